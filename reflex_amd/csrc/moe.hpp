// MoE data movement and activation kernels.
//
// rfxq_moe_gather / rfxq_moe_scatter_add keep the semantics of the reference's
// `moe_gather_kernel` / `moe_scatter_add_kernel` (src/kernels_cuda/elementwise.cu:
// 175-222): dst[a,:] = src[perm[a],:] and dst[row[a],:] += w[a] * src[a,:] (no
// atomics; rows unique within one launch). rfxq_silu_and_mul is
// src/kernels_cuda/silu_and_mul.cu:7-23 (g / (1 + expf(-g)) * u).
//
// rfxq_moe_combine is the grouped pipeline's replacement for 128 per-expert
// scatter-adds: every token sums its k routed expert outputs in increasing
// expert order with the same fma, which is the order and rounding the
// reference's per-expert launch sequence produces (dense.rs:1549-1556 walks
// experts 0..E-1 and each launch adds into the zeroed output).
#pragma once
#include "common.hpp"

extern "C" __global__ __launch_bounds__(256) void rfxq_moe_gather(const float* __restrict__ src,
                                                                 const uint32_t* __restrict__ perm_row,
                                                                 float* __restrict__ dst, uint32_t num,
                                                                 uint32_t hidden) {
    const uint64_t total = (uint64_t)num * hidden;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256u) {
        const uint64_t a = i / hidden, c = i % hidden;
        dst[i] = src[(uint64_t)perm_row[a] * hidden + c];
    }
}

extern "C" __global__ __launch_bounds__(256) void rfxq_moe_scatter_add(const float* __restrict__ src,
                                                                      const uint32_t* __restrict__ dest_row,
                                                                      const float* __restrict__ weight,
                                                                      float* __restrict__ dst, uint32_t num,
                                                                      uint32_t hidden) {
    const uint64_t total = (uint64_t)num * hidden;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256u) {
        const uint64_t a = i / hidden, c = i % hidden;
        float* p = dst + (uint64_t)dest_row[a] * hidden + c;
        *p = fmaf(weight[a], src[i], *p);
    }
}

extern "C" __global__ __launch_bounds__(256) void rfxq_silu_and_mul(const float* __restrict__ gate,
                                                                   const float* __restrict__ up,
                                                                   float* __restrict__ out, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256u) {
        const float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

// out[t,:] = sum_j w[t,j] * pair_out[idx[t,j],:] for j in 0..k (pairs sorted
// by expert), evaluated as fma(w, v, acc) from acc = 0. With `vec` (hidden a
// multiple of 4, 16-byte aligned rows) a workgroup takes whole tokens, four
// columns per lane, the k rows' loads issued together; else one element per
// lane. Same operations in the same order either way.
extern "C" __global__ __launch_bounds__(256) void rfxq_moe_combine(const float* __restrict__ pair_out,
                                                                  const int32_t* __restrict__ idx,
                                                                  const float* __restrict__ w,
                                                                  float* __restrict__ out, uint32_t tokens,
                                                                  uint32_t k, uint32_t hidden, uint32_t vec) {
    if (vec) {
        for (uint32_t t = blockIdx.x; t < tokens; t += gridDim.x) {
            const uint64_t tk = (uint64_t)t * k;
            for (uint32_t c = 4u * threadIdx.x; c < hidden; c += 1024u) {
                float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
                for (uint32_t j = 0; j < k; j++) {
                    const int32_t p = idx[tk + j];
                    if (p >= 0) {
                        const float wj = w[tk + j];
                        const float4 v = *reinterpret_cast<const float4*>(pair_out + (uint64_t)p * hidden + c);
                        acc.x = fmaf(wj, v.x, acc.x);
                        acc.y = fmaf(wj, v.y, acc.y);
                        acc.z = fmaf(wj, v.z, acc.z);
                        acc.w = fmaf(wj, v.w, acc.w);
                    }
                }
                *reinterpret_cast<float4*>(out + (uint64_t)t * hidden + c) = acc;
            }
        }
        return;
    }
    const uint64_t total = (uint64_t)tokens * hidden;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256u) {
        const uint64_t t = i / hidden, c = i % hidden;
        float acc = 0.0f;
        for (uint32_t j = 0; j < k; j++) {
            const int32_t p = idx[t * k + j];
            if (p >= 0) acc = fmaf(w[t * k + j], pair_out[(uint64_t)p * hidden + c], acc);
        }
        out[i] = acc;
    }
}

// ---------------------------------------------------------------- device routing
//
// The grouped MoE pipeline with routing on the device: router logits stay in
// device memory (the reference copies them to the host, dense.rs:1602-1605,
// and uploads per-expert row lists, :1539-1546). rfxq_moe_route does the
// routing, rfxq_moe_plan the grouping and the MMQ descriptor tables; the
// MMQ, SiLU, quantize and combine launches that follow read those tables.

constexpr uint32_t kRouteMaxE = 1024;    // experts per lane: up to 16
constexpr uint32_t kPlanMaxPairs = 16384;  // sort keys in LDS

// route_top_k_with_norm (src/moe.rs:47-98), one wave per token: softmax of
// the logits (max subtracted; the sum over lanes then a butterfly, so it can
// differ from a sequential sum in the last bit), the k best by probability
// descending then expert index ascending, renormalised by their sum (in
// selection order) when `normalize`; weights multiplied by `scale`.
// Selection by rank rather than k rounds of a wave-wide arg-max (each a
// chain of cross-lane shuffles): the probabilities go to LDS and every
// expert counts those that precede it (greater, or equal at a lower index);
// the experts of rank < k are the selection, in rank order. A NaN
// probability ranks below every number, so the k indices are always valid
// experts (such a token's weights are NaN).
constexpr uint32_t kRouteLds = kRouteMaxE + 128u;  // floats per wave: probabilities, then k (p, e) slots
// One wave routes token t (all 64 lanes take part); `sp` is the wave's
// kRouteLds floats of LDS.
__device__ __forceinline__ void moe_route_token(const float* __restrict__ logits, uint32_t t, uint32_t E,
                                                uint32_t k, uint32_t normalize, float scale,
                                                int32_t* __restrict__ idx, float* __restrict__ wts, float* sp) {
    const uint32_t lane = threadIdx.x & 63u;
    const float* l = logits + (uint64_t)t * E;
    constexpr uint32_t J = kRouteMaxE / 64u;
    float p[J];
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
        const uint32_t e = lane + 64u * j;
        p[j] = e < E ? l[e] : -INFINITY;
        mx = fmaxf(mx, p[j]);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    float sum = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
        const uint32_t e = lane + 64u * j;
        p[j] = e < E ? expf(p[j] - mx) : 0.0f;
        sum += p[j];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 64);
    // ranking values: the probability, NaN as -0.5 (below every probability)
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
        const uint32_t e = lane + 64u * j;
        if (e < E) {
            p[j] = p[j] / sum;
            sp[e] = p[j] == p[j] ? p[j] : -0.5f;
        } else if (e < ((E + 3u) & ~3u)) {
            sp[e] = -1.0f;  // padding to whole float4s: precedes nothing
        }
    }
    float* slot_p = sp + kRouteMaxE;
    int32_t* slot_e = reinterpret_cast<int32_t*>(sp + kRouteMaxE + 64u);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
        const uint32_t e = lane + 64u * j;
        if (64u * j < E) {  // wave-uniform
            const float mine = e < E ? sp[e] : 0.0f;
            // experts below this chunk precede on >=, above it on >, and
            // within it on > or (== at a lower index)
            const uint32_t lo = 64u * j, hi = min(64u * j + 64u, (E + 3u) & ~3u), end = (E + 3u) & ~3u;
            uint32_t r = 0;
#pragma unroll 8
            for (uint32_t c = 0; c < lo; c += 4u) {
                const float4 q = *reinterpret_cast<const float4*>(sp + c);
                r += (uint32_t)(q.x >= mine) + (uint32_t)(q.y >= mine) + (uint32_t)(q.z >= mine) +
                     (uint32_t)(q.w >= mine);
            }
#pragma unroll 4
            for (uint32_t c = lo; c < hi; c += 4u) {
                const float4 q = *reinterpret_cast<const float4*>(sp + c);
                r += (q.x > mine || (q.x == mine && c < e)) ? 1u : 0u;
                r += (q.y > mine || (q.y == mine && c + 1u < e)) ? 1u : 0u;
                r += (q.z > mine || (q.z == mine && c + 2u < e)) ? 1u : 0u;
                r += (q.w > mine || (q.w == mine && c + 3u < e)) ? 1u : 0u;
            }
#pragma unroll 8
            for (uint32_t c = hi; c < end; c += 4u) {
                const float4 q = *reinterpret_cast<const float4*>(sp + c);
                r += (uint32_t)(q.x > mine) + (uint32_t)(q.y > mine) + (uint32_t)(q.z > mine) +
                     (uint32_t)(q.w > mine);
            }
            if (e < E && r < k) {
                slot_p[r] = p[j];
                slot_e[r] = (int32_t)e;
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
    float top_sum = 0.0f;  // in selection order
    for (uint32_t s = 0; s < k; s++) top_sum += slot_p[s];
    if (lane < k) {
        const float sel_p = slot_p[lane];
        const float wv = normalize ? sel_p / top_sum : sel_p;
        idx[(uint64_t)t * k + lane] = slot_e[lane];
        wts[(uint64_t)t * k + lane] = wv * scale;
    }
}

extern "C" __global__ __launch_bounds__(256) void rfxq_moe_route(const float* __restrict__ logits, uint32_t tokens,
                                                                uint32_t E, uint32_t k, uint32_t normalize,
                                                                float scale, int32_t* __restrict__ idx,
                                                                float* __restrict__ wts) {
    __shared__ __attribute__((aligned(16))) float sp[4][kRouteLds];
    const uint32_t t = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (t >= tokens) return;
    moe_route_token(logits, t, E, k, normalize, scale, idx, wts, sp[threadIdx.x >> 6]);
}

// Grouping and descriptor tables, one workgroup of 1024 threads: the pairs
// (token t, slot j) in the order (expert, t*k + j) by a stable counting sort;
// then
//   pair_row[q]       token of the pair at sorted position q (MMQ row gather)
//   comb_idx/comb_w   per token, its pairs' positions and weights in
//                     increasing expert order (the combine's order)
//   descs_gu[2e], [2e+1], descs_dn[e]  the gate, up and down MMQ descriptors
//                     of expert e, from templates whose per-expert fields
//                     (weights, rows, outputs, tile counts, workgroup
//                     offsets) are filled here.
struct MoePlanArgs {
    const int32_t* idx;
    const float* wts;
    int32_t* pair_row;
    int32_t* comb_idx;
    float* comb_w;
    MmqDesc* descs_gu;
    MmqDesc* descs_dn;
    MmqDesc tg, tu, td;         // templates (m, rows, wg_begin filled per expert)
    uint64_t w_stride_gu;       // bytes between experts in gate / up
    uint64_t w_stride_dn;       // ... in down
    uint32_t tokens, k, E, bm_dn;  // bm_dn: row tile of the down projection
    uint32_t bm, ffn, hidden, f16;  // bm: row tile of gate / up; f16: descriptors read the f16 activation layout
    // GEMV form (few tokens; gemv_gu NULL: not written): per sorted pair q,
    // gemv_gu[2q], [2q+1] = gate, up of its token's row, gemv_dn[q] = down of
    // the pair's SiLU·up row, from templates whose w, x and y are the bases
    GemvDesc* gemv_gu;
    GemvDesc* gemv_dn;
    GemvDesc vg, vu, vd;
    // routing in this launch (few tokens; NULL: idx / wts come from
    // rfxq_moe_route): one wave per token writes idx and wts first
    const float* logits;
    uint32_t normalize;
    float scale;
};

extern "C" __global__ __launch_bounds__(1024) void rfxq_moe_plan(MoePlanArgs a) {
    __shared__ uint16_t pe[kPlanMaxPairs];                        // expert of each pair
    __shared__ __attribute__((aligned(16))) float pw[kPlanMaxPairs];  // its weight (first: routing scratch)
    static_assert(4u * kRouteLds <= kPlanMaxPairs, "routing scratch inside pw");
    __shared__ uint32_t start[kRouteMaxE + 1], cnt[kRouteMaxE];
    const uint32_t tid = threadIdx.x, P = a.tokens * a.k;
    if (a.logits) {
        float (*sp)[kRouteLds] = reinterpret_cast<float (*)[kRouteLds]>(pw);
        if (tid < 256u)
            for (uint32_t t = tid >> 6; t < a.tokens; t += 4u)
                moe_route_token(a.logits, t, a.E, a.k, a.normalize, a.scale, const_cast<int32_t*>(a.idx),
                                const_cast<float*>(a.wts), sp[tid >> 6]);
        __syncthreads();  // (a workgroup barrier orders the global writes for the reads below)
    }
    // Stable counting sort of the pairs by expert: the pairs' experts and
    // weights read once into LDS; a histogram and its exclusive scan give each
    // expert's first position; then, chunk by chunk, a pair's rank among the
    // lanes of its wave with the same expert comes from ballots over the
    // expert's bits and the waves before it from per-wave counts in LDS.
    // The pair's sorted position q is written where it is used: its row
    // gather (pair_row[q]), its combine slot (the rank of its expert among
    // its token's experts) and, in the GEMV form, its descriptors.
    __shared__ uint32_t base[kRouteMaxE];
    __shared__ uint16_t wcnt[16][kRouteMaxE];
    const uint32_t E = a.E, lane = tid & 63u, wave = tid >> 6;
    for (uint32_t e = tid; e < E; e += 1024u) base[e] = 0u;
#pragma unroll 4
    for (uint32_t i = tid; i < P; i += 1024u) {
        pe[i] = (uint16_t)min((uint32_t)a.idx[i], E - 1u);
        pw[i] = a.wts[i];
    }
    __syncthreads();
    for (uint32_t i = tid; i < P; i += 1024u) atomicAdd(&base[pe[i]], 1u);
    __syncthreads();
    const uint32_t hist = tid < E ? base[tid] : 0u;
    for (uint32_t off = 1; off < E; off <<= 1) {
        const uint32_t o = (tid < E && tid >= off) ? base[tid - off] : 0u;
        __syncthreads();
        if (tid < E) base[tid] += o;
        __syncthreads();
    }
    if (tid < E) {
        base[tid] -= hist;  // inclusive -> exclusive
        start[tid] = base[tid];
        cnt[tid] = hist;
    }
    for (uint32_t c0 = 0; c0 < P; c0 += 1024u) {
        for (uint32_t j = tid; j < 16u * E; j += 1024u) wcnt[j / E][j % E] = 0u;
        __syncthreads();
        const uint32_t i = c0 + tid;
        const bool valid = i < P;
        const uint32_t e = valid ? (uint32_t)pe[i] : 0u;
        uint64_t same = __ballot(valid);
#pragma unroll
        for (uint32_t bit = 0; bit < 10u; bit++) {  // E <= 1024
            const uint64_t ones = __ballot((e >> bit) & 1u);
            same &= ((e >> bit) & 1u) ? ones : ~ones;
        }
        const uint32_t rank = (uint32_t)__popcll(same & ((1ull << lane) - 1ull));
        if (valid && rank == 0u) wcnt[wave][e] = (uint16_t)__popcll(same);
        __syncthreads();
        if (valid) {
            uint32_t q = base[e] + rank;
            for (uint32_t w = 0; w < wave; w++) q += wcnt[w][e];
            const uint32_t t = i / a.k;
            a.pair_row[q] = (int32_t)t;
            uint32_t slot = 0;
            for (uint32_t j = 0; j < a.k; j++) slot += (uint32_t)pe[t * a.k + j] < e;
            a.comb_idx[(uint64_t)t * a.k + slot] = (int32_t)q;
            a.comb_w[(uint64_t)t * a.k + slot] = pw[i];
            if (a.gemv_gu) {
                GemvDesc* dg = a.gemv_gu + 2u * q;
                GemvDesc* du = dg + 1;
                GemvDesc* dd = a.gemv_dn + q;
                const uint32_t* tg = reinterpret_cast<const uint32_t*>(&a.vg);
                const uint32_t* tu = reinterpret_cast<const uint32_t*>(&a.vu);
                const uint32_t* td = reinterpret_cast<const uint32_t*>(&a.vd);
#pragma unroll
                for (uint32_t f = 0; f < sizeof(GemvDesc) / 4u; f++) {
                    reinterpret_cast<uint32_t*>(dg)[f] = tg[f];
                    reinterpret_cast<uint32_t*>(du)[f] = tu[f];
                    reinterpret_cast<uint32_t*>(dd)[f] = td[f];
                }
                dg->w = a.vg.w + (uint64_t)e * a.w_stride_gu;
                du->w = a.vu.w + (uint64_t)e * a.w_stride_gu;
                dd->w = a.vd.w + (uint64_t)e * a.w_stride_dn;
                dg->x = du->x = a.vg.x + (uint64_t)t * a.hidden;
                dg->y = a.vg.y + (uint64_t)q * a.ffn;
                du->y = a.vu.y + (uint64_t)q * a.ffn;
                dd->x = a.vd.x + (uint64_t)q * a.ffn;
                dd->y = a.vd.y + (uint64_t)q * a.hidden;
            }
        }
        __syncthreads();
        if (tid < E) {
            uint32_t n = 0;
            for (uint32_t w = 0; w < 16u; w++) n += wcnt[w][tid];
            base[tid] += n;
        }
        __syncthreads();  // (the next chunk clears wcnt)
    }
    __syncthreads();
    // per expert (one thread each): rows, tiles; workgroup offsets by an
    // inclusive scan over the experts (Hillis-Steele in LDS)
    __shared__ uint32_t scan_gu[kRouteMaxE], scan_dn[kRouteMaxE];
    const uint32_t tn_f = a.tg.tiles_n, tn_h = a.td.tiles_n;  // column tiles of gate / up and of down
    uint32_t m = 0, tm = 0, tmd = 0;
    if (tid < a.E) {
        m = cnt[tid];
        tm = (m + a.bm - 1u) / a.bm;
        tmd = (m + a.bm_dn - 1u) / a.bm_dn;
        scan_gu[tid] = 2u * tm * tn_f;
        scan_dn[tid] = tmd * tn_h;
    }
    __syncthreads();
    for (uint32_t off = 1; off < a.E; off <<= 1) {
        uint32_t vg = 0, vd = 0;
        if (tid < a.E && tid >= off) {
            vg = scan_gu[tid - off];
            vd = scan_dn[tid - off];
        }
        __syncthreads();
        if (tid < a.E) {
            scan_gu[tid] += vg;
            scan_dn[tid] += vd;
        }
        __syncthreads();
    }
    if (tid < a.E) {
        const uint32_t e = tid;
        const uint32_t st = m ? start[e] : 0u;  // (an expert with no rows has no tiles)
        const uint32_t wg_gu = scan_gu[e] - 2u * tm * tn_f, wg_dn = scan_dn[e] - tmd * tn_h;
        // descriptors from the templates, filled in place in global memory
        MmqDesc* g = a.descs_gu + 2u * e;
        MmqDesc* u = g + 1;
        MmqDesc* d = a.descs_dn + e;
        {
            const uint32_t* tg = reinterpret_cast<const uint32_t*>(&a.tg);
            const uint32_t* tu = reinterpret_cast<const uint32_t*>(&a.tu);
            const uint32_t* td = reinterpret_cast<const uint32_t*>(&a.td);
            uint32_t* pg = reinterpret_cast<uint32_t*>(g);
            uint32_t* pu = reinterpret_cast<uint32_t*>(u);
            uint32_t* pd = reinterpret_cast<uint32_t*>(d);
#pragma unroll
            for (uint32_t i = 0; i < sizeof(MmqDesc) / 4u; i++) {
                pg[i] = tg[i];
                pu[i] = tu[i];
                pd[i] = td[i];
            }
        }
        g->w = a.tg.w + (uint64_t)e * a.w_stride_gu;
        u->w = a.tu.w + (uint64_t)e * a.w_stride_gu;
        d->w = a.td.w + (uint64_t)e * a.w_stride_dn;
        g->rows = u->rows = a.pair_row + st;
        g->m = u->m = d->m = m;
        g->tiles_m = u->tiles_m = tm;
        d->tiles_m = tmd;
        g->y = a.tg.y + (uint64_t)st * a.ffn;
        u->y = a.tu.y + (uint64_t)st * a.ffn;
        if (a.f16) {  // xh rows of 2*ffn bytes, xsx records of ffn/256 * 32 bytes, xrs
            d->xq = a.td.xq + (uint64_t)st * a.ffn * 2u;
            d->xds = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(a.td.xds) +
                                                       (uint64_t)st * (a.ffn / 256u) * 32u);
            d->xrs = a.td.xrs + st;
        } else {
            d->xq = a.td.xq + (uint64_t)st * a.ffn;
            d->xds = a.td.xds + (uint64_t)st * (a.ffn / 32u);
        }
        d->y = a.td.y + (uint64_t)st * a.hidden;
        g->wg_begin = wg_gu;
        u->wg_begin = wg_gu + tm * tn_f;
        d->wg_begin = wg_dn;
    }
}
