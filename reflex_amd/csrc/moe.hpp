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
// multiple of 4, 16-byte aligned rows) a workgroup takes 1024 columns of a
// token, four per lane, the k rows' loads issued together; else one element
// per lane. Same operations in the same order either way.
extern "C" __global__ __launch_bounds__(256) void rfxq_moe_combine(const float* __restrict__ pair_out,
                                                                  const int32_t* __restrict__ idx,
                                                                  const float* __restrict__ w,
                                                                  float* __restrict__ out, uint32_t tokens,
                                                                  uint32_t k, uint32_t hidden, uint32_t vec) {
    if (vec) {
        // a workgroup per (token, 1024-column chunk); every one of the k
        // rows' loads is issued (an absent pair reads row 0 and keeps acc
        // by a select), so they are in flight together
        const uint32_t chunks = (hidden + 1023u) / 1024u;
        for (uint32_t b = blockIdx.x; b < tokens * chunks; b += gridDim.x) {
            const uint32_t t = b / chunks;
            const uint64_t tk = (uint64_t)t * k;
            const uint32_t c = (b % chunks) * 1024u + 4u * threadIdx.x;
            if (c < hidden) {
                float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 8
                for (uint32_t j = 0; j < k; j++) {
                    const int32_t p = idx[tk + j];
                    const bool has = p >= 0;
                    const float wj = w[tk + j];
                    const float4 v = *reinterpret_cast<const float4*>(pair_out + (uint64_t)(has ? p : 0) * hidden + c);
                    acc.x = has ? fmaf(wj, v.x, acc.x) : acc.x;
                    acc.y = has ? fmaf(wj, v.y, acc.y) : acc.y;
                    acc.z = has ? fmaf(wj, v.z, acc.z) : acc.z;
                    acc.w = has ? fmaf(wj, v.w, acc.w) : acc.w;
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

// route_top_k_with_norm (src/moe.rs:47-98), one workgroup of G threads per
// token: softmax of the logits (max subtracted; the sum by wave 0 as lane
// sums over its experts l, l + 64, ... then group_sum's lane reduction, so it
// can differ from a sequential sum in the last bit; the decode router sums
// in the same order, so both give the same probabilities), the k best by
// probability descending then expert index ascending, renormalised by their
// sum (in selection order) when `normalize`; weights multiplied by `scale`.
// Selection by rank: the ranking values go to LDS and every expert counts
// those that precede it (greater, or equal at a lower index), the count split
// over all G threads (G / E threads per expert, each over a slice of the
// experts, summed by LDS atomics); the experts of rank < k are the selection,
// in rank order. A NaN probability ranks below every number (value -0.5), so
// the k indices are always valid experts (such a token's weights are NaN).
struct RouteLds {
    float rv[kRouteMaxE];      // ranking values (padding to whole float4s: -1)
    float pv[kRouteMaxE];      // probabilities
    uint32_t rank[kRouteMaxE];
    float slot_p[64];
    int32_t slot_e[64];
    float red[16];             // per-wave maxima, then the sum
};

template <uint32_t G>
__device__ __forceinline__ void moe_route_token(const float* __restrict__ logits, uint32_t t, uint32_t E,
                                                uint32_t k, uint32_t normalize, float scale,
                                                int32_t* __restrict__ idx, float* __restrict__ wts, RouteLds& L) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const float* l = logits + (uint64_t)t * E;
    // max (exact in any order)
    float mx = -INFINITY;
    for (uint32_t e = tid; e < E; e += G) {
        const float v = l[e];
        L.pv[e] = v;
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    if (lane == 0u) L.red[wave] = mx;
    for (uint32_t e = tid; e < E; e += G) L.rank[e] = 0u;
    __syncthreads();
    mx = L.red[0];
#pragma unroll
    for (uint32_t w = 1; w < G / 64u; w++) mx = fmaxf(mx, L.red[w]);
    for (uint32_t e = tid; e < E; e += G) L.pv[e] = expf(L.pv[e] - mx);
    __syncthreads();
    if (wave == 0u) {
        float sum = 0.0f;
        for (uint32_t e = lane; e < E; e += 64u) sum += L.pv[e];
        sum = group_sum<64>(sum);
        if (lane == 0u) L.red[0] = sum;
    }
    __syncthreads();
    const float sum = L.red[0];
    const uint32_t E4 = (E + 3u) & ~3u;
    for (uint32_t e = tid; e < E4; e += G) {
        if (e < E) {
            const float p = L.pv[e] / sum;
            L.pv[e] = p;
            L.rv[e] = p == p ? p : -0.5f;
        } else {
            L.rv[e] = -1.0f;  // precedes nothing
        }
    }
    __syncthreads();
    // S slices of the experts per expert (S = G / E, at least 1)
    const uint32_t S = G >= 2u * E ? G / E : 1u;
    const uint32_t chunk = ((E4 / 4u + S - 1u) / S) * 4u;
    for (uint32_t i = tid; i < E * S; i += G) {
        const uint32_t e = i % E, c0 = (i / E) * chunk, c1 = min(E4, c0 + chunk);
        const float mine = L.rv[e];
        uint32_t r = 0;
        for (uint32_t c = c0; c < c1; c += 4u) {
            const float4 q = *reinterpret_cast<const float4*>(L.rv + c);
            r += (q.x > mine || (q.x == mine && c < e)) ? 1u : 0u;
            r += (q.y > mine || (q.y == mine && c + 1u < e)) ? 1u : 0u;
            r += (q.z > mine || (q.z == mine && c + 2u < e)) ? 1u : 0u;
            r += (q.w > mine || (q.w == mine && c + 3u < e)) ? 1u : 0u;
        }
        if (S > 1u) atomicAdd(&L.rank[e], r);
        else L.rank[e] = r;
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += G) {
        const uint32_t r = L.rank[e];
        if (r < k) {
            L.slot_p[r] = L.pv[e];
            L.slot_e[r] = (int32_t)e;
        }
    }
    __syncthreads();
    if (tid < k) {
        float top_sum = 0.0f;  // in selection order
        for (uint32_t s2 = 0; s2 < k; s2++) top_sum += L.slot_p[s2];
        const float sel_p = L.slot_p[tid];
        const float wv = normalize ? sel_p / top_sum : sel_p;
        idx[(uint64_t)t * k + tid] = L.slot_e[tid];
        wts[(uint64_t)t * k + tid] = wv * scale;
    }
    __syncthreads();  // the scratch is free again
}

// With xh set, the workgroup then writes its token's row of x in the f16
// activation layout (rfxq_act_f16_wg's row, the same values), so the grouped
// MMQ path needs no launch of its own for it.
extern "C" __global__ __launch_bounds__(256) void rfxq_moe_route(const float* __restrict__ logits, uint32_t tokens,
                                                                uint32_t E, uint32_t k, uint32_t normalize,
                                                                float scale, int32_t* __restrict__ idx,
                                                                float* __restrict__ wts, const float* __restrict__ x,
                                                                uint32_t hidden, uint16_t* __restrict__ xh,
                                                                uint16_t* __restrict__ xsx, float* __restrict__ xrs) {
    __shared__ __attribute__((aligned(16))) RouteLds L;
    moe_route_token<256>(logits, blockIdx.x, E, k, normalize, scale, idx, wts, L);
    if (xh) act_f16_row_wg(QuantSrcPlain{x, hidden, nullptr}, blockIdx.x, hidden, xh, xsx, xrs, nullptr);
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
    // 1: group the pairs in any order within an expert (places by LDS
    // atomics, then a prefix sum of the counts); 0: a stable sort (token
    // order within an expert)
    uint32_t any_order;
    // 1: gate and up in one descriptor per expert (MmqDesc::gu_pair; the
    // template tg carries the pair fields, tu the up weights' base)
    uint32_t gu_pair;
};

// Exclusive prefix sum of v over the 1024 threads of the workgroup (every
// thread takes part): wave scans, then the wave totals (`tot`: 16 words of
// LDS). Integer adds, so the grouping does not matter.
__device__ __forceinline__ uint32_t plan_scan(uint32_t v, uint32_t* tot) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    // inclusive within each 16-lane row (DPP row_shr 1, 2, 4, 8: lanes
    // shifted in from outside the row add 0), then the earlier rows' totals
    uint32_t x = v;
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, false);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, false);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, false);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, false);
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)x, 15);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)x, 31);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)x, 47);
    const uint32_t row = lane >> 4;
    x += (row >= 1u ? r0 : 0u) + (row >= 2u ? r1 : 0u) + (row >= 3u ? r2 : 0u);
    if (lane == 63u) tot[wave] = x;
    __syncthreads();
    uint32_t pre = 0;
    for (uint32_t w = 0; w < wave; w++) pre += tot[w];
    __syncthreads();  // tot is free again
    return pre + x - v;
}

extern "C" __global__ __launch_bounds__(1024) void rfxq_moe_plan(MoePlanArgs a) {
    __shared__ uint16_t pe[kPlanMaxPairs];                        // expert of each pair
    __shared__ __attribute__((aligned(16))) float pw[kPlanMaxPairs];  // its weight (first: routing scratch)
    static_assert(sizeof(RouteLds) <= sizeof(float) * kPlanMaxPairs, "routing scratch inside pw");
    __shared__ uint32_t start[kRouteMaxE + 1], cnt[kRouteMaxE];
    const uint32_t tid = threadIdx.x, P = a.tokens * a.k;
    if (a.logits) {
        // (its workgroup barriers order the global writes for the reads below)
        RouteLds& L = *reinterpret_cast<RouteLds*>(pw);
        for (uint32_t t = 0; t < a.tokens; t++)
            moe_route_token<1024>(a.logits, t, a.E, a.k, a.normalize, a.scale, const_cast<int32_t*>(a.idx),
                                  const_cast<float*>(a.wts), L);
    }
    // Grouping with `any_order` (the grouped MMQ form): below. Otherwise a
    // stable counting sort of the pairs by expert: the pairs' experts and
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
    __shared__ uint32_t tot[16];
    if (a.any_order) {
        // A pair's place among its expert's rows is its order of arrival at
        // an LDS counter, which changes from call to call; no result depends
        // on it: each output row of the expert GEMMs is computed from its own
        // activation row alone, and the combine sums a token's pairs in
        // expert order from comb_idx.
        uint16_t* inv = &wcnt[0][0];  // pair index at each place (the sort's counts are not used here)
        static_assert(sizeof(wcnt) >= kPlanMaxPairs * sizeof(uint16_t), "inverse places in wcnt");
        for (uint32_t e = tid; e < E; e += 1024u) cnt[e] = 0u;
        __syncthreads();
        uint32_t my_pos[kPlanMaxPairs / 1024u];
#pragma unroll
        for (uint32_t u = 0; u < kPlanMaxPairs / 1024u; u++) {
            const uint32_t i = tid + 1024u * u;
            if (i < P) {
                const uint32_t e = min((uint32_t)a.idx[i], E - 1u);
                pe[i] = (uint16_t)e;
                pw[i] = a.wts[i];
                my_pos[u] = atomicAdd(&cnt[e], 1u);
            }
        }
        __syncthreads();
        const uint32_t hist = tid < E ? cnt[tid] : 0u;
        const uint32_t first = plan_scan(hist, tot);
        if (tid < E) start[tid] = first;
        __syncthreads();
#pragma unroll
        for (uint32_t u = 0; u < kPlanMaxPairs / 1024u; u++) {
            const uint32_t i = tid + 1024u * u;
            if (i < P) {
                const uint32_t e = pe[i], t = i / a.k;
                const uint32_t q = start[e] + my_pos[u];
                inv[q] = (uint16_t)i;
                uint32_t slot = 0;
                for (uint32_t j = 0; j < a.k; j++) slot += (uint32_t)pe[t * a.k + j] < e;
                a.comb_idx[(uint64_t)t * a.k + slot] = (int32_t)q;
                a.comb_w[(uint64_t)t * a.k + slot] = pw[i];
            }
        }
        // pair_row[q] = token of the pair at place q, stored in place order
        // (one CU's scattered dword stores to P places cost several us)
        __syncthreads();
        for (uint32_t q = tid; q < P; q += 1024u) a.pair_row[q] = (int32_t)(inv[q] / a.k);
    } else {
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
        const uint32_t first = plan_scan(hist, tot);
        if (tid < E) {
            base[tid] = first;
            start[tid] = first;
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
    }
    __syncthreads();
    if (a.gemv_gu) return;  // the GEMV form runs no MMQ launch
    // per expert (one thread each): rows, tiles; workgroup offsets by
    // exclusive scans over the experts
    const uint32_t tn_f = a.tg.tiles_n, tn_h = a.td.tiles_n;  // column tiles of gate / up and of down
    uint32_t m = 0, tm = 0, tmd = 0;
    if (tid < a.E) {
        m = cnt[tid];
        tm = (m + a.bm - 1u) / a.bm;
        tmd = (m + a.bm_dn - 1u) / a.bm_dn;
    }
    const uint32_t gpe = a.gu_pair ? 1u : 2u;  // gate/up descriptors per expert
    const uint32_t wg_gu = plan_scan(gpe * tm * tn_f, tot), wg_dn = plan_scan(tmd * tn_h, tot);
    // Descriptors from the templates, 128 experts at a time: filled in LDS
    // (the pairs' weights are no longer needed: their space holds them),
    // then stored with consecutive threads on consecutive words (one thread
    // per expert writing its own descriptors scatters every store).
    constexpr uint32_t kChunk = 128, kDw = sizeof(MmqDesc) / 4u;
    static_assert(sizeof(pw) >= 3u * kChunk * sizeof(MmqDesc), "descriptor staging in pw");
    MmqDesc* stg = reinterpret_cast<MmqDesc*>(pw);  // [2 kChunk] gate/up, then [kChunk] down
    for (uint32_t c0 = 0; c0 < a.E; c0 += kChunk) {
        const uint32_t nc = min(kChunk, a.E - c0);
        __syncthreads();  // (the previous chunk's copies have read the staging)
        if (tid >= c0 && tid < c0 + nc) {
            const uint32_t e = tid;
            const uint32_t st = m ? start[e] : 0u;  // (an expert with no rows has no tiles)
            MmqDesc* g = stg + gpe * (e - c0);
            MmqDesc* u = g + 1;  // (not used for a pair)
            MmqDesc* d = stg + 2u * kChunk + (e - c0);
            {
                const uint32_t* tg = reinterpret_cast<const uint32_t*>(&a.tg);
                const uint32_t* tu = reinterpret_cast<const uint32_t*>(&a.tu);
                const uint32_t* td = reinterpret_cast<const uint32_t*>(&a.td);
                uint32_t* pg = reinterpret_cast<uint32_t*>(g);
                uint32_t* pu = reinterpret_cast<uint32_t*>(u);
                uint32_t* pd = reinterpret_cast<uint32_t*>(d);
#pragma unroll
                for (uint32_t i = 0; i < kDw; i++) {
                    pg[i] = tg[i];
                    if (!a.gu_pair) pu[i] = tu[i];
                    pd[i] = td[i];
                }
            }
            g->w = a.tg.w + (uint64_t)e * a.w_stride_gu;
            if (a.gu_pair) g->w_up = a.tu.w + (uint64_t)e * a.w_stride_gu;
            else u->w = a.tu.w + (uint64_t)e * a.w_stride_gu;
            d->w = a.td.w + (uint64_t)e * a.w_stride_dn;
            g->rows = a.pair_row + st;
            g->m = d->m = m;
            g->tiles_m = tm;
            d->tiles_m = tmd;
            g->y = a.tg.y + (uint64_t)st * a.ffn;
            if (!a.gu_pair) {
                u->rows = a.pair_row + st;
                u->m = m;
                u->tiles_m = tm;
                u->y = a.tu.y + (uint64_t)st * a.ffn;
            }
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
            if (!a.gu_pair) u->wg_begin = wg_gu + tm * tn_f;
            d->wg_begin = wg_dn;
        }
        __syncthreads();
        const uint32_t* sw = reinterpret_cast<const uint32_t*>(stg);
        uint32_t* gu_out = reinterpret_cast<uint32_t*>(a.descs_gu + gpe * c0);
        uint32_t* dn_out = reinterpret_cast<uint32_t*>(a.descs_dn + c0);
        for (uint32_t i = tid; i < gpe * nc * kDw; i += 1024u) gu_out[i] = sw[i];
        for (uint32_t i = tid; i < nc * kDw; i += 1024u) dn_out[i] = sw[2u * kChunk * kDw + i];
    }
}
