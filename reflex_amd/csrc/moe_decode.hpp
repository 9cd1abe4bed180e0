// MoE decode (a few tokens) in two launches.
//
// The grouped expert FFN of `moe_ffn_grouped` (src/model/dense.rs:1509-1559)
// at decode sizes: every routed pair (token t, slot j -> expert e) needs
// gate/up GEMVs of its token's row, SiLU·up (silu_and_mul.cu:7-23), a down
// GEMV of that, and the weighted sum over the token's k pairs in increasing
// expert order (dense.rs:1549-1556). At one token the expert weights (21 MB at
// config 5) stream in a few microseconds, so launches, not bytes, set the
// time; this pipeline has two:
//
//   rfxq_moe_dec_gu    workgroup = (token, slot, block of rows): routes the
//                      token (every wave of it, identically, moe_route_wave;
//                      or reads a routing the host uploaded), stages the
//                      token's x in LDS
//                      (f16, as the decode GEMV does), computes its rows of
//                      the gate and up projections of the slot's expert and
//                      writes s = silu(gate) * up.
//   rfxq_moe_dec_down  workgroup = (token, block of output rows): stages the
//                      token's k rows of s (one row of k * ffn values), lane
//                      groups compute each (row, slot) dot with its expert's
//                      down weights, and one thread per row adds the k values
//                      weighted, in increasing expert order, fma from 0 (the
//                      order and rounding of rfxq_moe_combine).
//
// Weights are read straight from the stacked expert tensors (a buffer
// resource over all experts: the host keeps them below 4 GiB) into registers,
// one unit (64 weights; a 32-block for Q8_0) per lane at a time in batches of
// four, and contracted with the decode GEMV's unit dots (gemv.hpp), so the
// arithmetic per pair is the GEMV's.
#pragma once
#include "common.hpp"
#include "gemv.hpp"
#include "moe.hpp"

// A unit's bytes from global memory (offset `o` of its block start in the
// buffer), laid out as the LDS fetches of gemv.hpp produce them.
template <typename T>
RFXQ_DEV typename T::Raw moe_fetch(rsrc_t r, uint32_t o, uint32_t unit);

template <>
RFXQ_DEV Q4K::Raw moe_fetch<Q4K>(rsrc_t r, uint32_t o, uint32_t unit) {
    const uint32_t q = o + 16u + 32u * (unit & 3u);
    return Q4K::Raw{bld16(r, o), bld16(r, q), bld16(r, q + 16u)};
}

template <>
RFXQ_DEV Q6K::Raw moe_fetch<Q6K>(rsrc_t r, uint32_t o, uint32_t unit) {
    const uint32_t g = unit & 3u, n = g >> 1, hs = g & 1u;
    const uint32_t a4 = o & ~3u;
    const uint32_t pa = a4 + 64u * n + 16u * hs, ph = a4 + 128u + 32u * n + 16u * hs;
    Q6K::Raw w;
    w.sh = o & 3u;
    w.a = Seg{bld16(r, pa), bld4(r, pa + 16u)};
    w.c = Seg{bld16(r, pa + 32u), bld4(r, pa + 48u)};
    w.h = Seg{bld16(r, ph), bld4(r, ph + 16u)};
    w.sw = bld16(r, a4 + 192u);
    w.tail = bld4(r, a4 + 208u);
    return w;
}

template <>
RFXQ_DEV Q80::Raw moe_fetch<Q80>(rsrc_t r, uint32_t o, uint32_t) {
    const uint32_t a4 = o & ~3u;
    return Q80::Raw{bld16(r, a4), bld16(r, a4 + 16u), bld4(r, a4 + 32u), o & 3u};
}

// gemv_x_load without branches: every load issued (a buffer resource returns
// zeros past x), so the compiler can count them and later waits do not wait
// for loads issued after them (such as the first weights)
RFXQ_DEV void moe_x_load(const float* x, uint32_t k, XRegs& xr, uint32_t tid) {
    const rsrc_t r = make_rsrc(x, k * 4u);
#pragma unroll
    for (uint32_t i = 0; i < kGemvMaxK / 1024u; i++) {
        const u4_t v = bld16(r, 16u * tid + 4096u * i);
        xr.v[i] = make_float4(as_f32(v.x), as_f32(v.y), as_f32(v.z), as_f32(v.w));
    }
}

struct MoeDecArgs {
    const float* x;        // [tokens][hidden]
    const float* logits;   // [tokens][E] router logits on the device; NULL: idx / wts hold the routing
    int32_t* idx;          // [tokens][k] experts (in selection order)
    float* wts;            // [tokens][k] their weights (times the weight scale)
    const uint8_t* wg;     // stacked gate [E][ffn][hidden], up, down [E][hidden][ffn]
    const uint8_t* wu;
    const uint8_t* wd;
    uint64_t eb_gu, eb_dn;  // bytes per expert
    float* s;              // [tokens][k][ffn] silu(gate) * up
    float* out;            // [tokens][hidden]
    uint32_t tokens, E, k, hidden, ffn, normalize;
    float scale;
    uint32_t nb1, nr1;     // gate/up: row blocks per slot, rows per block (of each projection)
    uint32_t nb2, nr2;     // down: row blocks per token, rows per block
    uint32_t lds_x1, lds_x2;  // byte offsets of the staged x in LDS
    // host routing of up to kDecInlinePairs pairs carried in the kernel
    // arguments (n_inline != 0: read instead of idx / wts; no upload)
    uint32_t n_inline;
    int32_t h_idx[32];
    float h_w[32];
};
constexpr uint32_t kDecInlinePairs = 32;

// buffer resource over a stacked tensor whose data may start 2 bytes past a
// dword: base rounded down, the remainder (*sh) added to every offset
RFXQ_DEV rsrc_t moe_rsrc(const uint8_t* p, uint64_t bytes, uint32_t* sh) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    *sh = (uint32_t)(a & 3u);
    return make_rsrc(reinterpret_cast<const void*>(a - *sh), (uint32_t)((bytes + *sh + 3u) & ~3ull));
}

// One row of `K` weights at byte offset `ro` dotted with the staged x from
// unit `xu` on: units li, li + LPR, ... of the row, in batches of four. The
// first batch's loads are issued by fetch0, before the x staging, so they
// are in flight during it.
template <typename T, int LPR>
struct MoeRowDot {
    typename T::Raw raw[4];
    rsrc_t r;
    uint32_t ro, U, li;
    __device__ __forceinline__ MoeRowDot(rsrc_t r_, uint32_t ro_, uint32_t K, uint32_t li_)
        : r(r_), ro(ro_), U(K / (T::QK / T::UPB) / LPR), li(li_) {}
    // every load issued (units past the row repeat the last one), so that
    // the compiler counts them and waits for earlier loads do not wait for them
    __device__ __forceinline__ void fetch(uint32_t u0) {
#pragma unroll
        for (uint32_t q = 0; q < 4u; q++) {
            const uint32_t unit = li + min(u0 + q, U - 1u) * LPR;
            raw[q] = moe_fetch<T>(r, ro + T::unit_off(unit), unit);
        }
    }
    __device__ __forceinline__ void fetch0() { fetch(0u); }
    __device__ __forceinline__ float dot(uint32_t xu, const uint32_t* lds_x, const float* lds_s, uint32_t magic) {
        float acc = 0.0f;
        for (uint32_t u0 = 0; u0 < U; u0 += 4u) {
            if (u0) fetch(u0);
#pragma unroll
            for (uint32_t q = 0; q < 4u; q++)
                if (u0 + q < U) {
                    const uint32_t unit = li + (u0 + q) * LPR;
                    typename T::XV xv;
                    T::loadx(lds_x, lds_s, xu + unit, xv);
                    acc += T::dot(raw[q], unit, xv, magic);
                }
        }
        return acc;
    }
};

// the wave's maximum of 32-bit signed integers in every lane: DPP steps
// (folded into v_max_i32) within each row, then the row swaps across rows
// (all in vector registers: no round trip through scalar ones)
RFXQ_DEV int32_t wave_max_i32(int32_t v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
    const auto a = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = max((int32_t)a[0], (int32_t)a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return max((int32_t)b[0], (int32_t)b[1]);
}

// float -> int32 of the same order (signed compare): negative floats have
// their magnitude bits flipped
RFXQ_DEV int32_t order_key(float f) {
    const int32_t b = __builtin_bit_cast(int32_t, f);
    return b ^ ((b >> 31) & 0x7FFFFFFF);
}

constexpr uint32_t kDecRouteMaxE = 256;  // experts the one-wave router takes (4 per lane)

// route_top_k_with_norm (src/moe.rs:47-98) of one token by one wave (no
// barrier, no LDS): softmax with the maximum subtracted (expf, the sum by a
// fixed wave reduction), probabilities p = v / sum, and the k best by p
// descending then index ascending (a NaN p ranks below every number),
// renormalised by their sum in selection order when `normalize`, times
// `scale`. Lane l holds experts l + 64 i. Each of the k rounds takes the
// wave-wide maximum of the ranking keys (the integer order of p; NaN p as
// -0.5, absent experts as -2, taken ones INT32_MIN) and, among the experts
// holding it, the lowest index: the first set bit of the ballots of chunks
// i = 0, 1, ... (p is never -0.0, so equal keys are the reference's ties).
// Deterministic, so every wave of a token finds the same routing. Returns
// slot `slot`'s expert; lanes < k write idx / wts when `write`.
struct RouteLogits {
    float v[kDecRouteMaxE / 64u];
};
// the token's logits, lane l holding experts l + 64 i (all loads in flight at
// once: a buffer resource reads 0 past the row)
RFXQ_DEV void moe_route_load(const float* __restrict__ logits, uint32_t t, uint32_t E, RouteLogits& rl) {
    const uint32_t lane = threadIdx.x & 63u;
    const rsrc_t lr = make_rsrc(logits + (uint64_t)t * E, E * 4u);
#pragma unroll
    for (uint32_t i = 0; i < kDecRouteMaxE / 64u; i++) rl.v[i] = as_f32(bld4(lr, 4u * (lane + 64u * i)));
}

// NV = ceil(E / 64) chunks of experts per lane (1, 2 or 4), so no chunk
// loop tests E. Only the writing wave needs every pick's probability; the
// others need pick `slot` alone and stop there.
template <uint32_t NV>
RFXQ_DEV int32_t moe_route_wave_n(const RouteLogits& rl, uint32_t t, uint32_t E, uint32_t k, uint32_t normalize,
                                  float scale, int32_t* __restrict__ idx, float* __restrict__ wts, uint32_t slot,
                                  bool write) {
    const uint32_t lane = threadIdx.x & 63u;
    float v[NV];
#pragma unroll
    for (uint32_t i = 0; i < NV; i++) v[i] = rl.v[i];
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t i = 0; i < NV; i++) mx = lane + 64u * i < E ? fmaxf(mx, v[i]) : mx;
    mx = wave_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < NV; i++) {
        v[i] = lane + 64u * i < E ? expf(v[i] - mx) : 0.0f;
        sum += v[i];  // (absent experts add 0)
    }
    sum = group_sum<64>(sum);
    // ranking keys: the order of p (a NaN p as -0.5, absent experts as -2;
    // taken ones INT32_MIN), compared as integers
    int32_t rk[NV];
#pragma unroll
    for (uint32_t i = 0; i < NV; i++) {
        v[i] = v[i] / sum;
        rk[i] = order_key(lane + 64u * i < E ? (v[i] == v[i] ? v[i] : -0.5f) : -2.0f);
    }
    float my_p = 0.0f, top_sum = 0.0f;
    int32_t my_e = 0, pick = 0;
    const uint32_t rounds = write ? k : slot + 1u;
    for (uint32_t r = 0; r < rounds; r++) {
        int32_t m = rk[0];
#pragma unroll
        for (uint32_t i = 1; i < NV; i++) m = max(m, rk[i]);
        m = wave_max_i32(m);
        // the lowest expert holding the maximum
        uint32_t be = 0xFFFFFFFFu;
#pragma unroll
        for (uint32_t i = 0; i < NV; i++) {
            const uint64_t bits = __ballot(rk[i] == m);
            if (be == 0xFFFFFFFFu && bits) be = 64u * i + (uint32_t)__builtin_ctzll(bits);
        }
        be = __builtin_amdgcn_readfirstlane(be);
#pragma unroll
        for (uint32_t i = 0; i < NV; i++) rk[i] = lane + 64u * i == be ? INT32_MIN : rk[i];  // taken
        if (r == slot) pick = (int32_t)be;
        if (write) {
            // the winner's probability, read by its lane and broadcast
            const uint32_t owner = be & 63u, oi = be >> 6;
            float pv = v[0];
#pragma unroll
            for (uint32_t i = 1; i < NV; i++) pv = i == oi ? v[i] : pv;
            pv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv), owner));
            top_sum += pv;  // in selection order
            if (lane == r) {
                my_p = pv;
                my_e = (int32_t)be;
            }
        }
    }
    if (write && lane < k) {
        idx[(uint64_t)t * k + lane] = my_e;
        wts[(uint64_t)t * k + lane] = (normalize ? my_p / top_sum : my_p) * scale;
    }
    return pick;
}

RFXQ_DEV int32_t moe_route_wave(const RouteLogits& rl, uint32_t t, uint32_t E, uint32_t k, uint32_t normalize,
                                float scale, int32_t* __restrict__ idx, float* __restrict__ wts, uint32_t slot,
                                bool write) {
    if (E <= 64u) return moe_route_wave_n<1>(rl, t, E, k, normalize, scale, idx, wts, slot, write);
    if (E <= 128u) return moe_route_wave_n<2>(rl, t, E, k, normalize, scale, idx, wts, slot, write);
    return moe_route_wave_n<4>(rl, t, E, k, normalize, scale, idx, wts, slot, write);
}

template <typename T, int LPR>
RFXQ_DEV void moe_dec_gu(const MoeDecArgs& a, uint8_t* lds) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    // uniform: the wave picks the weight tensor, whose V# must stay scalar
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t per_t = a.k * a.nb1;
    const uint32_t t = blockIdx.x / per_t, j = (blockIdx.x / a.nb1) % a.k, b = blockIdx.x % a.nb1;
    const float* xt = a.x + (uint64_t)t * a.hidden;
    // loads in the order they are needed (the wait for one also waits for
    // every load issued before it): the routing, then x (staged after the
    // first weight loads are issued)
    RouteLogits lg;
    int32_t e_raw = 0;
    if (a.logits) moe_route_load(a.logits, t, a.E, lg);
    else e_raw = a.n_inline ? a.h_idx[t * a.k + j] : a.idx[(uint64_t)t * a.k + j];
    __builtin_amdgcn_sched_barrier(0);  // (keeps the x loads after these)
    XRegs xr;
    moe_x_load(xt, a.hidden, xr, tid);
    // every wave routes the token itself (no barrier) as far as its slot;
    // one wave per token routes it again in full, while its weights are in
    // flight, and writes the routing for the down launch
    const bool writer = a.logits && wave == 0u && j == 0u && b == 0u;
    if (a.logits) e_raw = moe_route_wave(lg, t, a.E, a.k, a.normalize, a.scale, a.idx, a.wts, j, false);
    int32_t e = e_raw;
    e = __builtin_amdgcn_readfirstlane(min((uint32_t)e, a.E - 1u));
    // waves 0-1: gate rows, waves 2-3: up rows (a wave-uniform weight tensor);
    // the first weights are requested before x is staged
    constexpr uint32_t RPW = 64u / LPR;
    const uint32_t gi = lane / LPR, li = lane % LPR, p = wave >> 1;
    const uint32_t rl = (wave & 1u) * RPW + gi;
    const uint32_t r = min(b * a.nr1 + rl, a.ffn - 1u);
    const uint32_t row_bytes = a.hidden / T::QK * T::BB;
    uint32_t sh;
    const rsrc_t rs = moe_rsrc(p ? a.wu : a.wg, (uint64_t)a.E * a.eb_gu, &sh);
    MoeRowDot<T, LPR> rd(rs, sh + (uint32_t)(e * a.eb_gu) + r * row_bytes, a.hidden, li);
    rd.fetch0();
    if (writer) (void)moe_route_wave(lg, t, a.E, a.k, a.normalize, a.scale, a.idx, a.wts, j, true);
    uint32_t* lds_x = reinterpret_cast<uint32_t*>(lds + a.lds_x1);
    float* lds_s = reinterpret_cast<float*>(lds_x + a.hidden / 2u);
    float* lds_p = lds_s + a.hidden / 16u;  // 4 floats: the stage's wave maxima
    float* res = lds_p + 4;                 // [2][nr1] gate, up rows
    const float inv = gemv_stage_x(xt, a.hidden, T::XHI, xr, lds_x, lds_s, lds_p, tid);
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    float acc = rd.dot(0u, lds_x, lds_s, magic);
    acc = group_sum<LPR>(acc);
    if (li == 0u) lds_st32(lds_addr(res + p * a.nr1 + rl), __builtin_bit_cast(uint32_t, acc * inv));
    lds_barrier();
    if (tid < a.nr1) {
        const uint32_t row = b * a.nr1 + tid;
        if (row < a.ffn) {
            const float g = __builtin_bit_cast(float, lds_ld32(lds_addr(res + tid)));
            const float u = __builtin_bit_cast(float, lds_ld32(lds_addr(res + a.nr1 + tid)));
            a.s[((uint64_t)t * a.k + j) * a.ffn + row] = (g / (1.0f + expf(-g))) * u;
        }
    }
}

template <typename T, int LPR>
RFXQ_DEV void moe_dec_down(const MoeDecArgs& a, uint8_t* lds) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t t = blockIdx.x / a.nb2, b = blockIdx.x % a.nb2;
    const uint32_t K2 = a.k * a.ffn;
    const float* st = a.s + (uint64_t)t * K2;
    // the token's experts and weights (loaded first: waiting for them must not
    // wait for the staged row's loads), and the combine order (increasing
    // expert, then slot)
    int32_t* le = reinterpret_cast<int32_t*>(lds);
    float* lw = reinterpret_cast<float*>(le + 64);
    uint32_t* ord = reinterpret_cast<uint32_t*>(lw + 64);
    // lane group gi = (row, slot) item: row rl = item / k, slot j = item % k;
    // each lane loads its slot's expert itself, so its first weights are
    // requested as soon as that arrives (before the LDS tables, the combine
    // order and the staging of x)
    constexpr uint32_t RPW = 64u / LPR;
    const uint32_t gi = lane / LPR, li = lane % LPR;
    const uint32_t item = wave * RPW + gi, rl = item / a.k, j = item % a.k;
    uint32_t e_slot, my_e = 0, my_w = 0;
    if (a.n_inline) {  // the host's routing in the kernel arguments
        const int32_t* hi = &a.h_idx[0] + t * a.k;
        const float* hw = &a.h_w[0] + t * a.k;
        e_slot = (uint32_t)hi[min(j, a.k - 1u)];
        if (tid < a.k) {
            my_e = (uint32_t)hi[tid];
            my_w = __builtin_bit_cast(uint32_t, hw[tid]);
        }
    } else {
        const rsrc_t ri = make_rsrc(a.idx + (uint64_t)t * a.k, a.k * 4u), rw = make_rsrc(a.wts + (uint64_t)t * a.k, a.k * 4u);
        e_slot = bld4(ri, 4u * min(j, a.k - 1u));
        my_e = bld4(ri, 4u * (tid & 63u));
        my_w = bld4(rw, 4u * (tid & 63u));
    }
    __builtin_amdgcn_sched_barrier(0);  // (keeps the row's loads after these)
    XRegs xr;
    moe_x_load(st, K2, xr, tid);
    const uint32_t r = min(b * a.nr2 + rl, a.hidden - 1u);
    const uint32_t row_bytes = a.ffn / T::QK * T::BB;
    const uint32_t upp = a.ffn / (T::QK / T::UPB);  // units per slot in the staged row
    uint32_t sh;
    const rsrc_t rs = moe_rsrc(a.wd, (uint64_t)a.E * a.eb_dn, &sh);
    const uint32_t e = min(e_slot, a.E - 1u);
    MoeRowDot<T, LPR> rd(rs, sh + (uint32_t)(e * a.eb_dn) + r * row_bytes, a.ffn, li);
    rd.fetch0();  // (items past the rows fetch a valid row; their dots are not used)
    if (tid < a.k) {
        le[tid] = (int32_t)min(my_e, a.E - 1u);
        lw[tid] = as_f32(my_w);
    }
    __syncthreads();
    if (tid < a.k) {
        const int32_t me = le[tid];
        uint32_t rank = 0;
        for (uint32_t i = 0; i < a.k; i++) rank += (le[i] < me || (le[i] == me && i < tid)) ? 1u : 0u;
        ord[rank] = tid;
    }
    uint32_t* lds_x = reinterpret_cast<uint32_t*>(lds + a.lds_x2);
    float* lds_s = reinterpret_cast<float*>(lds_x + K2 / 2u);
    float* lds_p = lds_s + K2 / 16u;
    float* v = lds_p + 4;  // [nr2][k] per-slot row values
    const float inv = gemv_stage_x(st, K2, T::XHI, xr, lds_x, lds_s, lds_p, tid);  // (its barriers order ord too)
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    float acc = 0.0f;
    if (rl < a.nr2) acc = rd.dot(j * upp, lds_x, lds_s, magic);
    acc = group_sum<LPR>(acc);
    if (li == 0u && rl < a.nr2) lds_st32(lds_addr(v + item), __builtin_bit_cast(uint32_t, acc * inv));
    lds_barrier();
    if (tid < a.nr2) {
        const uint32_t row = b * a.nr2 + tid;
        if (row < a.hidden) {
            float y = 0.0f;
            for (uint32_t q = 0; q < a.k; q++) {
                const uint32_t jj = ord[q];
                y = fmaf(lw[jj], __builtin_bit_cast(float, lds_ld32(lds_addr(v + tid * a.k + jj))), y);
            }
            a.out[(uint64_t)t * a.hidden + row] = y;
        }
    }
}

// one kernel per (weight type, lanes per row): LPR in {4, 8, 16, 32}
#define RFXQ_MOE_DEC(TY, T, LPR)                                                                          \
    extern "C" __global__ __launch_bounds__(256) void rfxq_moe_dec_gu_##TY##_##LPR(MoeDecArgs a) {         \
        extern __shared__ __attribute__((aligned(16))) uint8_t moe_dec_lds[];                             \
        moe_dec_gu<T, LPR>(a, moe_dec_lds);                                                               \
    }                                                                                                     \
    extern "C" __global__ __launch_bounds__(256) void rfxq_moe_dec_down_##TY##_##LPR(MoeDecArgs a) {       \
        extern __shared__ __attribute__((aligned(16))) uint8_t moe_dec_lds[];                             \
        moe_dec_down<T, LPR>(a, moe_dec_lds);                                                             \
    }
RFXQ_MOE_DEC(q4k, Q4K, 4)
RFXQ_MOE_DEC(q4k, Q4K, 8)
RFXQ_MOE_DEC(q4k, Q4K, 16)
RFXQ_MOE_DEC(q4k, Q4K, 32)
RFXQ_MOE_DEC(q6k, Q6K, 4)
RFXQ_MOE_DEC(q6k, Q6K, 8)
RFXQ_MOE_DEC(q6k, Q6K, 16)
RFXQ_MOE_DEC(q6k, Q6K, 32)
RFXQ_MOE_DEC(q8_0, Q80, 4)
RFXQ_MOE_DEC(q8_0, Q80, 8)
RFXQ_MOE_DEC(q8_0, Q80, 16)
RFXQ_MOE_DEC(q8_0, Q80, 32)

// rfxq_moe_route's work with one wave per token (at most kDecRouteMaxE
// experts, k <= 64; x rows of up to kActRegK values): the token's logits and
// its row of x are requested together, the wave routes the token
// (moe_route_wave, every pick and weight written: the same probabilities,
// picks and weights as rfxq_moe_route) and, with xh, writes the row's f16
// layout (act_f16_row's arithmetic). No barrier: waves past the last token
// return at once.
extern "C" __global__ __launch_bounds__(256) void rfxq_moe_route_w(const float* __restrict__ logits, uint32_t tokens,
                                                                  uint32_t E, uint32_t k, uint32_t normalize,
                                                                  float scale, int32_t* __restrict__ idx,
                                                                  float* __restrict__ wts, const float* __restrict__ x,
                                                                  uint32_t hidden, uint16_t* __restrict__ xh,
                                                                  uint16_t* __restrict__ xsx, float* __restrict__ xrs) {
    const uint32_t t = __builtin_amdgcn_readfirstlane(blockIdx.x * 4u + (threadIdx.x >> 6));
    if (t >= tokens) return;
    RouteLogits lg;
    moe_route_load(logits, t, E, lg);
    float4 v[kActRowRegs];
    const QuantSrcPlain src{x, hidden, nullptr};
    if (xh) act_f16_row_load(src, t, hidden, v);
    (void)moe_route_wave(lg, t, E, k, normalize, scale, idx, wts, 0u, true);
    if (xh) act_f16_row_put(v, t, hidden, xh, xsx, xrs, nullptr);
}
