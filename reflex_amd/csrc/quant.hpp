// Activation quantization to int8 per 32 elements with an f16 scale and sum
// (the Q8_1 block of src/dequant.rs:228-240: d, s, qs[32]), using ggml's
// published quantize_row_q8_1_ref rounding: d = amax / 127, id = d ? 1/d : 0,
// q = roundf(x * id). The sum field holds the block's exact activation sum in
// units of d, s = f16(sum(x) * id) (|s| <= 32*127, so it cannot overflow f16),
// rather than ggml's d*sum(q): the MMQ epilogue multiplies d*s by each weight
// block's constant part, which removes that part's quantization error (about
// half of the total for Q4_K). sum(x) is taken in f32 in a fixed order: lane
// partials ((x0+x1)+x2)+x3 over 8 lanes, then a butterfly over lane distance
// 4, 2, 1. The reference has no activation
// quantizer (its prefill casts to f16, src/kernels_cuda/convert.cu:91); this
// is the input stage of the int8 MMQ GEMM.
//
// Layout for the GEMM: xq [rows][k] int8 (row stride ldq bytes) and xds
// [rows][k/32] u32 = d_bits | s_bits << 16. Optional `src_rows` gathers
// x rows (x row src_rows[r] -> output row r).
#pragma once
#include "common.hpp"

// Sources of the values to quantize: a lane loads four consecutive values
// of a row (row r, elements [c, c + 4)).
struct QuantSrcPlain {  // x[src_rows[r] or r][c], row stride ldx
    const float* x;
    uint32_t ldx;
    const int32_t* src_rows;
    __device__ __forceinline__ float4 load(uint32_t r, uint32_t c) const {
        const uint32_t sr = src_rows ? (uint32_t)src_rows[r] : r;
        return *reinterpret_cast<const float4*>(x + (uint64_t)sr * ldx + c);
    }
};

// Rows [0, rows) of one activation, spread over `nwaves` waves (this one is
// wave_global); 8 lanes per 32-block. `yout` (optional) receives the values
// quantized, f32 [rows][k] (the producer's own output).
template <class Src>
RFXQ_DEV void quant_q8_1_rows(const Src& src, uint32_t rows, uint32_t k, int8_t* __restrict__ xq, uint32_t ldq,
                              uint32_t* __restrict__ xds, float* __restrict__ yout, uint64_t wave_global,
                              uint64_t nwaves) {
    const uint32_t nblk = k / 32u;
    const uint64_t total = (uint64_t)rows * nblk;
    const uint32_t lane = threadIdx.x & 63u;
    for (uint64_t b0 = wave_global * 8u; b0 < total; b0 += nwaves * 8u) {
        const uint64_t bi = b0 + (lane >> 3);
        const bool valid = bi < total;
        const uint64_t bb = valid ? bi : total - 1u;
        const uint32_t row = (uint32_t)(bb / nblk), blk = (uint32_t)(bb % nblk);
        const uint32_t part = lane & 7u;
        const float4 v = src.load(row, 32u * blk + 4u * part);
        if (yout && valid) *reinterpret_cast<float4*>(yout + (uint64_t)row * k + 32u * blk + 4u * part) = v;
        float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        // the block's maximum in all 8 lanes (DPP within the lane group)
        amax = fmaxf(amax, RFXQ_DPP(amax, 0xB1));
        amax = fmaxf(amax, RFXQ_DPP(amax, 0x4E));
        amax = fmaxf(amax, RFXQ_DPP(amax, 0x141));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const int q0 = (int)roundf(v.x * id), q1 = (int)roundf(v.y * id);
        const int q2 = (int)roundf(v.z * id), q3 = (int)roundf(v.w * id);
        float sum = ((v.x + v.y) + v.z) + v.w;
        // lane distance 4, 2, 1 for the group's first lane (the one that
        // stores it): row_shl:4, then quad_perm swaps of 2 and 1
        sum += RFXQ_DPP(sum, 0x104);
        sum += RFXQ_DPP(sum, 0x4E);
        sum += RFXQ_DPP(sum, 0xB1);
        if (valid) {
            const uint32_t packed = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) |
                                    ((uint32_t)(q2 & 0xFF) << 16) | ((uint32_t)(q3 & 0xFF) << 24);
            *reinterpret_cast<uint32_t*>(xq + (uint64_t)row * ldq + 32u * blk + 4u * part) = packed;
            if (part == 0u) {
                const uint32_t dbits = __builtin_bit_cast(uint16_t, (half_t)d);
                // round the product to f32 first (no fused single-rounding mixed mad)
                float sid = sum * id;
                asm volatile("" : "+v"(sid));
                const uint32_t sbits = __builtin_bit_cast(uint16_t, (half_t)sid);
                xds[(uint64_t)row * nblk + blk] = dbits | (sbits << 16);
            }
        }
    }
}

// ---------------------------------------------------------------- f16 activations
//
// The input stage of the f16-activation prefill kernels (mmqh.hpp): one wave
// per row. It finds max |x| of the row; e = ilogb(max) - 8 (clamped to
// [-120, 120]; 0 for an all-zero or non-finite maximum) so that the scaled
// row's largest value lies in [256, 512), then writes
//   xh  [rows][k] f16 = RNE(x * 2^-e), groups of four stored (x0, x2), (x1, x3)
//   xsx [rows][k/256][16] f16: per 32-block b of the super-block, the sum of
//       the block's 32 f16 values (f32: lane partials ((h0+h1)+h2)+h3 over 8
//       lanes, then a butterfly over lane distance 1, 2, 4) as hi[b] = f16(S),
//       lo[b] = f16(S - hi)
//   xrs [rows] f32 = 2^e
// and, optionally, the source values themselves to yout (f32 [rows][k]).
// row exponent of the f16 layout from the row's max |x|
RFXQ_DEV int act_f16_exp(float mx) {
    mx = wave_max(mx);
    return (mx > 0.0f && mx <= 3.4028235e38f) ? min(max(ilogbf(mx) - 8, -120), 120) : 0;
}

RFXQ_DEV float absmax4(float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); }

// the f16 layout of one row's four values at column c (lane's chunk)
RFXQ_DEV void act_f16_chunk(float4 v, uint32_t lane, uint32_t c, uint64_t ro, uint32_t r, uint32_t nsb, float scale,
                            uint16_t* __restrict__ xh, uint16_t* __restrict__ xsx, float* __restrict__ yout) {
    if (yout) *reinterpret_cast<float4*>(yout + ro + c) = v;
    const half_t h0 = (half_t)(v.x * scale), h1 = (half_t)(v.y * scale);
    const half_t h2 = (half_t)(v.z * scale), h3 = (half_t)(v.w * scale);
    uint2 hv;
    hv.x = h2_bits(h2_t{h0, h2});
    hv.y = h2_bits(h2_t{h1, h3});
    *reinterpret_cast<uint2*>(xh + ro + c) = hv;
    float s = (((float)h0 + (float)h1) + (float)h2) + (float)h3;
    // lane distance 1, 2 (quad_perm swaps), then the other quad's sum by
    // row_half_mirror: the same additions as a butterfly for the group's
    // first lane, which stores it (every lane of a quad holds the same sum)
    s = group_sum<8>(s);
    if ((lane & 7u) == 0u) {
        const uint32_t blk = c / 32u;
        const half_t hi = (half_t)s;
        const half_t lo = (half_t)(s - (float)hi);
        uint16_t* rec = xsx + ((uint64_t)r * nsb + blk / 8u) * 16u;
        rec[blk & 7u] = __builtin_bit_cast(uint16_t, hi);
        rec[8u + (blk & 7u)] = __builtin_bit_cast(uint16_t, lo);
    }
}

// Rows of up to kActRegK values are read once, into registers; longer rows
// are read twice (the maximum, then the layout).
constexpr uint32_t kActRegK = 4096;

// act_f16_row's register form (k <= kActRegK) in two steps, so a caller can
// put the row's loads in flight beside other loads
constexpr uint32_t kActRowRegs = kActRegK / 256u;
template <class Src>
RFXQ_DEV void act_f16_row_load(const Src& src, uint32_t r, uint32_t k, float4 (&v)[kActRowRegs]) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t nsb = k / 256u;
#pragma unroll
    for (uint32_t i = 0; i < kActRowRegs; i++)
        if (i < nsb) v[i] = src.load(r, 4u * lane + 256u * i);
}

RFXQ_DEV void act_f16_row_put(const float4 (&v)[kActRowRegs], uint32_t r, uint32_t k, uint16_t* __restrict__ xh,
                              uint16_t* __restrict__ xsx, float* __restrict__ xrs, float* __restrict__ yout) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t ro = (uint64_t)r * k;
    const uint32_t nsb = k / 256u;
    float mx = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < kActRowRegs; i++)
        if (i < nsb) mx = fmaxf(mx, absmax4(v[i]));
    const int e = act_f16_exp(mx);
    const float scale = ldexpf(1.0f, -e);
#pragma unroll
    for (uint32_t i = 0; i < kActRowRegs; i++)
        if (i < nsb) act_f16_chunk(v[i], lane, 4u * lane + 256u * i, ro, r, nsb, scale, xh, xsx, yout);
    if (lane == 0u) xrs[r] = ldexpf(1.0f, e);
}

template <class Src>
RFXQ_DEV void act_f16_row(const Src& src, uint32_t r, uint32_t k, uint16_t* __restrict__ xh,
                          uint16_t* __restrict__ xsx, float* __restrict__ xrs, float* __restrict__ yout) {
    if (k <= kActRegK) {
        float4 v[kActRowRegs];
        act_f16_row_load(src, r, k, v);
        act_f16_row_put(v, r, k, xh, xsx, xrs, yout);
        return;
    }
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t ro = (uint64_t)r * k;
    const uint32_t nsb = k / 256u;
    float mx = 0.0f;
    for (uint32_t c = 4u * lane; c < k; c += 256u) mx = fmaxf(mx, absmax4(src.load(r, c)));
    const int e = act_f16_exp(mx);
    const float scale = ldexpf(1.0f, -e);
    for (uint32_t c = 4u * lane; c < k; c += 256u) act_f16_chunk(src.load(r, c), lane, c, ro, r, nsb, scale, xh, xsx, yout);
    if (lane == 0u) xrs[r] = ldexpf(1.0f, e);
}

// One row by the whole 256-thread workgroup: thread t takes the four values
// at 4t + 1024i, held in registers up to 16384 values (longer rows are read
// twice); the row maximum
// combines the four waves through LDS. Same layouts and arithmetic as
// act_f16_row (the block sums are formed by the same 8 lanes in the same
// order), so the result does not depend on which form wrote it.
template <class Src>
RFXQ_DEV void act_f16_row_wg(const Src& src, uint32_t r, uint32_t k, uint16_t* __restrict__ xh,
                             uint16_t* __restrict__ xsx, float* __restrict__ xrs, float* __restrict__ yout) {
    __shared__ float wmax[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint64_t ro = (uint64_t)r * k;
    const uint32_t nsb = k / 256u;
    constexpr uint32_t NC = 16;  // rows up to 16384 values stay in registers
    float4 v[NC];
    float mx = 0.0f;
    const bool reg = k <= NC * 1024u;
    if (reg) {
#pragma unroll
        for (uint32_t i = 0; i < NC; i++) {
            const uint32_t c = 4u * tid + 1024u * i;
            if (c < k) v[i] = src.load(r, c);
        }
#pragma unroll
        for (uint32_t i = 0; i < NC; i++)
            if (4u * tid + 1024u * i < k) mx = fmaxf(mx, absmax4(v[i]));
    } else {
        for (uint32_t c = 4u * tid; c < k; c += 1024u) mx = fmaxf(mx, absmax4(src.load(r, c)));
    }
    mx = wave_max(mx);
    if (lane == 0u) wmax[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    __syncthreads();  // wmax is reused by the next row
    const int e = act_f16_exp(mx);
    const float scale = ldexpf(1.0f, -e);
    if (reg) {
#pragma unroll
        for (uint32_t i = 0; i < NC; i++) {
            const uint32_t c = 4u * tid + 1024u * i;
            if (c < k) act_f16_chunk(v[i], lane, c, ro, r, nsb, scale, xh, xsx, yout);
        }
    } else {
        for (uint32_t c = 4u * tid; c < k; c += 1024u) act_f16_chunk(src.load(r, c), lane, c, ro, r, nsb, scale, xh, xsx, yout);
    }
    if (tid == 0u) xrs[r] = ldexpf(1.0f, e);
}

// Rows per workgroup of the f16 activation kernels: a row per wave (4 per
// workgroup) for many short rows, a whole workgroup per row otherwise (few
// rows, or rows too long for one wave's registers). The host sizes grids by
// the same rule.
RFXQ_DEV bool act_wave_rows(uint32_t rows, uint32_t k) { return k <= kActRegK && rows >= 128u; }

template <class Src>
RFXQ_DEV void act_f16_rows(const Src& src, uint32_t rows, uint32_t k, uint32_t b, uint32_t nb,
                           uint16_t* __restrict__ xh, uint16_t* __restrict__ xsx, float* __restrict__ xrs,
                           float* __restrict__ yout) {
    if (act_wave_rows(rows, k)) {
        for (uint32_t r = b * 4u + (threadIdx.x >> 6); r < rows; r += nb * 4u)
            act_f16_row(src, r, k, xh, xsx, xrs, yout);
    } else {
        for (uint32_t r = b; r < rows; r += nb) act_f16_row_wg(src, r, k, xh, xsx, xrs, yout);
    }
}

extern "C" __global__ __launch_bounds__(256) void rfxq_act_f16(const float* __restrict__ x, uint32_t ldx,
                                                              const int32_t* __restrict__ src_rows, uint32_t rows,
                                                              uint32_t k, uint16_t* __restrict__ xh,
                                                              uint16_t* __restrict__ xsx, float* __restrict__ xrs) {
    const QuantSrcPlain src{x, ldx, src_rows};
    for (uint32_t r = blockIdx.x * 4u + (threadIdx.x >> 6); r < rows; r += gridDim.x * 4u)
        act_f16_row(src, r, k, xh, xsx, xrs, nullptr);
}

// the same with a row per workgroup (few or long rows; a kernel of its own:
// its registers would otherwise limit the row-per-wave kernel's occupancy)
extern "C" __global__ __launch_bounds__(256) void rfxq_act_f16_wg(const float* __restrict__ x, uint32_t ldx,
                                                                 const int32_t* __restrict__ src_rows, uint32_t rows,
                                                                 uint32_t k, uint16_t* __restrict__ xh,
                                                                 uint16_t* __restrict__ xsx, float* __restrict__ xrs) {
    const QuantSrcPlain src{x, ldx, src_rows};
    for (uint32_t r = blockIdx.x; r < rows; r += gridDim.x) act_f16_row_wg(src, r, k, xh, xsx, xrs, nullptr);
}

// Several activations in one launch (grouped GEMMs): workgroups
// [wg_begin, wg_begin + wgs) of the grid take activation i.
struct ActF16Desc {
    const float* x;
    uint16_t* xh;
    uint16_t* xsx;
    float* xrs;
    uint32_t rows, k, wg_begin, wgs;
};

RFXQ_DEV const ActF16Desc& act_f16_pick(const ActF16Desc* __restrict__ table, uint32_t ndesc) {
    uint32_t lo = 0, hi = ndesc - 1u;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1u) >> 1;
        if (table[mid].wg_begin <= blockIdx.x) lo = mid;
        else hi = mid - 1u;
    }
    return table[lo];
}

extern "C" __global__ __launch_bounds__(256) void rfxq_act_f16_multi(const ActF16Desc* __restrict__ table,
                                                                    uint32_t ndesc) {
    const ActF16Desc d = act_f16_pick(table, ndesc);
    const QuantSrcPlain src{d.x, d.k, nullptr};
    for (uint32_t r = (blockIdx.x - d.wg_begin) * 4u + (threadIdx.x >> 6); r < d.rows; r += d.wgs * 4u)
        act_f16_row(src, r, d.k, d.xh, d.xsx, d.xrs, nullptr);
}

extern "C" __global__ __launch_bounds__(256) void rfxq_act_f16_multi_wg(const ActF16Desc* __restrict__ table,
                                                                       uint32_t ndesc) {
    const ActF16Desc d = act_f16_pick(table, ndesc);
    const QuantSrcPlain src{d.x, d.k, nullptr};
    for (uint32_t r = blockIdx.x - d.wg_begin; r < d.rows; r += d.wgs) act_f16_row_wg(src, r, d.k, d.xh, d.xsx, d.xrs, nullptr);
}

extern "C" __global__ __launch_bounds__(256) void rfxq_quantize_q8_1(const float* __restrict__ x, uint32_t ldx,
                                                                    const int32_t* __restrict__ src_rows,
                                                                    uint32_t rows, uint32_t k,
                                                                    int8_t* __restrict__ xq, uint32_t ldq,
                                                                    uint32_t* __restrict__ xds) {
    quant_q8_1_rows(QuantSrcPlain{x, ldx, src_rows}, rows, k, xq, ldq, xds, nullptr,
                    ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6, ((uint64_t)gridDim.x * blockDim.x) >> 6);
}

// Several activations in one launch (grouped GEMMs): workgroups
// [wg_begin, wg_begin + wgs) of the grid take activation i.
struct QuantDesc {
    const float* x;
    int8_t* xq;
    uint32_t* xds;
    uint32_t rows, k, wg_begin, wgs;
};

extern "C" __global__ __launch_bounds__(256) void rfxq_quantize_q8_1_multi(const QuantDesc* __restrict__ table,
                                                                          uint32_t ndesc) {
    uint32_t lo = 0, hi = ndesc - 1u;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1u) >> 1;
        if (table[mid].wg_begin <= blockIdx.x) lo = mid;
        else hi = mid - 1u;
    }
    const QuantDesc d = table[lo];
    const uint32_t wg = blockIdx.x - d.wg_begin;
    quant_q8_1_rows(QuantSrcPlain{d.x, d.k, nullptr}, d.rows, d.k, d.xq, d.k, d.xds, nullptr,
                    ((uint64_t)wg * blockDim.x + threadIdx.x) >> 6, ((uint64_t)d.wgs * blockDim.x) >> 6);
}

// ---------------------------------------------------------------- fused producers
//
// The activation producers of the prefill GEMMs write the quantized layouts
// directly (and, optionally, their own f32 output), so the activation is not
// written in f32 and read back by a separate quantize launch.

// RMSNorm (src/kernels_cuda/rmsnorm.cu:18-55 with rmsnorm.cuh:17-41):
// y = (x * r) * g, r = 1 / sqrtf(sum_sq / k + eps), sum_sq accumulated by one
// thread per row in index order as fused multiply-adds (the reference's
// order and contraction, so y is bit-identical to its output).
constexpr uint32_t kNormRowsPerWg = 4;

struct QuantSrcRms {
    const float* x;
    const float* g;
    const float* rinv;  // per row of the workgroup (LDS)
    uint32_t k;
    __device__ __forceinline__ float4 load(uint32_t r, uint32_t c) const {
        const float4 v = *reinterpret_cast<const float4*>(x + (uint64_t)r * k + c);
        const float4 w = *reinterpret_cast<const float4*>(g + c);
        const float s = rinv[r];
        return make_float4((v.x * s) * w.x, (v.y * s) * w.y, (v.z * s) * w.z, (v.w * s) * w.w);
    }
};

extern "C" __global__ __launch_bounds__(256) void rfxq_rmsnorm_q8_1(const float* __restrict__ x,
                                                                   const float* __restrict__ g, uint32_t rows,
                                                                   uint32_t k, float eps, int8_t* __restrict__ xq,
                                                                   uint32_t* __restrict__ xds,
                                                                   uint16_t* __restrict__ xh,
                                                                   uint16_t* __restrict__ xsx,
                                                                   float* __restrict__ xrs,
                                                                   float* __restrict__ y) {
    // The rows pass through LDS in chunks of kNormChunk floats, double
    // buffered: waves 1-3 copy chunk c + 1 (coalesced) while lanes 0..nr-1
    // of wave 0 run the chain of fused multiply-adds over chunk c from LDS
    // (one lane per row; the order is fixed, so the chain is the bound).
    constexpr uint32_t kNormChunk = 1024;
    constexpr uint32_t kRowF4 = kNormChunk / 4u + 1u;  // +1 float4: rows start on different banks
    __shared__ float4 stage[2][kNormRowsPerWg * kRowF4];
    __shared__ float rinv[kNormRowsPerWg];
    const uint32_t r0 = blockIdx.x * kNormRowsPerWg;
    const uint32_t nr = min(kNormRowsPerWg, rows - r0);
    const uint32_t tid = threadIdx.x, nchunks = (k + kNormChunk - 1u) / kNormChunk;
    auto copy = [&](uint32_t c, uint32_t t0, uint32_t nt) {
        const uint32_t c0 = c * kNormChunk, len4 = min(kNormChunk, k - c0) / 4u;  // k is a multiple of 256
        for (uint32_t i = t0; i < nr * len4; i += nt) {
            const uint32_t r = i / len4, j = i - r * len4;
            stage[c & 1u][r * kRowF4 + j] = *reinterpret_cast<const float4*>(x + (uint64_t)(r0 + r) * k + c0 + 4u * j);
        }
    };
    copy(0, tid, 256u);
    __syncthreads();
    float sum_sq = 0.0f;
    for (uint32_t c = 0; c < nchunks; c++) {
        if (tid >= 64u) {
            if (c + 1u < nchunks) copy(c + 1u, tid - 64u, 192u);
        } else if (tid < nr) {
            const float4* sr = &stage[c & 1u][tid * kRowF4];
            const uint32_t len4 = min(kNormChunk, k - c * kNormChunk) / 4u;
#pragma unroll 8
            for (uint32_t j = 0; j < len4; j++) {
                const float4 v = sr[j];
                sum_sq = __builtin_fmaf(v.x, v.x, sum_sq);
                sum_sq = __builtin_fmaf(v.y, v.y, sum_sq);
                sum_sq = __builtin_fmaf(v.z, v.z, sum_sq);
                sum_sq = __builtin_fmaf(v.w, v.w, sum_sq);
            }
        }
        __syncthreads();
    }
    if (tid < nr) rinv[tid] = 1.0f / sqrtf(sum_sq / (float)k + eps);
    __syncthreads();
    const uint64_t o = (uint64_t)r0 * k, nblk = k / 32u;
    const QuantSrcRms src{x + o, g, rinv, k};
    // int8 layout (8 lanes per 32-block), then the f16 layout (one wave per
    // row); the producer's own output y is written by the first pass run
    if (xq) quant_q8_1_rows(src, nr, k, xq + o, k, xds + r0 * nblk, y ? y + o : nullptr, threadIdx.x >> 6, 4u);
    const uint32_t wv = threadIdx.x >> 6;
    if (xh && wv < nr)
        act_f16_row(src, wv, k, xh + o, xsx + r0 * (nblk / 8u) * 16u, xrs + r0, (!xq && y) ? y + o : nullptr);
}

// SiLU(gate) * up (src/kernels_cuda/silu_and_mul.cu:7-23: g / (1 + expf(-g)) * u)
struct QuantSrcSilu {
    const float* gate;
    const float* up;
    uint32_t k;
    __device__ __forceinline__ float4 load(uint32_t r, uint32_t c) const {
        const uint64_t i = (uint64_t)r * k + c;
        const float4 g = *reinterpret_cast<const float4*>(gate + i);
        const float4 u = *reinterpret_cast<const float4*>(up + i);
        return make_float4((g.x / (1.0f + expf(-g.x))) * u.x, (g.y / (1.0f + expf(-g.y))) * u.y,
                           (g.z / (1.0f + expf(-g.z))) * u.z, (g.w / (1.0f + expf(-g.w))) * u.w);
    }
};

extern "C" __global__ __launch_bounds__(256) void rfxq_silu_and_mul_q8_1(const float* __restrict__ gate,
                                                                        const float* __restrict__ up,
                                                                        uint32_t rows, uint32_t k,
                                                                        int8_t* __restrict__ xq,
                                                                        uint32_t* __restrict__ xds,
                                                                        uint16_t* __restrict__ xh,
                                                                        uint16_t* __restrict__ xsx,
                                                                        float* __restrict__ xrs,
                                                                        float* __restrict__ y) {
    const QuantSrcSilu src{gate, up, k};
    if (xq)
        quant_q8_1_rows(src, rows, k, xq, k, xds, y, ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6,
                        ((uint64_t)gridDim.x * blockDim.x) >> 6);
    if (xh) act_f16_rows(src, rows, k, blockIdx.x, gridDim.x, xh, xsx, xrs, xq ? nullptr : y);
}
