// Decode GEMV y[N] = W[N,K] . x[K] straight from Q4_K / Q6_K / Q8_0 blocks.
//
// Replaces `gemv_q4k_r1_kernel`, `gemv_q6k_r1_kernel`, `gemv_q6k_kernel`
// (src/kernels_cuda/gemv_q4k.cu:170-337,461-509) and `gemv_q8_0_direct_kernel`
// (src/kernels_cuda/gemv_q8_0.cu:193-230), and the fused multi-projection
// launch of `Model::gemv_qkv_to` (src/model/kernels.rs:1761): one launch runs a
// table of independent GEMVs (descriptors), each with its own weight, x and y.
//
// Design (wave64, gfx950):
//  * Each 256-thread workgroup owns a contiguous tile of output rows of one
//    descriptor. Its prologue converts x once into LDS as f16, pair-permuted
//    (see pair_perm) and, for Q4_K, with the high-nibble runs pre-scaled by
//    1/16, plus per-16 sums of those f16 values.
//  * Weights stream with 16-byte loads. A packed byte word is turned into two
//    f16 values by masking a nibble (or byte) into the mantissa of 1024.0
//    (0x6400 | q == 1024 + q), and contracted with v_dot2_f32_f16 against the
//    matching x pair. The 1024 offset (and Q6_K's -32, Q8_0's +128 bias) is
//    removed per run with the run's x sum, so per weight the inner loop costs
//    about one VALU op instead of a convert plus an FMA.
//  * A row is covered by LPR lanes (a power of two); each lane owns U "units"
//    of 64 weights (Q4_K/Q6_K: a quarter super-block; Q8_0: one 32-block), and
//    the LPR partial sums are combined with a lane-group reduction.
//
// Numerics: weights take the exact dequantized values (d*sc*q - dmin*m as two
// f32 products), activations are rounded to f16 (relative 2^-11), products
// accumulate in f32. The result is within 1e-4 (relative to the output row's
// L2 norm) of the f64 host reference; it is not bit-identical to the
// reference's f32 kernel, which accumulates in a different order anyway.
#pragma once
#include "common.hpp"

struct GemvDesc {
    const uint8_t* w;  // raw blocks, row-major [n][k / QK]
    const float* x;    // [k] f32
    float* y;          // [n] f32
    uint32_t k, n, type, lpr_log2;
    uint32_t rows_per_wg, wg_begin, pad0, pad1;
};

#define GEMV_INLINE 4
struct GemvArgs {
    const GemvDesc* table;  // device table when ndesc > GEMV_INLINE
    uint32_t ndesc, pad;
    GemvDesc inl[GEMV_INLINE];
};

// ---------------------------------------------------------------- prologue

// x -> LDS f16 (pair-permuted; Q4_K high-nibble runs scaled by 1/16) and the
// per-16 sums of the stored f16 values (computed with the same dot2 op).
RFXQ_DEV void gemv_stage_x(const float* __restrict__ x, uint32_t k, bool prescale_hi, uint32_t* lds_x,
                           float* lds_s) {
    const uint32_t tid = threadIdx.x;
    for (uint32_t e = 4u * tid; e < k; e += 1024u) {
        const float4 v = *reinterpret_cast<const float4*>(x + e);
        const float sc = (prescale_hi && (e & 32u)) ? 0.0625f : 1.0f;
        const h2_t a = {(half_t)(v.x * sc), (half_t)(v.z * sc)};
        const h2_t b = {(half_t)(v.y * sc), (half_t)(v.w * sc)};
        uint2 st;
        st.x = h2_bits(a);
        st.y = h2_bits(b);
        *reinterpret_cast<uint2*>(lds_x + e / 2u) = st;
    }
    __syncthreads();
    const uint32_t ng = k / 16u;
    for (uint32_t g = tid; g < ng; g += 256u) {
        const uint4 p0 = *reinterpret_cast<const uint4*>(lds_x + 8u * g);
        const uint4 p1 = *reinterpret_cast<const uint4*>(lds_x + 8u * g + 4u);
        const uint32_t one2 = 0x3C003C00u;
        float s = 0.0f;
        s = dot2(p0.x, one2, s);
        s = dot2(p0.y, one2, s);
        s = dot2(p0.z, one2, s);
        s = dot2(p0.w, one2, s);
        s = dot2(p1.x, one2, s);
        s = dot2(p1.y, one2, s);
        s = dot2(p1.z, one2, s);
        s = dot2(p1.w, one2, s);
        lds_s[g] = s;
    }
    __syncthreads();
}

// ---------------------------------------------------------------- Q4_K unit

// 64 weights: qs bytes [32g, 32g+32) of one super-block = sub-blocks 2g (low
// nibbles) and 2g+1 (high nibbles). xl/xh: 16 dwords each of pair-permuted x.
struct XQ4 {
    uint4 l[4], h[4];
};

RFXQ_DEV void load_x_q4k(const uint32_t* lds_x, uint32_t xoff, XQ4& x) {
    const uint4* p = reinterpret_cast<const uint4*>(lds_x + xoff / 2u);
#pragma unroll
    for (int i = 0; i < 4; i++) x.l[i] = p[i];
#pragma unroll
    for (int i = 0; i < 4; i++) x.h[i] = p[4 + i];
}

RFXQ_DEV uint32_t u4_at(const uint4* a, int j) {
    const uint4 v = a[j >> 2];
    return (j & 3) == 0 ? v.x : (j & 3) == 1 ? v.y : (j & 3) == 2 ? v.z : v.w;
}

RFXQ_DEV float q4k_unit(const u4_t hdr, const u4_t qa, const u4_t qb, uint32_t g, const XQ4& x, const float* s) {
    const uint32_t sh = (g & 1u) * 16u;
    const uint32_t a = hdr.y >> sh, b = hdr.z >> sh, c = hdr.w >> sh;
    uint32_t sc1, sc2, m1, m2;
    if (g < 2u) {
        sc1 = a & 63u;
        sc2 = (a >> 8) & 63u;
        m1 = b & 63u;
        m2 = (b >> 8) & 63u;
    } else {
        sc1 = (c & 0xFu) | ((a >> 2) & 0x30u);
        sc2 = ((c >> 8) & 0xFu) | ((a >> 10) & 0x30u);
        m1 = ((c >> 4) & 0xFu) | ((b >> 2) & 0x30u);
        m2 = ((c >> 12) & 0xFu) | ((b >> 10) & 0x30u);
    }
    const float d = f16_bits_to_f32(hdr.x);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    const float d1 = d * (float)sc1, d2 = d * (float)sc2;
    const float mm1 = dmin * (float)m1, mm2 = dmin * (float)m2;

    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    float rl0 = 0.f, rl1 = 0.f, rh0 = 0.f, rh1 = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t v = q[j], v8 = v >> 8;
        rl0 = dot2((v & 0x000F000Fu) | 0x64006400u, u4_at(x.l, 2 * j), rl0);
        rl1 = dot2((v8 & 0x000F000Fu) | 0x64006400u, u4_at(x.l, 2 * j + 1), rl1);
        rh0 = dot2((v & 0x00F000F0u) | 0x64006400u, u4_at(x.h, 2 * j), rh0);
        rh1 = dot2((v8 & 0x00F000F0u) | 0x64006400u, u4_at(x.h, 2 * j + 1), rh1);
    }
    const float slo = s[0] + s[1], shi = s[2] + s[3];
    const float lo = d1 * (rl0 + rl1) - (1024.0f * d1 + mm1) * slo;
    const float hi = d2 * (rh0 + rh1) - (1024.0f * d2 + 16.0f * mm2) * shi;
    return lo + hi;
}

// ---------------------------------------------------------------- Q6_K unit

// 16 bytes at byte offset o of a 2-byte-aligned block base p (pa = p & ~3,
// sh = p & 3), read as dwords from the dword-aligned base and realigned.
// Never reads past o + 20 from p's dword-aligned base, i.e. stays inside the
// block for o <= 176.
RFXQ_DEV u4_t seg16(const uint8_t* pa, uint32_t o, uint32_t sh) {
    const u4_t v = ld16_a4(pa + o);
    const uint32_t e = *reinterpret_cast<const uint32_t*>(pa + o + 16);
    u4_t r;
    r.x = alignbyte(v.y, v.x, sh);
    r.y = alignbyte(v.z, v.y, sh);
    r.z = alignbyte(v.w, v.z, sh);
    r.w = alignbyte(e, v.w, sh);
    return r;
}

struct XQ6 {
    uint4 r[4][2];  // 4 runs of 16 elements: 8 dwords each
};

RFXQ_DEV void load_x_q6k(const uint32_t* lds_x, uint32_t xoff, XQ6& x) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint4* p = reinterpret_cast<const uint4*>(lds_x + (xoff + 32u * t) / 2u);
        x.r[t][0] = p[0];
        x.r[t][1] = p[1];
    }
}

// 64 weights of one super-block: half n = g >> 1, positions l in [16*(g&1), +16)
// of its four 32-runs (src/dequant.rs:414-444 layout).
RFXQ_DEV float q6k_unit(const uint8_t* blk, uint32_t g, const XQ6& x, const float* s) {
    const uint32_t n = g >> 1, hs = g & 1u;
    const uintptr_t addr = reinterpret_cast<uintptr_t>(blk);
    const uint8_t* pa = reinterpret_cast<const uint8_t*>(addr & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(addr & 3u);
    const u4_t a = seg16(pa, 64u * n + 16u * hs, sh);
    const u4_t c = seg16(pa, 64u * n + 32u + 16u * hs, sh);
    const u4_t h = seg16(pa, 128u + 32u * n + 16u * hs, sh);
    // scales (bytes 192..207) and d (208..209) without reading past byte 209
    const u4_t sw = ld16_a4(pa + 192);
    uint32_t tail;
    if (sh) tail = *reinterpret_cast<const uint32_t*>(pa + 208);
    else tail = *reinterpret_cast<const uint16_t*>(blk + 208);
    const uint32_t s0 = alignbyte(sw.y, sw.x, sh), s1 = alignbyte(sw.z, sw.y, sh);
    const uint32_t s2 = alignbyte(sw.w, sw.z, sh), s3 = alignbyte(tail, sw.w, sh);
    const float d = f16_bits_to_f32(sh ? (tail >> 16) : tail);
    const uint32_t W0 = n ? s2 : s0, W1 = n ? s3 : s1;
    const int sc0 = (int)(int8_t)(W0 >> (8u * hs));
    const int sc1 = (int)(int8_t)(W0 >> (8u * hs + 16u));
    const int sc2 = (int)(int8_t)(W1 >> (8u * hs));
    const int sc3 = (int)(int8_t)(W1 >> (8u * hs + 16u));

    const uint32_t A[4] = {a.x, a.y, a.z, a.w}, C[4] = {c.x, c.y, c.z, c.w}, H[4] = {h.x, h.y, h.z, h.w};
    float r0 = 0.f, r1 = 0.f, r2 = 0.f, r3 = 0.f;
    const uint32_t M4 = 0x000F000Fu, M2 = 0x00300030u, MG = 0x64006400u;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t av = A[j], cv = C[j], hv = H[j];
        const uint32_t xe0 = u4_at(x.r[0], 2 * j), xo0 = u4_at(x.r[0], 2 * j + 1);
        const uint32_t xe1 = u4_at(x.r[1], 2 * j), xo1 = u4_at(x.r[1], 2 * j + 1);
        const uint32_t xe2 = u4_at(x.r[2], 2 * j), xo2 = u4_at(x.r[2], 2 * j + 1);
        const uint32_t xe3 = u4_at(x.r[3], 2 * j), xo3 = u4_at(x.r[3], 2 * j + 1);
        r0 = dot2((av & M4) | ((hv << 4) & M2) | MG, xe0, r0);
        r0 = dot2(((av >> 8) & M4) | ((hv >> 4) & M2) | MG, xo0, r0);
        r1 = dot2((cv & M4) | ((hv << 2) & M2) | MG, xe1, r1);
        r1 = dot2(((cv >> 8) & M4) | ((hv >> 6) & M2) | MG, xo1, r1);
        r2 = dot2(((av >> 4) & M4) | (hv & M2) | MG, xe2, r2);
        r2 = dot2(((av >> 12) & M4) | ((hv >> 8) & M2) | MG, xo2, r2);
        r3 = dot2(((cv >> 4) & M4) | ((hv >> 2) & M2) | MG, xe3, r3);
        r3 = dot2(((cv >> 12) & M4) | ((hv >> 10) & M2) | MG, xo3, r3);
    }
    const float ds0 = d * (float)sc0, ds1 = d * (float)sc1, ds2 = d * (float)sc2, ds3 = d * (float)sc3;
    float acc = ds0 * r0 - (1056.0f * ds0) * s[0];
    acc += ds1 * r1 - (1056.0f * ds1) * s[2];
    acc += ds2 * r2 - (1056.0f * ds2) * s[4];
    acc += ds3 * r3 - (1056.0f * ds3) * s[6];
    return acc;
}

// ---------------------------------------------------------------- Q8_0 unit

struct XQ8 {
    uint4 v[4];
};

RFXQ_DEV void load_x_q8(const uint32_t* lds_x, uint32_t xoff, XQ8& x) {
    const uint4* p = reinterpret_cast<const uint4*>(lds_x + xoff / 2u);
#pragma unroll
    for (int i = 0; i < 4; i++) x.v[i] = p[i];
}

// One 34-byte block (2-byte aligned), never reading past its last byte.
RFXQ_DEV float q8_0_unit(const uint8_t* blk, const XQ8& x, const float* s) {
    const uintptr_t addr = reinterpret_cast<uintptr_t>(blk);
    const uint8_t* pa = reinterpret_cast<const uint8_t*>(addr & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(addr & 3u);
    const u4_t w0 = ld16_a4(pa), w1 = ld16_a4(pa + 16);
    uint32_t w8;
    if (sh) w8 = *reinterpret_cast<const uint32_t*>(pa + 32);
    else w8 = *reinterpret_cast<const uint16_t*>(blk + 32);
    const uint32_t w[9] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w, w8};
    const float d = f16_bits_to_f32(sh ? (w0.x >> 16) : w0.x);
    float r0 = 0.f, r1 = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t q = sh ? w[j + 1] : alignbyte(w[j + 1], w[j], 2u);
        const uint32_t v = q ^ 0x80808080u;
        r0 = dot2((v & 0x00FF00FFu) | 0x64006400u, u4_at(x.v, 2 * j), r0);
        r1 = dot2(((v >> 8) & 0x00FF00FFu) | 0x64006400u, u4_at(x.v, 2 * j + 1), r1);
    }
    return d * ((r0 + r1) - 1152.0f * (s[0] + s[1]));
}

// ---------------------------------------------------------------- row loops

template <uint32_t TY, int LPR>
RFXQ_DEV void gemv_rows(const GemvDesc& dsc, uint32_t row_begin, uint32_t row_end, const uint32_t* lds_x,
                        const float* lds_s) {
    constexpr int RPI = 64 / LPR;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t sub = lane / LPR, li = lane % LPR;
    const uint32_t k = dsc.k;
    const uint32_t units = TY == TY_Q8_0 ? k / 32u : k / 64u;
    const uint32_t U = units / LPR;
    const uint64_t row_bytes = TY == TY_Q4K ? (uint64_t)(k / 256u) * 144u
                             : TY == TY_Q6K ? (uint64_t)(k / 256u) * 210u
                                            : (uint64_t)(k / 32u) * 34u;
    const uint8_t* __restrict__ w = dsc.w;
    float* __restrict__ y = dsc.y;

    auto unit_xoff = [&](uint32_t unit) -> uint32_t {
        if (TY == TY_Q8_0) return unit * 32u;
        const uint32_t b = unit >> 2, g = unit & 3u;
        return TY == TY_Q4K ? 256u * b + 64u * g : 256u * b + 128u * (g >> 1) + 16u * (g & 1u);
    };
    auto unit_ptr = [&](uint32_t row, uint32_t unit) -> const uint8_t* {
        const uint64_t off = (uint64_t)row * row_bytes;
        if (TY == TY_Q8_0) return w + off + (uint64_t)unit * 34u;
        return w + off + (uint64_t)(unit >> 2) * (TY == TY_Q4K ? 144u : 210u);
    };

    if (U == 1u) {
        // The lane's x slice is the same for every row: keep it in registers.
        const uint32_t unit = li;
        const uint32_t xoff = unit_xoff(unit);
        const float* s = lds_s + xoff / 16u;
        XQ4 x4;
        XQ6 x6;
        XQ8 x8;
        float sv[8];
        if (TY == TY_Q4K) {
            load_x_q4k(lds_x, xoff, x4);
            for (int i = 0; i < 4; i++) sv[i] = s[i];
        } else if (TY == TY_Q6K) {
            load_x_q6k(lds_x, xoff, x6);
            for (int i = 0; i < 8; i++) sv[i] = s[i];
        } else {
            load_x_q8(lds_x, xoff, x8);
            for (int i = 0; i < 2; i++) sv[i] = s[i];
        }
        for (uint32_t base = row_begin + wave * RPI; base < row_end; base += 4u * RPI) {
            const uint32_t row = base + sub;
            const uint32_t rr = row < row_end ? row : row_end - 1u;
            const uint8_t* p = unit_ptr(rr, unit);
            float acc;
            if (TY == TY_Q4K) {
                const uint32_t g = unit & 3u;
                acc = q4k_unit(ld16(p), ld16(p + 16 + 32u * g), ld16(p + 32 + 32u * g), g, x4, sv);
            } else if (TY == TY_Q6K) {
                acc = q6k_unit(p, unit & 3u, x6, sv);
            } else {
                acc = q8_0_unit(p, x8, sv);
            }
            acc = group_sum<LPR>(acc);
            if (li == 0u && row < row_end) y[row] = acc;
        }
    } else {
        for (uint32_t base = row_begin + wave * RPI; base < row_end; base += 4u * RPI) {
            const uint32_t row = base + sub;
            const uint32_t rr = row < row_end ? row : row_end - 1u;
            float acc = 0.0f;
            for (uint32_t u = 0; u < U; u++) {
                const uint32_t unit = li + u * LPR;
                const uint32_t xoff = unit_xoff(unit);
                const float* s = lds_s + xoff / 16u;
                const uint8_t* p = unit_ptr(rr, unit);
                if (TY == TY_Q4K) {
                    XQ4 x4;
                    load_x_q4k(lds_x, xoff, x4);
                    const uint32_t g = unit & 3u;
                    acc += q4k_unit(ld16(p), ld16(p + 16 + 32u * g), ld16(p + 32 + 32u * g), g, x4, s);
                } else if (TY == TY_Q6K) {
                    XQ6 x6;
                    load_x_q6k(lds_x, xoff, x6);
                    acc += q6k_unit(p, unit & 3u, x6, s);
                } else {
                    XQ8 x8;
                    load_x_q8(lds_x, xoff, x8);
                    acc += q8_0_unit(p, x8, s);
                }
            }
            acc = group_sum<LPR>(acc);
            if (li == 0u && row < row_end) y[row] = acc;
        }
    }
}

template <uint32_t TY>
RFXQ_DEV void gemv_dispatch_lpr(const GemvDesc& d, uint32_t rb, uint32_t re, const uint32_t* lx, const float* ls) {
    switch (d.lpr_log2) {
        case 2: gemv_rows<TY, 4>(d, rb, re, lx, ls); break;
        case 3: gemv_rows<TY, 8>(d, rb, re, lx, ls); break;
        case 4: gemv_rows<TY, 16>(d, rb, re, lx, ls); break;
        case 5: gemv_rows<TY, 32>(d, rb, re, lx, ls); break;
        default: gemv_rows<TY, 64>(d, rb, re, lx, ls); break;
    }
}

RFXQ_DEV GemvDesc gemv_pick(const GemvArgs& a, uint32_t wg) {
    if (a.ndesc <= GEMV_INLINE) {
        GemvDesc d = a.inl[0];
        if (a.ndesc > 1 && wg >= a.inl[1].wg_begin) d = a.inl[1];
        if (a.ndesc > 2 && wg >= a.inl[2].wg_begin) d = a.inl[2];
        if (a.ndesc > 3 && wg >= a.inl[3].wg_begin) d = a.inl[3];
        return d;
    }
    uint32_t lo = 0, hi = a.ndesc - 1u;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1u) >> 1;
        if (a.table[mid].wg_begin <= wg) lo = mid;
        else hi = mid - 1u;
    }
    return a.table[lo];
}

extern "C" __global__ __launch_bounds__(256) void rfxq_gemv(GemvArgs args) {
    extern __shared__ uint32_t lds[];
    const GemvDesc d = gemv_pick(args, blockIdx.x);
    const uint32_t rb = (blockIdx.x - d.wg_begin) * d.rows_per_wg;
    const uint32_t re = min(d.n, rb + d.rows_per_wg);
    uint32_t* lds_x = lds;
    float* lds_s = reinterpret_cast<float*>(lds + d.k / 2u);
    gemv_stage_x(d.x, d.k, d.type == TY_Q4K, lds_x, lds_s);
    if (d.type == TY_Q4K) gemv_dispatch_lpr<TY_Q4K>(d, rb, re, lds_x, lds_s);
    else if (d.type == TY_Q6K) gemv_dispatch_lpr<TY_Q6K>(d, rb, re, lds_x, lds_s);
    else gemv_dispatch_lpr<TY_Q8_0>(d, rb, re, lds_x, lds_s);
}
