// Decode GEMV y[N] = W[N,K] . x[K] straight from Q4_K / Q6_K / Q8_0 blocks.
//
// Replaces `gemv_q4k_r1_kernel`, `gemv_q6k_r1_kernel`, `gemv_q6k_kernel`
// (src/kernels_cuda/gemv_q4k.cu:170-337,461-509) and `gemv_q8_0_direct_kernel`
// (src/kernels_cuda/gemv_q8_0.cu:193-230), and the fused multi-projection
// launch of `Model::gemv_qkv_to` (src/model/kernels.rs:1761): one launch runs a
// table of independent GEMVs (descriptors), each with its own weight, x and y.
//
// Design (wave64, gfx950):
//  * Each 256-thread workgroup owns a small contiguous tile of output rows
//    (tens of KB of weights) of one descriptor; its four waves work
//    independently (no barriers), so tiles can be small enough to spread any
//    GEMV over the whole chip and keep many loads in flight per CU.
//  * Each lane converts the x values of its unit to f16 registers,
//    pair-permuted and, for Q4_K high-nibble runs, pre-scaled by 1/16, plus
//    per-16 sums of those f16 values.
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
    uint32_t pad0, pad1, pad2, pad3;
};

#define GEMV_INLINE 4
struct GemvArgs {
    const GemvDesc* table;  // the descriptors (NULL: the first ndesc <= GEMV_INLINE of inl)
    const uint4* ranges;    // optional: per workgroup {d0, it0, d1, it1}
    uint32_t ndesc, part_floats;
    uint32_t iters_each;    // without ranges: every descriptor's row iterations, when all share them (else 0)
    uint32_t pad;
    GemvDesc inl[GEMV_INLINE];
};

// ---------------------------------------------------------------- prologue

// x -> LDS f16 (pair-permuted; the runs of high-nibble codes scaled by 1/16:
// elements with bit `hi` of their index set, hi = 32 for Q4_K, 64 for Q6_K, 0
// for none) and the per-16 sums of the stored f16 values (computed with the
// same dot2 op). x (at most kGemvMaxK elements, 16 per lane) is loaded into
// registers by gemv_x_load before the weight loads are issued, all at once,
// so staging costs one L2 round trip; the barriers wait on LDS only, weight
// loads issued before stay in flight.
constexpr uint32_t kGemvMaxK = 16384;
struct XRegs {
    float4 v[kGemvMaxK / 1024u];
};

RFXQ_DEV void gemv_x_load(const float* __restrict__ x, uint32_t k, XRegs& xr, uint32_t tid) {
#pragma unroll
    for (uint32_t i = 0; i < kGemvMaxK / 1024u; i++) {
        const uint32_t e = 4u * tid + 1024u * i;
        if (e < k) xr.v[i] = ldf4(x + e);
    }
}

RFXQ_DEV void gemv_x_put(uint32_t* lds_x, uint32_t e, float4 v, uint32_t hi, float scale) {
    const float sc = (e & hi) ? 0.0625f * scale : scale;
    const h2_t a = {(half_t)(v.x * sc), (half_t)(v.z * sc)};
    const h2_t b = {(half_t)(v.y * sc), (half_t)(v.w * sc)};
    lds_st64(lds_addr(lds_x) + 2u * e, u2_t{h2_bits(a), h2_bits(b)});
}

RFXQ_DEV void gemv_x_sums(const uint32_t* lds_x, float* lds_s, uint32_t k, uint32_t tid) {
    const uint32_t ng = k / 16u;
    for (uint32_t g = tid; g < ng; g += 256u) {
        u4_t p0, p1;
        lds_ld2x128(lds_addr(lds_x) + 32u * g, p0, p1);
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
        lds_st32(lds_addr(lds_s) + 4u * g, __builtin_bit_cast(uint32_t, s));
    }
}

// Returns the factor that undoes a range scaling of x: activations whose
// magnitude reaches 2^15 would overflow f16, so in that (rare) case x is
// staged again multiplied by an exact power of two 2^-s and row results are
// multiplied by 2^s when stored; otherwise it is 1 and nothing changes.
// lds_p (the row results, free while staging) carries the waves' maxima.
RFXQ_DEV float gemv_stage_x(const float* __restrict__ x, uint32_t k, uint32_t hi, const XRegs& xr,
                            uint32_t* lds_x, float* lds_s, float* lds_p, uint32_t tid) {
    float amax = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < kGemvMaxK / 1024u; i++) {
        const uint32_t e = 4u * tid + 1024u * i;
        if (e < k) {
            gemv_x_put(lds_x, e, xr.v[i], hi, 1.0f);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(xr.v[i].x), fabsf(xr.v[i].y)), fmaxf(fabsf(xr.v[i].z), fabsf(xr.v[i].w))));
        }
    }
    amax = wave_max(amax);
    if ((tid & 63u) == 0u) lds_st32(lds_addr(lds_p) + 4u * (tid >> 6), __builtin_bit_cast(uint32_t, amax));
    lds_barrier();
    {
        const u4_t m4 = lds_ld128(lds_addr(lds_p));
        amax = fmaxf(fmaxf(as_f32(m4.x), as_f32(m4.y)), fmaxf(as_f32(m4.z), as_f32(m4.w)));
    }
    gemv_x_sums(lds_x, lds_s, k, tid);
    lds_barrier();
    float inv = 1.0f;
    if (amax >= 32768.0f && amax <= 3.0e38f) {  // workgroup-uniform
        int ex;
        (void)frexpf(amax, &ex);  // amax < 2^ex
        const float scale = ldexpf(1.0f, 14 - ex);
        inv = ldexpf(1.0f, ex - 14);
        for (uint32_t e = 4u * tid; e < k; e += 1024u) gemv_x_put(lds_x, e, ldf4(x + e), hi, scale);
        lds_barrier();
        gemv_x_sums(lds_x, lds_s, k, tid);
        lds_barrier();
    }
    return inv;
}

RFXQ_DEV uint32_t u4_at(const uint4* a, int j) {
    const uint4 v = a[j >> 2];
    return (j & 3) == 0 ? v.x : (j & 3) == 1 ? v.y : (j & 3) == 2 ? v.z : v.w;
}

// ---------------------------------------------------------------- per-type units
//
// A "unit" is one lane's share of one row: 64 weights for Q4_K / Q6_K (a
// quarter super-block), 32 for Q8_0 (one block). Each type provides
//   Raw      the unit's raw bytes as loaded (kept in registers while in flight)
//   XV       the unit's x values (from LDS) and x sums
//   fetch()  read a unit's bytes from an LDS copy of its row chunk
//   loadx()  read the unit's x from LDS
//   dot()    the unit's contribution to the row's dot product

struct Q4K {
    static constexpr uint32_t QK = 256, BB = 144, UPB = 4;  // units per block
    static constexpr uint32_t XHI = 32;    // x of high-nibble runs staged / 16
    static constexpr bool ALIGNED = true;  // blocks (and rows) start 16-byte aligned
    static constexpr int NJ = 3;           // 1 KB copy instructions per item (64 x 36 B)
    struct Raw {
        u4_t hdr, qa, qb;
    };
    struct XV {
        uint4 l[4], h[4];
        float s[4];
    };
    static RFXQ_DEV uint32_t xoff(uint32_t unit) { return 256u * (unit >> 2) + 64u * (unit & 3u); }
    // byte offset of the unit's block within a row
    static RFXQ_DEV uint32_t unit_off(uint32_t unit) { return (unit >> 2) * BB; }
    // the unit's bytes from its block at slot byte o (16-byte aligned)
    static RFXQ_DEV Raw fetch(const uint8_t* slot, uint32_t o, uint32_t unit) {
        const uint32_t a = lds_addr(slot) + o;
        const uint32_t q = a + 16u + 32u * (unit & 3u);
        Raw r;
        asm volatile(
            "ds_read_b128 %0, %3\n\t"
            "ds_read_b128 %1, %4\n\t"
            "ds_read_b128 %2, %4 offset:16\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(r.hdr), "=&v"(r.qa), "=&v"(r.qb)
            : "v"(a), "v"(q)
            : "memory");
        return r;
    }
    static RFXQ_DEV void loadx(const uint32_t* lds_x, const float* lds_s, uint32_t unit, XV& x) {
        const uint32_t o = xoff(unit);
        const uint32_t a = lds_addr(lds_x) + 2u * o;
        u4_t v[8];
        lds_ld4x128(a, v[0], v[1], v[2], v[3]);
        lds_ld4x128(a + 64u, v[4], v[5], v[6], v[7]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x.l[i] = as_uint4(v[i]);
            x.h[i] = as_uint4(v[4 + i]);
        }
        const u4_t sm = lds_ld128(lds_addr(lds_s) + 4u * (o / 16u));
        x.s[0] = as_f32(sm.x);
        x.s[1] = as_f32(sm.y);
        x.s[2] = as_f32(sm.z);
        x.s[3] = as_f32(sm.w);
    }
    // qs bytes [32g, 32g+32) = sub-blocks 2g (low nibbles) and 2g+1 (high).
    // The 6-bit scales/mins of sub-blocks j = 2g, 2g+1 (g = unit & 3, fixed
    // per lane) are decoded without branches: bytes (q[j], q[j+4], q[j-4]) of
    // the 12-byte table sit in a = hdr.y, b = hdr.z, c = hdr.w, 16*(g&1) bits
    // up; j < 4 takes the low 6 bits of a (scales) and b (mins), j >= 4 takes
    // a nibble of c plus the top 2 bits of a (scales) or b (mins).
    static RFXQ_DEV float dot(const Raw& r, uint32_t unit, const XV& x, uint32_t MG) {
#pragma clang fp contract(off)
        const uint32_t g = unit & 3u;
        const uint32_t sh = (g & 1u) * 16u;
        const bool low = g < 2u;
        const uint32_t a = r.hdr.y >> sh, b = r.hdr.z >> sh, c = r.hdr.w >> sh;
        const uint32_t mlo = low ? 0x3F3Fu : 0x0F0Fu, mhi = low ? 0u : 0x3030u;
        const uint32_t SC = ((low ? a : c) & mlo) | ((a >> 2) & mhi);
        const uint32_t M = (((low ? b : c) >> (low ? 0u : 4u)) & mlo) | ((b >> 2) & mhi);
        const float d = f16_bits_to_f32(r.hdr.x);
        const float dmin = f16_bits_to_f32(r.hdr.x >> 16);
        const float d1 = d * (float)(SC & 0xFFu), d2 = d * (float)((SC >> 8) & 0xFFu);
        const float mm1 = dmin * (float)(M & 0xFFu), mm2 = dmin * (float)((M >> 8) & 0xFFu);
        const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        float rl0 = 0.f, rl1 = 0.f, rh0 = 0.f, rh1 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t v = q[j], v8 = v >> 8;
            rl0 = dot2((v & 0x000F000Fu) | MG, u4_at(x.l, 2 * j), rl0);
            rl1 = dot2((v8 & 0x000F000Fu) | MG, u4_at(x.l, 2 * j + 1), rl1);
            rh0 = dot2((v & 0x00F000F0u) | MG, u4_at(x.h, 2 * j), rh0);
            rh1 = dot2((v8 & 0x00F000F0u) | MG, u4_at(x.h, 2 * j + 1), rh1);
        }
        const float slo = x.s[0] + x.s[1], shi = x.s[2] + x.s[3];
        const float lo = fmaf(d1, rl0 + rl1, -(fmaf(1024.0f, d1, mm1) * slo));
        const float hi = fmaf(d2, rh0 + rh1, -(fmaf(1024.0f, d2, 16.0f * mm2) * shi));
        return lo + hi;
    }
};

// 16 bytes at byte offset o of a 2-byte-aligned block: four dwords from the
// dword-aligned offset below plus one more, realigned by sh = 0 or 2 bytes.
struct Seg {
    u4_t v;
    uint32_t e;
};

RFXQ_DEV u4_t seg_align(const Seg& s, uint32_t sh) {
    u4_t r;
    r.x = alignbyte(s.v.y, s.v.x, sh);
    r.y = alignbyte(s.v.z, s.v.y, sh);
    r.z = alignbyte(s.v.w, s.v.z, sh);
    r.w = alignbyte(s.e, s.v.w, sh);
    return r;
}

struct Q6K {
    static constexpr uint32_t QK = 256, BB = 210, UPB = 4;
    static constexpr uint32_t XHI = 64;   // x of the high-nibble runs (64..127 of each 128) staged / 16
    static constexpr bool ALIGNED = false;  // blocks are 2-byte aligned
    static constexpr int NJ = 4;            // 64 x 52.5 B plus per-row alignment slack
    struct Raw {
        Seg a, c, h;
        u4_t sw;
        uint32_t tail, sh;
    };
    struct XV {
        uint4 r[4][2];
        float s[4];
    };
    // half n = g >> 1, positions [16*(g&1), +16) of the four 32-runs
    static RFXQ_DEV uint32_t xoff(uint32_t unit) {
        const uint32_t g = unit & 3u;
        return 256u * (unit >> 2) + 128u * (g >> 1) + 16u * (g & 1u);
    }
    static RFXQ_DEV uint32_t unit_off(uint32_t unit) { return (unit >> 2) * BB; }
    // dword-aligned reads (the block may start 2 bytes past a dword)
    static RFXQ_DEV Raw fetch(const uint8_t* slot, uint32_t o, uint32_t unit) {
        const uint32_t g = unit & 3u, n = g >> 1, hs = g & 1u;
        const uint32_t a4 = lds_addr(slot) + (o & ~3u);
        const uint32_t pa = a4 + 64u * n + 16u * hs, ph = a4 + 128u + 32u * n + 16u * hs;
        Raw r;
        r.sh = o & 3u;
        u2_t a01, a23, c01, c23, h01, h23, s01, s23, ae_ce, he_t;
        asm volatile(
            "ds_read2_b32 %0, %10 offset1:1\n\t"
            "ds_read2_b32 %1, %10 offset0:2 offset1:3\n\t"
            "ds_read2_b32 %2, %10 offset0:8 offset1:9\n\t"
            "ds_read2_b32 %3, %10 offset0:10 offset1:11\n\t"
            "ds_read2_b32 %4, %11 offset1:1\n\t"
            "ds_read2_b32 %5, %11 offset0:2 offset1:3\n\t"
            "ds_read2_b32 %6, %12 offset0:48 offset1:49\n\t"
            "ds_read2_b32 %7, %12 offset0:50 offset1:51\n\t"
            "ds_read2_b32 %8, %10 offset0:4 offset1:12\n\t"
            "ds_read2_b32 %9, %11 offset0:4\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(a01), "=&v"(a23), "=&v"(c01), "=&v"(c23), "=&v"(h01), "=&v"(h23), "=&v"(s01), "=&v"(s23),
              "=&v"(ae_ce), "=&v"(he_t)
            : "v"(pa), "v"(ph), "v"(a4)
            : "memory");
        uint32_t tail;
        asm volatile("ds_read_b32 %0, %1 offset:208\n\ts_waitcnt lgkmcnt(0)" : "=&v"(tail) : "v"(a4) : "memory");
        r.a = Seg{u4_t{a01.x, a01.y, a23.x, a23.y}, ae_ce.x};
        r.c = Seg{u4_t{c01.x, c01.y, c23.x, c23.y}, ae_ce.y};
        r.h = Seg{u4_t{h01.x, h01.y, h23.x, h23.y}, he_t.x};
        r.sw = u4_t{s01.x, s01.y, s23.x, s23.y};
        r.tail = tail;
        return r;
    }
    static RFXQ_DEV void loadx(const uint32_t* lds_x, const float* lds_s, uint32_t unit, XV& x) {
        const uint32_t o = xoff(unit);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            u4_t v0, v1;
            lds_ld2x128(lds_addr(lds_x) + 2u * (o + 32u * t), v0, v1);
            x.r[t][0] = as_uint4(v0);
            x.r[t][1] = as_uint4(v1);
            x.s[t] = __builtin_bit_cast(float, lds_ld32(lds_addr(lds_s) + 4u * (o / 16u + 2u * t)));
        }
    }
    // runs 0, 1 (low nibbles of ql) as 1024 + q with the qh bits at 4-5;
    // runs 2, 3 (high nibbles) as 1024 + 16q with the qh bits at 8-9, against
    // x staged / 16: each pair is two v_and_or_b32 and one dot2, the shifted
    // qh words shared by a low and a high run
    static RFXQ_DEV float dot(const Raw& r, uint32_t unit, const XV& x, uint32_t MG) {
#pragma clang fp contract(off)
        const uint32_t g = unit & 3u, n = g >> 1, hs = g & 1u, sh = r.sh;
        const u4_t a = seg_align(r.a, sh), c = seg_align(r.c, sh), h = seg_align(r.h, sh);
        const uint32_t s0 = alignbyte(r.sw.y, r.sw.x, sh), s1 = alignbyte(r.sw.z, r.sw.y, sh);
        const uint32_t s2 = alignbyte(r.sw.w, r.sw.z, sh), s3 = alignbyte(r.tail, r.sw.w, sh);
        const float d = f16_bits_to_f32(alignbyte(r.tail, r.tail, sh));
        const uint32_t W0 = n ? s2 : s0, W1 = n ? s3 : s1;
        const int sc0 = (int)(int8_t)(W0 >> (8u * hs));
        const int sc1 = (int)(int8_t)(W0 >> (8u * hs + 16u));
        const int sc2 = (int)(int8_t)(W1 >> (8u * hs));
        const int sc3 = (int)(int8_t)(W1 >> (8u * hs + 16u));
        const uint32_t A[4] = {a.x, a.y, a.z, a.w}, C[4] = {c.x, c.y, c.z, c.w}, H[4] = {h.x, h.y, h.z, h.w};
        float r0 = 0.f, r1 = 0.f, r2 = 0.f, r3 = 0.f;
        uint32_t ml = 0x000F000Fu, mq = 0x00300030u, mlh = 0x00F000F0u, mqh = 0x03000300u;
        asm volatile("" : "+v"(ml), "+v"(mq), "+v"(mlh), "+v"(mqh));
        auto ao = [](uint32_t v, uint32_t m, uint32_t c2) {
            uint32_t o;
            asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(o) : "v"(v), "v"(m), "v"(c2));
            return o;
        };
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t av = A[j], cv = C[j], hv = H[j];
            const uint32_t a8 = av >> 8, c8 = cv >> 8;
            const uint32_t h4l = hv << 4, h4r = hv >> 4, h2l = hv << 2, h6r = hv >> 6;
            r0 = dot2(ao(av, ml, ao(h4l, mq, MG)), u4_at(x.r[0], 2 * j), r0);
            r0 = dot2(ao(a8, ml, ao(h4r, mq, MG)), u4_at(x.r[0], 2 * j + 1), r0);
            r1 = dot2(ao(cv, ml, ao(h2l, mq, MG)), u4_at(x.r[1], 2 * j), r1);
            r1 = dot2(ao(c8, ml, ao(h6r, mq, MG)), u4_at(x.r[1], 2 * j + 1), r1);
            r2 = dot2(ao(av, mlh, ao(h4l, mqh, MG)), u4_at(x.r[2], 2 * j), r2);
            r2 = dot2(ao(a8, mlh, ao(h4r, mqh, MG)), u4_at(x.r[2], 2 * j + 1), r2);
            r3 = dot2(ao(cv, mlh, ao(h2l, mqh, MG)), u4_at(x.r[3], 2 * j), r3);
            r3 = dot2(ao(c8, mlh, ao(h6r, mqh, MG)), u4_at(x.r[3], 2 * j + 1), r3);
        }
        // runs 0, 1: sum (1024 + q) x - 1056 sum x; runs 2, 3: sum (64 + q) x -
        // 96 sum x = r - 1536 sum(x / 16), the staged sums being of x / 16
        const float ds0 = d * (float)sc0, ds1 = d * (float)sc1, ds2 = d * (float)sc2, ds3 = d * (float)sc3;
        float acc = fmaf(ds0, r0, -((1056.0f * ds0) * x.s[0]));
        acc += fmaf(ds1, r1, -((1056.0f * ds1) * x.s[1]));
        acc += fmaf(ds2, r2, -((1536.0f * ds2) * x.s[2]));
        acc += fmaf(ds3, r3, -((1536.0f * ds3) * x.s[3]));
        return acc;
    }
};

struct Q80 {
    static constexpr uint32_t QK = 32, BB = 34, UPB = 1;
    static constexpr uint32_t XHI = 0;
    static constexpr bool ALIGNED = false;  // blocks are 2-byte aligned
    static constexpr int NJ = 3;            // 64 x 34 B plus per-row alignment slack
    struct Raw {
        u4_t w0, w1;
        uint32_t w8, sh;
    };
    struct XV {
        uint4 v[4];
        float s[2];
    };
    static RFXQ_DEV uint32_t xoff(uint32_t unit) { return unit * 32u; }
    static RFXQ_DEV uint32_t unit_off(uint32_t unit) { return unit * BB; }
    // one 34-byte block (2-byte aligned): 9 dwords from the dword-aligned offset
    static RFXQ_DEV Raw fetch(const uint8_t* slot, uint32_t o, uint32_t) {
        const uint32_t a4 = lds_addr(slot) + (o & ~3u);
        Raw r;
        r.sh = o & 3u;
        u2_t d01, d23, d45, d67;
        asm volatile(
            "ds_read2_b32 %0, %5 offset1:1\n\t"
            "ds_read2_b32 %1, %5 offset0:2 offset1:3\n\t"
            "ds_read2_b32 %2, %5 offset0:4 offset1:5\n\t"
            "ds_read2_b32 %3, %5 offset0:6 offset1:7\n\t"
            "ds_read_b32 %4, %5 offset:32\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(d01), "=&v"(d23), "=&v"(d45), "=&v"(d67), "=&v"(r.w8)
            : "v"(a4)
            : "memory");
        r.w0 = u4_t{d01.x, d01.y, d23.x, d23.y};
        r.w1 = u4_t{d45.x, d45.y, d67.x, d67.y};
        return r;
    }
    static RFXQ_DEV void loadx(const uint32_t* lds_x, const float* lds_s, uint32_t unit, XV& x) {
        const uint32_t o = xoff(unit);
        u4_t v[4];
        lds_ld4x128(lds_addr(lds_x) + 2u * o, v[0], v[1], v[2], v[3]);
#pragma unroll
        for (int i = 0; i < 4; i++) x.v[i] = as_uint4(v[i]);
        const u2_t sm = lds_ld64(lds_addr(lds_s) + 4u * (o / 16u));
        x.s[0] = as_f32(sm.x);
        x.s[1] = as_f32(sm.y);
    }
    static RFXQ_DEV float dot(const Raw& r, uint32_t, const XV& x, uint32_t MG) {
#pragma clang fp contract(off)
        const uint32_t sh = r.sh;
        const uint32_t w[9] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w, r.w8};
        const float d = f16_bits_to_f32(alignbyte(r.w0.x, r.w0.x, sh));
        float r0 = 0.f, r1 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t q = sh ? w[j + 1] : alignbyte(w[j + 1], w[j], 2u);
            const uint32_t v = q ^ 0x80808080u;
            r0 = dot2((v & 0x00FF00FFu) | MG, u4_at(x.v, 2 * j), r0);
            r1 = dot2(((v >> 8) & 0x00FF00FFu) | MG, u4_at(x.v, 2 * j + 1), r1);
        }
        return d * fmaf(-1152.0f, x.s[0] + x.s[1], r0 + r1);
    }
};

// ---------------------------------------------------------------- row loop

// Weight ring: each wave owns kRing slots of kSlotBytes in LDS. One item (one
// unit per lane: RPI rows x the row chunk of LPR units) is copied into a slot
// by NJ asynchronous 1 KB copies in which consecutive lanes take consecutive
// 16-byte pieces of the rows (fully coalesced, and no VGPRs held while the
// copy is in flight); each lane then reads its own unit from the slot. Every
// slot is its own array, so the compiler's wait counting knows which copy a
// read depends on and waits for exactly that one.
constexpr uint32_t kSlotBytes = 4096;
#ifndef RFXQ_GEMV_RING
#define RFXQ_GEMV_RING 2
#endif
constexpr int kRing = RFXQ_GEMV_RING;
__shared__ __attribute__((aligned(16))) uint8_t gemv_ring0[4][kSlotBytes];
__shared__ __attribute__((aligned(16))) uint8_t gemv_ring1[4][kSlotBytes];
#if RFXQ_GEMV_RING > 2
__shared__ __attribute__((aligned(16))) uint8_t gemv_ring2[4][kSlotBytes];
#endif
#if RFXQ_GEMV_RING > 3
__shared__ __attribute__((aligned(16))) uint8_t gemv_ring3[4][kSlotBytes];
#endif


// Offset for copies past a wave's last item: beyond any weight buffer's range
// (the host keeps weights below it), so the copy writes zeros and fetches
// nothing.
constexpr uint32_t kPastEnd = 0xFFFFF000u;

// Rows are covered by lane groups of LPR lanes; lane li owns units li + u*LPR,
// u < U. The wave's rows are row_begin + wave*RPI + sub + it*4*RPI (sub =
// lane / LPR, it < n_it). Work items run pass by pass: pass u walks all of
// the wave's rows with unit li + u*LPR, so a lane only ever holds the x slice
// of one unit in registers (reloaded from LDS at each pass start). Row
// results go to an LDS row buffer by lane li == 0 of the group; with U > 1
// the partial is carried there between passes (always the same thread, so
// program order is enough) and added in pass order, so the result does not
// depend on tiling. The buffer is stored to y, coalesced, at the end.
template <typename T, int LPR>
RFXQ_DEV void gemv_rows(const GemvDesc& dsc, uint32_t row_begin, uint32_t row_end, bool restage, uint32_t* lds_x,
                        float* lds_s, float* lds_p) {
#pragma clang fp contract(off)
    constexpr int RPI = 64 / LPR;
    constexpr int NJ = T::NJ;
    // opaque to the optimiser: keeps the lane-derived values of every type and
    // LPR variant from being hoisted out of the segment loop (all of them
    // would then stay live across it)
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t sub = lane / LPR, li = lane % LPR;
    const uint32_t k = dsc.k, n = dsc.n;
    const uint32_t units = k / (T::QK / T::UPB);
    const uint32_t U = units / LPR;
    const uint32_t row_bytes = (k / T::QK) * T::BB;
    // dword-aligned V# base (Q6_K / Q8_0 data may start 2 bytes past one), the
    // remainder added to every offset, range rounded up to whole dwords (the
    // last dword never crosses a page, so reading all of it is safe)
    const uintptr_t wa = reinterpret_cast<uintptr_t>(dsc.w);
    const uint32_t wsh = (uint32_t)(wa & 3u);
    const rsrc_t wr = make_rsrc(reinterpret_cast<const void*>(wa - wsh), (wsh + n * row_bytes + 3u) & ~3u);
    const rsrc_t yr = make_rsrc(dsc.y, n * 4u);
    const uint32_t base0 = row_begin + wave * RPI;
    const uint32_t stride = 4u * RPI;
    // wave-uniform (the scalar unit runs the item loop)
    const uint32_t n_it = __builtin_amdgcn_readfirstlane(base0 < row_end ? (row_end - base0 + stride - 1u) / stride : 0u);
    const uint32_t n_items = n_it * U;
    const uint32_t row_step = stride * row_bytes;  // bytes between row iterations
    const uint32_t chunk = T::unit_off(LPR);       // one row's bytes of an item
    const uint32_t out0 = lds_addr(lds_p);  // row results (and partials), by row - row_begin

    // Slot layout: row r of the item at r * ppr * 16 bytes, its chunk copied
    // from the dword at or below its start (sh = start & 3 bytes of slack).
    const uint32_t ppr = T::ALIGNED ? chunk / 16u : (chunk + 3u + 15u) / 16u;
    uint32_t prb[NJ], pc[NJ];
    bool pv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t p = 64u * j + lane, r = p / ppr;
        pv[j] = r < (uint32_t)RPI;
        prb[j] = r * row_bytes;
        pc[j] = 16u * (p - r * ppr);
    }
    const uint32_t uo = sub * ppr * 16u + T::unit_off(li);  // this lane's unit in a slot
    uint8_t* const ring[kRing] = {gemv_ring0[wave], gemv_ring1[wave]
#if RFXQ_GEMV_RING > 2
                                  , gemv_ring2[wave]
#endif
#if RFXQ_GEMV_RING > 3
                                  , gemv_ring3[wave]
#endif
    };

    // next item to copy: pass lu, row iteration lit; S = buffer offset of the
    // item's first row chunk (scalar)
    const uint32_t S0 = wsh + base0 * row_bytes;
    uint32_t lu = n_it ? 0u : U, lit = 0, lS = S0;
    auto advance = [&](uint32_t& u, uint32_t& it, uint32_t& S) {
        S += row_step;
        if (++it == n_it) {
            it = 0;
            u++;
            S = S0 + u * chunk;
        }
    };
    uint32_t slotS[kRing];
    auto issue = [&](int t) {
        const bool valid = lu < U;
        slotS[t] = lS;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            uint32_t g = lS + prb[j];
            if (!T::ALIGNED) g &= ~3u;
            g += pc[j];
            dma16_stream(wr, ring[t] + 1024 * j, valid && pv[j] ? g : kPastEnd);
        }
        advance(lu, lit, lS);
    };

    // Stores share vmcnt with the copies and may complete out of order with
    // them, which would break the counted waits below: none may be in flight
    // (the previous segment's are drained here), and results go to LDS and
    // are stored after the last wait.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    XRegs xr;
    gemv_x_load(dsc.x, k, xr, tid);
#pragma unroll
    for (int t = 0; t < kRing; t++) issue(t);
    if (restage) lds_barrier();  // every wave is done with the previous segment's x
    const float y_scale = gemv_stage_x(dsc.x, k, T::XHI, xr, lds_x, lds_s, lds_p, tid);

    // f16 1024.0 in both halves, kept in a VGPR: gfx9 VOP3 takes at most one
    // SGPR/constant, so (v & mask) | magic is one v_and_or_b32 only this way
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    typename T::XV xv;
    T::loadx(lds_x, lds_s, li, xv);
    uint32_t cu = 0, cit = 0;  // item being computed
    for (uint32_t t0 = 0; t0 < n_items; t0 += kRing) {
#pragma unroll
        for (int t = 0; t < kRing; t++) {
            if (t0 + t < n_items) {
                const uint32_t unit = li + cu * LPR;
                const uint32_t sh = T::ALIGNED ? 0u : ((slotS[t] + sub * row_bytes) & 3u);
                // the copies are counted in order: slot t's are done once at
                // most those of the other kRing - 1 slots are outstanding
                // (stores issued since only make this wait longer)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kRing - 1) * NJ) : "memory");
                const typename T::Raw rr = T::fetch(ring[t], uo + sh, unit);
                issue(t);  // the slot's reads are done (fetch waits for them): refill it during the math
                float acc = T::dot(rr, unit, xv, magic);
                acc = group_sum<LPR>(acc);
                const uint32_t row = base0 + sub + cit * stride;
                if (li == 0u && row < row_end) {
                    const uint32_t pa = out0 + 4u * (row - row_begin);
                    if (cu > 0u) acc = __builtin_bit_cast(float, lds_ld32(pa)) + acc;
                    lds_st32(pa, __builtin_bit_cast(uint32_t, acc));
                }
                if (++cit == n_it) {
                    cit = 0;
                    if (++cu < U) T::loadx(lds_x, lds_s, li + cu * LPR, xv);
                }
            }
        }
    }
    // no copy may land in LDS after the workgroup is gone (or in the next
    // segment's reads)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    for (uint32_t i = tid; i < row_end - row_begin; i += 256u)
        bst4f(yr, (row_begin + i) * 4u, __builtin_bit_cast(float, lds_ld32(out0 + 4u * i)) * y_scale);
}

template <typename T>
RFXQ_DEV void gemv_dispatch_lpr(const GemvDesc& d, uint32_t rb, uint32_t re, bool rs, uint32_t* lx, float* ls,
                                float* lp) {
    switch (d.lpr_log2) {
        case 2: gemv_rows<T, 4>(d, rb, re, rs, lx, ls, lp); break;
        case 3: gemv_rows<T, 8>(d, rb, re, rs, lx, ls, lp); break;
        case 4: gemv_rows<T, 16>(d, rb, re, rs, lx, ls, lp); break;
        case 5: gemv_rows<T, 32>(d, rb, re, rs, lx, ls, lp); break;
        default: gemv_rows<T, 64>(d, rb, re, rs, lx, ls, lp); break;
    }
}

// Rows of a descriptor are handed out in row iterations of 4 * (64 / LPR)
// rows (one lane group per wave and row). The launch has a fixed number of
// workgroups (about as many as the chip holds at once); workgroup g walks a
// contiguous range of the launch's iterations in descriptor order, [first,
// last) with first = (d0, it0), last = (d1, it1), crossing descriptors where
// needed (x is restaged in LDS at each crossing). With an iteration table the
// ranges are balanced by bytes on the host; without one (inline descriptors,
// or a table written on the device) by iteration count.
RFXQ_DEV uint32_t gemv_iters(const GemvDesc& d) {
    const uint32_t rows_iter = 256u >> d.lpr_log2;
    return (d.n + rows_iter - 1u) / rows_iter;
}

// (a pointer into the kernel arguments, so a runtime index is a scalar load
// rather than a register copy of the whole array)
RFXQ_DEV const GemvDesc* gemv_desc(const GemvArgs& a, uint32_t i) {
    return a.table ? a.table + i : &a.inl[0] + i;
}

// A descriptor read into scalar registers: every field is marked wave-uniform,
// so the weight buffer's V# stays in SGPRs (a V# the compiler thinks may
// differ per lane turns each buffer load into a loop over lanes).
RFXQ_DEV GemvDesc gemv_uniform(const GemvDesc* p) {
    struct Words {
        uint32_t v[sizeof(GemvDesc) / 4];
    };
    Words w = *reinterpret_cast<const Words*>(p);
#pragma unroll
    for (uint32_t i = 0; i < sizeof(GemvDesc) / 4; i++) w.v[i] = __builtin_amdgcn_readfirstlane(w.v[i]);
    return __builtin_bit_cast(GemvDesc, w);
}

// LDS: [part_floats] row results of the current segment, then x as f16
// (k * 2 bytes) and the per-16 x sums (k / 4 bytes).
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void rfxq_gemv(GemvArgs args) {
    extern __shared__ uint32_t lds[];
    uint32_t d0, it0, d1, it1;
    if (args.ranges) {
        const uint4 r = args.ranges[blockIdx.x];
        d0 = __builtin_amdgcn_readfirstlane(r.x);
        it0 = __builtin_amdgcn_readfirstlane(r.y);
        d1 = __builtin_amdgcn_readfirstlane(r.z);
        it1 = __builtin_amdgcn_readfirstlane(r.w);
    } else {
        // no range table: iterations split evenly by count, descriptor
        // counts from iters_each or read from the descriptors (inline or a
        // table; a table the device just wrote costs a round trip per read)
        const uint32_t ie = args.iters_each;
        uint32_t total = 0;
        if (ie) total = ie * args.ndesc;
        else
            for (uint32_t i = 0; i < args.ndesc; i++) total += gemv_iters(*gemv_desc(args, i));
        uint32_t g0 = (uint32_t)(((uint64_t)total * blockIdx.x) / gridDim.x);
        uint32_t g1 = (uint32_t)(((uint64_t)total * (blockIdx.x + 1u)) / gridDim.x);
        if (ie) {
            d0 = min(g0 / ie, args.ndesc - 1u);
            g0 -= d0 * ie;
            d1 = g1 ? min((g1 - 1u) / ie, args.ndesc - 1u) : 0u;
            g1 -= d1 * ie;
        } else {
            d0 = 0;
            for (uint32_t c; d0 + 1u < args.ndesc && g0 >= (c = gemv_iters(*gemv_desc(args, d0)));) {
                g0 -= c;
                d0++;
            }
            d1 = 0;
            for (uint32_t c; d1 + 1u < args.ndesc && g1 > (c = gemv_iters(*gemv_desc(args, d1)));) {
                g1 -= c;
                d1++;
            }
        }
        it0 = __builtin_amdgcn_readfirstlane(g0);
        it1 = __builtin_amdgcn_readfirstlane(g1);
        d0 = __builtin_amdgcn_readfirstlane(d0);
        d1 = __builtin_amdgcn_readfirstlane(d1);
    }
    bool restage = false;
    for (uint32_t di = d0; di <= d1; di++) {
        const GemvDesc d = gemv_uniform(gemv_desc(args, di));
        const uint32_t a = di == d0 ? it0 : 0u;
        const uint32_t b = di == d1 ? it1 : gemv_iters(d);
        if (a >= b) continue;
        const uint32_t rows_iter = 256u >> d.lpr_log2;
        const uint32_t rb = a * rows_iter, re = min(d.n, b * rows_iter);
        float* lds_p = reinterpret_cast<float*>(lds);
        uint32_t* lds_x = lds + args.part_floats;
        float* lds_s = reinterpret_cast<float*>(lds_x + d.k / 2u);
        if (d.type == TY_Q4K) gemv_dispatch_lpr<Q4K>(d, rb, re, restage, lds_x, lds_s, lds_p);
        else if (d.type == TY_Q6K) gemv_dispatch_lpr<Q6K>(d, rb, re, restage, lds_x, lds_s, lds_p);
        else gemv_dispatch_lpr<Q80>(d, rb, re, restage, lds_x, lds_s, lds_p);
        restage = true;
    }
}

