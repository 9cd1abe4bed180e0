// MMQ prefill GEMM: Y[M,N] = X[M,K] . W[N,K]^T with X quantized per 32 to int8
// (Q8_1: quant.hpp) and W raw Q4_K / Q6_K / Q8_0 blocks, contracted on the
// gfx950 int8 matrix cores (v_mfma_i32_32x32x32_i8: one MFMA = one 32-element
// activation block) with the per-block scale and min corrections applied in
// f32. Replaces the reference's f16 tensor-core prefill
// `gemm_q{4,6}k_mma_*_kernel` (src/kernels_cuda/gemm_q_mma.cu:299-764) and its
// split-K reduce (:769-783), and serves `Model::gemm` (src/model/kernels.rs:2197)
// and the per-expert `expert_gemm` (src/model/dense.rs:1103) as one grouped
// launch over a descriptor table.
//
// Per 32-block s of super-block sb, for output (m, n):
//   D = sum_{k in s} qa[m,k] * code[n,k]                    (exact int32, MFMA)
//   Q4_K: code = q - 8 (centered), and with c_s = 8*d*sc_s - dmin*m_s
//         y += da[m,s] * (d*sc_s)[n] * D  +  Sx[m,s] * c_s[n]
//         where Sx = d * s is the block's exact activation sum (the sum
//         field, stored in units of d), so the weights' constant part sees
//         unquantized activations.
//   Q6_K: D folds the two 16-run scales: D = sc_lo*D_lo + sc_hi*D_hi;
//         y += da[m,s] * d[n] * D
//   Q8_0: y += da[m,s] * d[n,s] * D
// The constant term of a Q4_K super-block is four f32 MFMAs (32x32x2, K = 2
// of the 8 sub-blocks each) into the same f32 accumulators. The scale
// products da[m,s] * dw[n,s] come from an f16 MFMA per tile and block
// (scale_products), so the per-element epilogue is one convert and one FMA:
// the VALU, not the int8 matrix core, bounds this kernel.
//
// Tile: 128 (M) x 128 (N) per 256-thread workgroup; each wave owns 64 x 64 =
// 2 x 2 MFMA tiles. Activation scales for the tile's 128 rows are staged in
// LDS once per super-block; A (int8 activations) and B (unpacked weights) go
// straight from global memory into MFMA operand registers (lane l holds row /
// column l%32 and the 16 K-values [16*(l/32), +16) of the 32-block).
// Split-K writes partial tiles to a workspace reduced in fixed order.
#pragma once
#include "common.hpp"

struct MmqDesc {
    const uint8_t* w;       // raw blocks [n][k/QK]
    const int8_t* xq;       // quantized activations [rows_src][ldq]
    const uint32_t* xds;    // [rows_src][k/32] d | s << 16
    const int32_t* rows;    // optional [m] source rows (gather); null = identity
    float* y;               // [splits][m][ldy] (splits > 1: workspace)
    uint32_t m, n, k, type;
    uint32_t ldq, ldy, tiles_m, tiles_n;
    uint32_t splits, sb_per_split, wg_begin;
    // 1: a gate/up pair (the Q4_K f16 tiles, mmqh.hpp): w holds the gate
    // weights, w_up the up weights of the same shape, and y receives
    // s = silu(gate) * up [m][n]; tiles are 128 columns wide
    uint32_t gu_pair;
    union {
        int32_t* dots_out;      // [m][n][k/32] for the rfxq_mmq_dots_* test hook (int8 kernels)
        const uint8_t* w_up;    // gu_pair: the up weights
    };
    const float* xrs;       // f16-activation kernels (mmqh.hpp): [m] row scales 2^e
};

#define MMQ_INLINE 2
struct MmqArgs {
    const MmqDesc* table;
    uint32_t ndesc, pad;
    MmqDesc inl[MMQ_INLINE];
};

#define MMQ_BN 128

RFXQ_DEV v16i_t mfma_i8(v4i_t a, v4i_t b) {
    const v16i_t z = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
}

RFXQ_DEV v4i_t as_v4i(u4_t v) { return __builtin_bit_cast(v4i_t, v); }

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
RFXQ_DEV h8_t as_h8(u4_t v) { return __builtin_bit_cast(h8_t, v); }

// Scale products S[m,n] = da[m] * dw[n] of one 32-block for a 32x32 tile, in
// the int8 MFMA's accumulator layout, from one f16 MFMA (32x32x16): lanes
// 0-31 carry K-slots 0-7 of row / column l%32, lanes 32-63 slots 8-15 (zero).
// Every product is exact in f32 (f16 x f16), and the sum over slots is of
// at most 6 such terms. This replaces a VALU multiply per output element and
// block; the epilogue is then one convert and one FMA.
RFXQ_DEV v16f_t scale_products(u4_t a, u4_t b) {
    const v16f_t z = {};
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(as_h8(a), as_h8(b), z, 0, 0, 0);
}

// f16 bits of x twice in one dword
RFXQ_DEV uint32_t h2_dup(uint32_t bits16) { return (bits16 & 0xFFFFu) * 0x00010001u; }

// ---------------------------------------------------------------- weights

// Q4_K: integer 6-bit scales of sub-blocks 2g and 2g+1 (get_scale_min_k4,
// src/dequant.rs:39-47)
RFXQ_DEV void q4k_pair_sc(const u4_t hdr, uint32_t g, uint32_t& sc1, uint32_t& sc2) {
    const uint32_t sh = (g & 1u) * 16u;
    const uint32_t a = hdr.y >> sh, c = hdr.w >> sh;
    if (g < 2u) {
        sc1 = a & 63u;
        sc2 = (a >> 8) & 63u;
    } else {
        sc1 = (c & 0xFu) | ((a >> 2) & 0x30u);
        sc2 = ((c >> 8) & 0xFu) | ((a >> 10) & 0x30u);
    }
}

// B operand of scale_products for a Q4_K sub-block: slot k (k < 6) holds
// d * 2^k if bit k of the 6-bit scale is set, else 0, so the slots sum to
// d * sc exactly. d2[t] = (d * 4^t, d * 2 * 4^t) as f16 pairs.
// The bit masks come from a 64-entry LDS table (mmq_scale_masks), one read
// instead of six bit tests.
RFXQ_DEV u4_t q4k_scale_operand(const uint32_t d2[3], uint32_t sc, const u4_t* masks) {
    const u4_t m = masks[sc];
    return u4_t{d2[0] & m.x, d2[1] & m.y, d2[2] & m.z, 0u};
}

// masks[sc] for sc in [0, 64): f16 lane k of the three dwords is all ones
// when bit k of sc is set
RFXQ_DEV void mmq_fill_scale_masks(u4_t* masks) {
    const uint32_t sc = threadIdx.x;
    if (sc < 64u) {
        auto pair = [&](uint32_t k) {
            return ((sc >> k) & 1u ? 0xFFFFu : 0u) | ((sc >> (k + 1u)) & 1u ? 0xFFFF0000u : 0u);
        };
        masks[sc] = u4_t{pair(0), pair(2), pair(4), 0u};
    }
}

// Constant part of the centered Q4_K weights, c_s = 8*(d*sc_s) - dmin*m_s
// (w = d*sc*q - dmin*m = d*sc*(q - 8) + c), for the sub-blocks s = 2t + h,
// t = 0..3, that this lane feeds to the K=2 f32 MFMAs.
RFXQ_DEV void q4k_offsets(const u4_t hdr, uint32_t h, float c[4]) {
    const float d = f16_bits_to_f32(hdr.x), dmin = f16_bits_to_f32(hdr.x >> 16);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        // j = 2t + h; bytes: q[j] of scales 0-3 (hdr.y) or 4-7 (hdr.z), q[j+4], q[j-4]
        const uint32_t j = 2u * t + h;
        uint32_t sc, m;
        if (t < 2) {  // j < 4
            sc = (hdr.y >> (8u * j)) & 63u;
            m = (hdr.z >> (8u * j)) & 63u;
        } else {      // j >= 4, e = j - 4
            const uint32_t e = j - 4u;
            sc = ((hdr.w >> (8u * e)) & 0xFu) | (((hdr.y >> (8u * e + 6u)) & 3u) << 4);
            m = ((hdr.w >> (8u * e + 4u)) & 0xFu) | (((hdr.z >> (8u * e + 6u)) & 3u) << 4);
        }
        c[t] = 8.0f * (d * (float)sc) - dmin * (float)m;
    }
}

RFXQ_DEV u4_t nib_lo(u4_t v) { return v & 0x0F0F0F0Fu; }
RFXQ_DEV u4_t nib_hi(u4_t v) { return (v >> 4) & 0x0F0F0F0Fu; }
// bytes q in [0, 15] -> q - 8 as int8: q + 0x78 stays below 0x100 (no carry
// between bytes), and flipping bit 7 maps it to q - 8 in two's complement
RFXQ_DEV u4_t center8(u4_t q) { return (q + 0x78787878u) ^ 0x80808080u; }

// Q8_0: one 34-byte block (2-byte aligned, never read past its end); returns
// the lane's 16 quants (K half h) and the f16 bits of d.
RFXQ_DEV u4_t load_q8_0_half(const uint8_t* blk, uint32_t h, uint32_t& dbits) {
    const uintptr_t addr = reinterpret_cast<uintptr_t>(blk);
    const uint8_t* pa = reinterpret_cast<const uint8_t*>(addr & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(addr & 3u);
    const u4_t w0 = ld16_a4(pa), w1 = ld16_a4(pa + 16);
    uint32_t w8;
    if (sh) w8 = *reinterpret_cast<const uint32_t*>(pa + 32);
    else w8 = *reinterpret_cast<const uint16_t*>(blk + 32);
    dbits = (sh ? (w0.x >> 16) : w0.x) & 0xFFFFu;
    // qs dword j = bytes [2+4j, 6+4j) of the block; the lane needs j = 4h..4h+3,
    // i.e. dwords W0..W4 = w[4h .. 4h+4] of the dword-aligned read.
    const uint32_t W0 = h ? w1.x : w0.x, W1 = h ? w1.y : w0.y, W2 = h ? w1.z : w0.z, W3 = h ? w1.w : w0.w;
    const uint32_t W4 = h ? w8 : w1.x;
    u4_t q;
    if (sh) {
        q.x = W1;
        q.y = W2;
        q.z = W3;
        q.w = W4;
    } else {
        q.x = alignbyte(W1, W0, 2u);
        q.y = alignbyte(W2, W1, 2u);
        q.z = alignbyte(W3, W2, 2u);
        q.w = alignbyte(W4, W3, 2u);
    }
    return q;
}

RFXQ_DEV u4_t seg16_mmq(const uint8_t* pa, uint32_t o, uint32_t sh) {
    const u4_t v = ld16_a4(pa + o);
    const uint32_t e = *reinterpret_cast<const uint32_t*>(pa + o + 16);
    u4_t r;
    r.x = alignbyte(v.y, v.x, sh);
    r.y = alignbyte(v.z, v.y, sh);
    r.z = alignbyte(v.w, v.z, sh);
    r.w = alignbyte(e, v.w, sh);
    return r;
}

// Signed Q6_K codes (q6 - 32) of run t for the lane's 16 positions, from the
// ql segment (low or high nibbles) and the qh segment.
RFXQ_DEV u4_t q6_codes(u4_t ql, u4_t qh, uint32_t t) {
    const u4_t lo = (t & 2u) ? nib_hi(ql) : nib_lo(ql);
    const u4_t hb = ((qh >> (2u * t)) & 0x03030303u) << 4;
    return (((lo | hb) | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

RFXQ_DEV int sbyte(uint32_t w, uint32_t byte) { return (int)(int8_t)(w >> (8u * byte)); }

// MI: 32-row MFMA tiles per wave along M (the workgroup tile is 64*MI x 128).
template <uint32_t TY, bool DOTS, int MI>
RFXQ_DEV void mmq_tile(const MmqDesc& ds, uint32_t t_local, float* lds_da, float* lds_sx, u4_t* lds_masks) {
    constexpr uint32_t BM = 64u * MI, WM = 32u * MI;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t wm = wave & 1u, wn = wave >> 1;
    const uint32_t h = lane >> 5, l32 = lane & 31u;
    const uint32_t lo_mask = h ? 0u : 0xFFFFFFFFu;  // scale-product K-slots live in lanes 0-31

    const uint32_t ks = t_local % ds.splits;
    const uint32_t rest = t_local / ds.splits;
    const uint32_t tm = rest % ds.tiles_m, tn = rest / ds.tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * MMQ_BN;
    if (TY == TY_Q4K && !DOTS) mmq_fill_scale_masks(lds_masks);  // ready after the first barrier
    const uint32_t nsb = ds.k / 256u;
    const uint32_t sb0 = ks * ds.sb_per_split;
    const uint32_t sb1 = min(nsb, sb0 + ds.sb_per_split);
    const uint32_t nkb = ds.k / 32u;
    const uint64_t row_bytes = TY == TY_Q4K ? (uint64_t)nsb * 144u : TY == TY_Q6K ? (uint64_t)nsb * 210u
                                                                                 : (uint64_t)nkb * 34u;

    const uint8_t* arow[MI];
#pragma unroll
    for (int i = 0; i < MI; i++) {
        uint32_t m = m0 + WM * wm + 32u * i + l32;
        m = m < ds.m ? m : ds.m - 1u;
        const uint32_t src = ds.rows ? (uint32_t)ds.rows[m] : m;
        arow[i] = reinterpret_cast<const uint8_t*>(ds.xq) + (uint64_t)src * ds.ldq + 16u * h;
    }
    const uint8_t* brow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        uint32_t n = n0 + 64u * wn + 32u * j + l32;
        n = n < ds.n ? n : ds.n - 1u;
        brow[j] = ds.w + (uint64_t)n * row_bytes;
    }
    // activation-scale staging: BM rows x 2 halves of a super-block's 8 blocks
    constexpr int ST = (2 * BM + 255) / 256;
    const uint32_t* st_src[ST];
#pragma unroll
    for (int q = 0; q < ST; q++) {
        const uint32_t r2 = tid + 256u * q;
        uint32_t m = m0 + (r2 >> 1);
        m = m < ds.m ? m : ds.m - 1u;
        const uint32_t src = ds.rows ? (uint32_t)ds.rows[m] : m;
        st_src[q] = ds.xds + (uint64_t)src * nkb + 4u * (r2 & 1u);
    }

    v16f_t acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = v16f_t{};

    // Software pipeline: the activation operands of the next block pair (and,
    // for Q4_K, its weight quants and the next super-block's header) are
    // loaded while the current pair's MFMAs and epilogue run.
    u4_t a_nx[2][MI], qv_nx[2], hdr_nx[2];
    auto load_a = [&](uint32_t sbx, uint32_t gx, u4_t a[2][MI]) {
#pragma unroll
        for (int e = 0; e < 2; e++)
#pragma unroll
            for (int i = 0; i < MI; i++) a[e][i] = ld16(arow[i] + 256u * sbx + 32u * (2u * gx + e));
    };
    // Q4_K quants of group gx: 16 bytes [16h, +16)
    auto load_q4 = [&](uint32_t sbx, uint32_t gx, u4_t q[2]) {
#pragma unroll
        for (int j = 0; j < 2; j++) q[j] = ld16(brow[j] + (uint64_t)sbx * 144u + 16u + 32u * gx + 16u * h);
    };
    if (sb0 < sb1) {
        load_a(sb0, 0u, a_nx);
        if (TY == TY_Q4K) {
            load_q4(sb0, 0u, qv_nx);
#pragma unroll
            for (int j = 0; j < 2; j++) hdr_nx[j] = ld16(brow[j] + (uint64_t)sb0 * 144u);
        }
    }

    for (uint32_t sb = sb0; sb < sb1; sb++) {
        // ---- activation scales of the tile's 128 rows: da as f32 [s][row], s_a as f16 [row][s]
#pragma unroll
        for (int q = 0; q < ST; q++) {
            const uint32_t r2 = tid + 256u * q;
            if (r2 >= 2u * BM) break;
            const uint32_t st_r = r2 >> 1, st_part = r2 & 1u;
            const u4_t v = *reinterpret_cast<const u4_t*>(st_src[q] + 8u * sb);
            lds_da[(4u * st_part + 0u) * BM + st_r] = f16_bits_to_f32(v.x);
            lds_da[(4u * st_part + 1u) * BM + st_r] = f16_bits_to_f32(v.y);
            lds_da[(4u * st_part + 2u) * BM + st_r] = f16_bits_to_f32(v.z);
            lds_da[(4u * st_part + 3u) * BM + st_r] = f16_bits_to_f32(v.w);
            // block activation sums d * s (s = sum(x)/d in f16), f32 [row][s]
            float4 sx;
            sx.x = f16_bits_to_f32(v.x) * f16_bits_to_f32(v.x >> 16);
            sx.y = f16_bits_to_f32(v.y) * f16_bits_to_f32(v.y >> 16);
            sx.z = f16_bits_to_f32(v.z) * f16_bits_to_f32(v.z >> 16);
            sx.w = f16_bits_to_f32(v.w) * f16_bits_to_f32(v.w >> 16);
            *reinterpret_cast<float4*>(lds_sx + st_r * 8u + 4u * st_part) = sx;
        }
        __syncthreads();

        u4_t hdr[2];
        uint32_t q6sh[2];
        const uint8_t* q6pa[2];
        uint32_t q6sc[2][4];
        uint32_t q6dbits[2];
        if (TY == TY_Q4K) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                hdr[j] = hdr_nx[j];
                if (sb + 1u < sb1) hdr_nx[j] = ld16(brow[j] + (uint64_t)(sb + 1u) * 144u);
            }
        } else if (TY == TY_Q6K) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint8_t* blk = brow[j] + (uint64_t)sb * 210u;
                const uintptr_t addr = reinterpret_cast<uintptr_t>(blk);
                q6pa[j] = reinterpret_cast<const uint8_t*>(addr & ~(uintptr_t)3);
                q6sh[j] = (uint32_t)(addr & 3u);
                const u4_t sw = ld16_a4(q6pa[j] + 192);
                uint32_t tail;
                if (q6sh[j]) tail = *reinterpret_cast<const uint32_t*>(q6pa[j] + 208);
                else tail = *reinterpret_cast<const uint16_t*>(blk + 208);
                q6sc[j][0] = alignbyte(sw.y, sw.x, q6sh[j]);
                q6sc[j][1] = alignbyte(sw.z, sw.y, q6sh[j]);
                q6sc[j][2] = alignbyte(sw.w, sw.z, q6sh[j]);
                q6sc[j][3] = alignbyte(tail, sw.w, q6sh[j]);
                q6dbits[j] = (q6sh[j] ? (tail >> 16) : tail) & 0xFFFFu;
            }
        }

        // B operands of the scale products (lanes 32-63 carry zero K-slots)
        uint32_t d2[2][3];  // Q4_K: (d, 2d), (4d, 8d), (16d, 32d) as f16 pairs
#pragma unroll
        for (int j = 0; j < 2; j++) {
            if (TY == TY_Q4K) {
                const float d = f16_bits_to_f32(hdr[j].x);
#pragma unroll
                for (int t = 0; t < 3; t++) {
                    const h2_t v = {(half_t)(d * (float)(1u << (2 * t))), (half_t)(d * (float)(2u << (2 * t)))};
                    d2[j][t] = h2_bits(v) & lo_mask;
                }
            }
        }

#pragma unroll 1
        for (uint32_t g = 0; g < 4; g++) {
            // this step's prefetched operands; issue the next step's loads
            u4_t a_cur[2][MI], qv_cur[2];
#pragma unroll
            for (int e = 0; e < 2; e++)
#pragma unroll
                for (int i = 0; i < MI; i++) a_cur[e][i] = a_nx[e][i];
#pragma unroll
            for (int j = 0; j < 2; j++) qv_cur[j] = qv_nx[j];
            {
                const bool last_g = g == 3u;
                const uint32_t sbn = last_g ? sb + 1u : sb, gn = last_g ? 0u : g + 1u;
                if (sbn < sb1) {
                    load_a(sbn, gn, a_nx);
                    if (TY == TY_Q4K) load_q4(sbn, gn, qv_nx);
                }
            }
            // per 32-block pair (2g, 2g+1): B operands and weight scales
            u4_t bw[2][2];
            uint32_t wsb[2][2];  // Q4_K: 6-bit sub-block scale; Q6_K / Q8_0: f16 bits of d
            int scl[2][2], sch[2][2];  // Q6_K: scales of the two 16-runs
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if (TY == TY_Q4K) {
                    const u4_t qv = qv_cur[j];
                    bw[j][0] = center8(nib_lo(qv));
                    bw[j][1] = center8(nib_hi(qv));
                    q4k_pair_sc(hdr[j], g, wsb[j][0], wsb[j][1]);
                } else if (TY == TY_Q6K) {
                    const uint32_t n = g >> 1, t0 = 2u * (g & 1u);
                    const u4_t qla = seg16_mmq(q6pa[j], 64u * n + 16u * h, q6sh[j]);
                    const u4_t qlc = seg16_mmq(q6pa[j], 64u * n + 32u + 16u * h, q6sh[j]);
                    const u4_t qh = seg16_mmq(q6pa[j], 128u + 32u * n + 16u * h, q6sh[j]);
                    bw[j][0] = q6_codes(qla, qh, t0);
                    bw[j][1] = q6_codes(qlc, qh, t0 + 1u);
                    // scales sc[8n + hh + 2t]: dword (2n + (t>>1)), byte (hh + 2(t&1))
                    const uint32_t wv = n ? (g & 1u ? q6sc[j][3] : q6sc[j][2]) : (g & 1u ? q6sc[j][1] : q6sc[j][0]);
                    scl[j][0] = sbyte(wv, 0);
                    sch[j][0] = sbyte(wv, 1);
                    scl[j][1] = sbyte(wv, 2);
                    sch[j][1] = sbyte(wv, 3);
                    wsb[j][0] = q6dbits[j];
                    wsb[j][1] = q6dbits[j];
                } else {
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        bw[j][e] = load_q8_0_half(brow[j] + (uint64_t)(8u * sb + 2u * g + e) * 34u, h, wsb[j][e]);
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const uint32_t s = 2u * g + e;
                v4i_t a[MI];
#pragma unroll
                for (int i = 0; i < MI; i++) a[i] = as_v4i(a_cur[e][i]);
                // scale-product A operands: each row tile's activation scale
                // (f16), in slots 0-5 for Q4_K (against d * 2^k), slot 0 otherwise
                u4_t sa[MI];
#pragma unroll
                for (int i = 0; i < MI; i++) {
                    sa[i] = u4_t{0u, 0u, 0u, 0u};
                    if (!DOTS) {
                        const float da = lds_da[s * BM + WM * wm + 32u * i + l32];
                        const uint32_t dab = (uint32_t)__builtin_bit_cast(uint16_t, (half_t)da) & lo_mask;
                        if (TY == TY_Q4K) {
                            const uint32_t p = h2_dup(dab);
                            sa[i] = u4_t{p, p, p, 0u};
                        } else {
                            sa[i].x = dab;
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    u4_t sbo = {};
                    if (!DOTS)
                        sbo = TY == TY_Q4K ? q4k_scale_operand(d2[j], wsb[j][e], lds_masks)
                                           : u4_t{wsb[j][e] & lo_mask, 0u, 0u, 0u};
#pragma unroll
                    for (int i = 0; i < MI; i++) {
                        v16i_t D;
                        if (TY == TY_Q6K) {
                            const u4_t z = {0u, 0u, 0u, 0u};
                            const v16i_t D0 = mfma_i8(a[i], as_v4i(h ? z : bw[j][e]));
                            const v16i_t D1 = mfma_i8(a[i], as_v4i(h ? bw[j][e] : z));
#pragma unroll
                            for (int r = 0; r < 16; r++) D[r] = D0[r] * scl[j][e] + D1[r] * sch[j][e];
                        } else {
                            D = mfma_i8(a[i], as_v4i(bw[j][e]));
                        }
                        if (DOTS) {
                            const uint32_t col = n0 + 64u * wn + 32u * j + l32;
#pragma unroll
                            for (int r = 0; r < 16; r++) {
                                const uint32_t row = m0 + WM * wm + 32u * i + 8u * (r >> 2) + 4u * h + (r & 3);
                                if (row < ds.m && col < ds.n)
                                    ds.dots_out[((uint64_t)row * ds.n + col) * nkb + 8u * sb + s] =
                                        D[r];
                            }
                        } else {
                            const v16f_t S = scale_products(sa[i], sbo);
#pragma unroll
                            for (int r = 0; r < 16; r++)
                                acc[i][j][r] = fmaf((float)D[r], S[r], acc[i][j][r]);
                        }
                    }
                }
            }
        }
        if (TY == TY_Q4K && !DOTS) {
            // constant part: acc += sum_s Sx[m,s] * c_s[n] over this super-block,
            // as four K=2 f32 MFMAs (lane half h carries sub-blocks 2t + h)
            float cw[2][4];
#pragma unroll
            for (int j = 0; j < 2; j++) q4k_offsets(hdr[j], h, cw[j]);
#pragma unroll
            for (int i = 0; i < MI; i++) {
                const float* sxp = lds_sx + (WM * wm + 32u * i + l32) * 8u + h;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const float sx = sxp[2 * t];
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(sx, cw[j][t], acc[i][j], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }

    if (DOTS) return;
    float* y = ds.y + (uint64_t)ks * ds.m * ds.ldy;
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t col = n0 + 64u * wn + 32u * j + l32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = m0 + WM * wm + 32u * i + 8u * (r >> 2) + 4u * h + (r & 3);
                if (row < ds.m && col < ds.n) y[(uint64_t)row * ds.ldy + col] = acc[i][j][r];
            }
        }
}

// The descriptor of workgroup `wg`: the last one whose wg_begin is at or
// below it (descriptors with no tiles share the next one's wg_begin and are
// skipped). A workgroup past the last descriptor's tiles (launch grids that
// are upper bounds, for tables built on the device) returns at once.
// Workgroups the descriptors of a launch use (the last one's end)
RFXQ_DEV uint32_t mmq_tile_count(const MmqArgs& a) {
    const MmqDesc* l = (a.ndesc <= MMQ_INLINE ? a.inl : a.table) + (a.ndesc - 1u);
    return __builtin_amdgcn_readfirstlane(l->wg_begin + l->tiles_m * l->tiles_n * l->splits);
}

RFXQ_DEV MmqDesc mmq_pick(const MmqArgs& a, uint32_t wg) {
    if (a.ndesc <= MMQ_INLINE) {
        MmqDesc d = a.inl[0];
        if (a.ndesc > 1 && wg >= a.inl[1].wg_begin) d = a.inl[1];
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

// The GEMM kernels are held to 2 waves per SIMD (no spills at this budget) so
// that one wave's epilogue overlaps another's MFMAs and loads; the block-dot
// test hooks keep the default budget. (MI = 4, 256-row tiles, needs more than
// the 256 registers of 2 waves per SIMD and spills.)
#define RFXQ_MMQ_ENTRY(NAME, TY, DOTS, WPE, MI)                              \
    extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE))) void NAME(MmqArgs args) { \
        __shared__ float lds_da[8 * 64 * MI];                                 \
        __shared__ float lds_sx[64 * MI * 8];                                 \
        __shared__ u4_t lds_masks[64];                                        \
        const MmqDesc d = mmq_pick(args, blockIdx.x);                         \
        if (blockIdx.x - d.wg_begin >= d.tiles_m * d.tiles_n * d.splits) return; \
        mmq_tile<TY, DOTS, MI>(d, blockIdx.x - d.wg_begin, lds_da, lds_sx, lds_masks); \
    }
RFXQ_MMQ_ENTRY(rfxq_mmq_q4k, TY_Q4K, false, 2, 2)
RFXQ_MMQ_ENTRY(rfxq_mmq_q6k, TY_Q6K, false, 2, 2)
RFXQ_MMQ_ENTRY(rfxq_mmq_q8_0, TY_Q8_0, false, 2, 2)
// 64-row tiles for short row groups (MoE experts at tens of rows each)
RFXQ_MMQ_ENTRY(rfxq_mmq_q4k_m64, TY_Q4K, false, 2, 1)
RFXQ_MMQ_ENTRY(rfxq_mmq_q6k_m64, TY_Q6K, false, 2, 1)
RFXQ_MMQ_ENTRY(rfxq_mmq_q8_0_m64, TY_Q8_0, false, 2, 1)
RFXQ_MMQ_ENTRY(rfxq_mmq_dots_q4k, TY_Q4K, true, 1, 2)
RFXQ_MMQ_ENTRY(rfxq_mmq_dots_q6k, TY_Q6K, true, 1, 2)
RFXQ_MMQ_ENTRY(rfxq_mmq_dots_q8_0, TY_Q8_0, true, 1, 2)

// y[i] = sum_z ws[z][i], added in split order (deterministic).
extern "C" __global__ __launch_bounds__(256) void rfxq_splitk_reduce(const float* __restrict__ ws,
                                                                    float* __restrict__ y, uint64_t n,
                                                                    uint32_t splits) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256u) {
        float s = ws[i];
        // eight loads in flight per round trip, added in split order
        for (uint32_t z0 = 1; z0 < splits; z0 += 8u) {
            float v[8];
#pragma unroll
            for (uint32_t u = 0; u < 8u; u++) v[u] = z0 + u < splits ? ws[(uint64_t)(z0 + u) * n + i] : 0.0f;
#pragma unroll
            for (uint32_t u = 0; u < 8u; u++)
                if (z0 + u < splits) s += v[u];
        }
        y[i] = s;
    }
}

// Several split-K reduces in one launch: item i takes workgroups
// [wg_begin, next item's wg_begin) and sums its splits as rfxq_splitk_reduce.
struct ReduceItem {
    const float* ws;
    float* y;
    uint32_t n, splits, wg_begin, wgs;
};
#define REDUCE_INLINE 32
struct ReduceArgs {
    uint32_t count, pad;
    ReduceItem items[REDUCE_INLINE];
};

extern "C" __global__ __launch_bounds__(256) void rfxq_splitk_reduce_multi(ReduceArgs a) {
    uint32_t it = 0;
    for (uint32_t j = 1; j < a.count; j++)
        if (a.items[j].wg_begin <= blockIdx.x) it = j;
    const ReduceItem r = a.items[it];
    const uint64_t n = r.n;
    for (uint64_t i = (uint64_t)(blockIdx.x - r.wg_begin) * 256u + threadIdx.x; i < n; i += (uint64_t)r.wgs * 256u) {
        float s = r.ws[i];
        for (uint32_t z0 = 1; z0 < r.splits; z0 += 8u) {
            float v[8];
#pragma unroll
            for (uint32_t u = 0; u < 8u; u++) v[u] = z0 + u < r.splits ? r.ws[(uint64_t)(z0 + u) * n + i] : 0.0f;
#pragma unroll
            for (uint32_t u = 0; u < 8u; u++)
                if (z0 + u < r.splits) s += v[u];
        }
        r.y[i] = s;
    }
}
