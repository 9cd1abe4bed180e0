// Prefill GEMM Y = X . W^T on f16 MFMAs with f16 activations: the default
// kernels of the MMQ path for Q4_K and Q6_K weights (they replace the
// reference's gemm_q_mma_impl, src/kernels_cuda/gemm_q_mma.cu:299-764, at the
// same call sites: Model::gemm, kernels.rs:2197).
//
// Activations (written by rfxq_act_f16 or a fused producer, quant.hpp):
//   xh  [rows][k] f16 = x * 2^-e_row, rounded to nearest even; within each
//       group of four the values are stored (x0, x2), (x1, x3)
//   xsx [rows][k/256] records of 16 f16: Sx_b = sum of block b's 32 xh
//       values (f32, fixed order) as hi[8] = f16(Sx), lo[8] = f16(Sx - hi)
//   xrs [rows] f32 = 2^e_row, with e_row = ilogb(max |x_row|) - 8, so every
//       row's largest value lands in [256, 512): no f16 overflow for any
//       finite activation, and no subnormals above 2^-22 of the row maximum.
//
// Q4_K (src/dequant.rs:339-367): w = d*sc_b*q - dmin*m_b for the 6-bit
// (sc_b, m_b) of 32-block b and 4-bit codes q. Written as
//   w = d*sc_b*(q - 8) + C_b,     C_b = 8*d*sc_b - dmin*m_b,
//   y[i,j] = 2^e_j * ( sum_k xh[j,k] * f16(d*sc_b*(q-8)) + sum_b C_b * Sx_b[j] ).
// The weight operand f16(16*(q - 8) * f16(d*sc_b/16)) is built from the
// nibble by an and-or into the mantissa of an f16 1024.0 (1024 + 16q), an
// exact add of -1152, and one multiply. The constant part is one 32x32x16
// f16 MFMA per super-block (K slots: C_0..7 against Sx hi, C_0..7 against
// Sx lo). Everything accumulates in one f32 accumulator in the matrix core:
// no per-block or per-super-block epilogue on the VALU.
//
// Q4_K tile: 128 activation rows x 256 weight columns per 256-thread
// workgroup (two per CU); wave w owns weight columns [64w, +64) against all
// 128 rows: eight 32x32 MFMA tiles, A = weights, B = activations (lane l holds
// activation row l%32 of its tile and 16 weight columns), so each activation
// operand read from LDS feeds two MFMAs and each converted weight operand
// four. Data moves in 64-k stages through a 2-slot LDS ring: activations
// [128][64] f16 (16 KB, 16-byte chunks XOR-swizzled by row/2) and weight
// quants [256][32 B] (8 KB, halves swizzled by column/8), plus the super-block
// headers [256][16 B] and Sx records [128][32 B] with the first stage of a
// super-block (56 KB). Every lane loads its share of stage s + 1 into
// registers with plain buffer loads while stage s computes, in two halves
// written to the other slot at mid-stage and at its end; one barrier per
// stage. (The LDS-DMA path, buffer_load ... lds, measured slower here: it
// throttles the MFMA stream of the same CU.) Activation rows are gathered
// through MmqDesc::rows when set (MoE expert groups).
//
// Q6_K tile: 128 x 128 per 256-thread workgroup with a 3-slot LDS-DMA ring
// (see the Q6_K section below).
#pragma once
#include "common.hpp"
#include "mmq.hpp"

namespace mmqh {

constexpr uint32_t BM = 128, BN = 256, kThreads = 256;
constexpr uint32_t kAct = 16384, kCodes = 8192;
constexpr uint32_t kSlot = kAct + kCodes;
constexpr uint32_t kHdr = 4096, kSx = 4096;
constexpr uint32_t kLds = 2 * kSlot + kHdr + kSx;
static_assert(kLds <= 81920, "two workgroups per CU");

// f16 of an f32, round to nearest even, as the low 16 bits
RFXQ_DEV uint32_t f16_rne(float v) { return __builtin_bit_cast(uint16_t, (half_t)v); }
RFXQ_DEV uint32_t pack16(uint32_t lo, uint32_t hi) { return (lo & 0xFFFFu) | (hi << 16); }

// the 6-bit scales and mins of sub-blocks 0..7 (get_scale_min_k4,
// src/dequant.rs:39-47) from header dwords y, z, w (bytes 4..15)
RFXQ_DEV void q4k_scales_mins(const u4_t hdr, float (&sc)[8], float (&mn)[8]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        sc[j] = (float)((hdr.y >> (8 * j)) & 63u);
        mn[j] = (float)((hdr.z >> (8 * j)) & 63u);
        sc[j + 4] = (float)(((hdr.w >> (8 * j)) & 0xFu) | (((hdr.y >> (8 * j + 6)) & 3u) << 4));
        mn[j + 4] = (float)(((hdr.w >> (8 * j + 4)) & 0xFu) | (((hdr.z >> (8 * j + 6)) & 3u) << 4));
    }
}

// Per super-block operands of one weight column: the constant-part A operand
// (C_0..7 as f16 pairs) and the eight block multipliers f16(d*sc_b/16),
// packed two per dword (block 2p low, 2p + 1 high).
RFXQ_DEV void q4k_sb_operands(const u4_t hdr, u4_t& cop, u4_t& dsc) {
    float sc[8], mn[8];
    q4k_scales_mins(hdr, sc, mn);
    const float d = f16_bits_to_f32(hdr.x), dmin = f16_bits_to_f32(hdr.x >> 16);
    uint32_t c[8], s[8];
#pragma unroll
    for (int b = 0; b < 8; b++) {
        c[b] = f16_rne(__builtin_fmaf(8.0f * d, sc[b], -(dmin * mn[b])));
        s[b] = f16_rne(d * sc[b] * 0.0625f);
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {
        cop[p] = pack16(c[2 * p], c[2 * p + 1]);
        dsc[p] = pack16(s[2 * p], s[2 * p + 1]);
    }
}

// (v, v) from the low (H = 0) or high (H = 1) f16 of a dword
template <int H>
RFXQ_DEV uint32_t splat16(uint32_t v) {
    return __builtin_amdgcn_perm(v, v, H ? 0x03020302u : 0x01000100u);
}

// Weight operand of one 16-k step: codes of block E (0: low nibbles, 1: high)
// of the step's two quant dwords, as f16 pairs f16(16*(q - 8) * s) in the
// activations' (q0, q2), (q1, q3) order. 16*(q - 8) is exact in f16, so the
// multiply is the only rounding.
template <int E>
RFXQ_DEV u4_t q4k_codes_f16(uint32_t v0, uint32_t v1, uint32_t s) {
    const uint32_t M = 0x00F000F0u, MG = 0x64006400u;
    uint32_t w[4];
    if (E == 0) {
        w[0] = ((v0 << 4) & M) | MG;
        w[1] = ((v0 >> 4) & M) | MG;
        w[2] = ((v1 << 4) & M) | MG;
        w[3] = ((v1 >> 4) & M) | MG;
    } else {
        w[0] = (v0 & M) | MG;
        w[1] = ((v0 >> 8) & M) | MG;
        w[2] = (v1 & M) | MG;
        w[3] = ((v1 >> 8) & M) | MG;
    }
    const h2_t off = {(half_t)-1152.0f, (half_t)-1152.0f};
    const h2_t sv = as_h2(s);
    u4_t r;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        h2_t c = as_h2(w[t]) + off;
        asm("" : "+v"(c));  // keep the exact add and the rounding multiply apart (no fma)
        r[t] = h2_bits(c * sv);
    }
    return r;
}

// Activation row read for output row r: rows past the matrix read the last
// row (their results are not stored), and a gathered GEMM (MoE expert groups)
// reads the source row rows[r].
RFXQ_DEV uint32_t act_row(const MmqDesc& ds, uint32_t r) {
    r = r < ds.m ? r : ds.m - 1u;
    return ds.rows ? (uint32_t)ds.rows[r] : r;
}

// y rows of one 32-row activation tile: acc[r] is weight column
// 8*(r/4) + 4*h + r%4 of the 32-column tile starting at c_base
RFXQ_DEV void store_tile(const MmqDesc& ds, float* y, uint32_t row, uint32_t c_base, uint32_t h, const v16f_t& acc,
                         float scale, bool vec) {
    if (row >= ds.m) return;
    float* yr = y + (uint64_t)row * ds.ldy;
#pragma unroll
    for (int q4 = 0; q4 < 4; q4++) {
        const uint32_t c0 = c_base + 8u * q4 + 4u * h;
        const float a0 = acc[4 * q4] * scale, a1 = acc[4 * q4 + 1] * scale;
        const float a2 = acc[4 * q4 + 2] * scale, a3 = acc[4 * q4 + 3] * scale;
        if (vec && c0 + 3u < ds.n) {
            *reinterpret_cast<float4*>(yr + c0) = make_float4(a0, a1, a2, a3);
        } else {
            if (c0 < ds.n) yr[c0] = a0;
            if (c0 + 1u < ds.n) yr[c0 + 1u] = a1;
            if (c0 + 2u < ds.n) yr[c0 + 2u] = a2;
            if (c0 + 3u < ds.n) yr[c0 + 3u] = a3;
        }
    }
}

// Asynchronous copies global -> LDS (buffer_load ... lds): lane l's 16 (4)
// bytes land at lds + 16l (4l). Issued from inline asm so that the compiler
// does not see LDS writes in flight: its own LDS reads then need no vmcnt
// waits, and the ring is ordered by the explicit vmcnt waits and barriers
// of the main loop. M0 (the LDS base) is saved and restored around the copy.
typedef uint32_t sdesc_t __attribute__((ext_vector_type(4)));
RFXQ_DEV void dma16(sdesc_t r, uint32_t lds, uint32_t voff, uint32_t soff) {
    uint32_t keep;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
        : "=&s"(keep)
        : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(r), "s"(__builtin_amdgcn_readfirstlane(soff))
        : "memory");
}
RFXQ_DEV void dma4(sdesc_t r, uint32_t lds, uint32_t voff, uint32_t soff) {
    uint32_t keep;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dword %2, %3, %4 offen lds\n\ts_mov_b32 m0, %0"
        : "=&s"(keep)
        : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(r), "s"(__builtin_amdgcn_readfirstlane(soff))
        : "memory");
}

// raw buffer descriptor (base, stride 0, num_records = bytes) in SGPRs:
// offsets at or past `bytes` read zeros
RFXQ_DEV sdesc_t uniform_desc(const void* p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uintptr_t>(p);
    return sdesc_t{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
                   (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)),
                   (uint32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000u};
}

RFXQ_DEV uint32_t bperm(uint32_t lane, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute((int)(lane << 2), (int)v);
}

// an f16 value as f32 in a register, hidden from instruction selection (which
// would otherwise fold the conversion back into every v_fma_mix_f32)
RFXQ_DEV float f16_opaque(uint32_t bits16) {
    float f = f16_bits_to_f32(bits16);
    asm("" : "+v"(f));
    return f;
}

RFXQ_DEV v16f_t mfma16(u4_t a, u4_t b, v16f_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(as_h8(a), as_h8(b), c, 0, 0, 0);
}

// ---------------------------------------------------------------- Q6_K
//
// A Q6_K super-block (ql[128], qh[64], scales[16] i8, d; src/dequant.rs:414-445)
// has no constant part: w = d * sc * (q - 32), with one scale per 16 codes.
// The scale goes into the weight operand, but sc*(q - 32) reaches 4096 in
// magnitude and needs 12 significant bits, one more than f16 holds; split by
// the code's low bit, q - 32 = (q & ~1) - 32 + (q & 1):
//   hi = sc * ((q & ~1) - 32)   (even, |hi| <= 4096: exact in f16)
//   lo = sc * (q & 1)           (|lo| <= 128)
// Both operands are exact, so the four chained 32x32x16 f16 MFMAs of a
// 32-block add exact products of f16 activations and the exact weights
// sc*(q - 32) into the super-block accumulator t; per super-block y += d * t,
// and the row scale 2^e at the end.
//
// A 64-k stage g = 2n + s of a super-block takes blocks A = 4n + s (low
// nibbles of ql[64n + 32s + l], qh[32n + l] bits 2s..2s+1) and B = A + 2
// (high nibbles, bits 2s+4..2s+5), l in [0, 32); lane half h holds positions
// l in [16h, 16h + 16), whose scales are sc[8n + 2s + h] (A) and
// sc[8n + 4 + 2s + h] (B). Blocks are 210 bytes, so a super-block starts at
// a 2-byte offset when its index is odd (rows are 4-byte aligned: the host
// requires an even super-block count per row): the ql and qh ranges are
// copied as 9-dword windows from the aligned address below and realigned
// with v_alignbyte after the LDS read.

// Q6_K kernel: 128x128 tiles; per LDS slot activations [128][64] f16 and the
// code windows [128][72 B]; headers [128][20 B]
constexpr uint32_t kBM6 = 128, kBN6 = 128;
constexpr uint32_t kCodes6 = 128u * 18u * 4u;
constexpr uint32_t kHdr6 = 128u * 5u * 4u;

// hi and lo operands of one 16-k step of block E (0: A, low nibbles; 1: B,
// high nibbles) from the step's ql dwords l0, l1 and qh dwords q0, q1 (code
// positions p..p+7): (q & ~1) << 4 and (q & 1) << 4 are placed in the
// mantissa of an f16 1024.0, then (1024 + 16x) * (sc/16) + off gives
// sc*(x - 32) with off = -96 sc (hi) and sc*x with off = -64 sc (lo), exact.
// tab = (sc/16, -96 sc, -64 sc) as f16 pairs. Pairs follow the activations'
// (p0, p2), (p1, p3) order.
template <int E, int S>
RFXQ_DEV void q6k_step_codes(uint32_t l0, uint32_t l1, uint32_t q0, uint32_t q1, const u4_t tab, u4_t& hi, u4_t& lo) {
    const uint32_t MH = 0x00E000E0u, MQ = 0x03000300u, ML = 0x00100010u, MG = 0x64006400u;
    uint32_t mh[4], ml[4];
    const uint32_t ls[2] = {l0, l1}, qs[2] = {q0, q1};
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t L = ls[u], Q = qs[u];
        uint32_t m02, m13, h02, h13;
        if (E == 0) {
            m02 = L << 4;
            m13 = L >> 4;
            h02 = Q << (8 - 2 * S);
            h13 = Q >> (2 * S);
        } else {
            m02 = L;
            m13 = L >> 8;
            h02 = Q << (4 - 2 * S);
            h13 = Q >> (2 * S + 4);
        }
        mh[2 * u] = (m02 & MH) | (h02 & MQ) | MG;
        mh[2 * u + 1] = (m13 & MH) | (h13 & MQ) | MG;
        ml[2 * u] = (m02 & ML) | MG;
        ml[2 * u + 1] = (m13 & ML) | MG;
    }
    const h2_t s = as_h2(tab.x), oh = as_h2(tab.y), ol = as_h2(tab.z);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        hi[t] = h2_bits(__builtin_elementwise_fma(as_h2(mh[t]), s, oh));
        lo[t] = h2_bits(__builtin_elementwise_fma(as_h2(ml[t]), s, ol));
    }
}

// (sc/16, -96 sc, -64 sc) of a signed 8-bit scale, each as an f16 pair
RFXQ_DEV u4_t q6k_tab(int sc) {
    const float f = (float)sc;
    const half_t a = (half_t)(f * 0.0625f), b = (half_t)(f * -96.0f), c = (half_t)(f * -64.0f);
    const h2_t s = {a, a}, oh = {b, b}, ol = {c, c};
    return u4_t{h2_bits(s), h2_bits(oh), h2_bits(ol), 0u};
}

// the weight operands of stage s of a half: [block][step] hi and lo
template <int S>
RFXQ_DEV void q6k_stage_operands(const uint32_t* V, const uint32_t* H, const u4_t tabA, const u4_t tabB,
                                 u4_t (&hi)[2][2], u4_t (&lo)[2][2]) {
#pragma unroll
    for (int st = 0; st < 2; st++) {
        q6k_step_codes<0, S>(V[2 * st], V[2 * st + 1], H[2 * st], H[2 * st + 1], tabA, hi[0][st], lo[0][st]);
        q6k_step_codes<1, S>(V[2 * st], V[2 * st + 1], H[2 * st], H[2 * st + 1], tabB, hi[1][st], lo[1][st]);
    }
}

constexpr uint32_t kSlotQ6 = kAct + kCodes6;
constexpr uint32_t kLdsQ6 = 3u * kSlotQ6 + kHdr6;

}  // namespace mmqh


// One 128x256 tile (and one split-K range) of Y = X . W^T for Q4_K weights.
RFXQ_DEV void mmqh_q4k_tile(const MmqDesc& dv, uint32_t t_local, uint8_t* lds) {
    using namespace mmqh;
    MmqDesc ds = dv;
    {
        uint32_t* p = reinterpret_cast<uint32_t*>(&ds);
#pragma unroll
        for (uint32_t i = 0; i < sizeof(MmqDesc) / 4u; i++) p[i] = __builtin_amdgcn_readfirstlane(p[i]);
        t_local = __builtin_amdgcn_readfirstlane(t_local);
    }
    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, h = lane >> 5;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);

    const uint32_t ks = t_local % ds.splits;
    const uint32_t rest = t_local / ds.splits;
    const uint32_t tm = rest % ds.tiles_m, tn = rest / ds.tiles_m;
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t nsb = ds.k / 256u;
    const uint32_t sb0 = ks * ds.sb_per_split;
    const uint32_t sb1 = min(nsb, sb0 + ds.sb_per_split);
    const uint32_t row_bytes = nsb * 144u;
    const uint32_t rec_bytes = nsb * 32u;
    uint8_t* const hdr_lds = lds + 2u * kSlot;
    uint8_t* const sx_lds = hdr_lds + kHdr;

    // Weight columns past the matrix read past the buffer: zeros, no fault.
    // Activation rows are clamped or gathered (act_row): always in bounds.
    const rsrc_t r_act = make_rsrc(ds.xq, 0xFFFFFFFFu);
    const rsrc_t r_w = make_rsrc(ds.w, ds.n * row_bytes);
    const rsrc_t r_sx = make_rsrc(ds.xds, 0xFFFFFFFFu);
    // Staged pieces (stage 0 of super-block 0). Activations: piece
    // 256u + tid is chunk tid%8 of row 32u + tid/8 (LDS + 4096u); LDS chunk
    // c of row r holds logical chunk c ^ ((r/2)%8). Quants: piece 256u + tid
    // is half tid%2 of column 128u + tid/2 (LDS + 4096u), stored at half
    // (tid%2) ^ ((column/8)%2). Headers: column tid. Sx: half tid%2 of row tid/2.
    const uint32_t ra = tid >> 3, ca = tid & 7u;
    uint32_t g_act[4];
#pragma unroll
    for (int u = 0; u < 4; u++) g_act[u] = act_row(ds, m0 + ra + 32u * u) * ds.ldq + 16u * ca;
    const uint32_t l_act = ra * 128u + 16u * (ca ^ ((ra >> 1) & 7u));
    const uint32_t cq = tid >> 1, pq = tid & 1u;
    const uint32_t g_cod = (n0 + cq) * row_bytes + 16u + 16u * pq;
    const uint32_t l_cod = kAct + cq * 32u + 16u * (pq ^ ((cq >> 3) & 1u));
    const uint32_t g_hdr = (n0 + tid) * row_bytes;
    const uint32_t g_sx = act_row(ds, m0 + (tid >> 1)) * rec_bytes + 16u * (tid & 1u);
    const uint32_t nst = 4u * (sb1 - sb0);

    // the staged loads of a stage in two halves: activations u = 2H, 2H + 1
    // and quants u = H; the super-block headers and Sx records ride with
    // half 0 of its first stage
    u4_t sa[2], sq, shd, ssx;
    // Loads are issued unconditionally so that the compiler's wait counts stay
    // exact across the loop: past the last stage a lane reloads the last stage
    // (in bounds; its copy in LDS is never read).
    auto load_half = [&](uint32_t st, int H) {
        const uint32_t sl = min(st, nst - 1u);
        const uint32_t sb = sb0 + (sl >> 2), g = sl & 3u;
#pragma unroll
        for (int u = 0; u < 2; u++)
            sa[u] = __builtin_amdgcn_raw_buffer_load_b128(r_act, g_act[2 * H + u], 512u * sb + 128u * g, 0);
        sq = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_cod, 144u * sb + 32u * g + 128u * H * row_bytes, 0);
        if (H == 0 && (st & 3u) == 0u) {
            shd = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_hdr, 144u * sb, 0);
            ssx = __builtin_amdgcn_raw_buffer_load_b128(r_sx, g_sx, 32u * sb, 0);
        }
    };
    auto store_half = [&](uint32_t st, int H) {
        uint8_t* S = lds + (st & 1u) * kSlot;
#pragma unroll
        for (int u = 0; u < 2; u++) *reinterpret_cast<u4_t*>(S + l_act + 4096u * (2u * H + u)) = sa[u];
        *reinterpret_cast<u4_t*>(S + l_cod + 4096u * H) = sq;
        if (H == 0 && (st & 3u) == 0u) {
            reinterpret_cast<u4_t*>(hdr_lds)[tid] = shd;
            reinterpret_cast<u4_t*>(sx_lds)[tid] = ssx;
        }
    };

    v16f_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i][0] = acc[i][1] = v16f_t{};
    // LDS read offsets (16-byte units): activations of row l32 of row tile 0,
    // logical chunk 4e + 2h + step; quants and header of column 64w + 32j + l32
    uint32_t a_act[2][2];
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) a_act[e][s2] = l32 * 8u + ((4u * e + 2u * h + s2) ^ ((l32 >> 1) & 7u));
    uint32_t a_codes[2], col[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        col[j] = 64u * w + 32u * j + l32;
        a_codes[j] = kAct / 16u + 2u * col[j] + (h ^ ((col[j] >> 3) & 1u));
    }
    u4_t dsc[2] = {};

    if (nst > 0u) {
        load_half(0u, 0);
        store_half(0u, 0);
        load_half(0u, 1);
        store_half(0u, 1);
    }
    __syncthreads();
    for (uint32_t st0 = 0; st0 < nst; st0 += 4u) {
#pragma unroll
        for (uint32_t g = 0; g < 4u; g++) {
            const uint32_t st = st0 + g;
            load_half(st + 1u, 0);
            const u4_t* S16 = reinterpret_cast<const u4_t*>(lds + (st & 1u) * kSlot);
            if (g == 0u) {
                // super-block start: the columns' multipliers, and the
                // constant part C_b * Sx_b into the accumulators
                u4_t cop[2];
#pragma unroll
                for (int j = 0; j < 2; j++) q4k_sb_operands(reinterpret_cast<const u4_t*>(hdr_lds)[col[j]], cop[j], dsc[j]);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const u4_t sxo = reinterpret_cast<const u4_t*>(sx_lds)[2u * (32u * i + l32) + h];
                    acc[i][0] = mfma16(cop[0], sxo, acc[i][0]);
                    acc[i][1] = mfma16(cop[1], sxo, acc[i][1]);
                }
            }
            u4_t q[2];
#pragma unroll
            for (int j = 0; j < 2; j++) q[j] = S16[a_codes[j]];
            uint32_t sm[2][2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                sm[0][j] = splat16<0>(dsc[j][g]);
                sm[1][j] = splat16<1>(dsc[j][g]);
            }
            // four 16-k steps t = 2e + s2 (block 2g + e, positions 16s2..),
            // software pipelined: the operands of step t + 1 are read and built
            // while the eight MFMAs of step t run
            auto wop = [&](int t, int j) {
                const int e = t >> 1, s2 = t & 1;
                return e ? q4k_codes_f16<1>(q[j][2 * s2], q[j][2 * s2 + 1], sm[1][j])
                         : q4k_codes_f16<0>(q[j][2 * s2], q[j][2 * s2 + 1], sm[0][j]);
            };
            u4_t Xc[4], Wc[2];
#pragma unroll
            for (int i = 0; i < 4; i++) Xc[i] = S16[256u * i + a_act[0][0]];
            Wc[0] = wop(0, 0);
            Wc[1] = wop(0, 1);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if (t == 2) {
                    // first half of stage st + 1 to LDS, second half's loads
                    __builtin_amdgcn_sched_barrier(0);
                    store_half(st + 1u, 0);
                    load_half(st + 1u, 1);
                    __builtin_amdgcn_sched_barrier(0);
                }
                u4_t Xn[4], Wn[2];
                if (t < 3) {
                    const int e = (t + 1) >> 1, s2 = (t + 1) & 1;
#pragma unroll
                    for (int i = 0; i < 4; i++) Xn[i] = S16[256u * i + a_act[e][s2]];
                    Wn[0] = wop(t + 1, 0);
                    Wn[1] = wop(t + 1, 1);
                }
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    acc[i][0] = mfma16(Wc[0], Xc[i], acc[i][0]);
                    acc[i][1] = mfma16(Wc[1], Xc[i], acc[i][1]);
                }
                if (t < 3) {
                    // interleave: per MFMA one LDS read (first four) and a few VALU ops
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < 4; i++) Xc[i] = Xn[i];
                    Wc[0] = Wn[0];
                    Wc[1] = Wn[1];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            store_half(st + 1u, 1);
            __syncthreads();
        }
    }

    float* y = ds.y + (uint64_t)ks * ds.m * ds.ldy;
    const bool vec = (ds.ldy & 3u) == 0u && ((uintptr_t)ds.y & 15u) == 0u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = m0 + 32u * i + l32;
        const float scale = row < ds.m ? ds.xrs[act_row(ds, row)] : 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++) store_tile(ds, y, row, n0 + 64u * w + 32u * j, h, acc[i][j], scale, vec);
    }
}

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void rfxq_mmqh_q4k(MmqArgs args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[mmqh::kLds];
    if (blockDim.x != mmqh::kThreads) return;  // the tile assumes exactly kThreads lanes
    const MmqDesc d = mmq_pick(args, blockIdx.x);
    if (blockIdx.x - d.wg_begin >= d.tiles_m * d.tiles_n * d.splits) return;
    mmqh_q4k_tile(d, blockIdx.x - d.wg_begin, lds);
}

// One 128x128 tile (and one split-K range) of Y = X . W^T for Q6_K weights,
// f16 activations.
RFXQ_DEV void mmqh_q6k_tile(const MmqDesc& dv, uint32_t t_local, uint8_t* lds) {
    using namespace mmqh;
    MmqDesc ds = dv;
    {
        uint32_t* p = reinterpret_cast<uint32_t*>(&ds);
#pragma unroll
        for (uint32_t i = 0; i < sizeof(MmqDesc) / 4u; i++) p[i] = __builtin_amdgcn_readfirstlane(p[i]);
        t_local = __builtin_amdgcn_readfirstlane(t_local);
    }
    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, h = lane >> 5;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);

    const uint32_t ks = t_local % ds.splits;
    const uint32_t rest = t_local / ds.splits;
    const uint32_t tm = rest % ds.tiles_m, tn = rest / ds.tiles_m;
    const uint32_t m0 = tm * kBM6, n0 = tn * kBN6;
    const uint32_t nsb = ds.k / 256u;
    const uint32_t sb0 = ks * ds.sb_per_split;
    const uint32_t sb1 = min(nsb, sb0 + ds.sb_per_split);
    const uint32_t row_bytes = nsb * 210u;

    const uint32_t L = __builtin_amdgcn_readfirstlane(lds_addr(lds));
    const uint32_t Lhdr = L + 3u * kSlotQ6;

    const sdesc_t r_act = uniform_desc(ds.xq, 0xFFFFFFFFu);  // rows clamped or gathered (act_row)
    const sdesc_t r_w = uniform_desc(ds.w, ds.n * row_bytes);
    // activations: as the Q4_K kernel, but logical chunks 4-7 (block B) sit
    // 128 bytes after chunks 0-3 (block A) in the f16 row
    uint32_t o_act[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t c = (lane & 7u) ^ (lane >> 4) ^ ((q & 1) ? 4u : 0u);
        o_act[q] = act_row(ds, m0 + 32u * w + 8u * q + (lane >> 3)) * ds.ldq + 16u * c + (c >= 4u ? 64u : 0u);
    }
    // code windows: dword j of column c's window is copy lane 9c + j of the
    // wave (five copies, the last on lanes 0-31); headers likewise 5 dwords
    uint32_t o_c[5], o_h[3];
#pragma unroll
    for (int q = 0; q < 5; q++) {
        const uint32_t lp = 64u * q + lane;
        o_c[q] = (n0 + 32u * w + lp / 9u) * row_bytes + 4u * (lp % 9u);
    }
#pragma unroll
    for (int q = 0; q < 3; q++) {
        const uint32_t lp = 64u * q + lane;
        o_h[q] = (n0 + 32u * w + lp / 5u) * row_bytes + 4u * (lp % 5u);
    }
    const uint32_t nst = 4u * (sb1 - sb0);
    // copies of stage st: 14 per wave, 17 when it opens a super-block
    auto issue = [&](uint32_t st) {
        const uint32_t sb = sb0 + (st >> 2), g = st & 3u, n = g >> 1, s = g & 1u, slot = st % 3u;
        const uint32_t Ls = __builtin_amdgcn_readfirstlane(L + slot * kSlotQ6);
        const uint32_t base = 210u * sb - 2u * (sb & 1u);  // 4-byte aligned
#pragma unroll
        for (int q = 0; q < 4; q++)
            dma16(r_act, Ls + 1024u * (4u * w + q), o_act[q], 512u * sb + 64u * (4u * n + s));
        const uint32_t Lc = Ls + kAct + 2304u * w;
#pragma unroll
        for (int q = 0; q < 4; q++) dma4(r_w, Lc + 256u * q, o_c[q], base + 64u * n + 32u * s);
        if (h == 0u) dma4(r_w, Lc + 1024u, o_c[4], base + 64u * n + 32u * s);
#pragma unroll
        for (int q = 0; q < 4; q++) dma4(r_w, Lc + 1152u + 256u * q, o_c[q], base + 128u + 32u * n);
        if (h == 0u) dma4(r_w, Lc + 1152u + 1024u, o_c[4], base + 128u + 32u * n);
        if (g == 0u) {
            const uint32_t Lh = Lhdr + 640u * w;
            dma4(r_w, Lh, o_h[0], base + 192u);
            dma4(r_w, Lh + 256u, o_h[1], base + 192u);
            if (h == 0u) dma4(r_w, Lh + 512u, o_h[2], base + 192u);
        }
    };

    v16f_t acc[4], t[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        acc[i] = v16f_t{};
        t[i] = v16f_t{};
    }
    uint32_t a_act[2][2];
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) a_act[e][s2] = l32 * 8u + ((4u * e + 2u * h + s2) ^ ((l32 >> 1) & 7u));
    const uint32_t a_codes = (kAct + 2304u * w) / 4u + 9u * l32 + 4u * h;
    uint32_t scw[4] = {0u, 0u, 0u, 0u}, dbits = 0u;

    if (nst > 0u) issue(0u);
    if (nst > 1u) issue(1u);
    for (uint32_t st = 0; st < nst; st++) {
        if (st + 1u < nst) {
            if (((st + 1u) & 3u) == 0u) asm volatile("s_waitcnt vmcnt(17)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(14)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (st + 2u < nst) issue(st + 2u);

        const uint32_t sb = sb0 + (st >> 2), g = st & 3u, n = g >> 1, s = g & 1u;
        const uint32_t sh = 2u * (sb & 1u);  // byte offset of the block in the windows
        const uint8_t* S = lds + (st % 3u) * kSlotQ6;
        const u4_t* S16 = reinterpret_cast<const u4_t*>(S);
        if (g == 0u) {
            const uint32_t* hp = reinterpret_cast<const uint32_t*>(lds + 3u * kSlotQ6 + 640u * w) + 5u * l32;
            uint32_t hw[5];
#pragma unroll
            for (int j = 0; j < 5; j++) hw[j] = hp[j];
#pragma unroll
            for (int j = 0; j < 4; j++) scw[j] = __builtin_amdgcn_alignbyte(hw[j + 1], hw[j], sh);
            dbits = (hw[4] >> (8u * sh)) & 0xFFFFu;
        }
        const uint32_t* cp = reinterpret_cast<const uint32_t*>(S) + a_codes;
        uint32_t V[4], H[4];
        {
            uint32_t c[5], e[5];
#pragma unroll
            for (int j = 0; j < 5; j++) {
                c[j] = cp[j];
                e[j] = cp[288 + j];
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                V[j] = __builtin_amdgcn_alignbyte(c[j + 1], c[j], sh);
                H[j] = __builtin_amdgcn_alignbyte(e[j + 1], e[j], sh);
            }
        }
        const uint32_t bsh = 8u * (2u * s + h);
        const u4_t tabA = q6k_tab((int)(int8_t)(scw[2 * n] >> bsh));
        const u4_t tabB = q6k_tab((int)(int8_t)(scw[2 * n + 1] >> bsh));
        u4_t hi[2][2], lo[2][2];
        if (s) q6k_stage_operands<1>(V, H, tabA, tabB, hi, lo);
        else q6k_stage_operands<0>(V, H, tabA, tabB, hi, lo);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u4_t* xp = S16 + 256u * i;
            const u4_t xa0 = xp[a_act[0][0]], xa1 = xp[a_act[0][1]];
            const u4_t xb0 = xp[a_act[1][0]], xb1 = xp[a_act[1][1]];
            t[i] = mfma16(hi[0][0], xa0, t[i]);
            t[i] = mfma16(lo[0][0], xa0, t[i]);
            t[i] = mfma16(hi[0][1], xa1, t[i]);
            t[i] = mfma16(lo[0][1], xa1, t[i]);
            t[i] = mfma16(hi[1][0], xb0, t[i]);
            t[i] = mfma16(lo[1][0], xb0, t[i]);
            t[i] = mfma16(hi[1][1], xb1, t[i]);
            t[i] = mfma16(lo[1][1], xb1, t[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (g == 3u) {
            uint32_t dd[16];
#pragma unroll
            for (int r = 0; r < 16; r++) dd[r] = bperm(8u * (r >> 2) + 4u * h + (r & 3), dbits);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float d = f16_opaque(dd[r]);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    acc[i][r] = __builtin_fmaf(t[i][r], d, acc[i][r]);
                    t[i][r] = 0.0f;
                }
            }
        }
    }

    float* y = ds.y + (uint64_t)ks * ds.m * ds.ldy;
    const bool vec = (ds.ldy & 3u) == 0u && ((uintptr_t)ds.y & 15u) == 0u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = m0 + 32u * i + l32;
        const float scale = row < ds.m ? ds.xrs[act_row(ds, row)] : 0.0f;
        store_tile(ds, y, row, n0 + 32u * w, h, acc[i], scale, vec);
    }
}

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void rfxq_mmqh_q6k(MmqArgs args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[mmqh::kLdsQ6];
    const MmqDesc d = mmq_pick(args, blockIdx.x);
    if (blockIdx.x - d.wg_begin >= d.tiles_m * d.tiles_n * d.splits) return;
    mmqh_q6k_tile(d, blockIdx.x - d.wg_begin, lds);
}
