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
// Tiles: (32 MT) activation rows x 256 weight columns per 256-thread
// workgroup, MT = 4 (128-row tiles, two workgroups per CU) or MT = 1 (32-row
// tiles: few-row GEMMs and small expert groups). Wave w owns weight columns
// [64w, +64) against all rows: 2 MT 32x32 MFMA tiles, A = weights,
// B = activations (lane l holds activation row l%32 of its tile and 16
// weight columns), so each activation operand read from LDS feeds two MFMAs
// and each converted weight operand MT. Data moves in 64-k stages:
//   - weights go straight to registers: no other wave reads a wave's columns,
//     so each lane loads its own 16-byte pieces of the stage one stage ahead
//     (plain buffer loads) and converts them there;
//   - activations [BM][64] f16 (16-byte chunks XOR-swizzled by row/2) and,
//     with the first stage of a super-block, the Sx records [BM][32 B] pass
//     through a 2-slot LDS ring: every lane loads its share of stage s + 1
//     into registers while stage s computes and writes it to the other slot;
//     one barrier per stage.
// (The LDS-DMA path, buffer_load ... lds, measured slower here: it throttles
// the MFMA stream of the same CU.) Activation rows are gathered through
// MmqDesc::rows when set (MoE expert groups). The Q6_K tile (below) has the
// same layout and pipeline with its own weight operands.
#pragma once
#include "common.hpp"
#include "mmq.hpp"


namespace mmqh {

// MT = 32-row tiles per wave (4: 128-row workgroup tiles; 1: 32-row tiles,
// the fused few-row form and small expert groups: weights read once per 32
// rows)
constexpr uint32_t BN = 256, kThreads = 256;
template <int MT>
struct Tile {
    static constexpr uint32_t BM = 32u * MT;
    static constexpr uint32_t kAct = BM * 128u;  // activation stage: BM rows x 64 f16
};

// Tile pipeline. Activations (and Q4_K's Sx records) are copied straight
// into LDS (buffer_load ... lds) kActDepth - 1 stages ahead, into
// kActDepth stage buffers that are distinct LDS objects, so that the
// compiler's wait counting sees that a stage's reads do not alias the copies
// in flight; weights go to registers WA stages ahead (2, or 1 where two
// stages of weight registers would not fit). Stage s issues stage s + WA's
// weight loads, then stage s + 3's copies (with the Sx records when s + 3
// starts a super-block). A stage ends with a counted wait for the next
// stage's copies, which were issued two stages earlier, and a barrier; the
// count is the operations issued after them, fixed by the stage's position g
// in its super-block because every stage issues the same loads whatever its
// position in the range (the last stage's data again past the range's end).
// The prologue issues the copies of stages 0-2 and the weights of stages
// 0..WA-1 in the same order (copies 0, 1, weights 0, copies 2 for WA = 1;
// copies 0, weights 0, copies 1, weights 1, copies 2 for WA = 2). W0..W3:
// vector-memory operations of a stage's weight loads at positions 0..3; SX:
// 1 when the Sx records are copied.
constexpr int kActDepth = 4;
struct ActLds {
    u4_t* a[kActDepth];  // stage buffers, BM x 128 bytes each
    u4_t* sx;            // the Sx records of one super-block: one 16-byte piece per thread
    float* sc;           // the rows' scales 2^e, for the stores
};
// stage buffer w (wave-uniform) of the pointers, by selects on the values:
// an index that is not a constant, or a member call, would put the pointers
// in scratch memory
RFXQ_DEV u4_t* pick_buf(u4_t* a0, u4_t* a1, u4_t* a2, u4_t* a3, uint32_t w) {
    return w == 0u ? a0 : w == 1u ? a1 : w == 2u ? a2 : a3;
}
template <int N>
RFXQ_DEV void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
template <int MT, int WA, int W0, int W1, int W2, int W3, int SX>
struct StagePipe {
    static_assert(WA == 1 || WA == 2, "weights one or two stages ahead");
    static constexpr int w_at(int p) { return p == 0 ? W0 : p == 1 ? W1 : p == 2 ? W2 : W3; }
    static constexpr int issued(int g) {  // operations stage g issues
        return w_at((g + WA) & 3) + MT + (((g + 3) & 3) == 0 ? SX : 0);
    }
    // after stage 0's copies (with its Sx): the weights of stages 0..WA-1,
    // the copies of stages 1 and 2
    static constexpr int kPrologue = W0 + (WA == 2 ? W1 : 0) + 2 * MT;
    // after stage g + 1's copies: stage g - 1's and stage g's operations
    static constexpr int after(int g) { return issued((g + 3) & 3) + issued(g); }
    static_assert(after(2) <= 63 && kPrologue <= 63, "vmcnt holds 6 bits");
    RFXQ_DEV static void prologue_end() {
        vm_wait<kPrologue>();
        lds_barrier();
    }
    RFXQ_DEV static void stage_end(uint32_t g) {
        if (g == 0u) vm_wait<after(0)>();
        else if (g == 1u) vm_wait<after(1)>();
        else if (g == 2u) vm_wait<after(2)>();
        else vm_wait<after(3)>();
        lds_barrier();
    }
};
// the activation chunk a lane copies: LDS chunk c of row r holds logical
// chunk c ^ ((r / 2) % 8), and a wave's copy writes its lanes' 16-byte
// pieces in lane order (piece tid = chunk tid % 8 of row tid / 8)
RFXQ_DEV uint32_t act_chunk(uint32_t tid) { return (tid & 7u) ^ ((tid >> 4) & 7u); }

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
// (C_0..7 as f16 pairs) and the eight block multipliers, packed two per dword
// (block 2p low, 2p + 1 high): f16(d*sc_b) for the low-nibble blocks (even
// b), f16(d*sc_b/16) for the high-nibble ones (the codes' scales 1 and 16).
RFXQ_DEV void q4k_sb_operands(const u4_t hdr, u4_t& cop, u4_t& dsc) {
    float sc[8], mn[8];
    q4k_scales_mins(hdr, sc, mn);
    const float d = f16_bits_to_f32(hdr.x), dmin = f16_bits_to_f32(hdr.x >> 16);
    uint32_t c[8], s[8];
#pragma unroll
    for (int b = 0; b < 8; b++) {
        c[b] = f16_rne(__builtin_fmaf(8.0f * d, sc[b], -(dmin * mn[b])));
        s[b] = f16_rne(d * sc[b] * ((b & 1) ? 0.0625f : 1.0f));
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
// of the step's two quant dwords, as f16 pairs f16((q - 8) * s) in the
// activations' (q0, q2), (q1, q3) order, s = f16(d*sc) (E = 0) or
// f16(d*sc/16) (E = 1): the nibble is and-or'ed into the mantissa of an f16
// 1024.0 where it already sits (bits 0-3: 1024 + q; bits 4-7: 1024 + 16q),
// an exact add of -1032 (-1152) centres it, and one multiply rounds. `m` is
// the nibble mask of E, `mg` the f16 pair (1024, 1024), `v0s`/`v1s` the
// dwords shifted right by 8 (shared by both blocks); all in VGPRs so that
// each code dword is one v_and_or_b32.
template <int E>
RFXQ_DEV u4_t q4k_codes_f16(uint32_t v0, uint32_t v1, uint32_t v0s, uint32_t v1s, uint32_t s, uint32_t m,
                            uint32_t mg) {
    const uint32_t w[4] = {(v0 & m) | mg, (v0s & m) | mg, (v1 & m) | mg, (v1s & m) | mg};
    const h2_t off = E ? h2_t{(half_t)-1152.0f, (half_t)-1152.0f} : h2_t{(half_t)-1032.0f, (half_t)-1032.0f};
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

// First activation row of the tile's buffer resource: the tile's own first
// row (m0) when rows are not gathered, so that offsets stay within 32 bits
// for any row count; 0 for a gathered GEMM, whose source rows can be any
// (the host keeps those activations under 4 GiB).
RFXQ_DEV uint32_t act_base(const MmqDesc& ds, uint32_t m0) { return ds.rows ? 0u : m0; }

// The accumulator of a 32x32 output tile (mfma16: A = activations, B =
// weights): lane (l32, h) holds weight column l32 and activation rows
// 8 q4 + 4 h + r (q4, r in [0, 4)) as acc[4 q4 + r]. Stored as dwords: the
// 32 lanes of a half write one row's 32 consecutive columns (128 contiguous
// bytes per row and instruction). `row` = the tile's row 4h, `sc` = the LDS
// scales 2^e of rows row..row+27. Outputs are written once and not read
// back by the kernel: non-temporal stores.
RFXQ_DEV void store_tile(const MmqDesc& ds, float* y, uint32_t row, uint32_t col, const v16f_t& acc,
                         const float* sc, bool scale = true) {
    if (col >= ds.n) return;
    float* yc = y + col;
#pragma unroll
    for (int q4 = 0; q4 < 4; q4++) {
        const float4 s4 = *reinterpret_cast<const float4*>(sc + 8 * q4);
        const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t m = row + 8u * q4 + r;
            if (m < ds.m) __builtin_nontemporal_store(scale ? acc[4 * q4 + r] * sv[r] : acc[4 * q4 + r], yc + (uint64_t)m * ds.ldy);
        }
    }
}

// A wave's MT x 2 accumulator tiles (rows m0 + 32i, columns c0 + 32j) with
// 16-byte stores: each tile passes through the wave's 4 KB LDS region `buf`
// (free once the tile loop is over) as a row-major 32x32 array whose column
// index is xor'ed with 4 (R % 8) in row R (whole float4 groups stay
// together), and lane (t + 4k, h) then reads and stores row 8q4 + 4h + t,
// columns 4k..4k+3: eight lanes per 128-byte row piece and a quarter of the
// dword stores' instructions (4-5% of the 0.6B prefill set). Outputs whose
// rows are not 16-byte aligned take the dword stores.
template <int MT, int JMASK = 3>
RFXQ_DEV void store_wave(const MmqDesc& ds, float* y, uint32_t m0, uint32_t c0, const v16f_t (&acc)[MT][2],
                         const float* sc, u4_t* buf, bool scale = true) {
    const uint32_t lane = threadIdx.x & 63u, l32 = lane & 31u, h = lane >> 5;
    if ((ds.ldy & 3u) != 0u || (reinterpret_cast<uintptr_t>(y) & 15u) != 0u) {
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                if (JMASK >> j & 1)
                    store_tile(ds, y, m0 + 32u * i + 4u * h, c0 + 32u * j + l32, acc[i][j], sc + 32u * i + 4u * h, scale);
        return;
    }
    float* bf = reinterpret_cast<float*>(buf);
    const uint32_t t = l32 & 3u, k = l32 >> 2;
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            if (!(JMASK >> j & 1)) continue;
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t R = 8u * q4 + 4u * h + r;
                    bf[32u * R + (l32 ^ ((R & 7u) << 2))] = acc[i][j][4 * q4 + r];
                }
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const uint32_t R = 8u * q4 + 4u * h + t;
                f4v_t v = *reinterpret_cast<const f4v_t*>(bf + 32u * R + ((4u * k) ^ ((R & 7u) << 2)));
                if (scale) v *= sc[32u * i + R];
                const uint32_t m = m0 + 32u * i + R, c = c0 + 32u * j + 4u * k;
                if (m >= ds.m) continue;
                float* yr = y + (uint64_t)m * ds.ldy;
                if (c + 3u < ds.n) {
                    __builtin_nontemporal_store(v, reinterpret_cast<f4v_t*>(yr + c));
                } else {
#pragma unroll
                    for (uint32_t u = 0; u < 4u; u++)
                        if (c + u < ds.n) __builtin_nontemporal_store(v[u], yr + c + u);
                }
            }
        }
}

// Workgroup b of a g-workgroup launch as a tile index such that the tiles
// each XCD runs are contiguous: workgroups go round-robin to the 8 XCDs, and
// neighbouring tiles (the row tiles of one column tile, then the next column
// tile) share weight and activation reads in that XCD's L2.
RFXQ_DEV uint32_t xcd_tile(uint32_t b, uint32_t g) {
    const uint32_t x = b & 7u, slot = b >> 3, q = g >> 3, r = g & 7u;
    return (x < r ? x * (q + 1u) : r * (q + 1u) + (x - r) * q) + slot;
}

// c += w . x over one 16-k step: w = weight operand (32 columns), x =
// activation operand (32 rows); the result's rows are the activation rows
// (A = x, B = w), see store_tile
RFXQ_DEV v16f_t mfma16(u4_t w, u4_t x, v16f_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(as_h8(x), as_h8(w), c, 0, 0, 0);
}

// ---------------------------------------------------------------- Q6_K
//
// A Q6_K super-block (ql[128], qh[64], scales[16] i8, d; src/dequant.rs:414-445)
// has no constant part: w = d * sc * (q - 32), one int8 scale per 16 codes.
// The weight operand is f16((q - 32) * f16(d*sc)): the 6-bit code is and-or'ed
// into the mantissa of an f16 1024.0 (low nibble from ql, two high bits from
// qh), an exact add centres it, and one multiply rounds, as for Q4_K.
//
// A 64-k stage g = 2n + s of a super-block takes the 32-code groups A = s and
// B = s + 2 of half n (elements 128n + 32s + l and 128n + 64 + 32s + l, l in
// [0, 32)): low and high nibbles of ql[64n + 32s + l], bits 2s, 2s + 4 of
// qh[32n + l]. Lane half h holds positions l in [16h, 16h + 16), whose scales
// are sc[8n + 2s + h] (A) and sc[8n + 4 + 2s + h] (B). Blocks are 210 bytes,
// so a super-block starts 0 or 2 bytes past a dword; its 16-byte pieces are
// read with single unaligned buffer loads (the HSA unaligned access mode).

// (a & m) | c in one instruction (instruction selection would otherwise
// merge two of them into an or3 of two ands)
RFXQ_DEV uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(c));
    return r;
}

// Weight operand of one 16-k step of a stage's group A (E = 0) or B (E = 1)
// from ql dwords l0, l1 (and l0s, l1s = the same >> 8) and qh dwords shifted
// so that the group's two bits of bytes 0 and 2 (qa0, qa1) and of bytes 1
// and 3 (qb0, qb1) sit at bits 4-5 (E = 0) or 8-9 (E = 1): the code goes into
// the mantissa of an f16 1024.0 where its low nibble already sits (A: bits
// 0-3, 1024 + q; B: bits 4-7, 1024 + 16q), an exact add of -1056 (-1536)
// centres it, and one multiply by s (f16(d*sc), or f16(d*sc/16) for B)
// rounds. Pairs follow the activations' (p0, p2), (p1, p3) order; the masks
// and mg = the f16 pair (1024, 1024) are VGPRs so that each half is one
// v_and_or_b32.
template <int E>
RFXQ_DEV u4_t q6k_codes_f16(uint32_t l0, uint32_t l1, uint32_t l0s, uint32_t l1s, uint32_t qa0, uint32_t qa1,
                            uint32_t qb0, uint32_t qb1, uint32_t s, uint32_t ml, uint32_t mq, uint32_t mg) {
    const uint32_t w[4] = {and_or(l0, ml, and_or(qa0, mq, mg)), and_or(l0s, ml, and_or(qb0, mq, mg)),
                           and_or(l1, ml, and_or(qa1, mq, mg)), and_or(l1s, ml, and_or(qb1, mq, mg))};
    const h2_t off = E ? h2_t{(half_t)-1536.0f, (half_t)-1536.0f} : h2_t{(half_t)-1056.0f, (half_t)-1056.0f};
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

// The eight block multipliers of lane half h of one column: f16(d * sc[2i + h])
// for i = 0..7, divided by 16 for the B groups (i = 2, 3, 6, 7: codes placed
// at 16q), packed two per dword (i = 2p low, 2p + 1 high); sc = the 16 int8
// scales, d = the f16 bits of d.
RFXQ_DEV u4_t q6k_multipliers(u4_t sc, uint32_t dbits, uint32_t h) {
    const float d = f16_bits_to_f32(dbits);
    uint32_t m[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t byte = 2u * i + h;  // scale index; dword byte/4, byte byte%4
        const int sv = (int)(int8_t)(sc[i >> 1] >> (8u * (byte & 3u)));
        m[i] = f16_rne(d * (float)sv * ((i & 2) ? 0.0625f : 1.0f));
    }
    return u4_t{pack16(m[0], m[1]), pack16(m[2], m[3]), pack16(m[4], m[5]), pack16(m[6], m[7])};
}

}  // namespace mmqh


// One (32 MT)x256 tile (and one split-K range) of Y = X . W^T for Q4_K weights.
template <int MT>
RFXQ_DEV void mmqh_q4k_rows(const MmqDesc& ds, uint32_t m0, uint32_t n0, uint32_t ks, const mmqh::ActLds& L) {
    using namespace mmqh;
    constexpr uint32_t BM = Tile<MT>::BM;
    // weight loads per stage: the code pieces of two stages (four loads) at
    // even positions, with the headers at position 0; none at odd ones
    constexpr int WA = 2;
    using Pipe = StagePipe<MT, WA, 6, 0, 4, 0, 1>;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, h = lane >> 5;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsb = ds.k / 256u;
    const uint32_t sb0 = ks * ds.sb_per_split;
    const uint32_t sb1 = min(nsb, sb0 + ds.sb_per_split);
    const uint32_t row_bytes = nsb * 144u;
    const uint32_t rec_bytes = nsb * 32u;

    // Buffers start at the tile (tile_base): 32-bit offsets for any matrix
    // size. Weight columns past the matrix read past the buffer: zeros, no
    // fault. Activation rows are clamped or gathered (act_row): in bounds.
    const uint32_t rb = act_base(ds, m0);
    const rsrc_t r_act = make_rsrc(ds.xq + (uint64_t)rb * ds.ldq, 0xFFFFFFFFu);
    // a gate/up pair: waves 0-1 the gate columns [n0, n0 + 128), waves 2-3
    // the same columns of up
    const bool pair = ds.gu_pair != 0u;
    const bool upw = pair && w >= 2u;
    const uint32_t wc = pair ? (w & 1u) : w;  // the wave's 64-column block
    const rsrc_t r_w = make_rsrc((upw ? ds.w_up : ds.w) + (uint64_t)n0 * row_bytes,
                                 min(pair ? BN / 2u : BN, ds.n - n0) * row_bytes);
    const rsrc_t r_sx =
        make_rsrc(reinterpret_cast<const uint8_t*>(ds.xds) + (uint64_t)rb * rec_bytes, 0xFFFFFFFFu);
    // Staged activations, copied straight into LDS (buffer_load ... lds: the
    // 64 lanes of a wave write 1 KB in lane order): piece 256u + tid of a
    // stage buffer is chunk tid%8 of row 32u + tid/8; LDS chunk c of row r
    // holds logical chunk c ^ ((r/2)%8), so the lane fetches that one.
    // Sx: piece tid = half tid%2 of row tid/2 (rows past the tile's BM repeat
    // its last row; never read).
    const uint32_t ra = tid >> 3;
    uint32_t g_act[MT];
#pragma unroll
    for (int u = 0; u < MT; u++) g_act[u] = (act_row(ds, m0 + ra + 32u * u) - rb) * ds.ldq + 16u * act_chunk(tid);
    const uint32_t g_sx = (act_row(ds, m0 + min(tid >> 1, BM - 1u)) - rb) * rec_bytes + 16u * (tid & 1u);
    // Weights go straight to registers (no other wave reads a wave's
    // columns), two stages at a time: for n-tile j, load A covers columns
    // 64w + 32j + [0, 16) and load B the next 16, each lane 16 of the 64
    // quant bytes the two stages take from its column, lane (l32, h) piece
    // 2 (l32 / 16) + h of column l32 % 16 (16 columns x 64 contiguous bytes
    // per load: 4.8-5.0 TB/s streamed, against 3.0-3.6 TB/s for one stage's
    // 32 bytes of 32 columns per load). One v_permlane16_swap per dword then
    // gives the two stages' operands: lane (l32, h) holds half h of the 32
    // quant bytes of column 64w + 32j + l32 for each stage. Each lane also
    // loads its column's 16-byte header with the first stage of each
    // super-block.
    uint32_t col[2], g_q[2], g_h[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        col[j] = 64u * wc + 32u * j + l32;
        g_h[j] = col[j] * row_bytes;
        g_q[j] = (64u * wc + 32u * j + (l32 & 15u)) * row_bytes + 16u + 32u * (l32 >> 4) + 16u * h;
    }
    const uint32_t g_qb = 16u * row_bytes;  // load B: 16 columns on
    const uint32_t nst = 4u * (sb1 - sb0);

    // Every stage issues the same copies and loads whatever its position, so
    // the wait counts below hold: past the last stage a lane copies the last
    // stage again (in bounds; into a buffer no stage reads any more).
    // Activations run kActDepth - 1 stages ahead, weights one.
    auto copy_act = [&](uint32_t st, u4_t* buf, bool sx) {
        const uint32_t sl = min(st, nst - 1u);
        const uint32_t sb = sb0 + (sl >> 2), g = sl & 3u;
#pragma unroll
        for (int u = 0; u < MT; u++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_act, RFXQ_LDSP(buf + 256u * u + 64u * w), 16, g_act[u],
                                                     512u * sb + 128u * g, 0, 0);
        if (sx)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_sx, RFXQ_LDSP(L.sx + 64u * w), 16, g_sx, 32u * sb, 0, 0);
    };
    // weights of two stage pairs (by pair: loads A, B of each n-tile), a
    // super-block's headers; load_w takes an even stage st: stages st, st + 1
    u4_t qp[2][2][2], hn[2];
    auto load_w = [&](uint32_t st, bool hdr) {
        const uint32_t sl = min(st, nst - 2u);
        const uint32_t sb = sb0 + (sl >> 2), g = sl & 3u;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            qp[(st >> 1) & 1u][j][0] = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_q[j], 144u * sb + 32u * g, 0);
            qp[(st >> 1) & 1u][j][1] = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_q[j] + g_qb, 144u * sb + 32u * g, 0);
        }
        if (hdr)
#pragma unroll
            for (int j = 0; j < 2; j++) hn[j] = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_h[j], 144u * sb, 0);
    };

    v16f_t acc[MT][2];
#pragma unroll
    for (int i = 0; i < MT; i++) acc[i][0] = acc[i][1] = v16f_t{};
    // LDS read offsets (16-byte units): activations of row l32 of row tile 0,
    // logical chunk 4e + 2h + step
    uint32_t a_act[2][2];
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) a_act[e][s2] = l32 * 8u + ((4u * e + 2u * h + s2) ^ ((l32 >> 1) & 7u));
    u4_t dsc[2] = {}, q[2] = {};
    // code-extraction constants, kept in VGPRs (VOP3 takes no literal here)
    uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, mg = 0x64006400u;
    asm("" : "+v"(mlo), "+v"(mhi), "+v"(mg));

    // the rows' scales 2^e (for the stores) read now, written to LDS after
    // the loop: a buffer load, so no wait before the first stage covers them
    float row_scale = 0.0f;
    if (tid < BM && m0 + tid < ds.m)
        row_scale = as_f32(bld4(make_rsrc(ds.xrs, 0xFFFFFFFFu), 4u * act_row(ds, m0 + tid)));
    // prologue: stages 0-2 copied (with stage 0's Sx), stages 0-1's weights
    copy_act(0u, L.a[0], true);
    load_w(0u, true);
    copy_act(1u, L.a[1], false);
    copy_act(2u, L.a[2], false);
    Pipe::prologue_end();
    u4_t q_odd[2] = {};  // the odd stage's operands, from the pair's swap
    for (uint32_t st0 = 0; st0 < nst; st0 += 4u) {
#pragma unroll
        for (uint32_t g = 0; g < 4u; g++) {
            const uint32_t st = st0 + g;
            u4_t hdr[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if ((g & 1u) == 0u) {
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const auto r = __builtin_amdgcn_permlane16_swap(qp[g >> 1][j][0][d], qp[g >> 1][j][1][d],
                                                                       false, false);
                        q[j][d] = r[0];
                        q_odd[j][d] = r[1];
                    }
                } else {
                    q[j] = q_odd[j];
                }
                if (g == 0u) hdr[j] = hn[j];
            }
            // (even stages) the weights of stages st + 2, st + 3 into the
            // pair registers stages st - 2, st - 1 used; then stage st + 3's
            // activations into the buffer stage st - 1 used (every wave is
            // past it: the barrier that ended stage st - 1), with its Sx when
            // it starts a super-block. (The weights first: their use then
            // waits only for them.)
            if ((g & 1u) == 0u) load_w(st + 2u, g == 2u);
            copy_act(st + 3u, L.a[(g + 3u) & 3u], g == 1u);
            const u4_t* S16 = L.a[g];
            if (g == 0u) {
                // super-block start: the columns' multipliers, and the
                // constant part C_b * Sx_b into the accumulators
                u4_t cop[2];
#pragma unroll
                for (int j = 0; j < 2; j++) q4k_sb_operands(hdr[j], cop[j], dsc[j]);
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    const u4_t sxo = L.sx[2u * (32u * i + l32) + h];
                    acc[i][0] = mfma16(cop[0], sxo, acc[i][0]);
                    acc[i][1] = mfma16(cop[1], sxo, acc[i][1]);
                }
            }
            uint32_t sm[2][2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                sm[0][j] = splat16<0>(dsc[j][g]);
                sm[1][j] = splat16<1>(dsc[j][g]);
            }
            // four 16-k steps t = 2e + s2 (block 2g + e, positions 16s2..),
            // software pipelined: the operands of step t + 1 are read and built
            // while the eight MFMAs of step t run
            uint32_t qs8[2][4];
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int u = 0; u < 4; u++) qs8[j][u] = q[j][u] >> 8;
            auto wop = [&](int t, int j) {
                const int e = t >> 1, s2 = t & 1;
                const uint32_t a0 = q[j][2 * s2], a1 = q[j][2 * s2 + 1], b0 = qs8[j][2 * s2], b1 = qs8[j][2 * s2 + 1];
                return e ? q4k_codes_f16<1>(a0, a1, b0, b1, sm[1][j], mhi, mg)
                         : q4k_codes_f16<0>(a0, a1, b0, b1, sm[0][j], mlo, mg);
            };
            u4_t Xc[MT], Wc[2];
#pragma unroll
            for (int i = 0; i < MT; i++) Xc[i] = S16[256u * i + a_act[0][0]];
            Wc[0] = wop(0, 0);
            Wc[1] = wop(0, 1);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                u4_t Xn[MT], Wn[2];
                if (t < 3) {
                    const int e = (t + 1) >> 1, s2 = (t + 1) & 1;
#pragma unroll
                    for (int i = 0; i < MT; i++) Xn[i] = S16[256u * i + a_act[e][s2]];
                    Wn[0] = wop(t + 1, 0);
                    Wn[1] = wop(t + 1, 1);
                }
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    acc[i][0] = mfma16(Wc[0], Xc[i], acc[i][0]);
                    acc[i][1] = mfma16(Wc[1], Xc[i], acc[i][1]);
                }
                if (t < 3) {
                    // interleave: per MFMA one LDS read (first MT) and a few VALU ops
#pragma unroll
                    for (int u = 0; u < MT; u++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                    }
#pragma unroll
                    for (int u = 0; u < MT; u++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < MT; i++) Xc[i] = Xn[i];
                    Wc[0] = Wn[0];
                    Wc[1] = Wn[1];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            // stage st + 1's copies done (issued two stages ago; after them
            // came stage st - 1's and stage st's copies and loads), then every
            // wave past this stage's reads
            Pipe::stage_end(g);
        }
    }
    // no copy may land in LDS after the workgroup is gone
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (tid < BM) L.sc[tid] = row_scale;
    lds_barrier();

    float* y = ds.y + (uint64_t)ks * ds.m * ds.ldy;
    if (!pair) {
        store_wave<MT>(ds, y, m0, n0 + 64u * w, acc, L.sc, pick_buf(L.a[0], L.a[1], L.a[2], L.a[3], w));
        return;
    }
    // gate/up pair: the two waves of a 64-column block split the epilogue.
    // The gate wave passes its j = 1 tiles to the up wave, the up wave its
    // j = 0 tiles to the gate wave, through the stage buffers (tile (i, j) of
    // the block c in buffer 2c + j at 4 KB i, each lane's 16 values at 64
    // bytes lane: both waves' accumulators have one layout); each then
    // stores s = silu(g) * u for its 32 columns, g and u the scaled outputs
    // (silu_and_mul.cu:7-23: g / (1 + expf(-g)) * u), unscaled.
    const int keep = upw ? 1 : 0;  // the j-tile this wave finishes
#pragma unroll
    for (int i = 0; i < MT; i++) {
        float* b = reinterpret_cast<float*>(pick_buf(L.a[0], L.a[1], L.a[2], L.a[3], 2u * wc + (1u - keep))) +
                   1024u * i + 16u * lane;
        const v16f_t& v = acc[i][1 - keep];
#pragma unroll
        for (int r = 0; r < 16; r += 4) *reinterpret_cast<f4v_t*>(b + r) = f4v_t{v[r], v[r + 1], v[r + 2], v[r + 3]};
    }
    lds_barrier();
    {
#pragma clang fp contract(off)
#pragma unroll
        for (int i = 0; i < MT; i++) {
            const float* b = reinterpret_cast<const float*>(pick_buf(L.a[0], L.a[1], L.a[2], L.a[3], 2u * wc + keep)) +
                             1024u * i + 16u * lane;
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const f4v_t pv = *reinterpret_cast<const f4v_t*>(b + 4 * q4);
                const float4 s4 = *reinterpret_cast<const float4*>(L.sc + 32u * i + 4u * h + 8u * q4);
                const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float mine = acc[i][keep][4 * q4 + r] * sv[r], other = pv[r] * sv[r];
                    const float g = upw ? other : mine, u = upw ? mine : other;
                    acc[i][keep][4 * q4 + r] = (g / (1.0f + expf(-g))) * u;
                }
            }
        }
    }
    lds_barrier();  // every passed tile read before the stores reuse the buffers
    if (upw)
        store_wave<MT, 2>(ds, y, m0, n0 + 64u * wc, acc, L.sc, pick_buf(L.a[0], L.a[1], L.a[2], L.a[3], w), false);
    else
        store_wave<MT, 1>(ds, y, m0, n0 + 64u * wc, acc, L.sc, pick_buf(L.a[0], L.a[1], L.a[2], L.a[3], w), false);
}

template <int MT>
RFXQ_DEV void mmqh_q6k_rows(const MmqDesc& ds, uint32_t m0, uint32_t n0, uint32_t ks, const mmqh::ActLds& ls);
template <int MT>
RFXQ_DEV void mmqh_q80_rows(const MmqDesc& ds, uint32_t m0, uint32_t n0, uint32_t ks, const mmqh::ActLds& lds);

// One (32 MT)x256 tile (and one split-K range): the descriptor made uniform,
// the tile decoded, and the rows computed by the body of as many 32-row tiles
// as the tile has rows (a ragged last tile, or an expert group of 33 rows in
// a 64-row tile, runs no MFMAs on absent rows).
template <int MT, int TY>
RFXQ_DEV void mmqh_tile(const MmqDesc& dv, uint32_t t_local, const mmqh::ActLds& lds) {
    MmqDesc ds = dv;
    {
        uint32_t* p = reinterpret_cast<uint32_t*>(&ds);
#pragma unroll
        for (uint32_t i = 0; i < sizeof(MmqDesc) / 4u; i++) p[i] = __builtin_amdgcn_readfirstlane(p[i]);
        t_local = __builtin_amdgcn_readfirstlane(t_local);
    }
    const uint32_t ks = t_local % ds.splits;
    const uint32_t rest = t_local / ds.splits;
    const uint32_t tm = rest % ds.tiles_m, tn = rest / ds.tiles_m;
    const uint32_t m0 = tm * 32u * MT, n0 = tn * (ds.gu_pair ? mmqh::BN / 2u : mmqh::BN);
    const uint32_t sub = min((uint32_t)MT, (ds.m - m0 + 31u) / 32u);  // 32-row tiles with rows
    auto run = [&](auto mt) {
        constexpr int M = decltype(mt)::value;
        if constexpr (TY == TY_Q4K) mmqh_q4k_rows<M>(ds, m0, n0, ks, lds);
        else if constexpr (TY == TY_Q6K) mmqh_q6k_rows<M>(ds, m0, n0, ks, lds);
        else mmqh_q80_rows<M>(ds, m0, n0, ks, lds);
    };
    if constexpr (MT >= 4) {
        if (sub >= 4u) return run(std::integral_constant<int, 4>{});
        if (sub == 3u) return run(std::integral_constant<int, 3>{});
    }
    if constexpr (MT >= 2)
        if (sub >= 2u) return run(std::integral_constant<int, 2>{});
    run(std::integral_constant<int, 1>{});
}

// The tiles of a launch are spread over the XCDs by their real count: a grid
// sized by an upper bound (device-written MoE tables) would otherwise leave
// the XCDs that own the tail of the tile range without work.
#define RFXQ_MMQH_ENTRY(NAME, TILE, MT, WPE)                                                                \
    extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE))) void NAME(MmqArgs args) { \
        __shared__ __attribute__((aligned(16))) u4_t a0[mmqh::Tile<MT>::kAct / 16u];                          \
        __shared__ __attribute__((aligned(16))) u4_t a1[mmqh::Tile<MT>::kAct / 16u];                          \
        __shared__ __attribute__((aligned(16))) u4_t a2[mmqh::Tile<MT>::kAct / 16u];                          \
        __shared__ __attribute__((aligned(16))) u4_t a3[mmqh::Tile<MT>::kAct / 16u];                          \
        __shared__ __attribute__((aligned(16))) u4_t sx[mmqh::kThreads];                                     \
        __shared__ __attribute__((aligned(16))) float sc[mmqh::Tile<MT>::BM];                                \
        if (blockDim.x != mmqh::kThreads) return; /* the tile assumes exactly kThreads lanes */               \
        const uint32_t tiles = min(gridDim.x, mmq_tile_count(args));                                        \
        if (blockIdx.x >= tiles) return;                                                                     \
        const uint32_t b = mmqh::xcd_tile(blockIdx.x, tiles);                                               \
        const MmqDesc d = mmq_pick(args, b);                                                                 \
        if (b - d.wg_begin >= d.tiles_m * d.tiles_n * d.splits) return;                                     \
        const mmqh::ActLds lds{{a0, a1, a2, a3}, sx, sc};                                                    \
        mmqh_tile<MT, TILE>(d, b - d.wg_begin, lds);                                                          \
    }
RFXQ_MMQH_ENTRY(rfxq_mmqh_q4k, TY_Q4K, 4, 2)
RFXQ_MMQH_ENTRY(rfxq_mmqh_q4k_m32, TY_Q4K, 1, 4)
RFXQ_MMQH_ENTRY(rfxq_mmqh_q4k_m64, TY_Q4K, 2, 3)

// One (32 MT)x256 tile (and one split-K range) of Y = X . W^T for Q6_K weights:
// the Q4_K tile's layout and pipeline, with the Q6_K weight operands.
template <int MT>
RFXQ_DEV void mmqh_q6k_rows(const MmqDesc& ds, uint32_t m0, uint32_t n0, uint32_t ks, const mmqh::ActLds& ls) {
    using namespace mmqh;
    constexpr uint32_t BM = Tile<MT>::BM;
    // weight loads per stage: the ql pieces; the qh pieces at even positions;
    // the scales and d at position 0
    constexpr int WA = MT == 4 ? 1 : 2;  // (128-row tiles: two stages of registers would spill)
    using Pipe = StagePipe<MT, WA, 8, 2, 4, 2, 0>;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, h = lane >> 5;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsb = ds.k / 256u;
    const uint32_t sb0 = ks * ds.sb_per_split;
    const uint32_t sb1 = min(nsb, sb0 + ds.sb_per_split);
    const uint32_t row_bytes = nsb * 210u;  // 2 mod 4 for an odd nsb

    // The weights' buffer starts at the dword at or below the tile's first
    // column (2-byte aligned); sh0 = the bytes between. Columns start 0 or 2
    // bytes past a dword, super-blocks too: the 16-byte pieces are read with
    // unaligned loads. Columns past the matrix read zeros.
    const uintptr_t wa = reinterpret_cast<uintptr_t>(ds.w + (uint64_t)n0 * row_bytes);
    const uint32_t sh0 = (uint32_t)(wa & 3u);
    const uint32_t rb = act_base(ds, m0);
    const rsrc_t r_act = make_rsrc(ds.xq + (uint64_t)rb * ds.ldq, 0xFFFFFFFFu);
    const rsrc_t r_w = make_rsrc(reinterpret_cast<const void*>(wa - sh0), min(BN, ds.n - n0) * row_bytes + sh0);
    const uint32_t ra = tid >> 3;
    // activations: the Q4_K tile's staging, but the stage's logical chunks 4-7
    // (group B) sit 128 bytes after chunks 0-3 (group A) in the f16 row
    uint32_t g_act[MT];
    const uint32_t lc = act_chunk(tid), cofs = 16u * lc + (lc >= 4u ? 64u : 0u);
#pragma unroll
    for (int u = 0; u < MT; u++) g_act[u] = (act_row(ds, m0 + ra + 32u * u) - rb) * ds.ldq + cofs;
    // Weights straight to registers: lane (l32, h) of n-tile j loads, per
    // stage, positions [16h, 16h + 16) of the ql and qh pieces of column
    // 64w + 32j + l32 (five dwords each), and with the first stage of a
    // super-block its scales and d.
    uint32_t col[2], g_c[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        col[j] = 64u * w + 32u * j + l32;
        g_c[j] = col[j] * row_bytes + 16u * h;
    }
    const uint32_t nst = 4u * (sb1 - sb0);

    // ql pieces of WA stages (by stage); qh, scales and d are copied out in
    // the stage that issues their next load
    u4_t qln[WA][2], qhn[2], scn[2];
    uint32_t dn[2];
    auto copy_act = [&](uint32_t st, u4_t* buf) {
        const uint32_t sl = min(st, nst - 1u);
        const uint32_t sb = sb0 + (sl >> 2), g = sl & 3u;
        const uint32_t n = g >> 1, s = g & 1u;
#pragma unroll
        for (int u = 0; u < MT; u++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_act, RFXQ_LDSP(buf + 256u * u + 64u * w), 16, g_act[u],
                                                     512u * sb + 256u * n + 64u * s, 0, 0);
    };
    // 16-byte loads at 2-byte-aligned offsets (unaligned access mode)
    auto load_w = [&](uint32_t st) {
        const uint32_t sl = min(st, nst - 1u);
        const uint32_t sb = sb0 + (sl >> 2), g = sl & 3u;
        const uint32_t n = g >> 1, s = g & 1u;
        const uint32_t base = 210u * sb + sh0;
        // the qh piece of half n serves both of its stages: loaded with s = 0
#pragma unroll
        for (int j = 0; j < 2; j++) {
            qln[st % WA][j] = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_c[j], base + 64u * n + 32u * s, 0);
            if ((st & 1u) == 0u) qhn[j] = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_c[j], base + 128u + 32u * n, 0);
        }
        if ((st & 3u) == 0u) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                scn[j] = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_c[j] - 16u * h, base + 192u, 0);
                dn[j] = __builtin_amdgcn_raw_buffer_load_b16(r_w, g_c[j] - 16u * h, base + 208u, 0);
            }
        }
    };

    v16f_t acc[MT][2];
#pragma unroll
    for (int i = 0; i < MT; i++) acc[i][0] = acc[i][1] = v16f_t{};
    uint32_t a_act[2][2];
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) a_act[e][s2] = l32 * 8u + ((4u * e + 2u * h + s2) ^ ((l32 >> 1) & 7u));
    u4_t mult[2] = {}, L[2], Q[2];
    uint32_t mla = 0x000F000Fu, mqa = 0x00300030u, mlb = 0x00F000F0u, mqb = 0x03000300u, mg = 0x64006400u;
    asm("" : "+v"(mla), "+v"(mqa), "+v"(mlb), "+v"(mqb), "+v"(mg));

    float row_scale = 0.0f;  // written to LDS after the loop (as for Q4_K)
    if (tid < BM && m0 + tid < ds.m) row_scale = as_f32(bld4(make_rsrc(ds.xrs, 0xFFFFFFFFu), 4u * act_row(ds, m0 + tid)));
    copy_act(0u, ls.a[0]);
    if constexpr (WA == 1) {
        copy_act(1u, ls.a[1]);
        load_w(0u);
    } else {
        load_w(0u);
        copy_act(1u, ls.a[1]);
        load_w(1u);
    }
    copy_act(2u, ls.a[2]);
    Pipe::prologue_end();
    for (uint32_t st0 = 0; st0 < nst; st0 += 4u) {
#pragma unroll
        for (uint32_t g = 0; g < 4u; g++) {
            const uint32_t st = st0 + g;
            const uint32_t n = g >> 1, s = g & 1u;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                L[j] = qln[g % WA][j];
                if (s == 0u) Q[j] = qhn[j];
                if (g == 0u) mult[j] = q6k_multipliers(scn[j], dn[j], h);
            }
            load_w(st + WA);
            copy_act(st + 3u, ls.a[(g + 3u) & 3u]);
            const u4_t* S16 = ls.a[g];
            // groups A (e = 0) and B (e = 1): multipliers i = 4n + s + 2e
            uint32_t sm[2][2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                sm[0][j] = s ? splat16<1>(mult[j][2 * n]) : splat16<0>(mult[j][2 * n]);
                sm[1][j] = s ? splat16<1>(mult[j][2 * n + 1]) : splat16<0>(mult[j][2 * n + 1]);
            }
            // shifted copies of the stage's code dwords (see q6k_codes_f16)
            uint32_t Ls[2][4], Qa[2][4], Qb[2][4];
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    Ls[j][u] = L[j][u] >> 8;
                    Qa[j][u] = s ? Q[j][u] << 2 : Q[j][u] << 4;
                    Qb[j][u] = s ? Q[j][u] >> 6 : Q[j][u] >> 4;
                }
            auto wop = [&](int t, int j) {
                const int e = t >> 1, u = 2 * (t & 1);
                if (e == 0)
                    return q6k_codes_f16<0>(L[j][u], L[j][u + 1], Ls[j][u], Ls[j][u + 1], Qa[j][u], Qa[j][u + 1],
                                            Qb[j][u], Qb[j][u + 1], sm[0][j], mla, mqa, mg);
                return q6k_codes_f16<1>(L[j][u], L[j][u + 1], Ls[j][u], Ls[j][u + 1], Qa[j][u], Qa[j][u + 1],
                                        Qb[j][u], Qb[j][u + 1], sm[1][j], mlb, mqb, mg);
            };
            u4_t Xc[MT], Wc[2];
#pragma unroll
            for (int i = 0; i < MT; i++) Xc[i] = S16[256u * i + a_act[0][0]];
            Wc[0] = wop(0, 0);
            Wc[1] = wop(0, 1);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                u4_t Xn[MT], Wn[2];
                if (t < 3) {
                    const int e = (t + 1) >> 1, s2 = (t + 1) & 1;
#pragma unroll
                    for (int i = 0; i < MT; i++) Xn[i] = S16[256u * i + a_act[e][s2]];
                    Wn[0] = wop(t + 1, 0);
                    Wn[1] = wop(t + 1, 1);
                }
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    acc[i][0] = mfma16(Wc[0], Xc[i], acc[i][0]);
                    acc[i][1] = mfma16(Wc[1], Xc[i], acc[i][1]);
                }
                if (t < 3) {
#pragma unroll
                    for (int u = 0; u < MT; u++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                    }
#pragma unroll
                    for (int u = 0; u < MT; u++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < MT; i++) Xc[i] = Xn[i];
                    Wc[0] = Wn[0];
                    Wc[1] = Wn[1];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            Pipe::stage_end(g);
        }
    }
    // no copy may land in LDS after the workgroup is gone
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (tid < BM) ls.sc[tid] = row_scale;
    lds_barrier();

    float* y = ds.y + (uint64_t)ks * ds.m * ds.ldy;
    const float* sc = ls.sc;
    store_wave<MT>(ds, y, m0, n0 + 64u * w, acc, sc, pick_buf(ls.a[0], ls.a[1], ls.a[2], ls.a[3], w));
}

RFXQ_MMQH_ENTRY(rfxq_mmqh_q6k, TY_Q6K, 4, 2)
RFXQ_MMQH_ENTRY(rfxq_mmqh_q6k_m32, TY_Q6K, 1, 3)
RFXQ_MMQH_ENTRY(rfxq_mmqh_q6k_m64, TY_Q6K, 2, 2)

// ---------------------------------------------------------------- Q8_0
//
// A Q8_0 block (src/dequant.rs:220-226) is an f16 d and 32 int8 codes:
// w = d * q. The weight operand is f16(q * d), rounded once from an exact
// product: the code byte, its sign bit flipped (q + 128), is permuted into
// the mantissa of an f16 1024.0 (1024 + q + 128), an exact add of -1152
// leaves q, and one multiply by the f16 pair (d, d) rounds. A 64-k stage is
// two blocks (e = 0, 1); lane half h holds codes [16h, 16h + 16) of each, so
// step t = 2e + s2 takes codes 32e + 16h + 8 s2 + [0, 8), the activations'
// logical chunk 4e + 2h + s2, as for Q4_K. Blocks are 34 bytes, so the
// stage's block pair (68 bytes) starts on a dword when the weights do: then
// lane half h reads it with dword-aligned loads (bytes [16h, +20) and
// [36 + 16h, +16), and the dword holding the d of the other half) and shifts
// block 0's codes by two bytes (v_alignbyte; unaligned 16-byte loads ran the
// kernel ~1.5x slower). Weights that start 2 bytes past a dword take the
// unaligned loads. Split-K ranges count in units of 256 weights (8 blocks,
// four stages), as for the K-quants.

namespace mmqh {
// f16 pairs f16(q * d) of one code dword v (bytes q0..q3, signs flipped by
// the caller: v ^ 0x80808080) in the activations' (q0, q2), (q1, q3) order
RFXQ_DEV u2_t q80_codes_f16(uint32_t v, h2_t dv, uint32_t mg) {
    const h2_t off = h2_t{(half_t)-1152.0f, (half_t)-1152.0f};
    h2_t a = as_h2(__builtin_amdgcn_perm(mg, v, 0x04020400u)) + off;
    h2_t b = as_h2(__builtin_amdgcn_perm(mg, v, 0x04030401u)) + off;
    asm("" : "+v"(a), "+v"(b));  // keep the exact adds and the rounding multiplies apart (no fma)
    return u2_t{h2_bits(a * dv), h2_bits(b * dv)};
}
}  // namespace mmqh

// One (32 MT)x256 tile (and one split-K range) of Y = X . W^T for Q8_0 weights:
// the Q4_K tile's activation staging and MFMA schedule, with Q8_0 operands.
template <int MT, bool AL>
RFXQ_DEV void mmqh_q80_rows_t(const MmqDesc& ds, uint32_t m0, uint32_t n0, uint32_t ks, const mmqh::ActLds& ls) {
    using namespace mmqh;
    constexpr uint32_t BM = Tile<MT>::BM;
    // weights two stages ahead in the 96- and 128-row bodies; one in the
    // smaller ones, whose entries cap the registers lower
    constexpr int WA = MT >= 3 ? 2 : 1;
    using Pipe = StagePipe<MT, WA, 8, 8, 8, 8, 0>;  // weight loads: four per column and stage
    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, h = lane >> 5;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsb = ds.k / 256u;
    const uint32_t sb0 = ks * ds.sb_per_split;
    const uint32_t sb1 = min(nsb, sb0 + ds.sb_per_split);
    const uint32_t row_bytes = nsb * 272u;

    // weights: the dword at or below the tile's first column (2-byte aligned)
    const uintptr_t wa = reinterpret_cast<uintptr_t>(ds.w + (uint64_t)n0 * row_bytes);
    const uint32_t sh0 = (uint32_t)(wa & 3u);
    const uint32_t rb = act_base(ds, m0);
    const rsrc_t r_act = make_rsrc(ds.xq + (uint64_t)rb * ds.ldq, 0xFFFFFFFFu);
    const rsrc_t r_w = make_rsrc(reinterpret_cast<const void*>(wa - sh0), min(BN, ds.n - n0) * row_bytes + sh0);
    const uint32_t ra = tid >> 3;
    uint32_t g_act[MT];
#pragma unroll
    for (int u = 0; u < MT; u++) g_act[u] = (act_row(ds, m0 + ra + 32u * u) - rb) * ds.ldq + 16u * act_chunk(tid);
    // lane (l32, h) of n-tile j: column 64w + 32j + l32, codes [16h, +16) of
    // each block, and each block's d
    // (the lane-varying parts of an offset go in the VGPR offset: a
    // lane-varying SGPR offset would make the compiler loop over lanes)
    uint32_t g_c[2], g_q[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        g_c[j] = (64u * w + 32u * j + l32) * row_bytes + sh0;
        g_q[j] = g_c[j] + (AL ? 16u * h : 2u + 16u * h);
    }
    const uint32_t e_off = h ? 0u : 32u;  // aligned form: the dword with the other half's d
    const uint32_t nst = 4u * (sb1 - sb0);

    // raw stage data per column, of two stages (by stage parity): unaligned
    // form qn = codes of blocks 0, 1 and dn = their d; aligned form qn[0] =
    // bytes [16h, +16), qn[1] = bytes [36 + 16h, +16), dn[0] = the dword after
    // qn[0], dn[1] = the other d's dword
    u4_t qn_[WA][2][2];
    uint32_t dn_[WA][2][2];
    auto copy_act = [&](uint32_t st, u4_t* buf) {
        const uint32_t sl = min(st, nst - 1u);
        const uint32_t sb = sb0 + (sl >> 2), g = sl & 3u;
#pragma unroll
        for (int u = 0; u < MT; u++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_act, RFXQ_LDSP(buf + 256u * u + 64u * w), 16, g_act[u],
                                                     512u * sb + 128u * g, 0, 0);
    };
    auto load_w = [&](uint32_t st) {
        const uint32_t sl = min(st, nst - 1u);
        auto& qn = qn_[st % WA];
        auto& dn = dn_[st % WA];
        const uint32_t blk = 8u * sb0 + 2u * sl;  // the stage's first block in the row
        if constexpr (AL) {
            const uint32_t o = 34u * blk;  // dword aligned (blk is even)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                qn[j][0] = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_q[j], o, 0);
                dn[j][0] = __builtin_amdgcn_raw_buffer_load_b32(r_w, g_q[j], o + 16u, 0);
                qn[j][1] = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_q[j], o + 36u, 0);
                dn[j][1] = __builtin_amdgcn_raw_buffer_load_b32(r_w, g_c[j] + e_off, o, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t o = 34u * (blk + e);
                    qn[j][e] = __builtin_amdgcn_raw_buffer_load_b128(r_w, g_q[j], o, 0);
                    dn[j][e] = __builtin_amdgcn_raw_buffer_load_b16(r_w, g_c[j], o, 0);
                }
        }
    };

    v16f_t acc[MT][2];
#pragma unroll
    for (int i = 0; i < MT; i++) acc[i][0] = acc[i][1] = v16f_t{};
    uint32_t a_act[2][2];
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) a_act[e][s2] = l32 * 8u + ((4u * e + 2u * h + s2) ^ ((l32 >> 1) & 7u));
    uint32_t mg = 0x64646464u, sgn = 0x80808080u;
    asm("" : "+v"(mg), "+v"(sgn));

    float row_scale = 0.0f;  // written to LDS after the loop (as for Q4_K)
    if (tid < BM && m0 + tid < ds.m) row_scale = as_f32(bld4(make_rsrc(ds.xrs, 0xFFFFFFFFu), 4u * act_row(ds, m0 + tid)));
    copy_act(0u, ls.a[0]);
    if constexpr (WA == 1) {
        copy_act(1u, ls.a[1]);
        load_w(0u);
    } else {
        load_w(0u);
        copy_act(1u, ls.a[1]);
        load_w(1u);
    }
    copy_act(2u, ls.a[2]);
    Pipe::prologue_end();
    for (uint32_t st0 = 0; st0 < nst; st0 += 4u) {
#pragma unroll
        for (uint32_t g = 0; g < 4u; g++) {
            const uint32_t st = st0 + g;
            const auto& qn = qn_[g % WA];
            const auto& dn = dn_[g % WA];
            u4_t q[2][2];
            h2_t dv[2][2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if constexpr (AL) {
                    const u4_t a = qn[j][0];
                    const uint32_t b = dn[j][0], e = dn[j][1];
                    q[j][0] = u4_t{alignbyte(a.y, a.x, 2u), alignbyte(a.z, a.y, 2u), alignbyte(a.w, a.z, 2u),
                                   alignbyte(b, a.w, 2u)} ^ u4_t{sgn, sgn, sgn, sgn};
                    q[j][1] = qn[j][1] ^ u4_t{sgn, sgn, sgn, sgn};
                    dv[j][0] = as_h2(splat16<0>(h ? e : a.x));
                    dv[j][1] = as_h2(h ? splat16<1>(b) : splat16<1>(e));
                } else {
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        q[j][e] = qn[j][e] ^ u4_t{sgn, sgn, sgn, sgn};
                        dv[j][e] = as_h2(splat16<0>(dn[j][e]));
                    }
                }
            }
            load_w(st + WA);
            copy_act(st + 3u, ls.a[(g + 3u) & 3u]);
            const u4_t* S16 = ls.a[g];
            auto wop = [&](int t, int j) {
                const int e = t >> 1, s2 = t & 1;
                const u2_t lo = q80_codes_f16(q[j][e][2 * s2], dv[j][e], mg);
                const u2_t hi = q80_codes_f16(q[j][e][2 * s2 + 1], dv[j][e], mg);
                return u4_t{lo.x, lo.y, hi.x, hi.y};
            };
            u4_t Xc[MT], Wc[2];
#pragma unroll
            for (int i = 0; i < MT; i++) Xc[i] = S16[256u * i + a_act[0][0]];
            Wc[0] = wop(0, 0);
            Wc[1] = wop(0, 1);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                u4_t Xn[MT], Wn[2];
                if (t < 3) {
                    const int e = (t + 1) >> 1, s2 = (t + 1) & 1;
#pragma unroll
                    for (int i = 0; i < MT; i++) Xn[i] = S16[256u * i + a_act[e][s2]];
                    Wn[0] = wop(t + 1, 0);
                    Wn[1] = wop(t + 1, 1);
                }
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    acc[i][0] = mfma16(Wc[0], Xc[i], acc[i][0]);
                    acc[i][1] = mfma16(Wc[1], Xc[i], acc[i][1]);
                }
                if (t < 3) {
#pragma unroll
                    for (int u = 0; u < MT; u++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                    }
#pragma unroll
                    for (int u = 0; u < MT; u++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < MT; i++) Xc[i] = Xn[i];
                    Wc[0] = Wn[0];
                    Wc[1] = Wn[1];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            Pipe::stage_end(g);
        }
    }
    // no copy may land in LDS after the workgroup is gone
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (tid < BM) ls.sc[tid] = row_scale;
    lds_barrier();

    float* y = ds.y + (uint64_t)ks * ds.m * ds.ldy;
    const float* sc = ls.sc;
    store_wave<MT>(ds, y, m0, n0 + 64u * w, acc, sc, pick_buf(ls.a[0], ls.a[1], ls.a[2], ls.a[3], w));
}

template <int MT>
RFXQ_DEV void mmqh_q80_rows(const MmqDesc& ds, uint32_t m0, uint32_t n0, uint32_t ks, const mmqh::ActLds& lds) {
    if ((reinterpret_cast<uintptr_t>(ds.w) & 3u) == 0u) mmqh_q80_rows_t<MT, true>(ds, m0, n0, ks, lds);
    else mmqh_q80_rows_t<MT, false>(ds, m0, n0, ks, lds);
}

RFXQ_MMQH_ENTRY(rfxq_mmqh_q8_0, TY_Q8_0, 4, 2)
RFXQ_MMQH_ENTRY(rfxq_mmqh_q8_0_m32, TY_Q8_0, 1, 4)
RFXQ_MMQH_ENTRY(rfxq_mmqh_q8_0_m64, TY_Q8_0, 2, 3)

// One launch of 32-row tiles over GEMMs of Q4_K and Q6_K weights (a layer's
// Q4_K projections with its Q6_K v / down at a few rows): each tile runs the
// body of its descriptor's type (a uniform branch; the same code and results
// as the per-type entries), so a few-row layer is one launch, not two (one
// Qwen3-0.6B layer at 12 rows: 28.8 -> 19.3 us). Not for the larger tiles:
// the 128-row bodies together spill registers (the 0.6B set at 512 rows gained
// nothing, and an 8B layer, whose Q6_K GEMMs then lose their split-K, lost
// 8%), and the 64-row ones run at different occupancies per type.
#define RFXQ_MMQH_MIX_ENTRY(NAME, MT, WPE)                                                                  \
    extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE))) void NAME(MmqArgs args) { \
        __shared__ __attribute__((aligned(16))) u4_t a0[mmqh::Tile<MT>::kAct / 16u];                          \
        __shared__ __attribute__((aligned(16))) u4_t a1[mmqh::Tile<MT>::kAct / 16u];                          \
        __shared__ __attribute__((aligned(16))) u4_t a2[mmqh::Tile<MT>::kAct / 16u];                          \
        __shared__ __attribute__((aligned(16))) u4_t a3[mmqh::Tile<MT>::kAct / 16u];                          \
        __shared__ __attribute__((aligned(16))) u4_t sx[mmqh::kThreads];                                     \
        __shared__ __attribute__((aligned(16))) float sc[mmqh::Tile<MT>::BM];                                \
        if (blockDim.x != mmqh::kThreads) return; /* the tile assumes exactly kThreads lanes */               \
        const uint32_t tiles = min(gridDim.x, mmq_tile_count(args));                                        \
        if (blockIdx.x >= tiles) return;                                                                     \
        const uint32_t b = mmqh::xcd_tile(blockIdx.x, tiles);                                               \
        const MmqDesc d = mmq_pick(args, b);                                                                 \
        if (b - d.wg_begin >= d.tiles_m * d.tiles_n * d.splits) return;                                     \
        const mmqh::ActLds lds{{a0, a1, a2, a3}, sx, sc};                                                    \
        const uint32_t ty = __builtin_amdgcn_readfirstlane(d.type);                                         \
        if (ty == TY_Q6K) mmqh_tile<MT, TY_Q6K>(d, b - d.wg_begin, lds);                                      \
        else mmqh_tile<MT, TY_Q4K>(d, b - d.wg_begin, lds);                                                    \
    }
RFXQ_MMQH_MIX_ENTRY(rfxq_mmqh_mix_m32, 1, 3)
