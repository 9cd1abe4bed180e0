// Q4_K prefill GEMM on exact f16 MFMAs with a transposed tile: the default
// Q4_K kernel of the MMQ path (src/kernels_cuda/gemm_q_mma.cu:299-764 is the
// reference's f16 prefill kernel it replaces; same call sites as mmq.hpp).
//
// Inputs are the same Q8_1 activations as the int8 kernel, in two derived
// layouts written by the quantizer: xh, the int8 values as f16 (group of four
// stored (q0, q2), (q1, q3)), and xsc, one 64-byte record per row and
// super-block: da[8] (the blocks' f16 scales), then Sx' = Sx * 2^-6 split
// exactly into f16 hi[8] and lo[8] (Sx = da * s, the block's activation sum,
// f32-exact; hi = f16(Sx'), lo = f16(Sx' - hi); the 2^-6 keeps sums up to 4e6
// in range and is undone by the 2^6 in the integer scale operands).
//
// For a Q4_K super-block with d, dmin, 6-bit (sc_b, m_b) and codes q:
//   w = d*sc_b*(q - 8) + (8*d*sc_b - dmin*m_b)
//   y[i,j] += d[j] * ( sum_b da_b[i] * D_b[i,j] + sum_b 8*sc_b[j]*Sx_b[i] )
//           - dmin[j] * sum_b m_b[j]*Sx_b[i]
// with D_b = sum_{k in b} qa[i,k] * sc_b[j]*(q[j,k] - 8). Every operand of
// D_b is an integer that f16 holds exactly (|qa| <= 127, |sc*(q-8)| <= 504),
// so the two 32x32x16 f16 MFMAs of a block return D_b exactly in f32
// (|D_b| <= 32*127*504 < 2^24), the same integers as the int8 kernel's
// block dots scaled by sc_b. The sums over b of 8*sc_b*Sx_b and m_b*Sx_b are
// one f16 MFMA each per super-block (K = 16 slots: hi and lo halves of Sx
// against the integer scales), exact products summed in f32.
//
// Per element the VALU does one FMA per 32-block (t += D_b * da_b, da_b one
// f32 value per lane because the lane owns one activation row) and two per
// super-block (acc += d*t, acc -= dmin*v): about half of the int8 kernel's
// epilogue (convert + FMA per block, plus a scale-product MFMA).
//
// Tile: 128 activation rows x 128 weight columns per 256-thread workgroup;
// wave w owns weight columns [32w, +32) against all 128 rows (four 32x32
// MFMA tiles, A = weights, B = activations, so lane l holds row l%32 of its
// tile and 16 weight columns). Operands stream through LDS by asynchronous
// copies (buffer_load ... lds) in a 3-slot ring of block pairs (K = 64):
// slot = activations [128][64] f16 (16 KB, 16-byte chunks XOR-swizzled by
// row) + weight quants [128][32 B] (4 KB) + da of the pair [128][2] (512 B).
// Super-block headers and Sx records ride with the pair g = 0 copy into a
// single buffer that is read only while that pair is current.
#pragma once
#include "common.hpp"
#include "mmq.hpp"

namespace mmq2 {

constexpr uint32_t BM = 128, BN = 128;
constexpr uint32_t kAct = 16384, kCodes = 4096, kDa = 512;
constexpr uint32_t kSlot = kAct + kCodes + kDa;
constexpr uint32_t kHdr = 2048, kSx = 4096, kTab = 512;
constexpr uint32_t kLds = 3 * kSlot + kHdr + kSx + kTab;

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

// two small integers (exact in f16) as an f16 pair, low half first
RFXQ_DEV uint32_t int_pair_f16(uint32_t lo, uint32_t hi) {
    const h2_t x = {(half_t)(float)lo, (half_t)(float)hi};
    return h2_bits(x);
}

// Q4_K scales of sub-blocks 0..7 (get_scale_min_k4, src/dequant.rs:39-47) as
// the A operands of the super-block constant MFMAs: 8*sc_b*2^6 and m_b*2^6,
// f16 (exact: at most 6 significant bits), against the activations' Sx*2^-6
RFXQ_DEV void q4k_const_operands(const u4_t hdr, u4_t& usc, u4_t& um) {
    uint32_t sc[8], m[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        sc[j] = (hdr.y >> (8 * j)) & 63u;
        m[j] = (hdr.z >> (8 * j)) & 63u;
        sc[j + 4] = ((hdr.w >> (8 * j)) & 0xFu) | (((hdr.y >> (8 * j + 6)) & 3u) << 4);
        m[j + 4] = ((hdr.w >> (8 * j + 4)) & 0xFu) | (((hdr.z >> (8 * j + 6)) & 3u) << 4);
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {
        usc[p] = int_pair_f16(512u * sc[2 * p], 512u * sc[2 * p + 1]);
        um[p] = int_pair_f16(64u * m[2 * p], 64u * m[2 * p + 1]);
    }
}

// f16 operands sc*(q - 8) of one 16-k step from the step's two quant dwords:
// the nibble is placed at bits 4-7 of an f16 1024.0 (1024 + 16q), then
// (1024 + 16q) * (sc/16) - 72*sc = sc*(q - 8), exact. tab = (sc/16, -72*sc)
// as f16 pairs. Pairs follow the activations' (q0, q2), (q1, q3) order.
template <int E>
RFXQ_DEV u4_t q4k_step_codes(uint32_t v0, uint32_t v1, u2_t tab) {
    const uint32_t M = 0x00F000F0u, MG = 0x64006400u;
    uint32_t w[4];
    if (E == 0) {  // low nibbles
        w[0] = ((v0 << 4) & M) | MG;
        w[1] = ((v0 >> 4) & M) | MG;
        w[2] = ((v1 << 4) & M) | MG;
        w[3] = ((v1 >> 4) & M) | MG;
    } else {       // high nibbles
        w[0] = (v0 & M) | MG;
        w[1] = ((v0 >> 8) & M) | MG;
        w[2] = (v1 & M) | MG;
        w[3] = ((v1 >> 8) & M) | MG;
    }
    const h2_t s = as_h2(tab.x), o = as_h2(tab.y);
    u4_t r;
#pragma unroll
    for (int t = 0; t < 4; t++) r[t] = h2_bits(__builtin_elementwise_fma(as_h2(w[t]), s, o));
    return r;
}

}  // namespace mmq2

// One 128x128 tile (and one split-K range) of Y = X . W^T for Q4_K weights.
RFXQ_DEV void mmq2_q4k_tile(const MmqDesc& dv, uint32_t t_local, uint8_t* lds) {
    using namespace mmq2;
    // the descriptor is wave-uniform: keep every field in SGPRs
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
    const uint32_t rec_bytes = nsb * 64u;  // xsc row

    const uint32_t L = __builtin_amdgcn_readfirstlane(lds_addr(lds));
    const uint32_t Lhdr = L + 3u * kSlot, Lsx = Lhdr + kHdr;

    // (sc/16, -72*sc) f16 pairs for sc in [0, 64)
    if (tid < 64u) {
        const h2_t s = {(half_t)((float)tid * 0.0625f), (half_t)((float)tid * 0.0625f)};
        const h2_t o = {(half_t)(-72.0f * (float)tid), (half_t)(-72.0f * (float)tid)};
        reinterpret_cast<u2_t*>(lds + 3u * kSlot + kHdr + kSx)[tid] = u2_t{h2_bits(s), h2_bits(o)};
    }
    __syncthreads();

    // copy sources and per-lane offsets. Rows and columns past the matrix
    // read past the buffer (zeros, no fault): nothing is clamped.
    const sdesc_t r_act = uniform_desc(ds.xq, ds.m * ds.ldq);
    const sdesc_t r_w = uniform_desc(ds.w, ds.n * row_bytes);
    const sdesc_t r_sc = uniform_desc(ds.xds, ds.m * rec_bytes);
    // activations: copy q of wave w fills rows r = 32w + 8q + lane/8; LDS
    // chunk lane%8 of row r holds logical chunk (lane%8) ^ swz(r) with
    // swz(r) = (r/2)%8 = (lane/16) ^ (4 if q is odd), so 16 consecutive rows
    // read at one logical chunk cover all 64 banks
    const uint32_t o_row = (m0 + 32u * w + (lane >> 3)) * ds.ldq;
    const uint32_t o_act[2] = {o_row + 16u * ((lane & 7u) ^ (lane >> 4)), o_row + 16u * ((lane & 7u) ^ (lane >> 4) ^ 4u)};
    const uint32_t s64 = 64u * w + lane;
    // weight quants: slot s = 2*col + p holds 16-byte half p ^ ((col/8) & 1)
    const uint32_t o_codes = (n0 + (s64 >> 1)) * row_bytes + 16u + 16u * ((s64 & 1u) ^ ((s64 >> 4) & 1u));
    const uint32_t o_da = (m0 + 32u * w + l32) * rec_bytes;
    const uint32_t o_hdr = (n0 + 32u * w + l32) * row_bytes;
    const uint32_t o_sx = (m0 + (s64 & 127u)) * rec_bytes + 16u + 16u * (s64 >> 7);
    const uint32_t nst = 4u * (sb1 - sb0);
    // copies of stage st: 6 per wave, 8 when it opens a super-block (the
    // 4-byte and header copies run on lanes 0-31)
    auto issue = [&](uint32_t st) {
        const uint32_t sb = sb0 + (st >> 2), g = st & 3u, slot = st % 3u;
        const uint32_t Ls = __builtin_amdgcn_readfirstlane(L + slot * kSlot);
#pragma unroll
        for (int q = 0; q < 4; q++)
            dma16(r_act, Ls + 1024u * (4u * w + q), o_act[q & 1], 512u * sb + 128u * g + 8u * q * ds.ldq);
        dma16(r_w, Ls + kAct + 1024u * w, o_codes, 144u * sb + 32u * g);
        if (h == 0u) dma4(r_sc, Ls + kAct + kCodes + 128u * w, o_da, 64u * sb + 4u * g);
        if (g == 0u) {
            if (h == 0u) dma16(r_w, Lhdr + 512u * w, o_hdr, 144u * sb);
            dma16(r_sc, Lsx + 1024u * w, o_sx, 64u * sb);
        }
    };

    v16f_t acc[4], t[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        acc[i] = v16f_t{};
        t[i] = v16f_t{};
    }
    // LDS read offsets (16-byte units) of the lane: activations of row l32 of
    // row tile 0, chunk 4e + 2h + step; weight quants of column 32w + l32
    uint32_t a_act[2][2];
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) a_act[e][s2] = l32 * 8u + ((4u * e + 2u * h + s2) ^ ((l32 >> 1) & 7u));
    const uint32_t col = 32u * w + l32;
    const uint32_t a_codes = kAct / 16u + col * 2u + (h ^ ((col >> 3) & 1u));
    const uint32_t a_da = (kAct + kCodes) / 4u + l32;
    const u2_t* tab = reinterpret_cast<const u2_t*>(lds + 3u * kSlot + kHdr + kSx);
    u4_t hdr = {};

    if (nst > 0u) issue(0u);
    if (nst > 1u) issue(1u);
    for (uint32_t st = 0; st < nst; st++) {
        // own copies of stage st done (those of st + 1 may remain), then
        // everyone's; slot (st + 2) % 3 is free once all waves pass
        if (st + 1u < nst) {
            if (((st + 1u) & 3u) == 0u) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (st + 2u < nst) issue(st + 2u);

        const uint32_t g = st & 3u;
        const uint8_t* S = lds + (st % 3u) * kSlot;
        const u4_t* S16 = reinterpret_cast<const u4_t*>(S);
        if (g == 0u) {
            // super-block start: header of the lane's weight column, constant
            // part -dmin * sum m_b Sx_b into acc and 8 sum sc_b Sx_b into t
            hdr = reinterpret_cast<const u4_t*>(lds + 3u * kSlot)[col];
            u4_t usc, um;
            q4k_const_operands(hdr, usc, um);
            uint32_t dd[16];
#pragma unroll
            for (int r = 0; r < 16; r++) dd[r] = bperm(8u * (r >> 2) + 4u * h + (r & 3), hdr.x);
            const u4_t* sxp = reinterpret_cast<const u4_t*>(lds + 3u * kSlot + kHdr) + 128u * h + l32;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const u4_t sxo = sxp[32 * i];
                t[i] = mfma16(usc, sxo, v16f_t{});
                const v16f_t v = mfma16(um, sxo, v16f_t{});
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][r] = __builtin_fmaf(v[r], -f16_opaque(dd[r] >> 16), acc[i][r]);
            }
        }
        const uint32_t* da_p = reinterpret_cast<const uint32_t*>(S) + a_da;
        uint32_t da[4];
#pragma unroll
        for (int i = 0; i < 4; i++) da[i] = da_p[32 * i];
        const u4_t q = S16[a_codes];
        uint32_t sc0, sc1;
        q4k_pair_sc(hdr, g, sc0, sc1);
        const u2_t tab0 = tab[sc0], tab1 = tab[sc1];
        // weight operands of both blocks (2g: low nibbles, 2g + 1: high) and
        // both 16-k steps
        const u4_t w00 = q4k_step_codes<0>(q.x, q.y, tab0), w01 = q4k_step_codes<0>(q.z, q.w, tab0);
        const u4_t w10 = q4k_step_codes<1>(q.x, q.y, tab1), w11 = q4k_step_codes<1>(q.z, q.w, tab1);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u4_t* xp = S16 + 256u * i;  // row tile i: 32 rows x 128 B
            const v16f_t D0 = mfma16(w01, xp[a_act[0][1]], mfma16(w00, xp[a_act[0][0]], v16f_t{}));
            const v16f_t D1 = mfma16(w11, xp[a_act[1][1]], mfma16(w10, xp[a_act[1][0]], v16f_t{}));
            // the block scales as f32 once (v_fma_mix_f32 with an f16 operand
            // issues at a lower rate than v_fmac_f32)
            const float da0 = f16_opaque(da[i]), da1 = f16_opaque(da[i] >> 16);
#pragma unroll
            for (int r = 0; r < 16; r++) t[i][r] = __builtin_fmaf(D1[r], da1, __builtin_fmaf(D0[r], da0, t[i][r]));
        }
        if (g == 3u) {
            uint32_t dd[16];
#pragma unroll
            for (int r = 0; r < 16; r++) dd[r] = bperm(8u * (r >> 2) + 4u * h + (r & 3), hdr.x);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float d = f16_opaque(dd[r]);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i][r] = __builtin_fmaf(t[i][r], d, acc[i][r]);
            }
        }
    }

    float* y = ds.y + (uint64_t)ks * ds.m * ds.ldy;
    const bool vec = (ds.ldy & 3u) == 0u && ((uintptr_t)ds.y & 15u) == 0u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = m0 + 32u * i + l32;
        if (row >= ds.m) continue;
        float* yr = y + (uint64_t)row * ds.ldy;
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const uint32_t c0 = n0 + 32u * w + 8u * q4 + 4u * h;
            if (vec && c0 + 3u < ds.n) {
                *reinterpret_cast<float4*>(yr + c0) =
                    make_float4(acc[i][4 * q4], acc[i][4 * q4 + 1], acc[i][4 * q4 + 2], acc[i][4 * q4 + 3]);
            } else {
#pragma unroll
                for (int s4 = 0; s4 < 4; s4++)
                    if (c0 + s4 < ds.n) yr[c0 + s4] = acc[i][4 * q4 + s4];
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void rfxq_mmq2_q4k(MmqArgs args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[mmq2::kLds];
    const MmqDesc d = mmq_pick(args, blockIdx.x);
    if (blockIdx.x - d.wg_begin >= d.tiles_m * d.tiles_n * d.splits) return;
    mmq2_q4k_tile(d, blockIdx.x - d.wg_begin, lds);
}

// ---------------------------------------------------------------------------
// Q6_K prefill GEMM on exact f16 MFMAs (rfxq_mmq2_q6k), same tile, ring and
// activation layouts as the Q4_K kernel above.
//
// A Q6_K super-block (ql[128], qh[64], scales[16] i8, d; src/dequant.rs:414-445)
// has no constant part: w = d * sc * (q - 32), with one scale per 16 codes.
// The scale goes into the weight operand, but sc*(q - 32) reaches 4096 in
// magnitude and needs 12 significant bits, one more than f16 holds; split by
// the code's low bit, q - 32 = (q & ~1) - 32 + (q & 1):
//   hi = sc * ((q & ~1) - 32)   (even, |hi| <= 4096: exact in f16)
//   lo = sc * (q & 1)           (|lo| <= 128)
// and D_b = sum_k qa * hi + sum_k qa * lo is four chained 32x32x16 f16 MFMAs
// per 32-block, exact in f32 (|D_b| <= 32*127*4096 < 2^24): the int8
// kernel's scaled block dot sc_lo*D_lo + sc_hi*D_hi. Then, per element,
//   t += da_b * D_b,   and per super-block   y += d * t.
//
// A 64-k stage g = 2n + s of a super-block takes blocks A = 4n + s (low
// nibbles of ql[64n + 32s + l], qh[32n + l] bits 2s..2s+1) and B = A + 2
// (high nibbles, bits 2s+4..2s+5), l in [0, 32); lane half h holds positions
// l in [16h, 16h + 16), whose scales are sc[8n + 2s + h] (A) and
// sc[8n + 4 + 2s + h] (B). Blocks are 210 bytes, so a super-block starts at
// a 2-byte offset when its index is odd (rows are 4-byte aligned: the host
// requires an even super-block count per row): the ql and qh ranges are
// copied as 9-dword windows from the aligned address below and realigned
// with v_alignbyte after the LDS read. LDS per slot: activations 16 KB, code
// windows 128 x 72 B, block scales 512 B; headers (scales, d) 128 x 20 B.

namespace mmq2 {

constexpr uint32_t kCodes6 = 128u * 18u * 4u;
constexpr uint32_t kSlot6 = kAct + kCodes6 + kDa;
constexpr uint32_t kHdr6 = 128u * 5u * 4u;
constexpr uint32_t kLds6 = 3u * kSlot6 + kHdr6;

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

}  // namespace mmq2

// One 128x128 tile (and one split-K range) of Y = X . W^T for Q6_K weights.
RFXQ_DEV void mmq2_q6k_tile(const MmqDesc& dv, uint32_t t_local, uint8_t* lds) {
    using namespace mmq2;
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
    const uint32_t row_bytes = nsb * 210u;
    const uint32_t rec_bytes = nsb * 64u;

    const uint32_t L = __builtin_amdgcn_readfirstlane(lds_addr(lds));
    const uint32_t Lhdr = L + 3u * kSlot6;

    const sdesc_t r_act = uniform_desc(ds.xq, ds.m * ds.ldq);
    const sdesc_t r_w = uniform_desc(ds.w, ds.n * row_bytes);
    const sdesc_t r_sc = uniform_desc(ds.xds, ds.m * rec_bytes);
    // activations: as the Q4_K kernel, but logical chunks 4-7 (block B) sit
    // 128 bytes after chunks 0-3 (block A) in the f16 row
    const uint32_t o_row = (m0 + 32u * w + (lane >> 3)) * ds.ldq;
    uint32_t o_act[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const uint32_t c = (lane & 7u) ^ (lane >> 4) ^ (e ? 4u : 0u);
        o_act[e] = o_row + 16u * c + (c >= 4u ? 64u : 0u);
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
    const uint32_t o_da = (m0 + 32u * w + l32) * rec_bytes + 48u;
    const uint32_t nst = 4u * (sb1 - sb0);
    // copies of stage st: 15 per wave, 18 when it opens a super-block
    auto issue = [&](uint32_t st) {
        const uint32_t sb = sb0 + (st >> 2), g = st & 3u, n = g >> 1, s = g & 1u, slot = st % 3u;
        const uint32_t Ls = __builtin_amdgcn_readfirstlane(L + slot * kSlot6);
        const uint32_t base = 210u * sb - 2u * (sb & 1u);  // 4-byte aligned
#pragma unroll
        for (int q = 0; q < 4; q++)
            dma16(r_act, Ls + 1024u * (4u * w + q), o_act[q & 1], 512u * sb + 64u * (4u * n + s) + 8u * q * ds.ldq);
        const uint32_t Lc = Ls + kAct + 2304u * w;
#pragma unroll
        for (int q = 0; q < 4; q++) dma4(r_w, Lc + 256u * q, o_c[q], base + 64u * n + 32u * s);
        if (h == 0u) dma4(r_w, Lc + 1024u, o_c[4], base + 64u * n + 32u * s);
#pragma unroll
        for (int q = 0; q < 4; q++) dma4(r_w, Lc + 1152u + 256u * q, o_c[q], base + 128u + 32u * n);
        if (h == 0u) dma4(r_w, Lc + 1152u + 1024u, o_c[4], base + 128u + 32u * n);
        if (h == 0u) dma4(r_sc, Ls + kAct + kCodes6 + 128u * w, o_da, 64u * sb + 4u * g);
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
    const uint32_t a_da = (kAct + kCodes6) / 4u + l32;
    uint32_t scw[4] = {0u, 0u, 0u, 0u}, dbits = 0u;

    if (nst > 0u) issue(0u);
    if (nst > 1u) issue(1u);
    for (uint32_t st = 0; st < nst; st++) {
        if (st + 1u < nst) {
            if (((st + 1u) & 3u) == 0u) asm volatile("s_waitcnt vmcnt(18)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(15)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (st + 2u < nst) issue(st + 2u);

        const uint32_t sb = sb0 + (st >> 2), g = st & 3u, n = g >> 1, s = g & 1u;
        const uint32_t sh = 2u * (sb & 1u);  // byte offset of the block in the windows
        const uint8_t* S = lds + (st % 3u) * kSlot6;
        const u4_t* S16 = reinterpret_cast<const u4_t*>(S);
        if (g == 0u) {
            const uint32_t* hp = reinterpret_cast<const uint32_t*>(lds + 3u * kSlot6 + 640u * w) + 5u * l32;
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
        const uint32_t* da_p = reinterpret_cast<const uint32_t*>(S) + a_da;
        uint32_t da[4];
#pragma unroll
        for (int i = 0; i < 4; i++) da[i] = da_p[32 * i];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u4_t* xp = S16 + 256u * i;
            const u4_t xa0 = xp[a_act[0][0]], xa1 = xp[a_act[0][1]];
            const u4_t xb0 = xp[a_act[1][0]], xb1 = xp[a_act[1][1]];
            v16f_t DA = mfma16(hi[0][0], xa0, v16f_t{});
            DA = mfma16(lo[0][0], xa0, DA);
            DA = mfma16(hi[0][1], xa1, DA);
            DA = mfma16(lo[0][1], xa1, DA);
            v16f_t DB = mfma16(hi[1][0], xb0, v16f_t{});
            DB = mfma16(lo[1][0], xb0, DB);
            DB = mfma16(hi[1][1], xb1, DB);
            DB = mfma16(lo[1][1], xb1, DB);
            const float da0 = f16_opaque(da[i]), da1 = f16_opaque(da[i] >> 16);
#pragma unroll
            for (int r = 0; r < 16; r++) t[i][r] = __builtin_fmaf(DB[r], da1, __builtin_fmaf(DA[r], da0, t[i][r]));
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
        if (row >= ds.m) continue;
        float* yr = y + (uint64_t)row * ds.ldy;
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const uint32_t c0 = n0 + 32u * w + 8u * q4 + 4u * h;
            if (vec && c0 + 3u < ds.n) {
                *reinterpret_cast<float4*>(yr + c0) =
                    make_float4(acc[i][4 * q4], acc[i][4 * q4 + 1], acc[i][4 * q4 + 2], acc[i][4 * q4 + 3]);
            } else {
#pragma unroll
                for (int s4 = 0; s4 < 4; s4++)
                    if (c0 + s4 < ds.n) yr[c0 + s4] = acc[i][4 * q4 + s4];
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void rfxq_mmq2_q6k(MmqArgs args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[mmq2::kLds6];
    const MmqDesc d = mmq_pick(args, blockIdx.x);
    if (blockIdx.x - d.wg_begin >= d.tiles_m * d.tiles_n * d.splits) return;
    mmq2_q6k_tile(d, blockIdx.x - d.wg_begin, lds);
}
