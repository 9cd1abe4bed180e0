// Q4_K prefill GEMM on exact f16 MFMAs with a transposed tile: the default
// Q4_K kernel of the MMQ path (src/kernels_cuda/gemm_q_mma.cu:299-764 is the
// reference's f16 prefill kernel it replaces; same call sites as mmq.hpp).
//
// Inputs are the same Q8_1 activations as the int8 kernel, in two derived
// layouts written by the quantizer: xh, the int8 values as f16 (group of four
// stored (q0, q2), (q1, q3)), and xsc, one 48-byte record per row and
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
    const uint32_t rec_bytes = nsb * 48u;  // xsc row

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
        if (h == 0u) dma4(r_sc, Ls + kAct + kCodes + 128u * w, o_da, 48u * sb + 4u * g);
        if (g == 0u) {
            if (h == 0u) dma16(r_w, Lhdr + 512u * w, o_hdr, 144u * sb);
            dma16(r_sc, Lsx + 1024u * w, o_sx, 48u * sb);
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
    mmq2_q4k_tile(d, blockIdx.x - d.wg_begin, lds);
}
