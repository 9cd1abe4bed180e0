// Device-side helpers shared by every kernel of the gfx950 code object.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half_t;
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));
typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

#define RFXQ_DEV static __device__ __forceinline__

// ggml type ids (GGUF on-disk values).
enum : uint32_t { TY_Q8_0 = 8, TY_Q4K = 12, TY_Q6K = 14 };

RFXQ_DEV float f16_bits_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(half_t, (uint16_t)(bits16 & 0xFFFFu));
}

RFXQ_DEV h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
RFXQ_DEV uint32_t h2_bits(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// 2-way f16 dot with f32 accumulate (v_dot2_f32_f16).
RFXQ_DEV float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Four dwords from a 16-byte-aligned global address.
RFXQ_DEV u4_t ld16(const uint8_t* p) { return *reinterpret_cast<const u4_t*>(p); }

// Four dwords from a dword-aligned global address.
RFXQ_DEV u4_t ld16_a4(const uint8_t* p) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    u4_t r;
    r.x = q[0];
    r.y = q[1];
    r.z = q[2];
    r.w = q[3];
    return r;
}

RFXQ_DEV uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t shift_bytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift_bytes);
}

// Sum over groups of `width` consecutive lanes (width a power of two <= 64);
// every lane of the group ends with the group sum.
template <int WIDTH>
RFXQ_DEV float group_sum(float v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Index of element e inside a run stored pair-permuted: within each group of
// four, elements (0,1,2,3) live at (0,2,1,3), so one dword holds the f16 pair
// (e, e+2) that a masked packed byte word produces.
RFXQ_DEV uint32_t pair_perm(uint32_t e) { return (e & ~3u) | ((e & 1u) << 1) | ((e >> 1) & 1u); }
