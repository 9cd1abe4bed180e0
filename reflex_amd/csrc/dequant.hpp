// Coalesced dequantization: raw GGUF blocks -> f32 or f16, one lane per element.
//
// Every value is computed with the reference's own expression and rounding
// order (src/dequant.rs:339-367 Q4_K `d1 * q - m1`, :414-444 Q6_K `d * sc * q`,
// :220-226 Q8_0 `q * d`), with FP contraction disabled, so the f32 output is
// bit-identical to the host dequantizer; the f16 output is the RNE rounding of
// that f32 value. Replaces `dequantize_{q4k,q6k}_coalesced{,_f16}_kernel`
// (src/kernels_cuda/gemv_q4k.cu:359-448) and `dequantize_q8_0_coalesced{,_f16}`
// (src/kernels_cuda/gemv_q8_0.cu:253-282).
#pragma once
#include "common.hpp"

template <typename T>
RFXQ_DEV T store_cvt(float v);
template <> __device__ __forceinline__ float store_cvt<float>(float v) { return v; }
// The empty asm keeps the f32 value opaque so the narrowing is a plain RNE
// conversion: fusing the producing multiply into a mixed-precision mad with a
// +0 addend would turn -0.0 (a Q6_K block with d = 0) into +0.0.
template <> __device__ __forceinline__ half_t store_cvt<half_t>(float v) {
    asm volatile("" : "+v"(v));
    return (half_t)v;
}

RFXQ_DEV void q4k_scale_min(uint32_t j, const uint8_t* q, uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = q[j] & 63u;
        m = q[j + 4] & 63u;
    } else {
        sc = (q[j + 4] & 0xFu) | ((uint32_t)(q[j - 4] >> 6) << 4);
        m = (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
    }
}

RFXQ_DEV float le16(const uint8_t* p) { return f16_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

RFXQ_DEV float dq_q4k_elem(const uint8_t* blk, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t g = e >> 6, hi = (e >> 5) & 1u, l = e & 31u;
    uint32_t sc, m;
    q4k_scale_min(2u * g + hi, blk + 4, sc, m);
    const float d1 = le16(blk) * (float)sc;
    const float m1 = le16(blk + 2) * (float)m;
    const uint8_t q = blk[16 + 32u * g + l];
    const float qf = (float)(hi ? (q >> 4) : (q & 0xF));
    const float t = d1 * qf;
    return t - m1;
}

RFXQ_DEV float dq_q6k_elem(const uint8_t* blk, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t n = e >> 7, t = (e >> 5) & 3u, l = e & 31u;
    const uint8_t ql = blk[64u * n + l + ((t & 1u) ? 32u : 0u)];
    const uint8_t qh = blk[128u + 32u * n + l];
    const int lo = (t & 2u) ? (ql >> 4) : (ql & 0xF);
    const int q = (int)(lo | (((qh >> (2u * t)) & 3) << 4)) - 32;
    const int8_t sc = (int8_t)blk[192u + 8u * n + (l >> 4) + 2u * t];
    const float d = le16(blk + 208);
    const float ds = d * (float)sc;
    return ds * (float)q;
}

RFXQ_DEV float dq_q8_0_elem(const uint8_t* blk, uint32_t e) {
#pragma clang fp contract(off)
    return (float)(int8_t)blk[2 + e] * le16(blk);
}

// grid-stride over super-blocks: 256 threads, one element each.
template <typename T, uint32_t TY>
RFXQ_DEV void dequant_k_body(const uint8_t* __restrict__ blocks, T* __restrict__ y, uint32_t num_blocks) {
    const uint32_t bb = TY == TY_Q4K ? 144u : 210u;
    for (uint32_t b = blockIdx.x; b < num_blocks; b += gridDim.x) {
        const uint8_t* blk = blocks + (uint64_t)b * bb;
        const float v = TY == TY_Q4K ? dq_q4k_elem(blk, threadIdx.x) : dq_q6k_elem(blk, threadIdx.x);
        y[(uint64_t)b * 256u + threadIdx.x] = store_cvt<T>(v);
    }
}

// Q8_0: 8 blocks of 32 per 256-thread group.
template <typename T>
RFXQ_DEV void dequant_q8_0_body(const uint8_t* __restrict__ blocks, T* __restrict__ y, uint32_t num_blocks) {
    const uint32_t groups = (num_blocks + 7u) / 8u;
    for (uint32_t g = blockIdx.x; g < groups; g += gridDim.x) {
        const uint32_t b = g * 8u + (threadIdx.x >> 5);
        if (b < num_blocks) {
            const float v = dq_q8_0_elem(blocks + (uint64_t)b * 34u, threadIdx.x & 31u);
            y[(uint64_t)b * 32u + (threadIdx.x & 31u)] = store_cvt<T>(v);
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void rfxq_dequant_q4k_f32(const uint8_t* b, float* y, uint32_t n) {
    dequant_k_body<float, TY_Q4K>(b, y, n);
}
extern "C" __global__ __launch_bounds__(256) void rfxq_dequant_q4k_f16(const uint8_t* b, half_t* y, uint32_t n) {
    dequant_k_body<half_t, TY_Q4K>(b, y, n);
}
extern "C" __global__ __launch_bounds__(256) void rfxq_dequant_q6k_f32(const uint8_t* b, float* y, uint32_t n) {
    dequant_k_body<float, TY_Q6K>(b, y, n);
}
extern "C" __global__ __launch_bounds__(256) void rfxq_dequant_q6k_f16(const uint8_t* b, half_t* y, uint32_t n) {
    dequant_k_body<half_t, TY_Q6K>(b, y, n);
}
extern "C" __global__ __launch_bounds__(256) void rfxq_dequant_q8_0_f32(const uint8_t* b, float* y, uint32_t n) {
    dequant_q8_0_body<float>(b, y, n);
}
extern "C" __global__ __launch_bounds__(256) void rfxq_dequant_q8_0_f16(const uint8_t* b, half_t* y, uint32_t n) {
    dequant_q8_0_body<half_t>(b, y, n);
}
