// MoE data movement and activation kernels.
//
// rfxq_moe_gather / rfxq_moe_scatter_add keep the semantics of the reference's
// `moe_gather_kernel` / `moe_scatter_add_kernel` (src/kernels_cuda/elementwise.cu:
// 175-222): dst[a,:] = src[perm[a],:] and dst[row[a],:] += w[a] * src[a,:] (no
// atomics; rows unique within one launch). rfxq_silu_and_mul is
// src/kernels_cuda/silu_and_mul.cu:7-23 (g / (1 + expf(-g)) * u).
//
// rfxq_moe_combine is the grouped pipeline's replacement for 128 per-expert
// scatter-adds: every token sums its k routed expert outputs in increasing
// expert order with the same fma, which is the order and rounding the
// reference's per-expert launch sequence produces (dense.rs:1549-1556 walks
// experts 0..E-1 and each launch adds into the zeroed output).
#pragma once
#include "common.hpp"

extern "C" __global__ __launch_bounds__(256) void rfxq_moe_gather(const float* __restrict__ src,
                                                                 const uint32_t* __restrict__ perm_row,
                                                                 float* __restrict__ dst, uint32_t num,
                                                                 uint32_t hidden) {
    const uint64_t total = (uint64_t)num * hidden;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256u) {
        const uint64_t a = i / hidden, c = i % hidden;
        dst[i] = src[(uint64_t)perm_row[a] * hidden + c];
    }
}

extern "C" __global__ __launch_bounds__(256) void rfxq_moe_scatter_add(const float* __restrict__ src,
                                                                      const uint32_t* __restrict__ dest_row,
                                                                      const float* __restrict__ weight,
                                                                      float* __restrict__ dst, uint32_t num,
                                                                      uint32_t hidden) {
    const uint64_t total = (uint64_t)num * hidden;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256u) {
        const uint64_t a = i / hidden, c = i % hidden;
        float* p = dst + (uint64_t)dest_row[a] * hidden + c;
        *p = fmaf(weight[a], src[i], *p);
    }
}

extern "C" __global__ __launch_bounds__(256) void rfxq_silu_and_mul(const float* __restrict__ gate,
                                                                   const float* __restrict__ up,
                                                                   float* __restrict__ out, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256u) {
        const float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

// out[t,:] = sum_j w[t,j] * pair_out[idx[t,j],:] for j in 0..k (pairs sorted
// by expert), evaluated as fma(w, v, acc) from acc = 0.
extern "C" __global__ __launch_bounds__(256) void rfxq_moe_combine(const float* __restrict__ pair_out,
                                                                  const int32_t* __restrict__ idx,
                                                                  const float* __restrict__ w,
                                                                  float* __restrict__ out, uint32_t tokens,
                                                                  uint32_t k, uint32_t hidden) {
    const uint64_t total = (uint64_t)tokens * hidden;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256u) {
        const uint64_t t = i / hidden, c = i % hidden;
        float acc = 0.0f;
        for (uint32_t j = 0; j < k; j++) {
            const int32_t p = idx[t * k + j];
            if (p >= 0) acc = fmaf(w[t * k + j], pair_out[(uint64_t)p * hidden + c], acc);
        }
        out[i] = acc;
    }
}
