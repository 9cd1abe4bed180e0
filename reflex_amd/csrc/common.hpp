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
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

#define RFXQ_DEV static __device__ __forceinline__

// ggml type ids (GGUF on-disk values).
enum : uint32_t { TY_Q8_0 = 8, TY_Q4K = 12, TY_Q6K = 14 };

RFXQ_DEV float f16_bits_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(half_t, (uint16_t)(bits16 & 0xFFFFu));
}

// Bits of a u32 as f32. Takes its argument by value: __builtin_bit_cast
// applied directly to an ext-vector element (v.y) reads element 0 in this
// compiler, so vector elements go through here.
RFXQ_DEV float as_f32(uint32_t v) { return __builtin_bit_cast(float, v); }

RFXQ_DEV h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
RFXQ_DEV uint32_t h2_bits(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// 2-way f16 dot with f32 accumulate (v_dot2_f32_f16).
RFXQ_DEV float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Global-address-space loads/stores: generic (flat) accesses would also count
// against the LDS counter, making every LDS wait wait on HBM loads too.
#define RFXQ_GLOBAL __attribute__((address_space(1)))
typedef uint32_t u4a4_t __attribute__((ext_vector_type(4), aligned(4)));

// Four dwords from a 16-byte-aligned global address.
RFXQ_DEV u4_t ld16(const void* p) { return *(const RFXQ_GLOBAL u4_t*)p; }
// Four dwords from a dword-aligned global address.
RFXQ_DEV u4_t ld16_a4(const void* p) { return *(const RFXQ_GLOBAL u4a4_t*)p; }
// Two dwords from an 8-byte-aligned global address.
RFXQ_DEV u2_t ld8(const void* p) { return *(const RFXQ_GLOBAL u2_t*)p; }
RFXQ_DEV uint32_t ld4(const void* p) { return *(const RFXQ_GLOBAL uint32_t*)p; }
RFXQ_DEV uint32_t ld2(const void* p) { return *(const RFXQ_GLOBAL uint16_t*)p; }
typedef float f4v_t __attribute__((ext_vector_type(4)));
RFXQ_DEV float4 ldf4(const float* p) {
    const f4v_t v = *(const RFXQ_GLOBAL f4v_t*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
RFXQ_DEV void stf(float* p, float v) { *(RFXQ_GLOBAL float*)p = v; }

// Raw buffer access (gfx9 V#: base, stride 0, num_records = bytes): 32-bit
// offsets, and reads at or past num_records return 0 instead of faulting.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
RFXQ_DEV rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
RFXQ_DEV u4_t bld16(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
RFXQ_DEV uint32_t bld4(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
RFXQ_DEV void bst4f(rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, 0);
}

// 32-bit LDS address of a pointer into shared memory
RFXQ_DEV uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Workgroup barrier that orders LDS only: earlier LDS accesses of the wave are
// complete, global loads and asynchronous copies may still be in flight
// (__syncthreads would also wait for those, as they write LDS).
RFXQ_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// LDS accesses hidden from the compiler's wait counting. A compiler-visible
// LDS access that may alias a buffer_load ... lds destination makes it wait
// for every copy in flight (vmcnt(0)); kernels that stream weights through LDS
// copies use these for their other LDS traffic and order the copies with
// explicit vmcnt waits. Reads wait for their own data (lgkmcnt(0)); their
// outputs are early-clobber, as the reads land after later ones issue.
RFXQ_DEV void lds_st32(uint32_t a, uint32_t v) { asm volatile("ds_write_b32 %0, %1" ::"v"(a), "v"(v) : "memory"); }
RFXQ_DEV void lds_st64(uint32_t a, u2_t v) { asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(v) : "memory"); }
RFXQ_DEV uint32_t lds_ld32(uint32_t a) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a) : "memory");
    return v;
}
RFXQ_DEV u2_t lds_ld64(uint32_t a) {
    u2_t v;
    asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a) : "memory");
    return v;
}
RFXQ_DEV u4_t lds_ld128(uint32_t a) {
    u4_t v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a) : "memory");
    return v;
}
// two 16-byte reads at a and a + 16
RFXQ_DEV void lds_ld2x128(uint32_t a, u4_t& v0, u4_t& v1) {
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v0), "=&v"(v1)
                 : "v"(a)
                 : "memory");
}
// four 16-byte reads at a, a + 16, a + 32, a + 48
RFXQ_DEV void lds_ld4x128(uint32_t a, u4_t& v0, u4_t& v1, u4_t& v2, u4_t& v3) {
    asm volatile(
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:16\n\t"
        "ds_read_b128 %2, %4 offset:32\n\tds_read_b128 %3, %4 offset:48\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
        : "v"(a)
        : "memory");
}
RFXQ_DEV uint4 as_uint4(u4_t v) { return make_uint4(v.x, v.y, v.z, v.w); }

// Asynchronous copy global -> LDS (buffer_load ... lds): each lane's `size`
// bytes from its own buffer offset land at lds_base + lane * size. lds_base
// must be wave-uniform. Lanes reading past the buffer write zeros.
#define RFXQ_LDSP(p) ((__attribute__((address_space(3))) void*)(p))
RFXQ_DEV void dma16(rsrc_t r, void* lds_base, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, RFXQ_LDSP(lds_base), 16, off, 0, 0, 0);
}

// the same copy marked non-temporal (cache policy nt): for data read once,
// such as decode weights streamed from HBM
RFXQ_DEV void dma16_stream(rsrc_t r, void* lds_base, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, RFXQ_LDSP(lds_base), 16, off, 0, 0, 2);
}


RFXQ_DEV uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t shift_bytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift_bytes);
}

// DPP lane moves (row = 16 lanes): quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror, row_mirror.
#define RFXQ_DPP(v, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, false))

// Sum over groups of WIDTH consecutive lanes (a power of two <= 64). Within a
// 16-lane row the sum uses DPP (every lane of the group ends with it); across
// rows the gfx950 row swaps: v_permlane16_swap gives every lane of rows 2i,
// 2i + 1 the pair row0 + row1 of its half (32), v_permlane32_swap every lane
// the two halves' sum, lower half first (64). (Every lane of a row holds the
// same value by then, so the lane alignment of the swaps does not matter.)
template <int WIDTH>
RFXQ_DEV float group_sum(float v) {
    if (WIDTH >= 2) v += RFXQ_DPP(v, 0xB1);
    if (WIDTH >= 4) v += RFXQ_DPP(v, 0x4E);
    if (WIDTH >= 8) v += RFXQ_DPP(v, 0x141);
    if (WIDTH >= 16) v += RFXQ_DPP(v, 0x140);
    if (WIDTH >= 32) {
        const uint32_t b = __builtin_bit_cast(uint32_t, v);
        const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
        v = __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
    }
    if (WIDTH >= 64) {
        const uint32_t b = __builtin_bit_cast(uint32_t, v);
        const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
        v = __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
    }
    return v;
}

// wave-wide maximum (every lane ends with it; order-independent): DPP
// steps leave each 16-lane row's maximum in its lanes, then the four rows'
// are read out (no LDS round trip, as a swizzle across rows would take)
RFXQ_DEV float wave_max(float v) {
    v = fmaxf(v, RFXQ_DPP(v, 0xB1));
    v = fmaxf(v, RFXQ_DPP(v, 0x4E));
    v = fmaxf(v, RFXQ_DPP(v, 0x141));
    v = fmaxf(v, RFXQ_DPP(v, 0x140));
    const int b = __builtin_bit_cast(int, v);
    return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))),
                 fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48))));
}

// Index of element e inside a run stored pair-permuted: within each group of
// four, elements (0,1,2,3) live at (0,2,1,3), so one dword holds the f16 pair
// (e, e+2) that a masked packed byte word produces.
RFXQ_DEV uint32_t pair_perm(uint32_t e) { return (e & ~3u) | ((e & 1u) << 1) | ((e >> 1) & 1u); }
