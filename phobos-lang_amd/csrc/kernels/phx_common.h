// Shared device-side helpers for the gfx950 leaf kernels.
//
// Every kernel keeps the reference's exploded-memref parameter list
// (phobos-pod/src/engine.rs:582-630, phobos-bench/src/main.rs:308-323):
// each tensor<T>[d0..dr-1] parameter expands to
//   (T* alloc, T* aligned, IDX offset, IDX size[0..r-1], IDX stride[0..r-1])
// with IDX = int32_t, or int64_t for kernels the reference compiles with a
// wide index (@tensorcore, phobos-lang/src/lib.rs:47-49).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "phx_geometry.h"

#define PHX_MEMREF1(T, n, IDX) T *n##_alloc, T *n##_ptr, IDX n##_off, IDX n##_s0, IDX n##_st0
#define PHX_MEMREF2(T, n, IDX)                                                          \
    T *n##_alloc, T *n##_ptr, IDX n##_off, IDX n##_s0, IDX n##_s1, IDX n##_st0, IDX n##_st1
#define PHX_MEMREF3(T, n, IDX)                                                          \
    T *n##_alloc, T *n##_ptr, IDX n##_off, IDX n##_s0, IDX n##_s1, IDX n##_s2, IDX n##_st0, \
        IDX n##_st1, IDX n##_st2

typedef _Float16 phx_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 phx_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 phx_h2 __attribute__((ext_vector_type(2)));
typedef float phx_f4 __attribute__((ext_vector_type(4)));
typedef float phx_f16v __attribute__((ext_vector_type(16)));
typedef uint32_t phx_u4 __attribute__((ext_vector_type(4)));
typedef uint32_t phx_u2 __attribute__((ext_vector_type(2)));

// Linear workgroup id over a 1-3D grid and the total count.
__device__ __forceinline__ uint32_t phx_block_linear() {
    return blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
}
__device__ __forceinline__ uint32_t phx_block_count() {
    return gridDim.x * gridDim.y * gridDim.z;
}

// Workgroups are dispatched round-robin over the 8 XCDs (block b lands on
// XCD b % 8).  Renumber so that the i-th block of an XCD gets consecutive
// work items: neighbouring output tiles then share that XCD's L2.
__device__ __forceinline__ uint32_t phx_xcd_swizzle(uint32_t b, uint32_t nblocks) {
    const uint32_t XCD = 8;
    if (nblocks % XCD != 0) return b;
    return (b % XCD) * (nblocks / XCD) + b / XCD;
}

__device__ __forceinline__ uint32_t phx_pack_h2(float lo, float hi) {
    phx_h2 v;
    v.x = (_Float16)lo;   // v_cvt_f16_f32: round to nearest even
    v.y = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, v);
}
