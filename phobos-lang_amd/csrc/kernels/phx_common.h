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

// The split-K epilogue shared by the GEMM code objects: acc = W[0] + W[1] +
// ... + W[S-1] over S partial-sum planes of M x N f32 (in that order, so the
// result does not depend on timing), then C = fl(fl(alpha*acc) +
// fl(beta*c_old)) with C not read when beta == 0, rounded once to the output
// type.  Four consecutive elements per thread (N is a multiple of 4, C's
// rows are 16-byte (f32) or 8-byte (f16) aligned), block-stride over the
// M x N/4 groups.  Compiled -ffp-contract=off: every mul and add rounds.
template <typename TO>
__device__ __forceinline__ void phx_splitk_reduce(const float *W, int32_t S, TO *C, int64_t ldc,
                                                  int64_t M, int64_t N, float alpha, float beta) {
    const int64_t ng = M * (N / 4), plane = M * N;
    for (int64_t gi = (int64_t)phx_block_linear() * blockDim.x + threadIdx.x; gi < ng;
         gi += (int64_t)phx_block_count() * blockDim.x) {
        const int64_t e = gi * 4;
        const int64_t r = e / N, c = e % N;
        phx_f4 acc = *(const phx_f4 *)(W + e);
        for (int32_t sp = 1; sp < S; ++sp) acc = acc + *(const phx_f4 *)(W + sp * plane + e);
        TO *dst = C + r * ldc + c;
        phx_f4 o = alpha * acc;
        if constexpr (sizeof(TO) == 4) {
            if (beta != 0.0f) o = o + beta * *(const phx_f4 *)dst;
            *(phx_f4 *)dst = o;
        } else {
            if (beta != 0.0f) {
                const phx_h4 h = *(const phx_h4 *)dst;
                o = o + beta * (phx_f4){(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
            }
            *(phx_h4 *)dst =
                (phx_h4){(_Float16)o[0], (_Float16)o[1], (_Float16)o[2], (_Float16)o[3]};
        }
    }
}
