// saxpy leaf kernel for gfx950: out[i] = fl(fl(alpha * x[i]) + y[i]).
//
// Reference: examples/saxpy_fp32.ph:1-5 (one program per BLOCK elements);
// the multiply and the add are separately rounded and never contracted into
// an FMA (phobos-lang/src/codegen/tile.rs:1786-1794; exact check at
// phobos-bench/src/main.rs:1176-1188).  This file is compiled with
// -ffp-contract=off so `alpha * x + y` stays v_mul_f32 + v_add_f32.
//
// MI355X design: a pure HBM stream (12 bytes per element).  Each thread moves
// PHX_SAXPY_VEC 16-byte vectors per block step, issuing every load before any
// store so each wave keeps 2*VEC independent 16-byte loads in flight; blocks
// stride over the array, so any grid size is correct.  `out` may alias `y`
// (y = alpha*x + y): each element is read and then written by one thread.
// The descriptor's offset and stride are honoured; non-unit strides or
// misaligned bases fall back to a scalar loop.
#include "phx_common.h"

// Streaming hints: non-temporal loads/stores keep the single-use stream from
// evicting other data.
#ifndef PHX_SAXPY_PLAIN
#define PHX_LOAD(p) __builtin_nontemporal_load(p)
#define PHX_STORE(v, p) __builtin_nontemporal_store(v, p)
#else
#define PHX_LOAD(p) (*(p))
#define PHX_STORE(v, p) (*(p) = (v))
#endif

extern "C" __global__ __launch_bounds__(PHX_SAXPY_THREADS) void saxpy(
    PHX_MEMREF1(float, x, int32_t), PHX_MEMREF1(float, y, int32_t),
    PHX_MEMREF1(float, o, int32_t), float alpha) {
    const float *x = x_ptr + x_off;
    const float *y = y_ptr + y_off;
    float *o = o_ptr + o_off;
    const int64_t n = x_s0;
    const uint32_t tid = threadIdx.x;
    const uint32_t nblk = phx_block_count();
    const uint32_t bid = phx_block_linear();

    const bool vec_ok = x_st0 == 1 && y_st0 == 1 && o_st0 == 1 &&
                        ((((uintptr_t)x) | ((uintptr_t)y) | ((uintptr_t)o)) & 15) == 0;
    if (vec_ok) {
        const int64_t nv = n >> 2;  // float4 count
        const phx_f4 *xv = (const phx_f4 *)x;
        const phx_f4 *yv = (const phx_f4 *)y;
        phx_f4 *ov = (phx_f4 *)o;
        const int64_t step = (int64_t)nblk * (PHX_SAXPY_THREADS * PHX_SAXPY_VEC);
        for (int64_t base = (int64_t)bid * (PHX_SAXPY_THREADS * PHX_SAXPY_VEC) + tid; base < nv;
             base += step) {
            phx_f4 xr[PHX_SAXPY_VEC], yr[PHX_SAXPY_VEC];
#pragma unroll
            for (int u = 0; u < PHX_SAXPY_VEC; ++u) {
                const int64_t i = base + (int64_t)u * PHX_SAXPY_THREADS;
                if (i < nv) {
                    xr[u] = PHX_LOAD(xv + i);
                    yr[u] = PHX_LOAD(yv + i);
                }
            }
#pragma unroll
            for (int u = 0; u < PHX_SAXPY_VEC; ++u) {
                const int64_t i = base + (int64_t)u * PHX_SAXPY_THREADS;
                if (i < nv) {
                    phx_f4 r = alpha * xr[u];
                    r = r + yr[u];
                    PHX_STORE(r, ov + i);
                }
            }
        }
        // ragged tail (n % 4 elements), owned by block 0
        if (bid == 0) {
            const int64_t i = nv * 4 + tid;
            if (i < n) {
                float p = alpha * x[i];
                o[i] = p + y[i];
            }
        }
        return;
    }
    const int64_t step = (int64_t)nblk * PHX_SAXPY_THREADS;
    for (int64_t i = (int64_t)bid * PHX_SAXPY_THREADS + tid; i < n; i += step) {
        float p = alpha * x[(int64_t)i * x_st0];
        o[(int64_t)i * o_st0] = p + y[(int64_t)i * y_st0];
    }
}
