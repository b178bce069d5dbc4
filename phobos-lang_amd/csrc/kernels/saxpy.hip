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
// stride over the array in chunks, so any grid size is correct.  `out` may alias `y`
// (y = alpha*x + y): each element is read and then written by one thread.
// The descriptor's offset and stride are honoured; non-unit strides or
// misaligned bases fall back to a scalar loop.
#include "phx_common.h"

// Streaming loads and stores go through buffer instructions with the
// non-temporal bit (nt): the single-use stream does not displace other data,
// the 32-bit offsets keep the address arithmetic to one VALU op per access,
// and this measured 1-2 % faster on MI355X than global loads with the same
// hint (plain loads and stores are 15 % slower).  A workgroup's chunk gets its
// own buffer resource, so arrays beyond 4 GiB are covered.
#define PHX_NT 2  // cache-policy operand: nt

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sx_rsrc(const float *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

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
        constexpr uint32_t CH = PHX_SAXPY_THREADS * PHX_SAXPY_VEC;  // float4 per block step
        for (int64_t c = bid; c * CH < nv; c += nblk) {
            const int64_t e0 = c * CH * 4;  // first element of this chunk
            const int64_t left = nv * 4 - e0;
            const uint32_t bytes = (uint32_t)((left < (int64_t)CH * 4 ? left : (int64_t)CH * 4) * 4);
            const __amdgpu_buffer_rsrc_t rx = sx_rsrc(x + e0, bytes);
            const __amdgpu_buffer_rsrc_t ry = sx_rsrc(y + e0, bytes);
            const __amdgpu_buffer_rsrc_t ro = sx_rsrc(o + e0, bytes);
            // out-of-range float4s (the last chunk) read as 0 and are not stored
            phx_f4 xr[PHX_SAXPY_VEC], yr[PHX_SAXPY_VEC];
#pragma unroll
            for (int u = 0; u < PHX_SAXPY_VEC; ++u) {
                const uint32_t off = (tid + u * PHX_SAXPY_THREADS) * 16;
                xr[u] = __builtin_bit_cast(phx_f4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, PHX_NT));
                yr[u] = __builtin_bit_cast(phx_f4, __builtin_amdgcn_raw_buffer_load_b128(ry, off, 0, PHX_NT));
            }
#pragma unroll
            for (int u = 0; u < PHX_SAXPY_VEC; ++u) {
                const uint32_t off = (tid + u * PHX_SAXPY_THREADS) * 16;
                phx_f4 r = alpha * xr[u];
                r = r + yr[u];
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(phx_u4, r), ro, off, 0, PHX_NT);
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
