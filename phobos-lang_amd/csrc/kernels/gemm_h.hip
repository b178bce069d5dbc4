// f16-operand GEMM leaf kernels for gfx950: C = alpha * A@B + beta * C.
//
// Built twice from this file:
//   -DPHX_GEMM_TC   gemm_fp16tc_fp32acc.ph: f32 tensors; A and B are rounded
//                   to f16 (RNE) once, while being staged into LDS
//                   (phobos-lang/src/codegen/matmul.rs:2170-2231); f32
//                   accumulation; f32 epilogue and output.
//   (default)       gemm_fp16.ph: f16 tensors.  The reference accumulates in
//                   f16 WMMA fragments (codegen/mod.rs:2120-2155); MFMA has no
//                   f16-accumulate mode, so this kernel accumulates in f32 (more
//                   accurate) and rounds once to f16 after the f32 epilogue
//                   truncf(alpha*acc + beta*c) (matmul.rs:1014-1025).
// Both take the reference's wide (i64) exploded-memref descriptors
// (launch_gemm, phobos-bench/src/main.rs:290-327).
//
// Epilogue: C = fl(fl(alpha*acc) + fl(beta*c_old)) with separately rounded
// operations (matmul.rs:384-403; this file is compiled -ffp-contract=off).
// When beta == 0 the old C is not read (BLAS convention); for finite C this
// differs from the reference only in the sign of an exactly-zero result.
//
// MI355X design
//   * 256x128 output tile, K step 32, 256 threads = 4 waves (2x2) of 128x64,
//     each 4x2 v_mfma_f32_32x32x16_f16 tiles (128 f32 accumulators).  LDS is
//     72 KiB (f16) / 48 KiB (tc) and a wave stays under 256 registers, so two
//     workgroups share each CU and cover each other's barrier, LDS and load stalls
//     (at 4096^2: 512 tiles, two per CU, all resident at once).
//   * A is staged As[m][k] (64-byte rows); an MFMA A operand (8 consecutive k
//     of one row) is one ds_read_b128.  B stays row-major Bs[k][n] (256-byte
//     rows) and its operand is read with gfx950's transposing
//     ds_read_b64_tr_b16: in a 16-lane group, lane s supplies 4 halves of row
//     k0 + s/4 at column n0 + 4*(s%4), and lane i receives B[k0..k0+3][n0+i].
//     Two such reads give a lane its 8 consecutive k.  Staging is therefore a
//     plain 16-byte copy for both operands.
//   * gfx950's LDS serves 64 banks (256 bytes) per clock.  The 16-byte chunk
//     index is XOR-swizzled so every 16-lane (b128) or 32-lane (b64) group
//     hits distinct banks: As chunk ^ ((row >> 2) & 3), Bs chunk ^ 4*(row % 4).
//   * f16 inputs are copied global -> LDS directly (buffer_load ... lds, no
//     VGPR staging) into a ring of three 24 KiB stages: K step t+2 is in
//     flight while step t computes; each wave waits for its own copies
//     (vmcnt) before the raw barrier that publishes a stage.  The tc variant
//     (f32 inputs, converted to f16 on the way) stages through registers with
//     a double-buffered LDS.  Both issue a K slice's LDS reads ahead of its
//     MFMAs (fenced, since the wave issues in order).
//   * Workgroups are renumbered XCD-major and grouped 8 tile-rows deep, so the
//     64 workgroups of one XCD cover an 8x8 block of tiles and share A/B
//     panels in that XCD's L2.
#include "phx_common.h"

#ifdef PHX_GEMM_TC
typedef float TIn;
typedef float TOut;
#else
typedef _Float16 TIn;
typedef _Float16 TOut;
#endif

#define BM PHX_H_BM  // 256
#define BN PHX_H_BN  // 128
#define BK PHX_H_BK  // 32
#define NT PHX_H_THREADS
#define WM 128  // wave tile rows
#define WN 64   // wave tile cols
#define GROUP_M 8

#define A_ROW_BYTES (BK * 2)             // 64
#define B_ROW_BYTES (BN * 2)             // 256
#define A_BYTES (BM * A_ROW_BYTES)       // 16 KiB
#define B_BYTES (BK * B_ROW_BYTES)       // 8 KiB
#define STAGE_BYTES (A_BYTES + B_BYTES)  // 24 KiB
#define EP_PITCH 68                      // epilogue LDS row pitch (floats)

typedef __fp16 phx_fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) phx_fp16x4 *phx_lds_h4p;

__device__ __forceinline__ uint32_t a_off(uint32_t row, uint32_t chunk) {
    return row * A_ROW_BYTES + ((chunk ^ ((row >> 2) & 3)) << 4);
}
__device__ __forceinline__ uint32_t b_off(uint32_t row, uint32_t chunk) {
    return row * B_ROW_BYTES + ((chunk ^ ((row & 3) << 2)) << 4);
}

// Buffer resource over `bytes` bytes from p (gfx9 dword3 = 0x00020000).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t phx_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

template <typename V>
__device__ __forceinline__ V buf_load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}

// Global loads of one K step.  Thread t stages
//   A: rows i*64 + t/4 (i < 4), 16-byte chunk t%4 (8 k values);
//   B: rows t/16 and t/16 + 16, chunk t%16 (8 n values).
struct Stage {
#ifdef PHX_GEMM_TC
    phx_f4 a[4][2];
    phx_f4 b[2][2];
#else
    phx_u4 a[4];
    phx_u4 b[2];
#endif
};

__device__ __forceinline__ void load_stage(Stage &st, const TIn *A, int64_t lda, const TIn *B,
                                           int64_t ldb, uint32_t m0, uint32_t n0, uint32_t k0,
                                           uint32_t voa, uint32_t vob) {
    const uint32_t esz = sizeof(TIn);
    const __amdgpu_buffer_rsrc_t ra =
        phx_rsrc(A + (int64_t)m0 * lda + k0, (uint32_t)((BM - 1) * lda + BK) * esz);
    const __amdgpu_buffer_rsrc_t rb =
        phx_rsrc(B + (int64_t)k0 * ldb + n0, (uint32_t)((BK - 1) * ldb + BN) * esz);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t so = (uint32_t)(i * 64 * lda) * esz;
#ifdef PHX_GEMM_TC
        st.a[i][0] = buf_load<phx_f4>(ra, voa, so);
        st.a[i][1] = buf_load<phx_f4>(ra, voa + 16, so);
#else
        st.a[i] = buf_load<phx_u4>(ra, voa, so);
#endif
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t so = (uint32_t)(i * 16 * ldb) * esz;
#ifdef PHX_GEMM_TC
        st.b[i][0] = buf_load<phx_f4>(rb, vob, so);
        st.b[i][1] = buf_load<phx_f4>(rb, vob + 16, so);
#else
        st.b[i] = buf_load<phx_u4>(rb, vob, so);
#endif
    }
}

#ifdef PHX_GEMM_TC
__device__ __forceinline__ phx_u4 to_h8(const phx_f4 &lo, const phx_f4 &hi) {
    phx_u4 v;
    v.x = phx_pack_h2(lo.x, lo.y);
    v.y = phx_pack_h2(lo.z, lo.w);
    v.z = phx_pack_h2(hi.x, hi.y);
    v.w = phx_pack_h2(hi.z, hi.w);
    return v;
}
#endif

__device__ __forceinline__ void store_stage(const Stage &st, char *stage, uint32_t tid) {
    char *As = stage, *Bs = stage + A_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#ifdef PHX_GEMM_TC
        const phx_u4 v = to_h8(st.a[i][0], st.a[i][1]);
#else
        const phx_u4 v = st.a[i];
#endif
        *(phx_u4 *)(As + a_off(i * 64 + (tid >> 2), tid & 3)) = v;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#ifdef PHX_GEMM_TC
        const phx_u4 v = to_h8(st.b[i][0], st.b[i][1]);
#else
        const phx_u4 v = st.b[i];
#endif
        *(phx_u4 *)(Bs + b_off(i * 16 + (tid >> 4), tid & 15)) = v;
    }
}

struct Frags {
    phx_h8 a[4];
    phx_h8 b[2];
};

// Operands of K slice s (k = 16s .. 16s+15) for this wave.
//   A: lane l reads row wm + 32i + l%32, k = 16s + 8*(l/32) .. +7.
//   B: lane l needs column wn + 32j + l%32 at the same 8 k; two transposing
//      reads (k +0..3, +4..7) from the lane's 16-lane group q = l/16, which
//      covers columns 16*(q%2) .. +15 and k half q/2.
__device__ __forceinline__ void read_frags(Frags &f, const char *stage, uint32_t s, uint32_t wm,
                                           uint32_t wn, uint32_t lane) {
    const char *As = stage;
    const char *Bs = stage + A_BYTES;
    const uint32_t lrow = lane & 31, g = lane >> 5;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        f.a[i] = *(const phx_h8 *)(As + a_off(wm + i * 32 + lrow, 2 * s + g));
    const uint32_t q = lane >> 4, sl = lane & 15;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t col = wn + j * 32 + 16 * (q & 1) + 4 * (sl & 3);  // halves
        phx_fp16x4 h[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t row = 16 * s + 8 * (q >> 1) + 4 * t + (sl >> 2);
            const uint32_t off = b_off(row, col >> 3) + ((col & 7) << 1);
            h[t] = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                (phx_lds_h4p)((__attribute__((address_space(3))) char *)(Bs + off)));
        }
        phx_h4 lo = __builtin_bit_cast(phx_h4, h[0]);
        phx_h4 hi = __builtin_bit_cast(phx_h4, h[1]);
        f.b[j] = (phx_h8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
}

__device__ __forceinline__ void mfma_slice(phx_f16v (&acc)[4][2], const Frags &f) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// Epilogue, staged through LDS so every global access is a 16-byte row
// chunk: each pass parks alpha*acc for RP rows of every wave's tile in `ep`
// (row pitch EP_PITCH floats, so the two lane halves hit different banks) and
// reads it back row-wise.  acc[i][j][r] sits at tile row 32i + 8*(r/4) +
// 4*lgrp + r%4, column 32j + lrow.  Uses 4 * RP * EP_PITCH * 4 bytes of LDS.
template <int RP>
__device__ __forceinline__ void epilogue(const phx_f16v (&acc)[4][2], float *ep_all, TOut *C,
                                         int64_t ldc, uint32_t m0, uint32_t n0, uint32_t wm,
                                         uint32_t wn, float alpha, float beta, uint32_t wave,
                                         uint32_t lane) {
    const uint32_t lrow = lane & 31, lgrp = lane >> 5;
    float *ep = ep_all + wave * (RP * EP_PITCH);
#pragma unroll
    for (int pass = 0; pass < WM / RP; ++pass) {
        __syncthreads();  // the previous pass (or the main loop) is done with LDS
        const int i = (pass * RP) / 32;
        const int r0 = ((pass * RP) % 32) / 2;  // first accumulator register of this pass
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = r0; r < r0 + RP / 2; ++r)
                ep[(8 * (r >> 2) + 4 * lgrp + (r & 3) - 2 * r0) * EP_PITCH + 32 * j + lrow] =
                    alpha * acc[i][j][r];
        __syncthreads();
        // RP rows x 64 values; a lane moves 8 consecutive values of a row
#pragma unroll
        for (int rr = 0; rr < RP / 8; ++rr) {
            const uint32_t row = rr * 8 + (lane >> 3), c8 = (lane & 7) * 8;
            const float *src = ep + row * EP_PITCH + c8;
            const phx_f4 v0 = *(const phx_f4 *)src, v1 = *(const phx_f4 *)(src + 4);
            TOut *dst = C + (int64_t)(m0 + wm + pass * RP + row) * ldc + n0 + wn + c8;
#ifdef PHX_GEMM_TC
            phx_f4 o0 = v0, o1 = v1;
            if (beta != 0.0f) {
                const phx_f4 c0 = *(const phx_f4 *)dst, c1 = *(const phx_f4 *)(dst + 4);
                o0 = v0 + beta * c0;
                o1 = v1 + beta * c1;
            }
            *(phx_f4 *)dst = o0;
            *(phx_f4 *)(dst + 4) = o1;
#else
            float o[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            if (beta != 0.0f) {
                const phx_h8 c = *(const phx_h8 *)dst;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float cb = beta * (float)c[e];
                    o[e] = o[e] + cb;
                }
            }
            phx_h8 h;
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (_Float16)o[e];
            *(phx_h8 *)dst = h;
#endif
        }
    }
    __syncthreads();  // LDS is reused by the next tile
}

#ifndef PHX_GEMM_TC
// ------------------------------------------------------------------ f16 path
// f16 inputs go global -> LDS directly (buffer_load ... lds: lane l of a
// 64-lane load writes LDS bytes base + 16l .. +15 from its own global
// address, so the XOR-swizzled layouts are built by choosing each lane's
// source).  Three 24 KiB stages, each its own LDS array so the compiler's
// LDS-DMA tracking tells them apart; K step t+2 is in flight while step t
// computes.  A wave waits for its own copies of a stage (vmcnt) before the
// barrier that publishes it; the raw s_barrier carries no memory fence, so
// nothing waits for the younger copies still in flight.
#define DMA_PER_STEP 6  // buffer_load ... lds per wave per K step (4 A + 2 B)

typedef __attribute__((address_space(3))) void *phx_lds_vp;

// s_waitcnt with only vmcnt = n (expcnt and lgkmcnt left at their maxima)
#define PHX_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

// Copies K step kt of A and B into stage `dst` (per-lane offsets voa/vob,
// wave w's share of the stage).
__device__ __forceinline__ void dma_step(char *dst, const TIn *A, int64_t lda, const TIn *B,
                                         int64_t ldb, uint32_t m0, uint32_t n0, uint32_t k0,
                                         uint32_t voa, uint32_t vob, uint32_t wave) {
    const __amdgpu_buffer_rsrc_t ra =
        phx_rsrc(A + (int64_t)m0 * lda + k0, (uint32_t)((BM - 1) * lda + BK) * 2);
    const __amdgpu_buffer_rsrc_t rb =
        phx_rsrc(B + (int64_t)k0 * ldb + n0, (uint32_t)((BK - 1) * ldb + BN) * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i)  // A chunks wave*256 + i*64 + lane
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ra, (phx_lds_vp)(dst + (wave * 256 + i * 64) * 16), 16, voa,
            (int)((uint32_t)((wave * 64 + i * 16) * lda) * 2), 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)  // B chunks wave*128 + i*64 + lane
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rb, (phx_lds_vp)(dst + A_BYTES + (wave * 128 + i * 64) * 16), 16, vob,
            (int)((uint32_t)((wave * 8 + i * 4) * ldb) * 2), 0, 0);
}

// One K step on stage `cur`; issues the copy of step kt+2 into `fill`.
__device__ __forceinline__ void dma_k_step(phx_f16v (&acc)[4][2], const char *cur, char *fill,
                                           const TIn *A, int64_t lda, const TIn *B, int64_t ldb,
                                           uint32_t m0, uint32_t n0, uint32_t kt, uint32_t nk,
                                           uint32_t voa, uint32_t vob, uint32_t wm, uint32_t wn,
                                           uint32_t wave, uint32_t lane) {
    if (kt + 1 < nk)
        PHX_WAIT_VMCNT(DMA_PER_STEP);  // own copies of step kt landed (kt+1 may fly)
    else
        PHX_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();  // everyone's step kt visible; step kt-1 reads done
    if (kt + 2 < nk) dma_step(fill, A, lda, B, ldb, m0, n0, (kt + 2) * BK, voa, vob, wave);
    Frags f0, f1;
    read_frags(f0, cur, 0, wm, wn, lane);
    read_frags(f1, cur, 1, wm, wn, lane);
    __builtin_amdgcn_sched_barrier(0);
    mfma_slice(acc, f0);
    __builtin_amdgcn_sched_barrier(0);
    mfma_slice(acc, f1);
    __builtin_amdgcn_sched_barrier(0);
}
#endif

extern "C" __global__ __launch_bounds__(NT, 2) void gemm(PHX_MEMREF2(TIn, a, int64_t),
                                                          PHX_MEMREF2(TIn, b, int64_t),
                                                          PHX_MEMREF2(TOut, c, int64_t),
                                                          float alpha, float beta) {
#ifdef PHX_GEMM_TC
    __shared__ __attribute__((aligned(16))) char lds[2][STAGE_BYTES];
#else
    __shared__ __attribute__((aligned(16))) char stg0[STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) char stg1[STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) char stg2[STAGE_BYTES];
#endif

    const int64_t M = a_s0, K = a_s1, N = b_s1;
    // Uniform preconditions (validated on the host by phx_check_shape; a
    // launch that breaks them writes nothing).
    if (blockDim.x != NT || M % BM || N % BN || K % BK || M <= 0 || N <= 0 || K <= 0 ||
        b_s0 != K || c_s0 != M || c_s1 != N || a_st1 != 1 || b_st1 != 1 || c_st1 != 1)
        return;

    const TIn *A = a_ptr + a_off;
    const TIn *B = b_ptr + b_off;
    TOut *C = c_ptr + c_off;
    const int64_t lda = a_st0, ldb = b_st0, ldc = c_st0;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = tid >> 6;
    const uint32_t wm = (wave >> 1) * WM;
    const uint32_t wn = (wave & 1) * WN;
    const uint32_t tiles_n = (uint32_t)(N / BN);
    const uint32_t tiles_m = (uint32_t)(M / BM);
    const uint32_t ntiles = tiles_m * tiles_n;
    const uint32_t nblk = phx_block_count();
    const uint32_t nk = (uint32_t)(K / BK);
#ifdef PHX_GEMM_TC
    // per-lane byte offsets of the staging loads (see Stage)
    const uint32_t voa = (uint32_t)(((tid >> 2) * lda + (tid & 3) * 8) * sizeof(TIn));
    const uint32_t vob = (uint32_t)(((tid >> 4) * ldb + (tid & 15) * 8) * sizeof(TIn));
#else
    // per-lane byte offsets of the LDS copies (see dma_step): the chunk a
    // lane fetches is the logical chunk its swizzled LDS slot holds.
    const uint32_t voa =
        (uint32_t)(((lane >> 2) * lda + 8 * ((lane & 3) ^ ((lane >> 4) & 3))) * 2);
    const uint32_t vob =
        (uint32_t)(((lane >> 4) * ldb + 8 * ((lane & 15) ^ (4 * ((lane >> 4) & 3)))) * 2);
#endif

    for (uint32_t t = phx_block_linear(); t < ntiles; t += nblk) {
        const uint32_t ts = nblk == ntiles ? phx_xcd_swizzle(t, ntiles) : t;
        const uint32_t gsz = GROUP_M * tiles_n;
        const uint32_t g0 = (ts / gsz) * GROUP_M;
        const uint32_t gm = (tiles_m - g0) < GROUP_M ? (tiles_m - g0) : GROUP_M;
        const uint32_t tm = g0 + (ts % gsz) % gm;
        const uint32_t tn = (ts % gsz) / gm;
        const uint32_t m0 = tm * BM, n0 = tn * BN;

        phx_f16v acc[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

#ifdef PHX_GEMM_TC
        Stage st;
        load_stage(st, A, lda, B, ldb, m0, n0, 0, voa, vob);
        store_stage(st, lds[0], tid);
        __syncthreads();

        for (uint32_t kt = 0; kt < nk; ++kt) {
            const char *cur = lds[kt & 1];
            Frags f0, f1;
            read_frags(f0, cur, 0, wm, wn, lane);
            if (kt + 1 < nk) load_stage(st, A, lda, B, ldb, m0, n0, (kt + 1) * BK, voa, vob);
            read_frags(f1, cur, 1, wm, wn, lane);
            __builtin_amdgcn_sched_barrier(0);
            mfma_slice(acc, f0);
            __builtin_amdgcn_sched_barrier(0);
            mfma_slice(acc, f1);
            __builtin_amdgcn_sched_barrier(0);
            if (kt + 1 < nk) store_stage(st, lds[(kt + 1) & 1], tid);
            __syncthreads();
        }
        epilogue<32>(acc, (float *)&lds[0][0], C, ldc, m0, n0, wm, wn, alpha, beta, wave, lane);
#else
        dma_step(stg0, A, lda, B, ldb, m0, n0, 0, voa, vob, wave);
        if (nk > 1) dma_step(stg1, A, lda, B, ldb, m0, n0, BK, voa, vob, wave);
        uint32_t kt = 0;
        for (; kt + 2 < nk; kt += 3) {
            dma_k_step(acc, stg0, stg2, A, lda, B, ldb, m0, n0, kt, nk, voa, vob, wm, wn, wave, lane);
            dma_k_step(acc, stg1, stg0, A, lda, B, ldb, m0, n0, kt + 1, nk, voa, vob, wm, wn, wave,
                       lane);
            dma_k_step(acc, stg2, stg1, A, lda, B, ldb, m0, n0, kt + 2, nk, voa, vob, wm, wn, wave,
                       lane);
        }
        if (kt < nk)
            dma_k_step(acc, stg0, stg2, A, lda, B, ldb, m0, n0, kt, nk, voa, vob, wm, wn, wave, lane);
        if (kt + 1 < nk)
            dma_k_step(acc, stg1, stg0, A, lda, B, ldb, m0, n0, kt + 1, nk, voa, vob, wm, wn, wave,
                       lane);
        PHX_WAIT_VMCNT(0);
        epilogue<16>(acc, (float *)stg0, C, ldc, m0, n0, wm, wn, alpha, beta, wave, lane);
#endif
    }
}
