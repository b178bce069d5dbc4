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
//   * 256x256 output tile per workgroup, 256 threads = 4 waves (2x2), each wave
//     a 128x128 sub-tile = 4x4 v_mfma_f32_32x32x16_f16 tiles whose 256 f32
//     accumulators live in AGPRs.  At 4096^3 this is 256 tiles: one per CU.
//   * K step 64.  A is staged as As[m][k], B transposed to Bs[n][k], so every
//     MFMA operand is one ds_read_b128 (8 consecutive k of one row/column).
//     Rows are 128 bytes; the 16-byte chunk index is XOR-swizzled with
//     (row & 7), which makes both the staging writes and the operand reads
//     bank-conflict free.
//   * B (row-major [K,N]) is transposed in registers: each thread loads an 8x8
//     block (8 rows of 16 bytes) and re-packs it with v_perm into 8 k-runs.
//   * LDS double buffer (2 x 64 KiB); the next K step's global loads are in
//     flight while the current step's 64 MFMAs per wave run; one barrier per
//     K step.
//   * Workgroups are renumbered XCD-major and grouped 4 tile-rows deep so the
//     32 workgroups of one XCD cover a 4x8 block of tiles and share A/B panels
//     in that XCD's L2.
#include "phx_common.h"

#ifdef PHX_GEMM_TC
typedef float TIn;
typedef float TOut;
#else
typedef _Float16 TIn;
typedef _Float16 TOut;
#endif

#define BM PHX_H_BM
#define BN PHX_H_BN
#define BK PHX_H_BK
#define NT PHX_H_THREADS
#define WM 128  // wave tile rows
#define WN 128  // wave tile cols
#define GROUP_M 4

// LDS: [buffer][row][64 halves], 16-byte chunks swizzled by (row & 7).
#define LDS_ROW_BYTES (BK * 2)
#define LDS_TILE_BYTES (BM * LDS_ROW_BYTES)

__device__ __forceinline__ uint32_t lds_off(uint32_t row, uint32_t chunk) {
    return row * LDS_ROW_BYTES + ((chunk ^ (row & 7)) << 4);
}

// Global loads of one K step, held in registers until written to LDS.
struct Stage {
#ifdef PHX_GEMM_TC
    phx_f4 a[8][2];  // 8 row-chunks, each 8 floats
    phx_f4 b[8][2];  // 8 rows of the 8x8 block, each 8 floats
#else
    phx_u4 a[8];     // 8 row-chunks of 8 halves
    phx_u4 b[8];     // 8 rows of the 8x8 block, 8 halves each
#endif
};

__device__ __forceinline__ void load_stage(Stage &st, const TIn *A, int64_t lda, const TIn *B,
                                           int64_t ldb, uint32_t m0, uint32_t n0, uint32_t k0,
                                           uint32_t tid) {
    // A: row = i*32 + tid/8, chunk (8 k values) = tid%8
    const uint32_t ar = tid >> 3, ac = tid & 7;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const TIn *p = A + (int64_t)(m0 + i * 32 + ar) * lda + k0 + ac * 8;
#ifdef PHX_GEMM_TC
        st.a[i][0] = *(const phx_f4 *)p;
        st.a[i][1] = *(const phx_f4 *)(p + 4);
#else
        st.a[i] = *(const phx_u4 *)p;
#endif
    }
    // B: 8x8 block, k rows 8*(tid%8)+i, n cols 8*(tid/8)..+7
    const uint32_t bk = tid & 7, bn = tid >> 3;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const TIn *p = B + (int64_t)(k0 + bk * 8 + i) * ldb + n0 + bn * 8;
#ifdef PHX_GEMM_TC
        st.b[i][0] = *(const phx_f4 *)p;
        st.b[i][1] = *(const phx_f4 *)(p + 4);
#else
        st.b[i] = *(const phx_u4 *)p;
#endif
    }
}

#ifndef PHX_GEMM_TC
// Selects the low (hi=0) or high (hi=1) halves of two dwords: {lo16(x), lo16(y)}.
__device__ __forceinline__ uint32_t pk_lo(uint32_t x, uint32_t y) {
    return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t pk_hi(uint32_t x, uint32_t y) {
    return __builtin_amdgcn_perm(y, x, 0x07060302u);
}
#endif

__device__ __forceinline__ void store_stage(const Stage &st, char *As, char *Bs, uint32_t tid) {
    const uint32_t ar = tid >> 3, ac = tid & 7;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#ifdef PHX_GEMM_TC
        phx_u4 v;
        v.x = phx_pack_h2(st.a[i][0].x, st.a[i][0].y);
        v.y = phx_pack_h2(st.a[i][0].z, st.a[i][0].w);
        v.z = phx_pack_h2(st.a[i][1].x, st.a[i][1].y);
        v.w = phx_pack_h2(st.a[i][1].z, st.a[i][1].w);
#else
        phx_u4 v = st.a[i];
#endif
        *(phx_u4 *)(As + lds_off(i * 32 + ar, ac)) = v;
    }
    // Transpose the 8x8 block: output column j (n = 8*bn + j) holds
    // k = 8*bk .. 8*bk+7.
    const uint32_t bk = tid & 7, bn = tid >> 3;
#ifdef PHX_GEMM_TC
    float e[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        e[i][0] = st.b[i][0].x; e[i][1] = st.b[i][0].y; e[i][2] = st.b[i][0].z; e[i][3] = st.b[i][0].w;
        e[i][4] = st.b[i][1].x; e[i][5] = st.b[i][1].y; e[i][6] = st.b[i][1].z; e[i][7] = st.b[i][1].w;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        phx_u4 v;
        v.x = phx_pack_h2(e[0][j], e[1][j]);
        v.y = phx_pack_h2(e[2][j], e[3][j]);
        v.z = phx_pack_h2(e[4][j], e[5][j]);
        v.w = phx_pack_h2(e[6][j], e[7][j]);
        *(phx_u4 *)(Bs + lds_off(bn * 8 + j, bk)) = v;
    }
#else
    // row i dword d holds halves (n=2d, n=2d+1).  Column j=2d+h of rows
    // (i, i+1) packs as pk_lo/pk_hi of dword d of those rows.
    uint32_t r[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        r[i][0] = st.b[i].x; r[i][1] = st.b[i].y; r[i][2] = st.b[i].z; r[i][3] = st.b[i].w;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        phx_u4 lo, hi;
        lo.x = pk_lo(r[0][d], r[1][d]); hi.x = pk_hi(r[0][d], r[1][d]);
        lo.y = pk_lo(r[2][d], r[3][d]); hi.y = pk_hi(r[2][d], r[3][d]);
        lo.z = pk_lo(r[4][d], r[5][d]); hi.z = pk_hi(r[4][d], r[5][d]);
        lo.w = pk_lo(r[6][d], r[7][d]); hi.w = pk_hi(r[6][d], r[7][d]);
        *(phx_u4 *)(Bs + lds_off(bn * 8 + 2 * d, bk)) = lo;
        *(phx_u4 *)(Bs + lds_off(bn * 8 + 2 * d + 1, bk)) = hi;
    }
#endif
}

extern "C" __global__ __launch_bounds__(NT, 1) void gemm(PHX_MEMREF2(TIn, a, int64_t),
                                                          PHX_MEMREF2(TIn, b, int64_t),
                                                          PHX_MEMREF2(TOut, c, int64_t),
                                                          float alpha, float beta) {
    __shared__ __attribute__((aligned(16))) char lds[2][2][LDS_TILE_BYTES];

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
    const uint32_t wm = (wave >> 1) * WM;  // wave row offset in tile
    const uint32_t wn = (wave & 1) * WN;
    const uint32_t tiles_n = (uint32_t)(N / BN);
    const uint32_t ntiles = (uint32_t)(M / BM) * tiles_n;
    const uint32_t nblk = phx_block_count();
    const uint32_t nk = (uint32_t)(K / BK);

    const uint32_t lrow = lane & 31;  // MFMA operand row/col within a 32 tile
    const uint32_t lgrp = lane >> 5;  // k half (0/1) inside a 16-wide k slice

    for (uint32_t t = phx_block_linear(); t < ntiles; t += nblk) {
        const uint32_t ts = nblk == ntiles ? phx_xcd_swizzle(t, ntiles) : t;
        // grouped ordering: GROUP_M tile-rows per group
        const uint32_t tiles_m = ntiles / tiles_n;
        const uint32_t gsz = GROUP_M * tiles_n;
        const uint32_t g0 = (ts / gsz) * GROUP_M;
        const uint32_t gm = (tiles_m - g0) < GROUP_M ? (tiles_m - g0) : GROUP_M;
        const uint32_t tm = g0 + (ts % gsz) % gm;
        const uint32_t tn = (ts % gsz) / gm;
        const uint32_t m0 = tm * BM, n0 = tn * BN;

        phx_f16v acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

        Stage st;
        load_stage(st, A, lda, B, ldb, m0, n0, 0, tid);
        store_stage(st, lds[0][0], lds[0][1], tid);
        __syncthreads();

        for (uint32_t kt = 0; kt < nk; ++kt) {
            const uint32_t cur = kt & 1;
            if (kt + 1 < nk) load_stage(st, A, lda, B, ldb, m0, n0, (kt + 1) * BK, tid);
            const char *As = lds[cur][0];
            const char *Bs = lds[cur][1];
#pragma unroll
            for (uint32_t s = 0; s < BK / 16; ++s) {
                const uint32_t chunk = 2 * s + lgrp;
                phx_h8 af[4], bf[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    af[i] = *(const phx_h8 *)(As + lds_off(wm + i * 32 + lrow, chunk));
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    bf[j] = *(const phx_h8 *)(Bs + lds_off(wn + j * 32 + lrow, chunk));
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] =
                            __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
            if (kt + 1 < nk) store_stage(st, lds[cur ^ 1][0], lds[cur ^ 1][1], tid);
            __syncthreads();
        }

        // Epilogue.  acc[i][j][r]: row = 8*(r/4) + 4*lgrp + r%4, col = lrow.
        const bool read_c = beta != 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t col = n0 + wn + j * 32 + lrow;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * lgrp + (r & 3);
                    TOut *pc = C + (int64_t)row * ldc + col;
                    float v = alpha * acc[i][j][r];
                    if (read_c) {
                        float cb = beta * (float)*pc;
                        v = v + cb;
                    }
                    *pc = (TOut)v;
                }
            }
        }
    }
}
