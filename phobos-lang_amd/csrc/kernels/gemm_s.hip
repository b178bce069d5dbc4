// f32 GEMM leaf kernels for gfx950 on the f32 matrix cores.
//
// Built twice from this file:
//   -DPHX_GEMM_FP32        gemm_fp32.ph, entry "gemm":
//                          C = fl(fl(alpha*acc) + fl(beta*c_old))
//                          (phobos-lang/src/codegen/matmul.rs:384-403)
//   -DPHX_MATMUL_CLUSTER   the two leaves clustergen synthesises from
//                          matmul_cluster_fp32.ph (phobos-cluster/src/clustergen.rs):
//                          "matmul"      step leaf, C = fl(fl(alpha*acc) + c_old),
//                                        an implicit beta of 1 (:1363-1399); its
//                                        beta parameter is carried but unused;
//                          "matmul_init" init leaf, C = fl(beta*c_old) (:1292-1360).
// All take the reference's i32 exploded-memref descriptors (gemm_fp32.ph has no
// @tensorcore; every pod leaf is compiled at the default 32-bit index,
// phobos-sched/src/server.rs:696-714).  acc is an f32 sum of exact f32
// products (v_mfma_f32_32x32x2_f32); the reference sums with fma.rn, so the
// two agree to f32 summation-order rounding (and exactly on integer data).
//
// MI355X design
//   * 128x128 output tile, K step 32, 256 threads = 4 waves (2x2) of 64x64,
//     each 2x2 v_mfma_f32_32x32x2_f32 tiles (64 accumulators).  LDS is 2 x 32
//     KiB, so two workgroups share a CU.
//   * The MFMA's 2-wide k slice is permuted so that a lane's four consecutive
//     MFMAs read four consecutive k from one ds_read_b128: lane group g of MFMA
//     s uses k = 8q + 4g + s.  A is staged As[m][k], B transposed to Bs[n][k]
//     (a free 4x4 register transpose); 128-byte rows with the 16-byte chunk
//     XOR-swizzled by ((row >> 1) & 7) keep writes and reads conflict free
//     on the 64-bank LDS.
//   * Double-buffered LDS with the next K step's loads in flight during the
//     current step's MFMAs; XCD-aware grouped tile order as in gemm_h.hip.
#include "phx_common.h"

#define BM PHX_S_BM
#define BN PHX_S_BN
#define BK PHX_S_BK
#define NT PHX_S_THREADS
#define WM 64
#define WN 64
#define GROUP_M 4
#define LDS_ROW_BYTES (BK * 4)
#define LDS_TILE_BYTES (BM * LDS_ROW_BYTES)

__device__ __forceinline__ uint32_t lds_off(uint32_t row, uint32_t chunk) {
    return row * LDS_ROW_BYTES + ((chunk ^ ((row >> 1) & 7)) << 4);
}

struct Stage {
    phx_f4 a[4];
    phx_f4 b[4];
};

__device__ __forceinline__ void load_stage(Stage &st, const float *A, int64_t lda, const float *B,
                                           int64_t ldb, uint32_t m0, uint32_t n0, uint32_t k0,
                                           uint32_t tid) {
    const uint32_t ar = tid >> 3, ac = tid & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        st.a[i] = *(const phx_f4 *)(A + (int64_t)(m0 + i * 32 + ar) * lda + k0 + ac * 4);
    const uint32_t bk = tid & 7, bn = tid >> 3;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        st.b[i] = *(const phx_f4 *)(B + (int64_t)(k0 + bk * 4 + i) * ldb + n0 + bn * 4);
}

__device__ __forceinline__ void store_stage(const Stage &st, char *As, char *Bs, uint32_t tid) {
    const uint32_t ar = tid >> 3, ac = tid & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i) *(phx_f4 *)(As + lds_off(i * 32 + ar, ac)) = st.a[i];
    const uint32_t bk = tid & 7, bn = tid >> 3;
    phx_f4 c0 = {st.b[0].x, st.b[1].x, st.b[2].x, st.b[3].x};
    phx_f4 c1 = {st.b[0].y, st.b[1].y, st.b[2].y, st.b[3].y};
    phx_f4 c2 = {st.b[0].z, st.b[1].z, st.b[2].z, st.b[3].z};
    phx_f4 c3 = {st.b[0].w, st.b[1].w, st.b[2].w, st.b[3].w};
    *(phx_f4 *)(Bs + lds_off(bn * 4 + 0, bk)) = c0;
    *(phx_f4 *)(Bs + lds_off(bn * 4 + 1, bk)) = c1;
    *(phx_f4 *)(Bs + lds_off(bn * 4 + 2, bk)) = c2;
    *(phx_f4 *)(Bs + lds_off(bn * 4 + 3, bk)) = c3;
}

// STEP: cluster step leaf (implicit beta 1), else the plain gemm epilogue.
template <bool STEP>
__device__ __forceinline__ void gemm_s_body(const float *A, int64_t lda, const float *B,
                                            int64_t ldb, float *C, int64_t ldc, int64_t M,
                                            int64_t N, int64_t K, float alpha, float beta,
                                            char (*lds)[2][LDS_TILE_BYTES]) {
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
    const uint32_t lrow = lane & 31;
    const uint32_t lgrp = lane >> 5;

    for (uint32_t t = phx_block_linear(); t < ntiles; t += nblk) {
        const uint32_t ts = nblk == ntiles ? phx_xcd_swizzle(t, ntiles) : t;
        const uint32_t gsz = GROUP_M * tiles_n;
        const uint32_t g0 = (ts / gsz) * GROUP_M;
        const uint32_t gm = (tiles_m - g0) < GROUP_M ? (tiles_m - g0) : GROUP_M;
        const uint32_t tm = g0 + (ts % gsz) % gm;
        const uint32_t tn = (ts % gsz) / gm;
        const uint32_t m0 = tm * BM, n0 = tn * BN;

        phx_f16v acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
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
            for (uint32_t q = 0; q < BK / 8; ++q) {
                const uint32_t chunk = 2 * q + lgrp;
                phx_f4 af[2], bf[2];
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    af[i] = *(const phx_f4 *)(As + lds_off(wm + i * 32 + lrow, chunk));
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    bf[j] = *(const phx_f4 *)(Bs + lds_off(wn + j * 32 + lrow, chunk));
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s],
                                                                             acc[i][j], 0, 0, 0);
            }
            if (kt + 1 < nk) store_stage(st, lds[cur ^ 1][0], lds[cur ^ 1][1], tid);
            __syncthreads();
        }

        // acc[i][j][r]: row = 8*(r/4) + 4*lgrp + r%4, col = lrow
        if (STEP || beta != 0.0f) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t col = n0 + wn + j * 32 + lrow;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const uint32_t row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * lgrp + (r & 3);
                        float *pc = C + (int64_t)row * ldc + col;
                        float v = alpha * acc[i][j][r];
                        float cb = STEP ? *pc : beta * *pc;
                        *pc = v + cb;
                    }
                }
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t col = n0 + wn + j * 32 + lrow;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const uint32_t row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * lgrp + (r & 3);
                        C[(int64_t)row * ldc + col] = alpha * acc[i][j][r];
                    }
                }
        }
    }
}

#define GEMM_S_PRELUDE                                                                        \
    __shared__ __attribute__((aligned(16))) char lds[2][2][LDS_TILE_BYTES];                   \
    const int64_t M = a_s0, K = a_s1, N = b_s1;                                               \
    if (blockDim.x != NT || M % BM || N % BN || K % BK || M <= 0 || N <= 0 || K <= 0 ||       \
        b_s0 != K || c_s0 != M || c_s1 != N || a_st1 != 1 || b_st1 != 1 || c_st1 != 1)       \
        return;

#ifdef PHX_GEMM_FP32
extern "C" __global__ __launch_bounds__(NT, 2) void gemm(PHX_MEMREF2(float, a, int32_t),
                                                          PHX_MEMREF2(float, b, int32_t),
                                                          PHX_MEMREF2(float, c, int32_t),
                                                          float alpha, float beta) {
    GEMM_S_PRELUDE
    gemm_s_body<false>(a_ptr + a_off, a_st0, b_ptr + b_off, b_st0, c_ptr + c_off, c_st0, M, N, K,
                       alpha, beta, lds);
}
#endif

#ifdef PHX_MATMUL_CLUSTER
extern "C" __global__ __launch_bounds__(NT, 2) void matmul(PHX_MEMREF2(float, a, int32_t),
                                                            PHX_MEMREF2(float, b, int32_t),
                                                            PHX_MEMREF2(float, c, int32_t),
                                                            float alpha, float beta) {
    GEMM_S_PRELUDE
    gemm_s_body<true>(a_ptr + a_off, a_st0, b_ptr + b_off, b_st0, c_ptr + c_off, c_st0, M, N, K,
                      alpha, beta, lds);
}

// C = fl(beta * C) over a [M, N] tile: an HBM stream of 8 bytes per element.
extern "C" __global__ __launch_bounds__(PHX_EW_THREADS) void matmul_init(
    PHX_MEMREF2(float, c, int32_t), float beta) {
    if (blockDim.x != PHX_EW_THREADS || c_st1 != 1) return;
    float *C = c_ptr + c_off;
    const int64_t rows = c_s0, cols = c_s1, ld = c_st0;
    const uint32_t nblk = phx_block_count(), bid = phx_block_linear(), tid = threadIdx.x;
    if (ld == cols && (((uintptr_t)C) & 15) == 0) {
        const int64_t n = rows * cols, nv = n >> 2;
        phx_f4 *cv = (phx_f4 *)C;
        const int64_t per = PHX_EW_BLOCK_ELEMS / 4;  // float4 per block step
        for (int64_t base = (int64_t)bid * per + tid; base < nv; base += (int64_t)nblk * per) {
            phx_f4 r[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (base + u * PHX_EW_THREADS < nv) r[u] = cv[base + u * PHX_EW_THREADS];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (base + u * PHX_EW_THREADS < nv) cv[base + u * PHX_EW_THREADS] = beta * r[u];
        }
        if (bid == 0 && nv * 4 + tid < n) C[nv * 4 + tid] = beta * C[nv * 4 + tid];
        return;
    }
    const int64_t n = rows * cols;
    for (int64_t i = (int64_t)bid * PHX_EW_THREADS + tid; i < n; i += (int64_t)nblk * PHX_EW_THREADS) {
        const int64_t r = i / cols, cidx = i % cols;
        C[r * ld + cidx] = beta * C[r * ld + cidx];
    }
}
#endif
