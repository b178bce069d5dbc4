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
//   * 256x256 output tile per workgroup, one workgroup per CU, 4 waves in a
//     2x2 arrangement, each owning 128x128 = 4x4 v_mfma_f32_32x32x2_f32 tiles
//     whose 256 accumulators live in AGPRs.  K step 16: 128 MFMAs (8192
//     matrix-core cycles) per wave per step, so one barrier per step costs
//     little.
//   * Ragged shapes (M any, N and K multiples of 4, so every 16-byte chunk is
//     whole): each step's buffer resources end at the last row / column that
//     exists, so rows past M and B rows past K read zeros (the range check
//     covers the scalar offset too); A chunks past K in the last, partial K
//     step take an out-of-range lane offset and read zeros; tiles crossing M
//     or N are stored masked.  Columns of B past N in a row are read but only
//     reach output columns that are not stored.
//   * The MFMA's 2-wide k slice is permuted so that a lane's four consecutive
//     MFMAs read four consecutive k: lane group g of MFMA s uses k = 8q + 4g +
//     s.  A is staged As[m][k] (64-byte rows, 16-byte chunks XOR (row>>2)&3),
//     so an A operand for 4 MFMAs is one ds_read_b128.  B stays row-major
//     Bs[k][n] (1 KiB rows); its operand is four ds_read_b32 (one per k), and
//     rows whose k differs by 4 (the two lane groups) are offset by 128 bytes
//     (chunk XOR 8 when bit 2 of k is set), so all 64 lanes hit distinct banks.
//   * Both operands are copied global -> LDS directly (buffer_load ... lds, 16
//     bytes per lane) into a ring of 3 stages of 32 KiB; step k+3 is issued
//     into the stage step k just released.  Copies of steps past K read an
//     empty buffer resource (zeros), which keeps every wait count constant.
//   * Software pipeline as in the f16 GEMM: the MFMAs of k-group 0 run while
//     group 1's operands are read; then the wait for the next step and the
//     barrier; then group 1's MFMAs while the next step's group-0 operands are
//     read and the copy of step k+3 is issued.
//   * Workgroups are renumbered XCD-major and grouped 4 tile-rows deep.
#include "phx_common.h"

#define NT PHX_S_THREADS
#define GROUP_M 4
#define NSTG 3
#define EP_RP 8  // epilogue rows per pass

typedef __attribute__((address_space(3))) void *phx_lds_vp;

#define PHX_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))
#define PHX_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (((n) >> 4) << 14))
#define SGB(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
#define G_MFMA 0x008
#define G_VMEM 0x020
#define G_DSR 0x100

__device__ __forceinline__ __amdgpu_buffer_rsrc_t phx_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

// One tiling: a TM x TN output tile per workgroup of 4 waves in a 2 x 2
// arrangement (each WM x WN = MI x NJ MFMA tiles of 32 x 32), K steps of TK.
// TK = 8, 16 or 32 (1, 2 or 4 k-groups of 8 per step); TM, TN multiples of
// 64.  The tilings the reference's autotuner chooses among are its
// @autotune(TILE_M, TILE_N in [32, 256], TILE_K in [4, 32]) dims
// (examples/gemm_fp32.ph:1); the built-in plan is 256 x 256 x 16.
template <int TM_, int TN_, int TK_>
struct Tile {
    static constexpr int TM = TM_, TN = TN_, TK = TK_;
    static constexpr int WM = TM / 2, WN = TN / 2;
    static constexpr int MI = WM / 32, NJ = WN / 32;
    static constexpr int CA = TK / 4;    // 16-byte chunks per A row
    static constexpr int RA = 64 / TK;   // A rows per 256 bytes (one LDS bank sweep)
    static constexpr int NQ = TK / 8;    // k-groups per step
    static constexpr int A_BYTES = TM * TK * 4;
    static constexpr int B_ROW = TN * 4;
    static constexpr int B_BYTES = TK * B_ROW;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int A_COPIES = A_BYTES / 4096;  // 1 KiB copies per wave per step
    static constexpr int B_COPIES = B_BYTES / 4096;
    static constexpr int DMA = A_COPIES + B_COPIES;
    static constexpr int A_RPC = 64 / CA;      // A rows per copy
    static constexpr int B_LPR = TN / 4;       // lanes per B row in a copy
    static constexpr int B_RPC = 64 / B_LPR;   // B rows per copy
    static constexpr int NMF = 4 * MI * NJ;    // MFMAs per k-group
    static constexpr int RD = MI + 4 * NJ;     // LDS operand reads per k-group
    static constexpr int EP_PITCH = WN + 8;    // epilogue LDS row pitch (floats)
    static constexpr int EP_LPR = WN / 4;      // lanes per epilogue row
    static constexpr int EP_RPI = 64 / EP_LPR; // rows per epilogue store
    static constexpr int OCC = MI * NJ * 16 <= 128 ? 2 : 1;  // workgroups per CU
    static_assert(TK == 8 || TK == 16 || TK == 32, "TK");
    static_assert(TM % 64 == 0 && TN % 64 == 0 && TN <= 256, "TM, TN");
    static_assert(A_COPIES >= 1 && B_COPIES >= 1 && A_BYTES % 4096 == 0 && B_BYTES % 4096 == 0,
                  "whole copies per wave");
    static_assert(CA < 8 || A_COPIES % 2 == 0, "TK = 32: A copies come in pairs");
    static_assert(4 * EP_RP * EP_PITCH * 4 <= NSTG * STAGE, "epilogue fits in the stages");
};

// A is staged As[m][k] (TK*4-byte rows) with 16-byte chunks XOR ((row / RA) &
// (CA - 1)), so the 16 rows one ds_read_b128 quarter-wave reads at one
// logical chunk land in 16 distinct 16-byte slots of the 256-byte bank sweep.
template <class T>
__device__ __forceinline__ uint32_t a_off(uint32_t row, uint32_t chunk) {
    return row * (T::TK * 4) + ((chunk ^ ((row / T::RA) & (T::CA - 1))) << 4);
}
// B stays row-major Bs[k][n]; rows whose k differs by 4 (the two lane groups
// of an operand read) are offset by 128 bytes.
template <class T>
__device__ __forceinline__ uint32_t b_off(uint32_t row, uint32_t chunk) {
    return row * T::B_ROW + ((chunk ^ (((row >> 2) & 1) << 3)) << 4);
}

// Operands of k-group q (k = 8q .. 8q+7) for this wave: a[i] = A row wm +
// 32i + lane%32, k = 8q + 4g .. +3; b[j][s] = B[8q + 4g + s][wn + 32j + lane%32].
template <class T>
struct Frags {
    phx_f4 a[T::MI];
    float b[T::NJ][4];
};

template <class T>
__device__ __forceinline__ void read_frags(Frags<T> &f, const char *stage, uint32_t q,
                                           uint32_t wm, uint32_t wn, uint32_t lane) {
    const char *As = stage, *Bs = stage + T::A_BYTES;
    const uint32_t lrow = lane & 31, g = lane >> 5;
#pragma unroll
    for (int i = 0; i < T::MI; ++i)
        f.a[i] = *(const phx_f4 *)(As + a_off<T>(wm + 32 * i + lrow, 2 * q + g));
#pragma unroll
    for (int j = 0; j < T::NJ; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t row = 8 * q + 4 * g + s, col = wn + 32 * j + lrow;
            f.b[j][s] = *(const float *)(Bs + b_off<T>(row, col >> 2) + 4 * (col & 3));
        }
}

// MFMA order: s outermost, then (i, j): MI*NJ independent accumulators
// between two updates of the same one.
template <class T>
__device__ __forceinline__ void mfma_all(phx_f16v (&acc)[T::MI][T::NJ], const Frags<T> &f) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < T::MI; ++i)
#pragma unroll
            for (int j = 0; j < T::NJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[i][s], f.b[j][s], acc[i][j],
                                                                 0, 0, 0);
}

// Copies K step k0 of A and B into stage dst.  Copy c of the workgroup (c =
// wave * COPIES + i) fills 1 KiB of LDS, lane l the l-th 16-byte slot: for A
// rows c*A_RPC + l/CA, physical chunk l%CA; for B rows c*B_RPC + l/B_LPR,
// physical chunk l%B_LPR.  Each lane fetches the logical chunk its swizzled
// slot holds.  Rows past M (A) and past K (B) read zeros through the
// resource bounds; in the last, partial K step A chunks past K take an
// out-of-range offset and read zeros.
template <class T>
__device__ __forceinline__ void dma_step(char *dst, const float *A, int64_t lda, const float *B,
                                         int64_t ldb, int64_t M, int64_t N, int64_t K, uint32_t m0,
                                         uint32_t n0, uint32_t k0, uint32_t wave, uint32_t lane) {
    const bool in = (int64_t)k0 < K;
    const int64_t mrows = M - m0 < T::TM ? M - m0 : T::TM;
    const int64_t kr = in ? K - k0 : 0;  // columns of this step that exist
    const int64_t kw = kr < T::TK ? kr : T::TK;
    const __amdgpu_buffer_rsrc_t ra = phx_rsrc(
        A + (int64_t)m0 * lda + (in ? k0 : 0), in ? (uint32_t)(((mrows - 1) * lda + kw) * 4) : 0);
    // B rows are full reads even when the tile crosses N: columns past N land
    // in output columns that are not stored; the resource ends at the
    // matrix's last element.
    const int64_t brem = (K - (in ? k0 : 0) - 1) * ldb + (N - n0);
    const int64_t bmax = (int64_t)(T::TK - 1) * ldb + T::TN;
    const uint32_t bbytes = (uint32_t)((brem < bmax ? brem : bmax) * 4);
    const __amdgpu_buffer_rsrc_t rb =
        phx_rsrc(B + (int64_t)(in ? k0 : 0) * ldb + n0, in ? bbytes : 0);
    const uint32_t ar = lane / T::CA, apc = lane % T::CA;
#pragma unroll
    for (int i = 0; i < T::A_COPIES; ++i) {
        // copy c's first row is 4c row-sweeps in, so only 4c & (CA - 1)
        // (0, or 4 for odd copies when CA = 8) enters the swizzle
        const uint32_t x = (4 * i) & (T::CA - 1);
        const uint32_t c = apc ^ ((x + ar / T::RA) & (T::CA - 1));
        const uint32_t va = 4 * c < (uint32_t)kw ? (uint32_t)(ar * lda * 4 + c * 16) : 0x80000000u;
        const uint32_t row0 = (wave * T::A_COPIES + i) * T::A_RPC;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ra, (phx_lds_vp)(dst + (wave * T::A_COPIES + i) * 1024), 16, va,
            (int)((uint32_t)(row0 * lda) * 4), 0, 0);
    }
    const uint32_t br = lane / T::B_LPR, bpc = lane % T::B_LPR;
#pragma unroll
    for (int i = 0; i < T::B_COPIES; ++i) {
        const uint32_t row0 = (wave * T::B_COPIES + i) * T::B_RPC;
        const uint32_t c = bpc ^ ((((row0 + br) >> 2) & 1) << 3);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rb, (phx_lds_vp)(dst + T::A_BYTES + (wave * T::B_COPIES + i) * 1024), 16,
            br * (uint32_t)ldb * 4 + c * 16, (int)((uint32_t)(row0 * ldb) * 4), 0, 0);
    }
}

// Interleave of one k-group's MFMAs with the operand reads for the next
// group (and, in the step's last group, the copies of step kt+3).
template <class T, bool COPIES>
__device__ __forceinline__ void sched_group() {
#pragma unroll
    for (int i = 0; i < T::NMF; ++i) {
        SGB(G_MFMA, 1);
        if (i < T::RD) SGB(G_DSR, 1);
        if (COPIES && i >= T::RD && i < T::RD + T::DMA) SGB(G_VMEM, 1);
    }
    if constexpr (T::RD > T::NMF) SGB(G_DSR, T::RD - T::NMF);
    if constexpr (COPIES && T::RD + T::DMA > T::NMF) {
        constexpr int left = T::RD >= T::NMF ? T::DMA : T::RD + T::DMA - T::NMF;
        SGB(G_VMEM, left);
    }
}

// One K step: each k-group's MFMAs run while the next group's operands are
// read; before the last group, the wait for this wave's copies of step kt+1
// and the barrier, after which the next step's group 0 is read and step
// kt+3 is copied into the stage this step releases.  F0 holds group 0 on
// entry; on exit it holds the next step's group 0.
template <class T>
__device__ __forceinline__ void k_step(phx_f16v (&acc)[T::MI][T::NJ], Frags<T> &F0,
                                       Frags<T> &F1, char *cur, const char *nxt, const float *A,
                                       int64_t lda, const float *B, int64_t ldb, int64_t M,
                                       int64_t N, int64_t K, uint32_t m0, uint32_t n0,
                                       uint32_t kt, uint32_t wm, uint32_t wn, uint32_t wave,
                                       uint32_t lane) {
#pragma unroll
    for (int q = 0; q < T::NQ; ++q) {
        Frags<T> &Fc = (q & 1) ? F1 : F0;  // this group's operands
        Frags<T> &Fn = (q & 1) ? F0 : F1;  // the next group's
        if (q < T::NQ - 1) {
            read_frags<T>(Fn, cur, q + 1, wm, wn, lane);
            mfma_all<T>(acc, Fc);
            sched_group<T, false>();
        } else {
            __builtin_amdgcn_sched_barrier(0);
            // own copies of kt+1 landed, reads of cur done
            PHX_WAIT_VM_LGKM0((NSTG - 2) * T::DMA);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            read_frags<T>(Fn, nxt, 0, wm, wn, lane);
            dma_step<T>(cur, A, lda, B, ldb, M, N, K, m0, n0, (kt + NSTG) * T::TK, wave, lane);
            mfma_all<T>(acc, Fc);
            sched_group<T, true>();
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (T::NQ & 1) {  // the next step's group 0 was read into F1
        const Frags<T> t = F0;
        F0 = F1;
        F1 = t;
    }
}

// Epilogue: per wave, passes of EP_RP rows x WN columns through a private
// LDS region; a lane then moves 4 consecutive values of a row.  STEP: the
// cluster step leaf (C += alpha*acc), else C = alpha*acc + beta*C (C not read
// when beta == 0).
template <class T, bool STEP>
__device__ __forceinline__ void epilogue(const phx_f16v (&acc)[T::MI][T::NJ], float *ep_all,
                                         float *C, int64_t ldc, int64_t M, int64_t N, uint32_t m0,
                                         uint32_t n0, uint32_t wm, uint32_t wn, float alpha,
                                         float beta, uint32_t wave, uint32_t lane) {
    const uint32_t lrow = lane & 31, lgrp = lane >> 5;
    float *ep = ep_all + wave * (EP_RP * T::EP_PITCH);
#pragma unroll
    for (int pass = 0; pass < T::WM / EP_RP; ++pass) {
        const int i = (pass * EP_RP) / 32;
        const int r0 = ((pass * EP_RP) % 32) / 2;
#pragma unroll
        for (int j = 0; j < T::NJ; ++j)
#pragma unroll
            for (int r = r0; r < r0 + EP_RP / 2; ++r)
                ep[(8 * (r >> 2) + 4 * lgrp + (r & 3) - 2 * r0) * T::EP_PITCH + 32 * j + lrow] =
                    alpha * acc[i][j][r];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int rr = 0; rr < EP_RP / T::EP_RPI; ++rr) {
            const uint32_t row = rr * T::EP_RPI + lane / T::EP_LPR;
            const uint32_t c4 = (lane % T::EP_LPR) * 4;
            const int64_t grow = (int64_t)m0 + wm + pass * EP_RP + row;
            const int64_t gcol = (int64_t)n0 + wn + c4;
            if (grow < M && gcol < N) {
                const phx_f4 v = *(const phx_f4 *)(ep + row * T::EP_PITCH + c4);
                float *dst = C + grow * ldc + gcol;
                phx_f4 o = v;
                if (STEP) {
                    o = v + *(const phx_f4 *)dst;
                } else if (beta != 0.0f) {
                    const phx_f4 c = *(const phx_f4 *)dst;
                    o = v + beta * c;
                }
                *(phx_f4 *)dst = o;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// Tiles t0, t0 + tstride, ... of C (the regular entries walk them with the
// linear block id over the whole grid; the split-K entry with blockIdx.x).
template <class T, bool STEP>
__device__ __forceinline__ void gemm_s_body(const float *A, int64_t lda, const float *B,
                                            int64_t ldb, float *C, int64_t ldc, int64_t M,
                                            int64_t N, int64_t K, float alpha, float beta,
                                            char *stg, uint32_t t0, uint32_t tstride) {
    char *const S[NSTG] = {stg, stg + T::STAGE, stg + 2 * T::STAGE};
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = (wave >> 1) * T::WM;
    const uint32_t wn = (wave & 1) * T::WN;
    const uint32_t tiles_n = (uint32_t)((N + T::TN - 1) / T::TN);
    const uint32_t tiles_m = (uint32_t)((M + T::TM - 1) / T::TM);
    const uint32_t ntiles = tiles_m * tiles_n;
    const uint32_t nblk = tstride;
    const uint32_t nk = (uint32_t)((K + T::TK - 1) / T::TK);

    for (uint32_t t = t0; t < ntiles; t += nblk) {
        const uint32_t ts = nblk == ntiles ? phx_xcd_swizzle(t, ntiles) : t;
        const uint32_t gsz = GROUP_M * tiles_n;
        const uint32_t g0 = (ts / gsz) * GROUP_M;
        const uint32_t gm = (tiles_m - g0) < GROUP_M ? (tiles_m - g0) : GROUP_M;
        const uint32_t tm = g0 + (ts % gsz) % gm;
        const uint32_t tn = (ts % gsz) / gm;
        const uint32_t m0 = tm * T::TM, n0 = tn * T::TN;

        phx_f16v acc[T::MI][T::NJ];
#pragma unroll
        for (int i = 0; i < T::MI; ++i)
#pragma unroll
            for (int j = 0; j < T::NJ; ++j)
                acc[i][j] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        Frags<T> F0, F1;
#pragma unroll
        for (int p = 0; p < NSTG; ++p)
            dma_step<T>(S[p], A, lda, B, ldb, M, N, K, m0, n0, p * T::TK, wave, lane);
        PHX_WAIT_VMCNT((NSTG - 1) * T::DMA);
        __builtin_amdgcn_s_barrier();
        read_frags<T>(F0, S[0], 0, wm, wn, lane);
        uint32_t kt = 0;
        for (; kt + NSTG <= nk; kt += NSTG) {
#pragma unroll
            for (int u = 0; u < NSTG; ++u)
                k_step<T>(acc, F0, F1, S[u], S[(u + 1) % NSTG], A, lda, B, ldb, M, N, K, m0, n0,
                          kt + u, wm, wn, wave, lane);
        }
#pragma unroll
        for (int u = 0; u < NSTG - 1; ++u)
            if (kt + u < nk)
                k_step<T>(acc, F0, F1, S[u], S[(u + 1) % NSTG], A, lda, B, ldb, M, N, K, m0, n0,
                          kt + u, wm, wn, wave, lane);
        PHX_WAIT_VMCNT(0);
        __syncthreads();
        epilogue<T, STEP>(acc, (float *)stg, C, ldc, M, N, m0, n0, wm, wn, alpha, beta, wave,
                          lane);
        __syncthreads();
    }
}

typedef Tile<PHX_S_TILE, PHX_S_TILE, PHX_S_BK> Base;  // 256 x 256 x 16

#define GEMM_S_PRELUDE(T)                                                                     \
    __shared__ __attribute__((aligned(16))) char stg[NSTG * T::STAGE];                        \
    const int64_t M = a_s0, K = a_s1, N = b_s1;                                               \
    if (blockDim.x != NT || N % PHX_S_NK_MULT || K % PHX_S_NK_MULT || M <= 0 || N <= 0 ||  \
        K <= 0 || b_s0 != K || c_s0 != M || c_s1 != N || a_st1 != 1 || b_st1 != 1 ||         \
        c_st1 != 1 || (a_st0 | b_st0 | c_st0) % 4 ||                                         \
        ((uintptr_t)(a_ptr + a_off) | (uintptr_t)(b_ptr + b_off) | (uintptr_t)(c_ptr + c_off)) & 15) \
        return;

#ifdef PHX_GEMM_FP32
extern "C" __global__ __launch_bounds__(NT, 1) void gemm(PHX_MEMREF2(float, a, int32_t),
                                                          PHX_MEMREF2(float, b, int32_t),
                                                          PHX_MEMREF2(float, c, int32_t),
                                                          float alpha, float beta) {
    GEMM_S_PRELUDE(Base)
    gemm_s_body<Base, false>(a_ptr + a_off, a_st0, b_ptr + b_off, b_st0, c_ptr + c_off, c_st0, M,
                             N, K, alpha, beta, stg, phx_block_linear(), phx_block_count());
}

// The other tilings of the gemm_fp32 launch plan (phx_plan variant 1 ..):
// entry gemm_t<TM>x<TN>k<TK>, the same parameters and arithmetic as "gemm"
// over TM x TN tiles and K steps of TK.  Each output is the same f32 sum of
// exact products in a different order only where TK differs (the k-groups
// of 8 are summed in order in every tiling).
// workgroups per CU a tiling's registers allow (Tile::OCC, without the
// commas a template argument list would put into __launch_bounds__)
#define GEMM_S_OCC(AREA) ((AREA) <= 128 * 256 ? 2 : 1)
#define GEMM_S_VARIANT(VM, VN, VK)                                                            \
    extern "C" __global__ __launch_bounds__(NT, GEMM_S_OCC(VM * VN)) void                    \
        gemm_t##VM##x##VN##k##VK(PHX_MEMREF2(float, a, int32_t), PHX_MEMREF2(float, b, int32_t), \
                                 PHX_MEMREF2(float, c, int32_t), float alpha, float beta) {   \
        typedef Tile<VM, VN, VK> T;                                                           \
        static_assert(T::OCC == GEMM_S_OCC(VM * VN), "occupancy");                            \
        GEMM_S_PRELUDE(T)                                                                     \
        gemm_s_body<T, false>(a_ptr + a_off, a_st0, b_ptr + b_off, b_st0, c_ptr + c_off,      \
                              c_st0, M, N, K, alpha, beta, stg, phx_block_linear(),           \
                              phx_block_count());                                             \
    }
GEMM_S_VARIANT(256, 128, 16)
GEMM_S_VARIANT(128, 256, 16)
GEMM_S_VARIANT(128, 128, 16)
GEMM_S_VARIANT(128, 128, 32)
GEMM_S_VARIANT(128, 128, 8)
GEMM_S_VARIANT(256, 256, 8)
GEMM_S_VARIANT(64, 64, 16)

// Split-K for shapes with too few output tiles to fill the GPU (the host
// picks the split; see phx_runtime.cpp).  Workgroup (x, y) computes tiles
// x, x + gridDim.x, ... over the K columns [y * kchunk, min(K, (y+1) * kchunk))
// and stores the raw f32 sums to W + y * M * N (row-major, row pitch N): the
// tile kernel on the sub-matrices A[:, k0:k1] and B[k0:k1, :] with alpha 1
// and beta 0.  gemm_splitk_reduce then applies the epilogue.
extern "C" __global__ __launch_bounds__(NT, 1) void gemm_splitk(const float *A, const float *B,
                                                                 float *W, int64_t lda,
                                                                 int64_t ldb, int64_t M,
                                                                 int64_t N, int64_t K,
                                                                 int64_t kchunk) {
    __shared__ __attribute__((aligned(16))) char stg[NSTG * Base::STAGE];
    const int64_t k0 = (int64_t)blockIdx.y * kchunk;
    if (blockDim.x != NT || k0 >= K || kchunk % Base::TK) return;
    const int64_t kc = K - k0 < kchunk ? K - k0 : kchunk;
    gemm_s_body<Base, false>(A + k0, lda, B + k0 * ldb, ldb, W + (int64_t)blockIdx.y * M * N, N,
                             M, N, kc, 1.0f, 0.0f, stg, blockIdx.x, gridDim.x);
}

extern "C" __global__ __launch_bounds__(256) void gemm_splitk_reduce(const float *W, int32_t S,
                                                                      float *C, int64_t ldc,
                                                                      int64_t M, int64_t N,
                                                                      float alpha, float beta) {
    phx_splitk_reduce(W, S, C, ldc, M, N, alpha, beta);
}
#endif

#ifdef PHX_MATMUL_CLUSTER
extern "C" __global__ __launch_bounds__(NT, 1) void matmul(PHX_MEMREF2(float, a, int32_t),
                                                            PHX_MEMREF2(float, b, int32_t),
                                                            PHX_MEMREF2(float, c, int32_t),
                                                            float alpha, float beta) {
    GEMM_S_PRELUDE(Base)
    gemm_s_body<Base, true>(a_ptr + a_off, a_st0, b_ptr + b_off, b_st0, c_ptr + c_off, c_st0, M,
                            N, K, alpha, beta, stg, phx_block_linear(), phx_block_count());
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
