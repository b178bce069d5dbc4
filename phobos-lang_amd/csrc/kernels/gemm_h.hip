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
//   * 256x256 output tile per workgroup, one workgroup per CU (at 4096^2: 256
//     tiles, one wave of workgroups).  4 waves in a 2x2 arrangement, each
//     owning 128x128 = 4x4 v_mfma_f32_32x32x16_f16 tiles whose 256 f32
//     accumulators live in AGPRs.  Per K slice of 16 a wave reads 8 KiB of
//     operands from LDS for 16 MFMAs, half the LDS traffic per flop of a
//     128x64 wave tile.
//   * K step 32.  A is staged As[m][k] (64-byte rows); an MFMA A operand (8
//     consecutive k of one row) is one ds_read_b128.  B stays row-major
//     Bs[k][n] (512-byte rows) and its operand is read with gfx950's
//     transposing ds_read_b64_tr_b16: in a 16-lane group, lane s supplies 4
//     halves of row k0 + s/4 at column n0 + 4*(s%4), and lane i receives
//     B[k0..k0+3][n0+i].  Two such reads give a lane its 8 consecutive k.
//     Staging is therefore a plain 16-byte copy for both operands.
//   * gfx950's LDS serves 64 banks (256 bytes) per clock.  The 16-byte chunk
//     index is XOR-swizzled so every 16-lane (b128) or 32-lane (b64) group
//     hits distinct banks: As chunk ^ ((row >> 2) & 3), Bs chunk ^ 4*(row % 4).
//   * Software pipeline, one barrier per K step: the MFMAs of slice 0 run
//     while the slice-1 operands are read; then each wave waits for its own
//     copies of the next step and for its reads, and passes the barrier; the
//     MFMAs of slice 1 run while the next step's slice-0 operands are read.
//     gemm_fp16 copies global -> LDS directly into a 4-stage ring, step k+3
//     into the stage of step k-1 (free once step k-1's barrier has passed),
//     A's copies during the first half and B's during the second (1.5%
//     faster than a 3-stage ring with all copies in the second half).
//     Fences (sched_barrier / sched_group_barrier) fix the interleave, so the
//     single wave per SIMD keeps its matrix pipe fed.
//   * gemm_fp16tc: f32 operands are loaded into registers two steps ahead
//     and converted into a 3-stage LDS ring; the f16 data of step k+2 goes
//     into the stage of step k-1, which is free once step k-1's barrier has
//     passed, so A's conversions and loads ride with the first half's MFMAs
//     and B's with the second half's (6% faster than a 2-stage ring that put
//     them all in the second half).
//   * Workgroups are renumbered XCD-major and grouped 4 tile-rows deep, so the
//     32 workgroups of one XCD cover a 4x8 block of tiles and share A/B
//     panels in that XCD's L2.
//   * Ragged shapes (M any; N a multiple of one 16-byte chunk, 4 f32 or 8
//     f16 elements; K a multiple of 8, the k extent of a lane's chunk, so
//     the partial last K step masks whole chunks): each step's buffer resources end at the last row and
//     column that exist, so rows of A past M and rows of B past K read zeros
//     (the range check covers the scalar offset too); A chunks past K in the
//     last, partial K step take an out-of-range lane offset and read zeros;
//     stores are masked to M x N.  B columns past N in a row are read but
//     only reach output columns that are not stored.
#include "phx_common.h"

#ifdef PHX_GEMM_TC
typedef float TIn;
typedef float TOut;
#else
typedef _Float16 TIn;
typedef _Float16 TOut;
#endif

#define BM PHX_H_BM  // 256
#define BN PHX_H_BN  // 256
#define BK PHX_H_BK  // 32
#define NT PHX_H_THREADS
#define WM 128
#define WN 128
#define GROUP_M 4   // tile rows per swizzle group

#define A_ROW_BYTES (BK * 2)             // 64
#define B_ROW_BYTES (BN * 2)             // 512
#define A_BYTES (BM * A_ROW_BYTES)       // 16 KiB
#define B_BYTES (BK * B_ROW_BYTES)       // 16 KiB
#define STAGE_BYTES (A_BYTES + B_BYTES)  // 32 KiB
#define EP_RP 8                         // epilogue rows per pass
#define EP_PITCH 136                     // epilogue LDS row pitch (floats)

typedef __fp16 phx_fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) phx_fp16x4 *phx_lds_h4p;
typedef __attribute__((address_space(3))) void *phx_lds_vp;

// s_waitcnt fields: vmcnt [3:0]+[15:14], expcnt [6:4], lgkmcnt [11:8]
#define PHX_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))
#define PHX_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (((n) >> 4) << 14))
#define SGB(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
#define G_MFMA 0x008
#define G_VALU 0x002
#define G_VMEM 0x020
#define G_DSR 0x100
#define G_DSW 0x200

__device__ __forceinline__ uint32_t a_off(uint32_t row, uint32_t chunk) {
    return row * A_ROW_BYTES + ((chunk ^ ((row >> 2) & 3)) << 4);
}
__device__ __forceinline__ uint32_t b_off(uint32_t row, uint32_t chunk) {
    return row * B_ROW_BYTES + ((chunk ^ ((row & 3) << 2)) << 4);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t phx_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

struct Frags {
    phx_h8 a[4];
    phx_h8 b[4];
};

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
    for (int j = 0; j < 4; ++j) {
        const uint32_t col = wn + j * 32 + 16 * (q & 1) + 4 * (sl & 3);
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

__device__ __forceinline__ void mfma_all(phx_f16v (&acc)[4][4], const Frags &f) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// Epilogue: per wave, 8 passes of 16 rows x 128 columns through a private
// LDS region; a lane then moves 4 consecutive values of a row.  C is written
// (and, for beta != 0, read) through a buffer resource over the tile's rows
// that exist, so stores to rows past M fall out of range and are dropped; a
// lane whose 4 columns lie past N gets an out-of-range column offset, fixed
// for the tile.  No per-store test: an explicit bounds check on every store
// cost gemm_fp16 5% through its branches and exec-mask updates.  R (ragged)
// false: the tile lies inside C and stores go through plain pointers.
template <bool R, typename TO>
__device__ __forceinline__ void epilogue(const phx_f16v (&acc)[4][4], float *ep_all, TO *C,
                                         int64_t ldc, int64_t M, int64_t N, uint32_t m0,
                                         uint32_t n0, uint32_t wm, uint32_t wn, float alpha,
                                         float beta, uint32_t wave, uint32_t lane) {
    const uint32_t lrow = lane & 31, lgrp = lane >> 5;
    float *ep = ep_all + wave * (EP_RP * EP_PITCH);
    const uint32_t ml = (uint32_t)M - m0;
    const uint32_t rows = ml < BM ? ml : BM;  // rows of the tile that exist
    const __amdgpu_buffer_rsrc_t rc =
        phx_rsrc(C + (int64_t)m0 * ldc, rows * (uint32_t)ldc * (uint32_t)sizeof(TO));
    // lane part of the offset (row wm + lane/32, its 4 columns); a store adds
    // the uniform row step in the scalar offset.  The empty asm keeps the
    // compiler from hoisting per-store offsets out of the tile loop, where
    // they would stay live (and spill) across the K loop.
    const uint32_t pitch = (uint32_t)ldc * (uint32_t)sizeof(TO);
    const uint32_t col = n0 + wn + (lane & 31) * 4;
    uint32_t voff = (wm + (lane >> 5)) * pitch +
                    (col < (uint32_t)N ? col * (uint32_t)sizeof(TO) : 0x80000000u);
    asm volatile("" : "+v"(voff));
#pragma unroll
    for (int pass = 0; pass < WM / EP_RP; ++pass) {
        const int i = (pass * EP_RP) / 32;
        const int r0 = ((pass * EP_RP) % 32) / 2;  // first accumulator register of this pass
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = r0; r < r0 + EP_RP / 2; ++r)
                ep[(8 * (r >> 2) + 4 * lgrp + (r & 3) - 2 * r0) * EP_PITCH + 32 * j + lrow] =
                    alpha * acc[i][j][r];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int rr = 0; rr < EP_RP / 2; ++rr) {
            const uint32_t row = rr * 2 + (lane >> 5), c4 = (lane & 31) * 4;
            const phx_f4 v = *(const phx_f4 *)(ep + row * EP_PITCH + c4);
            // row of the tile * pitch + column: < 2^31 in range (the host
            // limits 257 rows of C to 2 GiB); + 2^31 when the column is past N
            const int so = (int)((pass * EP_RP + rr * 2) * pitch);
            TO *dst = C + (int64_t)(m0 + wm + pass * EP_RP + row) * ldc + n0 + wn + c4;
            if constexpr (sizeof(TO) == 4) {  // f32 output
            phx_f4 o = v;
            if (beta != 0.0f) {
                const phx_f4 c = R ? __builtin_bit_cast(phx_f4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                    rc, (int)voff, so, 0))
                                   : *(const phx_f4 *)dst;
                o = v + beta * c;
            }
            if (R)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(phx_u4, o), rc, (int)voff, so, 0);
            else
                *(phx_f4 *)dst = o;
            } else {  // f16 output
            float o[4] = {v.x, v.y, v.z, v.w};
            if (beta != 0.0f) {
                const phx_h4 c = R ? __builtin_bit_cast(phx_h4, __builtin_amdgcn_raw_buffer_load_b64(
                                                                    rc, (int)voff, so, 0))
                                   : *(const phx_h4 *)dst;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float cb = beta * (float)c[e];
                    o[e] = o[e] + cb;
                }
            }
            phx_h4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = (_Float16)o[e];
            if (R)
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(phx_u2, h), rc, (int)voff, so, 0);
            else
                *(phx_h4 *)dst = h;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

#ifdef PHX_GEMM_TC
// ------------------------------------------------------------------ tc path
// f32 inputs are staged through registers and rounded to f16 (RNE) on the
// way into LDS.  Thread t stages f16 chunks c = i*256 + t (i < 4) of A (row
// c/4, chunk c%4) and of B (row c/32, chunk c%32); each chunk is two 16-byte
// f32 loads.  Step t lives in LDS stage t % 3 and, while in flight, in
// register set t % 2.
#define ESZ 4u
struct Chunk { phx_f4 lo, hi; };
__device__ __forceinline__ Chunk load_chunk(__amdgpu_buffer_rsrc_t r, uint32_t vo, int so) {
    Chunk c;
    c.lo = __builtin_bit_cast(phx_f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, so, 0));
    c.hi = __builtin_bit_cast(phx_f4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo + 16, so, 0));
    return c;
}
__device__ __forceinline__ phx_u4 pack(const Chunk &c) {
    phx_u4 v;
    v.x = phx_pack_h2(c.lo.x, c.lo.y);
    v.y = phx_pack_h2(c.lo.z, c.lo.w);
    v.z = phx_pack_h2(c.hi.x, c.hi.y);
    v.w = phx_pack_h2(c.hi.z, c.hi.w);
    return v;
}
struct Regs {
    Chunk a[4];
    Chunk b[4];
};

#endif

// Buffer resources of one K step: A rows m0 .. min(M, m0 + BM) - 1 and B
// columns n0 .. min(N, n0 + BN) - 1, K columns / rows k0 .. min(K, k0 + BK) - 1;
// steps past K get an empty resource (every access reads zero).
// (32-bit arithmetic: the host limits the extents so that 256 rows of either
// operand span less than 2 GiB.  The clamps are unsigned mins behind an
// in-range test: a signed clamp becomes v_med3_i32, which moves these
// wave-uniform values, and the resources built from them, into VGPRs.)
template <bool R>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t a_rsrc(const TIn *A, uint32_t lda, uint32_t M,
                                                         uint32_t K, uint32_t m0, uint32_t k0) {
    if (!R) {  // whole tiles: BM rows x BK columns, or nothing past K
        const bool in = k0 < K;
        return phx_rsrc(A + (int64_t)m0 * lda + (in ? k0 : 0),
                        in ? ((BM - 1) * lda + BK) * (uint32_t)sizeof(TIn) : 0u);
    }
    const uint32_t kl = K - k0, ml = M - m0;
    const uint32_t kw = kl < BK ? kl : BK, mr = ml < BM ? ml : BM;
    // a resource past K has no records; its base is then never dereferenced
    const uint32_t in = 0u - (uint32_t)(k0 < K);  // all ones in range: no branch
    return phx_rsrc(A + (int64_t)m0 * lda + k0, ((mr - 1) * lda + kw) * (uint32_t)sizeof(TIn) & in);
}
template <bool R>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t b_rsrc(const TIn *B, uint32_t ldb, uint32_t N,
                                                         uint32_t K, uint32_t n0, uint32_t k0) {
    if (!R) {
        const bool in = k0 < K;
        return phx_rsrc(B + (int64_t)(in ? k0 : 0) * ldb + n0,
                        in ? ((BK - 1) * ldb + BN) * (uint32_t)sizeof(TIn) : 0u);
    }
    const uint32_t kl = K - k0, nl = N - n0;
    const uint32_t kw = kl < BK ? kl : BK, nc = nl < BN ? nl : BN;
    const uint32_t in = 0u - (uint32_t)(k0 < K);
    return phx_rsrc(B + (int64_t)k0 * ldb + n0, ((kw - 1) * ldb + nc) * (uint32_t)sizeof(TIn) & in);
}
// A lane's A offset in step k0: its full-step offset vo, or in the last,
// partial step (K % BK columns left) vo_tail, which is out of range (reads
// zero) for the lanes whose chunk lies past K.  vo_tail is fixed per kernel.
template <bool R>
__device__ __forceinline__ uint32_t a_lane_off(uint32_t vo, uint32_t vo_tail, uint32_t K,
                                               uint32_t k0) {
    return !R || k0 + BK <= K ? vo : vo_tail;
}
__device__ __forceinline__ uint32_t a_tail_off(uint32_t vo, uint32_t kc, uint32_t K) {
    const uint32_t kwl = K % BK;
    return kwl == 0 || kc < kwl ? vo : 0x80000000u;
}

#ifdef PHX_GEMM_TC

template <bool RG>
__device__ __forceinline__ void load_regs(Regs &R, const TIn *A, int64_t lda, const TIn *B,
                                          int64_t ldb, int64_t M, int64_t N, int64_t K,
                                          uint32_t m0, uint32_t n0, uint32_t k0, uint32_t voa,
                                          uint32_t voa_t, uint32_t vob) {
    const __amdgpu_buffer_rsrc_t ra = a_rsrc<RG>(A, lda, M, K, m0, k0);
    const __amdgpu_buffer_rsrc_t rb = b_rsrc<RG>(B, ldb, N, K, n0, k0);
    const uint32_t va = a_lane_off<RG>(voa, voa_t, K, k0);
#pragma unroll
    for (int i = 0; i < 4; ++i) R.a[i] = load_chunk(ra, va, (int)((uint32_t)(i * 64 * lda) * ESZ));
#pragma unroll
    for (int i = 0; i < 4; ++i) R.b[i] = load_chunk(rb, vob, (int)((uint32_t)(i * 8 * ldb) * ESZ));
}

__device__ __forceinline__ void store_regs(const Regs &R, char *stage, uint32_t tid) {
    char *As = stage, *Bs = stage + A_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i) *(phx_u4 *)(As + a_off(i * 64 + (tid >> 2), tid & 3)) = pack(R.a[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) *(phx_u4 *)(Bs + b_off(i * 8 + (tid >> 5), tid & 31)) = pack(R.b[i]);
}

__device__ __forceinline__ void mfma_one(phx_f16v (&acc)[4][4], const Frags &f, int m) {
    acc[m >> 2][m & 3] =
        __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[m >> 2], f.b[m & 3], acc[m >> 2][m & 3], 0, 0, 0);
}

__device__ __forceinline__ void read_a(Frags &f, const char *stage, uint32_t s, uint32_t wm,
                                       uint32_t lane, int i) {
    f.a[i] = *(const phx_h8 *)(stage + a_off(wm + i * 32 + (lane & 31), 2 * s + (lane >> 5)));
}

__device__ __forceinline__ void read_b(Frags &f, const char *stage, uint32_t s, uint32_t wn,
                                       uint32_t lane, int j) {
    const char *Bs = stage + A_BYTES;
    const uint32_t q = lane >> 4, sl = lane & 15;
    const uint32_t col = wn + j * 32 + 16 * (q & 1) + 4 * (sl & 3);
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


// Slot plan of a tc3 half: which of the 16 MFMA slots carries operand read
// r (0-3: A fragments, 4-7: B fragments) and which carries chunk c (0-3:
// convert, store and reload).  Returns 0 for nothing, 1 + r for a read,
// 9 + c for a chunk.  The chunks sit on every fourth slot with reads in
// between (1% faster than reads first and the chunks in one run after them).
__device__ constexpr int tc_slot(int m) {
    return (m % 4 == 2) ? 9 + m / 4 : (m < 11 ? 1 + (m - (m > 2) - (m > 6) - (m > 10)) : 0);
}

// Three-stage form: the f16 data of step kt+2 goes into the stage step kt-1
// used, which every wave has finished reading once step kt-1's barrier has
// passed, so it can be written during both halves of step kt.  Each half
// then carries half of the loads and conversions next to its 16 MFMAs
// (A's in the first, B's in the second) instead of all of them landing in
// the second half, where the queued loads stalled the in-order MFMA issue.
template <bool RG>
__device__ __forceinline__ void tc3_step(phx_f16v (&acc)[4][4], Frags &F0, Frags &F1,
                                         const char *cur, const char *nxt, char *fill, Regs &R,
                                         const TIn *A, int64_t lda, const TIn *B, int64_t ldb,
                                         int64_t M, int64_t N, int64_t K, uint32_t m0, uint32_t n0,
                                         uint32_t kt, uint32_t voa, uint32_t voa_t, uint32_t vob,
                                         uint32_t wm, uint32_t wn, uint32_t tid, uint32_t lane) {
    const uint32_t k4 = (kt + 4) * BK;
    char *As = fill, *Bs = fill + A_BYTES;
    {
        const __amdgpu_buffer_rsrc_t ra = a_rsrc<RG>(A, lda, M, K, m0, k4);
        const uint32_t va = a_lane_off<RG>(voa, voa_t, K, k4);
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            mfma_one(acc, F0, m);
            const int sl = tc_slot(m);
            if (sl >= 1 && sl <= 4) {
                read_a(F1, cur, 1, wm, lane, sl - 1);
            } else if (sl >= 5 && sl <= 8) {
                read_b(F1, cur, 1, wn, lane, sl - 5);
            } else if (sl >= 9) {
                const int i = sl - 9;
                *(phx_u4 *)(As + a_off(i * 64 + (tid >> 2), tid & 3)) = pack(R.a[i]);
                R.a[i] = load_chunk(ra, va, (int)((uint32_t)(i * 64 * lda) * ESZ));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    PHX_WAIT_VM_LGKM0(63);  // reads of cur and this wave's LDS writes done
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    {
        const __amdgpu_buffer_rsrc_t rb = b_rsrc<RG>(B, ldb, N, K, n0, k4);
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            mfma_one(acc, F1, m);
            const int sl = tc_slot(m);
            if (sl >= 1 && sl <= 4) {
                read_a(F0, nxt, 0, wm, lane, sl - 1);
            } else if (sl >= 5 && sl <= 8) {
                read_b(F0, nxt, 0, wn, lane, sl - 5);
            } else if (sl >= 9) {
                const int i = sl - 9;
                *(phx_u4 *)(Bs + b_off(i * 8 + (tid >> 5), tid & 31)) = pack(R.b[i]);
                R.b[i] = load_chunk(rb, vob, (int)((uint32_t)(i * 8 * ldb) * ESZ));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}
#else
// ------------------------------------------------------------------ f16 path
// f16 inputs go global -> LDS directly (buffer_load ... lds: lane l of a
// 64-lane copy writes LDS bytes base + 16l .. +15 from its own global
// address, so the XOR-swizzled layouts are built by choosing each lane's
// source) into a ring of 4 stages, each its own LDS array so the compiler's
// LDS-DMA tracking tells them apart.  Step t+3 is copied into the stage step
// t-1 used, once every wave is past the barrier that ends its reads.  Copies
// of K steps past the end read through an empty buffer resource (zeros) into
// stages nobody reads, which keeps every wait count constant.
#define NSTG 4
#define DMA_PER_STEP 8  // copies per wave per K step (4 A + 4 B)

// PARTS: 1 = A's copies, 2 = B's, 3 = both
template <bool RG, int PARTS = 3>
__device__ __forceinline__ void dma_step(char *dst, const TIn *A, int64_t lda, const TIn *B,
                                         int64_t ldb, int64_t M, int64_t N, int64_t K, uint32_t m0,
                                         uint32_t n0, uint32_t k0, uint32_t voa, uint32_t voa_t,
                                         uint32_t vob0, uint32_t vob1, uint32_t wave) {
    const __amdgpu_buffer_rsrc_t ra = a_rsrc<RG>(A, lda, M, K, m0, k0);
    const __amdgpu_buffer_rsrc_t rb = b_rsrc<RG>(B, ldb, N, K, n0, k0);
    const uint32_t va = a_lane_off<RG>(voa, voa_t, K, k0);
#pragma unroll
    for (int i = 0; i < 4; ++i)  // A chunks wave*256 + i*64 + lane: row wave*64 + i*16 + lane/4
        if (PARTS & 1)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (phx_lds_vp)(dst + (wave * 256 + i * 64) * 16), 16, va,
                (int)((uint32_t)((wave * 64 + i * 16) * lda) * 2), 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i)  // B chunks wave*256 + i*64 + lane: row wave*8 + 2i + lane/32
        if (PARTS & 2)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (phx_lds_vp)(dst + A_BYTES + (wave * 256 + i * 64) * 16), 16,
                (i & 1) ? vob1 : vob0, (int)((uint32_t)((wave * 8 + i * 2) * ldb) * 2), 0, 0);
}

// Four-stage form: the copies of step kt+3 go into the stage of step kt-1,
// which is free once step kt-1's barrier has passed, so A's copies ride with
// the first half's MFMAs and B's with the second half's.
template <bool RG>
__device__ __forceinline__ void dma4_k_step(phx_f16v (&acc)[4][4], Frags &F0, Frags &F1,
                                            const char *cur, const char *nxt, char *fill,
                                            const TIn *A, int64_t lda, const TIn *B, int64_t ldb,
                                            int64_t M, int64_t N, int64_t K, uint32_t m0,
                                            uint32_t n0, uint32_t kt,
                                            uint32_t voa, uint32_t voa_t, uint32_t vob0, uint32_t vob1,
                                            uint32_t wm, uint32_t wn, uint32_t wave,
                                            uint32_t lane) {
    read_frags(F1, cur, 1, wm, wn, lane);
    dma_step<RG, 1>(fill, A, lda, B, ldb, M, N, K, m0, n0, (kt + 3) * BK, voa, voa_t, vob0, vob1, wave);
    mfma_all(acc, F0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        SGB(G_MFMA, 1);
        if (i < 12) SGB(G_DSR, 1);
        if ((i & 3) == 1) SGB(G_VMEM, 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    // own copies of step kt+1 landed: step kt+2 (8) and kt+3's A part (4) may be in flight
    PHX_WAIT_VM_LGKM0(DMA_PER_STEP + DMA_PER_STEP / 2);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(F0, nxt, 0, wm, wn, lane);
    dma_step<RG, 2>(fill, A, lda, B, ldb, M, N, K, m0, n0, (kt + 3) * BK, voa, voa_t, vob0, vob1, wave);
    mfma_all(acc, F1);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        SGB(G_MFMA, 1);
        if (i < 12) SGB(G_DSR, 1);
        if ((i & 3) == 1) SGB(G_VMEM, 1);
    }
    __builtin_amdgcn_sched_barrier(0);
}
#endif

// The kernel body.  RG (ragged): M, N or K is not a whole number of tiles,
// so operand resources end at the matrix edges, A chunks past K in the last
// step read zero and C is stored through a bounded resource; whole-tile
// shapes run the instance without any of that (the masks cost gemm_fp16tc
// 2% when always on).
// Tiles t0, t0 + tstride, ... of C (the regular entry walks them with the
// linear block id over the whole grid; the split-K entry with blockIdx.x).
template <bool RG, typename TO>
__device__ __forceinline__ void gemm_body(const TIn *A, const TIn *B, TO *C, int64_t lda,
                                          int64_t ldb, int64_t ldc, int64_t M, int64_t N,
                                          int64_t K, float alpha, float beta, uint32_t t0,
                                          uint32_t tstride,
#ifdef PHX_GEMM_TC
                                          char *stg
#else
                                          char *stg0, char *stg1, char *stg2, char *stg3
#endif
) {
#ifdef PHX_GEMM_TC
    char *const stg0 = stg;  // the epilogue's staging area
#else
    char *const S[NSTG] = {stg0, stg1, stg2, stg3};
#endif

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = (wave >> 1) * WM;
    const uint32_t wn = (wave & 1) * WN;
    const uint32_t tiles_n = (uint32_t)((N + BN - 1) / BN);
    const uint32_t tiles_m = (uint32_t)((M + BM - 1) / BM);
    const uint32_t ntiles = tiles_m * tiles_n;
    const uint32_t nblk = tstride;
    const uint32_t nk = (uint32_t)((K + BK - 1) / BK);
#ifdef PHX_GEMM_TC
    const uint32_t voa = (uint32_t)(((tid >> 2) * lda + (tid & 3) * 8) * ESZ);
    const uint32_t voa_t = a_tail_off(voa, (tid & 3) * 8, K);  // 8 k per chunk, K % 8 == 0
    const uint32_t vob = (uint32_t)(((tid >> 5) * ldb + (tid & 31) * 8) * ESZ);
#else
    const uint32_t voa =
        (uint32_t)(((lane >> 2) * lda + 8 * ((lane & 3) ^ ((lane >> 4) & 3))) * 2);
    const uint32_t voa_t = a_tail_off(voa, 8 * ((lane & 3) ^ ((lane >> 4) & 3)), K);
    // B row parity within the 4-row swizzle period: 2*(i&1) + lane/32
    const uint32_t vob0 =
        (uint32_t)(((lane >> 5) * ldb + 8 * ((lane & 31) ^ (4 * (lane >> 5)))) * 2);
    const uint32_t vob1 =
        (uint32_t)(((lane >> 5) * ldb + 8 * ((lane & 31) ^ (4 * (2 + (lane >> 5))))) * 2);
#endif

    for (uint32_t t = t0; t < ntiles; t += nblk) {
        const uint32_t ts = nblk == ntiles ? phx_xcd_swizzle(t, ntiles) : t;
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
        Frags F0, F1;

#ifdef PHX_GEMM_TC
        // prologue: steps 0 and 1 into LDS stages 0 and 1, steps 2 and 3 in
        // flight; step t lives in stage t % 3 and register set t % 2
        Regs R0, R1;
        load_regs<RG>(R0, A, lda, B, ldb, M, N, K, m0, n0, 0, voa, voa_t, vob);
        load_regs<RG>(R1, A, lda, B, ldb, M, N, K, m0, n0, BK, voa, voa_t, vob);
        store_regs(R0, stg, tid);
        store_regs(R1, stg + STAGE_BYTES, tid);
        load_regs<RG>(R0, A, lda, B, ldb, M, N, K, m0, n0, 2 * BK, voa, voa_t, vob);
        load_regs<RG>(R1, A, lda, B, ldb, M, N, K, m0, n0, 3 * BK, voa, voa_t, vob);
        PHX_WAIT_VM_LGKM0(63);
        __builtin_amdgcn_s_barrier();
        read_frags(F0, stg, 0, wm, wn, lane);
#define TC3(cur, nxt, fill, R, t)                                                               \
        tc3_step<RG>(acc, F0, F1, cur, nxt, fill, R, A, lda, B, ldb, M, N, K, m0, n0, t, voa, voa_t, vob, wm, wn, \
                 tid, lane)
        // stage bases rotate at run time (uniform values), so the LDS
        // addresses are one per-lane offset plus a scalar base instead of a
        // register set per stage
        uint32_t s0 = 0, s1 = STAGE_BYTES, s2 = 2 * STAGE_BYTES;
        uint32_t kt = 0;
        for (; kt + 2 <= nk; kt += 2) {
            TC3(stg + s0, stg + s1, stg + s2, R0, kt);
            TC3(stg + s1, stg + s2, stg + s0, R1, kt + 1);
            const uint32_t t = s0;  // advance by two stages
            s0 = s2;
            s2 = s1;
            s1 = t;
        }
        if (kt < nk) TC3(stg + s0, stg + s1, stg + s2, R0, kt);
#undef TC3
        PHX_WAIT_VMCNT(0);
        __syncthreads();
        epilogue<RG, TO>(acc, (float *)stg0, C, ldc, M, N, m0, n0, wm, wn, alpha, beta, wave, lane);
        __syncthreads();
#else
#pragma unroll
        for (int p = 0; p < 3; ++p)  // prologue: steps 0 .. 2 in flight
            dma_step<RG>(S[p], A, lda, B, ldb, M, N, K, m0, n0, p * BK, voa, voa_t, vob0, vob1, wave);
        PHX_WAIT_VMCNT(2 * DMA_PER_STEP);
        __builtin_amdgcn_s_barrier();
        read_frags(F0, stg0, 0, wm, wn, lane);
        uint32_t kt = 0;
        for (; kt + 4 <= nk; kt += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                dma4_k_step<RG>(acc, F0, F1, S[u], S[(u + 1) % 4], S[(u + 3) % 4], A, lda, B, ldb, M,
                            N, K, m0, n0, kt + u, voa, voa_t, vob0, vob1, wm, wn, wave, lane);
        }
#pragma unroll
        for (int u = 0; u < 3; ++u)
            if (kt + u < nk)
                dma4_k_step<RG>(acc, F0, F1, S[u], S[(u + 1) % 4], S[(u + 3) % 4], A, lda, B, ldb, M,
                            N, K, m0, n0, kt + u, voa, voa_t, vob0, vob1, wm, wn, wave, lane);
        PHX_WAIT_VMCNT(0);
        __syncthreads();
        epilogue<RG, TO>(acc, (float *)stg0, C, ldc, M, N, m0, n0, wm, wn, alpha, beta, wave, lane);
        __syncthreads();
#endif
    }
}

extern "C" __global__ __launch_bounds__(NT, 1) void gemm(PHX_MEMREF2(TIn, a, int64_t),
                                                          PHX_MEMREF2(TIn, b, int64_t),
                                                          PHX_MEMREF2(TOut, c, int64_t),
                                                          float alpha, float beta) {
#ifdef PHX_GEMM_TC
    __shared__ __attribute__((aligned(16))) char stg[3 * STAGE_BYTES];
#else
    __shared__ __attribute__((aligned(16))) char stg0[STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) char stg1[STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) char stg2[STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) char stg3[STAGE_BYTES];
#endif

    const int64_t M = a_s0, K = a_s1, N = b_s1;
#ifdef PHX_GEMM_TC
    constexpr int64_t NMULT = PHX_TC_N_MULT, KMULT = PHX_TC_K_MULT;
#else
    constexpr int64_t NMULT = PHX_H16_NK_MULT, KMULT = PHX_H16_NK_MULT;
#endif
    if (blockDim.x != NT || N % NMULT || K % KMULT || M <= 0 || N <= 0 || K <= 0 || b_s0 != K ||
        c_s0 != M || c_s1 != N || a_st1 != 1 || b_st1 != 1 || c_st1 != 1 ||
        a_st0 % KMULT || (b_st0 | c_st0) % NMULT || M > INT32_MAX ||
        (BM + 1) * (a_st0 > b_st0 ? a_st0 : b_st0) * (int64_t)sizeof(TIn) > INT32_MAX ||
        (BM + 1) * c_st0 * (int64_t)sizeof(TOut) > INT32_MAX ||
        ((uintptr_t)(a_ptr + a_off) | (uintptr_t)(b_ptr + b_off) | (uintptr_t)(c_ptr + c_off)) & 15)
        return;

    const TIn *A = a_ptr + a_off;
    const TIn *B = b_ptr + b_off;
    TOut *C = c_ptr + c_off;
    const int64_t lda = a_st0, ldb = b_st0, ldc = c_st0;
#ifdef PHX_GEMM_TC
#define GEMM_LDS stg
#else
#define GEMM_LDS stg0, stg1, stg2, stg3
#endif
    if (M % BM == 0 && N % BN == 0 && K % BK == 0)  // uniform
        gemm_body<false, TOut>(A, B, C, lda, ldb, ldc, M, N, K, alpha, beta, phx_block_linear(),
                               phx_block_count(), GEMM_LDS);
    else
        gemm_body<true, TOut>(A, B, C, lda, ldb, ldc, M, N, K, alpha, beta, phx_block_linear(),
                              phx_block_count(), GEMM_LDS);
}

// Split-K for shapes with too few output tiles to fill the GPU (the host
// picks the split; see phx_runtime.cpp).  Workgroup (x, y) computes tiles
// x, x + gridDim.x, ... over the K columns [y * kchunk, min(K, (y+1) * kchunk))
// and stores the raw f32 sums to W + y * M * N (row-major, row pitch N):
// the tile kernel run on the sub-matrices A[:, k0:k1] and B[k0:k1, :] with
// alpha 1 and beta 0, so C is not read.  kchunk is a multiple of BK, so each
// chunk starts 16-byte aligned; a chunk's partial last step is masked as the
// last step of any K is.  gemm_splitk_reduce then applies the epilogue.
extern "C" __global__ __launch_bounds__(NT, 1) void gemm_splitk(const TIn *A, const TIn *B,
                                                                 float *W, int64_t lda,
                                                                 int64_t ldb, int64_t M,
                                                                 int64_t N, int64_t K,
                                                                 int64_t kchunk) {
#ifdef PHX_GEMM_TC
    __shared__ __attribute__((aligned(16))) char stg[3 * STAGE_BYTES];
#else
    __shared__ __attribute__((aligned(16))) char stg0[STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) char stg1[STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) char stg2[STAGE_BYTES];
    __shared__ __attribute__((aligned(16))) char stg3[STAGE_BYTES];
#endif
    const int64_t k0 = (int64_t)blockIdx.y * kchunk;
    if (blockDim.x != NT || k0 >= K || kchunk % BK) return;
    const int64_t kc = K - k0 < kchunk ? K - k0 : kchunk;
    const TIn *As = A + k0;
    const TIn *Bs = B + k0 * ldb;
    float *Ws = W + (int64_t)blockIdx.y * M * N;
    if (M % BM == 0 && N % BN == 0 && kc % BK == 0)
        gemm_body<false, float>(As, Bs, Ws, lda, ldb, N, M, N, kc, 1.0f, 0.0f, blockIdx.x,
                                gridDim.x, GEMM_LDS);
    else
        gemm_body<true, float>(As, Bs, Ws, lda, ldb, N, M, N, kc, 1.0f, 0.0f, blockIdx.x,
                               gridDim.x, GEMM_LDS);
}
#undef GEMM_LDS

extern "C" __global__ __launch_bounds__(256) void gemm_splitk_reduce(const float *W, int32_t S,
                                                                      TOut *C, int64_t ldc,
                                                                      int64_t M, int64_t N,
                                                                      float alpha, float beta) {
    phx_splitk_reduce(W, S, C, ldc, M, N, alpha, beta);
}

#ifdef PHX_GEMM_TC
// ------------------------------------------------- eight-wave tc kernel
// gemm_w8 / gemm_w8_splitk: gemm_fp16tc_fp32acc with two waves per SIMD,
// at every shape the one-wave kernels take (ragged edges masked as there).  The one-wave-per-SIMD kernel above issues
// its f32 operand loads and its MFMAs from one instruction stream; when the
// CU's load path is saturated (64 KiB of f32 per K step, as many cycles as
// the step's MFMAs) a load that cannot issue holds up the MFMAs behind it,
// and the two run one after the other.  A microbenchmark on MI355X (one
// workgroup per CU, L2-resident data, the tc per-step load volume and MFMA
// count): 244 us with one wave per SIMD doing both, against 178 us with two
// waves per SIMD (either split into a loading and a computing wave, or both
// doing half of each), where MFMA-only runs 127 us and loads-only 160 us.
// So here 8 waves own 128 x 64 of the 256 x 256 tile each (4 x 2
// v_mfma_f32_32x32x16_f16 tiles, 128 f32 accumulators), every wave loads
// and converts its share of the operands, and a stalled load in one wave
// leaves the SIMD to the other wave's MFMAs.  Three LDS stages and one
// register set of f32 loads (248 VGPRs per wave); one barrier per step.
// Measured at 4096^3: 130-135 us against 139-142 us for the one-wave kernel
// (same box, alternating), bit-identical output.  Probe builds put the rest
// on the load path: without the MFMAs 105 us, without the loads 90 us.
#define W8_NT 512
// MFMA positions (of 8 per half step) of the A and B chunks, and of the
// first of the six operand reads for the other slice
#ifndef W8_A0
#define W8_A0 0
#define W8_A1 4
#define W8_B0 0
#define W8_B1 4
#endif
#ifndef W8_RD
#define W8_RD 1
#endif
#define W8_WM 128
#define W8_WN 64

struct Frags8 {
    phx_h8 a[4];
    phx_h8 b[2];
};

__device__ __forceinline__ void w8_mfma(phx_f16v (&acc)[4][2], const Frags8 &f, int m) {
    acc[m >> 1][m & 1] =
        __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[m >> 1], f.b[m & 1], acc[m >> 1][m & 1], 0, 0, 0);
}

// C = fl(fl(alpha*acc) + fl(beta*c)) over a wave's 128 x 64 block at (r0,
// c0), rounded once to the output type; C is not read when beta == 0.  Lane
// l holds column 32j + l%32 and rows 32i + 8(r/4) + 4(l/32) + r%4; a store
// writes two row segments of 32 elements.  RG: C is read and written
// through a buffer resource over the block's rows that exist, and a lane
// whose column lies past N gets an out-of-range column offset (as in the
// one-wave epilogue: no per-store test).
template <bool RG, typename TO>
__device__ __forceinline__ void w8_epilogue(const phx_f16v (&acc)[4][2], TO *C, int64_t ldc,
                                            int64_t M, int64_t N, uint32_t r0, uint32_t c0,
                                            float alpha, float beta, uint32_t lane) {
    static_assert(sizeof(TO) == 4, "gemm_w8 stores f32");
    const uint32_t lrow = 4 * (lane >> 5), lcol = lane & 31;
    if constexpr (RG) {
        if ((int64_t)r0 >= M) return;  // the whole block lies past M (uniform)
        const uint32_t ml = (uint32_t)(M - r0);
        const uint32_t rows = ml < W8_WM ? ml : W8_WM;
        const uint32_t pitch = (uint32_t)ldc * (uint32_t)sizeof(TO);
        const __amdgpu_buffer_rsrc_t rc = phx_rsrc(C + (int64_t)r0 * ldc, rows * pitch);
        uint32_t vo[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t col = c0 + 32 * j + lcol;
            vo[j] = lrow * pitch + (col < (uint32_t)N ? col * (uint32_t)sizeof(TO) : 0x80000000u);
        }
        asm volatile("" : "+v"(vo[0]), "+v"(vo[1]));  // not hoisted into the K loop
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    // row step of the block: < 128 rows, so < 2^31 with the column
                    const int so = (int)((32 * i + 8 * (r >> 2) + (r & 3)) * pitch);
                    float o = alpha * acc[i][j][r];
                    if (beta != 0.0f) {
                        const float c = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(rc, (int)vo[j], so, 0));
                        const float cb = beta * c;
                        o = o + cb;
                    }
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, o), rc,
                                                          (int)vo[j], so, 0);
                }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = r0 + 32 * i + 8 * (r >> 2) + lrow + (r & 3);
                const int64_t col = c0 + 32 * j + lcol;
                TO *dst = C + row * ldc + col;
                float o = alpha * acc[i][j][r];
                if (beta != 0.0f) {
                    const float cb = beta * (float)*dst;
                    o = o + cb;
                }
                *dst = (TO)o;
            }
}

// operand read r of a slice: 0-3 the A fragments, 4-5 the B fragments
__device__ __forceinline__ void w8_read(Frags8 &f, const char *stage, uint32_t s, uint32_t wm,
                                        uint32_t wn, uint32_t lane, int r) {
    if (r < 4) {
        f.a[r] = *(const phx_h8 *)(stage + a_off(wm + r * 32 + (lane & 31), 2 * s + (lane >> 5)));
    } else {  // B columns wn + 32j + lane%32 through two transposing reads
        const int j = r - 4;
        const char *Bs = stage + A_BYTES;
        const uint32_t q = lane >> 4, sl = lane & 15;
        const uint32_t col = wn + j * 32 + 16 * (q & 1) + 4 * (sl & 3);
        phx_fp16x4 h[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t row = 16 * s + 8 * (q >> 1) + 4 * t + (sl >> 2);
            const uint32_t off = b_off(row, col >> 3) + ((col & 7) << 1);
            h[t] = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                (phx_lds_h4p)((__attribute__((address_space(3))) char *)(Bs + off)));
        }
        const phx_h4 lo = __builtin_bit_cast(phx_h4, h[0]);
        const phx_h4 hi = __builtin_bit_cast(phx_h4, h[1]);
        f.b[j] = (phx_h8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
}

struct Regs8 {
    Chunk a[2];
    Chunk b[2];
};

// Thread t's chunks of a step: A chunk i = row 128 i + t/4, k chunk t%4;
// B chunk i = k row 16 i + t/32, n chunk t%32.  Each chunk is 8 f32 (two
// 16-byte loads), rounded to one 16-byte f16 chunk in LDS.
__device__ __forceinline__ void w8_load_a(Regs8 &R, __amdgpu_buffer_rsrc_t ra, uint32_t voa,
                                          uint32_t lda, int i) {  // voa: this step's lane offset
    R.a[i] = load_chunk(ra, voa, (int)((uint32_t)(i * 128 * lda) * ESZ));
}
__device__ __forceinline__ void w8_load_b(Regs8 &R, __amdgpu_buffer_rsrc_t rb, uint32_t vob,
                                          uint32_t ldb, int i) {
    R.b[i] = load_chunk(rb, vob, (int)((uint32_t)(i * 16 * ldb) * ESZ));
}
__device__ __forceinline__ void w8_store_a(const Regs8 &R, char *stage, uint32_t tid, int i) {
    *(phx_u4 *)(stage + a_off(i * 128 + (tid >> 2), tid & 3)) = pack(R.a[i]);
}
__device__ __forceinline__ void w8_store_b(const Regs8 &R, char *stage, uint32_t tid, int i) {
    *(phx_u4 *)(stage + A_BYTES + b_off(i * 16 + (tid >> 5), tid & 31)) = pack(R.b[i]);
}

// One K step kt over three LDS stages: cur holds step kt, nxt step kt+1,
// and fill receives step kt+2, converted from R while step kt+3's loads are
// issued into R (the data of step kt+2 was loaded during step kt-1).  First
// half: slice 0's MFMAs (F0) with slice 1's operand reads (into F1) and A's
// two chunks; the barrier; second half: slice 1's MFMAs with the next
// step's slice-0 reads (from nxt, into F0) and B's two chunks.  fill was
// last read during step kt-1, before the barrier of that step.  In each half
// the two chunks go with MFMAs 0 and 4, half a half apart, so the CU's load
// path sees the step's loads in four evenly spaced bursts (measured: 1-2%
// faster than chunks at MFMAs 0 and 2, bit-identical).
__device__ __forceinline__ void w8_chunk(Regs8 &R, char *fill, __amdgpu_buffer_rsrc_t ra,
                                         __amdgpu_buffer_rsrc_t rb, uint32_t voa, uint32_t vob,
                                         uint32_t lda, uint32_t ldb, uint32_t tid, int c) {
    if (c < 2) {
        w8_store_a(R, fill, tid, c);
        w8_load_a(R, ra, voa, lda, c);
    } else {
        w8_store_b(R, fill, tid, c - 2);
        w8_load_b(R, rb, vob, ldb, c - 2);
    }
}

template <bool RG>
__device__ __forceinline__ void w8_step(phx_f16v (&acc)[4][2], Frags8 &F0, Frags8 &F1,
                                        const char *cur, const char *nxt, char *fill, Regs8 &R,
                                        const TIn *A, uint32_t lda, const TIn *B, uint32_t ldb,
                                        uint32_t M, uint32_t N, uint32_t K, uint32_t m0,
                                        uint32_t n0, uint32_t kt, uint32_t voa, uint32_t voa_t,
                                        uint32_t vob, uint32_t wm, uint32_t wn, uint32_t tid,
                                        uint32_t lane) {
    const uint32_t kn = (kt + 3) * BK;  // the step whose data the reloads fetch
    const __amdgpu_buffer_rsrc_t ra = a_rsrc<RG>(A, lda, M, K, m0, kn);
    const __amdgpu_buffer_rsrc_t rb = b_rsrc<RG>(B, ldb, N, K, n0, kn);
    const uint32_t va = a_lane_off<RG>(voa, voa_t, K, kn);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        w8_mfma(acc, F0, m);
        if (m >= W8_RD && m < W8_RD + 6) w8_read(F1, cur, 1, wm, wn, lane, m - W8_RD);
        if (m == W8_A0 || m == W8_A1) w8_chunk(R, fill, ra, rb, va, vob, lda, ldb, tid, m == W8_A0 ? 0 : 1);
        __builtin_amdgcn_sched_barrier(0);
    }
    PHX_WAIT_VM_LGKM0(63);  // this wave's F1 reads and fill stores are done
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        w8_mfma(acc, F1, m);
        if (m >= W8_RD && m < W8_RD + 6) w8_read(F0, nxt, 0, wm, wn, lane, m - W8_RD);
        if (m == W8_B0 || m == W8_B1) w8_chunk(R, fill, ra, rb, va, vob, lda, ldb, tid, m == W8_B0 ? 2 : 3);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The eight-wave body over tiles t0, t0 + tstride, ... (as gemm_body).  RG:
// M, N or K is not a whole number of tiles; the operand resources then end
// at the matrix edges, A's chunks past K in the last step read zero, and
// the epilogue skips rows and columns past the edges.
#define W8S(CUR, NXT, FILL, KT)                                                              \
    w8_step<RG>(acc, F0, F1, CUR, NXT, FILL, R, A, lda, B, ldb, (uint32_t)M, (uint32_t)N,     \
                (uint32_t)K, m0, n0, KT, voa, voa_t, vob, wm, wn, tid, lane)
template <bool RG, typename TO>
__device__ __forceinline__ void w8_body(const TIn *A, const TIn *B, TO *C, uint32_t lda,
                                        uint32_t ldb, int64_t ldc, int64_t M, int64_t N,
                                        int64_t K, float alpha, float beta, uint32_t t0,
                                        uint32_t tstride, char *stg) {
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = (wave >> 2) * W8_WM, wn = (wave & 3) * W8_WN;
    const uint32_t tiles_n = (uint32_t)((N + BN - 1) / BN), tiles_m = (uint32_t)((M + BM - 1) / BM);
    const uint32_t ntiles = tiles_m * tiles_n, nblk = tstride;
    const uint32_t nk = (uint32_t)((K + BK - 1) / BK);
    const uint32_t voa = ((tid >> 2) * lda + (tid & 3) * 8) * ESZ;
    const uint32_t voa_t = a_tail_off(voa, (tid & 3) * 8, (uint32_t)K);  // 8 k per chunk, K % 8 == 0
    const uint32_t vob = ((tid >> 5) * ldb + (tid & 31) * 8) * ESZ;
    char *const S0 = stg, *const S1 = stg + STAGE_BYTES, *const S2 = stg + 2 * STAGE_BYTES;

    for (uint32_t t = t0; t < ntiles; t += nblk) {
        const uint32_t ts = nblk == ntiles ? phx_xcd_swizzle(t, ntiles) : t;
        const uint32_t gsz = GROUP_M * tiles_n;
        const uint32_t g0 = (ts / gsz) * GROUP_M;
        const uint32_t gm = (tiles_m - g0) < GROUP_M ? (tiles_m - g0) : GROUP_M;
        const uint32_t m0 = (g0 + (ts % gsz) % gm) * BM, n0 = ((ts % gsz) / gm) * BN;

        phx_f16v acc[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        Frags8 F0, F1;
        Regs8 R;
        {   // prologue: steps 0 and 1 into stages 0 and 1, step 2 in flight in R
            for (int p = 0; p < 3; ++p) {
                const __amdgpu_buffer_rsrc_t ra = a_rsrc<RG>(A, lda, (uint32_t)M, (uint32_t)K, m0, p * BK);
                const __amdgpu_buffer_rsrc_t rb = b_rsrc<RG>(B, ldb, (uint32_t)N, (uint32_t)K, n0, p * BK);
                const uint32_t va = a_lane_off<RG>(voa, voa_t, (uint32_t)K, p * BK);
                char *prev = stg + (p - 1) * STAGE_BYTES;  // step p-1's stage
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    if (p > 0) w8_store_a(R, prev, tid, i);
                    w8_load_a(R, ra, va, lda, i);
                    if (p > 0) w8_store_b(R, prev, tid, i);
                    w8_load_b(R, rb, vob, ldb, i);
                }
            }
        }
        PHX_WAIT_VM_LGKM0(63);
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int r = 0; r < 6; ++r) w8_read(F0, S0, 0, wm, wn, lane, r);
        uint32_t kt = 0;
        for (; kt + 3 <= nk; kt += 3) {
            W8S(S0, S1, S2, kt);
            W8S(S1, S2, S0, kt + 1);
            W8S(S2, S0, S1, kt + 2);
        }
        if (kt < nk) W8S(S0, S1, S2, kt);
        if (kt + 1 < nk) W8S(S1, S2, S0, kt + 1);
        PHX_WAIT_VMCNT(0);  // the loads past K (zeros) before the stages are reused
        __syncthreads();

        w8_epilogue<RG, TO>(acc, C, ldc, M, N, m0 + wm, n0 + wn, alpha, beta, lane);
    }
}
#undef W8S

// The operand checks both eight-wave entries share with gemm (the host
// refuses what fails them before launching).
#define W8_SHAPE_OK(LDA, LDB, LDC, TO)                                                        \
    (blockDim.x == W8_NT && N % PHX_TC_N_MULT == 0 && K % PHX_TC_K_MULT == 0 && M > 0 &&     \
     N > 0 && K > 0 && (LDA) % PHX_TC_K_MULT == 0 && ((LDB) | (LDC)) % PHX_TC_N_MULT == 0 && \
     M <= INT32_MAX && (BM + 1) * ((LDA) > (LDB) ? (LDA) : (LDB)) * (int64_t)sizeof(TIn) <= INT32_MAX && \
     (BM + 1) * (LDC) * (int64_t)sizeof(TO) <= INT32_MAX)

extern "C" __global__ __launch_bounds__(W8_NT, 1) void gemm_w8(PHX_MEMREF2(TIn, a, int64_t),
                                                                PHX_MEMREF2(TIn, b, int64_t),
                                                                PHX_MEMREF2(TOut, c, int64_t),
                                                                float alpha, float beta) {
    __shared__ __attribute__((aligned(16))) char stg[3 * STAGE_BYTES];
    const int64_t M = a_s0, K = a_s1, N = b_s1;
    if (!W8_SHAPE_OK(a_st0, b_st0, c_st0, TOut) || b_s0 != K || c_s0 != M || c_s1 != N ||
        a_st1 != 1 || b_st1 != 1 || c_st1 != 1 ||
        ((uintptr_t)(a_ptr + a_off) | (uintptr_t)(b_ptr + b_off) | (uintptr_t)(c_ptr + c_off)) & 15)
        return;
    const TIn *A = a_ptr + a_off;
    const TIn *B = b_ptr + b_off;
    TOut *C = c_ptr + c_off;
    if (M % BM == 0 && N % BN == 0 && K % BK == 0)  // uniform
        w8_body<false, TOut>(A, B, C, (uint32_t)a_st0, (uint32_t)b_st0, c_st0, M, N, K, alpha,
                             beta, phx_block_linear(), phx_block_count(), stg);
    else
        w8_body<true, TOut>(A, B, C, (uint32_t)a_st0, (uint32_t)b_st0, c_st0, M, N, K, alpha,
                            beta, phx_block_linear(), phx_block_count(), stg);
}

// Split-K on the eight-wave body: the same contract as gemm_splitk (raw f32
// sums of K columns [y * kchunk, min(K, (y+1) * kchunk)) to W + y * M * N).
extern "C" __global__ __launch_bounds__(W8_NT, 1) void gemm_w8_splitk(const TIn *A, const TIn *B,
                                                                       float *W, int64_t lda,
                                                                       int64_t ldb, int64_t M,
                                                                       int64_t N, int64_t K,
                                                                       int64_t kchunk) {
    __shared__ __attribute__((aligned(16))) char stg[3 * STAGE_BYTES];
    const int64_t k0 = (int64_t)blockIdx.y * kchunk;
    if (!W8_SHAPE_OK(lda, ldb, N, float) || k0 >= K || kchunk % BK) return;
    const int64_t kc = K - k0 < kchunk ? K - k0 : kchunk;
    const TIn *As = A + k0;
    const TIn *Bs = B + k0 * ldb;
    float *Ws = W + (int64_t)blockIdx.y * M * N;
    if (M % BM == 0 && N % BN == 0 && kc % BK == 0)
        w8_body<false, float>(As, Bs, Ws, (uint32_t)lda, (uint32_t)ldb, N, M, N, kc, 1.0f, 0.0f,
                              blockIdx.x, gridDim.x, stg);
    else
        w8_body<true, float>(As, Bs, Ws, (uint32_t)lda, (uint32_t)ldb, N, M, N, kc, 1.0f, 0.0f,
                             blockIdx.x, gridDim.x, stg);
}
#endif
