// Flash-attention leaf kernels for gfx950 (FlashAttention-2 online softmax).
//
// Built twice from this file:
//   -DPHX_FLASH_F16   flash_attention_fp16.ph: f16 Q/K/V/O, f32 m/l/acc,
//                     m starts at -65504 (:23), P is rounded to f16 for P.V
//                     while l sums the f32 P, O is rounded f32 -> f16 on store.
//   -DPHX_FLASH_F32   flash_attention_fp32.ph: f32 everywhere, m starts at
//                     -3e8.  Runs on the f32 matrix cores with no f16
//                     rounding (the exact-f32 semantics of the .ph source).
// Per key block (examples/flash_attention_fp16.ph:26-46):
//   s = q.k^T * scale; mnew = max(m, rowmax s); p = exp(s - mnew);
//   corr = exp(m - mnew); l = l*corr + rowsum p; acc = acc*corr + p.v; m = mnew
// and O = acc / l at the end.  exp(x) is evaluated as exp2(x * log2 e) on
// v_exp_f32, with the scale folded in: the running max is kept in units of
// log2, m2 = m * log2e, and p = exp2(fma(s, scale*log2e, -m2)), which is the
// same quantity as the reference's ex2.approx(x * log2e) formulation
// (phobos-lang/src/codegen/tile.rs:1027-1061) up to f32 rounding.
//
// Entry points: "flash_attention" keeps the one-head .ph signature
// (tensor[N, D] x 4 + scale, wide i64 descriptors, launch_flash at
// phobos-bench/src/main.rs:334-371); "flash_attention_bh" takes [BH, N, D]
// tensors and runs every head in one launch (grid.y = heads).
//
// MI355X design (f16)
//   * 128 queries per workgroup, 4 waves x 32 queries, 64 keys per step, D=64.
//   * Each wave computes S^T = K . Q^T with v_mfma_f32_32x32x16_f16 (K from
//     LDS is the A operand, Q^T lives in 16 VGPRs as the B operand), so a lane
//     holds 32 scores of ONE query; the row max/sum is a register reduction
//     plus one swap with lane^32.
//   * O^T = V^T . P^T: P^T is the B operand straight from the score registers
//     (cvt to f16, no LDS round trip); V^T comes from LDS, staged transposed
//     with bits 2 and 3 of the key index swapped so each lane's 8 keys are
//     one ds_read_b128.  The per-query rescale is then a per-lane scalar.
//   * K and V^T are double-buffered in LDS (2 x 16 KiB), next block's global
//     loads in flight during the current block's 16 MFMAs per wave.
//   * Workgroups are renumbered XCD-major so all blocks of one head share an
//     XCD and its L2.
#include "phx_common.h"

#define BR PHX_FA_BR
#define BC PHX_FA_BC
#define D PHX_FA_D
#define NT PHX_FA_THREADS

#define LOG2E 1.4426950408889634f

#ifdef PHX_FLASH_F16
typedef _Float16 T;
#define M_INIT (-65504.0f)
#define ROW_BYTES (D * 2)  // K rows (64 d) and V^T rows (64 keys): 128 bytes
#else
typedef float T;
#define M_INIT (-300000000.0f)
#define ROW_BYTES (D * 4)  // 256 bytes
#endif
#define TILE_BYTES (BC * ROW_BYTES)  // BC == D == 64 rows
// two workgroups (8 waves) per CU for the f16 path
#ifdef PHX_FLASH_F16
#define FA_MIN_BLOCKS 2
#else
#define FA_MIN_BLOCKS 1
#endif

// LDS serves 64 banks x 4 bytes per clock on gfx950, so a 16-lane group of a
// 16-byte access must hit 16 distinct 16-byte slots of a 256-byte line.
// 128-byte rows: two rows share a line, XOR the chunk with (row>>1)&7;
// 256-byte rows: XOR with row&15.
__device__ __forceinline__ uint32_t lds_off(uint32_t row, uint32_t chunk) {
#ifdef PHX_FLASH_F16
    return row * ROW_BYTES + ((chunk ^ ((row >> 1) & 7)) << 4);
#else
    return row * ROW_BYTES + ((chunk ^ (row & 15)) << 4);
#endif
}

__device__ __forceinline__ float shfl_xor32(float v) { return __shfl_xor(v, 32, 64); }

#ifdef PHX_FLASH_F16
// ---------------------------------------------------------------- f16 path
// Threads 0-127 stage V^T, threads 128-255 stage K; 4 x 16-byte buffer loads
// each.  K runs one block ahead of V: during block j the LDS holds K_{j+1}
// (for the next scores) and V_j (for this block's P.V).
struct Stage {
    phx_u4 r[4];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t phx_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

// V thread v (0..127): c = v/32 (16-key group), h = (v/16)%2, b' = (v/8)%2,
// db = v%8: rows key = 16c + 8b' + 4h + i (i<4), d = 8db..8db+7.
// K thread u (0..127): rows i*16 + u/8 (i<4), 16-byte chunk u%8.
// vo: this thread's byte offset inside a block (see flash_block).
__device__ __forceinline__ void load_stage(Stage &st, __amdgpu_buffer_rsrc_t rk,
                                           __amdgpu_buffer_rsrc_t rv, uint32_t kbytes_row,
                                           uint32_t vbytes_row, uint32_t kblk, uint32_t vblk,
                                           bool kval, bool vval, uint32_t vo, uint32_t tid) {
    if (tid < 128) {
        if (vval) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                st.r[i] = __builtin_bit_cast(
                    phx_u4, __builtin_amdgcn_raw_buffer_load_b128(
                                rv, (int)(vo + i * vbytes_row), (int)(vblk * BC * vbytes_row), 0));
        }
    } else if (kval) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            st.r[i] = __builtin_bit_cast(
                phx_u4, __builtin_amdgcn_raw_buffer_load_b128(
                            rk, (int)(vo + i * 16 * kbytes_row), (int)(kblk * BC * kbytes_row), 0));
    }
}

__device__ __forceinline__ uint32_t pk_lo(uint32_t x, uint32_t y) {
    return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t pk_hi(uint32_t x, uint32_t y) {
    return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

__device__ __forceinline__ void store_stage(const Stage &st, char *Ks, char *Vt, bool kval,
                                            bool vval, uint32_t tid) {
    if (tid < 128) {
        if (!vval) return;
        const uint32_t v = tid;
        const uint32_t db = v & 7, bp = (v >> 3) & 1, h = (v >> 4) & 1, c = v >> 5;
        // keys 16c + 8b' + 4h + i  ->  position 16c + 8h + 4b' + i: chunk 2c+h, half bp
        const uint32_t chunk = 2 * c + h;
        uint32_t r[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r[i][0] = st.r[i].x; r[i][1] = st.r[i].y; r[i][2] = st.r[i].z; r[i][3] = st.r[i].w;
        }
#pragma unroll
        for (int dd = 0; dd < 4; ++dd) {
            phx_u2 lo, hi;
            lo.x = pk_lo(r[0][dd], r[1][dd]);
            lo.y = pk_lo(r[2][dd], r[3][dd]);
            hi.x = pk_hi(r[0][dd], r[1][dd]);
            hi.y = pk_hi(r[2][dd], r[3][dd]);
            const uint32_t d0 = 8 * db + 2 * dd;
            *(phx_u2 *)(Vt + lds_off(d0, chunk) + 8 * bp) = lo;
            *(phx_u2 *)(Vt + lds_off(d0 + 1, chunk) + 8 * bp) = hi;
        }
    } else {
        if (!kval) return;
        const uint32_t u = tid - 128;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t row = i * 16 + (u >> 3), ch = u & 7;
            *(phx_u4 *)(Ks + lds_off(row, ch)) = st.r[i];
        }
    }
}

// S^T = K . Q^T for one key block: sT[t] holds keys 32t + 8(r/4) + 4g + r%4
// of query lq.
__device__ __forceinline__ void scores(phx_f16v (&sT)[2], const phx_h8 (&kf)[2][4],
                                       const phx_h8 (&qf)[4]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        sT[t] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < 4; ++s)
            sT[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t][s], qf[s], sT[t], 0, 0, 0);
    }
}

__device__ __forceinline__ void read_k(phx_h8 (&kf)[2][4], const char *Ks, uint32_t lq,
                                       uint32_t g) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s)
            kf[t][s] = *(const phx_h8 *)(Ks + lds_off(32 * t + lq, 2 * s + g));
}

// The running max is raised only when a row's block max exceeds it by more
// than RESCALE_SLACK (in log2 units), so the O/l rescale (32 multiplies) is
// skipped on almost every block; p = exp2(s*c - m) then stays <= 2^8, which
// f16 P and f32 l hold exactly as well as the reference's per-block update.
// O = acc / l is the same quantity either way.
#define RESCALE_SLACK 8.0f

__device__ __forceinline__ void flash_block(const T *Q, const T *Kp, const T *Vp, T *O,
                                            int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                                            uint32_t Nk, uint32_t q0, float scale,
                                            char (*lds)[2][TILE_BYTES]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t lq = lane & 31, g = lane >> 5;
    const uint32_t myq = q0 + wave * 32 + lq;
    const float c2 = scale * LOG2E;
    const uint32_t nkb = Nk / BC;

    // buffer views of this head's K and V
    const uint32_t kbr = (uint32_t)(ldk * 2), vbr = (uint32_t)(ldv * 2);
    const __amdgpu_buffer_rsrc_t rk = phx_rsrc(Kp, (uint32_t)((Nk - 1) * kbr + D * 2));
    const __amdgpu_buffer_rsrc_t rv = phx_rsrc(Vp, (uint32_t)((Nk - 1) * vbr + D * 2));
    uint32_t vo;
    if (tid < 128) {
        const uint32_t v = tid, db = v & 7, bp = (v >> 3) & 1, h = (v >> 4) & 1, c = v >> 5;
        vo = (16 * c + 8 * bp + 4 * h) * vbr + 16 * db;
    } else {
        const uint32_t u = tid - 128;
        vo = (u >> 3) * kbr + 16 * (u & 7);
    }

    // Q^T operand: s-step s covers d = 16s + 8g .. +7
    phx_h8 qf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = *(const phx_h8 *)(Q + (int64_t)myq * ldq + 16 * s + 8 * g);

    phx_f16v acc[2];
    acc[0] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    acc[1] = acc[0];
    float m2 = M_INIT * LOG2E;
    float l = 0.0f;

    // prologue: K_0, V_0 -> buffer 0; K_1 -> buffer 1
    Stage st;
    load_stage(st, rk, rv, kbr, vbr, 0, 0, true, true, vo, tid);
    store_stage(st, lds[0][0], lds[0][1], true, true, tid);
    load_stage(st, rk, rv, kbr, vbr, 1, 0, nkb > 1, false, vo, tid);
    store_stage(st, lds[1][0], lds[1][1], nkb > 1, false, tid);
    __syncthreads();

    phx_f16v sT[2];
    {
        phx_h8 kf[2][4];
        read_k(kf, lds[0][0], lq, g);
        scores(sT, kf, qf);
    }

    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const uint32_t cur = kb & 1, nxt = cur ^ 1;
        const bool more = kb + 1 < nkb;
        // global loads of K_{kb+2} and V_{kb+1}, stored at the end of this block
        load_stage(st, rk, rv, kbr, vbr, kb + 2, kb + 1, kb + 2 < nkb, more, vo, tid);

        // next block's scores go to the MFMA pipe while this block's softmax
        // runs on the VALU
        phx_f16v sN[2];
        {
            phx_h8 kf[2][4];
            if (more) read_k(kf, lds[nxt][0], lq, g);
            if (more) scores(sN, kf, qf);
        }
        __builtin_amdgcn_sched_barrier(0);

        float mx = sT[0][0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sT[0][r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sT[1][r]);
        mx = fmaxf(mx, shfl_xor32(mx)) * c2;
        if (__ballot(mx > m2 + RESCALE_SLACK)) {  // wave-uniform
            const float m2new = fmaxf(m2, mx);
            const float corr = __builtin_amdgcn_exp2f(m2 - m2new);
            l = l * corr;
            acc[0] = acc[0] * corr;
            acc[1] = acc[1] * corr;
            m2 = m2new;
        }
        float ps = 0.0f;
        phx_h8 pf[4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                phx_h8 v;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sT[t][8 * hh + j], c2, -m2));
                    ps += p;
                    v[j] = (_Float16)p;
                }
                pf[2 * t + hh] = v;
            }
        ps += shfl_xor32(ps);
        l = l + ps;
        // O^T[dt] += V^T[dt rows, 16 keys of block c] . P^T
        const char *Vt = lds[cur][1];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
                const phx_h8 vf = *(const phx_h8 *)(Vt + lds_off(32 * dt + lq, 2 * c + g));
                acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[c], acc[dt], 0, 0, 0);
            }
        if (more) {
            sT[0] = sN[0];
            sT[1] = sN[1];
        }
        // K_{kb+2} -> buffer cur (its K_kb was used for the scores one block
        // ago); V_{kb+1} -> buffer nxt (its V_{kb-1} is done).
        store_stage(st, lds[cur][0], lds[nxt][1], kb + 2 < nkb, more, tid);
        __syncthreads();
    }

    // acc[dt][r]: d = 32dt + 8(r/4) + 4g + r%4, query lq.
    T *orow = O + (int64_t)myq * ldo;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            phx_h4 v;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) v[rr] = (_Float16)(acc[dt][4 * b + rr] / l);
            *(phx_h4 *)(orow + 32 * dt + 8 * b + 4 * g) = v;
        }
}
#else
// ---------------------------------------------------------------- f32 path
// K rows / V^T rows are 64 floats (256 B, 16 chunks).  Waves 0-1 stage V^T
// via 4x4 register transposes, waves 2-3 stage K; 8 x 16-byte loads each.
struct Stage {
    phx_f4 r[8];
};

__device__ __forceinline__ void load_stage(Stage &st, const T *Kp, const T *Vp, int64_t ldk,
                                           int64_t ldv, uint32_t key0, uint32_t tid) {
    if (tid < 128) {
        // two 4x4 blocks: keys 4kq..4kq+3 (kq = v/16 and kq+8), d = 4*(v%16)..
        const uint32_t v = tid, dq = v & 15, kq = v >> 4;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                st.r[4 * h + i] =
                    *(const phx_f4 *)(Vp + (int64_t)(key0 + 4 * (kq + 8 * h) + i) * ldv + 4 * dq);
    } else {
        const uint32_t u = tid - 128;  // 64 rows x 16 chunks = 1024 = 128 x 8
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t row = i * 8 + (u >> 4), ch = u & 15;
            st.r[i] = *(const phx_f4 *)(Kp + (int64_t)(key0 + row) * ldk + 4 * ch);
        }
    }
}

__device__ __forceinline__ void store_stage(const Stage &st, char *Ks, char *Vt, uint32_t tid) {
    if (tid < 128) {
        const uint32_t v = tid, dq = v & 15, kq = v >> 4;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const phx_f4 *b = &st.r[4 * h];
            const uint32_t chunk = kq + 8 * h;  // keys 4*chunk .. +3
            phx_f4 c0 = {b[0].x, b[1].x, b[2].x, b[3].x};
            phx_f4 c1 = {b[0].y, b[1].y, b[2].y, b[3].y};
            phx_f4 c2 = {b[0].z, b[1].z, b[2].z, b[3].z};
            phx_f4 c3 = {b[0].w, b[1].w, b[2].w, b[3].w};
            *(phx_f4 *)(Vt + lds_off(4 * dq + 0, chunk)) = c0;
            *(phx_f4 *)(Vt + lds_off(4 * dq + 1, chunk)) = c1;
            *(phx_f4 *)(Vt + lds_off(4 * dq + 2, chunk)) = c2;
            *(phx_f4 *)(Vt + lds_off(4 * dq + 3, chunk)) = c3;
        }
    } else {
        const uint32_t u = tid - 128;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t row = i * 8 + (u >> 4), ch = u & 15;
            *(phx_f4 *)(Ks + lds_off(row, ch)) = st.r[i];
        }
    }
}

__device__ __forceinline__ void flash_block(const T *Q, const T *Kp, const T *Vp, T *O,
                                            int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                                            uint32_t Nk, uint32_t q0, float scale,
                                            char (*lds)[2][TILE_BYTES]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t lq = lane & 31, g = lane >> 5;
    const uint32_t myq = q0 + wave * 32 + lq;
    const float c2 = scale * LOG2E;

    // Q^T operand: MFMA (q', s) uses d = 8q' + 4g + s.
    phx_f4 qf[8];
#pragma unroll
    for (int qq = 0; qq < 8; ++qq) qf[qq] = *(const phx_f4 *)(Q + (int64_t)myq * ldq + 8 * qq + 4 * g);

    phx_f16v acc[2];
    acc[0] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    acc[1] = acc[0];
    float m2 = M_INIT * LOG2E;
    float l = 0.0f;

    const uint32_t nkb = Nk / BC;
    Stage st;
    load_stage(st, Kp, Vp, ldk, ldv, 0, tid);
    store_stage(st, lds[0][0], lds[0][1], tid);
    __syncthreads();

    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const uint32_t cur = kb & 1;
        if (kb + 1 < nkb) load_stage(st, Kp, Vp, ldk, ldv, (kb + 1) * BC, tid);
        const char *Ks = lds[cur][0];
        const char *Vt = lds[cur][1];

        phx_f16v sT[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            sT[t] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int qq = 0; qq < 8; ++qq) {
                phx_f4 kf = *(const phx_f4 *)(Ks + lds_off(32 * t + lq, 2 * qq + g));
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    sT[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[s], qf[qq][s], sT[t], 0, 0, 0);
            }
        }
        float mx = sT[0][0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sT[0][r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sT[1][r]);
        mx = fmaxf(mx, shfl_xor32(mx));
        const float m2new = fmaxf(m2, mx * c2);
        const float corr = __builtin_amdgcn_exp2f(m2 - m2new);
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sT[t][r], c2, -m2new));
                ps += p;
                sT[t][r] = p;
            }
        ps += shfl_xor32(ps);
        l = l * corr + ps;
        m2 = m2new;
        acc[0] = acc[0] * corr;
        acc[1] = acc[1] * corr;
        // P^T operand: lane holds keys 32t + 8b + 4g + s = sT[t][4b + s];
        // V^T row d, chunk (8t + 2b + g) holds keys 32t + 8b + 4g .. +3.
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    phx_f4 vf = *(const phx_f4 *)(Vt + lds_off(32 * dt + lq, 8 * t + 2 * b + g));
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[s], sT[t][4 * b + s],
                                                                       acc[dt], 0, 0, 0);
                }

        if (kb + 1 < nkb) store_stage(st, lds[cur ^ 1][0], lds[cur ^ 1][1], tid);
        __syncthreads();
    }

    T *orow = O + (int64_t)myq * ldo;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            phx_f4 v;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) v[rr] = acc[dt][4 * b + rr] / l;
            *(phx_f4 *)(orow + 32 * dt + 8 * b + 4 * g) = v;
        }
}
#endif

extern "C" __global__ __launch_bounds__(NT, FA_MIN_BLOCKS) void flash_attention(PHX_MEMREF2(T, q, int64_t),
                                                                  PHX_MEMREF2(T, k, int64_t),
                                                                  PHX_MEMREF2(T, v, int64_t),
                                                                  PHX_MEMREF2(T, o, int64_t),
                                                                  float scale) {
    __shared__ __attribute__((aligned(16))) char lds[2][2][TILE_BYTES];
    const int64_t Nq = q_s0, Nk = k_s0;
    if (blockDim.x != NT || q_s1 != D || k_s1 != D || v_s1 != D || o_s1 != D || v_s0 != Nk ||
        o_s0 != Nq || Nq % BR || Nk % BC || Nq <= 0 || Nk <= 0 || q_st1 != 1 || k_st1 != 1 ||
        v_st1 != 1 || o_st1 != 1)
        return;
    const uint32_t nrb = (uint32_t)(Nq / BR);
    for (uint32_t rb = phx_block_linear(); rb < nrb; rb += phx_block_count())
        flash_block(q_ptr + q_off, k_ptr + k_off, v_ptr + v_off, o_ptr + o_off, q_st0, k_st0,
                    v_st0, o_st0, (uint32_t)Nk, rb * BR, scale, lds);
}

extern "C" __global__ __launch_bounds__(NT, FA_MIN_BLOCKS) void flash_attention_bh(PHX_MEMREF3(T, q, int64_t),
                                                                     PHX_MEMREF3(T, k, int64_t),
                                                                     PHX_MEMREF3(T, v, int64_t),
                                                                     PHX_MEMREF3(T, o, int64_t),
                                                                     float scale) {
    __shared__ __attribute__((aligned(16))) char lds[2][2][TILE_BYTES];
    const int64_t H = q_s0, Nq = q_s1, Nk = k_s1;
    if (blockDim.x != NT || k_s0 != H || v_s0 != H || o_s0 != H || q_s2 != D || k_s2 != D ||
        v_s2 != D || o_s2 != D || v_s1 != Nk || o_s1 != Nq || Nq % BR || Nk % BC || Nq <= 0 ||
        Nk <= 0 || H <= 0 || q_st2 != 1 || k_st2 != 1 || v_st2 != 1 || o_st2 != 1)
        return;
    const uint32_t nrb = (uint32_t)(Nq / BR);
    const uint32_t nwork = nrb * (uint32_t)H;
    const uint32_t nblk = phx_block_count();
    for (uint32_t w = phx_block_linear(); w < nwork; w += nblk) {
        const uint32_t ws = nblk == nwork ? phx_xcd_swizzle(w, nwork) : w;
        const uint32_t h = ws / nrb, rb = ws % nrb;
        flash_block(q_ptr + q_off + h * q_st0, k_ptr + k_off + h * k_st0,
                    v_ptr + v_off + h * v_st0, o_ptr + o_off + h * o_st0, q_st1, k_st1, v_st1,
                    o_st1, (uint32_t)Nk, rb * BR, scale, lds);
    }
}
