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
// K and V are both staged as plain 16-byte row copies (K by threads 128-255,
// V by threads 0-127, 4 buffer loads each).  K runs one block ahead of V:
// during block j the LDS holds K_{j+1} (for the next scores) and V_j.
struct Stage {
    phx_u4 r[4];
};

typedef __fp16 phx_fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) phx_fp16x4 *phx_lds_h4p;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t phx_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

// V rows (128 bytes) are read with ds_read_b64_tr_b16: a 32-lane service
// group touches 4 consecutive rows x 64 bytes, so rows 2 apart are shifted by
// 64 bytes to land on distinct banks.
__device__ __forceinline__ uint32_t v_off(uint32_t row, uint32_t chunk) {
    return row * ROW_BYTES + ((chunk ^ (((row >> 1) & 1) << 2)) << 4);
}

// Thread u of a 128-thread half stages rows i*16 + u/8 (i < 4), chunk u%8.
__device__ __forceinline__ void load_stage(Stage &st, __amdgpu_buffer_rsrc_t r, uint32_t rowb,
                                           uint32_t blk, bool val, uint32_t vo) {
    if (!val) return;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        st.r[i] = __builtin_bit_cast(
            phx_u4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(vo + i * 16 * rowb),
                                                          (int)(blk * BC * rowb), 0));
}

__device__ __forceinline__ void store_stage(const Stage &st, char *Ks, char *Vs, bool kval,
                                            bool vval, uint32_t tid) {
    const uint32_t u = tid & 127, ch = u & 7;
    if (tid < 128) {
        if (!vval) return;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *(phx_u4 *)(Vs + v_off(i * 16 + (u >> 3), ch)) = st.r[i];
    } else {
        if (!kval) return;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *(phx_u4 *)(Ks + lds_off(i * 16 + (u >> 3), ch)) = st.r[i];
    }
}

// S^T = K . Q^T for one key block: sT[t] holds keys 32t + 8(r/4) + 4g + r%4
// of query lq.
__device__ __forceinline__ void scores(phx_f16v (&sT)[2], const char *Ks, const phx_h8 (&qf)[4],
                                       uint32_t lq, uint32_t g) {
    phx_h8 kf[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s)
            kf[t][s] = *(const phx_h8 *)(Ks + lds_off(32 * t + lq, 2 * s + g));
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        sT[t] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < 4; ++s)
            sT[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t][s], qf[s], sT[t], 0, 0, 0);
    }
}

// The running max is raised only when a row's block max exceeds it by more
// than RESCALE_SLACK (in log2 units), so the O/l rescale is skipped on almost
// every block; p = exp2(s*c - m) then stays <= 2^8, which f16 P and f32 l
// hold as well as the reference's per-block update.  O = acc / l is the same
// quantity either way.
#define RESCALE_SLACK 8.0f

struct FlashState {
    phx_f16v acc[2];
    float m2, l;
};

// One key block: issue the next block's scores (K_{kb+1}, MFMA pipe), then
// this block's softmax (VALU) and P.V (V_kb); stage K_{kb+2} / V_{kb+1}.
__device__ __forceinline__ void flash_step(FlashState &fs, phx_f16v (&sT)[2], phx_f16v (&sN)[2],
                                           Stage &st, char (*lds)[2][TILE_BYTES],
                                           const phx_h8 (&qf)[4], __amdgpu_buffer_rsrc_t rk,
                                           __amdgpu_buffer_rsrc_t rv, uint32_t kbr, uint32_t vbr,
                                           uint32_t vo, uint32_t kb, uint32_t nkb, float c2,
                                           uint32_t tid, uint32_t lane) {
    const uint32_t lq = lane & 31, g = lane >> 5;
    const uint32_t cur = kb & 1, nxt = cur ^ 1;
    const bool more = kb + 1 < nkb;
    if (tid < 128)
        load_stage(st, rv, vbr, kb + 1, more, vo);
    else
        load_stage(st, rk, kbr, kb + 2, kb + 2 < nkb, vo);
    if (more) scores(sN, lds[nxt][0], qf, lq, g);
    __builtin_amdgcn_sched_barrier(0);

    float mx = sT[0][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sT[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sT[1][r]);
    mx = fmaxf(mx, shfl_xor32(mx)) * c2;
    if (__ballot(mx > fs.m2 + RESCALE_SLACK)) {  // wave-uniform
        const float m2new = fmaxf(fs.m2, mx);
        const float corr = __builtin_amdgcn_exp2f(fs.m2 - m2new);
        fs.l = fs.l * corr;
        fs.acc[0] = fs.acc[0] * corr;
        fs.acc[1] = fs.acc[1] * corr;
        fs.m2 = m2new;
    }
    // P (f16) and its row sum: v_dot2_f32_f16 against (1, 1) adds the two
    // f16 values of a pair into an f32 sum.
    const phx_h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    float ps = 0.0f;
    phx_h8 pf[4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            phx_h8 v;
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const float p0 =
                    __builtin_amdgcn_exp2f(__builtin_fmaf(sT[t][8 * hh + j], c2, -fs.m2));
                const float p1 =
                    __builtin_amdgcn_exp2f(__builtin_fmaf(sT[t][8 * hh + j + 1], c2, -fs.m2));
                const phx_h2 pp = {(_Float16)p0, (_Float16)p1};
                ps = __builtin_amdgcn_fdot2(pp, ones, ps, false);
                v[j] = pp.x;
                v[j + 1] = pp.y;
            }
            pf[2 * t + hh] = v;
        }
    ps += shfl_xor32(ps);
    fs.l = fs.l + ps;

    // O^T[dt] += V^T[32 d rows, 16 keys of block c] . P^T.  The A operand
    // of lane group g holds keys 16c + 4g + 0..3 and 16c + 8 + 4g + 0..3 (the
    // order P's registers have), read as two transposing 4-key runs.
    const char *Vs = lds[cur][1];
    const uint32_t q = lane >> 4, sl = lane & 15;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
            const uint32_t col = 32 * dt + 16 * (q & 1) + 4 * (sl & 3);  // d
            phx_fp16x4 h[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint32_t row = 16 * c + 8 * t + 4 * (q >> 1) + (sl >> 2);  // key
                const uint32_t off = v_off(row, col >> 3) + ((col & 7) << 1);
                h[t] = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                    (phx_lds_h4p)((__attribute__((address_space(3))) char *)(Vs + off)));
            }
            const phx_h4 lo = __builtin_bit_cast(phx_h4, h[0]);
            const phx_h4 hi = __builtin_bit_cast(phx_h4, h[1]);
            const phx_h8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            fs.acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[c], fs.acc[dt], 0, 0, 0);
        }
    // K_{kb+2} -> buffer cur (its K_kb fed the scores one block ago);
    // V_{kb+1} -> buffer nxt (its V_{kb-1} is done).
    store_stage(st, lds[cur][0], lds[nxt][1], kb + 2 < nkb, more, tid);
    __syncthreads();
}

__device__ __forceinline__ void flash_block(const T *Q, const T *Kp, const T *Vp, T *O,
                                            int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                                            uint32_t Nk, uint32_t q0, float scale,
                                            char (*lds)[2][TILE_BYTES]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t lq = lane & 31, g = lane >> 5;
    const uint32_t myq = q0 + wave * 32 + lq;
    const float c2 = scale * LOG2E;
    const uint32_t nkb = Nk / BC;

    // buffer views of this head's K and V; vo = this thread's staging offset
    const uint32_t kbr = (uint32_t)(ldk * 2), vbr = (uint32_t)(ldv * 2);
    const __amdgpu_buffer_rsrc_t rk = phx_rsrc(Kp, (uint32_t)((Nk - 1) * kbr + D * 2));
    const __amdgpu_buffer_rsrc_t rv = phx_rsrc(Vp, (uint32_t)((Nk - 1) * vbr + D * 2));
    const uint32_t u = tid & 127;
    const uint32_t vo = (u >> 3) * (tid < 128 ? vbr : kbr) + 16 * (u & 7);

    // Q^T operand: s-step s covers d = 16s + 8g .. +7
    phx_h8 qf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[s] = *(const phx_h8 *)(Q + (int64_t)myq * ldq + 16 * s + 8 * g);

    FlashState fs;
    fs.acc[0] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    fs.acc[1] = fs.acc[0];
    fs.m2 = M_INIT * LOG2E;
    fs.l = 0.0f;

    // prologue: V_0 -> buffer 0 (threads 0-127), K_0 -> buffer 0 then K_1 ->
    // buffer 1 (threads 128-255)
    Stage st;
    if (tid < 128) {
        load_stage(st, rv, vbr, 0, true, vo);
        store_stage(st, lds[0][0], lds[0][1], false, true, tid);
    } else {
        load_stage(st, rk, kbr, 0, true, vo);
        store_stage(st, lds[0][0], lds[0][1], true, false, tid);
        load_stage(st, rk, kbr, 1, nkb > 1, vo);
        store_stage(st, lds[1][0], lds[1][1], nkb > 1, false, tid);
    }
    __syncthreads();

    phx_f16v s0[2], s1[2];
    scores(s0, lds[0][0], qf, lq, g);
    uint32_t kb = 0;
    for (; kb + 1 < nkb; kb += 2) {
        flash_step(fs, s0, s1, st, lds, qf, rk, rv, kbr, vbr, vo, kb, nkb, c2, tid, lane);
        flash_step(fs, s1, s0, st, lds, qf, rk, rv, kbr, vbr, vo, kb + 1, nkb, c2, tid, lane);
    }
    if (kb < nkb) flash_step(fs, s0, s1, st, lds, qf, rk, rv, kbr, vbr, vo, kb, nkb, c2, tid, lane);

    // acc[dt][r]: d = 32dt + 8(r/4) + 4g + r%4, query lq.
    T *orow = O + (int64_t)myq * ldo;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            phx_h4 v;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) v[rr] = (_Float16)(fs.acc[dt][4 * b + rr] / fs.l);
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
