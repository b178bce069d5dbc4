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
//   * 256 queries per workgroup, 8 waves x 32 queries, 64 keys per step,
//     D = 64; two workgroups per CU, so four waves per SIMD.
//   * Each wave computes S^T = K . Q^T with v_mfma_f32_32x32x16_f16 (K from
//     LDS is the A operand, Q^T lives in 16 VGPRs as the B operand), so a lane
//     holds 32 scores of ONE query; the row sum is a register reduction plus
//     one swap with lane^32, and the row max is only taken when needed.
//   * O^T = V^T . P^T: P^T is the B operand straight from the score registers
//     (cvt to f16, no LDS round trip); V^T comes from LDS through the
//     transposing ds_read_b64_tr_b16.  The per-query rescale is then a
//     per-lane scalar.
//   * K and V reach LDS by direct global->LDS copies into a 4-stage ring.
//   * Workgroups are renumbered XCD-major so all blocks of one head share an
//     XCD and its L2.
//   * Measured on MI355X: at these shapes the card runs at its 1.4 kW power
//     limit (socket power 1346 W, shader clock ~1.8 GHz instead of 2.4), so
//     the time per head is set by the energy per block.  Staggered and
//     software-pipelined schedules with two waves per SIMD ran no faster than
//     this plain four-waves-per-SIMD form.
#include "phx_common.h"

#define BR PHX_FA_BR
#define BC PHX_FA_BC
#define D PHX_FA_D
#ifdef PHX_FLASH_F16
#define NT PHX_FA16_THREADS
#else
#define NT PHX_FA_THREADS
#endif

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
// second __launch_bounds__ operand: waves per SIMD the register budget must allow
#ifdef PHX_FLASH_F16
#define FA_WAVES_PER_SIMD 4  // two 8-wave workgroups per CU: <= 128 registers per wave
#else
#define FA_WAVES_PER_SIMD 2  // two 4-wave workgroups per CU: <= 256 registers per wave
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


// v = x of lane l combined with x of lane l^32: gfx950's v_permlane32_swap
// exchanges the two 32-lane halves in one VALU op (no LDS round trip).
__device__ __forceinline__ float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                    __builtin_bit_cast(uint32_t, x), false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float xor32_add(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                    __builtin_bit_cast(uint32_t, x), false, false);
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

typedef __attribute__((address_space(3))) void *phx_lds_vp;
// s_waitcnt fields: vmcnt [3:0]+[15:14], expcnt [6:4], lgkmcnt [11:8]
#define PHX_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

__device__ __forceinline__ __amdgpu_buffer_rsrc_t phx_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

// Buffer resource from the first row of key block blk to the end of the K or
// V matrix: a block's copies only reach its own 64 rows, so rows past Nk (a
// partial last block) read zero, and a block past the end has no records.
// (No min over the block's rows: this form keeps the copy schedule of the
// full-block loop as it was, measured 4% faster than a clamped row count.)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kv_rsrc(const T *P, int64_t ld, uint32_t Nk,
                                                          uint32_t blk) {
    const bool in = blk * BC < Nk;
    const uint32_t r0 = in ? blk * BC : 0;
    const uint32_t bytes = (uint32_t)(((Nk - 1 - r0) * ld + D) * sizeof(T));
    return phx_rsrc(P + (int64_t)r0 * ld, bytes & (0u - (uint32_t)in));  // no branch
}

// Scores of keys past Nk in a partial last block become -inf (p = 0): the
// score accumulators start from this bias (0 for a key that exists, -inf
// past Nk) instead of zero, so the masked scores come straight out of the
// MFMA chain with no register beyond the accumulators.  A lane's score
// register r of tile t holds key 32t + 8(r/4) + 4g + r%4 (both precisions'
// S^T layouts).  kv: keys of the block that exist, 0 < kv <= 64.  A per-lane
// limit and a bit select keep the compiler from materialising 32 key indices
// and compare masks, and the empty asm keeps it from hoisting the 32 bias
// values (loop-invariant when kv is) to the kernel's entry, where they would
// stay live, and spill, across the whole key loop.
__device__ __forceinline__ void key_bias(phx_f16v (&sc)[2], uint32_t kv, uint32_t g) {
    int32_t lim = (int32_t)kv - 4 * (int32_t)g;  // key 32t+8(r/4)+r%4 must be < lim
    asm volatile("" : "+v"(lim));
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int32_t c = 32 * t + 8 * (r >> 2) + (r & 3);
            const uint32_t keep = (uint32_t)((c - lim) >> 31);  // all ones when c < lim
            sc[t][r] = __builtin_bit_cast(float, 0xff800000u & ~keep);
        }
}

// The same mask applied to finished scores (the f32 kernel, whose score
// accumulators start from the MFMA's inline zero on every full block).  A
// plain select on the element value: a __builtin_bit_cast of a vector
// element lvalue was compiled as a read of element 0.
__device__ __forceinline__ void mask_keys(phx_f16v (&sc)[2], uint32_t kv, uint32_t g) {
    int32_t lim = (int32_t)kv - 4 * (int32_t)g;
    asm volatile("" : "+v"(lim));
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float x = sc[t][r];
            sc[t][r] = 32 * t + 8 * (r >> 2) + (r & 3) < lim ? x : -__builtin_inff();
        }
}

// The softmax is evaluated as exp2(s * c2 - m2) with c2 = scale * log2e.  A
// negative scale is folded into Q (q -> -q, exact), so that c2 > 0 and the
// row max of s * c2 is c2 times the row max of s; c2 is at least FLT_MIN so
// a masked key's -inf score never meets a zero factor (scale 0 then gives
// equal weights, as exp(0 * s) does).
__device__ __forceinline__ float softmax_c2(float scale) {
    return fmaxf(fabsf(scale) * LOG2E, 1.17549435e-38f);
}

#ifdef PHX_FLASH_F16
// ---------------------------------------------------------------- f16 path
// 256 queries per workgroup: 8 waves x 32 queries, two workgroups per CU, so
// each SIMD holds four waves of at most 128 registers.  A wave's softmax is a
// chain of dependent VALU ops (fma -> exp -> cvt -> dot2) whose latency one
// or two waves per SIMD cannot hide; with four, the SIMD always has a wave
// ready to issue an MFMA while the others run their softmax.  Per 64-key
// block a wave runs 16 MFMAs (S^T: 8, O^T += V^T.P^T: 8) on 16 KiB of K/V
// operands read from LDS.
//
// K and V blocks are copied global -> LDS directly (buffer_load ... lds, 16
// bytes per lane; each wave copies 8 rows of K and 8 of V) into a ring of 4
// stages (K 8 KiB + V 8 KiB each): block i+3 is issued during block i (after
// its softmax), and one barrier per block publishes it.
#define WQ 32                  // queries per wave
#define NWAVE 8
#define QB (NWAVE * WQ)        // queries per workgroup
#define KV_ROW 128             // bytes per K or V row (64 f16)
#define KV_TILE (BC * KV_ROW)  // 8 KiB
#define STAGE_BYTES (2 * KV_TILE)
#define NSTAGE 4
#define DMA_PER_BLK 2          // copies per wave per key block (K + V)

typedef __fp16 phx_fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) phx_fp16x4 *phx_lds_h4p;

#define PHX_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (((n) >> 4) << 14))

#define SGB(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
#define G_MFMA 0x008
#define G_DSR 0x100

// K rows are read as b128 MFMA operands (16 lanes = 16 rows, one chunk):
// XOR the chunk with (row>>1)&7.  V rows are read with ds_read_b64_tr_b16 (a
// 32-lane group touches 4 consecutive rows x 64 bytes): rows 2 apart are
// shifted by 64 bytes.
__device__ __forceinline__ uint32_t k_off(uint32_t row, uint32_t chunk) {
    return row * KV_ROW + ((chunk ^ ((row >> 1) & 7)) << 4);
}
__device__ __forceinline__ uint32_t v_off(uint32_t row, uint32_t chunk) {
    return row * KV_ROW + ((chunk ^ (((row >> 1) & 1) << 2)) << 4);
}

// Copies K and V rows wave*8 .. +7 of key block blk into stage dst.  Lane l
// lands at LDS row wave*8 + l/8, physical chunk l%8; its source (vk, vv) is
// the logical chunk stored there.  Rows past Nk read zeros; blocks past the
// end read an empty buffer into a stage that is never consumed.
__device__ __forceinline__ void dma_block(char *dst, const T *Kp, const T *Vp, int64_t ldk,
                                          int64_t ldv, uint32_t Nk, uint32_t blk, uint32_t vk,
                                          uint32_t vv, uint32_t wave) {
    const __amdgpu_buffer_rsrc_t rk = kv_rsrc(Kp, ldk, Nk, blk);
    const __amdgpu_buffer_rsrc_t rv = kv_rsrc(Vp, ldv, Nk, blk);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (phx_lds_vp)(dst + wave * 8 * KV_ROW), 16, vk,
                                             (int)((uint32_t)(wave * 8 * ldk) * 2), 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (phx_lds_vp)(dst + KV_TILE + wave * 8 * KV_ROW),
                                             16, vv, (int)((uint32_t)(wave * 8 * ldv) * 2), 0, 0);
}

// RESCALE_SLACK: the running max is raised only when a row's block max
// exceeds it by more than 8 (log2 units), so the O/l rescale is skipped on
// almost every block; p = exp2(s*c2 - m2) then stays <= 2^8, which f16 P and
// f32 l hold as well as the reference's per-block update.  O = acc / l is the
// same quantity either way.
// Fast path: the row max is not computed on a block unless it is needed.  A
// lane's 32 p are computed at once with the current m2; when their sum is at
// most 2^8 no p exceeds 2^8 and the block needs no max.  Otherwise (a
// wave-uniform branch, rare after the first block) the row max is taken, rows
// whose max exceeds the slack are raised to it, their p recomputed and acc
// and l rescaled.  The first key block always takes the max: m2 starts at the
// first block's row max, as after the reference's first per-block update from
// m = -65504.
#define RESCALE_SLACK 8.0f
#define FAST_SUM_LIMIT 256.0f  // 2^RESCALE_SLACK

struct Flash16 {
    phx_f16v acc[2];  // [d tile]: d = 32dt + 8(r/4) + 4g + r%4, query lq
    float m2;         // running max (log2 units) of the lane's query
    float l;          // row sum over this lane's half of the keys; lanes l and
                      // l^32 hold the two halves of one query's sum, which
                      // are added once, after the last block
    phx_h8 qf[4];     // Q^T operand, d slice s: d = 16s + 8g .. +7
};

// S^T: s[t] holds keys 32t + 8(r/4) + 4g + r%4 of query lq.  K operands:
// K row 32t + lq, d 16s + 8g .. +7.  Two chains over the d slices.
// BIAS: the chain starts from sc's current contents (key_bias), else from 0.
template <bool BIAS = false>
__device__ __forceinline__ void scores(phx_f16v (&sc)[2], const char *Ks, const Flash16 &fs,
                                       uint32_t lq, uint32_t g) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const phx_h8 kf = *(const phx_h8 *)(Ks + k_off(32 * t + lq, 2 * s + g));
            sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                kf, fs.qf[s],
                (s || BIAS) ? sc[t] : (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}, 0,
                0, 0);
        }
    // each K operand is read two MFMAs ahead of its use, not all at once:
    // the wave has 128 registers
    SGB(G_DSR, 2);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        SGB(G_MFMA, 1);
        if (m < 6) SGB(G_DSR, 1);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// V^T operand for keys 16c + (4g + 0..3, 8 + 4g + 0..3) (the order P's
// registers have) and d rows 32dt + lane%32: two transposing 4-key reads.
__device__ __forceinline__ phx_h8 read_v(const char *Vs, int c, int dt, uint32_t lane) {
    const uint32_t q = lane >> 4, sl = lane & 15;
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
    return (phx_h8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// O^T += V^T . P^T, V^T operands from the stage's V block.
__device__ __forceinline__ void pv(phx_f16v (&acc)[2], const char *Vs, const phx_h8 (&pf)[4],
                                   uint32_t lane) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
            acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(read_v(Vs, c, dt, lane), pf[c], acc[dt],
                                                             0, 0, 0);
    SGB(G_DSR, 4);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        SGB(G_MFMA, 1);
        if (m < 6) SGB(G_DSR, 2);
    }
    __builtin_amdgcn_sched_barrier(0);
}

// exp2(s*c2 - m2) as f16 MFMA operands pf[c] (keys 16c + ...), and the sum
// of the f32 p values before their rounding to f16, as the reference sums
// l over the f32 P (examples/flash_attention_fp16.ph:37-38: s = exp(s -
// mnew); l += rowsum(s); P is rounded to f16 only for P.V).
__device__ __forceinline__ float softmax_p(phx_h8 (&pf)[4], const phx_f16v (&s)[2], float c2,
                                           float m2) {
    float part[4];  // one partial sum per key slice: four short dependency chains
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        phx_h8 v;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[c >> 1][8 * (c & 1) + j], c2, -m2));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[c >> 1][8 * (c & 1) + j + 1], c2, -m2));
            part[c] = j == 0 ? p0 + p1 : (part[c] + p0) + p1;
            const phx_h2 pp = {(_Float16)p0, (_Float16)p1};
            v[j] = pp.x;
            v[j + 1] = pp.y;
        }
        pf[c] = v;
    }
    return (part[0] + part[1]) + (part[2] + part[3]);
}

// max over a lane's 32 scores (a running chain, which the compiler turns into
// v_max3_f32), then across the two lane halves.
__device__ __forceinline__ float row_max(const phx_f16v (&s)[2]) {
    float m = s[0][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) m = fmaxf(m, s[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) m = fmaxf(m, s[1][r]);
    return xor32_max(m);
}

// One key block i: scores, fast-path P, P.V, and (rarely) the slow path,
// which recomputes the scores from the K block still in LDS so they need not
// stay live through P.V.
template <bool FIRST>
__device__ __forceinline__ void flash16_step(Flash16 &fs, const char *cur, char *fill,
                                             const T *Kp, const T *Vp, int64_t ldk, int64_t ldv,
                                             uint32_t Nk, uint32_t i, float c2, uint32_t vk,
                                             uint32_t vv, uint32_t wave, uint32_t lane) {
    const uint32_t lq = lane & 31, g = lane >> 5;
    PHX_WAIT_VM_LGKM0((NSTAGE - 2) * DMA_PER_BLK);  // own copies of block i landed
    __builtin_amdgcn_s_barrier();                     // everyone's block i landed, i-1 done
    __builtin_amdgcn_sched_barrier(0);
    phx_f16v sc[2];
    phx_h8 pf[4];
    if constexpr (FIRST) {  // m2 starts at block 0's row max: no fast path to try
        key_bias(sc, Nk < BC ? Nk : BC, g);  // block 0 may be partial: keys past Nk are -inf
        scores<true>(sc, cur, fs, lq, g);
        const float mx = row_max(sc) * c2;  // log2 units
        const float ps = softmax_p(pf, sc, c2, mx);
        dma_block(fill, Kp, Vp, ldk, ldv, Nk, i + NSTAGE - 1, vk, vv, wave);
        fs.m2 = mx;
        fs.l += ps;
        pv(fs.acc, cur + KV_TILE, pf, lane);
        return;
    }
    scores(sc, cur, fs, lq, g);
    float ps = softmax_p(pf, sc, c2, fs.m2);
    // block i+3's copies go out between the softmax and P.V, not at the top
    // of the step next to the score MFMAs' K reads: 298.6 against 306.1 us
    // on average over five alternations on one box, bit-identical
    dma_block(fill, Kp, Vp, ldk, ldv, Nk, i + NSTAGE - 1, vk, vv, wave);
    const bool slow = __ballot(!(ps <= FAST_SUM_LIMIT));  // wave-uniform; NaN too
    if (slow) {
#pragma unroll
        for (int c = 0; c < 4; ++c) pf[c] = (phx_h8){0, 0, 0, 0, 0, 0, 0, 0};
    } else {
        fs.l += ps;
    }
    pv(fs.acc, cur + KV_TILE, pf, lane);
    if (slow) {
        scores(sc, cur, fs, lq, g);
        const float mx = row_max(sc) * c2;  // block row max, log2 units
        const float m2n = mx > fs.m2 + RESCALE_SLACK ? mx : fs.m2;
        ps = softmax_p(pf, sc, c2, m2n);
        const float corr = __builtin_amdgcn_exp2f(fs.m2 - m2n);  // 1 where not raised
        fs.l = fs.l * corr;
        fs.acc[0] = fs.acc[0] * corr;
        fs.acc[1] = fs.acc[1] * corr;
        fs.m2 = m2n;
        fs.l += ps;
        pv(fs.acc, cur + KV_TILE, pf, lane);
    }
}

// The partial last key block after at least one full one (kv < 64 keys
// exist), outside the pipelined loop so the masking costs the full blocks
// nothing: scores start from the key bias (-inf past Nk), then the plain
// per-block update with the row max.  No copies are issued; all earlier ones
// are drained first.
__device__ __forceinline__ void flash16_last(Flash16 &fs, const char *cur, uint32_t kv, float c2,
                                             uint32_t lane) {
    const uint32_t lq = lane & 31, g = lane >> 5;
    PHX_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    phx_f16v sc[2];
    key_bias(sc, kv, g);
    scores<true>(sc, cur, fs, lq, g);
    const float mx = row_max(sc) * c2;  // finite: key 0 always exists
    const float m2n = mx > fs.m2 + RESCALE_SLACK ? mx : fs.m2;
    phx_h8 pf[4];
    const float ps = softmax_p(pf, sc, c2, m2n);
    const float corr = __builtin_amdgcn_exp2f(fs.m2 - m2n);
    fs.l = fs.l * corr;
    fs.acc[0] = fs.acc[0] * corr;
    fs.acc[1] = fs.acc[1] * corr;
    fs.m2 = m2n;
    fs.l += ps;
    pv(fs.acc, cur + KV_TILE, pf, lane);
}

// One block of queries q0 .. q0 + 255 over keys 0 .. Nk-1.  PART: instead of
// O, store each query's unnormalised accumulator (64 f32 at pacc + 64 q) and
// its running max (log2 units) and row sum (pml + 2 q), for flash_combine.
template <bool PART>
__device__ __forceinline__ void flash_block(const T *Q, const T *Kp, const T *Vp, T *O,
                                            int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                                            uint32_t Nq, uint32_t Nk, uint32_t q0, float scale,
                                            char *st,
                                            float *pacc, float *pml) {
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lq = lane & 31, g = lane >> 5;
    const uint32_t qw = q0 + wave * WQ;  // first query of this wave
    const float c2 = softmax_c2(scale);
    const uint32_t nkb = (Nk + BC - 1) / BC;
    char *S[NSTAGE];  // stage b % NSTAGE holds key block b
#pragma unroll
    for (int k = 0; k < NSTAGE; ++k) S[k] = st + k * STAGE_BYTES;

    // per-lane source offsets of the LDS copies (see dma_block): the K
    // swizzle depends on bit 2 of the row, i.e. on the wave's parity
    const uint32_t vk = (uint32_t)(((lane >> 3) * ldk +
                                    8 * ((lane & 7) ^ (4 * (wave & 1) + ((lane >> 4) & 3)))) * 2);
    const uint32_t vv =
        (uint32_t)(((lane >> 3) * ldv + 8 * ((lane & 7) ^ (((lane >> 4) & 1) << 2))) * 2);

#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) dma_block(S[p], Kp, Vp, ldk, ldv, Nk, p, vk, vv, wave);

    Flash16 fs;
    // Q rows past Nq read as zeros (their outputs are not stored)
    const __amdgpu_buffer_rsrc_t rq = phx_rsrc(Q, (uint32_t)(((Nq - 1) * ldq + D) * 2));
#pragma unroll
    for (int s = 0; s < 4; ++s)
        fs.qf[s] = __builtin_bit_cast(
            phx_h8, __builtin_amdgcn_raw_buffer_load_b128(
                        rq, (int)(((qw + lq) * ldq + 16 * s + 8 * g) * 2), 0, 0));
    if (scale < 0.0f) {  // wave-uniform
#pragma unroll
        for (int s = 0; s < 4; ++s) fs.qf[s] = -fs.qf[s];
    }
    fs.acc[0] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    fs.acc[1] = fs.acc[0];
    fs.m2 = M_INIT * LOG2E;  // replaced by the first block's row max
    fs.l = 0.0f;

    // block b lives in stage b % 4; the copy of block b + 3 goes into stage (b + 3) % 4.
    // The full blocks run pipelined; a partial last block (Nk % 64 keys) follows.
    // Block 0 (the first step, whose scores are masked when Nk < 64) always runs.
    const uint32_t nfull = Nk / BC;
    flash16_step<true>(fs, S[0], S[NSTAGE - 1], Kp, Vp, ldk, ldv, Nk, 0, c2, vk, vv, wave, lane);
    uint32_t i = 1;
    for (; i + NSTAGE <= nfull; i += NSTAGE) {
        flash16_step<false>(fs, S[1], S[0], Kp, Vp, ldk, ldv, Nk, i, c2, vk, vv, wave, lane);
        flash16_step<false>(fs, S[2], S[1], Kp, Vp, ldk, ldv, Nk, i + 1, c2, vk, vv, wave, lane);
        flash16_step<false>(fs, S[3], S[2], Kp, Vp, ldk, ldv, Nk, i + 2, c2, vk, vv, wave, lane);
        flash16_step<false>(fs, S[0], S[3], Kp, Vp, ldk, ldv, Nk, i + 3, c2, vk, vv, wave, lane);
    }
    if (i < nfull)
        flash16_step<false>(fs, S[1], S[0], Kp, Vp, ldk, ldv, Nk, i, c2, vk, vv, wave, lane);
    if (i + 1 < nfull)
        flash16_step<false>(fs, S[2], S[1], Kp, Vp, ldk, ldv, Nk, i + 1, c2, vk, vv, wave, lane);
    if (i + 2 < nfull)
        flash16_step<false>(fs, S[3], S[2], Kp, Vp, ldk, ldv, Nk, i + 2, c2, vk, vv, wave, lane);
    if (nfull > 0 && nfull < nkb) {  // wave-uniform
        const uint32_t kv = Nk - nfull * BC;
        flash16_last(fs, st + (nfull % NSTAGE) * STAGE_BYTES, kv, c2, lane);
    }
    // drain the copies of the blocks past the end before the LDS is reused
    PHX_WAIT_VMCNT(0);
    __syncthreads();

    // acc[dt][r]: d = 32dt + 8(r/4) + 4g + r%4, query qw + lq.
    fs.l = xor32_add(fs.l);  // both halves of the query's row sum
    const uint32_t q = qw + lq;
    if (PART && q < Nq) {
        float *arow = pacc + (int64_t)q * D;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                *(phx_f4 *)(arow + 32 * dt + 8 * b + 4 * g) =
                    (phx_f4){fs.acc[dt][4 * b], fs.acc[dt][4 * b + 1], fs.acc[dt][4 * b + 2],
                             fs.acc[dt][4 * b + 3]};
        if (g == 0) *(float2 *)(pml + 2 * (int64_t)q) = make_float2(fs.m2, fs.l);
    } else if (q < Nq) {
        T *orow = O + (int64_t)q * ldo;
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
}
#else
// ---------------------------------------------------------------- f32 path
// V^T rows are stored 4 apart by one instruction (the register transpose,
// rows 4dq + r) and read 16 consecutive at a time (the MFMA operands): XOR
// the chunk with ((row >> 2) ^ (row << 2)) & 15, i.e. the row's two 2-bit
// fields swapped.  SQ_LDS_BANK_CONFLICT reads 0 for both access sets with
// it on gfx950 (LDS microbenchmark of exactly these two patterns); row & 15
// costs the stores 24 conflict cycles per instruction, and (row ^ row>>2) & 15
// costs the reads 4, although both map each 16-lane group to 16 distinct
// 16-byte slots.
__device__ __forceinline__ uint32_t vt_off(uint32_t row, uint32_t chunk) {
    return row * ROW_BYTES + ((chunk ^ (((row >> 2) ^ (row << 2)) & 15)) << 4);
}
// K rows / V^T rows are 64 floats (256 B, 16 chunks).  K is copied global ->
// LDS directly (buffer_load ... lds: a 64-lane copy fills 4 rows; lane l lands
// at row r = l/16 (+4c), physical chunk l%16 and fetches the logical chunk
// (l%16) ^ (r & 15) stored there), 4 copies per wave, through a resource that
// ends at key Nk (rows past it read zero).  V^T is staged by all 256 threads,
// one 4x4 register transpose each: keys 4kq .. +3, d = 4dq .. +3.  In a
// partial last block V rows past Nk repeat row Nk-1 (finite; those keys'
// scores are masked to -inf, so their p is 0).
struct Stage {
    phx_f4 r[4];
};

__device__ __forceinline__ void dma_k(char *Ks, const T *Kp, int64_t ldk, uint32_t Nk,
                                      uint32_t blk, const uint32_t (&vk)[4], uint32_t wave) {
    const __amdgpu_buffer_rsrc_t rk = kv_rsrc(Kp, ldk, Nk, blk);
#pragma unroll
    for (int c = 0; c < 4; ++c)  // rows 16 wave + 4c .. +3
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rk, (phx_lds_vp)(Ks + (16 * wave + 4 * c) * ROW_BYTES), 16, vk[c],
            (int)((uint32_t)((16 * wave + 4 * c) * ldk) * 4), 0, 0);
}

template <bool CLAMP>
__device__ __forceinline__ void load_v_rows(Stage &st, const T *Vp, int64_t ldv, uint32_t Nk,
                                            uint32_t key0, uint32_t tid) {
    const uint32_t dq = tid & 15, kq = tid >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = key0 + 4 * kq + i;
        st.r[i] = *(const phx_f4 *)(Vp + (int64_t)(CLAMP ? (r < Nk ? r : Nk - 1) : r) * ldv + 4 * dq);
    }
}

__device__ __forceinline__ void load_v(Stage &st, const T *Vp, int64_t ldv, uint32_t Nk,
                                       uint32_t blk, uint32_t tid) {
    const uint32_t key0 = blk * BC;
    if (key0 + BC <= Nk)  // wave-uniform
        load_v_rows<false>(st, Vp, ldv, Nk, key0, tid);
    else
        load_v_rows<true>(st, Vp, ldv, Nk, key0, tid);
}

__device__ __forceinline__ void store_v(const Stage &st, char *Vt, uint32_t tid) {
    const uint32_t dq = tid & 15, kq = tid >> 4;  // keys 4*kq .. +3 = V^T chunk kq
    const phx_f4 *b = st.r;
    const phx_f4 c0 = {b[0].x, b[1].x, b[2].x, b[3].x};
    const phx_f4 c1 = {b[0].y, b[1].y, b[2].y, b[3].y};
    const phx_f4 c2 = {b[0].z, b[1].z, b[2].z, b[3].z};
    const phx_f4 c3 = {b[0].w, b[1].w, b[2].w, b[3].w};
    *(phx_f4 *)(Vt + vt_off(4 * dq + 0, kq)) = c0;
    *(phx_f4 *)(Vt + vt_off(4 * dq + 1, kq)) = c1;
    *(phx_f4 *)(Vt + vt_off(4 * dq + 2, kq)) = c2;
    *(phx_f4 *)(Vt + vt_off(4 * dq + 3, kq)) = c3;
}

#define RESCALE_SLACK 8.0f

// One block of queries q0 .. q0 + 127 over keys 0 .. Nk-1; PART as in the
// f16 path.
template <bool PART>
__device__ __forceinline__ void flash_block(const T *Q, const T *Kp, const T *Vp, T *O,
                                            int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo,
                                            uint32_t Nq, uint32_t Nk, uint32_t q0, float scale,
                                            char (*lds)[2][TILE_BYTES], float *pacc, float *pml) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t lq = lane & 31, g = lane >> 5;
    const uint32_t myq = q0 + wave * 32 + lq;
    const float c2 = softmax_c2(scale);

    // Q^T operand: MFMA (q', s) uses d = 8q' + 4g + s.  Rows past Nq read
    // zeros (their outputs are not stored).
    const __amdgpu_buffer_rsrc_t rq = phx_rsrc(Q, (uint32_t)(((Nq - 1) * ldq + D) * 4));
    const float qsign = scale < 0.0f ? -1.0f : 1.0f;  // exact
    phx_f4 qf[8];
#pragma unroll
    for (int qq = 0; qq < 8; ++qq)
        qf[qq] = qsign * __builtin_bit_cast(phx_f4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        rq, (int)((myq * ldq + 8 * qq + 4 * g) * 4), 0, 0));

    phx_f16v acc[2];
    acc[0] = (phx_f16v){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    acc[1] = acc[0];
    float m2 = M_INIT * LOG2E;
    float l = 0.0f;

    const uint32_t nkb = (Nk + BC - 1) / BC;
    // K copy sources of this lane: row lane/16 of copy c's 4-row group (rows
    // 16 wave + 4c + lane/16, so row & 15 = 4c + lane/16), logical chunk
    // (lane%16) ^ (row & 15)
    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    uint32_t vk[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        vk[c] = (uint32_t)(((lane >> 4) * ldk + 4 * ((lane & 15) ^ (4 * c + (lane >> 4)))) * 4);
    Stage st;
    dma_k(lds[0][0], Kp, ldk, Nk, 0, vk, wv);
    load_v(st, Vp, ldv, Nk, 0, tid);
    store_v(st, lds[0][1], tid);
    PHX_WAIT_VMCNT(0);
    __syncthreads();

    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const uint32_t cur = kb & 1;
        if (kb + 1 < nkb) {
            dma_k(lds[cur ^ 1][0], Kp, ldk, Nk, kb + 1, vk, wv);
            load_v(st, Vp, ldv, Nk, kb + 1, tid);
        }
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
        const uint32_t kv = Nk - kb * BC;  // keys of this block that exist (uniform)
        if (kv < BC) mask_keys(sT, kv, g);  // partial last block only
        float mx = sT[0][0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sT[0][r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sT[1][r]);
        mx = xor32_max(mx) * c2;
        // Lazy rescale: the running max is raised only when the block max
        // exceeds it by more than 8 (log2 units), so p <= 2^8 and O and l are
        // rescaled only on the rare block that raises some row's max.
        const bool raise = kb == 0 || mx > m2 + RESCALE_SLACK;
        const float m2new = raise ? mx : m2;
        float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sT[t][r], c2, -m2new));
                part[r & 3] += p;
                sT[t][r] = p;
            }
        if (__ballot(raise)) {  // wave-uniform
            const float corr = __builtin_amdgcn_exp2f(m2 - m2new);  // 1 where not raised
            l = l * corr;
            acc[0] = acc[0] * corr;
            acc[1] = acc[1] * corr;
        }
        l += xor32_add((part[0] + part[1]) + (part[2] + part[3]));
        m2 = m2new;
        // P^T operand: lane holds keys 32t + 8b + 4g + s = sT[t][4b + s];
        // V^T row d, chunk (8t + 2b + g) holds keys 32t + 8b + 4g .. +3.
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    phx_f4 vf = *(const phx_f4 *)(Vt + vt_off(32 * dt + lq, 8 * t + 2 * b + g));
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[s], sT[t][4 * b + s],
                                                                       acc[dt], 0, 0, 0);
                }

        if (kb + 1 < nkb) store_v(st, lds[cur ^ 1][1], tid);
        PHX_WAIT_VMCNT(0);  // this wave's K copies of block kb+1 landed
        __syncthreads();
    }

    if (myq >= Nq) return;
    if (PART) {
        float *arow = pacc + (int64_t)myq * D;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                *(phx_f4 *)(arow + 32 * dt + 8 * b + 4 * g) =
                    (phx_f4){acc[dt][4 * b], acc[dt][4 * b + 1], acc[dt][4 * b + 2],
                             acc[dt][4 * b + 3]};
        if (g == 0) *(float2 *)(pml + 2 * (int64_t)myq) = make_float2(m2, l);
        return;
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

#ifdef PHX_FLASH_F16
#define FA_QB QB  // queries per workgroup
// one array, so every stage address is a constant offset from one base
#define FA_LDS_DECL __shared__ __attribute__((aligned(16))) char st[NSTAGE][STAGE_BYTES];
#define FA_CALL(Qp, Kp, Vp, Op, ldq, ldk, ldv, ldo, Nq, Nk, q0) \
    flash_block<false>(Qp, Kp, Vp, Op, ldq, ldk, ldv, ldo, Nq, Nk, q0, scale, &st[0][0], nullptr, \
                       nullptr)
#define FA_CALL_PART(Qp, Kp, Vp, ldq, ldk, ldv, Nq, Nk, q0, pacc, pml)                    \
    flash_block<true>(Qp, Kp, Vp, nullptr, ldq, ldk, ldv, 0, Nq, Nk, q0, scale, &st[0][0], pacc, \
                      pml)
#else
#define FA_QB BR
#define FA_LDS_DECL __shared__ __attribute__((aligned(16))) char lds[2][2][TILE_BYTES];
#define FA_CALL(Qp, Kp, Vp, Op, ldq, ldk, ldv, ldo, Nq, Nk, q0) \
    flash_block<false>(Qp, Kp, Vp, Op, ldq, ldk, ldv, ldo, Nq, Nk, q0, scale, lds, nullptr, nullptr)
#define FA_CALL_PART(Qp, Kp, Vp, ldq, ldk, ldv, Nq, Nk, q0, pacc, pml) \
    flash_block<true>(Qp, Kp, Vp, nullptr, ldq, ldk, ldv, 0, Nq, Nk, q0, scale, lds, pacc, pml)
#endif

extern "C" __global__ __launch_bounds__(NT, FA_WAVES_PER_SIMD) void flash_attention(PHX_MEMREF2(T, q, int64_t),
                                                                  PHX_MEMREF2(T, k, int64_t),
                                                                  PHX_MEMREF2(T, v, int64_t),
                                                                  PHX_MEMREF2(T, o, int64_t),
                                                                  float scale) {
    FA_LDS_DECL
    const int64_t Nq = q_s0, Nk = k_s0;
    if (blockDim.x != NT || q_s1 != D || k_s1 != D || v_s1 != D || o_s1 != D || v_s0 != Nk ||
        o_s0 != Nq || Nq <= 0 || Nk <= 0 || q_st1 != 1 || k_st1 != 1 || v_st1 != 1 ||
        o_st1 != 1 || (q_st0 | k_st0 | v_st0 | o_st0) % 8 || Nq * q_st0 * 4 > INT32_MAX ||
        Nk * (k_st0 > v_st0 ? k_st0 : v_st0) * 4 > INT32_MAX)
        return;
    const uint32_t nrb = (uint32_t)((Nq + FA_QB - 1) / FA_QB);
    for (uint32_t rb = phx_block_linear(); rb < nrb; rb += phx_block_count())
        FA_CALL(q_ptr + q_off, k_ptr + k_off, v_ptr + v_off, o_ptr + o_off, q_st0, k_st0, v_st0,
                o_st0, (uint32_t)Nq, (uint32_t)Nk, rb * FA_QB);
}

extern "C" __global__ __launch_bounds__(NT, FA_WAVES_PER_SIMD) void flash_attention_bh(PHX_MEMREF3(T, q, int64_t),
                                                                     PHX_MEMREF3(T, k, int64_t),
                                                                     PHX_MEMREF3(T, v, int64_t),
                                                                     PHX_MEMREF3(T, o, int64_t),
                                                                     float scale) {
    FA_LDS_DECL
    const int64_t H = q_s0, Nq = q_s1, Nk = k_s1;
    if (blockDim.x != NT || k_s0 != H || v_s0 != H || o_s0 != H || q_s2 != D || k_s2 != D ||
        v_s2 != D || o_s2 != D || v_s1 != Nk || o_s1 != Nq || Nq <= 0 || Nk <= 0 || H <= 0 ||
        q_st2 != 1 || k_st2 != 1 || v_st2 != 1 || o_st2 != 1 ||
        (q_st1 | k_st1 | v_st1 | o_st1 | q_st0 | k_st0 | v_st0 | o_st0) % 8 ||
        Nq * q_st1 * 4 > INT32_MAX || Nk * (k_st1 > v_st1 ? k_st1 : v_st1) * 4 > INT32_MAX)
        return;
    const uint32_t nrb = (uint32_t)((Nq + FA_QB - 1) / FA_QB);
    const uint32_t nwork = nrb * (uint32_t)H;
    const uint32_t nblk = phx_block_count();
    for (uint32_t w = phx_block_linear(); w < nwork; w += nblk) {
        const uint32_t ws = nblk == nwork ? phx_xcd_swizzle(w, nwork) : w;
        const uint32_t h = ws / nrb, rb = ws % nrb;
        FA_CALL(q_ptr + q_off + h * q_st0, k_ptr + k_off + h * k_st0, v_ptr + v_off + h * v_st0,
                o_ptr + o_off + h * o_st0, q_st1, k_st1, v_st1, o_st1, (uint32_t)Nq, (uint32_t)Nk,
                rb * FA_QB);
    }
}

// Split keys, for launches with too few query blocks to fill the GPU (the
// host picks the split; see phx_runtime.cpp).  Workgroup (x, y) runs query
// block x % nrb of head x / nrb over keys [y * kchunk, min(Nk, (y+1) * kchunk))
// and stores each query's unnormalised accumulator, running max and row sum
// into the workspace W, laid out for splits s, heads h, queries q as
//   acc: W[((s * BH + h) * Nq + q) * 64 + d]
//   m, l: W[nsplit * BH * Nq * 64 + ((s * BH + h) * Nq + q) * 2 + {0, 1}].
// Each chunk is the same online softmax over its own keys (kchunk is a
// multiple of the 64-key block), so flash_combine only has to merge them.
// Head strides hq, hk, hv are in elements (0 for one head).
extern "C" __global__ __launch_bounds__(NT, FA_WAVES_PER_SIMD) void flash_attention_split(
    const T *Qb, const T *Kb, const T *Vb, float *W, int64_t BH, int64_t Nq, int64_t Nk,
    int64_t ldq, int64_t ldk, int64_t ldv, int64_t hq, int64_t hk, int64_t hv, int64_t kchunk,
    int32_t nsplit, float scale) {
    FA_LDS_DECL
    const uint32_t nrb = (uint32_t)((Nq + FA_QB - 1) / FA_QB);
    const int64_t k0 = (int64_t)blockIdx.y * kchunk;
    if (blockDim.x != NT || blockIdx.x >= nrb * (uint32_t)BH || k0 >= Nk || kchunk % BC) return;
    const uint32_t h = blockIdx.x / nrb, rb = blockIdx.x % nrb;
    const int64_t nk = Nk - k0 < kchunk ? Nk - k0 : kchunk;
    const int64_t plane = ((int64_t)blockIdx.y * BH + h) * Nq;
    float *pacc = W + plane * D;
    float *pml = W + (int64_t)nsplit * BH * Nq * D + plane * 2;
    FA_CALL_PART(Qb + h * hq, Kb + h * hk + k0 * ldk, Vb + h * hv + k0 * ldv, ldq, ldk, ldv,
                 (uint32_t)Nq, (uint32_t)nk, rb * FA_QB, pacc, pml);
}

// Merges the nsplit partial results of flash_attention_split: per query,
// M = max_s m_s, w_s = 2^(m_s - M), O = (sum_s w_s acc_s) / (sum_s w_s l_s),
// rounded once to T.  Four d of one query per thread; head stride ho and row
// stride ldo of O in elements.
extern "C" __global__ __launch_bounds__(256) void flash_combine(const float *W, int32_t nsplit,
                                                                T *O, int64_t BH, int64_t Nq,
                                                                int64_t ldo, int64_t ho) {
    const int64_t nq = BH * Nq, total = nq * (D / 4);
    const float *ml = W + (int64_t)nsplit * nq * D;
    for (int64_t i = (int64_t)phx_block_linear() * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)phx_block_count() * blockDim.x) {
        const int64_t hqi = i / (D / 4), d4 = i % (D / 4);
        float mx = ml[2 * hqi];
        for (int32_t s = 1; s < nsplit; ++s) mx = fmaxf(mx, ml[2 * (s * nq + hqi)]);
        float l = 0.0f;
        phx_f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int32_t s = 0; s < nsplit; ++s) {
            const float w = __builtin_amdgcn_exp2f(ml[2 * (s * nq + hqi)] - mx);
            l = l + w * ml[2 * (s * nq + hqi) + 1];
            acc = acc + w * *(const phx_f4 *)(W + (s * nq + hqi) * D + 4 * d4);
        }
        const int64_t h = hqi / Nq, q = hqi % Nq;
        T *dst = O + h * ho + q * ldo + 4 * d4;
#ifdef PHX_FLASH_F16
        *(phx_h4 *)dst = (phx_h4){(_Float16)(acc[0] / l), (_Float16)(acc[1] / l),
                                  (_Float16)(acc[2] / l), (_Float16)(acc[3] / l)};
#else
        *(phx_f4 *)dst = acc / l;
#endif
    }
}
