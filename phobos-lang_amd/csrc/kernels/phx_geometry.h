// Launch geometry shared by the gfx950 kernels and the host runtime.
//
// The reference derives each grid from the autotuned .ph tile sizes
// (phobos-bench/src/main.rs:500-508, 974-981, 1220-1223).  These kernels pick
// their own MI355X tiles, so the host asks phx_grid_for() instead; every
// kernel also walks its work items with a block-stride loop, so any grid the
// caller passes still computes the whole result.
#pragma once

// saxpy: 256 threads, each handling PHX_SAXPY_VEC float4 per block step.
#define PHX_SAXPY_THREADS 256
#ifndef PHX_SAXPY_VEC
#define PHX_SAXPY_VEC 4
#endif
#define PHX_SAXPY_BLOCK_ELEMS (PHX_SAXPY_THREADS * PHX_SAXPY_VEC * 4)

// GEMM shapes: M is any positive extent; N and K must be multiples of the
// element count of one 16-byte chunk of the operand type (4 for f32 storage,
// 8 for f16; K % 8 for gemm_fp16tc, whose lanes stage 8 k at a time), so
// every staged chunk is whole and every row starts 16-byte aligned.  Tiles crossing M, N or K are masked inside the kernels.  (The
// reference's own tiles need M and N multiples of 32 and K of its K tile.)

// f16-operand GEMMs (gemm_fp16, gemm_fp16tc_fp32acc): 256x256 output tile,
// K step 32, 256 threads = 4 waves in a 2x2 arrangement of 128x128.
#define PHX_H_BM 256
#define PHX_H_BN 256
#define PHX_H_BK 32
#define PHX_H_THREADS 256
#define PHX_TC_W8_THREADS 512  // gemm_w8, gemm_w8_splitk: the eight-wave tc kernels
#define PHX_TC_N_MULT 4    // gemm_fp16tc_fp32acc (f32 storage): N % 4, K % 8
#define PHX_TC_K_MULT 8
#define PHX_H16_NK_MULT 8  // gemm_fp16 (f16 storage): N % 8, K % 8

// f32 GEMM (gemm_fp32, cluster matmul): a workgroup computes a
// PHX_S_TILE x PHX_S_TILE output tile (4 waves of 128x128).
#define PHX_S_TILE 256
#define PHX_S_BK 16
#define PHX_S_THREADS 256
#define PHX_S_NK_MULT 4

// Split-K (gemm_fp32, gemm_fp16tc_fp32acc, gemm_fp16): when a GEMM has
// fewer than PHX_SPLIT_MIN_TILES output tiles of 256 x 256, its K range is
// cut into chunks of whole 32-deep steps computed by separate workgroups
// (gemm_splitk), whose f32 partial sums gemm_splitk_reduce adds in a fixed
// order.  gemm_fp32 aims at PHX_SPLIT_TARGET_F32 workgroups with chunks of
// at least PHX_SPLIT_MIN_STEPS_F32 steps; the f16 MFMA GEMMs, whose K steps
// are 8x cheaper, at PHX_SPLIT_TARGET_F16 workgroups with chunks of at least
// PHX_SPLIT_MIN_STEPS_F16 steps, or PHX_SPLIT_MIN_STEPS_F16_WIDE once a
// launch has PHX_SPLIT_WIDE_TILES tiles; at most PHX_SPLIT_MAX chunks.
// Measured on MI355X with the partial sums in a workspace the caller bound
// (HIP events, pinned split counts): gemm_fp16 512^3 16.6 us unsplit, 14.0
// at 2 chunks; 768^3 20.4 / 17.1 at 3; 1536^3 33.8 / 25.8 at 3; 512^2 x
// 2048 38.2 / 18.6 at 8; 256^2 x 4096 67.5 / 18.0 at 16; 2048^3 42.6 / 36.5
// at 2; and at 2048^2 x 1024 the split loses (26.5 / 28.5 at 2), as it does
// at 3072^2 x 1024 (31.5 / 53.8); gemm_fp16tc_fp32acc alike.
#define PHX_SPLIT_MIN_TILES 128
#define PHX_SPLIT_MAX 16
#define PHX_SPLIT_TARGET_F32 256
#define PHX_SPLIT_TARGET_F16 128
#define PHX_SPLIT_MIN_STEPS_F32 1
#define PHX_SPLIT_MIN_STEPS_F16 8
#define PHX_SPLIT_MIN_STEPS_F16_WIDE 32
#define PHX_SPLIT_WIDE_TILES 64
#define PHX_SPLIT_KSTEP 32

// gemm_fp32's built-in tiling (no pin): 256 x 256 x 16 when its tiles fill
// all PHX_S32_FULL_TILES CUs; else 64 x 64 x 16 (launch-plan variant
// PHX_S32_SMALL_VARIANT) when that gives at least PHX_S32_SMALL_MIN_TILES
// tiles, or at least PHX_S32_SMALL_SHORT_TILES with K <= PHX_S32_SHORT_K;
// else the split rule above.  Measured on MI355X (one box, HIP events): the
// small tile beats both the 256 x 256 tile and its split at 3072^2 x 1024
// (151 vs 260 us unsplit), 2048^3 (133 vs 160 split), 768^3 (18.5 vs 44),
// 1024^2 x 256 (9 vs 40) and 512^2 x 2048 (41 vs 58); the split stays ahead
// only with long K over few tiles (512^2 x 16384: 255 vs 300 us).
#define PHX_S32_FULL_TILES 256
#define PHX_S32_SMALL_VARIANT 7
#define PHX_S32_SMALL_TILE 64
#define PHX_S32_SMALL_MIN_TILES 128
#define PHX_S32_SMALL_SHORT_TILES 16
#define PHX_S32_SHORT_K 4096

#define PHX_REDUCE_THREADS 256

// Split keys (flash attention): when the (query block, head) work items
// cannot fill half of the PHX_FA_SLOTS workgroup slots (256 CUs x 2
// resident workgroups), the keys are cut into chunks of whole 64-key blocks
// run as separate workgroups (flash_attention_split) and merged by
// flash_combine: enough chunks for PHX_FLASH_SPLIT_TARGET workgroups, of at
// least PHX_FLASH_SPLIT_MIN_BLOCKS_F16 (f16) or _F32 (f32) blocks each, at
// most PHX_SPLIT_MAX.  Measured on MI355X with the partial results in a
// workspace the caller bound (HIP events, pinned chunk counts; best count
// in brackets): f16 one head 1024^2 16.2 us (3; 14.3 at 6) against 17.7 at the
// earlier rule's 2; 8192^2 34.4 (8) against 39.4 at 16; 4 heads 4096^2 32.2
// (4) against 36.3 at 8; f32 one head 1024^2 19.5 (8) against 41.2 at 2,
// 2048^2 27.0 (16) against 43.2 at 4.  One workgroup per CU (256) beat
// filling both slots of every CU, and short chunks beat the earlier floor of
// 8 blocks, whose tuning had a workspace allocation in every split launch.
#define PHX_FA_SLOTS 512
#define PHX_FLASH_SPLIT_TARGET 256
#define PHX_FLASH_SPLIT_MIN_BLOCKS_F16 5
#define PHX_FLASH_SPLIT_MIN_BLOCKS_F32 2
// Device bytes of the fixed scratch array behind the allocation-free flash
// entry point (phx_flash_attention_bh_noalloc): its split-key workspace.
#define PHX_SCRATCH_BYTES (16u << 20)

// matmul_init: element-wise, 256 threads x 4 float4.
#define PHX_EW_THREADS 256
#define PHX_EW_BLOCK_ELEMS (256 * 16)

// flash attention: any Nq >= 1 and Nk >= 1, D == 64; 64 keys per step (keys
// past Nk in the last step are masked out of the softmax).  f32: 128 query
// rows per workgroup (4 waves x 32).  f16: 256 query rows per workgroup (8
// waves x 32).  Query rows past Nq are computed from zero queries and not
// stored.
#define PHX_FA_BR 128
#define PHX_FA16_BR 256
#define PHX_FA_BC 64
#define PHX_FA_THREADS 256
#define PHX_FA16_THREADS 512  // f16: 8 waves x 32 queries
#define PHX_FA_D 64
