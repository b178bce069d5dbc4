/*
 * phobos_hip.h -- C ABI of the MI355X (gfx950) leaf-kernel backend.
 *
 * Everything is plain C: device addresses are uint64_t (the reference's
 * CUdeviceptr), streams and events are opaque handles, sizes are integers.
 * Every function returns 0 on success or a nonzero status (a HIP error code
 * where one exists, else PHX_E_*); phx_last_error() returns the message for
 * the calling thread.  No function here allocates device memory except the
 * ones named *_malloc / *_create, phx_init and the lazy load of a code object
 * on a kernel's first use (phx_module_load_*, phx_builtin_function, a
 * built-in's first launch).  Launches never allocate: a split launch's
 * partial results go to the caller-owned workspace bound to its stream
 * (phx_stream_set_workspace).
 *
 * The entry points replace, one for one, what the reference's host code does
 * through the cust CUDA driver API:
 *   - phobos-bench launches:  launch!(func<<<grid, block, 0, stream>>>(...))
 *       phobos-bench/src/main.rs:290-327 (gemm), 334-371 (flash),
 *       1227-1239 (saxpy)
 *   - phobos-pod COMPUTE:     Engine::launch, phobos-pod/src/engine.rs:542-653
 *   - module cache:           PtxCache, phobos-pod/src/ptx_cache.rs:12-82
 *   - device arena:           DeviceArena / TileStore,
 *                             phobos-pod/src/tile_store.rs:14-222
 *   - streams / events:       engine.rs:86, 172-174, 632-687
 */
#ifndef PHOBOS_HIP_H
#define PHOBOS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status codes */
#define PHX_OK 0
#define PHX_E_INVALID 1001     /* bad argument / shape the kernel does not take */
#define PHX_E_NOT_INIT 1002    /* phx_init not called */
#define PHX_E_NOT_FOUND 1003   /* code object or entry point missing */
#define PHX_E_EXHAUSTED 1004   /* arena exhausted (tile_store.rs:57-63) */
#define PHX_E_IO 1005          /* file:// storage error */
#define PHX_E_SEGMENT 1006     /* malformed segment / instruction */

/* ------------------------------------------------------------ kernel ids */
/* The leaf kernels of the reference examples (.ph files), one code object each; the entry name
 * inside is the .ph kernel name (main.rs:512, 761, 985, 1113, 1225;
 * clustergen.rs:1285, 1353). */
typedef enum {
    PHX_SAXPY_FP32 = 0,          /* saxpy_fp32.ph            entry "saxpy", i32 idx */
    PHX_GEMM_FP32 = 1,           /* gemm_fp32.ph             entry "gemm",  i32 idx */
    PHX_GEMM_FP16TC_FP32ACC = 2, /* gemm_fp16tc_fp32acc.ph   entry "gemm",  i64 idx */
    PHX_GEMM_FP16 = 3,           /* gemm_fp16.ph             entry "gemm",  i64 idx */
    PHX_FLASH_FP32 = 4,          /* flash_attention_fp32.ph  entry "flash_attention", i64 */
    PHX_FLASH_FP16 = 5,          /* flash_attention_fp16.ph  entry "flash_attention", i64 */
    PHX_MATMUL = 6,              /* matmul_cluster_fp32.ph step leaf "matmul", i32 */
    PHX_MATMUL_INIT = 7,         /* matmul_cluster_fp32.ph init leaf "matmul_init", i32 */
    PHX_FLASH_FP32_BH = 8,       /* "flash_attention_bh": [B*H, N, D] in one launch */
    PHX_FLASH_FP16_BH = 9,
    PHX_NUM_KERNELS = 10
} phx_kernel;

typedef void *phx_stream;   /* a hipStream_t; NULL = the legacy default stream */
typedef void *phx_event;    /* a hipEvent_t */
typedef void *phx_module;   /* a hipModule_t */
typedef void *phx_function; /* a hipFunction_t */
typedef struct phx_arena_s *phx_arena;

/* ------------------------------------------------------------ device */
/* cust::quick_init (main.rs:169).  Loads the built-in code objects from
 * code_object_dir (NULL: the directory holding this library, or
 * $PHX_CODE_OBJECT_DIR). */
int phx_init(int device, const char *code_object_dir);
int phx_shutdown(void);
const char *phx_last_error(void);
/* name: >=64 bytes.  cus, clock_khz, l2/lds bytes as reported by HIP. */
int phx_device_info(char *name, size_t name_len, int *cus, int *clock_khz, size_t *hbm_bytes,
                    int *lds_bytes_per_cu);
int phx_device_synchronize(void);

/* ------------------------------------------------------------ memory */
int phx_malloc(uint64_t *dptr, size_t bytes);
int phx_free(uint64_t dptr);
int phx_host_alloc(void **ptr, size_t bytes); /* pinned (hipHostMalloc) */
int phx_host_free(void *ptr);
int phx_memcpy_h2d(uint64_t dst, const void *src, size_t bytes);
int phx_memcpy_d2h(void *dst, uint64_t src, size_t bytes);
int phx_memcpy_d2d(uint64_t dst, uint64_t src, size_t bytes);
int phx_memcpy_h2d_async(uint64_t dst, const void *src, size_t bytes, phx_stream s);
int phx_memcpy_d2h_async(void *dst, uint64_t src, size_t bytes, phx_stream s);
/* cuMemsetD8Async (main.rs:268-282) */
int phx_memset_async(uint64_t dst, int value, size_t bytes, phx_stream s);

/* ------------------------------------------------------------ streams/events */
int phx_stream_create(phx_stream *s); /* non-blocking, default priority */
int phx_stream_destroy(phx_stream s);
int phx_stream_synchronize(phx_stream s);
/* Binds a caller-owned device buffer (256-byte aligned) as the workspace of
 * split launches on stream s (NULL: the legacy default stream); dptr 0 or
 * bytes 0 unbinds.  No counterpart in the reference, whose kernels never
 * split: it keeps the reference's ownership rule (the caller owns every
 * device buffer, tile_store.rs:14-83; a COMPUTE touches only arena tiles,
 * engine.rs:582-647) for the split launches of this backend.  A built-in
 * GEMM or flash launch that phx_split_plan would split runs with the largest
 * split whose workspace fits in the bound bytes, and unsplit when none fits
 * or nothing is bound (gemm_fp32 without a pin then takes its 64 x 64 x 16
 * tiling, which needs no workspace); it never allocates.  The buffer must stay valid until
 * every launch on s that may use it has completed; launches on one stream
 * run in order, so they can share it.  Unbinding (or phx_stream_destroy)
 * forgets it; the caller frees it. */
int phx_stream_set_workspace(phx_stream s, uint64_t dptr, size_t bytes);
int phx_stream_get_workspace(phx_stream s, uint64_t *dptr, size_t *bytes);
int phx_event_create(phx_event *e);
int phx_event_destroy(phx_event e);
int phx_event_record(phx_event e, phx_stream s);
/* 0 = complete, 1 = not ready, else error (engine.rs:655-687) */
int phx_event_query(phx_event e);
int phx_event_synchronize(phx_event e);
int phx_event_elapsed_ms(float *ms, phx_event start, phx_event stop);

/* ------------------------------------------------------------ modules */
/* PtxCache::insert / function (ptx_cache.rs:41-81) for gfx950 code objects. */
int phx_module_load_data(phx_module *m, const void *image, size_t bytes);
int phx_module_load_file(phx_module *m, const char *path);
int phx_module_unload(phx_module m);
int phx_module_get_function(phx_function *f, phx_module m, const char *name);
/* The built-in code object's entry for a kernel id. */
int phx_builtin_function(phx_function *f, phx_kernel k);
/* Index width (32 or 64) and block size the built-in kernel expects. */
int phx_kernel_abi(phx_kernel k, int *index_bits, uint32_t block[3]);

/* ------------------------------------------------------------ launch */
/* cuLaunchKernel semantics: one pointer per kernel parameter in args
 * (stream.launch, engine.rs:643-647; launch!, main.rs:308-323).
 * For a built-in kernel (phx_builtin_function, or phx_module_get_function on
 * a phx_module_load_file of a built-in code object) the runtime reads the
 * extents from the argument list, checks them as the kernel would, and
 * replaces grid, block and shared_bytes with its own (the reference caller's
 * saxpy 1024-thread blocks and flash @launch(128) are accepted).  A built-in
 * GEMM or flash launch whose problem cannot fill the GPU runs split over K
 * or over the keys (phx_split_plan) when s has a workspace bound
 * (phx_stream_set_workspace) that holds the split's partial results, else
 * unsplit. */
int phx_launch(phx_function f, const uint32_t grid[3], const uint32_t block[3],
               uint32_t shared_bytes, phx_stream s, void **args);

/* Grid and block a built-in kernel wants for the given problem.
 * dims: saxpy {n}; gemm/matmul {M, N, K}; matmul_init {M, N};
 * flash {Nq, Nk, D}; flash_bh {BH, Nq, Nk, D}.
 * Replaces the reference's config-derived grid (main.rs:500-508, 974-981,
 * 1220-1223; phobos-sched/src/lib.rs:380-429). */
int phx_grid_for(phx_kernel k, const int64_t *dims, int ndims, uint32_t grid[3],
                 uint32_t block[3]);
/* Kernel id of a built-in by the reference's names: the .ph file stem
 * ("saxpy_fp32", "gemm_fp32", "gemm_fp16tc_fp32acc", "gemm_fp16",
 * "flash_attention_fp32", "flash_attention_fp16", "matmul_cluster_fp32") and
 * the kernel's entry name ("saxpy", "gemm", "flash_attention",
 * "flash_attention_bh", "matmul", "matmul_init").  The stem is needed: three
 * .ph files export "gemm" (phobos-bench/src/main.rs:512, 761, 985;
 * clustergen.rs:1285, 1353).  PHX_E_INVALID for an unknown pair. */
int phx_kernel_by_name(phx_kernel *k, const char *ph_file, const char *entry);
/* phx_launch of the built-in phx_kernel_by_name names, with the caller's
 * void** argument list (the launch! macro's, main.rs:308-323).  block NULL
 * means the kernel's own workgroup size (phx_kernel_abi). */
int phx_launch_by_name(const char *ph_file, const char *entry, const uint32_t grid[3],
                       const uint32_t block[3], phx_stream s, void **args);
/* Validates that a built-in kernel accepts these dims (divisibility etc). */
int phx_check_shape(phx_kernel k, const int64_t *dims, int ndims);
/* The split a launch of k over dims (as phx_grid_for) runs with on a stream
 * whose bound workspace holds at least *workspace_bytes: *splits K
 * chunks (gemm_fp32, gemm_fp16tc_fp32acc, gemm_fp16) or key chunks (flash),
 * 1 for none, and the workspace bytes that needs (0 for none).  With a
 * smaller workspace a launch takes fewer chunks, down to none.  Other
 * kernels never split.  No counterpart in the reference, whose autotuner
 * picks tile sizes instead (phobos-bench/src/autotune.rs:98-192). */
int phx_split_plan(phx_kernel k, const int64_t *dims, int ndims, int *splits,
                   size_t *workspace_bytes);

/* A launch plan of a built-in kernel at one problem shape: the dims the
 * autotuner searches (phobos_amd.autotune).  The reference's autotuner picks
 * compile-time tile sizes by timing every choice
 * (phobos-bench/src/autotune.rs:98-192; the @autotune dims of the .ph
 * kernels); here each kernel has one tile shape and these are its choices:
 *   splits   K chunks (gemm_fp32, gemm_fp16tc_fp32acc, gemm_fp16) or key
 *            chunks (flash), 1 .. 16, 1 for none;
 *   variant  gemm_fp32: the tiling TILE_M x TILE_N x TILE_K (the .ph file's
 *            @autotune dims, examples/gemm_fp32.ph:1): 0 256x256x16 (the
 *            built-in tiling, the only one that splits), 1 256x128x16,
 *            2 128x256x16, 3 128x128x16, 4 128x128x32, 5 128x128x8,
 *            6 256x256x8, 7 64x64x16 (code object entries "gemm" and
 *            "gemm_t<M>x<N>k<K>");
 *            gemm_fp16tc_fp32acc: 0 the eight-wave kernels (entries
 *            "gemm_w8", "gemm_w8_splitk"), 1 the one-wave kernels ("gemm",
 *            "gemm_splitk"), split or not; 0 for every other kernel.
 * A launch uses the plan pinned for its kernel and dims, else the built-in
 * rule.  The PHX_GEMM_SPLIT, PHX_FLASH_SPLIT and PHX_GEMM_W8 environment
 * variables, which force a plan for measurement, take precedence over both. */
typedef struct {
    int32_t splits;
    int32_t variant;
} phx_plan;
/* The plan a launch of k over dims (as phx_grid_for) would use now. */
int phx_plan_get(phx_kernel k, const int64_t *dims, int ndims, phx_plan *plan);
/* Pins plan for k at dims (plan NULL removes the pin).  The one-head and
 * batched flash kernels of a precision share pins, the one-head dims meaning
 * one head.  PHX_E_INVALID for a kernel without choices, splits outside
 * 1 .. 16, a variant the kernel lacks, or a gemm_fp32 tiling other than 0
 * with splits above 1. */
int phx_plan_pin(phx_kernel k, const int64_t *dims, int ndims, const phx_plan *plan);
/* Removes every pin. */
int phx_plan_unpin_all(void);

/* --- Pod COMPUTE marshalling (engine.rs:582-630) ---
 * Each tile argument becomes the exploded memref
 *   (ptr, ptr, offset=0, sizes[rank], strides[rank] row-major)
 * at the kernel's index width; scalars are placed at their parameter
 * position `pos` as little-endian bit patterns (tile.rs:75-84: an f32 uses
 * the low 4 bytes of `bits`).  grid/cta are passed through unchanged. */
typedef struct {
    uint64_t addr;
    uint32_t rank; /* 1..3 */
    uint64_t shape[3];
} phx_tile_arg;

typedef struct {
    uint32_t pos;   /* parameter position among tiles+scalars */
    uint32_t bytes; /* 4 (f32/i32) or 8 (f64/i64) */
    uint64_t bits;
} phx_scalar_arg;

int phx_compute(phx_function f, int index_bits, const phx_tile_arg *tiles, uint32_t ntiles,
                const phx_scalar_arg *scalars, uint32_t nscalars, const uint32_t grid[3],
                const uint32_t cta[3], phx_stream s);

/* ------------------------------------------------------------ typed launches */
/* Each marshals the reference's exploded-memref argument list for the named
 * .ph kernel and launches its gfx950 code object on stream s. */

/* saxpy_fp32.ph: out = alpha*x + y; out may alias y (main.rs:1227-1239). */
int phx_saxpy(phx_stream s, uint64_t x, uint64_t y, uint64_t out, int64_t n, float alpha);

/* gemm (kernel = PHX_GEMM_FP32 | PHX_GEMM_FP16TC_FP32ACC | PHX_GEMM_FP16 |
 * PHX_MATMUL): C = alpha*A@B + beta*C, row-major A[M,K] B[K,N] C[M,N]
 * (launch_gemm, main.rs:290-327).  Element types follow the .ph signature:
 * f32 for FP32/FP16TC/MATMUL, f16 for FP16.  PHX_MATMUL is the cluster step
 * leaf C = alpha*A@B + C (beta is accepted and ignored, clustergen.rs:1363-1399). */
int phx_gemm(phx_stream s, phx_kernel k, uint64_t a, uint64_t b, uint64_t c, int64_t M,
             int64_t N, int64_t K, float alpha, float beta);

/* matmul_init leaf: C = beta*C over a [M, N] f32 tile (clustergen.rs:1292-1360). */
int phx_matmul_init(phx_stream s, uint64_t c, int64_t M, int64_t N, float beta);

/* flash_attention (kernel = PHX_FLASH_FP32 | PHX_FLASH_FP16): one head,
 * Q[Nq,D] K[Nk,D] V[Nk,D] O[Nq,D] (launch_flash, main.rs:334-371). */
int phx_flash_attention(phx_stream s, phx_kernel k, uint64_t q, uint64_t kk, uint64_t v,
                        uint64_t o, int64_t Nq, int64_t Nk, int64_t D, float scale);

/* flash_attention_bh: BH independent heads laid out [BH, N, D] (head stride
 * N*D), one launch.  No reference counterpart: the .ph signature is one
 * head; per head it is the same arithmetic as flash_attention. */
int phx_flash_attention_bh(phx_stream s, phx_kernel k, uint64_t q, uint64_t kk, uint64_t v,
                           uint64_t o, int64_t BH, int64_t Nq, int64_t Nk, int64_t D,
                           float scale);

/* ------------------------------------------------------------ arena */
/* DeviceArena (tile_store.rs:14-83): one device allocation, bump pointer,
 * exact size-class free lists, 256-byte alignment, 256-byte minimum class. */
size_t phx_size_class(size_t bytes);
int phx_arena_create(phx_arena *a, size_t bytes);
int phx_arena_destroy(phx_arena a);
int phx_arena_alloc(phx_arena a, size_t bytes, uint64_t *addr, size_t *cls);
int phx_arena_free(phx_arena a, uint64_t addr, size_t cls);
int phx_arena_can_alloc(phx_arena a, size_t bytes); /* 1 yes, 0 no */
int phx_arena_stats(phx_arena a, size_t *cap, size_t *bump, uint64_t *base);

/* ------------------------------------------------------------ no allocation */
/* phx_flash_attention_bh without any device allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, split plan, kernels and results (bit for bit)
 * as phx_flash_attention_bh on a stream whose bound workspace holds the
 * split; a launch split over the keys keeps its partial results in a fixed
 * PHX_SCRATCH_BYTES (16 MiB) device array that the library holds on each
 * initialised GPU until the process ends, instead of the stream's workspace
 * (it splits whether or not one is bound).  A split that needs more
 * scratch (phx_split_plan) returns PHX_E_INVALID; phx_flash_attention_bh
 * takes any size.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (several streams or
 * threads) race. */
int phx_flash_attention_bh_noalloc(phx_stream s, phx_kernel k, uint64_t q, uint64_t kk,
                                   uint64_t v, uint64_t o, int64_t BH, int64_t Nq, int64_t Nk,
                                   int64_t D, float scale);

/* ------------------------------------------------------------ inputs */
/* Lcg::unit_f32s (phobos-base/src/rng.rs:9-25) into host memory. */
int phx_lcg_fill_f32(uint64_t seed, size_t n, float *out);
/* The same stream continued: *state is the Lcg state (the seed before the
 * first call) and is advanced by n draws, so a tensor can be filled chunk by
 * chunk (phobos-tensor.rs:55-70). */
int phx_lcg_fill_f32_stream(uint64_t *state, size_t n, float *out);
/* Seeded N(0,1)*scale by Box-Muller over Lcg draws (this backend's input
 * convention for the BASELINE configs; the reference has no normal draw). */
int phx_normal_fill_f32(uint64_t seed, size_t n, double scale, float *out);
/* f32 -> f16 bit patterns, IEEE round-to-nearest-even (main.rs:682-693). */
int phx_f32_to_f16(size_t n, const float *in, uint16_t *out);
int phx_f16_to_f32(size_t n, const uint16_t *in, float *out);

/* ------------------------------------------------------------ pod segment */
/* One-pod executor for ALLOC/LOAD/COMPUTE/STORE/FREE segments
 * (Engine, phobos-pod/src/engine.rs:121-232, 355-398, 424-509).  The segment
 * is text, one instruction per line ('#' starts a comment), the fields of
 * phobos_v1_isa.proto / isa.rs:25-50:
 *   <iid> <deps|-> ALLOC   <tile> <d0xd1> f32
 *   <iid> <deps>   LOAD    <tile> <tensor> <off0,off1> <s0,s1>
 *   <iid> <deps>   COMPUTE <kernel> <tile:r|w|rmw,...> <pos:f32:0xBITS,...|-> <gx,gy,gz> <cx,cy,cz>
 *   <iid> <deps>   STORE   <tile> <tensor> <off0,off1> <s0,s1>
 *   <iid> <deps>   FREE    <tile> <expected_serves>
 * (deps: comma-separated iids; phx_segment_pb_to_text writes this form from
 * a wire Segment).  Kernels are the built-in ids or functions bound with
 * phx_pod_set_kernel_function.  LOAD/STORE use file:// f32 tensors
 * (storage.rs:22-79) staged through pinned host buffers with async copies. */
typedef struct phx_pod_s *phx_pod;
int phx_pod_create(phx_pod *p, size_t arena_bytes, int nstreams);
int phx_pod_destroy(phx_pod p);
/* The pod's device arena (for phx_arena_stats); owned by the pod.  Besides
 * the segment's tiles it holds the workspace of a split built-in COMPUTE
 * while that leaf runs. */
int phx_pod_get_arena(phx_pod p, phx_arena *a);
/* Registers a tensor id -> (uri, shape) for LOAD/STORE (JobManifest). */
int phx_pod_set_tensor(phx_pod p, uint32_t tensor, const char *uri, const uint64_t *shape,
                       uint32_t rank);
/* Binds a segment kernel id to a built-in kernel (SetKernels). */
int phx_pod_set_kernel(phx_pod p, uint32_t kernel_id, phx_kernel k);
/* Binds a segment kernel id to any loaded kernel (phx_module_load_data /
 * phx_module_get_function), in place of the PTX text a SetKernels or
 * GetKernel reply carries (phobos-pod/src/server.rs:189-225,
 * ptx_cache.rs:12-82).  Its COMPUTEs run with the instruction's own grid and
 * cta, and their tiles are marshalled with index_bits (32 or 64) wide
 * sizes and strides, as engine.rs:582-647 launches every kernel. */
int phx_pod_set_kernel_function(phx_pod p, uint32_t kernel_id, phx_function f, int index_bits);
/* Runs one segment to completion.  stats (nullable) receives
 * {n_alloc, n_load, n_compute, n_store, n_free, compute_ns, wall_ns, io_ns}.
 * compute_ns is device time with at least one COMPUTE running (the union of
 * the leaves' event intervals; leaves on different streams may overlap). */
int phx_pod_run_segment(phx_pod p, const char *segment_text, uint64_t stats[8]);

/* The scheduler's wire messages, protobuf-encoded (proto3 wire format):
 *   phx_pod_set_manifest_pb: a phobos.v1.JobManifest
 *     (phobos-cluster/proto/v1/phobos_v1_scheduler.proto:53-76), as the pod's
 *     server applies it (phobos-pod/src/server.rs:189-225): each TensorEntry
 *     is registered as with phx_pod_set_tensor (f32 file:// tensors); each
 *     KernelEntry is bound by entry-point name to a built-in leaf ("matmul",
 *     "matmul_init", "saxpy"); other names return PHX_E_NOT_FOUND and are
 *     bound by id with phx_pod_set_kernel or phx_pod_set_kernel_function.
 *     kernel_holders are ignored (no peer pods).
 *   phx_pod_run_segment_pb: a phobos.v1.Segment
 *     (phobos-cluster/proto/v1/phobos_v1_isa.proto:107-110), decoded with the
 *     checks of segment_from_proto (phobos-cluster/src/proto.rs:193-275) and
 *     run like phx_pod_run_segment (server.rs:239-248 -> engine.rs).  FETCH
 *     needs a peer pod and is rejected with PHX_E_SEGMENT. */
int phx_pod_set_manifest_pb(phx_pod p, const void *manifest, size_t bytes);
int phx_pod_run_segment_pb(phx_pod p, const void *segment, size_t bytes, uint64_t stats[8]);
/* Decodes an encoded phobos.v1.Segment (the same decoder) into the text form
 * phx_pod_run_segment takes; needs no device.  `needed` (nullable) receives
 * the text size including the NUL; text may be NULL to query it. */
int phx_segment_pb_to_text(const void *segment, size_t bytes, char *text, size_t cap,
                           size_t *needed);

#ifdef __cplusplus
}
#endif
#endif /* PHOBOS_HIP_H */
