// Host runtime of the MI355X leaf-kernel backend: the C ABI declared in
// include/phobos_hip.h.  Everything goes through the HIP module API
// (hipModuleLoad / hipModuleGetFunction / hipModuleLaunchKernel), the same
// path the reference takes through cust (Module::from_ptx + launch!), so the
// typed helpers below exercise exactly what a phobos-pod COMPUTE would.
#include "phx_internal.h"

#include <dlfcn.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <deque>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace phx {

static thread_local std::string g_err;

int set_error(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_error(hipError_t e, const char *what) {
    return set_error((int)e, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

struct KernelSpec {
    const char *file;
    const char *entry;
    int index_bits;
    uint32_t block;
};

// One code object per .ph source, as the reference compiles one module per
// kernel file; the entry name is the .ph kernel name.
static const KernelSpec kSpecs[PHX_NUM_KERNELS] = {
    {"saxpy_fp32.hsaco", "saxpy", 32, PHX_SAXPY_THREADS},
    {"gemm_fp32.hsaco", "gemm", 32, PHX_S_THREADS},
    {"gemm_fp16tc_fp32acc.hsaco", "gemm", 64, PHX_H_THREADS},
    {"gemm_fp16.hsaco", "gemm", 64, PHX_H_THREADS},
    {"flash_attention_fp32.hsaco", "flash_attention", 64, PHX_FA_THREADS},
    {"flash_attention_fp16.hsaco", "flash_attention", 64, PHX_FA16_THREADS},
    {"matmul_cluster_fp32.hsaco", "matmul", 32, PHX_S_THREADS},
    {"matmul_cluster_fp32.hsaco", "matmul_init", 32, PHX_EW_THREADS},
    {"flash_attention_fp32.hsaco", "flash_attention_bh", 64, PHX_FA_THREADS},
    {"flash_attention_fp16.hsaco", "flash_attention_bh", 64, PHX_FA16_THREADS},
};

struct State {
    bool init = false;
    int device = -1;
    std::string dir;
    std::unordered_map<std::string, hipModule_t> modules;  // file -> module
    // written under mu by builtin(), read without it by launch_raw()
    std::atomic<hipFunction_t> fns[PHX_NUM_KERNELS] = {};
    // Functions a caller got from its own load of a built-in code object
    // file (phx_module_load_file + phx_module_get_function), keyed to the
    // built-in they are; under mu.
    std::unordered_map<hipModule_t, std::string> module_files;  // module -> file name
    std::unordered_map<hipFunction_t, std::pair<int, hipModule_t>> aliases;
    std::unordered_map<std::string, hipFunction_t> aux;  // "file:entry" -> function
    std::mutex mu;
};
static State g;

// The built-in kernel id `f` is, or -1.
static int builtin_id(hipFunction_t f) {
    if (!f) return -1;
    for (int k = 0; k < PHX_NUM_KERNELS; ++k)
        if (g.fns[k].load(std::memory_order_acquire) == f) return k;
    std::lock_guard<std::mutex> lock(g.mu);
    auto it = g.aliases.find(f);
    return it == g.aliases.end() ? -1 : it->second.first;
}

static std::string default_dir() {
    if (const char *env = getenv("PHX_CODE_OBJECT_DIR")) return env;
    Dl_info info;
    if (dladdr((void *)&default_dir, &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        size_t slash = p.rfind('/');
        if (slash != std::string::npos) return p.substr(0, slash);
    }
    return ".";
}

static int ensure_init() {
    if (!g.init) return set_error(PHX_E_NOT_INIT, "phx_init has not been called");
    return PHX_OK;
}

int builtin(phx_kernel k, hipFunction_t *out) {
    if (int rc = ensure_init()) return rc;
    if ((int)k < 0 || k >= PHX_NUM_KERNELS)
        return set_error(PHX_E_INVALID, "unknown kernel id %d", (int)k);
    if (hipFunction_t f = g.fns[k].load(std::memory_order_acquire)) {
        *out = f;
        return PHX_OK;
    }
    std::lock_guard<std::mutex> lock(g.mu);
    if (!g.fns[k].load(std::memory_order_relaxed)) {
        const KernelSpec &s = kSpecs[k];
        hipModule_t mod;
        auto it = g.modules.find(s.file);
        if (it == g.modules.end()) {
            std::string path = g.dir + "/" + s.file;
            hipError_t e = hipModuleLoad(&mod, path.c_str());
            if (e != hipSuccess)
                return set_error(PHX_E_NOT_FOUND,
                                 "cannot load code object %s: %s (build the backend first)",
                                 path.c_str(), hipGetErrorString(e));
            g.modules[s.file] = mod;
        } else {
            mod = it->second;
        }
        hipFunction_t f;
        hipError_t e = hipModuleGetFunction(&f, mod, s.entry);
        if (e != hipSuccess)
            return set_error(PHX_E_NOT_FOUND, "entry '%s' not in %s: %s", s.entry, s.file,
                             hipGetErrorString(e));
        g.fns[k].store(f, std::memory_order_release);
    }
    *out = g.fns[k].load(std::memory_order_relaxed);
    return PHX_OK;
}

// Entry points of the built-in code objects that no .ph kernel names (the
// split-K and split-key kernels the runtime launches itself), by file and
// entry name; loaded on first use.
int aux_function(const char *file, const char *entry, hipFunction_t *out) {
    if (int rc = ensure_init()) return rc;
    std::lock_guard<std::mutex> lock(g.mu);
    const std::string key = std::string(file) + ":" + entry;
    auto fit = g.aux.find(key);
    if (fit != g.aux.end()) {
        *out = fit->second;
        return PHX_OK;
    }
    hipModule_t mod;
    auto it = g.modules.find(file);
    if (it == g.modules.end()) {
        std::string path = g.dir + "/" + file;
        hipError_t e = hipModuleLoad(&mod, path.c_str());
        if (e != hipSuccess)
            return set_error(PHX_E_NOT_FOUND, "cannot load code object %s: %s (build the backend first)",
                             path.c_str(), hipGetErrorString(e));
        g.modules[file] = mod;
    } else {
        mod = it->second;
    }
    hipFunction_t f;
    hipError_t e = hipModuleGetFunction(&f, mod, entry);
    if (e != hipSuccess)
        return set_error(PHX_E_NOT_FOUND, "entry '%s' not in %s: %s", entry, file,
                         hipGetErrorString(e));
    g.aux[key] = f;
    *out = f;
    return PHX_OK;
}

// ------------------------------------------------------------------ args
// Holds the values of an exploded-memref argument list at stable addresses
// plus the void* array hipModuleLaunchKernel reads.
struct ArgPack {
    std::deque<uint64_t> slots;  // deque: push_back keeps earlier addresses valid
    std::vector<void *> ptrs;
    explicit ArgPack(size_t cap) { ptrs.reserve(cap); }
    void push_bits(uint64_t v) {
        slots.push_back(v);
        ptrs.push_back(&slots.back());
    }
    void ptr(uint64_t p) { push_bits(p); }
    void idx(int64_t v, int bits) {
        if (bits == 32) {
            int32_t v32 = (int32_t)v;
            uint32_t u;
            memcpy(&u, &v32, 4);
            push_bits((uint64_t)u);  // little-endian: low 4 bytes hold the i32
        } else {
            uint64_t u;
            memcpy(&u, &v, 8);
            push_bits(u);
        }
    }
    void f32(float f) {
        uint32_t u;
        memcpy(&u, &f, 4);
        push_bits((uint64_t)u);
    }
    // (ptr, ptr, 0, sizes..., row-major strides...)
    void memref(uint64_t p, const int64_t *shape, int rank, int bits) {
        ptr(p);
        ptr(p);
        idx(0, bits);
        for (int i = 0; i < rank; ++i) idx(shape[i], bits);
        int64_t stride = 1;
        int64_t strides[4];
        for (int i = rank - 1; i >= 0; --i) {
            strides[i] = stride;
            stride *= shape[i];
        }
        for (int i = 0; i < rank; ++i) idx(strides[i], bits);
    }
};

// ------------------------------------------------------------------ raw launches
static int64_t arg_idx(void **args, int i, int bits) {
    if (bits == 32) {
        int32_t v;
        memcpy(&v, args[i], 4);
        return v;
    }
    int64_t v;
    memcpy(&v, args[i], 8);
    return v;
}

// Reads `n` rank-`rank` descriptors starting at args[0]; `esz` is the element
// size the offset is scaled by.
static void read_descs(void **args, int n, int rank, int bits, int esz, Desc *d) {
    int a = 0;
    for (int t = 0; t < n; ++t) {
        uint64_t aligned;
        memcpy(&aligned, args[a + 1], 8);
        d[t].ptr = aligned + (uint64_t)(arg_idx(args, a + 2, bits) * esz);
        for (int r = 0; r < rank; ++r) d[t].size[r] = arg_idx(args, a + 3 + r, bits);
        for (int r = 0; r < rank; ++r) d[t].stride[r] = arg_idx(args, a + 3 + rank + r, bits);
        a += 3 + 2 * rank;
    }
}

// The problem extents of a built-in kernel's launch, read from its argument
// list the way the kernel reads them, after the same consistency checks the
// kernel makes on entry (a launch that fails them would return without
// output, so it is refused here instead).
static int builtin_dims(phx_kernel k, void **args, int64_t *d, int *nd, Desc *t) {
    if (!args) return set_error(PHX_E_INVALID, "%s: null argument list", kSpecs[k].entry);
    const int bits = kSpecs[k].index_bits;
    auto bad = [&](const char *why) {
        return set_error(PHX_E_INVALID, "%s (%s): %s", kSpecs[k].entry, kSpecs[k].file, why);
    };
    switch (k) {
    case PHX_SAXPY_FP32:
        read_descs(args, 3, 1, bits, 4, t);
        if (t[1].size[0] != t[0].size[0] || t[2].size[0] != t[0].size[0])
            return bad("x, y and out differ in length");
        if (t[0].size[0] > 0 && (!t[0].ptr || !t[1].ptr || !t[2].ptr)) return bad("null operand");
        d[0] = t[0].size[0];
        *nd = 1;
        return PHX_OK;
    case PHX_GEMM_FP32:
    case PHX_GEMM_FP16TC_FP32ACC:
    case PHX_GEMM_FP16:
    case PHX_MATMUL: {
        read_descs(args, 3, 2, bits, k == PHX_GEMM_FP16 ? 2 : 4, t);
        const int64_t M = t[0].size[0], K = t[0].size[1], N = t[1].size[1];
        if (t[1].size[0] != K || t[2].size[0] != M || t[2].size[1] != N)
            return bad("A, B and C extents do not chain as [M,K] x [K,N] -> [M,N]");
        for (int i = 0; i < 3; ++i)
            if (t[i].stride[1] != 1) return bad("operands need a unit minor stride");
        const int nm = k == PHX_GEMM_FP16 ? PHX_H16_NK_MULT
                       : k == PHX_GEMM_FP16TC_FP32ACC ? PHX_TC_N_MULT : PHX_S_NK_MULT;
        const int km = k == PHX_GEMM_FP16TC_FP32ACC ? PHX_TC_K_MULT : nm;
        if (t[0].stride[0] % km || t[1].stride[0] % nm || t[2].stride[0] % nm)
            return bad("row strides must keep every row 16-byte aligned");
        if (!t[0].ptr || !t[1].ptr || !t[2].ptr) return bad("null operand");
        if ((t[0].ptr | t[1].ptr | t[2].ptr) & 15) return bad("operands must be 16-byte aligned");
        d[0] = M;
        d[1] = N;
        d[2] = K;
        *nd = 3;
        return PHX_OK;
    }
    case PHX_MATMUL_INIT:
        read_descs(args, 1, 2, bits, 4, t);
        if (t[0].stride[1] != 1) return bad("C needs a unit minor stride");
        if (t[0].size[0] * t[0].size[1] > 0 && !t[0].ptr) return bad("null operand");
        d[0] = t[0].size[0];
        d[1] = t[0].size[1];
        *nd = 2;
        return PHX_OK;
    case PHX_FLASH_FP32:
    case PHX_FLASH_FP16: {
        read_descs(args, 4, 2, bits, k == PHX_FLASH_FP16 ? 2 : 4, t);
        const int64_t Nq = t[0].size[0], Nk = t[1].size[0], D = t[0].size[1];
        if (t[1].size[1] != D || t[2].size[1] != D || t[3].size[1] != D || t[2].size[0] != Nk ||
            t[3].size[0] != Nq)
            return bad("Q, K, V and O extents disagree");
        for (int i = 0; i < 4; ++i)
            if (t[i].stride[1] != 1 || t[i].stride[0] % 8)
                return bad("operands need a unit minor stride and rows of whole 16-byte chunks");
        if (!t[0].ptr || !t[1].ptr || !t[2].ptr || !t[3].ptr) return bad("null operand");
        if ((t[0].ptr | t[1].ptr | t[2].ptr | t[3].ptr) & 15)
            return bad("operands must be 16-byte aligned");
        d[0] = Nq;
        d[1] = Nk;
        d[2] = D;
        *nd = 3;
        return PHX_OK;
    }
    case PHX_FLASH_FP32_BH:
    case PHX_FLASH_FP16_BH: {
        read_descs(args, 4, 3, bits, k == PHX_FLASH_FP16_BH ? 2 : 4, t);
        const int64_t H = t[0].size[0], Nq = t[0].size[1], Nk = t[1].size[1], D = t[0].size[2];
        for (int i = 1; i < 4; ++i)
            if (t[i].size[0] != H || t[i].size[2] != D) return bad("Q, K, V and O extents disagree");
        if (t[2].size[1] != Nk || t[3].size[1] != Nq) return bad("Q, K, V and O extents disagree");
        for (int i = 0; i < 4; ++i)
            if (t[i].stride[2] != 1 || (t[i].stride[0] | t[i].stride[1]) % 8)
                return bad("operands need a unit minor stride and rows of whole 16-byte chunks");
        if (!t[0].ptr || !t[1].ptr || !t[2].ptr || !t[3].ptr) return bad("null operand");
        if ((t[0].ptr | t[1].ptr | t[2].ptr | t[3].ptr) & 15)
            return bad("operands must be 16-byte aligned");
        d[0] = H;
        d[1] = Nq;
        d[2] = Nk;
        d[3] = D;
        *nd = 4;
        return PHX_OK;
    }
    default:
        return set_error(PHX_E_INVALID, "unknown kernel id %d", (int)k);
    }
}

// Plans pinned by phx_plan_pin, keyed by kernel family and problem dims:
// GEMMs by (kernel, M, N, K), flash by (precision, heads, Nq, Nk).
namespace {
struct PlanKey {
    int fam;
    int64_t a, b, c;
    bool operator==(const PlanKey &o) const {
        return fam == o.fam && a == o.a && b == o.b && c == o.c;
    }
};
struct PlanKeyHash {
    size_t operator()(const PlanKey &k) const {
        size_t h = (size_t)k.fam;
        for (int64_t v : {k.a, k.b, k.c}) h = h * 1000003u ^ (size_t)v;
        return h;
    }
};
std::mutex g_plan_mu;
std::unordered_map<PlanKey, phx_plan, PlanKeyHash> g_plans;

bool pinned_plan(const PlanKey &key, phx_plan *out) {  // out may be null
    std::lock_guard<std::mutex> lock(g_plan_mu);
    auto it = g_plans.find(key);
    if (it == g_plans.end()) return false;
    if (out) *out = it->second;
    return true;
}
bool is_gemm(phx_kernel k) {
    return k == PHX_GEMM_FP32 || k == PHX_GEMM_FP16TC_FP32ACC || k == PHX_GEMM_FP16;
}
bool is_flash(phx_kernel k) {
    return k == PHX_FLASH_FP16 || k == PHX_FLASH_FP32 || k == PHX_FLASH_FP16_BH ||
           k == PHX_FLASH_FP32_BH;
}
PlanKey gemm_key(phx_kernel k, int64_t M, int64_t N, int64_t K) { return {(int)k, M, N, K}; }
PlanKey flash_key(phx_kernel k, int64_t BH, int64_t Nq, int64_t Nk) {
    const bool f16 = k == PHX_FLASH_FP16 || k == PHX_FLASH_FP16_BH;
    return {f16 ? -1 : -2, BH, Nq, Nk};
}
}  // namespace

// Workspaces bound to streams by phx_stream_set_workspace: device memory
// the caller owns (a pod's arena slab, a bench's buffer).  A split launch on
// a stream takes its partial results from the stream's workspace and never
// allocates; a stream without one, or with one too small for any split, runs
// the unsplit kernel.
namespace {
struct Workspace {
    uint64_t ptr = 0;
    size_t bytes = 0;
};
std::mutex g_ws_mu;
std::unordered_map<hipStream_t, Workspace> g_ws;

Workspace stream_workspace(hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = g_ws.find(s);
    return it == g_ws.end() ? Workspace{} : it->second;
}

// Chunks a split of `units` (K steps or key blocks) into at most sp chunks of
// whole units really makes: ceil(units / ceil(units / sp)), so no chunk is
// empty.
int round_split(int64_t units, int64_t sp) {
    if (sp > units) sp = units;
    if (sp < 2) return 1;
    const int64_t per = (units + sp - 1) / sp;
    return (int)((units + per - 1) / per);
}

// The largest split of at most sp chunks of `units` whose workspace,
// bytes_per_chunk per chunk, fits in cap bytes; 1 when none does.
int fit_split(int64_t units, int sp, size_t bytes_per_chunk, size_t cap) {
    for (int64_t want = sp; want >= 2; --want) {
        const int r = round_split(units, want);
        if (r >= 2 && (size_t)r * bytes_per_chunk <= cap) return r;
    }
    return 1;
}
}  // namespace

// The tilings of gemm_fp32 (entries of gemm_fp32.hsaco), by phx_plan
// variant: the reference's autotuner picks TILE_M, TILE_N in [32, 256] and
// TILE_K in [4, 32] (examples/gemm_fp32.ph:1); variant 0 is the built-in
// 256 x 256 x 16 "gemm", the only one that also splits over K.
struct S32Tiling {
    const char *entry;
    int64_t tm, tn, tk;
};
static const S32Tiling kS32[] = {
    {"gemm", 256, 256, 16},           {"gemm_t256x128k16", 256, 128, 16},
    {"gemm_t128x256k16", 128, 256, 16}, {"gemm_t128x128k16", 128, 128, 16},
    {"gemm_t128x128k32", 128, 128, 32}, {"gemm_t128x128k8", 128, 128, 8},
    {"gemm_t256x256k8", 256, 256, 8},   {"gemm_t64x64k16", 64, 64, 16},
};
constexpr int kS32Variants = (int)(sizeof kS32 / sizeof kS32[0]);

// The built-in gemm_fp32 tiling (no pin): the 256 x 256 tile when it fills
// the GPU, else the 64 x 64 one where it measured faster than splitting K
// (phx_geometry.h), else 0 and the split rule.
static int s32_rule(int64_t M, int64_t N, int64_t K) {
    const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
    if (t256 >= PHX_S32_FULL_TILES) return 0;
    const int64_t ts = PHX_S32_SMALL_TILE;
    const int64_t tsmall = ((M + ts - 1) / ts) * ((N + ts - 1) / ts);
    if (tsmall >= PHX_S32_SMALL_MIN_TILES ||
        (tsmall >= PHX_S32_SMALL_SHORT_TILES && K <= PHX_S32_SHORT_K))
        return PHX_S32_SMALL_VARIANT;
    return 0;
}

// The gemm_fp32 tiling a launch at M x N x K uses: the pinned variant, else
// (unless PHX_GEMM_SPLIT forces a split of the 256 x 256 tiling) the
// built-in one.
static int s32_variant(int64_t M, int64_t N, int64_t K) {
    phx_plan pin;
    if (pinned_plan(gemm_key(PHX_GEMM_FP32, M, N, K), &pin))
        return pin.variant > 0 && pin.variant < kS32Variants ? pin.variant : 0;
    if (getenv("PHX_GEMM_SPLIT")) return 0;
    return s32_rule(M, N, K);
}

// How many K chunks a GEMM is split into (1: no split).  A GEMM whose
// 256 x 256 output tiles cannot fill half of the 256 CUs gets enough chunks
// to give its kernel's target number of workgroups, within its chunk-length
// floor and at most PHX_SPLIT_MAX chunks (phx_geometry.h).  PHX_GEMM_SPLIT=<n> in the environment
// forces n (1 turns the split off), for measurement.
int gemm_split(phx_kernel k, int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = ((M + PHX_H_BM - 1) / PHX_H_BM) * ((N + PHX_H_BN - 1) / PHX_H_BN);
    const int64_t steps = (K + PHX_SPLIT_KSTEP - 1) / PHX_SPLIT_KSTEP;
    int64_t sp;
    phx_plan pin;
    if (const char *env = getenv("PHX_GEMM_SPLIT")) {
        sp = atoi(env);
    } else if (pinned_plan(gemm_key(k, M, N, K), &pin)) {
        sp = pin.splits;
    } else {
        if (k == PHX_GEMM_FP32 && s32_rule(M, N, K) != 0) return 1;  // a smaller tile instead
        if (tiles >= PHX_SPLIT_MIN_TILES) return 1;
        const bool f32 = k == PHX_GEMM_FP32;
        const int64_t min_steps = f32                            ? PHX_SPLIT_MIN_STEPS_F32
                                  : tiles >= PHX_SPLIT_WIDE_TILES ? PHX_SPLIT_MIN_STEPS_F16_WIDE
                                                                  : PHX_SPLIT_MIN_STEPS_F16;
        sp = (f32 ? PHX_SPLIT_TARGET_F32 : PHX_SPLIT_TARGET_F16) / tiles;
        if (sp > steps / min_steps) sp = steps / min_steps;
        if (sp > PHX_SPLIT_MAX) sp = PHX_SPLIT_MAX;
    }
    // chunks of whole steps; drop chunks the rounding left empty
    return round_split(steps, sp);
}

// Whether a gemm_fp16tc_fp32acc launch runs the eight-wave kernels
// (gemm_w8, and gemm_w8_splitk for a split) rather than the one-wave ones
// (gemm, gemm_splitk): always, unless the plan pins variant 1.  Measured on
// one box, three alternations: 4096^3 139-141 against 147-154 us, 4000^3
// 134-140 against 146-154, 3000 x 5000 x 1000 49 against 51.5, split
// 2048^3 (2 chunks) 41.5 against 47.0, 512^3 (2) 14.6 against 16.6, and
// within 2% elsewhere (4088^3, 1000^3 and 640 x 768 x 4104 split 13 ways).
// gemm_fp16, whose operand
// copies are half the bytes and already overlap its MFMAs, measured the
// same with an eight-wave form (114-119 vs 115-118 us) and keeps its
// one-wave kernel.  PHX_GEMM_W8=0 in the environment turns it off, for
// measurement.
static bool gemm_w8(phx_kernel k, int64_t M, int64_t N, int64_t K) {
    if (k != PHX_GEMM_FP16TC_FP32ACC) return false;
    phx_plan pin;
    if (const char *env = getenv("PHX_GEMM_W8")) return atoi(env) != 0;
    return !(pinned_plan(gemm_key(k, M, N, K), &pin) && pin.variant == 1);
}

// K columns per chunk of a split into sp chunks (a multiple of 32).
static int64_t split_chunk(int64_t K, int sp) {
    const int64_t steps = (K + PHX_SPLIT_KSTEP - 1) / PHX_SPLIT_KSTEP;
    return ((steps + sp - 1) / sp) * PHX_SPLIT_KSTEP;
}

// Bytes of f32 partial sums a split GEMM needs.
size_t gemm_split_bytes(int64_t M, int64_t N, int sp) {
    return (size_t)sp * (size_t)M * (size_t)N * sizeof(float);
}

// The split-K launches over a caller-provided workspace of
// gemm_split_bytes(M, N, sp) bytes: gemm_splitk over (tiles, sp) workgroups,
// then gemm_splitk_reduce, both on stream s.
int launch_gemm_split_ws(phx_kernel k, const Desc *t, int64_t M, int64_t N, int64_t K,
                         float alpha, float beta, int sp, hipStream_t s, uint64_t ws) {
    const char *file = kSpecs[k].file;
    hipFunction_t fk, fr;
    const bool w8 = gemm_w8(k, M, N, K);
    if (int rc = aux_function(file, w8 ? "gemm_w8_splitk" : "gemm_splitk", &fk)) return rc;
    if (int rc = aux_function(file, "gemm_splitk_reduce", &fr)) return rc;
    const int64_t tiles = ((M + PHX_H_BM - 1) / PHX_H_BM) * ((N + PHX_H_BN - 1) / PHX_H_BN);
    uint64_t a = t[0].ptr, b = t[1].ptr, c = t[2].ptr;
    int64_t lda = t[0].stride[0], ldb = t[1].stride[0], ldc = t[2].stride[0];
    int64_t kchunk = split_chunk(K, sp);
    void *ka[] = {&a, &b, &ws, &lda, &ldb, &M, &N, &K, &kchunk};
    hipError_t e = hipModuleLaunchKernel(fk, (uint32_t)tiles, (uint32_t)sp, 1,
                                         w8 ? PHX_TC_W8_THREADS : PHX_H_THREADS, 1, 1, 0, s, ka,
                                         nullptr);
    if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel(gemm_splitk)");
    int32_t s32 = sp;
    void *ra[] = {&ws, &s32, &c, &ldc, &M, &N, &alpha, &beta};
    const int64_t groups = M * (N / 4);
    int64_t nb = (groups + PHX_REDUCE_THREADS - 1) / PHX_REDUCE_THREADS;
    if (nb > 8192) nb = 8192;
    e = hipModuleLaunchKernel(fr, (uint32_t)nb, 1, 1, PHX_REDUCE_THREADS, 1, 1, 0, s, ra, nullptr);
    if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel(gemm_splitk_reduce)");
    return PHX_OK;
}

// The split count a GEMM launch on a stream whose workspace holds cap bytes
// runs with: gemm_split's plan, cut to what fits.
static int gemm_split_fit(phx_kernel k, int64_t M, int64_t N, int64_t K, size_t cap) {
    const int sp = gemm_split(k, M, N, K);
    if (sp < 2) return 1;
    const int64_t steps = (K + PHX_SPLIT_KSTEP - 1) / PHX_SPLIT_KSTEP;
    return fit_split(steps, sp, gemm_split_bytes(M, N, 1), cap);
}

// How many key chunks a flash launch is split into (1: no split).
// PHX_FLASH_SPLIT=<n> in the environment forces n, for measurement.
static bool flash_f16(phx_kernel k) { return k == PHX_FLASH_FP16 || k == PHX_FLASH_FP16_BH; }
int flash_split(phx_kernel k, int64_t BH, int64_t Nq, int64_t Nk) {
    const int64_t qb = flash_f16(k) ? PHX_FA16_BR : PHX_FA_BR;
    const int64_t items = ((Nq + qb - 1) / qb) * BH;
    const int64_t nkb = (Nk + PHX_FA_BC - 1) / PHX_FA_BC;
    int64_t sp;
    phx_plan pin;
    if (const char *env = getenv("PHX_FLASH_SPLIT")) {
        sp = atoi(env);
    } else if (pinned_plan(flash_key(k, BH, Nq, Nk), &pin)) {
        sp = pin.splits;
    } else {
        if (2 * items >= PHX_FA_SLOTS) return 1;
        const int64_t min_blocks =
            flash_f16(k) ? PHX_FLASH_SPLIT_MIN_BLOCKS_F16 : PHX_FLASH_SPLIT_MIN_BLOCKS_F32;
        sp = PHX_FLASH_SPLIT_TARGET / items;
        if (sp > nkb / min_blocks) sp = nkb / min_blocks;
        if (sp > PHX_SPLIT_MAX) sp = PHX_SPLIT_MAX;
    }
    return round_split(nkb, sp);  // whole blocks per chunk; no empty chunk
}

// Bytes of partial results a split flash launch needs: per chunk and query,
// 64 accumulators plus the running max and row sum, all f32.
size_t flash_split_bytes(int64_t BH, int64_t Nq, int sp) {
    return (size_t)sp * (size_t)BH * (size_t)Nq * (PHX_FA_D + 2) * sizeof(float);
}

// The split-key launches over a caller-provided workspace of
// flash_split_bytes(BH, Nq, sp) bytes.  t: the Q, K, V, O descriptors, rank 2
// (one head) or rank 3 ([BH, N, D]).
int flash_split_functions(phx_kernel k, hipFunction_t *fs, hipFunction_t *fc) {
    if (int rc = aux_function(kSpecs[k].file, "flash_attention_split", fs)) return rc;
    return aux_function(kSpecs[k].file, "flash_combine", fc);
}

int launch_flash_split_ws(phx_kernel k, const Desc *t, int rank, int64_t BH, int64_t Nq,
                          int64_t Nk, float scale, int sp, hipStream_t s, uint64_t ws,
                          hipFunction_t fs, hipFunction_t fc) {
    const int64_t qb = flash_f16(k) ? PHX_FA16_BR : PHX_FA_BR;
    const int64_t items = ((Nq + qb - 1) / qb) * BH;
    const int64_t nkb = (Nk + PHX_FA_BC - 1) / PHX_FA_BC;
    int64_t kchunk = ((nkb + sp - 1) / sp) * PHX_FA_BC;
    uint64_t q = t[0].ptr, kk = t[1].ptr, v = t[2].ptr;
    const int r = rank - 2;  // index of the row stride
    int64_t ldq = t[0].stride[r], ldk = t[1].stride[r], ldv = t[2].stride[r], ldo = t[3].stride[r];
    int64_t hq = r ? t[0].stride[0] : 0, hk = r ? t[1].stride[0] : 0, hv = r ? t[2].stride[0] : 0;
    int64_t ho = r ? t[3].stride[0] : 0;
    int32_t nsplit = sp;
    void *sa[] = {&q, &kk, &v, &ws, &BH, &Nq, &Nk, &ldq, &ldk, &ldv, &hq, &hk, &hv, &kchunk,
                  &nsplit, &scale};
    hipError_t e = hipModuleLaunchKernel(fs, (uint32_t)items, (uint32_t)sp, 1, kSpecs[k].block, 1,
                                         1, 0, s, sa, nullptr);
    if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel(flash_attention_split)");
    uint64_t o = t[3].ptr;
    void *ca[] = {&ws, &nsplit, &o, &BH, &Nq, &ldo, &ho};
    const int64_t threads = BH * Nq * (PHX_FA_D / 4);
    int64_t nb = (threads + PHX_REDUCE_THREADS - 1) / PHX_REDUCE_THREADS;
    if (nb > 8192) nb = 8192;
    e = hipModuleLaunchKernel(fc, (uint32_t)nb, 1, 1, PHX_REDUCE_THREADS, 1, 1, 0, s, ca, nullptr);
    if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel(flash_combine)");
    return PHX_OK;
}

static int flash_split_fit(phx_kernel k, int64_t BH, int64_t Nq, int64_t Nk, size_t cap) {
    const int sp = flash_split(k, BH, Nq, Nk);
    if (sp < 2) return 1;
    const int64_t nkb = (Nk + PHX_FA_BC - 1) / PHX_FA_BC;
    return fit_split(nkb, sp, flash_split_bytes(BH, Nq, 1), cap);
}

int launch_raw(hipFunction_t f, const uint32_t grid[3], const uint32_t block[3], uint32_t shmem,
               hipStream_t s, void **args) {
    // A built-in kernel runs on this backend's own tiling, whatever geometry
    // the caller derived from the reference's tiles (e.g. saxpy's 1024-thread
    // blocks, flash's @launch(128)): its grid and workgroup come from
    // grid_for() over the extents in its own argument list.  The kernels
    // need no dynamic LDS, so the shared-memory size is ignored as well.
    if (int k = builtin_id(f); k >= 0) {
        int64_t d[4];
        int nd = 0;
        Desc t[4];
        if (int rc = builtin_dims((phx_kernel)k, args, d, &nd, t)) return rc;
        if (k == PHX_GEMM_FP32 || k == PHX_GEMM_FP16TC_FP32ACC || k == PHX_GEMM_FP16) {
            if (int rc = check_shape((phx_kernel)k, d, nd)) return rc;
            const Workspace w = stream_workspace(s);
            const int sp = gemm_split_fit((phx_kernel)k, d[0], d[1], d[2], w.bytes);
            // gemm_fp32's built-in plan split over K, but the stream has no
            // workspace for it: the 64 x 64 tiling fills the GPU without one
            // (256^2 x 8192: 151 us against 1.8 ms for one 256 x 256 tile)
            const bool no_room = k == PHX_GEMM_FP32 && sp == 1 &&
                                 gemm_split((phx_kernel)k, d[0], d[1], d[2]) > 1 &&
                                 !pinned_plan(gemm_key((phx_kernel)k, d[0], d[1], d[2]), nullptr) &&
                                 !getenv("PHX_GEMM_SPLIT");
            if (sp > 1) {
                float alpha, beta;  // the two f32 scalars after the three memrefs
                memcpy(&alpha, args[21], 4);
                memcpy(&beta, args[22], 4);
                return launch_gemm_split_ws((phx_kernel)k, t, d[0], d[1], d[2], alpha, beta, sp,
                                            s, w.ptr);
            }
            if (k == PHX_GEMM_FP32) {
                const int v = no_room ? PHX_S32_SMALL_VARIANT : s32_variant(d[0], d[1], d[2]);
                if (v) {
                    const S32Tiling &ti = kS32[v];
                    hipFunction_t fv;
                    if (int rc = aux_function(kSpecs[k].file, ti.entry, &fv)) return rc;
                    const uint32_t tiles = (uint32_t)(((d[0] + ti.tm - 1) / ti.tm) *
                                                      ((d[1] + ti.tn - 1) / ti.tn));
                    hipError_t e = hipModuleLaunchKernel(fv, tiles, 1, 1, PHX_S_THREADS, 1, 1, 0,
                                                         s, args, nullptr);
                    if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel(gemm tiling)");
                    return PHX_OK;
                }
            }
            if (gemm_w8((phx_kernel)k, d[0], d[1], d[2])) {
                hipFunction_t fw;
                if (int rc = aux_function(kSpecs[k].file, "gemm_w8", &fw)) return rc;
                const uint32_t tiles = (uint32_t)(((d[0] + PHX_H_BM - 1) / PHX_H_BM) *
                                                  ((d[1] + PHX_H_BN - 1) / PHX_H_BN));
                hipError_t e = hipModuleLaunchKernel(fw, tiles, 1, 1, PHX_TC_W8_THREADS, 1, 1, 0,
                                                     s, args, nullptr);
                if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel(gemm_w8)");
                return PHX_OK;
            }
        }
        if (k == PHX_FLASH_FP16 || k == PHX_FLASH_FP32 || k == PHX_FLASH_FP16_BH ||
            k == PHX_FLASH_FP32_BH) {
            if (int rc = check_shape((phx_kernel)k, d, nd)) return rc;
            const bool bh = nd == 4;
            const int64_t BH = bh ? d[0] : 1, Nq = d[bh], Nk = d[bh + 1];
            const Workspace w = stream_workspace(s);
            const int sp = flash_split_fit((phx_kernel)k, BH, Nq, Nk, w.bytes);
            if (sp > 1) {
                float scale;  // the f32 scalar after the four memrefs
                memcpy(&scale, args[bh ? 36 : 28], 4);
                hipFunction_t fs, fc;
                if (int rc = flash_split_functions((phx_kernel)k, &fs, &fc)) return rc;
                return launch_flash_split_ws((phx_kernel)k, t, bh ? 3 : 2, BH, Nq, Nk, scale, sp,
                                             s, w.ptr, fs, fc);
            }
        }
        uint32_t g2[3], b2[3];
        if (int rc = grid_for((phx_kernel)k, d, nd, g2, b2)) return rc;
        hipError_t e = hipModuleLaunchKernel(f, g2[0], g2[1], g2[2], b2[0], b2[1], b2[2], 0, s,
                                             args, nullptr);
        if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel");
        return PHX_OK;
    }
    if (!grid || !block) return set_error(PHX_E_INVALID, "null grid or block");
    hipError_t e = hipModuleLaunchKernel(f, grid[0], grid[1], grid[2], block[0], block[1],
                                         block[2], shmem, s, args, nullptr);
    if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel");
    return PHX_OK;
}

static bool fits_i32(int64_t v) { return v >= 0 && v <= INT32_MAX; }

int check_shape(phx_kernel k, const int64_t *d, int nd) {
    auto need = [&](int n) {
        if (nd != n)
            return set_error(PHX_E_INVALID, "kernel %d takes %d dims, got %d", (int)k, n, nd);
        for (int i = 0; i < n; ++i)
            if (d[i] < 0) return set_error(PHX_E_INVALID, "negative dimension %lld", (long long)d[i]);
        return PHX_OK;
    };
    switch (k) {
    case PHX_SAXPY_FP32:
        if (int rc = need(1)) return rc;
        if (!fits_i32(d[0])) return set_error(PHX_E_INVALID, "saxpy n=%lld exceeds i32 index", (long long)d[0]);
        return PHX_OK;
    case PHX_GEMM_FP16TC_FP32ACC:
    case PHX_GEMM_FP16:
    case PHX_GEMM_FP32:
    case PHX_MATMUL: {
        if (int rc = need(3)) return rc;
        const int nm = k == PHX_GEMM_FP16 ? PHX_H16_NK_MULT
                       : k == PHX_GEMM_FP16TC_FP32ACC ? PHX_TC_N_MULT
                                                      : PHX_S_NK_MULT;
        const int km = k == PHX_GEMM_FP16 ? PHX_H16_NK_MULT
                       : k == PHX_GEMM_FP16TC_FP32ACC ? PHX_TC_K_MULT
                                                      : PHX_S_NK_MULT;
        if (d[0] == 0 || d[1] == 0 || d[2] == 0 || d[1] % nm || d[2] % km)
            return set_error(PHX_E_INVALID,
                             "gemm needs M>0, N%%%d==0, K%%%d==0 (got %lld,%lld,%lld)", nm, km,
                             (long long)d[0], (long long)d[1], (long long)d[2]);
        if (kSpecs[k].index_bits == 32 &&
            (!fits_i32(d[0] * d[2]) || !fits_i32(d[2] * d[1]) || !fits_i32(d[0] * d[1])))
            return set_error(PHX_E_INVALID, "gemm extents exceed the i32 index");
        // per-tile buffer resources span up to 256 rows of a matrix
        const int64_t esz = k == PHX_GEMM_FP16 ? 2 : 4;
        if ((PHX_H_BM + 1) * (d[1] > d[2] ? d[1] : d[2]) * esz > INT32_MAX)
            return set_error(PHX_E_INVALID, "gemm rows too long (N or K = %lld)",
                             (long long)(d[1] > d[2] ? d[1] : d[2]));
        return PHX_OK;
    }
    case PHX_MATMUL_INIT:
        if (int rc = need(2)) return rc;
        if (!fits_i32(d[0] * d[1])) return set_error(PHX_E_INVALID, "matmul_init exceeds i32 index");
        return PHX_OK;
    case PHX_FLASH_FP32:
    case PHX_FLASH_FP16:
        if (int rc = need(3)) return rc;
        if (d[2] != PHX_FA_D || d[0] == 0 || d[1] == 0)
            return set_error(PHX_E_INVALID, "flash needs D==%d, Nq>0, Nk>0 (got Nq=%lld Nk=%lld D=%lld)",
                             PHX_FA_D, (long long)d[0], (long long)d[1], (long long)d[2]);
        if (d[0] * PHX_FA_D * 4 > INT32_MAX || d[1] * PHX_FA_D * 4 > INT32_MAX)
            return set_error(PHX_E_INVALID, "flash head exceeds 2 GiB (Nq=%lld Nk=%lld)",
                             (long long)d[0], (long long)d[1]);
        return PHX_OK;
    case PHX_FLASH_FP32_BH:
    case PHX_FLASH_FP16_BH:
        if (int rc = need(4)) return rc;
        if (d[0] == 0 || d[0] > 65535)
            return set_error(PHX_E_INVALID, "flash_bh needs 1 <= BH <= 65535");
        return check_shape(k == PHX_FLASH_FP32_BH ? PHX_FLASH_FP32 : PHX_FLASH_FP16, d + 1, 3);
    default:
        return set_error(PHX_E_INVALID, "unknown kernel id %d", (int)k);
    }
}

int grid_for(phx_kernel k, const int64_t *d, int nd, uint32_t grid[3], uint32_t block[3]) {
    if ((int)k < 0 || k >= PHX_NUM_KERNELS)
        return set_error(PHX_E_INVALID, "unknown kernel id %d", (int)k);
    if (int rc = check_shape(k, d, nd)) return rc;
    grid[0] = grid[1] = grid[2] = 1;
    block[0] = kSpecs[k].block;
    block[1] = block[2] = 1;
    switch (k) {
    case PHX_SAXPY_FP32: {
        int64_t b = (d[0] + PHX_SAXPY_BLOCK_ELEMS - 1) / PHX_SAXPY_BLOCK_ELEMS;
        grid[0] = (uint32_t)(b < 1 ? 1 : b);
        break;
    }
    case PHX_GEMM_FP16TC_FP32ACC:
    case PHX_GEMM_FP16:
        grid[0] = (uint32_t)(((d[0] + PHX_H_BM - 1) / PHX_H_BM) * ((d[1] + PHX_H_BN - 1) / PHX_H_BN));
        break;
    case PHX_GEMM_FP32: {
        const S32Tiling &ti = kS32[s32_variant(d[0], d[1], d[2])];
        grid[0] = (uint32_t)(((d[0] + ti.tm - 1) / ti.tm) * ((d[1] + ti.tn - 1) / ti.tn));
        break;
    }
    case PHX_MATMUL:
        grid[0] = (uint32_t)(((d[0] + PHX_S_TILE - 1) / PHX_S_TILE) *
                             ((d[1] + PHX_S_TILE - 1) / PHX_S_TILE));
        break;
    case PHX_MATMUL_INIT: {
        int64_t n = d[0] * d[1];
        int64_t b = (n + PHX_EW_BLOCK_ELEMS - 1) / PHX_EW_BLOCK_ELEMS;
        grid[0] = (uint32_t)(b < 1 ? 1 : b);
        break;
    }
    case PHX_FLASH_FP32:
        grid[0] = (uint32_t)((d[0] + PHX_FA_BR - 1) / PHX_FA_BR);
        break;
    case PHX_FLASH_FP16:
        grid[0] = (uint32_t)((d[0] + PHX_FA16_BR - 1) / PHX_FA16_BR);
        break;
    case PHX_FLASH_FP32_BH:
        grid[0] = (uint32_t)((d[1] + PHX_FA_BR - 1) / PHX_FA_BR);
        grid[1] = (uint32_t)d[0];
        break;
    case PHX_FLASH_FP16_BH:
        grid[0] = (uint32_t)((d[1] + PHX_FA16_BR - 1) / PHX_FA16_BR);
        grid[1] = (uint32_t)d[0];
        break;
    default:
        break;
    }
    return PHX_OK;
}

int kernel_abi(phx_kernel k, int *bits, uint32_t block[3]) {
    if ((int)k < 0 || k >= PHX_NUM_KERNELS)
        return set_error(PHX_E_INVALID, "unknown kernel id %d", (int)k);
    if (bits) *bits = kSpecs[k].index_bits;
    if (block) {
        block[0] = kSpecs[k].block;
        block[1] = block[2] = 1;
    }
    return PHX_OK;
}

}  // namespace phx

using namespace phx;

extern "C" {

const char *phx_last_error(void) { return g_err.c_str(); }

static int init_device(int device, const char *dir) {
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return hip_error(e, "hipSetDevice");
    e = hipFree(nullptr);  // force context creation
    if (e != hipSuccess) return hip_error(e, "hipFree(0)");
    std::lock_guard<std::mutex> lock(g.mu);
    if (g.init && g.device != device)
        return set_error(PHX_E_INVALID, "already initialised on device %d", g.device);
    g.device = device;
    g.dir = dir ? std::string(dir) : default_dir();
    g.init = true;
    return PHX_OK;
}

// The device set-up, then that of the allocation-free entry point
// (phx_scratch.hip), which loads functions and so needs the lock released.
int phx_init(int device, const char *dir) {
    if (int rc = init_device(device, dir)) return rc;
    return scratch_setup(device);
}

int phx_shutdown(void) {
    scratch_reset();
    {
        std::lock_guard<std::mutex> lock(g_ws_mu);
        g_ws.clear();
    }
    std::lock_guard<std::mutex> lock(g.mu);
    for (auto &kv : g.modules) (void)hipModuleUnload(kv.second);
    g.modules.clear();
    for (auto &f : g.fns) f.store(nullptr, std::memory_order_release);
    g.aux.clear();
    g.init = false;
    return PHX_OK;
}

int phx_device_info(char *name, size_t name_len, int *cus, int *clock_khz, size_t *hbm,
                    int *lds) {
    if (int rc = ensure_init()) return rc;
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, g.device);
    if (e != hipSuccess) return hip_error(e, "hipGetDeviceProperties");
    if (name && name_len) {
        snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
    }
    if (cus) *cus = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    if (hbm) *hbm = p.totalGlobalMem;
    if (lds) *lds = (int)p.maxSharedMemoryPerMultiProcessor;
    return PHX_OK;
}

int phx_device_synchronize(void) {
    hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipDeviceSynchronize");
}

// ------------------------------------------------------------------ memory
int phx_malloc(uint64_t *dptr, size_t bytes) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) return hip_error(e, "hipMalloc");
    *dptr = (uint64_t)(uintptr_t)p;
    return PHX_OK;
}
int phx_free(uint64_t dptr) {
    hipError_t e = hipFree((void *)(uintptr_t)dptr);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipFree");
}
int phx_host_alloc(void **ptr, size_t bytes) {
    hipError_t e = hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocDefault);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipHostMalloc");
}
int phx_host_free(void *ptr) {
    hipError_t e = hipHostFree(ptr);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipHostFree");
}
int phx_memcpy_h2d(uint64_t dst, const void *src, size_t bytes) {
    hipError_t e = hipMemcpy((void *)(uintptr_t)dst, src, bytes, hipMemcpyHostToDevice);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipMemcpy H2D");
}
int phx_memcpy_d2h(void *dst, uint64_t src, size_t bytes) {
    hipError_t e = hipMemcpy(dst, (const void *)(uintptr_t)src, bytes, hipMemcpyDeviceToHost);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipMemcpy D2H");
}
int phx_memcpy_d2d(uint64_t dst, uint64_t src, size_t bytes) {
    hipError_t e = hipMemcpy((void *)(uintptr_t)dst, (const void *)(uintptr_t)src, bytes,
                             hipMemcpyDeviceToDevice);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipMemcpy D2D");
}
int phx_memcpy_h2d_async(uint64_t dst, const void *src, size_t bytes, phx_stream s) {
    hipError_t e = hipMemcpyAsync((void *)(uintptr_t)dst, src, bytes, hipMemcpyHostToDevice,
                                  (hipStream_t)s);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipMemcpyAsync H2D");
}
int phx_memcpy_d2h_async(void *dst, uint64_t src, size_t bytes, phx_stream s) {
    hipError_t e = hipMemcpyAsync(dst, (const void *)(uintptr_t)src, bytes,
                                  hipMemcpyDeviceToHost, (hipStream_t)s);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipMemcpyAsync D2H");
}
int phx_memset_async(uint64_t dst, int value, size_t bytes, phx_stream s) {
    hipError_t e = hipMemsetAsync((void *)(uintptr_t)dst, value, bytes, (hipStream_t)s);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipMemsetAsync");
}

// ------------------------------------------------------------------ streams/events
int phx_stream_create(phx_stream *s) {
    hipStream_t h;
    hipError_t e = hipStreamCreateWithFlags(&h, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_error(e, "hipStreamCreateWithFlags");
    *s = (phx_stream)h;
    return PHX_OK;
}
int phx_stream_destroy(phx_stream s) {
    {
        std::lock_guard<std::mutex> lock(g_ws_mu);
        g_ws.erase((hipStream_t)s);
    }
    hipError_t e = hipStreamDestroy((hipStream_t)s);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipStreamDestroy");
}
int phx_stream_set_workspace(phx_stream s, uint64_t dptr, size_t bytes) {
    if (dptr & 255) return set_error(PHX_E_INVALID, "workspace must be 256-byte aligned");
    std::lock_guard<std::mutex> lock(g_ws_mu);
    if (!dptr || !bytes)
        g_ws.erase((hipStream_t)s);
    else
        g_ws[(hipStream_t)s] = Workspace{dptr, bytes};
    return PHX_OK;
}
int phx_stream_get_workspace(phx_stream s, uint64_t *dptr, size_t *bytes) {
    const Workspace w = stream_workspace((hipStream_t)s);
    if (dptr) *dptr = w.ptr;
    if (bytes) *bytes = w.bytes;
    return PHX_OK;
}
int phx_stream_synchronize(phx_stream s) {
    hipError_t e = hipStreamSynchronize((hipStream_t)s);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipStreamSynchronize");
}
int phx_event_create(phx_event *ev) {
    hipEvent_t h;
    hipError_t e = hipEventCreate(&h);
    if (e != hipSuccess) return hip_error(e, "hipEventCreate");
    *ev = (phx_event)h;
    return PHX_OK;
}
int phx_event_destroy(phx_event ev) {
    hipError_t e = hipEventDestroy((hipEvent_t)ev);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipEventDestroy");
}
int phx_event_record(phx_event ev, phx_stream s) {
    hipError_t e = hipEventRecord((hipEvent_t)ev, (hipStream_t)s);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipEventRecord");
}
int phx_event_query(phx_event ev) {
    hipError_t e = hipEventQuery((hipEvent_t)ev);
    if (e == hipSuccess) return 0;
    if (e == hipErrorNotReady) return 1;
    return hip_error(e, "hipEventQuery");
}
int phx_event_synchronize(phx_event ev) {
    hipError_t e = hipEventSynchronize((hipEvent_t)ev);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipEventSynchronize");
}
int phx_event_elapsed_ms(float *ms, phx_event a, phx_event b) {
    hipError_t e = hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipEventElapsedTime");
}

// ------------------------------------------------------------------ modules
int phx_module_load_data(phx_module *m, const void *image, size_t bytes) {
    if (int rc = ensure_init()) return rc;
    if (!image || !bytes) return set_error(PHX_E_INVALID, "empty code object image");
    hipModule_t h;
    hipError_t e = hipModuleLoadData(&h, image);
    if (e != hipSuccess) return hip_error(e, "hipModuleLoadData");
    *m = (phx_module)h;
    return PHX_OK;
}
int phx_module_load_file(phx_module *m, const char *path) {
    if (int rc = ensure_init()) return rc;
    hipModule_t h;
    hipError_t e = hipModuleLoad(&h, path);
    if (e != hipSuccess) return hip_error(e, "hipModuleLoad");
    *m = (phx_module)h;
    const char *base = strrchr(path, '/');
    std::lock_guard<std::mutex> lock(g.mu);
    g.module_files[h] = base ? base + 1 : path;
    return PHX_OK;
}
int phx_module_unload(phx_module m) {
    {
        std::lock_guard<std::mutex> lock(g.mu);
        g.module_files.erase((hipModule_t)m);
        for (auto it = g.aliases.begin(); it != g.aliases.end();)
            it = it->second.second == (hipModule_t)m ? g.aliases.erase(it) : std::next(it);
    }
    hipError_t e = hipModuleUnload((hipModule_t)m);
    return e == hipSuccess ? PHX_OK : hip_error(e, "hipModuleUnload");
}
int phx_module_get_function(phx_function *f, phx_module m, const char *name) {
    hipFunction_t h;
    hipError_t e = hipModuleGetFunction(&h, (hipModule_t)m, name);
    if (e != hipSuccess) return set_error(PHX_E_NOT_FOUND, "entry '%s': %s", name, hipGetErrorString(e));
    *f = (phx_function)h;
    // a caller's own load of a built-in code object gets the built-in's
    // launch geometry too (see launch_raw)
    std::lock_guard<std::mutex> lock(g.mu);
    auto it = g.module_files.find((hipModule_t)m);
    if (it != g.module_files.end())
        for (int k = 0; k < PHX_NUM_KERNELS; ++k)
            if (it->second == kSpecs[k].file && strcmp(name, kSpecs[k].entry) == 0)
                g.aliases[h] = {k, (hipModule_t)m};
    return PHX_OK;
}
int phx_builtin_function(phx_function *f, phx_kernel k) {
    hipFunction_t h;
    if (int rc = builtin(k, &h)) return rc;
    *f = (phx_function)h;
    return PHX_OK;
}
int phx_kernel_abi(phx_kernel k, int *index_bits, uint32_t block[3]) {
    return kernel_abi(k, index_bits, block);
}
int phx_kernel_by_name(phx_kernel *k, const char *ph_file, const char *entry) {
    if (!k || !ph_file || !entry) return set_error(PHX_E_INVALID, "kernel_by_name: null argument");
    const size_t n = strlen(ph_file);
    for (int i = 0; i < PHX_NUM_KERNELS; ++i) {
        const char *f = kSpecs[i].file;  // "<stem>.hsaco"
        if (strncmp(f, ph_file, n) == 0 && strcmp(f + n, ".hsaco") == 0 &&
            strcmp(kSpecs[i].entry, entry) == 0) {
            *k = (phx_kernel)i;
            return PHX_OK;
        }
    }
    return set_error(PHX_E_INVALID, "no built-in kernel %s:%s", ph_file, entry);
}
int phx_launch_by_name(const char *ph_file, const char *entry, const uint32_t grid[3],
                       const uint32_t block[3], phx_stream s, void **args) {
    phx_kernel k;
    if (int rc = phx_kernel_by_name(&k, ph_file, entry)) return rc;
    phx_function f;
    if (int rc = phx_builtin_function(&f, k)) return rc;
    uint32_t own[3] = {kSpecs[k].block, 1, 1};
    return phx_launch(f, grid, block ? block : own, 0, s, args);
}

// ------------------------------------------------------------------ launch
int phx_launch(phx_function f, const uint32_t grid[3], const uint32_t block[3],
               uint32_t shared_bytes, phx_stream s, void **args) {
    if (!f) return set_error(PHX_E_INVALID, "null function");
    return launch_raw((hipFunction_t)f, grid, block, shared_bytes, (hipStream_t)s, args);
}

int phx_grid_for(phx_kernel k, const int64_t *dims, int ndims, uint32_t grid[3],
                 uint32_t block[3]) {
    return grid_for(k, dims, ndims, grid, block);
}
int phx_check_shape(phx_kernel k, const int64_t *dims, int ndims) {
    return check_shape(k, dims, ndims);
}
int phx_split_plan(phx_kernel k, const int64_t *dims, int ndims, int *splits,
                   size_t *workspace_bytes) {
    if (int rc = check_shape(k, dims, ndims)) return rc;
    int sp = 1;
    size_t ws = 0;
    if (k == PHX_GEMM_FP32 || k == PHX_GEMM_FP16TC_FP32ACC || k == PHX_GEMM_FP16) {
        sp = gemm_split(k, dims[0], dims[1], dims[2]);
        if (sp > 1) ws = gemm_split_bytes(dims[0], dims[1], sp);
    } else if (k == PHX_FLASH_FP16 || k == PHX_FLASH_FP32 || k == PHX_FLASH_FP16_BH ||
               k == PHX_FLASH_FP32_BH) {
        const bool bh = ndims == 4;
        const int64_t BH = bh ? dims[0] : 1, Nq = dims[bh], Nk = dims[bh + 1];
        sp = flash_split(k, BH, Nq, Nk);
        if (sp > 1) ws = flash_split_bytes(BH, Nq, sp);
    }
    if (splits) *splits = sp;
    if (workspace_bytes) *workspace_bytes = ws;
    return PHX_OK;
}

int phx_plan_get(phx_kernel k, const int64_t *dims, int ndims, phx_plan *plan) {
    if (!plan) return set_error(PHX_E_INVALID, "null plan");
    if (int rc = check_shape(k, dims, ndims)) return rc;
    plan->splits = 1;
    plan->variant = 0;
    if (is_gemm(k)) {
        plan->splits = gemm_split(k, dims[0], dims[1], dims[2]);
        if (k == PHX_GEMM_FP16TC_FP32ACC && !gemm_w8(k, dims[0], dims[1], dims[2]))
            plan->variant = 1;
        if (k == PHX_GEMM_FP32 && plan->splits == 1)
            plan->variant = s32_variant(dims[0], dims[1], dims[2]);
    } else if (is_flash(k)) {
        const bool bh = ndims == 4;
        plan->splits = flash_split(k, bh ? dims[0] : 1, dims[bh], dims[bh + 1]);
    }
    return PHX_OK;
}

int phx_plan_pin(phx_kernel k, const int64_t *dims, int ndims, const phx_plan *plan) {
    if (int rc = check_shape(k, dims, ndims)) return rc;
    PlanKey key;
    if (is_gemm(k)) {
        key = gemm_key(k, dims[0], dims[1], dims[2]);
    } else if (is_flash(k)) {
        const bool bh = ndims == 4;
        key = flash_key(k, bh ? dims[0] : 1, dims[bh], dims[bh + 1]);
    } else {
        return set_error(PHX_E_INVALID, "kernel %d has no launch plan choices", (int)k);
    }
    if (plan) {
        if (plan->splits < 1 || plan->splits > PHX_SPLIT_MAX)
            return set_error(PHX_E_INVALID, "splits %d outside 1..%d", plan->splits, PHX_SPLIT_MAX);
        const bool tc1 = k == PHX_GEMM_FP16TC_FP32ACC && plan->variant == 1;
        const bool s32 = k == PHX_GEMM_FP32 && plan->variant > 0 && plan->variant < kS32Variants;
        if (plan->variant != 0 && !tc1 && !s32)
            return set_error(PHX_E_INVALID, "variant %d: kernel %d has no such variant",
                             plan->variant, (int)k);
        if (s32 && plan->splits != 1)
            return set_error(PHX_E_INVALID,
                             "gemm_fp32 tiling %d (%s) runs unsplit; only variant 0 splits",
                             plan->variant, kS32[plan->variant].entry);
    }
    std::lock_guard<std::mutex> lock(g_plan_mu);
    if (plan)
        g_plans[key] = *plan;
    else
        g_plans.erase(key);
    return PHX_OK;
}

int phx_plan_unpin_all(void) {
    std::lock_guard<std::mutex> lock(g_plan_mu);
    g_plans.clear();
    return PHX_OK;
}

int phx_compute(phx_function f, int bits, const phx_tile_arg *tiles, uint32_t ntiles,
                const phx_scalar_arg *scalars, uint32_t nscalars, const uint32_t grid[3],
                const uint32_t cta[3], phx_stream s) {
    if (!f) return set_error(PHX_E_INVALID, "null function");
    if (bits != 32 && bits != 64) return set_error(PHX_E_INVALID, "index_bits must be 32 or 64");
    ArgPack pack((size_t)ntiles * 9 + nscalars + 1);
    uint32_t total = ntiles + nscalars;
    uint32_t next_tile = 0;
    for (uint32_t pos = 0; pos < total; ++pos) {
        const phx_scalar_arg *sc = nullptr;
        for (uint32_t i = 0; i < nscalars; ++i)
            if (scalars[i].pos == pos) sc = &scalars[i];
        if (sc) {
            if (sc->bytes != 4 && sc->bytes != 8)
                return set_error(PHX_E_INVALID, "scalar at %u has %u bytes", pos, sc->bytes);
            pack.push_bits(sc->bytes == 4 ? (sc->bits & 0xffffffffu) : sc->bits);
            continue;
        }
        if (next_tile >= ntiles)
            return set_error(PHX_E_INVALID, "parameter %u: no tile left and no scalar at it", pos);
        const phx_tile_arg &t = tiles[next_tile++];
        if (t.rank < 1 || t.rank > 3) return set_error(PHX_E_INVALID, "tile rank %u", t.rank);
        int64_t shape[3];
        for (uint32_t i = 0; i < t.rank; ++i) {
            shape[i] = (int64_t)t.shape[i];
            if (bits == 32 && !fits_i32(shape[i]))
                return set_error(PHX_E_INVALID, "tile dim %lld exceeds the i32 index", (long long)shape[i]);
        }
        pack.memref(t.addr, shape, (int)t.rank, bits);
    }
    if (next_tile != ntiles) return set_error(PHX_E_INVALID, "%u tiles left unplaced", ntiles - next_tile);
    return launch_raw((hipFunction_t)f, grid, cta, 0, (hipStream_t)s, pack.ptrs.data());
}

// ------------------------------------------------------------------ typed launches
static int launch_builtin(phx_kernel k, const int64_t *dims, int nd, ArgPack &pack,
                          hipStream_t s) {
    hipFunction_t f;
    if (int rc = builtin(k, &f)) return rc;
    uint32_t grid[3], block[3];
    if (int rc = grid_for(k, dims, nd, grid, block)) return rc;
    return launch_raw(f, grid, block, 0, s, pack.ptrs.data());
}

int phx_saxpy(phx_stream s, uint64_t x, uint64_t y, uint64_t out, int64_t n, float alpha) {
    if (n > 0 && (!x || !y || !out)) return set_error(PHX_E_INVALID, "saxpy: null operand");
    int64_t d[1] = {n};
    ArgPack p(20);
    p.memref(x, d, 1, 32);
    p.memref(y, d, 1, 32);
    p.memref(out, d, 1, 32);
    p.f32(alpha);
    return launch_builtin(PHX_SAXPY_FP32, d, 1, p, (hipStream_t)s);
}

int phx_gemm(phx_stream s, phx_kernel k, uint64_t a, uint64_t b, uint64_t c, int64_t M,
             int64_t N, int64_t K, float alpha, float beta) {
    if (k != PHX_GEMM_FP32 && k != PHX_GEMM_FP16TC_FP32ACC && k != PHX_GEMM_FP16 &&
        k != PHX_MATMUL)
        return set_error(PHX_E_INVALID, "kernel %d is not a gemm", (int)k);
    if (!a || !b || !c) return set_error(PHX_E_INVALID, "gemm: null operand");
    if ((a | b | c) & 15) return set_error(PHX_E_INVALID, "gemm operands must be 16-byte aligned");
    int bits = kSpecs[k].index_bits;
    int64_t d[3] = {M, N, K};
    int64_t sa[2] = {M, K}, sb[2] = {K, N}, sc[2] = {M, N};
    ArgPack p(24);
    p.memref(a, sa, 2, bits);
    p.memref(b, sb, 2, bits);
    p.memref(c, sc, 2, bits);
    p.f32(alpha);
    p.f32(beta);
    return launch_builtin(k, d, 3, p, (hipStream_t)s);
}

int phx_matmul_init(phx_stream s, uint64_t c, int64_t M, int64_t N, float beta) {
    if (!c) return set_error(PHX_E_INVALID, "matmul_init: null operand");
    int64_t d[2] = {M, N};
    ArgPack p(10);
    p.memref(c, d, 2, 32);
    p.f32(beta);
    return launch_builtin(PHX_MATMUL_INIT, d, 2, p, (hipStream_t)s);
}

int phx_flash_attention(phx_stream s, phx_kernel k, uint64_t q, uint64_t kk, uint64_t v,
                        uint64_t o, int64_t Nq, int64_t Nk, int64_t D, float scale) {
    if (k != PHX_FLASH_FP32 && k != PHX_FLASH_FP16)
        return set_error(PHX_E_INVALID, "kernel %d is not a single-head flash", (int)k);
    if (!q || !kk || !v || !o) return set_error(PHX_E_INVALID, "flash: null operand");
    if ((q | kk | v | o) & 15) return set_error(PHX_E_INVALID, "flash operands must be 16-byte aligned");
    int64_t d[3] = {Nq, Nk, D};
    int64_t sq[2] = {Nq, D}, sk[2] = {Nk, D};
    ArgPack p(32);
    p.memref(q, sq, 2, 64);
    p.memref(kk, sk, 2, 64);
    p.memref(v, sk, 2, 64);
    p.memref(o, sq, 2, 64);
    p.f32(scale);
    return launch_builtin(k, d, 3, p, (hipStream_t)s);
}

int phx_flash_attention_bh(phx_stream s, phx_kernel k, uint64_t q, uint64_t kk, uint64_t v,
                           uint64_t o, int64_t BH, int64_t Nq, int64_t Nk, int64_t D,
                           float scale) {
    if (k != PHX_FLASH_FP32_BH && k != PHX_FLASH_FP16_BH)
        return set_error(PHX_E_INVALID, "kernel %d is not a batched flash", (int)k);
    if (!q || !kk || !v || !o) return set_error(PHX_E_INVALID, "flash: null operand");
    if ((q | kk | v | o) & 15) return set_error(PHX_E_INVALID, "flash operands must be 16-byte aligned");
    int64_t d[4] = {BH, Nq, Nk, D};
    int64_t sq[3] = {BH, Nq, D}, sk[3] = {BH, Nk, D};
    ArgPack p(44);
    p.memref(q, sq, 3, 64);
    p.memref(kk, sk, 3, 64);
    p.memref(v, sk, 3, 64);
    p.memref(o, sq, 3, 64);
    p.f32(scale);
    return launch_builtin(k, d, 4, p, (hipStream_t)s);
}

// ------------------------------------------------------------------ inputs
int phx_lcg_fill_f32_stream(uint64_t *state, size_t n, float *out) {
    if (!state || (n && !out)) return set_error(PHX_E_INVALID, "lcg stream: null argument");
    uint64_t st = *state;
    for (size_t i = 0; i < n; ++i) {
        st = st * 6364136223846793005ULL + 1442695040888963407ULL;
        out[i] = (float)(st >> 33) / 2147483648.0f - 1.0f;
    }
    *state = st;
    return PHX_OK;
}

int phx_lcg_fill_f32(uint64_t seed, size_t n, float *out) {
    uint64_t st = seed;
    return phx_lcg_fill_f32_stream(&st, n, out);
}

int phx_normal_fill_f32(uint64_t seed, size_t n, double scale, float *out) {
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        st = st * 6364136223846793005ULL + 1442695040888963407ULL;
        uint64_t a = st;
        st = st * 6364136223846793005ULL + 1442695040888963407ULL;
        uint64_t b = st;
        double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;
        double u2 = (double)(b >> 11) * 0x1.0p-53;
        double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = (float)(r * std::cos(two_pi * u2) * scale);
        if (i + 1 < n) out[i + 1] = (float)(r * std::sin(two_pi * u2) * scale);
    }
    return PHX_OK;
}

int phx_f32_to_f16(size_t n, const float *in, uint16_t *out) {
    for (size_t i = 0; i < n; ++i) {
        _Float16 h = (_Float16)in[i];  // IEEE RNE
        memcpy(&out[i], &h, 2);
    }
    return PHX_OK;
}
int phx_f16_to_f32(size_t n, const uint16_t *in, float *out) {
    for (size_t i = 0; i < n; ++i) {
        _Float16 h;
        memcpy(&h, &in[i], 2);
        out[i] = (float)h;
    }
    return PHX_OK;
}

}  // extern "C"
