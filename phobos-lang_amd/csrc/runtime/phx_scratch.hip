// The allocation-free variant of phx_flash_attention_bh, for callers that
// cannot allocate device memory: code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc.  It has no counterpart in the
// reference.
//
// phx_flash_attention_bh splits small launches over the keys when the
// caller has bound a workspace to the launch stream (phx_stream_set_workspace)
// for the split's partial accumulators, running maxima and row sums, and
// runs unsplit otherwise.  This entry point runs the built-in split plan and
// the same kernels whether or not a workspace is bound, with the workspace
// in a fixed array of PHX_SCRATCH_BYTES
// device memory that the library holds on each GPU it is initialised on,
// until the process ends.  Every call on a GPU shares that GPU's array:
// calls that overlap on one GPU (on different streams, or from several
// threads) race.  The array keeps the last call's contents; nothing in it
// has to start at zero, because each call writes every partial result it
// later reads (each split covers whole query blocks of every head and a
// non-empty key range).
#include "phx_internal.h"

#include <cstring>
#include <string>

namespace phx {

static __device__ __align__(256) char scratch[PHX_SCRATCH_BYTES];

// Device address of `scratch` on each device, from hipGetSymbolAddress: in
// host code the array's name is only a host-side stand-in.
constexpr int kMaxDevices = 64;
static uint64_t g_scratch[kMaxDevices];
// Functions the entry point launches, resolved at set-up so that a call
// loads no code object (a load allocates device memory).  Null when the
// code objects lack them; the entry point then reports PHX_E_NOT_FOUND.
static hipFunction_t g_bh[2], g_split[2], g_combine[2];  // [0]: f16, [1]: f32
static std::string g_missing;  // why a function could not be resolved

int scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices)
        return set_error(PHX_E_INVALID, "device %d: the scratch table holds %d devices", device,
                         kMaxDevices);
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // device is current
    if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
    g_scratch[device] = (uint64_t)(uintptr_t)p;
    const phx_kernel bh[2] = {PHX_FLASH_FP16_BH, PHX_FLASH_FP32_BH};
    g_missing.clear();
    for (int i = 0; i < 2; ++i) {
        if (builtin(bh[i], &g_bh[i]) ||
            flash_split_functions(bh[i], &g_split[i], &g_combine[i])) {
            g_bh[i] = g_split[i] = g_combine[i] = nullptr;
            g_missing = phx_last_error();  // the other entry points report it on use
        }
    }
    return PHX_OK;
}

void scratch_reset() {  // phx_shutdown: the functions are unloaded
    for (int i = 0; i < 2; ++i) g_bh[i] = g_split[i] = g_combine[i] = nullptr;
    for (auto &p : g_scratch) p = 0;
}

}  // namespace phx

using namespace phx;

extern "C" int phx_flash_attention_bh_noalloc(phx_stream s, phx_kernel k, uint64_t q,
                                              uint64_t kk, uint64_t v, uint64_t o, int64_t BH,
                                              int64_t Nq, int64_t Nk, int64_t D, float scale) {
    if (k != PHX_FLASH_FP16_BH && k != PHX_FLASH_FP32_BH)
        return set_error(PHX_E_INVALID, "kernel %d is not a batched flash", (int)k);
    if (!q || !kk || !v || !o) return set_error(PHX_E_INVALID, "flash: null operand");
    if ((q | kk | v | o) & 15) return set_error(PHX_E_INVALID, "flash operands must be 16-byte aligned");
    const int64_t d[4] = {BH, Nq, Nk, D};
    if (int rc = check_shape(k, d, 4)) return rc;
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_error(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices || !g_scratch[dev])
        return set_error(PHX_E_NOT_INIT, "phx_init has not set up device %d", dev);
    const int i = k == PHX_FLASH_FP16_BH ? 0 : 1;
    if (!g_bh[i] || !g_split[i] || !g_combine[i])
        return set_error(PHX_E_NOT_FOUND, "flash_attention_bh_noalloc: %s", g_missing.c_str());
    const int sp = flash_split(k, BH, Nq, Nk);
    if (sp > 1) {
        const size_t need = flash_split_bytes(BH, Nq, sp);
        if (need > PHX_SCRATCH_BYTES)
            return set_error(PHX_E_INVALID,
                             "flash_attention_bh_noalloc: BH=%lld Nq=%lld Nk=%lld splits the keys "
                             "%d ways and needs %zu bytes of scratch; the static scratch holds "
                             "%u (phx_flash_attention_bh takes any size)",
                             (long long)BH, (long long)Nq, (long long)Nk, sp, need,
                             (unsigned)PHX_SCRATCH_BYTES);
        Desc t[4];
        const uint64_t ptr[4] = {q, kk, v, o};
        const int64_t n[4] = {Nq, Nk, Nk, Nq};
        for (int j = 0; j < 4; ++j) {
            t[j].ptr = ptr[j];
            t[j].size[0] = BH;
            t[j].size[1] = n[j];
            t[j].size[2] = D;
            t[j].stride[0] = n[j] * D;
            t[j].stride[1] = D;
            t[j].stride[2] = 1;
        }
        return launch_flash_split_ws(k, t, 3, BH, Nq, Nk, scale, sp, (hipStream_t)s,
                                     g_scratch[dev], g_split[i], g_combine[i]);
    }
    // no split: the batched kernel itself, with the exploded-memref argument
    // list built on the stack
    uint64_t slots[37];
    void *args[37];
    int a = 0;
    const uint64_t ptr[4] = {q, kk, v, o};
    const int64_t n[4] = {Nq, Nk, Nk, Nq};
    for (int j = 0; j < 4; ++j) {
        const int64_t vals[9] = {0, 0, 0, BH, n[j], D, n[j] * D, D, 1};
        for (int r = 0; r < 9; ++r) {
            uint64_t u = r < 2 ? ptr[j] : 0;
            if (r >= 2) memcpy(&u, &vals[r], 8);
            slots[a] = u;
            args[a] = &slots[a];
            ++a;
        }
    }
    uint32_t sb;
    memcpy(&sb, &scale, 4);
    slots[a] = sb;
    args[a] = &slots[a];
    uint32_t grid[3], block[3];
    if (int rc = grid_for(k, d, 4, grid, block)) return rc;
    e = hipModuleLaunchKernel(g_bh[i], grid[0], grid[1], grid[2], block[0], block[1], block[2], 0,
                              (hipStream_t)s, args, nullptr);
    if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel(flash_attention_bh)");
    return PHX_OK;
}
