// Device arena: the counterpart of DeviceArena (phobos-pod/src/tile_store.rs:14-83).
// One hipMalloc'd slab, a bump pointer, and exact size-class free lists
// (256-byte alignment, 256-byte minimum class), so a 400 MiB supertile claims
// 400 MiB and three fit a 1200 MiB arena (tile_store.rs:228-242).  On MI355X
// the arena is sized to the segment's peak residency within the 288 GB HBM.
#include <unordered_map>
#include <vector>

#include "phx_internal.h"

using namespace phx;

static const size_t kAlign = 256;
static const size_t kMinClass = 256;

struct phx_arena_s {
    void *mem = nullptr;
    uint64_t base = 0;
    size_t cap = 0;
    size_t bump = 0;
    std::unordered_map<size_t, std::vector<uint64_t>> free;
};

extern "C" {

size_t phx_size_class(size_t bytes) {
    size_t c = (bytes + kAlign - 1) / kAlign * kAlign;
    if (c < bytes) c = SIZE_MAX / kAlign * kAlign;  // saturating, as div_ceil().saturating_mul()
    return c < kMinClass ? kMinClass : c;
}

int phx_arena_create(phx_arena *out, size_t bytes) {
    phx_arena a = new phx_arena_s;
    hipError_t e = hipMalloc(&a->mem, bytes ? bytes : kAlign);
    if (e != hipSuccess) {
        delete a;
        return hip_error(e, "arena hipMalloc");
    }
    a->base = (uint64_t)(uintptr_t)a->mem;
    a->cap = bytes;
    *out = a;
    return PHX_OK;
}

int phx_arena_destroy(phx_arena a) {
    if (!a) return PHX_OK;
    hipError_t e = hipFree(a->mem);
    delete a;
    return e == hipSuccess ? PHX_OK : hip_error(e, "arena hipFree");
}

int phx_arena_alloc(phx_arena a, size_t bytes, uint64_t *addr, size_t *cls) {
    if (!a) return set_error(PHX_E_INVALID, "null arena");
    size_t c = phx_size_class(bytes);
    auto it = a->free.find(c);
    if (it != a->free.end() && !it->second.empty()) {
        *addr = it->second.back();
        it->second.pop_back();
        if (cls) *cls = c;
        return PHX_OK;
    }
    size_t off = (a->bump + kAlign - 1) & ~(kAlign - 1);
    if (off + c > a->cap || off + c < off)
        return set_error(PHX_E_EXHAUSTED, "device arena exhausted (%zu MiB cap): need %zu more bytes",
                         a->cap >> 20, c);
    a->bump = off + c;
    *addr = a->base + off;
    if (cls) *cls = c;
    return PHX_OK;
}

int phx_arena_free(phx_arena a, uint64_t addr, size_t cls) {
    if (!a) return set_error(PHX_E_INVALID, "null arena");
    if (addr < a->base || addr >= a->base + a->cap)
        return set_error(PHX_E_INVALID, "address 0x%llx not in this arena", (unsigned long long)addr);
    a->free[cls].push_back(addr);
    return PHX_OK;
}

int phx_arena_can_alloc(phx_arena a, size_t bytes) {
    if (!a) return 0;
    size_t c = phx_size_class(bytes);
    auto it = a->free.find(c);
    if (it != a->free.end() && !it->second.empty()) return 1;
    size_t off = (a->bump + kAlign - 1) & ~(kAlign - 1);
    return off + c <= a->cap ? 1 : 0;
}

int phx_arena_stats(phx_arena a, size_t *cap, size_t *bump, uint64_t *base) {
    if (!a) return set_error(PHX_E_INVALID, "null arena");
    if (cap) *cap = a->cap;
    if (bump) *bump = a->bump;
    if (base) *base = a->base;
    return PHX_OK;
}

}  // extern "C"
