// Internal declarations shared by the runtime translation units.
#pragma once
#include <hip/hip_runtime.h>

#include "../kernels/phx_geometry.h"
#include "phobos_hip.h"

namespace phx {
// One exploded-memref descriptor read back out of a void** argument list, or
// built for a typed entry point.
struct Desc {
    uint64_t ptr = 0;  // aligned pointer + offset, in bytes
    int64_t size[3] = {0, 0, 0};
    int64_t stride[3] = {0, 0, 0};
};

int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_error(hipError_t e, const char *what);
int builtin(phx_kernel k, hipFunction_t *out);
int check_shape(phx_kernel k, const int64_t *d, int nd);
int grid_for(phx_kernel k, const int64_t *d, int nd, uint32_t grid[3], uint32_t block[3]);
int kernel_abi(phx_kernel k, int *bits, uint32_t block[3]);
int launch_raw(hipFunction_t f, const uint32_t grid[3], const uint32_t block[3], uint32_t shmem,
               hipStream_t s, void **args);
int aux_function(const char *file, const char *entry, hipFunction_t *out);
// split-key flash attention (phx_runtime.cpp)
int flash_split(phx_kernel k, int64_t BH, int64_t Nq, int64_t Nk);
size_t flash_split_bytes(int64_t BH, int64_t Nq, int sp);
int flash_split_functions(phx_kernel k, hipFunction_t *fs, hipFunction_t *fc);
int launch_flash_split_ws(phx_kernel k, const Desc *t, int rank, int64_t BH, int64_t Nq,
                          int64_t Nk, float scale, int sp, hipStream_t s, uint64_t ws,
                          hipFunction_t fs, hipFunction_t fc);
// the allocation-free entry point's per-device set-up (phx_scratch.hip)
int scratch_setup(int device);
void scratch_reset();
}  // namespace phx
