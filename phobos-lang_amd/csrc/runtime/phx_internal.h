// Internal declarations shared by the runtime translation units.
#pragma once
#include <hip/hip_runtime.h>

#include "../kernels/phx_geometry.h"
#include "phobos_hip.h"

namespace phx {
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_error(hipError_t e, const char *what);
int builtin(phx_kernel k, hipFunction_t *out);
int check_shape(phx_kernel k, const int64_t *d, int nd);
int grid_for(phx_kernel k, const int64_t *d, int nd, uint32_t grid[3], uint32_t block[3]);
int kernel_abi(phx_kernel k, int *bits, uint32_t block[3]);
int launch_raw(hipFunction_t f, const uint32_t grid[3], const uint32_t block[3], uint32_t shmem,
               hipStream_t s, void **args);
}  // namespace phx
