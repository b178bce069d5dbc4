// The loopback job's elementwise add leaf, c = a + b on f32 vectors
// (phobos-pod/examples/loopback.rs:24-30, kernel `add`, checked there bit for
// bit against the host's f32 sum at :135-156).
//
// Not one of the bench kernels: it is the kernel a caller hands the pod as a
// code object of its own (phx_module_load_data / phx_module_get_function,
// then phx_pod_set_kernel_function), which is how the pod runs kernels that
// are not built in.  The pod launches it with the COMPUTE's own grid and cta,
// like any kernel the reference's engine receives, so it strides over its
// extent with whatever grid arrives.  i32 exploded-memref descriptors (the
// pod leaves' default index width, phobos-sched/src/server.rs:696-714).
#include "phx_common.h"

extern "C" __global__ void add(PHX_MEMREF1(float, a, int32_t), PHX_MEMREF1(float, b, int32_t),
                               PHX_MEMREF1(float, c, int32_t)) {
    const int64_t n = c_s0;
    if (a_s0 != n || b_s0 != n) return;
    const float *A = a_ptr + a_off;
    const float *B = b_ptr + b_off;
    float *C = c_ptr + c_off;
    const int64_t step = (int64_t)phx_block_count() * blockDim.x;
    for (int64_t i = (int64_t)phx_block_linear() * blockDim.x + threadIdx.x; i < n; i += step)
        C[i * c_st0] = A[i * a_st0] + B[i * b_st0];
}
