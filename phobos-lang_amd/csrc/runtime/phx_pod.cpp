// placeholder, replaced by the segment executor
#include "phx_internal.h"
using namespace phx;
struct phx_pod_s {};
extern "C" {
int phx_pod_create(phx_pod *, size_t, int) { return set_error(PHX_E_INVALID, "pod: not built yet"); }
int phx_pod_destroy(phx_pod) { return PHX_OK; }
int phx_pod_set_tensor(phx_pod, uint32_t, const char *, const uint64_t *, uint32_t) { return set_error(PHX_E_INVALID, "pod: not built yet"); }
int phx_pod_set_kernel(phx_pod, uint32_t, phx_kernel) { return set_error(PHX_E_INVALID, "pod: not built yet"); }
int phx_pod_run_segment(phx_pod, const char *, uint64_t *) { return set_error(PHX_E_INVALID, "pod: not built yet"); }
}
