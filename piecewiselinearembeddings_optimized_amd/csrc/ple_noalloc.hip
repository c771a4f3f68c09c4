// ple_backward_launch_noalloc: the backward entry point for callers that
// cannot allocate device memory.  Its workspace is `scratch`, a file-scope
// device array of kScratchBytes that every GPU the library runs on holds
// until the process ends.
//
// In host code `scratch` names a host-side stand-in, not device memory: the
// device address comes from hipGetSymbolAddress, once per device (with that
// device current), and only that address is handed to the kernels.  All
// calls on one GPU share its array; the backward needs no initialised
// workspace, so nothing is cleared between calls, and calls that overlap on
// one GPU (different streams, or host threads) race on it.

#include <mutex>

#include "ple_internal.h"

static __device__ __align__(256) unsigned char scratch[PLE_NOALLOC_SCRATCH_BYTES];

namespace ple {
namespace {

constexpr size_t kScratchBytes = PLE_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call for that device).  PLE_OK or an error code.
int scratch_address(void **out) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (dev < 0 || dev >= kMaxDevices) return PLE_E_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        const hipError_t ge = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (ge != hipSuccess) return static_cast<int>(ge);
        if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return PLE_OK;
}

}  // namespace
}  // namespace ple

extern "C" {

int ple_backward_launch_noalloc(const void *grad_output, const float *x, const float *bin_edges,
                                const float *inv_bin_widths, const int32_t *n_bins, const float *weight,
                                const void *bin_indices, float *grad_x, float *grad_weight, float *grad_bias,
                                int64_t N, int64_t F, int64_t B, int64_t D, int grad_dtype, int quant_dtype,
                                void *stream) {
    // (sizes the C ABI rejects report 0 here and are rejected below)
    const size_t need = ple_backward_workspace_bytes(N, F, B, D);
    if (need > ple::kScratchBytes) return PLE_E_SCRATCH_LIMIT;
    void *ws = nullptr;
    if (need > 0) {
        const int rc = ple::scratch_address(&ws);
        if (rc != PLE_OK) return rc;
    }
    return ple_backward_launch(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices, grad_x,
                               grad_weight, grad_bias, N, F, B, D, grad_dtype, quant_dtype, ws, need, stream);
}

}  // extern "C"
