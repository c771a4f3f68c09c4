// The extern "C" entry points of include/ple_hip.h: argument checks that need
// no device, then the forward / backward launchers.

#include <atomic>
#include <mutex>
#include <vector>

#include "ple_internal.h"

namespace ple {

int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

namespace {

std::atomic<int> g_tuning[PLE_TUNE_COUNT];
std::atomic<uint32_t> g_tuning_epoch{0};

}  // namespace

int tuning(int knob) { return g_tuning[knob].load(std::memory_order_relaxed); }

uint32_t tuning_epoch() { return g_tuning_epoch.load(std::memory_order_relaxed); }

// Kernel timing: per timer, event pairs {begin, end} for up to `slots`
// launches, recorded on the launch stream around the main kernel.
namespace {

struct Timer {
    std::vector<hipEvent_t> ev;   // 2 * slots events: begin and end of launch i
    std::vector<char> done;       // slot i's launch was issued (its events are recorded)
    int slots = 0;
    int used = 0;
};

std::atomic<bool> g_timing{false};
std::mutex g_timer_mu;
Timer g_timers[PLE_TIMER_COUNT];

// Waits for every recorded stop event (launches still in flight record
// them), then destroys the events.
void timers_release() {
    for (Timer &t : g_timers) {
        for (int i = 0; i < t.used; ++i)
            if (t.done[i]) (void)hipEventSynchronize(t.ev[2 * i + 1]);
        for (hipEvent_t e : t.ev) (void)hipEventDestroy(e);
        t.ev.clear();
        t.done.clear();
        t.slots = t.used = 0;
    }
}

}  // namespace

TimerSlot timer_slot(int which) {
    if (!g_timing.load(std::memory_order_relaxed)) return TimerSlot{};
    std::lock_guard<std::mutex> lk(g_timer_mu);
    Timer &t = g_timers[which];
    if (t.used >= t.slots) return TimerSlot{};
    const TimerSlot ts{t.ev[2 * t.used], t.ev[2 * t.used + 1], which, t.used};
    t.done[t.used] = 0;
    ++t.used;
    return ts;
}

void timer_commit(const TimerSlot &ts) {
    if (ts.which < 0) return;
    std::lock_guard<std::mutex> lk(g_timer_mu);
    Timer &t = g_timers[ts.which];
    // (a slot of timers released in the meantime is gone)
    if (ts.index < t.used && t.ev[2 * ts.index] == ts.start) t.done[ts.index] = 1;
}

namespace {

// Zeros n floats (a kernel rather than hipMemsetAsync, so that a caller may
// capture the launch in a graph).
__global__ __launch_bounds__(256) void ple_zero_kernel(float *p, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256)
        p[i] = 0.0f;
}

hipError_t zero_floats(float *p, int64_t n, hipStream_t s) {
    if (!p || n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(ple_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

int check_common(int64_t N, int64_t F, int64_t B, int64_t D) {
    if (N < 0 || F < 1 || B < 1 || D < 1) return PLE_E_BAD_SHAPE;
    // (the kernels index per-feature tables and rows with 32-bit offsets)
    if (F > INT32_MAX / 2 || B > kMaxBins || D > INT32_MAX / 2) return PLE_E_TOO_LARGE;
    if (F * (B + 1) > INT32_MAX / 2 || F * B * 2 * D > INT32_MAX) return PLE_E_TOO_LARGE;
    if (N > INT64_MAX / (F * D)) return PLE_E_TOO_LARGE;
    return PLE_OK;
}

}  // namespace
}  // namespace ple

extern "C" {

int ple_abi_version(void) { return (1 << 16) | 4; }

int ple_bin_index_bytes(int64_t max_n_bins) { return ple::idx_bytes_for(max_n_bins); }

int ple_set_tuning(int knob, int value) {
    if (knob < 0 || knob >= PLE_TUNE_COUNT) return PLE_E_BAD_SHAPE;
    const int prev = ple::g_tuning[knob].exchange(value, std::memory_order_relaxed);
    ple::g_tuning_epoch.fetch_add(1, std::memory_order_relaxed);
    return prev;
}

int ple_timing_start(int slots) {
    if (slots < 0) return PLE_E_BAD_SHAPE;
    std::lock_guard<std::mutex> lk(ple::g_timer_mu);
    ple::g_timing.store(false, std::memory_order_relaxed);
    ple::timers_release();
    if (slots == 0) return PLE_OK;
    for (ple::Timer &t : ple::g_timers) {
        t.ev.resize(2 * static_cast<size_t>(slots), nullptr);
        t.done.assign(static_cast<size_t>(slots), 0);
        for (hipEvent_t &e : t.ev) {
            const hipError_t rc = hipEventCreate(&e);
            if (rc != hipSuccess) {
                e = nullptr;
                ple::timers_release();
                return static_cast<int>(rc);
            }
        }
        t.slots = slots;
    }
    ple::g_timing.store(true, std::memory_order_relaxed);
    return PLE_OK;
}

int ple_timing_stop(void) {
    ple::g_timing.store(false, std::memory_order_relaxed);
    return PLE_OK;
}

int ple_timing_read(int which, double *ms_total, int *count) {
    if (which < 0 || which >= PLE_TIMER_COUNT) return PLE_E_BAD_SHAPE;
    if (!ms_total || !count) return PLE_E_NULL_POINTER;
    std::lock_guard<std::mutex> lk(ple::g_timer_mu);
    const ple::Timer &t = ple::g_timers[which];
    double sum = 0.0;
    int n = 0;
    for (int i = 0; i < t.used; ++i) {
        if (!t.done[i]) continue;   // (the launch was not issued)
        hipError_t rc = hipEventSynchronize(t.ev[2 * i + 1]);
        float ms = 0.0f;
        if (rc == hipSuccess) rc = hipEventElapsedTime(&ms, t.ev[2 * i], t.ev[2 * i + 1]);
        if (rc != hipSuccess) return static_cast<int>(rc);
        sum += ms;
        ++n;
    }
    *ms_total = sum;
    *count = n;
    return PLE_OK;
}

const char *ple_error_string(int code) {
    switch (code) {
        case PLE_OK: return "success";
        case PLE_E_NULL_POINTER: return "a required pointer is NULL";
        case PLE_E_BAD_SHAPE: return "invalid shape (need N >= 0 and F, B, D >= 1)";
        case PLE_E_BAD_DTYPE: return "invalid dtype code";
        case PLE_E_BAD_INDEX_WIDTH: return "invalid bin index width";
        case PLE_E_TOO_LARGE:
            return "sizes exceed the supported range (max_n_bins <= 2^24, F * max_n_bins * D < 2^30; "
                   "module epilogues with ReLU or linear0: D <= 64)";
        case PLE_E_WORKSPACE: return "workspace is NULL, too small or not 256-byte aligned";
        case PLE_E_UNSUPPORTED: return "combination not supported (dtype or epilogue pairing)";
        case PLE_E_MISALIGNED: return "pointer misaligned for its element type";
        case PLE_E_SCRATCH_LIMIT:
            return "the sizes need more workspace than the no-allocation entry point's static scratch holds";
        default: break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "unknown error";
}

int ple_forward_launch(const float *x, const float *bin_edges, const float *inv_bin_widths,
                       const int32_t *n_bins, const float *weight, const float *bias,
                       void *output, void *bin_indices, int64_t N, int64_t F, int64_t B,
                       int64_t D, int quant_dtype, int output_dtype, void *stream) {
    const int rc = ple::check_common(N, F, B, D);
    if (rc != PLE_OK) return rc;
    if (!ple::valid_dtype(quant_dtype) || !ple::valid_dtype(output_dtype)) return PLE_E_BAD_DTYPE;
    if (N == 0) return PLE_OK;
    if (!x || !bin_edges || !inv_bin_widths || !n_bins || !weight || !output || !bin_indices)
        return PLE_E_NULL_POINTER;
    ple::ForwardRequest r;
    r.x = x; r.edges = bin_edges; r.iw = inv_bin_widths; r.nbins = n_bins; r.weight = weight;
    r.bias = bias; r.out = output; r.idx = bin_indices;
    r.N = N; r.F = F; r.B = B; r.D = D;
    r.quant = quant_dtype; r.out_dtype = output_dtype;
    r.stream = static_cast<hipStream_t>(stream);
    return ple::forward_run(r);
}

size_t ple_backward_workspace_bytes(int64_t N, int64_t F, int64_t B, int64_t D) {
    if (ple::check_common(N, F, B, D) != PLE_OK || N == 0) return 0;
    return ple::backward_workspace_bytes(N, F, B, D);
}

int ple_backward_launch(const void *grad_output, const float *x, const float *bin_edges,
                        const float *inv_bin_widths, const int32_t *n_bins,
                        const float *weight, const void *bin_indices, float *grad_x,
                        float *grad_weight, float *grad_bias, int64_t N, int64_t F,
                        int64_t B, int64_t D, int grad_dtype, int quant_dtype,
                        void *workspace, size_t workspace_bytes, void *stream) {
    const int rc = ple::check_common(N, F, B, D);
    if (rc != PLE_OK) return rc;
    if (!ple::valid_dtype(grad_dtype) || !ple::valid_dtype(quant_dtype)) return PLE_E_BAD_DTYPE;
    if (!grad_x && !grad_weight && !grad_bias) return PLE_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (N == 0) {
        // empty batch: the parameter gradients are zero
        hipError_t e = hipSuccess;
        if (grad_weight) e = ple::zero_floats(grad_weight, F * B * D, s);
        if (e == hipSuccess && grad_bias) e = ple::zero_floats(grad_bias, F * D, s);
        return e == hipSuccess ? PLE_OK : static_cast<int>(e);
    }
    if (!grad_output || !x || !bin_edges || !inv_bin_widths || !n_bins || !weight || !bin_indices)
        return PLE_E_NULL_POINTER;
    ple::BackwardRequest r;
    r.g = grad_output; r.x = x; r.edges = bin_edges; r.iw = inv_bin_widths; r.nbins = n_bins;
    r.weight = weight; r.idx = bin_indices; r.dx = grad_x; r.dw = grad_weight; r.db = grad_bias;
    r.N = N; r.F = F; r.B = B; r.D = D;
    r.grad_dtype = grad_dtype; r.quant = quant_dtype;
    r.workspace = workspace; r.workspace_bytes = workspace_bytes;
    r.stream = s;
    return ple::backward_run(r);
}

int ple_backward_plan_query(const void *grad_output, int64_t N, int64_t F, int64_t B, int64_t D,
                            int grad_dtype, int quant_dtype, int relu, int linear0,
                            ple_backward_plan_info_t *info) {
    const int rc = ple::check_common(N, F, B, D);
    if (rc != PLE_OK) return rc;
    if (!ple::valid_dtype(grad_dtype) || !ple::valid_dtype(quant_dtype)) return PLE_E_BAD_DTYPE;
    if (!info) return PLE_E_NULL_POINTER;
    if (grad_dtype != PLE_DTYPE_F32 && (quant_dtype != grad_dtype || relu || linear0)) return PLE_E_UNSUPPORTED;
    ple::BackwardRequest r{};
    // (any 16-byte aligned address stands for "aligned" when no gradient is given)
    r.g = grad_output ? grad_output : reinterpret_cast<const void *>(static_cast<uintptr_t>(256));
    static const float lin_marker = 0.0f;
    r.lin_w = linear0 ? &lin_marker : nullptr;
    r.relu = relu ? 1 : 0;
    r.N = N; r.F = F; r.B = B; r.D = D;
    r.grad_dtype = grad_dtype; r.quant = quant_dtype;
    return ple::backward_plan_info(r, info);
}

int ple_forward_epilogue_launch(const float *x, const float *bin_edges, const float *inv_bin_widths,
                                const int32_t *n_bins, const float *weight,
                                const ple_epilogue_t *epilogue, float *output, void *bin_indices,
                                int64_t N, int64_t F, int64_t B, int64_t D, int quant_dtype,
                                void *stream) {
    const int rc = ple::check_common(N, F, B, D);
    if (rc != PLE_OK) return rc;
    if (!ple::valid_dtype(quant_dtype)) return PLE_E_BAD_DTYPE;
    if (!epilogue) return PLE_E_NULL_POINTER;
    if ((epilogue->bias != nullptr) == (epilogue->lin_weight != nullptr)) return PLE_E_UNSUPPORTED;
    if (epilogue->lin_weight && !epilogue->lin_bias) return PLE_E_NULL_POINTER;
    if (N == 0) return PLE_OK;
    if (!x || !bin_edges || !inv_bin_widths || !n_bins || !weight || !output || !bin_indices)
        return PLE_E_NULL_POINTER;
    ple::ForwardRequest r;
    r.x = x; r.edges = bin_edges; r.iw = inv_bin_widths; r.nbins = n_bins; r.weight = weight;
    r.bias = epilogue->bias; r.lin_w = epilogue->lin_weight; r.lin_b = epilogue->lin_bias;
    r.relu = epilogue->relu ? 1 : 0; r.mask = epilogue->relu_mask;
    r.out = output; r.idx = bin_indices;
    r.N = N; r.F = F; r.B = B; r.D = D;
    r.quant = quant_dtype; r.out_dtype = PLE_DTYPE_F32;
    r.stream = static_cast<hipStream_t>(stream);
    return ple::forward_run(r);
}

int ple_backward_epilogue_launch(const float *grad_output, const float *x, const float *bin_edges,
                                 const float *inv_bin_widths, const int32_t *n_bins,
                                 const float *weight, const void *bin_indices,
                                 const ple_epilogue_t *epilogue, float *grad_x, float *grad_weight,
                                 float *grad_bias, float *grad_lin_weight, float *grad_lin_bias,
                                 int64_t N, int64_t F, int64_t B, int64_t D, int quant_dtype,
                                 void *workspace, size_t workspace_bytes, void *stream) {
    const int rc = ple::check_common(N, F, B, D);
    if (rc != PLE_OK) return rc;
    if (!ple::valid_dtype(quant_dtype)) return PLE_E_BAD_DTYPE;
    if (!epilogue) return PLE_E_NULL_POINTER;
    const bool lin = epilogue->lin_weight != nullptr;   // else version A (bias, lin_bias: not read)
    if (lin ? grad_bias != nullptr : (grad_lin_weight != nullptr || grad_lin_bias != nullptr))
        return PLE_E_UNSUPPORTED;
    float *db = lin ? grad_lin_bias : grad_bias;
    if (!grad_x && !grad_weight && !db && !grad_lin_weight) return PLE_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (N == 0) {
        hipError_t e = hipSuccess;
        if (grad_weight) e = ple::zero_floats(grad_weight, F * B * D, s);
        if (e == hipSuccess && db) e = ple::zero_floats(db, F * D, s);
        if (e == hipSuccess && grad_lin_weight) e = ple::zero_floats(grad_lin_weight, F * D, s);
        return e == hipSuccess ? PLE_OK : static_cast<int>(e);
    }
    if (!grad_output || !x || !bin_edges || !inv_bin_widths || !n_bins || !weight || !bin_indices)
        return PLE_E_NULL_POINTER;
    if (epilogue->relu && !epilogue->relu_mask) return PLE_E_NULL_POINTER;
    ple::BackwardRequest r;
    r.g = grad_output; r.x = x; r.edges = bin_edges; r.iw = inv_bin_widths; r.nbins = n_bins;
    r.weight = weight; r.idx = bin_indices; r.dx = grad_x; r.dw = grad_weight; r.db = db;
    r.relu = epilogue->relu ? 1 : 0; r.mask = epilogue->relu_mask;
    r.lin_w = epilogue->lin_weight; r.dlw = grad_lin_weight;
    r.N = N; r.F = F; r.B = B; r.D = D;
    r.grad_dtype = PLE_DTYPE_F32; r.quant = quant_dtype;
    r.workspace = workspace; r.workspace_bytes = workspace_bytes;
    r.stream = s;
    return ple::backward_run(r);
}

int ple_encode_launch(const float *x, const float *bin_edges, const float *inv_bin_widths,
                      const int32_t *n_bins, const int32_t *offsets, float *output, int64_t N,
                      int64_t F, int64_t B, int64_t total_bins, void *stream) {
    const int rc = ple::check_common(N, F, B, 1);
    if (rc != PLE_OK) return rc;
    if (total_bins < 1) return PLE_E_BAD_SHAPE;
    if (N == 0) return PLE_OK;
    if (N > INT64_MAX / total_bins) return PLE_E_TOO_LARGE;
    if (!x || !bin_edges || !inv_bin_widths || !n_bins || !offsets || !output) return PLE_E_NULL_POINTER;
    ple::EncodeRequest r;
    r.x = x; r.edges = bin_edges; r.iw = inv_bin_widths; r.nbins = n_bins; r.offsets = offsets;
    r.out = output;
    r.N = N; r.F = F; r.B = B; r.T = total_bins;
    r.stream = static_cast<hipStream_t>(stream);
    return ple::encode_run(r);
}

int ple_encode_backward_launch(const float *grad_output, const float *x, const float *bin_edges,
                               const float *inv_bin_widths, const int32_t *n_bins,
                               const int32_t *offsets, float *grad_x, int64_t N, int64_t F,
                               int64_t B, int64_t total_bins, void *stream) {
    const int rc = ple::check_common(N, F, B, 1);
    if (rc != PLE_OK) return rc;
    if (total_bins < 1) return PLE_E_BAD_SHAPE;
    if (N == 0) return PLE_OK;
    if (N > INT64_MAX / total_bins) return PLE_E_TOO_LARGE;
    if (!grad_output || !x || !bin_edges || !inv_bin_widths || !n_bins || !offsets || !grad_x)
        return PLE_E_NULL_POINTER;
    ple::EncodeRequest r;
    r.g = grad_output; r.x = x; r.edges = bin_edges; r.iw = inv_bin_widths; r.nbins = n_bins;
    r.offsets = offsets; r.out = grad_x;
    r.N = N; r.F = F; r.B = B; r.T = total_bins;
    r.stream = static_cast<hipStream_t>(stream);
    return ple::encode_backward_run(r);
}

}  // extern "C"
