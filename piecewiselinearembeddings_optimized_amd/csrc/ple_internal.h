// Host-side interfaces between the translation units of libple_hip.so.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <stddef.h>
#include <stdint.h>

#include "../../include/ple_hip.h"

namespace ple {

constexpr size_t kLdsMax = 160 * 1024;   // LDS per workgroup on gfx950
// Largest max_n_bins the entry points take (bin indices are int32 beyond
// 32768 bins, as in the reference; every table offset is 64-bit).
constexpr int64_t kMaxBins = int64_t{1} << 24;

int device_cu_count();

// Current value of a PLE_TUNE_* planner override (0: the planner's choice).
int tuning(int knob);
// Changes whenever a tuning knob is set (plans cached under an older epoch
// are stale).
uint32_t tuning_epoch();

// Kernel timing (ple_timing_*): the start / stop events of the next timed
// launch of timer `which` (PLE_TIMER_*), or two NULLs when timing is off or
// its slots are used up.  The events go to hipExtLaunchKernelGGL, which
// records them at the kernel's start and end; the launcher then commits the
// slot (timer_commit), and only committed slots are read back, so a launch
// that was never issued leaves no unrecorded events behind.
struct TimerSlot {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    int which = -1;
    int index = -1;
};
TimerSlot timer_slot(int which);
void timer_commit(const TimerSlot &ts);

inline int idx_bytes_for(int64_t B) { return B <= 256 ? 1 : (B <= 32768 ? 2 : 4); }

inline bool valid_dtype(int d) { return d == PLE_DTYPE_F32 || d == PLE_DTYPE_F16 || d == PLE_DTYPE_BF16; }

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct ForwardRequest {
    const float *x, *edges, *iw;
    const int32_t *nbins;
    const float *weight, *bias;
    const float *lin_w = nullptr, *lin_b = nullptr;   // version-B linear0
    int relu = 0;
    uint32_t *mask = nullptr;                          // ReLU pass bits
    void *out, *idx;
    int64_t N, F, B, D;
    int quant, out_dtype;
    hipStream_t stream;
};

// Validated request -> launch.  Returns PLE_OK, PLE_E_* or a hipError_t.
int forward_run(const ForwardRequest &r);

struct BackwardRequest {
    const void *g;
    const float *x, *edges, *iw;
    const int32_t *nbins;
    const float *weight;
    const void *idx;
    float *dx, *dw, *db;
    const uint32_t *mask = nullptr;    // ReLU pass bits of the forward
    int relu = 0;
    const float *lin_w = nullptr;      // version-B linear0 weight
    float *dlw = nullptr;              // its gradient (db then holds linear0's bias gradient)
    int64_t N, F, B, D;
    int grad_dtype, quant;
    void *workspace;
    size_t workspace_bytes;
    hipStream_t stream;
};

size_t backward_workspace_bytes(int64_t N, int64_t F, int64_t B, int64_t D);
int backward_run(const BackwardRequest &r);
// The plan backward_run would take (r's pointers other than g and the
// outputs are not read).
int backward_plan_info(const BackwardRequest &r, ple_backward_plan_info_t *info);

struct EncodeRequest {
    const float *x, *edges, *iw;
    const int32_t *nbins, *offsets;
    const float *g = nullptr;    // backward: grad_output [N, T]
    float *out;                  // forward: encoding [N, T]; backward: grad_x [N, F]
    int64_t N, F, B, T;
    hipStream_t stream;
};

int encode_run(const EncodeRequest &r);
int encode_backward_run(const EncodeRequest &r);

}  // namespace ple
