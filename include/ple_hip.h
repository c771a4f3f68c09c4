/*
 * C ABI of the MI355X (gfx950) piecewise-linear-embedding kernels.
 *
 * Plain pointers and sizes only; every device pointer refers to memory on the
 * device that is current on the calling thread, and every launch is enqueued
 * on `stream` (a hipStream_t; NULL = the null stream).  No entry point
 * allocates device memory or synchronises the host: scratch space is passed in
 * by the caller (see ple_backward_workspace_bytes).
 *
 * Return value: PLE_OK (0), a negative PLE_E_* argument error, or a positive
 * hipError_t from the launch.  ple_error_string() names every code.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   ple_forward_launch   <- ple_forward_cuda   csrc/forward_cuda.cu:687-860
 *                           (registered at csrc/ops.cpp:35-44, :62-75)
 *   ple_backward_launch  <- ple_backward_cuda  csrc/backward_cuda.cu:1528-1725
 *                           (registered at csrc/ops.cpp:46-58, :62-75)
 *   ple_encode_launch / ple_encode_backward_launch
 *                        <- upstream rtdl_num_embeddings.PiecewiseLinearEncoding
 *                           (external dependency of the reference, pinned at
 *                           requirements.txt:1; no operator counterpart)
 *   ple_forward_epilogue_launch / ple_backward_epilogue_launch
 *                        <- the module tail run as PyTorch ops after the
 *                           forward operator, src/rtdl_num_embeddings_cuda/
 *                           module.py:230-248 (no operator counterpart)
 * The reference exposes these only through the torch dispatcher; this ABI is
 * the layer under this build's own dispatcher registration, and is what a
 * ctypes / cgo / JNI binding would call.
 */
#ifndef PLE_HIP_H_
#define PLE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
enum {
    PLE_DTYPE_F32 = 0,
    PLE_DTYPE_F16 = 1,
    PLE_DTYPE_BF16 = 2,
};

/* error codes (negative: rejected before any launch) */
enum {
    PLE_OK = 0,
    PLE_E_NULL_POINTER = -1,
    PLE_E_BAD_SHAPE = -2,
    PLE_E_BAD_DTYPE = -3,
    PLE_E_BAD_INDEX_WIDTH = -4,
    PLE_E_TOO_LARGE = -5,
    PLE_E_WORKSPACE = -6,
    PLE_E_UNSUPPORTED = -7,
    PLE_E_MISALIGNED = -8,
    PLE_E_SCRATCH_LIMIT = -9,
};

/* Bytes of bin index per (sample, feature) for a given max_n_bins:
 * 1 up to 256 bins, 2 up to 32768, else 4 (reference _meta.py:14-19). */
int ple_bin_index_bytes(int64_t max_n_bins);

/*
 * Forward: for every (n, f)
 *   k      = searchsorted(bin_edges[f, :n_bins[f]+1], x[n, f], right) - 1,
 *            clamped to [0, n_bins[f]-1]                 -> bin_indices[n, f]
 *   frac   = (x[n, f] - bin_edges[f, k]) * inv_bin_widths[f, k]
 *   r      = fma(q(frac), q(weight[f, phys(k), :]), sum_{j<k} q(weight[f, j, :]))
 *   out    = round_quant(r) (+ bias[f, :])               -> output[n, f, :]
 * with q / round_quant = round trip through quant_dtype and
 * phys(k) = (k == n_bins[f]-1) ? max_n_bins-1 : k.
 *
 *   x               float32 [N, F]
 *   bin_edges       float32 [F, B+1]  (+inf padded past n_bins[f])
 *   inv_bin_widths  float32 [F, B]    (0 padded)
 *   n_bins          int32   [F]       (1 <= n_bins[f] <= B)
 *   weight          float32 [F, B, D]
 *   bias            float32 [F, D] or NULL (added after quantisation)
 *   output          output_dtype [N, F, D]
 *   bin_indices     [N, F] of ple_bin_index_bytes(B) bytes each (uint8 /
 *                   int16 / int32)
 *   quant_dtype     PLE_DTYPE_* used for q() and round_quant()
 *   output_dtype    PLE_DTYPE_* of the stored output
 * Supported pairings: output_dtype == quant_dtype with bias NULL (the
 * reference operator), or output_dtype == PLE_DTYPE_F32 with a bias (the
 * module's "x_ple + bias" fused into the store); others -> PLE_E_UNSUPPORTED.
 * N may be 0 (no launch).  F, B, D >= 1, any D (as the reference operator,
 * csrc/forward_cuda.cu:764-766: only the reference module asserts D <= 64);
 * B <= 2^24 and F * B * D < 2^30 (else PLE_E_TOO_LARGE).  Every such shape
 * runs: per-feature tables that fit LDS take the table kernel, larger ones
 * (many bins times a wide row) a kernel that keeps prefix checkpoints in LDS
 * and reads the weights from global memory -- bit-identical results; rows of
 * more than 64 lanes' columns are split into column chunks.
 */
int ple_forward_launch(const float *x, const float *bin_edges, const float *inv_bin_widths,
                       const int32_t *n_bins, const float *weight, const float *bias,
                       void *output, void *bin_indices, int64_t N, int64_t F, int64_t B,
                       int64_t D, int quant_dtype, int output_dtype, void *stream);

/* Scratch bytes ple_backward_launch needs for these sizes (0 is possible). */
size_t ple_backward_workspace_bytes(int64_t N, int64_t F, int64_t B, int64_t D);

/*
 * Backward of ple_forward_launch.
 *   grad_x[n, f]  = iw_k * <g, q(W[f, phys(k)])>
 *                   + [k > 0 and x == e_k] * iw_{k-1} * <g, q(W[f, k-1])>
 *   grad_weight[f, phys(k)] = sum_{bin=k} q(frac) g + sum_{bin>k} g
 *                   (slots no bin maps to are written as 0)
 *   grad_bias[f]  = sum_n grad_output[n, f]   (unrounded grad_output)
 * where g = grad_output rounded through quant_dtype (identity for F32).
 * Supported pairings: quant_dtype == grad_dtype (the reference operator,
 * whose gradient arrives in the forward's output dtype), or grad_dtype ==
 * PLE_DTYPE_F32 with any quant_dtype; others -> PLE_E_UNSUPPORTED.
 * Each of grad_x / grad_weight / grad_bias may be NULL (not computed).
 * Reductions are deterministic: a fixed summation order, no atomics on
 * floating-point data.
 *
 *   grad_output     grad_dtype [N, F, D]
 *   bin_indices     as produced by ple_forward_launch
 *   workspace       >= ple_backward_workspace_bytes(N, F, B, D) bytes,
 *                   256-byte aligned, contents need not be initialised
 * Shapes as for ple_forward_launch; all of them run (tables beyond the
 * sorted path's LDS take deterministic fallback kernels).
 */
int ple_backward_launch(const void *grad_output, const float *x, const float *bin_edges,
                        const float *inv_bin_widths, const int32_t *n_bins,
                        const float *weight, const void *bin_indices, float *grad_x,
                        float *grad_weight, float *grad_bias, int64_t N, int64_t F,
                        int64_t B, int64_t D, int grad_dtype, int quant_dtype,
                        void *workspace, size_t workspace_bytes, void *stream);

/*
 * ple_backward_launch without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a static device array of PLE_NOALLOC_SCRATCH_BYTES that each
 * GPU the library runs on holds until the process ends; sizes whose
 * ple_backward_workspace_bytes exceed it return PLE_E_SCRATCH_LIMIT before
 * any launch.  Nothing is allocated or freed.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams, other host
 * threads) race.  Arguments and results as ple_backward_launch.
 */
#define PLE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int ple_backward_launch_noalloc(const void *grad_output, const float *x, const float *bin_edges,
                                const float *inv_bin_widths, const int32_t *n_bins, const float *weight,
                                const void *bin_indices, float *grad_x, float *grad_weight, float *grad_bias,
                                int64_t N, int64_t F, int64_t B, int64_t D, int grad_dtype, int quant_dtype,
                                void *stream);

/*
 * The backward's launch plan for a shape, for benchmarks and memory
 * accounting; no counterpart in the reference (its launcher picks private,
 * sorted or atomic dW paths internally, csrc/backward_cuda.cu:1141-1463, and
 * reports nothing).  grad_output: the gradient that will be passed (its
 * alignment picks the lane width; NULL = 16-byte aligned); relu / linear0:
 * the module epilogue of ple_backward_epilogue_launch (0 for
 * ple_backward_launch).  Fills *info; returns PLE_OK or PLE_E_*.
 *   sorted             1: the fused sort + reduce + dx kernel; 0: the
 *                      fallback dx and histogram kernels
 *   chunks             sample chunks with dW / db partials in the workspace
 *                      (sorted path with 1 chunk: the gradient kernel writes
 *                      grad_weight / grad_bias itself, no finalize kernel)
 *   features_per_group features per gradient-kernel workgroup (sorted and
 *                      matrix-core paths)
 *   columns_per_lane   gradient elements a lane holds per row (sorted path)
 *   lanes_per_row      lanes that share a row (sorted path)
 *   threads            gradient-kernel workgroup size
 *   lds_bytes          gradient-kernel LDS per workgroup
 *   workspace_bytes    workspace a launch that writes grad_weight / grad_bias
 *                      needs (0 for grad_x alone)
 *   bins_per_window    bins whose tables and histogram cells a workgroup holds
 *                      in LDS (sorted path; B when all of them fit)
 *   windows            workgroups per feature group, one per window of bins
 *                      (sorted path; 1 when all bins fit)
 *   matrix_cores       1: the histograms as one-hot products on the matrix
 *                      cores (16-bit gradients in their own dtype, rows of 8,
 *                      16, 24 or 32 columns, at most 96 bins, at most 8
 *                      chunks); sorted is 0 then
 */
typedef struct ple_backward_plan_info {
    int sorted;
    int chunks;
    int features_per_group;
    int columns_per_lane;
    int lanes_per_row;
    int threads;
    size_t lds_bytes;
    size_t workspace_bytes;
    int bins_per_window;
    int windows;
    int matrix_cores;
} ple_backward_plan_info_t;
int ple_backward_plan_query(const void *grad_output, int64_t N, int64_t F, int64_t B, int64_t D,
                            int grad_dtype, int quant_dtype, int relu, int linear0,
                            ple_backward_plan_info_t *info);

/*
 * Module epilogue fused into the kernels.  No counterpart in the reference's
 * operator API: the reference module runs this tail as separate PyTorch ops
 * after its forward operator (src/rtdl_num_embeddings_cuda/module.py:230-248).
 *   version A:  v = x_ple + bias;             out = relu ? relu(v) : v
 *   version B:  out = (lin_bias + lin_weight * x) + (relu ? relu(x_ple) : x_ple)
 * where x_ple is ple_forward_launch's output (rounded through quant_dtype) and
 * the arithmetic after it is fp32 (the output is float32).  relu follows
 * torch.relu: NaN passes, v <= 0 gives 0.  With relu, relu_mask holds one bit
 * per element, bit (j % 32) of word [n, f, j / 32] set where the ReLU passed
 * its input; the forward writes it (when non-NULL) and the backward reads it.
 */
typedef struct ple_epilogue {
    const float *bias;          /* [F, D] or NULL (version A) */
    const float *lin_weight;    /* [F, D] or NULL: linear0 weight (version B) */
    const float *lin_bias;      /* [F, D] linear0 bias, required with lin_weight */
    int relu;                   /* 0 or 1 */
    uint32_t *relu_mask;        /* [N, F, ceil(D / 32)] uint32, see above */
} ple_epilogue_t;

/* Forward with an epilogue: exactly one of bias / lin_weight non-NULL;
 * output float32 [N, F, D]; other arguments as ple_forward_launch. */
int ple_forward_epilogue_launch(const float *x, const float *bin_edges, const float *inv_bin_widths,
                                const int32_t *n_bins, const float *weight,
                                const ple_epilogue_t *epilogue, float *output, void *bin_indices,
                                int64_t N, int64_t F, int64_t B, int64_t D, int quant_dtype,
                                void *stream);

/*
 * Backward of ple_forward_epilogue_launch (grad_output float32 [N, F, D]).
 * With g_ple = relu ? grad_output * pass : grad_output, rounded through
 * quant_dtype for grad_x / grad_weight as in ple_backward_launch, and
 * grad_x += <grad_output[n, f], lin_weight[f]> for version B;
 *   grad_bias[f]       = sum_n g_ple (unrounded)         (version A)
 *   grad_lin_weight[f] = sum_n grad_output[n, f] * x[n, f] (version B)
 *   grad_lin_bias[f]   = sum_n grad_output[n, f]           (version B)
 * The backward reads lin_weight (non-NULL: version B, else version A), relu
 * and relu_mask; bias and lin_bias are not read.  Any gradient pointer may be
 * NULL; grad_bias must be NULL for version B and the linear0 gradients NULL
 * for version A.  The workspace is sized by ple_backward_workspace_bytes.
 */
int ple_backward_epilogue_launch(const float *grad_output, const float *x, const float *bin_edges,
                                 const float *inv_bin_widths, const int32_t *n_bins,
                                 const float *weight, const void *bin_indices,
                                 const ple_epilogue_t *epilogue, float *grad_x, float *grad_weight,
                                 float *grad_bias, float *grad_lin_weight, float *grad_lin_bias,
                                 int64_t N, int64_t F, int64_t B, int64_t D, int quant_dtype,
                                 void *workspace, size_t workspace_bytes, void *stream);

/*
 * Dense piecewise-linear encoding: the output of the upstream
 * PiecewiseLinearEncoding module (rtdl_num_embeddings==0.0.12), which the
 * reference's module builds on; no counterpart in the reference's operators.
 * For feature f (n_bins[f] = n bins, b and frac as in ple_forward_launch) the
 * n components at columns offsets[f] .. offsets[f] + n - 1 of row n are
 *   1 (k < b), frac (k == b), 0 (k > b);   NaN x: all NaN.
 *   offsets         int32 [F], offsets[f] = sum_{j<f} n_bins[j]
 *   output          float32 [N, total_bins], total_bins = sum_f n_bins[f]
 * F * 8 * 8 + 4 bytes of per-feature tables must fit LDS (F <= 2500).
 */
int ple_encode_launch(const float *x, const float *bin_edges, const float *inv_bin_widths,
                      const int32_t *n_bins, const int32_t *offsets, float *output, int64_t N,
                      int64_t F, int64_t B, int64_t total_bins, void *stream);

/* Backward of ple_encode_launch: grad_x[n, f] = g[n, offsets[f] + b] * iw_b
 * (+ g[n, offsets[f] + b - 1] * iw_{b-1} when b > 0 and x == e_b). */
int ple_encode_backward_launch(const float *grad_output, const float *x, const float *bin_edges,
                               const float *inv_bin_widths, const int32_t *n_bins,
                               const int32_t *offsets, float *grad_x, int64_t N, int64_t F,
                               int64_t B, int64_t total_bins, void *stream);

/*
 * Planner overrides, for tuning sweeps and for tests that run every kernel
 * form on the same inputs.  No counterpart in the reference (its launchers
 * have no knobs).  Each knob holds 0 -- the planner's own choice, the default
 * -- or a forced value, read by every later launch of the process:
 *   PLE_TUNE_FWD_FS         features per forward workgroup (power of two)
 *   PLE_TUNE_FWD_WG_PER_CU  forward workgroups per CU the chunking aims for
 *   PLE_TUNE_FWD_FB         forward workgroup size (256 or 512 threads)
 *   PLE_TUNE_FWD_VEC        outputs per lane (1, 2 or 4; 16-bit outputs 8)
 *   PLE_TUNE_FWD_WIDE       1: the wide-table forward kernel for any shape
 *   PLE_TUNE_BWD_SIMPLE     1: the fallback backward kernels for any shape
 *   PLE_TUNE_BWD_SIMPLE_GLOBAL 1: their histogram cells in global memory
 *   PLE_TUNE_BWD_VEC        1: one gradient element per lane; 4: at most four
 *                           (no 8-element lanes for 16-bit gradients)
 *   PLE_TUNE_BWD_FS         features per backward sub-tile (1, 2, 4, 8, 16;
 *                           the matrix-core backward's groups: 1, 2, 4)
 *   PLE_TUNE_BWD_RB         reducer threads per backward workgroup (256 or 512)
 *   PLE_TUNE_BWD_WG_PER_CU  backward workgroups per CU
 *   PLE_TUNE_BWD_MFMA       1: no matrix-core backward (the sorted path for
 *                           16-bit gradients too); 2: the matrix-core backward
 *                           for every shape it can take (also past 8 chunks)
 * A forced value the shape cannot take is ignored.  Returns the knob's
 * previous value, or PLE_E_BAD_SHAPE for an unknown knob.  Not synchronised
 * with launches running on other threads.
 */
enum {
    PLE_TUNE_FWD_FS = 0,
    PLE_TUNE_FWD_WG_PER_CU = 1,
    PLE_TUNE_FWD_FB = 2,
    PLE_TUNE_FWD_VEC = 3,
    PLE_TUNE_FWD_WIDE = 4,
    PLE_TUNE_BWD_SIMPLE = 5,
    PLE_TUNE_BWD_SIMPLE_GLOBAL = 6,
    PLE_TUNE_BWD_VEC = 7,
    PLE_TUNE_BWD_FS = 8,
    PLE_TUNE_BWD_RB = 9,
    PLE_TUNE_BWD_WG_PER_CU = 10,
    PLE_TUNE_BWD_MFMA = 11,
    PLE_TUNE_COUNT = 12,
};
int ple_set_tuning(int knob, int value);

/*
 * Kernel timing, for benchmarks; no counterpart in the reference.  After
 * ple_timing_start(slots), each of the next `slots` launches of the forward
 * (resp. backward) entry points records a HIP event pair on its stream around
 * its main kernel: PLE_TIMER_FORWARD brackets the forward kernel,
 * PLE_TIMER_BACKWARD the backward's gradient kernel (the sorted-path kernel,
 * or the fallback path's dx and histogram kernels), not the finalize that
 * turns its partials into grad_weight / grad_bias.  ple_timing_read waits for
 * the recorded pairs and returns their summed duration in milliseconds and
 * their number.  ple_timing_stop ends recording; ple_timing_start(0) also
 * releases the events.  The events belong to the device current at
 * ple_timing_start.  Returns PLE_OK, PLE_E_* or a hipError_t.
 */
enum {
    PLE_TIMER_FORWARD = 0,
    PLE_TIMER_BACKWARD = 1,
    PLE_TIMER_COUNT = 2,
};
int ple_timing_start(int slots);
int ple_timing_stop(void);
int ple_timing_read(int which, double *ms_total, int *count);

/* Human-readable name of a return code (static storage). */
const char *ple_error_string(int code);

/* ABI version of this header: (major << 16) | minor. */
int ple_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PLE_HIP_H_ */
