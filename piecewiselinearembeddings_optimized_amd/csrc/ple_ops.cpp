// PyTorch dispatcher registration of the PLE operators (the Python extension
// module `_C`).  Host code only: it validates the tensors, allocates outputs
// and scratch with the ATen caching allocator, and calls the C ABI of
// include/ple_hip.h on the caller's current HIP stream.  No host
// synchronisation happens here.
//
// Schemas `forward` and `backward` are the reference's, string for string
// (reference csrc/ops.cpp:35-58), registered for the device key that HIP
// tensors carry in PyTorch-ROCm (`CUDA`, reference csrc/ops.cpp:62-75).  The
// validation messages are the reference's too
// (csrc/forward_cuda.cu:695-790, csrc/backward_cuda.cu:1539-1657), so
// callers that match on them keep working.
//
// `forward_with_bias` / `backward_with_bias` are this build's additions: the
// same computation with the module's bias add fused into the output store
// (reference module.py:238-239 does it as a separate PyTorch op) and the bias
// gradient produced by the backward pass.  `forward_epilogue` /
// `backward_epilogue` fuse the module's whole tail (module.py:230-248): the
// bias and ReLU of version A, or the ReLU and the linear0 residual of
// version B; with ReLU the forward also returns one pass bit per element
// (int32 words [N, F, ceil(D / 32)]) for the backward.

#include <Python.h>

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <hip/hip_runtime_api.h>

#include <tuple>

#include "../../include/ple_hip.h"

namespace {

int ple_dtype_of(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return PLE_DTYPE_F32;
        case at::kHalf: return PLE_DTYPE_F16;
        case at::kBFloat16: return PLE_DTYPE_BF16;
        default: return -1;
    }
}

at::ScalarType bin_index_scalar_type(int64_t max_n_bins) {
    return max_n_bins <= 256 ? at::kByte : (max_n_bins <= 32768 ? at::kShort : at::kInt);
}

// Makes `index` the current HIP device for the scope (the launch enqueues on
// that device's current stream).
class DeviceScope {
   public:
    explicit DeviceScope(c10::DeviceIndex index) {
        TORCH_CHECK(hipGetDevice(&prev_) == hipSuccess, "hipGetDevice failed");
        if (prev_ != index) {
            TORCH_CHECK(hipSetDevice(index) == hipSuccess, "hipSetDevice failed");
            changed_ = true;
        }
    }
    ~DeviceScope() {
        if (changed_) (void)hipSetDevice(prev_);
    }
    DeviceScope(const DeviceScope &) = delete;
    DeviceScope &operator=(const DeviceScope &) = delete;

   private:
    int prev_ = 0;
    bool changed_ = false;
};

void check_rc(int rc, const char *what) {
    TORCH_CHECK(rc == PLE_OK, what, " failed: ", ple_error_string(rc), " (code ", rc, ")");
}

void *current_stream(const at::Tensor &t) {
    return static_cast<void *>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_forward_inputs(const at::Tensor &x, const at::Tensor &bin_edges,
                          const at::Tensor &inv_bin_widths, const at::Tensor &n_bins,
                          const at::Tensor &weight) {
    TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
    TORCH_CHECK(bin_edges.is_cuda(), "bin_edges must be a CUDA tensor");
    TORCH_CHECK(inv_bin_widths.is_cuda(), "inv_bin_widths must be a CUDA tensor");
    TORCH_CHECK(n_bins.is_cuda(), "n_bins must be a CUDA tensor");
    TORCH_CHECK(weight.is_cuda(), "weight must be a CUDA tensor");
    TORCH_CHECK(x.device() == bin_edges.device() && x.device() == inv_bin_widths.device() &&
                    x.device() == n_bins.device() && x.device() == weight.device(),
                "All forward tensors must be on the same CUDA device");
    TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
    TORCH_CHECK(bin_edges.is_contiguous(), "bin_edges must be contiguous");
    TORCH_CHECK(inv_bin_widths.is_contiguous(), "inv_bin_widths must be contiguous");
    TORCH_CHECK(n_bins.is_contiguous(), "n_bins must be contiguous");
    TORCH_CHECK(weight.is_contiguous(), "weight must be contiguous");
    TORCH_CHECK(x.dim() == 2, "x must have shape [N, F]");
    TORCH_CHECK(bin_edges.dim() == 2, "bin_edges must have shape [F, B + 1]");
    TORCH_CHECK(inv_bin_widths.dim() == 2, "inv_bin_widths must have shape [F, B]");
    TORCH_CHECK(n_bins.dim() == 1, "n_bins must have shape [F]");
    TORCH_CHECK(weight.dim() == 3, "weight must have shape [F, B, D]");
    TORCH_CHECK(x.scalar_type() == at::kFloat, "x must be float32");
    TORCH_CHECK(bin_edges.scalar_type() == at::kFloat, "bin_edges must be float32");
    TORCH_CHECK(inv_bin_widths.scalar_type() == at::kFloat, "inv_bin_widths must be float32");
    TORCH_CHECK(n_bins.scalar_type() == at::kInt, "n_bins must be int32");
    TORCH_CHECK(weight.scalar_type() == at::kFloat, "weight parameters must be float32");
    const int64_t n_features = x.size(1);
    const int64_t max_n_bins = weight.size(1);
    const int64_t d_embedding = weight.size(2);
    TORCH_CHECK(n_features > 0, "n_features must be positive");
    TORCH_CHECK(max_n_bins > 0, "max_n_bins must be positive");
    TORCH_CHECK(d_embedding > 0, "d_embedding must be positive");
    TORCH_CHECK(weight.size(0) == n_features, "weight.size(0) must equal x.size(1)");
    TORCH_CHECK(bin_edges.size(0) == n_features, "bin_edges.size(0) must equal x.size(1)");
    TORCH_CHECK(bin_edges.size(1) == max_n_bins + 1, "bin_edges.size(1) must equal max_n_bins + 1");
    TORCH_CHECK(inv_bin_widths.size(0) == n_features, "inv_bin_widths.size(0) must equal x.size(1)");
    TORCH_CHECK(inv_bin_widths.size(1) == max_n_bins, "inv_bin_widths.size(1) must equal max_n_bins");
    TORCH_CHECK(n_bins.size(0) == n_features, "n_bins.size(0) must equal x.size(1)");
}

std::tuple<at::Tensor, at::Tensor> run_forward(const at::Tensor &x, const at::Tensor &bin_edges,
                                               const at::Tensor &inv_bin_widths,
                                               const at::Tensor &n_bins, const at::Tensor &weight,
                                               const at::Tensor *bias, at::ScalarType quant_dtype,
                                               at::ScalarType output_dtype) {
    const int64_t N = x.size(0), F = x.size(1), B = weight.size(1), D = weight.size(2);
    DeviceScope scope(x.device().index());
    at::Tensor output = at::empty({N, F, D}, weight.options().dtype(output_dtype));
    at::Tensor bin_indices = at::empty({N, F}, weight.options().dtype(bin_index_scalar_type(B)));
    if (output.numel() == 0) return {output, bin_indices};
    const int rc = ple_forward_launch(
        x.data_ptr<float>(), bin_edges.data_ptr<float>(), inv_bin_widths.data_ptr<float>(),
        n_bins.data_ptr<int32_t>(), weight.data_ptr<float>(),
        bias ? bias->data_ptr<float>() : nullptr, output.data_ptr(), bin_indices.data_ptr(), N, F, B,
        D, ple_dtype_of(quant_dtype), ple_dtype_of(output_dtype), current_stream(x));
    check_rc(rc, "ple_forward_launch");
    return {output, bin_indices};
}

// reference csrc/forward_cuda.cu:687-860
std::tuple<at::Tensor, at::Tensor> ple_forward(const at::Tensor &x, const at::Tensor &bin_edges,
                                               const at::Tensor &inv_bin_widths,
                                               const at::Tensor &n_bins, const at::Tensor &weight,
                                               at::ScalarType output_dtype) {
    check_forward_inputs(x, bin_edges, inv_bin_widths, n_bins, weight);
    TORCH_CHECK(output_dtype == at::kFloat || output_dtype == at::kHalf || output_dtype == at::kBFloat16,
                "output_dtype must be float32, float16, or bfloat16");
    return run_forward(x, bin_edges, inv_bin_widths, n_bins, weight, nullptr, output_dtype, output_dtype);
}

std::tuple<at::Tensor, at::Tensor> ple_forward_with_bias(const at::Tensor &x, const at::Tensor &bin_edges,
                                                         const at::Tensor &inv_bin_widths,
                                                         const at::Tensor &n_bins,
                                                         const at::Tensor &weight, const at::Tensor &bias,
                                                         at::ScalarType quant_dtype) {
    check_forward_inputs(x, bin_edges, inv_bin_widths, n_bins, weight);
    TORCH_CHECK(quant_dtype == at::kFloat || quant_dtype == at::kHalf || quant_dtype == at::kBFloat16,
                "quant_dtype must be float32, float16, or bfloat16");
    TORCH_CHECK(bias.is_cuda() && bias.device() == x.device(), "bias must be on the same CUDA device as x");
    TORCH_CHECK(bias.is_contiguous(), "bias must be contiguous");
    TORCH_CHECK(bias.scalar_type() == at::kFloat, "bias must be float32");
    TORCH_CHECK(bias.dim() == 2 && bias.size(0) == weight.size(0) && bias.size(1) == weight.size(2),
                "bias must have shape [F, D]");
    return run_forward(x, bin_edges, inv_bin_widths, n_bins, weight, &bias, quant_dtype, at::kFloat);
}

void check_param_fd(const at::Tensor &t, const at::Tensor &x, const at::Tensor &weight, const char *name) {
    TORCH_CHECK(t.is_cuda() && t.device() == x.device(), name, " must be on the same CUDA device as x");
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
    TORCH_CHECK(t.scalar_type() == at::kFloat, name, " must be float32");
    TORCH_CHECK(t.dim() == 2 && t.size(0) == weight.size(0) && t.size(1) == weight.size(2), name,
                " must have shape [F, D]");
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> ple_forward_epilogue(
    const at::Tensor &x, const at::Tensor &bin_edges, const at::Tensor &inv_bin_widths,
    const at::Tensor &n_bins, const at::Tensor &weight, const c10::optional<at::Tensor> &bias,
    const c10::optional<at::Tensor> &lin_weight, const c10::optional<at::Tensor> &lin_bias, bool relu,
    bool save_mask, at::ScalarType quant_dtype) {
    check_forward_inputs(x, bin_edges, inv_bin_widths, n_bins, weight);
    TORCH_CHECK(quant_dtype == at::kFloat || quant_dtype == at::kHalf || quant_dtype == at::kBFloat16,
                "quant_dtype must be float32, float16, or bfloat16");
    const bool has_bias = bias.has_value() && bias->defined();
    const bool has_lin = lin_weight.has_value() && lin_weight->defined();
    TORCH_CHECK(has_bias != has_lin, "exactly one of bias and lin_weight must be given");
    if (has_bias) check_param_fd(*bias, x, weight, "bias");
    if (has_lin) {
        TORCH_CHECK(lin_bias.has_value() && lin_bias->defined(), "lin_bias must be given with lin_weight");
        check_param_fd(*lin_weight, x, weight, "lin_weight");
        check_param_fd(*lin_bias, x, weight, "lin_bias");
    }
    const int64_t N = x.size(0), F = x.size(1), B = weight.size(1), D = weight.size(2);
    DeviceScope scope(x.device().index());
    at::Tensor output = at::empty({N, F, D}, weight.options().dtype(at::kFloat));
    at::Tensor bin_indices = at::empty({N, F}, weight.options().dtype(bin_index_scalar_type(B)));
    at::Tensor mask = (relu && save_mask) ? at::empty({N, F, (D + 31) / 32}, weight.options().dtype(at::kInt))
                                          : at::empty({0}, weight.options().dtype(at::kInt));
    if (output.numel() == 0) return {output, bin_indices, mask};
    ple_epilogue_t epi{};
    epi.bias = has_bias ? bias->data_ptr<float>() : nullptr;
    epi.lin_weight = has_lin ? lin_weight->data_ptr<float>() : nullptr;
    epi.lin_bias = has_lin ? lin_bias->data_ptr<float>() : nullptr;
    epi.relu = relu ? 1 : 0;
    epi.relu_mask = mask.numel() > 0 ? reinterpret_cast<uint32_t *>(mask.data_ptr<int32_t>()) : nullptr;
    const int rc = ple_forward_epilogue_launch(
        x.data_ptr<float>(), bin_edges.data_ptr<float>(), inv_bin_widths.data_ptr<float>(),
        n_bins.data_ptr<int32_t>(), weight.data_ptr<float>(), &epi, output.data_ptr<float>(),
        bin_indices.data_ptr(), N, F, B, D, ple_dtype_of(quant_dtype), current_stream(x));
    check_rc(rc, "ple_forward_epilogue_launch");
    return {output, bin_indices, mask};
}

void check_backward_inputs(const at::Tensor &grad_output, const at::Tensor &x, const at::Tensor &bin_edges,
                           const at::Tensor &inv_bin_widths, const at::Tensor &n_bins,
                           const at::Tensor &weight, const at::Tensor &bin_indices) {
    TORCH_CHECK(grad_output.is_cuda(), "grad_output must be CUDA");
    TORCH_CHECK(x.is_cuda(), "x must be CUDA");
    TORCH_CHECK(bin_edges.is_cuda(), "bin_edges must be CUDA");
    TORCH_CHECK(inv_bin_widths.is_cuda(), "inv_bin_widths must be CUDA");
    TORCH_CHECK(n_bins.is_cuda(), "n_bins must be CUDA");
    TORCH_CHECK(weight.is_cuda(), "weight must be CUDA");
    TORCH_CHECK(bin_indices.is_cuda(), "bin_indices must be CUDA");
    TORCH_CHECK(grad_output.device() == x.device() && x.device() == bin_edges.device() &&
                    x.device() == inv_bin_widths.device() && x.device() == n_bins.device() &&
                    x.device() == weight.device() && x.device() == bin_indices.device(),
                "All backward tensors must be on the same CUDA device");
    TORCH_CHECK(grad_output.is_contiguous(), "grad_output must be contiguous");
    TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
    TORCH_CHECK(bin_edges.is_contiguous(), "bin_edges must be contiguous");
    TORCH_CHECK(inv_bin_widths.is_contiguous(), "inv_bin_widths must be contiguous");
    TORCH_CHECK(n_bins.is_contiguous(), "n_bins must be contiguous");
    TORCH_CHECK(weight.is_contiguous(), "weight must be contiguous");
    TORCH_CHECK(bin_indices.is_contiguous(), "bin_indices must be contiguous");
    TORCH_CHECK(x.dim() == 2, "x must have shape [N, F]");
    TORCH_CHECK(grad_output.dim() == 3, "grad_output must have shape [N, F, D]");
    TORCH_CHECK(bin_edges.dim() == 2, "bin_edges must have shape [F, B+1]");
    TORCH_CHECK(inv_bin_widths.dim() == 2, "inv_bin_widths must have shape [F, B]");
    TORCH_CHECK(n_bins.dim() == 1, "n_bins must have shape [F]");
    TORCH_CHECK(weight.dim() == 3, "weight must have shape [F, B, D]");
    TORCH_CHECK(bin_indices.dim() == 2, "bin_indices must have shape [N, F]");
    TORCH_CHECK(x.scalar_type() == at::kFloat, "x must be float32");
    TORCH_CHECK(bin_edges.scalar_type() == at::kFloat, "bin_edges must be float32");
    TORCH_CHECK(inv_bin_widths.scalar_type() == at::kFloat, "inv_bin_widths must be float32");
    TORCH_CHECK(n_bins.scalar_type() == at::kInt, "n_bins must be int32");
    TORCH_CHECK(weight.scalar_type() == at::kFloat, "weight must be float32");
    TORCH_CHECK(grad_output.scalar_type() == at::kFloat || grad_output.scalar_type() == at::kHalf ||
                    grad_output.scalar_type() == at::kBFloat16,
                "grad_output must be float32, float16, or bfloat16");
    const int64_t batch_size = x.size(0);
    const int64_t n_features = x.size(1);
    const int64_t max_n_bins = weight.size(1);
    const int64_t d_embedding = weight.size(2);
    TORCH_CHECK(bin_indices.scalar_type() == bin_index_scalar_type(max_n_bins), "bin_indices has an invalid dtype");
    TORCH_CHECK(grad_output.size(0) == batch_size && grad_output.size(1) == n_features &&
                    grad_output.size(2) == d_embedding,
                "grad_output shape must be [N, F, D]");
    TORCH_CHECK(bin_indices.size(0) == batch_size && bin_indices.size(1) == n_features,
                "bin_indices shape must be [N, F]");
    TORCH_CHECK(weight.size(0) == n_features, "weight F mismatch");
    TORCH_CHECK(bin_edges.size(0) == n_features, "bin_edges F mismatch");
    TORCH_CHECK(bin_edges.size(1) == max_n_bins + 1, "bin_edges B mismatch");
    TORCH_CHECK(inv_bin_widths.size(0) == n_features, "inv_bin_widths F mismatch");
    TORCH_CHECK(inv_bin_widths.size(1) == max_n_bins, "inv_bin_widths B mismatch");
    TORCH_CHECK(n_bins.size(0) == n_features, "n_bins F mismatch");
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> run_backward(
    const at::Tensor &grad_output, const at::Tensor &x, const at::Tensor &bin_edges,
    const at::Tensor &inv_bin_widths, const at::Tensor &n_bins, const at::Tensor &weight,
    const at::Tensor &bin_indices, at::ScalarType quant_dtype, bool compute_grad_x,
    bool compute_grad_weight, bool compute_grad_bias) {
    const int64_t N = x.size(0), F = x.size(1), B = weight.size(1), D = weight.size(2);
    DeviceScope scope(x.device().index());
    // Every element of the requested gradients is written by the kernels
    // (slots of grad_weight that no bin maps to are stored as 0), except for
    // an empty batch, where the parameter gradients are plain zeros.
    at::Tensor grad_x = compute_grad_x ? at::empty_like(x) : at::empty({0}, x.options());
    at::Tensor grad_weight = compute_grad_weight ? (N == 0 ? at::zeros_like(weight) : at::empty_like(weight))
                                                 : at::empty({0}, weight.options());
    at::Tensor grad_bias = compute_grad_bias ? (N == 0 ? at::zeros({F, D}, weight.options())
                                                       : at::empty({F, D}, weight.options()))
                                             : at::empty({0}, weight.options());
    if (N == 0 || (!compute_grad_x && !compute_grad_weight && !compute_grad_bias))
        return {grad_x, grad_weight, grad_bias};
    const size_t ws_bytes = ple_backward_workspace_bytes(N, F, B, D);
    at::Tensor workspace = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, x.options().dtype(at::kByte));
    const int rc = ple_backward_launch(
        grad_output.data_ptr(), x.data_ptr<float>(), bin_edges.data_ptr<float>(),
        inv_bin_widths.data_ptr<float>(), n_bins.data_ptr<int32_t>(), weight.data_ptr<float>(),
        bin_indices.data_ptr(), compute_grad_x ? grad_x.data_ptr<float>() : nullptr,
        compute_grad_weight ? grad_weight.data_ptr<float>() : nullptr,
        compute_grad_bias ? grad_bias.data_ptr<float>() : nullptr, N, F, B, D,
        ple_dtype_of(grad_output.scalar_type()), ple_dtype_of(quant_dtype), workspace.data_ptr(), ws_bytes,
        current_stream(x));
    check_rc(rc, "ple_backward_launch");
    return {grad_x, grad_weight, grad_bias};
}

// reference csrc/backward_cuda.cu:1528-1725
std::tuple<at::Tensor, at::Tensor> ple_backward(const at::Tensor &grad_output, const at::Tensor &x,
                                                const at::Tensor &bin_edges, const at::Tensor &inv_bin_widths,
                                                const at::Tensor &n_bins, const at::Tensor &weight,
                                                const at::Tensor &bin_indices, bool compute_grad_x,
                                                bool compute_grad_weight) {
    check_backward_inputs(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices);
    auto r = run_backward(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices,
                          grad_output.scalar_type(), compute_grad_x, compute_grad_weight, false);
    return {std::get<0>(r), std::get<1>(r)};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> ple_backward_with_bias(
    const at::Tensor &grad_output, const at::Tensor &x, const at::Tensor &bin_edges,
    const at::Tensor &inv_bin_widths, const at::Tensor &n_bins, const at::Tensor &weight,
    const at::Tensor &bin_indices, at::ScalarType quant_dtype, bool compute_grad_x,
    bool compute_grad_weight, bool compute_grad_bias) {
    check_backward_inputs(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices);
    TORCH_CHECK(quant_dtype == at::kFloat || quant_dtype == at::kHalf || quant_dtype == at::kBFloat16,
                "quant_dtype must be float32, float16, or bfloat16");
    return run_backward(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices, quant_dtype,
                        compute_grad_x, compute_grad_weight, compute_grad_bias);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> ple_backward_epilogue(
    const at::Tensor &grad_output, const at::Tensor &x, const at::Tensor &bin_edges,
    const at::Tensor &inv_bin_widths, const at::Tensor &n_bins, const at::Tensor &weight,
    const at::Tensor &bin_indices, const at::Tensor &relu_mask, const c10::optional<at::Tensor> &lin_weight,
    bool relu, at::ScalarType quant_dtype, bool compute_grad_x, bool compute_grad_weight,
    bool compute_grad_bias, bool compute_grad_lin_weight, bool compute_grad_lin_bias) {
    check_backward_inputs(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices);
    TORCH_CHECK(grad_output.scalar_type() == at::kFloat, "grad_output must be float32");
    TORCH_CHECK(quant_dtype == at::kFloat || quant_dtype == at::kHalf || quant_dtype == at::kBFloat16,
                "quant_dtype must be float32, float16, or bfloat16");
    const bool has_lin = lin_weight.has_value() && lin_weight->defined();
    if (has_lin) check_param_fd(*lin_weight, x, weight, "lin_weight");
    TORCH_CHECK(!(has_lin && compute_grad_bias), "no bias gradient with lin_weight (version B has no bias)");
    TORCH_CHECK(has_lin || (!compute_grad_lin_weight && !compute_grad_lin_bias),
                "linear0 gradients need lin_weight");
    const int64_t N = x.size(0), F = x.size(1), B = weight.size(1), D = weight.size(2);
    if (relu) {
        TORCH_CHECK(relu_mask.is_cuda() && relu_mask.device() == x.device() && relu_mask.is_contiguous() &&
                        relu_mask.scalar_type() == at::kInt && relu_mask.dim() == 3 && relu_mask.size(0) == N &&
                        relu_mask.size(1) == F && relu_mask.size(2) == (D + 31) / 32,
                    "relu_mask must be the int32 [N, F, ceil(D / 32)] pass bits of the forward");
    }
    DeviceScope scope(x.device().index());
    auto fd = [&](bool want) {
        return want ? (N == 0 ? at::zeros({F, D}, weight.options()) : at::empty({F, D}, weight.options()))
                    : at::empty({0}, weight.options());
    };
    at::Tensor grad_x = compute_grad_x ? at::empty_like(x) : at::empty({0}, x.options());
    at::Tensor grad_weight = compute_grad_weight ? (N == 0 ? at::zeros_like(weight) : at::empty_like(weight))
                                                 : at::empty({0}, weight.options());
    at::Tensor grad_bias = fd(compute_grad_bias);
    at::Tensor grad_lw = fd(compute_grad_lin_weight);
    at::Tensor grad_lb = fd(compute_grad_lin_bias);
    if (N == 0 || (!compute_grad_x && !compute_grad_weight && !compute_grad_bias && !compute_grad_lin_weight &&
                   !compute_grad_lin_bias))
        return {grad_x, grad_weight, grad_bias, grad_lw, grad_lb};
    const size_t ws_bytes = ple_backward_workspace_bytes(N, F, B, D);
    at::Tensor workspace = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, x.options().dtype(at::kByte));
    // version B when lin_weight is given, else version A
    ple_epilogue_t epi{};
    epi.lin_weight = has_lin ? lin_weight->data_ptr<float>() : nullptr;
    epi.relu = relu ? 1 : 0;
    epi.relu_mask = relu ? reinterpret_cast<uint32_t *>(relu_mask.data_ptr<int32_t>()) : nullptr;
    const int rc = ple_backward_epilogue_launch(
        grad_output.data_ptr<float>(), x.data_ptr<float>(), bin_edges.data_ptr<float>(),
        inv_bin_widths.data_ptr<float>(), n_bins.data_ptr<int32_t>(), weight.data_ptr<float>(),
        bin_indices.data_ptr(), &epi, compute_grad_x ? grad_x.data_ptr<float>() : nullptr,
        compute_grad_weight ? grad_weight.data_ptr<float>() : nullptr,
        compute_grad_bias ? grad_bias.data_ptr<float>() : nullptr,
        compute_grad_lin_weight ? grad_lw.data_ptr<float>() : nullptr,
        compute_grad_lin_bias ? grad_lb.data_ptr<float>() : nullptr, N, F, B, D, ple_dtype_of(quant_dtype),
        workspace.data_ptr(), ws_bytes, current_stream(x));
    check_rc(rc, "ple_backward_epilogue_launch");
    return {grad_x, grad_weight, grad_bias, grad_lw, grad_lb};
}

void check_encode_tables(const at::Tensor &x, const at::Tensor &bin_edges, const at::Tensor &inv_bin_widths,
                         const at::Tensor &n_bins, const at::Tensor &offsets) {
    for (const at::Tensor *t : {&x, &bin_edges, &inv_bin_widths, &n_bins, &offsets}) {
        TORCH_CHECK(t->is_cuda() && t->device() == x.device(), "All encoding tensors must be on the same CUDA device");
        TORCH_CHECK(t->is_contiguous(), "encoding tensors must be contiguous");
    }
    TORCH_CHECK(x.dim() == 2 && x.scalar_type() == at::kFloat, "x must be float32 [N, F]");
    const int64_t F = x.size(1);
    TORCH_CHECK(bin_edges.dim() == 2 && bin_edges.size(0) == F && bin_edges.scalar_type() == at::kFloat,
                "bin_edges must be float32 [F, B + 1]");
    TORCH_CHECK(inv_bin_widths.dim() == 2 && inv_bin_widths.size(0) == F &&
                    inv_bin_widths.size(1) + 1 == bin_edges.size(1) && inv_bin_widths.scalar_type() == at::kFloat,
                "inv_bin_widths must be float32 [F, B]");
    TORCH_CHECK(n_bins.dim() == 1 && n_bins.size(0) == F && n_bins.scalar_type() == at::kInt, "n_bins must be int32 [F]");
    TORCH_CHECK(offsets.dim() == 1 && offsets.size(0) == F && offsets.scalar_type() == at::kInt,
                "offsets must be int32 [F]");
}

// The upstream PiecewiseLinearEncoding output (this build's addition).
at::Tensor ple_encode(const at::Tensor &x, const at::Tensor &bin_edges, const at::Tensor &inv_bin_widths,
                      const at::Tensor &n_bins, const at::Tensor &offsets, int64_t total_bins) {
    check_encode_tables(x, bin_edges, inv_bin_widths, n_bins, offsets);
    TORCH_CHECK(total_bins > 0, "total_bins must be positive");
    const int64_t N = x.size(0), F = x.size(1), B = inv_bin_widths.size(1);
    DeviceScope scope(x.device().index());
    at::Tensor out = at::empty({N, total_bins}, x.options());
    if (N == 0) return out;
    const int rc = ple_encode_launch(x.data_ptr<float>(), bin_edges.data_ptr<float>(), inv_bin_widths.data_ptr<float>(),
                                     n_bins.data_ptr<int32_t>(), offsets.data_ptr<int32_t>(), out.data_ptr<float>(), N,
                                     F, B, total_bins, current_stream(x));
    check_rc(rc, "ple_encode_launch");
    return out;
}

at::Tensor ple_encode_backward(const at::Tensor &grad_output, const at::Tensor &x, const at::Tensor &bin_edges,
                               const at::Tensor &inv_bin_widths, const at::Tensor &n_bins,
                               const at::Tensor &offsets) {
    check_encode_tables(x, bin_edges, inv_bin_widths, n_bins, offsets);
    TORCH_CHECK(grad_output.is_cuda() && grad_output.device() == x.device() && grad_output.is_contiguous() &&
                    grad_output.scalar_type() == at::kFloat && grad_output.dim() == 2 &&
                    grad_output.size(0) == x.size(0),
                "grad_output must be contiguous float32 [N, total_bins]");
    const int64_t N = x.size(0), F = x.size(1), B = inv_bin_widths.size(1), T = grad_output.size(1);
    DeviceScope scope(x.device().index());
    at::Tensor grad_x = at::empty_like(x);
    if (N == 0) return grad_x;
    const int rc = ple_encode_backward_launch(
        grad_output.data_ptr<float>(), x.data_ptr<float>(), bin_edges.data_ptr<float>(),
        inv_bin_widths.data_ptr<float>(), n_bins.data_ptr<int32_t>(), offsets.data_ptr<int32_t>(),
        grad_x.data_ptr<float>(), N, F, B, T, current_stream(x));
    check_rc(rc, "ple_encode_backward_launch");
    return grad_x;
}

}  // namespace

TORCH_LIBRARY(rtdl_num_embeddings_cuda, m) {
    m.def(
        "forward(Tensor x, Tensor bin_edges, Tensor inv_bin_widths, Tensor n_bins, Tensor weight, "
        "ScalarType output_dtype) -> (Tensor output, Tensor bin_indices)");
    m.def(
        "backward(Tensor grad_output, Tensor x, Tensor bin_edges, Tensor inv_bin_widths, Tensor n_bins, "
        "Tensor weight, Tensor bin_indices, bool compute_grad_x, bool compute_grad_weight) -> "
        "(Tensor grad_x, Tensor grad_weight)");
    m.def(
        "forward_with_bias(Tensor x, Tensor bin_edges, Tensor inv_bin_widths, Tensor n_bins, Tensor weight, "
        "Tensor bias, ScalarType quant_dtype) -> (Tensor output, Tensor bin_indices)");
    m.def(
        "backward_with_bias(Tensor grad_output, Tensor x, Tensor bin_edges, Tensor inv_bin_widths, "
        "Tensor n_bins, Tensor weight, Tensor bin_indices, ScalarType quant_dtype, bool compute_grad_x, "
        "bool compute_grad_weight, bool compute_grad_bias) -> (Tensor grad_x, Tensor grad_weight, "
        "Tensor grad_bias)");
    m.def(
        "forward_epilogue(Tensor x, Tensor bin_edges, Tensor inv_bin_widths, Tensor n_bins, Tensor weight, "
        "Tensor? bias, Tensor? lin_weight, Tensor? lin_bias, bool relu, bool save_mask, ScalarType quant_dtype) "
        "-> (Tensor output, Tensor bin_indices, Tensor relu_mask)");
    m.def(
        "backward_epilogue(Tensor grad_output, Tensor x, Tensor bin_edges, Tensor inv_bin_widths, "
        "Tensor n_bins, Tensor weight, Tensor bin_indices, Tensor relu_mask, Tensor? lin_weight, bool relu, "
        "ScalarType quant_dtype, bool compute_grad_x, bool compute_grad_weight, bool compute_grad_bias, "
        "bool compute_grad_lin_weight, bool compute_grad_lin_bias) -> (Tensor grad_x, Tensor grad_weight, "
        "Tensor grad_bias, Tensor grad_lin_weight, Tensor grad_lin_bias)");
    m.def(
        "encode(Tensor x, Tensor bin_edges, Tensor inv_bin_widths, Tensor n_bins, Tensor offsets, int total_bins) "
        "-> Tensor");
    m.def(
        "encode_backward(Tensor grad_output, Tensor x, Tensor bin_edges, Tensor inv_bin_widths, Tensor n_bins, "
        "Tensor offsets) -> Tensor");
}

TORCH_LIBRARY_IMPL(rtdl_num_embeddings_cuda, CUDA, m) {
    m.impl("forward", &ple_forward);
    m.impl("backward", &ple_backward);
    m.impl("forward_with_bias", &ple_forward_with_bias);
    m.impl("backward_with_bias", &ple_backward_with_bias);
    m.impl("forward_epilogue", &ple_forward_epilogue);
    m.impl("backward_epilogue", &ple_backward_epilogue);
    m.impl("encode", &ple_encode);
    m.impl("encode_backward", &ple_encode_backward);
}

// Importing the extension module runs the registrations above; the module
// itself exposes only the C ABI version of the kernel library it links.
static PyObject *abi_version(PyObject *, PyObject *) { return PyLong_FromLong(ple_abi_version()); }

static PyMethodDef kMethods[] = {
    {"abi_version", abi_version, METH_NOARGS, "ABI version of the linked kernel library."},
    {nullptr, nullptr, 0, nullptr},
};

static PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_C", "PLE operator registrations (HIP, gfx950).", -1,
                              kMethods};

PyMODINIT_FUNC PyInit__C(void) { return PyModule_Create(&kModule); }
