"""FakeTensor (meta) kernels of the PLE operators.

They state the shape / dtype contract of every operator without touching
data, so ``torch.compile(fullgraph=True)`` and meta-device tracing work.  The
checks and messages of ``forward`` / ``backward`` follow the reference
(``src/rtdl_num_embeddings_cuda/_meta.py:22-188``); the ``*_with_bias`` and
``*_epilogue`` operators are this build's fused variants.
"""

from __future__ import annotations

import torch
from torch import Tensor

SUPPORTED_OUTPUT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def bin_indices_dtype(max_n_bins: int) -> torch.dtype:
    """uint8 up to 256 bins, int16 up to 32768, int32 beyond (``_meta.py:14-19``)."""
    if max_n_bins <= 256:
        return torch.uint8
    if max_n_bins <= 32768:
        return torch.int16
    return torch.int32


def _check_forward_inputs(x, bin_edges, inv_bin_widths, n_bins, weight) -> None:
    torch._check(x.ndim == 2, lambda: "x must have shape [N, F]")
    torch._check(bin_edges.ndim == 2, lambda: "bin_edges must have shape [F, B + 1]")
    torch._check(inv_bin_widths.ndim == 2, lambda: "inv_bin_widths must have shape [F, B]")
    torch._check(n_bins.ndim == 1, lambda: "n_bins must have shape [F]")
    torch._check(weight.ndim == 3, lambda: "weight must have shape [F, B, D]")
    f_count, max_n_bins = weight.shape[0], weight.shape[1]
    torch._check(x.shape[1] == f_count, lambda: "x.shape[1] must equal weight.shape[0]")
    torch._check(bin_edges.shape[0] == f_count, lambda: "bin_edges.shape[0] must equal weight.shape[0]")
    torch._check(bin_edges.shape[1] == max_n_bins + 1, lambda: "bin_edges.shape[1] must equal weight.shape[1] + 1")
    torch._check(inv_bin_widths.shape[0] == f_count, lambda: "inv_bin_widths.shape[0] must equal weight.shape[0]")
    torch._check(inv_bin_widths.shape[1] == max_n_bins, lambda: "inv_bin_widths.shape[1] must equal weight.shape[1]")
    torch._check(n_bins.shape[0] == f_count, lambda: "n_bins.shape[0] must equal weight.shape[0]")
    torch._check(x.dtype == torch.float32, lambda: "x must be float32")
    torch._check(bin_edges.dtype == torch.float32, lambda: "bin_edges must be float32")
    torch._check(inv_bin_widths.dtype == torch.float32, lambda: "inv_bin_widths must be float32")
    torch._check(n_bins.dtype == torch.int32, lambda: "n_bins must be int32")
    torch._check(weight.dtype == torch.float32, lambda: "weight must be float32")


def _forward_outputs(x: Tensor, weight: Tensor, output_dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    out = torch.empty((x.shape[0], x.shape[1], weight.shape[2]), dtype=output_dtype, device=x.device)
    idx = torch.empty((x.shape[0], x.shape[1]), dtype=bin_indices_dtype(weight.shape[1]), device=x.device)
    return out, idx


@torch.library.register_fake("rtdl_num_embeddings_cuda::forward")
def _forward_fake(x, bin_edges, inv_bin_widths, n_bins, weight, output_dtype):
    _check_forward_inputs(x, bin_edges, inv_bin_widths, n_bins, weight)
    torch._check(output_dtype in SUPPORTED_OUTPUT_DTYPES, lambda: "Unsupported output dtype")
    return _forward_outputs(x, weight, output_dtype)


@torch.library.register_fake("rtdl_num_embeddings_cuda::forward_with_bias")
def _forward_with_bias_fake(x, bin_edges, inv_bin_widths, n_bins, weight, bias, quant_dtype):
    _check_forward_inputs(x, bin_edges, inv_bin_widths, n_bins, weight)
    torch._check(quant_dtype in SUPPORTED_OUTPUT_DTYPES, lambda: "Unsupported quant dtype")
    torch._check(bias.ndim == 2, lambda: "bias must have shape [F, D]")
    torch._check(bias.shape[0] == weight.shape[0], lambda: "bias must have shape [F, D]")
    torch._check(bias.shape[1] == weight.shape[2], lambda: "bias must have shape [F, D]")
    torch._check(bias.dtype == torch.float32, lambda: "bias must be float32")
    return _forward_outputs(x, weight, torch.float32)


def _check_backward_inputs(grad_output, x, weight, bin_indices) -> None:
    torch._check(grad_output.ndim == 3, lambda: "grad_output must have shape [N, F, D]")
    torch._check(grad_output.shape[0] == x.shape[0], lambda: "grad_output N mismatch")
    torch._check(grad_output.shape[1] == x.shape[1], lambda: "grad_output F mismatch")
    torch._check(grad_output.shape[2] == weight.shape[2], lambda: "grad_output D mismatch")
    torch._check(bin_indices.shape[0] == x.shape[0], lambda: "bin_indices N mismatch")
    torch._check(bin_indices.shape[1] == x.shape[1], lambda: "bin_indices F mismatch")
    torch._check(bin_indices.dtype == bin_indices_dtype(weight.shape[1]), lambda: "bin_indices has an invalid dtype")
    torch._check(grad_output.dtype in SUPPORTED_OUTPUT_DTYPES, lambda: "Unsupported grad_output dtype")


def _maybe(t: Tensor, like: Tensor, wanted: bool) -> Tensor:
    return torch.empty_like(like) if wanted else torch.empty((0,), dtype=like.dtype, device=like.device)


@torch.library.register_fake("rtdl_num_embeddings_cuda::backward")
def _backward_fake(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices,
                   compute_grad_x, compute_grad_weight):
    _check_backward_inputs(grad_output, x, weight, bin_indices)
    return _maybe(x, x, compute_grad_x), _maybe(weight, weight, compute_grad_weight)


@torch.library.register_fake("rtdl_num_embeddings_cuda::backward_with_bias")
def _backward_with_bias_fake(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices,
                             quant_dtype, compute_grad_x, compute_grad_weight, compute_grad_bias):
    _check_backward_inputs(grad_output, x, weight, bin_indices)
    torch._check(quant_dtype in SUPPORTED_OUTPUT_DTYPES, lambda: "Unsupported quant dtype")
    grad_bias = (
        torch.empty((weight.shape[0], weight.shape[2]), dtype=weight.dtype, device=weight.device)
        if compute_grad_bias
        else torch.empty((0,), dtype=weight.dtype, device=weight.device)
    )
    return _maybe(x, x, compute_grad_x), _maybe(weight, weight, compute_grad_weight), grad_bias


def _check_fd(t, weight, name: str) -> None:
    torch._check(t.ndim == 2, lambda: f"{name} must have shape [F, D]")
    torch._check(t.shape[0] == weight.shape[0], lambda: f"{name} must have shape [F, D]")
    torch._check(t.shape[1] == weight.shape[2], lambda: f"{name} must have shape [F, D]")
    torch._check(t.dtype == torch.float32, lambda: f"{name} must be float32")


def _mask_words(d_embedding) -> int:
    return (d_embedding + 31) // 32


@torch.library.register_fake("rtdl_num_embeddings_cuda::forward_epilogue")
def _forward_epilogue_fake(x, bin_edges, inv_bin_widths, n_bins, weight, bias, lin_weight, lin_bias, relu,
                           save_mask, quant_dtype):
    _check_forward_inputs(x, bin_edges, inv_bin_widths, n_bins, weight)
    torch._check(quant_dtype in SUPPORTED_OUTPUT_DTYPES, lambda: "Unsupported quant dtype")
    torch._check((bias is None) != (lin_weight is None), lambda: "exactly one of bias and lin_weight must be given")
    if bias is not None:
        _check_fd(bias, weight, "bias")
    if lin_weight is not None:
        torch._check(lin_bias is not None, lambda: "lin_bias must be given with lin_weight")
        _check_fd(lin_weight, weight, "lin_weight")
        _check_fd(lin_bias, weight, "lin_bias")
    out, idx = _forward_outputs(x, weight, torch.float32)
    if relu and save_mask:
        mask = torch.empty((x.shape[0], x.shape[1], _mask_words(weight.shape[2])), dtype=torch.int32,
                           device=x.device)
    else:
        mask = torch.empty((0,), dtype=torch.int32, device=x.device)
    return out, idx, mask


@torch.library.register_fake("rtdl_num_embeddings_cuda::backward_epilogue")
def _backward_epilogue_fake(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices, relu_mask,
                            lin_weight, relu, quant_dtype, compute_grad_x, compute_grad_weight,
                            compute_grad_bias, compute_grad_lin_weight, compute_grad_lin_bias):
    _check_backward_inputs(grad_output, x, weight, bin_indices)
    torch._check(grad_output.dtype == torch.float32, lambda: "grad_output must be float32")
    torch._check(quant_dtype in SUPPORTED_OUTPUT_DTYPES, lambda: "Unsupported quant dtype")
    if lin_weight is not None:
        _check_fd(lin_weight, weight, "lin_weight")
    torch._check(not (lin_weight is not None and compute_grad_bias),
                 lambda: "no bias gradient with lin_weight (version B has no bias)")
    torch._check(lin_weight is not None or not (compute_grad_lin_weight or compute_grad_lin_bias),
                 lambda: "linear0 gradients need lin_weight")
    if relu:
        torch._check(relu_mask.ndim == 3 and relu_mask.dtype == torch.int32,
                     lambda: "relu_mask must be the int32 [N, F, ceil(D / 32)] pass bits of the forward")

    def fd(wanted: bool) -> Tensor:
        shape = (weight.shape[0], weight.shape[2]) if wanted else (0,)
        return torch.empty(shape, dtype=weight.dtype, device=weight.device)

    return (_maybe(x, x, compute_grad_x), _maybe(weight, weight, compute_grad_weight), fd(compute_grad_bias),
            fd(compute_grad_lin_weight), fd(compute_grad_lin_bias))


@torch.library.register_fake("rtdl_num_embeddings_cuda::encode")
def _encode_fake(x, bin_edges, inv_bin_widths, n_bins, offsets, total_bins):
    torch._check(x.ndim == 2 and x.dtype == torch.float32, lambda: "x must be float32 [N, F]")
    torch._check(n_bins.shape[0] == x.shape[1], lambda: "n_bins must be int32 [F]")
    torch._check(offsets.shape[0] == x.shape[1], lambda: "offsets must be int32 [F]")
    torch._check(total_bins > 0, lambda: "total_bins must be positive")
    return torch.empty((x.shape[0], total_bins), dtype=torch.float32, device=x.device)


@torch.library.register_fake("rtdl_num_embeddings_cuda::encode_backward")
def _encode_backward_fake(grad_output, x, bin_edges, inv_bin_widths, n_bins, offsets):
    torch._check(grad_output.ndim == 2 and grad_output.shape[0] == x.shape[0],
                 lambda: "grad_output must be contiguous float32 [N, total_bins]")
    return torch.empty_like(x)
