"""Autograd formulas of the PLE operators.

``forward``: the same contract as the reference
(``src/rtdl_num_embeddings_cuda/_autograd.py:9-96``): the saved bin indices
are non-differentiable, grads are not materialised, and the backward operator
returns gradients for ``x`` (input 0) and ``weight`` (input 4) only.

``forward_with_bias``: additionally returns the bias gradient (input 5) from
the same backward launch; ``quant_dtype`` (input 6) is forwarded so the
backward rounds the gradient, the fraction and the weights like the forward
did.

``forward_epilogue``: gradients for ``x`` (0), ``weight`` (4), ``bias`` (5),
``lin_weight`` (6) and ``lin_bias`` (7) from one backward launch, which reads
the forward's ReLU pass bits (saved, non-differentiable).

``encode``: the gradient of ``x`` (input 0) from ``encode_backward``.

Double backward is not implemented (as in the reference).
"""

from __future__ import annotations

from typing import Any

import torch

_ops = torch.ops.rtdl_num_embeddings_cuda


def _setup_forward_context(ctx: Any, inputs, output) -> None:
    x, bin_edges, inv_bin_widths, n_bins, weight, _output_dtype = inputs
    _out, bin_indices = output
    ctx.save_for_backward(x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices)
    ctx.mark_non_differentiable(bin_indices)
    ctx.set_materialize_grads(False)


def _forward_backward(ctx: Any, grad_output, _grad_bin_indices):
    if grad_output is None:
        return None, None, None, None, None, None
    x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices = ctx.saved_tensors
    need_x = bool(ctx.needs_input_grad[0])
    need_w = bool(ctx.needs_input_grad[4])
    grad_x, grad_weight = _ops.backward(
        grad_output.contiguous(), x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices, need_x, need_w
    )
    return (grad_x if need_x else None, None, None, None, grad_weight if need_w else None, None)


torch.library.register_autograd(
    "rtdl_num_embeddings_cuda::forward",
    _forward_backward,
    setup_context=_setup_forward_context,
)


def _setup_forward_with_bias_context(ctx: Any, inputs, output) -> None:
    x, bin_edges, inv_bin_widths, n_bins, weight, _bias, quant_dtype = inputs
    _out, bin_indices = output
    ctx.save_for_backward(x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices)
    ctx.quant_dtype = quant_dtype
    ctx.mark_non_differentiable(bin_indices)
    ctx.set_materialize_grads(False)


def _forward_with_bias_backward(ctx: Any, grad_output, _grad_bin_indices):
    if grad_output is None:
        return None, None, None, None, None, None, None
    x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices = ctx.saved_tensors
    need_x = bool(ctx.needs_input_grad[0])
    need_w = bool(ctx.needs_input_grad[4])
    need_b = bool(ctx.needs_input_grad[5])
    grad_x, grad_weight, grad_bias = _ops.backward_with_bias(
        grad_output.contiguous(), x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices,
        ctx.quant_dtype, need_x, need_w, need_b,
    )
    return (
        grad_x if need_x else None,
        None,
        None,
        None,
        grad_weight if need_w else None,
        grad_bias if need_b else None,
        None,
    )


torch.library.register_autograd(
    "rtdl_num_embeddings_cuda::forward_with_bias",
    _forward_with_bias_backward,
    setup_context=_setup_forward_with_bias_context,
)


def _setup_forward_epilogue_context(ctx: Any, inputs, output) -> None:
    x, bin_edges, inv_bin_widths, n_bins, weight, _bias, lin_weight, _lin_bias, relu, save_mask, quant_dtype = inputs
    _out, bin_indices, relu_mask = output
    ctx.save_for_backward(x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices, relu_mask, lin_weight)
    ctx.relu = bool(relu)
    # (from the flag, not the mask's size: an empty batch saves an empty mask)
    ctx.saved_mask = bool(save_mask)
    ctx.quant_dtype = quant_dtype
    ctx.mark_non_differentiable(bin_indices, relu_mask)
    ctx.set_materialize_grads(False)


def _forward_epilogue_backward(ctx: Any, grad_output, _grad_bin_indices, _grad_relu_mask):
    if grad_output is None:
        return (None,) * 11
    x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices, relu_mask, lin_weight = ctx.saved_tensors
    need = [bool(ctx.needs_input_grad[i]) for i in (0, 4, 5, 6, 7)]
    if ctx.relu and not ctx.saved_mask:
        raise RuntimeError("forward_epilogue was called with save_mask=False; its ReLU cannot be differentiated")
    gx, gw, gb, glw, glb = _ops.backward_epilogue(
        grad_output.contiguous(), x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices, relu_mask,
        lin_weight, ctx.relu, ctx.quant_dtype, *need,
    )
    return (
        gx if need[0] else None, None, None, None, gw if need[1] else None, gb if need[2] else None,
        glw if need[3] else None, glb if need[4] else None, None, None, None,
    )


torch.library.register_autograd(
    "rtdl_num_embeddings_cuda::forward_epilogue",
    _forward_epilogue_backward,
    setup_context=_setup_forward_epilogue_context,
)


def _setup_encode_context(ctx: Any, inputs, output) -> None:
    x, bin_edges, inv_bin_widths, n_bins, offsets, _total = inputs
    ctx.save_for_backward(x, bin_edges, inv_bin_widths, n_bins, offsets)
    ctx.set_materialize_grads(False)


def _encode_backward(ctx: Any, grad_output):
    if grad_output is None or not ctx.needs_input_grad[0]:
        return (None,) * 6
    x, bin_edges, inv_bin_widths, n_bins, offsets = ctx.saved_tensors
    gx = _ops.encode_backward(grad_output.contiguous(), x, bin_edges, inv_bin_widths, n_bins, offsets)
    return gx, None, None, None, None, None


torch.library.register_autograd(
    "rtdl_num_embeddings_cuda::encode",
    _encode_backward,
    setup_context=_setup_encode_context,
)
