"""Drop-in ``CudaPiecewiseLinearEmbeddings`` module.

Same constructor, parameters, buffers and outputs as the reference module
(``src/rtdl_num_embeddings_cuda/module.py:10-248``), which subclasses
``rtdl_num_embeddings.PiecewiseLinearEmbeddings`` (version 0.0.12).  That
package is not a dependency here: its module structure -- ``linear0``
(version B), ``impl`` (encoding buffers), ``linear`` (per-feature linear
layer), ``activation`` -- is restated in this file so parameter names, buffer
names, initialisation order and the CPU computation stay the same.

On a HIP device the whole module runs through the fused operator
``forward_epilogue`` (one forward kernel, one backward launch):

* version A: ``relu?(x_ple + bias)`` fused into the kernel's store;
* version B: ``linear0(x) + relu?(x_ple)`` fused into the store, linear0's
  gradients produced by the same backward pass;
* with ReLU the forward keeps one pass bit per element for the backward.

Parameters that are not contiguous float32 ``[F, D]`` tensors fall back to
``forward`` plus the same tail in PyTorch.

Under CUDA/HIP autocast (float16 / bfloat16) the kernels round the fraction,
the weights and the result through the autocast dtype with fp32 accumulation,
and the bias is added afterwards in fp32, exactly as the reference's
``x_ple + self.linear.bias`` promotes.  On CPU the module computes the dense
upstream formulation with ordinary PyTorch ops (as the reference falls back to
its parent class, ``module.py:222-223``).
"""

from __future__ import annotations

import warnings
from typing import Literal

import torch
from torch import Tensor, nn
from torch.nn.parameter import Parameter

from ._meta import SUPPORTED_OUTPUT_DTYPES
from .bins import bin_tables, check_bins

_ops = torch.ops.rtdl_num_embeddings_cuda

MAX_D_EMBEDDING = 64


class LinearEmbeddings(nn.Module):
    """``x_linear[n, f] = bias[f] + weight[f] * x[n, f]`` (upstream ``LinearEmbeddings``)."""

    def __init__(self, n_features: int, d_embedding: int) -> None:
        super().__init__()
        self.weight = Parameter(torch.empty(n_features, d_embedding))
        self.bias = Parameter(torch.empty(n_features, d_embedding))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        bound = self.weight.shape[1] ** -0.5
        nn.init.uniform_(self.weight, -bound, bound)
        nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x: Tensor) -> Tensor:
        return torch.addcmul(self.bias, self.weight, x[..., None])


class NLinear(nn.Module):
    """F independent linear layers ``[Bmax] -> [d]`` (upstream ``_NLinear``)."""

    def __init__(self, n: int, in_features: int, out_features: int, bias: bool = True) -> None:
        super().__init__()
        self.weight = Parameter(torch.empty(n, in_features, out_features))
        self.bias = Parameter(torch.empty(n, out_features)) if bias else None
        self.reset_parameters()

    def reset_parameters(self) -> None:
        bound = self.weight.shape[-2] ** -0.5
        nn.init.uniform_(self.weight, -bound, bound)
        if self.bias is not None:
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x: Tensor) -> Tensor:
        if x.ndim != 3:
            raise ValueError("NLinear expects input of shape [batch, n, in_features]")
        y = (x.transpose(0, 1) @ self.weight).transpose(0, 1)
        if self.bias is not None:
            y = y + self.bias
        return y


class PiecewiseLinearEncodingBuffers(nn.Module):
    """Dense-encoding buffers (upstream ``_PiecewiseLinearEncodingImpl``).

    Component ``[f, slot]`` of the encoding is ``weight * x + bias`` with
    ``weight = 1 / width`` and ``bias = -left_edge / width``; the first
    ``n_f - 1`` bins occupy slots ``0 .. n_f - 2`` and the last bin slot
    ``Bmax - 1``; slots between are phantom (weight and bias 0).
    """

    def __init__(self, bins: list[Tensor]) -> None:
        super().__init__()
        n_features = len(bins)
        n_bins = [len(e) - 1 for e in bins]
        max_n_bins = max(n_bins)
        self.register_buffer("weight", torch.zeros(n_features, max_n_bins))
        self.register_buffer("bias", torch.zeros(n_features, max_n_bins))
        single = torch.tensor(n_bins) == 1
        self.register_buffer("single_bin_mask", single if bool(single.any()) else None)
        ragged = any(nb != n_bins[0] for nb in n_bins)
        mask = None
        if ragged:
            mask = torch.stack([
                torch.cat([
                    torch.ones(nb - 1, dtype=torch.bool),
                    torch.zeros(max_n_bins - nb, dtype=torch.bool),
                    torch.ones(1, dtype=torch.bool),
                ])
                for nb in n_bins
            ])
        self.register_buffer("mask", mask)
        for i, edges in enumerate(bins):
            width = edges.diff()
            w = 1.0 / width
            b = -edges[:-1] / width
            self.weight[i, -1] = w[-1]
            self.bias[i, -1] = b[-1]
            self.weight[i, : n_bins[i] - 1] = w[:-1]
            self.bias[i, : n_bins[i] - 1] = b[:-1]

    def get_max_n_bins(self) -> int:
        return self.weight.shape[-1]

    def forward(self, x: Tensor) -> Tensor:
        x = torch.addcmul(self.bias, self.weight, x[..., None])
        if x.shape[-1] > 1:
            last = x[..., -1:]
            last = (
                last.clamp_min(0.0)
                if self.single_bin_mask is None
                else torch.where(self.single_bin_mask[..., None], last, last.clamp_min(0.0))
            )
            x = torch.cat([x[..., :1].clamp_max(1.0), x[..., 1:-1].clamp(0.0, 1.0), last], dim=-1)
        return x


class CudaPiecewiseLinearEncoding(nn.Module):
    """Dense piecewise-linear encoding (upstream ``PiecewiseLinearEncoding``).

    Output ``[batch, total_n_bins]``, ``total_n_bins = sum_f n_f``: per feature
    its ``n_f`` components in bin order (the phantom slots of the padded layout
    dropped, as upstream's mask does).  On a HIP device the encoding and the
    gradient of ``x`` run in the ``encode`` / ``encode_backward`` kernels; on
    the CPU the upstream dense computation runs.  No parameters.
    """

    def __init__(self, bins: list[Tensor]) -> None:
        check_bins(bins)
        super().__init__()
        self.impl = PiecewiseLinearEncodingBuffers(bins)
        base_device = bins[0].device
        for i, e in enumerate(bins):
            if e.device != base_device:
                raise ValueError(
                    "All bin tensors must be on the same device. "
                    f"bins[0].device={base_device}, bins[{i}].device={e.device}"
                )
        edges, inv_w, n_bins = bin_tables(bins, device=base_device)
        offsets = torch.zeros_like(n_bins)
        offsets[1:] = torch.cumsum(n_bins, 0)[:-1]
        self.register_buffer("_cuda_bin_edges", edges, persistent=False)
        self.register_buffer("_cuda_inv_bin_widths", inv_w, persistent=False)
        self.register_buffer("_cuda_n_bins", n_bins, persistent=False)
        self.register_buffer("_cuda_offsets", offsets.to(torch.int32), persistent=False)
        self._total_n_bins = int(sum(int(e.numel()) - 1 for e in bins))

    def get_output_shape(self) -> torch.Size:
        return torch.Size((self._total_n_bins,))

    def forward(self, x: Tensor) -> Tensor:
        if x.ndim != 2:
            raise ValueError("Only inputs with shape [batch_size, n_features] are supported")
        if x.shape[1] != self._cuda_n_bins.shape[0]:
            raise ValueError(f"Expected {self._cuda_n_bins.shape[0]} numerical features, got {x.shape[1]}")
        if x.device.type != "cuda":
            enc = self.impl(x)
            return enc.flatten(-2) if self.impl.mask is None else enc[:, self.impl.mask]
        if x.device != self._cuda_bin_edges.device:
            raise RuntimeError("x and the module must be on the same CUDA device")
        if x.dtype != torch.float32:
            raise TypeError(f"The fused CUDA path requires float32 x. Got {x.dtype}.")
        if not x.is_contiguous():
            raise ValueError("The fused CUDA path requires contiguous x.")
        return _ops.encode(x, self._cuda_bin_edges, self._cuda_inv_bin_widths, self._cuda_n_bins,
                           self._cuda_offsets, self._total_n_bins)


class CudaPiecewiseLinearEmbeddings(nn.Module):
    """Piecewise-linear embeddings with the PLE branch fused on HIP devices.

    Contract on a HIP device (same as the reference):

    - ``x`` is contiguous float32 ``[batch, n_features]``;
    - parameters stay float32;
    - without autocast the output is float32; under float16 / bfloat16
      autocast the PLE branch is rounded through that dtype with fp32
      accumulation;
    - first-order autograd and ``torch.compile(fullgraph=True)`` work;
      double backward is not implemented.
    """

    def __init__(
        self,
        bins: list[Tensor],
        d_embedding: int,
        *,
        activation: bool,
        version: Literal[None, "A", "B"] = None,
    ) -> None:
        assert d_embedding <= MAX_D_EMBEDDING, "d_embedding must be less than or equal to 64"
        if d_embedding <= 0:
            raise ValueError(f"d_embedding must be a positive integer, however: d_embedding={d_embedding}")
        check_bins(bins)
        if version is None:
            warnings.warn(
                'The `version` argument is not provided, so version="A" is used for backward compatibility'
            )
            version = "A"
        if version not in ("A", "B"):
            raise ValueError(f'version must be "A" or "B", got {version!r}')
        super().__init__()
        n_features = len(bins)
        is_b = version == "B"
        # construction order fixes the RNG stream used by the initialisers
        self.linear0 = LinearEmbeddings(n_features, d_embedding) if is_b else None
        self.impl = PiecewiseLinearEncodingBuffers(bins)
        self.linear = NLinear(n_features, self.impl.get_max_n_bins(), d_embedding, bias=not is_b)
        if is_b:
            nn.init.zeros_(self.linear.weight)
        self.activation = nn.ReLU() if activation else None

        base_device = bins[0].device
        for i, e in enumerate(bins):
            if e.device != base_device:
                raise ValueError(
                    "All bin tensors must be on the same device. "
                    f"bins[0].device={base_device}, bins[{i}].device={e.device}"
                )
        edges, inv_w, n_bins_t = bin_tables(bins, device=base_device)
        # non-persistent: the state_dict stays that of the upstream module
        self.register_buffer("_cuda_bin_edges", edges, persistent=False)
        self.register_buffer("_cuda_inv_bin_widths", inv_w, persistent=False)
        self.register_buffer("_cuda_n_bins", n_bins_t, persistent=False)

    @property
    def n_features(self) -> int:
        return int(self.linear.weight.shape[0])

    @property
    def max_n_bins(self) -> int:
        return int(self.linear.weight.shape[1])

    @property
    def d_embedding(self) -> int:
        return int(self.linear.weight.shape[2])

    def get_output_shape(self) -> torch.Size:
        return torch.Size((self.n_features, self.d_embedding))

    def _cuda_output_dtype(self) -> torch.dtype:
        if torch.is_autocast_enabled("cuda"):
            dtype = torch.get_autocast_dtype("cuda")
            if dtype not in (torch.float16, torch.bfloat16):
                raise RuntimeError(f"CUDA autocast dtype must be float16 or bfloat16, got {dtype}")
            return dtype
        return torch.float32

    def _check_cuda_inputs(self, x: Tensor) -> None:
        if x.dtype != torch.float32:
            raise TypeError(f"The fused CUDA path requires float32 x. Got {x.dtype}.")
        if self.linear.weight.dtype != torch.float32:
            raise TypeError(
                f"The fused CUDA path requires float32 parameters. Got weight dtype {self.linear.weight.dtype}."
            )
        if not x.is_contiguous():
            raise ValueError("The fused CUDA path requires contiguous x.")
        for name in ("_cuda_bin_edges", "_cuda_inv_bin_widths", "_cuda_n_bins"):
            if not getattr(self, name).is_contiguous():
                raise RuntimeError(f"{name} must be contiguous")
        if not self.linear.weight.is_contiguous():
            raise RuntimeError("linear.weight must be contiguous")

    def _forward_cpu(self, x: Tensor) -> Tensor:
        x_linear = None if self.linear0 is None else self.linear0(x)
        x_ple = self.linear(self.impl(x))
        if self.activation is not None:
            x_ple = self.activation(x_ple)
        return x_ple if x_linear is None else x_linear + x_ple

    def forward(self, x: Tensor) -> Tensor:
        if x.ndim != 2:
            raise ValueError("Only inputs with shape [batch_size, n_features] are supported")
        if x.shape[1] != self.n_features:
            raise ValueError(f"Expected {self.n_features} numerical features, got {x.shape[1]}")
        if x.device.type != "cuda":
            return self._forward_cpu(x)
        if x.device != self._cuda_bin_edges.device:
            raise RuntimeError("x and the module must be on the same CUDA device")

        self._check_cuda_inputs(x)
        out_dtype = self._cuda_output_dtype()
        assert out_dtype in SUPPORTED_OUTPUT_DTYPES
        bias = self.linear.bias
        l0 = self.linear0
        shape_fd = (self.n_features, self.d_embedding)

        def fusable(t) -> bool:
            return t.dtype == torch.float32 and t.is_contiguous() and t.device == x.device and t.shape == shape_fd

        if l0 is None and bias is not None and fusable(bias):
            out, _, _ = _ops.forward_epilogue(
                x, self._cuda_bin_edges, self._cuda_inv_bin_widths, self._cuda_n_bins, self.linear.weight,
                bias, None, None, self.activation is not None, torch.is_grad_enabled(), out_dtype,
            )
            return out
        if l0 is not None and bias is None and fusable(l0.weight) and fusable(l0.bias):
            out, _, _ = _ops.forward_epilogue(
                x, self._cuda_bin_edges, self._cuda_inv_bin_widths, self._cuda_n_bins, self.linear.weight,
                None, l0.weight, l0.bias, self.activation is not None, torch.is_grad_enabled(), out_dtype,
            )
            return out

        # unfused tail: the reference's sequence of PyTorch ops
        x_linear = None if l0 is None else l0(x)
        x_ple, _ = _ops.forward(
            x, self._cuda_bin_edges, self._cuda_inv_bin_widths, self._cuda_n_bins, self.linear.weight, out_dtype,
        )
        if bias is not None:
            x_ple = x_ple + bias
        if self.activation is not None:
            x_ple = self.activation(x_ple)
        return x_ple if x_linear is None else x_linear + x_ple
