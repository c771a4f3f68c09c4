"""Dense upstream PLE algorithm in PyTorch float32 -- TEST INFRASTRUCTURE ONLY.

The CPU path the reference falls back to (``module.py:222-223`` calls the
parent ``rtdl_num_embeddings.PiecewiseLinearEmbeddings`` of version 0.0.12),
restated: ``addcmul(-left/width, 1/width, x)`` -> first / middle / last
clamps -> ``cat`` -> per-feature matmul over ``[F, N, Bmax] x [F, Bmax, d]``
-> ``+ bias``; backward through autograd.  ``bench.py`` times it on the host
cores as the CPU baseline.
"""

from __future__ import annotations

import numpy as np
import torch


class DensePLE:
    """Upstream-style dense PLE over fixed bins (float32, CPU)."""

    def __init__(self, bins, weight: np.ndarray, bias: np.ndarray | None):
        n_bins = [len(e) - 1 for e in bins]
        bmax = max(n_bins)
        f = len(bins)
        slope = torch.zeros(f, bmax)
        offset = torch.zeros(f, bmax)
        for i, e in enumerate(bins):
            e = torch.as_tensor(np.asarray(e, dtype=np.float32))
            width = e.diff()
            w = 1.0 / width
            b = -e[:-1] / width
            slope[i, -1], offset[i, -1] = w[-1], b[-1]
            slope[i, : n_bins[i] - 1] = w[:-1]
            offset[i, : n_bins[i] - 1] = b[:-1]
        self.slope, self.offset = slope, offset
        single = torch.tensor(n_bins) == 1
        self.single = single if bool(single.any()) else None
        self.weight = torch.tensor(weight, dtype=torch.float32, requires_grad=True)
        self.bias = None if bias is None else torch.tensor(bias, dtype=torch.float32, requires_grad=True)

    def encode(self, x: torch.Tensor) -> torch.Tensor:
        z = torch.addcmul(self.offset, self.slope, x[..., None])
        if z.shape[-1] > 1:
            last = z[..., -1:]
            last = last.clamp_min(0.0) if self.single is None else torch.where(
                self.single[..., None], last, last.clamp_min(0.0))
            z = torch.cat([z[..., :1].clamp_max(1.0), z[..., 1:-1].clamp(0.0, 1.0), last], dim=-1)
        return z

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = (self.encode(x).transpose(0, 1) @ self.weight).transpose(0, 1)
        return y if self.bias is None else y + self.bias

    def forward_backward(self, x: torch.Tensor, grad: torch.Tensor):
        """One training step's PLE work: forward, then dx, dW, db by autograd."""
        self.weight.grad = None
        if self.bias is not None:
            self.bias.grad = None
        x = x.detach().requires_grad_(True)
        out = self.forward(x)
        out.backward(grad)
        return out, x.grad, self.weight.grad, None if self.bias is None else self.bias.grad
