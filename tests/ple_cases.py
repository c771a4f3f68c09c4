"""Shared test inputs: the reference suite's bin sets, input sampler and
parameter initialisation, restated so the parity tests exercise the same cases
as the reference's own ``tests/test_correctness.py``.
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

with open(os.path.join(HERE, "golden", "reference_bin_sets.json")) as fh:
    _BIN_SETS = {k: v for k, v in json.load(fh).items() if not k.startswith("_")}

BIN_CASE_NAMES = ("equal", "ragged", "single_bin", "all_single_bin")
D_EMBEDDING_VALUES = (10, 15, 20)
SEED_VALUES = (42, 0, 1)

# tolerances of the reference suite (tests/test_correctness.py:18-28)
FORWARD_RTOL, FORWARD_ATOL = 2e-5, 2e-6
GRAD_RTOL, GRAD_ATOL = 9e-5, 9e-6
AMP_FORWARD_RTOL, AMP_FORWARD_ATOL = 8e-3, 8e-3
AMP_GRAD_RTOL, AMP_GRAD_ATOL = 2e-2, 2e-2

# tolerances of the build's parity bar: fp32 1e-5 relative / 1e-6 absolute,
# bf16 1e-2 relative, the relative part scaled by the sum of |terms| of each
# reduction (an fp32 sum in a different order cannot do better than that)
FP32_RTOL, FP32_ATOL = 1e-5, 1e-6
BF16_RTOL = 1e-2


def make_bins(case_name: str, dtype=torch.float32) -> list[torch.Tensor]:
    """Literal bin sets of ``tests/utils/generate_bins.py:18-84`` (reference)."""
    if case_name not in _BIN_SETS:
        raise ValueError(f"Unknown bin case: {case_name!r}")
    return [torch.tensor(e, dtype=dtype) for e in _BIN_SETS[case_name]]


def sample_features(bins, *, batch_size: int, seed: int) -> torch.Tensor:
    """Input sampler of ``tests/utils/generate_input.py:5-32`` (reference).

    Same torch RNG calls in the same order, so the same seed gives the same
    tensor: half ``randn * range + min``, a quarter below the first edge, a
    quarter above the last edge, stacked per feature.
    """
    torch.manual_seed(seed)
    assert batch_size % 4 == 0
    half, quarter = batch_size // 2, batch_size // 4
    cols = []
    for edges in bins:
        lo, hi = edges[0].item(), edges[-1].item()
        inside = torch.randn(half) * (hi - lo) + lo
        below = lo - torch.rand(quarter).abs() * (hi - lo)
        above = hi + torch.rand(quarter).abs() * (hi - lo)
        cols.append(torch.cat([inside, below, above]))
    return torch.stack(cols, dim=1)


@torch.no_grad()
def init_parameters_(module, *, seed: int) -> None:
    """Parameter re-initialisation of ``tests/test_correctness.py:45-76``."""
    torch.manual_seed(seed)
    if module.linear.weight.is_cuda:
        torch.cuda.manual_seed_all(seed)
    module.linear.weight.uniform_(0.05, 0.25)
    if module.linear.bias is not None:
        module.linear.bias.uniform_(0.10, 0.30)
    if module.linear0 is not None:
        module.linear0.weight.uniform_(-0.20, 0.20)
        module.linear0.bias.uniform_(-0.10, 0.10)


def with_edge_hits(x: torch.Tensor, bins, every: int = 7) -> torch.Tensor:
    """Copy of ``x`` where every ``every``-th row sits exactly on edges."""
    x = x.clone()
    for f, e in enumerate(bins):
        rows = torch.arange(0, x.shape[0], every)
        x[rows, f] = e[torch.arange(rows.numel()) % e.numel()].to(x.dtype)
    return x


def normwise_rel(actual, expected) -> float:
    """max |a - e| / max |e| over finite entries (relative error of the tensor)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    fin = np.isfinite(e)
    den = float(np.abs(e[fin]).max()) if fin.any() else 1.0
    return float(np.abs(a[fin] - e[fin]).max()) / (den if den > 0 else 1.0)


def close_scaled(actual, expected, abs_sum, rtol, atol) -> tuple[bool, float]:
    """``|a - e| <= atol + rtol * abs_sum`` elementwise (NaN == NaN, equal infs).

    Returns (ok, worst ratio of error to allowance).
    """
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    s = np.asarray(abs_sum, dtype=np.float64)
    both_nan = np.isnan(a) & np.isnan(e)
    same_inf = np.isinf(a) & np.isinf(e) & (np.sign(a) == np.sign(e))
    with np.errstate(invalid="ignore"):
        err = np.abs(a - e)
        allow = atol + rtol * np.where(np.isfinite(s), s, 0.0)
        ratio = np.where(both_nan | same_inf, 0.0, err / allow)
    ratio = np.where(np.isnan(ratio), np.inf, ratio)
    worst = float(ratio.max()) if ratio.size else 0.0
    return worst <= 1.0, worst
