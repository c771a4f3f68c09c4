"""Seeded synthetic workloads of the benchmark configurations.

``configs[0..4]`` of the build's baseline description:

0. plumbing: N=256, F=8, 48 bins, d=24, fp32; x ~ N(0, 1) (seed 0); edges are
   49 quantiles of 10k seeded N(0, 1) draws per feature; W, b ~ U(+-1/sqrt(48)).
1. forward / fwd+bwd headline: N=65536, F=128, 48 bins, d=32, fp32; x ~ N(0, 1);
   5% of the entries are replaced by an exact copy of one of the feature's
   edges (e_0 .. e_n, uniform), 1% are moved outside the edge range
   (e_0 - 3 (e_n - e_0) u or e_n + 3 (e_n - e_0) u, u ~ U(0, 1], 50/50).
2. ragged: N=16384, F=64, d=64; per-feature bin count ~ U{2..128}; features by
   thirds lognormal(0, 1) / U(-5, 5) / Poisson(3); edges = unique quantiles
   (duplicates collapse, down to a single bin).
3. contention: N=262144, F=32, 256 bins, d=16; 90% of x ~ N(c_f, 0.05) around a
   seeded centre, 10% ~ N(0, 1); edges from 10k N(0, 1) draws.
4. wide bf16: N=8192, F=1024, 96 bins, d=24; features 50/50 N(0, 1) /
   lognormal; W, b and the output in bf16 with fp32 accumulation.

Everything is generated with NumPy's PCG64 so the arrays are identical on every
machine.  ``n_samples`` shrinks a configuration for quick checks.  The
gradient is not generated here (it is as large as the output); callers draw it
where they need it.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

CONFIG_NAMES = ("c0_plumbing", "c1_headline", "c2_ragged", "c3_contention", "c4_wide_bf16")
FULL_SAMPLES = (256, 65536, 16384, 262144, 8192)


@dataclass
class Workload:
    name: str
    x: np.ndarray                 # float32 [N, F]
    bins: list                    # F float32 edge arrays
    edges: np.ndarray             # float32 [F, Bmax + 1], +inf padded
    inv_widths: np.ndarray        # float32 [F, Bmax], 0 padded
    n_bins: np.ndarray            # int32 [F]
    weight: np.ndarray            # float32 [F, Bmax, d]
    bias: np.ndarray              # float32 [F, d]
    quant: str = "f32"            # rounding dtype of the PLE branch
    meta: dict = field(default_factory=dict)

    @property
    def shape(self):
        n, f = self.x.shape
        return n, f, self.weight.shape[1], self.weight.shape[2]


def pad_bins(bins):
    """``[F, Bmax+1]`` +inf-padded edges, ``[F, Bmax]`` 0-padded fp32 inverse
    widths and int32 bin counts, as the module builds them."""
    n_bins = np.array([len(e) - 1 for e in bins], dtype=np.int32)
    bmax = int(n_bins.max())
    edges = np.full((len(bins), bmax + 1), np.inf, dtype=np.float32)
    inv_w = np.zeros((len(bins), bmax), dtype=np.float32)
    for f, e in enumerate(bins):
        e = np.asarray(e, dtype=np.float32)
        edges[f, : e.size] = e
        inv_w[f, : e.size - 1] = np.float32(1.0) / (e[1:] - e[:-1])
    return edges, inv_w, n_bins


def _quantile_edges(draws: np.ndarray, n_bins: int) -> np.ndarray:
    q = np.quantile(draws.astype(np.float64), np.linspace(0.0, 1.0, n_bins + 1))
    e = np.unique(q.astype(np.float32))
    return e


def _params(rng, f, bmax, d):
    bound = np.float32(bmax ** -0.5)
    w = rng.uniform(-bound, bound, size=(f, bmax, d)).astype(np.float32)
    b = rng.uniform(-bound, bound, size=(f, d)).astype(np.float32)
    return w, b


def _finish(name, x, bins, rng, d, quant="f32", meta=None):
    edges, inv_w, n_bins = pad_bins(bins)
    w, b = _params(rng, len(bins), edges.shape[1] - 1, d)
    return Workload(name, np.ascontiguousarray(x, dtype=np.float32), bins, edges, inv_w, n_bins, w, b,
                    quant=quant, meta=meta or {})


def config0(n_samples: int | None = None) -> Workload:
    n = n_samples or 256
    rng = np.random.default_rng(0)
    f, nb, d = 8, 48, 24
    x = rng.standard_normal((n, f)).astype(np.float32)
    bins = [_quantile_edges(rng.standard_normal(10_000), nb) for _ in range(f)]
    return _finish("c0_plumbing", x, bins, rng, d)


def config1(n_samples: int | None = None) -> Workload:
    n = n_samples or 65536
    rng = np.random.default_rng(1)
    f, nb, d = 128, 48, 32
    bins = [_quantile_edges(rng.standard_normal(10_000), nb) for _ in range(f)]
    x = rng.standard_normal((n, f)).astype(np.float32)
    for j, e in enumerate(bins):
        col = x[:, j]
        hit = rng.random(n) < 0.05
        col[hit] = e[rng.integers(0, e.size, size=int(hit.sum()))]
        out = (~hit) & (rng.random(n) < 0.01 / 0.95)
        m = int(out.sum())
        u = 1.0 - rng.random(m)                           # U(0, 1]
        span = float(e[-1] - e[0])
        below = rng.random(m) < 0.5
        col[out] = np.where(below, e[0] - 3.0 * span * u, e[-1] + 3.0 * span * u).astype(np.float32)
    return _finish("c1_headline", x, bins, rng, d)


def config2(n_samples: int | None = None) -> Workload:
    n = n_samples or 16384
    rng = np.random.default_rng(2)
    f, d = 64, 64
    kinds = [("lognormal", "uniform", "poisson")[j * 3 // f] for j in range(f)]
    bins, cols = [], []
    for j in range(f):
        nb = int(rng.integers(2, 129))
        kind = kinds[j]
        if kind == "lognormal":
            draw = lambda size: rng.lognormal(0.0, 1.0, size)      # noqa: E731
        elif kind == "uniform":
            draw = lambda size: rng.uniform(-5.0, 5.0, size)       # noqa: E731
        else:
            draw = lambda size: rng.poisson(3.0, size).astype(np.float64)  # noqa: E731
        bins.append(_quantile_edges(draw(10_000), nb))
        cols.append(draw(n).astype(np.float32))
    x = np.stack(cols, axis=1)
    return _finish("c2_ragged", x, bins, rng, d, meta={"kinds": kinds})


def config3(n_samples: int | None = None) -> Workload:
    n = n_samples or 262144
    rng = np.random.default_rng(3)
    f, nb, d = 32, 256, 16
    bins = [_quantile_edges(rng.standard_normal(10_000), nb) for _ in range(f)]
    centres = rng.uniform(-1.5, 1.5, size=f)
    x = np.empty((n, f), dtype=np.float32)
    for j in range(f):
        narrow = rng.random(n) < 0.9
        col = rng.standard_normal(n)
        col[narrow] = centres[j] + 0.05 * rng.standard_normal(int(narrow.sum()))
        x[:, j] = col.astype(np.float32)
    return _finish("c3_contention", x, bins, rng, d, meta={"centres": centres})


def config4(n_samples: int | None = None) -> Workload:
    n = n_samples or 8192
    rng = np.random.default_rng(4)
    f, nb, d = 1024, 96, 24
    bins, cols = [], []
    for j in range(f):
        if j % 2 == 0:
            draw = lambda size: rng.standard_normal(size)           # noqa: E731
        else:
            draw = lambda size: rng.lognormal(0.0, 1.0, size)       # noqa: E731
        bins.append(_quantile_edges(draw(10_000), nb))
        cols.append(draw(n).astype(np.float32))
    x = np.stack(cols, axis=1)
    return _finish("c4_wide_bf16", x, bins, rng, d, quant="bf16")


CONFIGS = (config0, config1, config2, config3, config4)


def make(index: int, n_samples: int | None = None) -> Workload:
    return CONFIGS[index](n_samples)


def algorithmic_bytes(n, f, bmax, d, out_bytes=4, w_bytes=4, b_bytes=4, idx_bytes=None, grad_bytes=None):
    """Compulsory HBM bytes of one forward and one backward pass.

    Forward: x, output, bin indices, edges, inverse widths, n_bins, W, b.
    Backward: grad_output, x, bin indices, edges + inverse widths + n_bins, W,
    dx, dW, db.  Each external tensor counted once; scratch excluded.
    """
    if idx_bytes is None:
        idx_bytes = 1 if bmax <= 256 else (2 if bmax <= 32768 else 4)
    if grad_bytes is None:
        grad_bytes = out_bytes
    fwd = (n * f * 4 + n * f * d * out_bytes + n * f * idx_bytes + f * (bmax + 1) * 4 + f * bmax * 4 + f * 4
           + f * bmax * d * w_bytes + f * d * b_bytes)
    bwd = (n * f * d * grad_bytes + n * f * 4 + n * f * idx_bytes + f * (2 * bmax + 2) * 4
           + f * bmax * d * w_bytes + n * f * 4 + f * bmax * d * 4 + f * d * 4)
    return fwd, bwd
