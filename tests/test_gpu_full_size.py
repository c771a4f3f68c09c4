"""The headline configuration c1 (N=65536, F=128, 48 bins, d=32, fp32) at its
full size, through checks whose cost does not grow past a few seconds:

* bin indices exact against the closed form (``oracle.ple_oracle.bin_indices``);
* 512 sampled sample rows bit-exact against the C mirror of the reference
  forward arithmetic;
* dx, dW and db against float64 closed forms evaluated on the GPU with torch
  (dW: per-bin sums of q(frac)·g plus the suffix sums of g over the higher bins,
  placed at the physical slots; dx: iw_k <g, q(W[phys k])> plus the lower bin's
  term for x on an inner edge; db: the sum of g), each within the fp32 bar
  ``|err| <= 1e-6 + 1e-5 * sum|terms|``;
* determinism (bitwise-equal repeats) and linearity in the gradient.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ple_oracle as po
from piecewiselinearembeddings_optimized_amd import workloads
from tests.ple_cases import FP32_ATOL, FP32_RTOL, close_scaled, normwise_rel

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def c1():
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    w = workloads.make(1)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    ins = (t(w.x), t(w.edges), t(w.inv_widths), t(w.n_bins), t(w.weight), t(w.bias))
    return w, ins, torch.ops.rtdl_num_embeddings_cuda


def _report(name, ok, worst):
    print(f"  {name}: worst error / allowance = {worst:.3g}", flush=True)
    assert ok, f"{name} outside tolerance (worst ratio {worst:.3g})"


def test_full_size_forward(c1, c_oracle):
    w, (x, e, iw, nb, wt, bt), ops = c1
    print(f"full-size forward {w.name} shape={w.shape}", flush=True)
    out, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), po.bin_indices(w.x, w.edges, w.n_bins))
    rows = np.sort(np.random.default_rng(11).choice(w.shape[0], 512, replace=False))
    mirror, _ = c_oracle.forward_f32(w.x[rows], w.edges, w.inv_widths, w.n_bins, w.weight, bias=w.bias)
    got = out[torch.from_numpy(rows).to(DEV)].cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), mirror.view(np.uint32))


def _reference_backward(x, e, iw, nb, wt, idx, g):
    """float64 closed forms of dx, dW, db and their sums of |terms| (torch on the GPU)."""
    n, f = x.shape
    B, d = wt.shape[1], wt.shape[2]
    k = idx.long()
    fidx = torch.arange(f, device=DEV).expand(n, f)
    e_k = e[fidx, k]
    iw_k = iw[fidx, k]
    frac = (x - e_k) * iw_k                          # fp32, as the kernels form it (no fma)
    g64 = g.double()
    key = (fidx * B + k).reshape(-1)
    bucket = torch.zeros(f * B, d, dtype=torch.float64, device=DEV)
    weighted = torch.zeros_like(bucket)
    bucket_abs = torch.zeros_like(bucket)
    weighted_abs = torch.zeros_like(bucket)
    fg = frac.double().unsqueeze(-1) * g64
    bucket.index_add_(0, key, g64.reshape(-1, d))
    weighted.index_add_(0, key, fg.reshape(-1, d))
    bucket_abs.index_add_(0, key, g64.abs().reshape(-1, d))
    weighted_abs.index_add_(0, key, fg.abs().reshape(-1, d))
    del fg

    def suffix(t):
        t = t.reshape(f, B, d)
        cs = t.cumsum(1)
        return cs[:, -1:, :] - cs                    # sum over the higher bins

    val = weighted.reshape(f, B, d) + suffix(bucket)
    val_abs = weighted_abs.reshape(f, B, d) + suffix(bucket_abs)
    dw = torch.zeros(f, B, d, dtype=torch.float64, device=DEV)
    dw_abs = torch.zeros_like(dw)
    for j, nfj in enumerate(nb.tolist()):
        nfj = max(1, min(int(nfj), B))
        dw[j, : nfj - 1] = val[j, : nfj - 1]
        dw_abs[j, : nfj - 1] = val_abs[j, : nfj - 1]
        dw[j, B - 1] = val[j, nfj - 1]
        dw_abs[j, B - 1] = val_abs[j, nfj - 1]
    db = g64.sum(0)
    db_abs = g64.abs().sum(0)

    # dx: the physical slot of bin k is B - 1 for the last real bin
    nbf = nb.long().clamp(1, B)[None, :].expand(n, f)
    phys = torch.where(k == nbf - 1, torch.full_like(k, B - 1), k)
    w64 = wt.double().reshape(f * B, d)
    prod = g64 * w64[(fidx * B + phys).reshape(-1)].reshape(n, f, d)
    dx = iw_k.double() * prod.sum(-1)
    dx_abs = iw_k.double() * prod.abs().sum(-1)
    del prod
    edge = (k > 0) & (x == e_k)
    if bool(edge.any()):
        kp = (k - 1).clamp(min=0)
        iw_p = iw[fidx, kp].double()
        prod = g64 * w64[(fidx * B + kp).reshape(-1)].reshape(n, f, d)
        dx = dx + torch.where(edge, iw_p * prod.sum(-1), torch.zeros_like(dx))
        dx_abs = dx_abs + torch.where(edge, iw_p * prod.abs().sum(-1), torch.zeros_like(dx))
        del prod
    return dx, dx_abs, dw, dw_abs, db, db_abs


def test_full_size_backward(c1):
    w, (x, e, iw, nb, wt, bt), ops = c1
    n, f, bmax, d = w.shape
    print(f"full-size backward {w.name} shape={w.shape}", flush=True)
    _, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    gen = torch.Generator(DEV).manual_seed(5)
    g = torch.randn((n, f, d), device=DEV, generator=gen)
    gx, gw, gb = ops.backward_with_bias(g, x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    # determinism: a second call gives the same bits
    gx2, gw2, gb2 = ops.backward_with_bias(g, x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    torch.cuda.synchronize()
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2) and torch.equal(gb, gb2)
    del gx2, gw2, gb2
    dx, dx_abs, dw, dw_abs, db, db_abs = _reference_backward(x, e, iw, nb, wt, idx, g)
    for name, got, ref, s in (("dx", gx, dx, dx_abs), ("dW", gw, dw, dw_abs), ("db", gb, db, db_abs)):
        _report(name, *close_scaled(got.cpu().numpy(), ref.cpu().numpy(), s.cpu().numpy(), FP32_RTOL, FP32_ATOL))
    # linearity in the gradient
    g2 = torch.randn((n, f, d), device=DEV, generator=gen)
    hx, hw, hb = ops.backward_with_bias(g2, x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    sx, sw, sb = ops.backward_with_bias(g + g2, x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    torch.cuda.synchronize()
    for name, s_, a_, b_ in (("dx", sx, gx, hx), ("dW", sw, gw, hw), ("db", sb, gb, hb)):
        rel = normwise_rel(s_.cpu().numpy(), (a_.double() + b_.double()).cpu().numpy())
        print(f"  linearity {name}: normwise relative error {rel:.3g}", flush=True)
        assert rel <= 1e-5
