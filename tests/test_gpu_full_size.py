"""Configurations c1-c4 at their full sizes (c1 N=65536 F=128 48 bins d=32;
c2 N=16384 F=64 ragged bins up to 128 d=64; c3 N=262144 F=32 256 bins d=16;
c4 N=8192 F=1024 96 bins d=24 in bf16), through checks whose cost does not
grow past a few seconds:

* bin indices exact against the closed form (``oracle.ple_oracle.bin_indices``);
* 512 sampled sample rows bit-exact against the C mirror of the reference
  forward arithmetic (fp32 with the fused bias; c4: bf16 output);
* dx, dW and db against float64 closed forms evaluated on the GPU with torch
  (dW: per-bin sums of q(frac)·g plus the suffix sums of g over the higher bins,
  placed at the physical slots; dx: iw_k <g, q(W[phys k])> plus the lower bin's
  term for x on an inner edge; db: the sum of g), each within the fp32 bar
  ``|err| <= 1e-6 + 1e-5 * sum|terms|``; c4 (bf16 gradient, bf16 rounding of W
  and frac, as the reference's low-precision path) within ``1e-2 * sum|terms|``
  of the bf16-aware closed form and within 1e-2 normwise of unrounded fp32
  math;
* determinism (bitwise-equal repeats; c3 is the contention configuration,
  90% of its samples in about 5% of the bins) and, for fp32, linearity in the
  gradient.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ple_oracle as po
from piecewiselinearembeddings_optimized_amd import workloads
from tests.ple_cases import BF16_RTOL, FP32_ATOL, FP32_RTOL, close_scaled, normwise_rel

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module", params=(1, 2, 3, 4), ids=lambda c: workloads.CONFIG_NAMES[c])
def cfg(request):
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    w = workloads.make(request.param)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    ins = (t(w.x), t(w.edges), t(w.inv_widths), t(w.n_bins), t(w.weight), t(w.bias))
    yield w, ins, torch.ops.rtdl_num_embeddings_cuda
    del ins
    torch.cuda.empty_cache()


def _report(name, ok, worst):
    print(f"  {name}: worst error / allowance = {worst:.3g}", flush=True)
    assert ok, f"{name} outside tolerance (worst ratio {worst:.3g})"


def test_full_size_forward(cfg, c_oracle):
    w, (x, e, iw, nb, wt, bt), ops = cfg
    bf16 = w.quant == "bf16"
    print(f"full-size forward {w.name} shape={w.shape} quant={w.quant}", flush=True)
    if bf16:
        out, idx = ops.forward(x, e, iw, nb, wt, torch.bfloat16)
    else:
        out, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), po.bin_indices(w.x, w.edges, w.n_bins))
    rows = np.sort(np.random.default_rng(11).choice(w.shape[0], 512, replace=False))
    mirror, _ = c_oracle.forward_f32(w.x[rows], w.edges, w.inv_widths, w.n_bins, w.weight,
                                     bias=None if bf16 else w.bias, quant=w.quant)
    got = out[torch.from_numpy(rows).to(DEV)].float().cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), mirror.view(np.uint32))


def _reference_backward(x, e, iw, nb, wt, idx, g, quant=None):
    """float64 closed forms of dx, dW, db and their sums of |terms| (torch on the GPU);
    with ``quant`` (a torch dtype) W and frac are rounded through it first."""
    n, f = x.shape
    B, d = wt.shape[1], wt.shape[2]
    k = idx.long()
    fidx = torch.arange(f, device=DEV).expand(n, f)
    e_k = e[fidx, k]
    iw_k = iw[fidx, k]
    frac = (x - e_k) * iw_k                          # fp32, as the kernels form it (no fma)
    if quant is not None:
        frac = frac.to(quant).float()
        wt = wt.to(quant).float()
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


def test_full_size_backward(cfg):
    w, (x, e, iw, nb, wt, bt), ops = cfg
    n, f, bmax, d = w.shape
    bf16 = w.quant == "bf16"
    print(f"full-size backward {w.name} shape={w.shape} quant={w.quant}", flush=True)
    gen = torch.Generator(DEV).manual_seed(5)
    g = torch.randn((n, f, d), device=DEV, generator=gen)
    if bf16:
        _, idx = ops.forward(x, e, iw, nb, wt, torch.bfloat16)
        g = g.bfloat16()

        def run(gg):
            gx_, gw_ = ops.backward(gg, x, e, iw, nb, wt, idx, True, True)
            return gx_, gw_, None
    else:
        _, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)

        def run(gg):
            return ops.backward_with_bias(gg, x, e, iw, nb, wt, idx, torch.float32, True, True, True)

    gx, gw, gb = run(g)
    # determinism: a second call gives the same bits
    gx2, gw2, gb2 = run(g)
    torch.cuda.synchronize()
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2) and (gb is None or torch.equal(gb, gb2))
    del gx2, gw2, gb2
    quant = torch.bfloat16 if bf16 else None
    dx, dx_abs, dw, dw_abs, db, db_abs = _reference_backward(x, e, iw, nb, wt, idx, g, quant)
    rtol, atol = (BF16_RTOL, 0.0) if bf16 else (FP32_RTOL, FP32_ATOL)
    checks = [("dx", gx, dx, dx_abs), ("dW", gw, dw, dw_abs)] + ([] if gb is None else [("db", gb, db, db_abs)])
    for name, got, ref, s in checks:
        _report(name, *close_scaled(got.cpu().numpy(), ref.cpu().numpy(), s.cpu().numpy(), rtol, atol))
    del dx, dx_abs, dw, dw_abs, db, db_abs
    if bf16:
        # against unrounded fp32 math (W and frac not rounded), normwise, at the bf16 bar
        rx, _, rw, _, _, _ = _reference_backward(x, e, iw, nb, wt, idx, g, None)
        for name, got, ref in (("dx", gx, rx), ("dW", gw, rw)):
            rel = normwise_rel(got.cpu().numpy(), ref.cpu().numpy())
            print(f"  {name} vs unrounded fp32 math: normwise relative error {rel:.3g}", flush=True)
            assert rel <= BF16_RTOL
        return
    # linearity in the gradient
    g2 = torch.randn((n, f, d), device=DEV, generator=gen)
    hx, hw, hb = run(g2)
    sx, sw, sb = run(g + g2)
    torch.cuda.synchronize()
    for name, s_, a_, b_ in (("dx", sx, gx, hx), ("dW", sw, gw, hw), ("db", sb, gb, hb)):
        rel = normwise_rel(s_.cpu().numpy(), (a_.double() + b_.double()).cpu().numpy())
        print(f"  linearity {name}: normwise relative error {rel:.3g}", flush=True)
        assert rel <= 1e-5


@pytest.fixture(scope="module")
def c4():
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    w = workloads.make(4)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    ins = (t(w.x), t(w.edges), t(w.inv_widths), t(w.n_bins), t(w.weight), t(w.bias))
    yield w, ins, torch.ops.rtdl_num_embeddings_cuda
    del ins
    torch.cuda.empty_cache()


def test_full_size_c4_with_bias(c4, c_oracle):
    """c4 as its configuration names it, with the bias b: the fused-bias
    operators with bf16 quantisation (the reference module under bf16 autocast,
    reference module.py:238-239: x_ple in bf16, + b in fp32).  Forward: sampled
    rows bit-exact against the C mirror (bf16-rounded x_ple, then + b in fp32).
    Backward with an fp32 gradient: dx and dW use the gradient rounded to bf16
    (at the bf16 bar of the bf16-aware closed form), db is the sum of the
    unrounded gradient (at the fp32 bar)."""
    w, (x, e, iw, nb, wt, bt), ops = c4
    n, f, bmax, d = w.shape
    print(f"full-size c4 with bias shape={w.shape}", flush=True)
    out, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.bfloat16)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), po.bin_indices(w.x, w.edges, w.n_bins))
    rows = np.sort(np.random.default_rng(12).choice(n, 256, replace=False))
    mirror, _ = c_oracle.forward_f32(w.x[rows], w.edges, w.inv_widths, w.n_bins, w.weight, bias=w.bias, quant="bf16")
    got = out[torch.from_numpy(rows).to(DEV)].cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), mirror.view(np.uint32))
    del out

    g = torch.randn((n, f, d), device=DEV, generator=torch.Generator(DEV).manual_seed(7))
    gx, gw, gb = ops.backward_with_bias(g, x, e, iw, nb, wt, idx, torch.bfloat16, True, True, True)
    gx2, gw2, gb2 = ops.backward_with_bias(g, x, e, iw, nb, wt, idx, torch.bfloat16, True, True, True)
    torch.cuda.synchronize()
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2) and torch.equal(gb, gb2)
    del gx2, gw2, gb2
    gq = g.bfloat16().float()
    dx, dx_abs, dw, dw_abs, _, _ = _reference_backward(x, e, iw, nb, wt, idx, gq, torch.bfloat16)
    for name, got_, ref, s in (("dx", gx, dx, dx_abs), ("dW", gw, dw, dw_abs)):
        _report(name, *close_scaled(got_.cpu().numpy(), ref.cpu().numpy(), s.cpu().numpy(), BF16_RTOL, 0.0))
    del dx, dx_abs, dw, dw_abs
    db = g.double().sum(0)
    db_abs = g.double().abs().sum(0)
    _report("db (unrounded gradient)", *close_scaled(gb.cpu().numpy(), db.cpu().numpy(), db_abs.cpu().numpy(),
                                                     FP32_RTOL, FP32_ATOL))


def test_full_size_c4_module_under_bf16_autocast(c4):
    """The module (version A, with its bias) at c4 size under bf16 autocast,
    as the reference module runs it there (module.py:145-158, 238-239): the
    output is fp32, its gradients land in .grad -- x.grad and weight.grad at
    the bf16 bar of the bf16-aware float64 closed form (the gradient reaches
    the operator rounded to bf16), bias.grad at the fp32 bar of the sum of the
    unrounded gradient."""
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings

    w, (x, e, iw, nb, wt, bt), ops = c4
    n, f, bmax, d = w.shape
    print(f"full-size c4 module under bf16 autocast shape={w.shape}", flush=True)
    bins = [torch.from_numpy(w.edges[j, : int(w.n_bins[j]) + 1].copy()) for j in range(f)]
    m = CudaPiecewiseLinearEmbeddings(bins, d, activation=False, version="A").to(DEV)
    with torch.no_grad():
        m.linear.weight.copy_(wt)
        m.linear.bias.copy_(bt)
    xr = x.clone().requires_grad_(True)
    g = torch.randn((n, f, d), device=DEV, generator=torch.Generator(DEV).manual_seed(8))
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = m(xr)
    assert out.dtype == torch.float32
    out.backward(g)
    torch.cuda.synchronize()
    # (the module's own padded tables: its inverse widths are its own computation)
    me, miw, mnb = m._cuda_bin_edges, m._cuda_inv_bin_widths, m._cuda_n_bins
    _, idx = ops.forward(x, me, miw, mnb, wt, torch.bfloat16)
    gq = g.bfloat16().float()
    dx, dx_abs, dw, dw_abs, _, _ = _reference_backward(x, me, miw, mnb, wt, idx, gq, torch.bfloat16)
    for name, got_, ref, s in (("x.grad", xr.grad, dx, dx_abs), ("weight.grad", m.linear.weight.grad, dw, dw_abs)):
        _report(name, *close_scaled(got_.cpu().numpy(), ref.cpu().numpy(), s.cpu().numpy(), BF16_RTOL, 0.0))
    del dx, dx_abs, dw, dw_abs
    db = g.double().sum(0)
    _report("bias.grad", *close_scaled(m.linear.bias.grad.cpu().numpy(), db.cpu().numpy(),
                                       g.double().abs().sum(0).cpu().numpy(), FP32_RTOL, FP32_ATOL))
