"""GPU parity of the dense encoding kernels (``encode`` / ``encode_backward``).

The output is the upstream ``PiecewiseLinearEncoding`` (restated; the
package is not installed).  Forward: bit-exact against the closed form
evaluated with the kernel's fp32 arithmetic in NumPy
(``oracle.ple_oracle.encoding_closed_form``, pinned against the dense
upstream formulation in ``tests/test_oracle.py``), special values included;
against the CPU module (upstream's dense arithmetic) within the rounding of
its ``addcmul``.  Backward: dx within the fp32 bar of the float64 closed form
(pinned against torch autograd of the dense form) and against autograd of the
CPU module away from exact edge hits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ple_oracle as po
from piecewiselinearembeddings_optimized_amd import workloads
from tests.ple_cases import FP32_ATOL, FP32_RTOL, close_scaled

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ops = None
REDUCED = {0: None, 1: 1024, 2: 2048, 4: 256}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    global ops
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    ops = torch.ops.rtdl_num_embeddings_cuda
    yield


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _tables(w):
    offs = po.encoding_offsets(w.n_bins).astype(np.int32)
    return _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(offs), int(np.sum(w.n_bins))


def _with_special(w):
    x = w.x.copy()
    n, f = x.shape
    rng = np.random.default_rng(9)
    for r in range(min(n, 64)):
        c = r % f
        k = rng.integers(0, int(w.n_bins[c]) + 1)
        x[r, c] = w.edges[c, k]                       # exact edge hits, both ends included
    x[min(n - 1, 64), 0] = np.nan
    x[min(n - 1, 65), 0] = np.inf
    x[min(n - 1, 66), 0] = -np.inf
    return x


@pytest.mark.parametrize("cfg", [0, 1, 2, 4])
def test_encode_matches_closed_form_bitwise(cfg):
    w = workloads.make(cfg, REDUCED[cfg])
    x = _with_special(w)
    print(f"encode {w.name} shape={w.shape} total_bins={int(np.sum(w.n_bins))}", flush=True)
    e, iw, nb, offs, total = _tables(w)
    out = ops.encode(_t(x), e, iw, nb, offs, total)
    torch.cuda.synchronize()
    assert out.shape == (x.shape[0], total) and out.dtype == torch.float32
    exp = po.encoding_closed_form(x, w.edges, w.inv_widths, w.n_bins, dtype=np.float32).astype(np.float32)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got, exp)                      # NaN where expected
    fin = ~np.isnan(exp)
    np.testing.assert_array_equal(got[fin].view(np.uint32), exp[fin].view(np.uint32))   # and every bit elsewhere


@pytest.mark.parametrize("case_name", ["equal", "ragged", "single_bin", "all_single_bin"])
def test_encoding_module_matches_cpu_module(case_name):
    from piecewiselinearembeddings_optimized_amd import CudaPiecewiseLinearEncoding
    from tests.ple_cases import make_bins, sample_features

    bins = make_bins(case_name)
    cpu = CudaPiecewiseLinearEncoding(bins)
    gpu = CudaPiecewiseLinearEncoding(bins).to(DEV)
    x = sample_features(bins, batch_size=256, seed=12)
    xc = x.clone().requires_grad_(True)
    xg = x.to(DEV).requires_grad_(True)
    oc, og = cpu(xc), gpu(xg)
    assert og.shape == oc.shape == (256,) + tuple(gpu.get_output_shape())
    # upstream computes (1/w) x + (-e/w) with addcmul: a few ulp of |x / w|
    scale = (x.abs()[:, :, None] + 1.0) * torch.tensor(po.pad_bins([b.numpy() for b in bins])[1]).max()
    torch.testing.assert_close(og.detach().cpu(), oc.detach(), rtol=1e-5, atol=float(scale.max()) * 1e-6)
    g = torch.randn(oc.shape, generator=torch.Generator().manual_seed(1))
    oc.backward(g)
    og.backward(g.to(DEV))
    torch.testing.assert_close(xg.grad.cpu(), xc.grad, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("cfg", [0, 1, 2, 4])
def test_encode_backward_matches_oracle(cfg):
    w = workloads.make(cfg, REDUCED[cfg])
    x = _with_special(w)
    x[~np.isfinite(x)] = 0.0                          # dx at NaN / inf is not specified upstream
    e, iw, nb, offs, total = _tables(w)
    g = np.random.default_rng(cfg).standard_normal((x.shape[0], total)).astype(np.float32)
    gx = ops.encode_backward(_t(g), _t(x), e, iw, nb, offs)
    torch.cuda.synchronize()
    ref, ref_abs = po.encoding_backward(g, x, w.edges, w.inv_widths, w.n_bins)
    ok, worst = close_scaled(gx.cpu().numpy(), ref, ref_abs, FP32_RTOL, FP32_ATOL)
    print(f"  dx: worst error / allowance = {worst:.3g}", flush=True)
    assert ok


def test_encode_autograd_and_c_abi():
    from piecewiselinearembeddings_optimized_amd import capi

    w = workloads.make(2, 512)
    e, iw, nb, offs, total = _tables(w)
    x = _t(w.x).requires_grad_(True)
    out = ops.encode(x, e, iw, nb, offs, total)
    g = torch.randn(out.shape, device=DEV, generator=torch.Generator(DEV).manual_seed(2))
    out.backward(g)
    direct = ops.encode_backward(g, x.detach(), e, iw, nb, offs)
    assert torch.equal(x.grad, direct)
    out2 = torch.empty_like(out)
    capi.encode(x.detach(), e, iw, nb, offs, out2)
    gx2 = torch.empty_like(direct)
    capi.encode_backward(g, x.detach(), e, iw, nb, offs, gx2)
    torch.cuda.synchronize()
    assert torch.equal(out2, out.detach()) and torch.equal(gx2, direct)
    with pytest.raises(capi.PleError) as ei:
        capi.encode(x.detach(), e, iw, nb, offs, torch.empty((512, 0), device=DEV))
    assert ei.value.code == -2


def test_opcheck_and_compile_encoding():
    from piecewiselinearembeddings_optimized_amd import CudaPiecewiseLinearEncoding
    from tests.ple_cases import make_bins, sample_features

    w = workloads.make(0, 64)
    e, iw, nb, offs, total = _tables(w)
    x = _t(w.x).requires_grad_(True)
    torch.library.opcheck(ops.encode.default, (x, e, iw, nb, offs, total))
    g = torch.randn((64, total), device=DEV)
    torch.library.opcheck(ops.encode_backward.default, (g, x.detach(), e, iw, nb, offs))
    torch._dynamo.reset()
    bins = make_bins("ragged")
    m = CudaPiecewiseLinearEncoding(bins).to(DEV)
    cm = torch.compile(m, fullgraph=True, dynamic=True, backend="aot_eager")
    for batch in (32, 48):
        xb = sample_features(bins, batch_size=batch, seed=batch).to(DEV)
        torch.testing.assert_close(cm(xb), m(xb), rtol=0, atol=0)
