"""GPU parity for per-feature tables beyond LDS, and for int32 bin indices.

The reference runs these shapes through its generic kernels (forward:
``csrc/forward_cuda.cu:293-425``, chosen at ``:478-512``; backward dx:
``csrc/backward_cuda.cu:343-492``, dW fallback ``:497-593``, chosen at
``:1274-1281,1361-1462``), and allocates int32 bin indices beyond 32768 bins
(``forward_cuda.cu:802-817``).  Here the forward takes the wide-table kernel
(prefix checkpoints in LDS, weights from global memory) and the backward the
fallback kernels (histogram cells in global memory when they exceed LDS).

Forward: bin indices exact and of the reference's dtype; float outputs
bit-exact against the C mirror of the reference arithmetic
(``oracle/ple_oracle.c``), which folds the prefix from bin 0 exactly as the
reference does.  Backward: dx, dW, db within the fp32 bar
(``|err| <= 1e-6 + 1e-5 * sum|terms|``) of the float64 oracle.  Forcing the
wide kernel or the global-cell histogram on shapes that fit LDS gives the same
bits as the LDS paths.
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
IDX_DTYPE = {1: torch.uint8, 2: torch.int16, 4: torch.int32}
QT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    global ops
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    ops = torch.ops.rtdl_num_embeddings_cuda
    yield


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def wide_case(n, f, bmax, d, seed):
    """Ragged per-feature edges (feature 0 has all bmax bins), x spread over
    every bin and 10% past either end, 10% exactly on an edge."""
    rng = np.random.default_rng(seed)
    bins = []
    for j in range(f):
        nb = bmax if j == 0 else int(rng.integers(max(1, bmax // 2), bmax + 1))
        e = np.cumsum(rng.uniform(0.05, 1.0, nb + 1)) - nb * 0.25
        bins.append(e.astype(np.float32))
    edges, iw, nbins = workloads.pad_bins(bins)
    x = np.empty((n, f), dtype=np.float32)
    for j, e in enumerate(bins):
        lo, hi = float(e[0]), float(e[-1])
        v = lo + (hi - lo) * rng.uniform(-0.05, 1.05, n)
        hit = rng.random(n) < 0.1
        v[hit] = e[rng.integers(0, e.size, int(hit.sum()))]
        x[:, j] = v
    wt = rng.uniform(-0.5, 0.5, (f, bmax, d)).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, (f, d)).astype(np.float32)
    return workloads.Workload(f"wide{n}x{f}x{bmax}x{d}", x, bins, edges, iw, nbins, wt, b)


def _inputs(w):
    return _t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight), _t(w.bias)


def _report(name, ok, worst):
    print(f"  {name}: worst error / allowance = {worst:.3g}", flush=True)
    assert ok, f"{name} outside tolerance (worst ratio {worst:.3g})"


def _check_backward(w, g, gx, gw, gb, c_oracle, quant="f32"):
    idx = po.bin_indices(w.x, w.edges, w.n_bins)
    ref = c_oracle.backward_f64(g, w.x, w.edges, w.inv_widths, w.n_bins, w.weight, idx, quant=quant)
    for name, got, key in (("dx", gx, "dx"), ("dW", gw, "dw"), ("db", gb, "db")):
        if got is not None:
            _report(name, *close_scaled(got.cpu().numpy(), ref[key], ref[key + "_abs"], FP32_RTOL, FP32_ATOL))


# (N, F, max bins, d): the shapes named for this path, then widths that take
# two- and one-column lanes, the int16 / int32 index boundary, and a table
# just past the LDS limit of the table kernel (320 bins at d = 64)
WIDE_SHAPES = [
    (2048, 4, 1024, 32), (2048, 4, 512, 64), (2048, 4, 4096, 16), (2048, 4, 40000, 4),
    (2048, 3, 32768, 2), (1024, 2, 32769, 3), (1500, 2, 320, 64), (1000, 3, 700, 62), (800, 2, 3000, 23),
]


@pytest.mark.parametrize("shape", WIDE_SHAPES, ids=[f"{n}x{f}x{b}x{d}" for n, f, b, d in WIDE_SHAPES])
def test_wide_tables_forward_and_backward(shape, c_oracle):
    n, f, bmax, d = shape
    w = wide_case(n, f, bmax, d, seed=sum(shape))
    print(f"wide tables {w.name}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, idx = ops.forward(x, e, iw, nb, wt, torch.float32)
    torch.cuda.synchronize()
    assert idx.dtype == IDX_DTYPE[po.bin_index_dtype(bmax).itemsize]
    mirror, midx = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), midx.astype(np.int64))
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), mirror.view(np.uint32))

    outb, idxb = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    mirror_b, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, bias=w.bias)
    np.testing.assert_array_equal(outb.cpu().numpy().view(np.uint32), mirror_b.view(np.uint32))
    assert torch.equal(idx, idxb)

    g = np.random.default_rng(sum(shape) + 1).standard_normal((n, f, d)).astype(np.float32)
    gx, gw, gb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    torch.cuda.synchronize()
    _check_backward(w, g, gx, gw, gb, c_oracle)
    # the reference operator's backward (dx, dW) and each gradient alone agree
    gx2, gw2 = ops.backward(_t(g), x, e, iw, nb, wt, idx, True, True)
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2)
    gx3, _, _ = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, False, False)
    _, gw3, gb3 = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, False, True, True)
    assert torch.equal(gx, gx3) and torch.equal(gw, gw3) and torch.equal(gb, gb3)


@pytest.mark.parametrize("quant", ["bf16", "f16"])
def test_wide_tables_16bit(quant, c_oracle):
    """16-bit outputs and gradients through the wide forward and the fallback
    backward: forward bits against the C mirror, backward at the fp32 bar of
    the quantisation-aware float64 oracle."""
    n, f, bmax, d = 1200, 3, 900, 24
    w = wide_case(n, f, bmax, d, seed=5)
    print(f"wide tables {w.name} {quant}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, idx = ops.forward(x, e, iw, nb, wt, QT[quant])
    assert out.dtype == QT[quant]
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant=quant)
    np.testing.assert_array_equal(out.float().cpu().numpy().view(np.uint32), mirror.view(np.uint32))
    g_h = torch.from_numpy(np.random.default_rng(6).standard_normal((n, f, d), dtype=np.float32)).to(QT[quant])
    gx, gw = ops.backward(g_h.to(DEV), x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    _check_backward(w, g_h.float().numpy(), gx, gw, None, c_oracle, quant=quant)


@pytest.mark.parametrize("version,relu", [("A", False), ("A", True), ("B", False), ("B", True)])
def test_wide_tables_module_epilogues(version, relu, c_oracle):
    """The fused module tails on a wide table: version A outputs and ReLU bits
    exact, version B within two fp32 roundings; gradients at the fp32 bar of
    the float64 module oracle."""
    n, f, bmax, d = 1000, 3, 1500, 40
    w = wide_case(n, f, bmax, d, seed=9)
    rng = np.random.default_rng(10)
    w0 = rng.uniform(-0.3, 0.3, (f, d)).astype(np.float32)
    b0 = rng.uniform(-0.3, 0.3, (f, d)).astype(np.float32)
    g = rng.standard_normal((n, f, d)).astype(np.float32)
    print(f"wide tables {w.name} version={version} relu={relu}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    bias = bt if version == "A" else None
    lw, lb = (_t(w0), _t(b0)) if version == "B" else (None, None)
    out, idx, mask = ops.forward_epilogue(x, e, iw, nb, wt, bias, lw, lb, relu, True, torch.float32)
    torch.cuda.synchronize()
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight)
    got = out.cpu().numpy()
    if version == "A":
        v = (mirror + w.bias[None]).astype(np.float32)
        passm = po.relu_pass(v)
        exp = np.where(passm, v, np.float32(0.0)) if relu else v
        np.testing.assert_array_equal(got.view(np.uint32), exp.astype(np.float32).view(np.uint32))
    else:
        passm = po.relu_pass(mirror)
        a = np.where(passm, mirror, np.float32(0.0)) if relu else mirror
        lin = b0[None].astype(np.float64) + w0[None].astype(np.float64) * w.x.astype(np.float64)[..., None]
        _report("out vs fp64", *close_scaled(got, lin + a, np.abs(lin) + np.abs(a), 2.0 ** -22, 0.0))
    if relu:
        np.testing.assert_array_equal(mask.cpu().numpy(), po.pack_pass_bits(passm))
    a_ = version == "A"
    grads = ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, mask, lw, relu, torch.float32,
                                  True, True, a_, not a_, not a_)
    torch.cuda.synchronize()
    ref = po.module_backward(g, w.x, (w.edges, w.inv_widths, w.n_bins), w.weight,
                             po.bin_indices(w.x, w.edges, w.n_bins), pass_mask=passm if relu else None,
                             has_bias=a_, linear0=(w0, b0) if not a_ else None)
    pairs = [("dx", grads[0], "dx"), ("dW", grads[1], "dw")]
    pairs += [("db", grads[2], "db")] if a_ else [("d lin_w", grads[3], "dlw"), ("d lin_b", grads[4], "dlb")]
    for name, got_t, key in pairs:
        _report(name, *close_scaled(got_t.cpu().numpy(), ref[key], ref[key + "_abs"], FP32_RTOL, FP32_ATOL))


@pytest.mark.parametrize("cfg,n", [(0, None), (1, 4096), (2, 2048), (4, 1024)])
def test_forced_wide_forward_matches_table_kernel(cfg, n, tune):
    """The wide-table kernel on shapes the table kernel takes (FWD_WIDE knob):
    the same indices and output bits, plain and with each fused tail."""
    w = workloads.make(cfg, n)
    print(f"forced wide forward {w.name} shape={w.shape}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    q = QT[w.quant]
    f, d = w.shape[1], w.shape[3]
    rng = np.random.default_rng(cfg)
    lw = _t(rng.uniform(-0.3, 0.3, (f, d)).astype(np.float32))
    lb = _t(rng.uniform(-0.3, 0.3, (f, d)).astype(np.float32))

    def run():
        res = [ops.forward(x, e, iw, nb, wt, q)]
        for bias, l0, relu in ((bt, None, False), (bt, None, True), (None, lw, False), (None, lw, True)):
            res.append(ops.forward_epilogue(x, e, iw, nb, wt, bias, l0, lb if l0 is not None else None, relu,
                                            True, q))
        torch.cuda.synchronize()
        return res

    base = run()
    tune("FWD_WIDE", 1)
    wide = run()
    for r0, r1 in zip(base, wide):
        for a, b in zip(r0, r1):
            assert a.dtype == b.dtype and a.shape == b.shape
            if a.is_floating_point():
                assert torch.equal(a.view(torch.int16) if a.element_size() == 2 else a.view(torch.int32),
                                   b.view(torch.int16) if b.element_size() == 2 else b.view(torch.int32))
            else:
                assert torch.equal(a, b)


@pytest.mark.parametrize("cfg,n", [(0, None), (1, 4096), (2, 2048), (3, 8192)])
def test_global_cell_histogram_matches_lds_cells(cfg, n, tune, c_oracle):
    """The fallback histogram with its cells in global memory (tables beyond
    LDS) and in LDS: the same fixed order per cell, so the same bits; both at
    the fp32 bar of the oracle."""
    w = workloads.make(cfg, n)
    nn, f, bmax, d = w.shape
    print(f"global-cell histogram {w.name} shape={w.shape}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    _, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    g = np.random.default_rng(40 + cfg).standard_normal((nn, f, d)).astype(np.float32)
    tune("BWD_SIMPLE", 1)
    lds = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    tune("BWD_SIMPLE_GLOBAL", 1)
    glob = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    torch.cuda.synchronize()
    for a, b in zip(lds, glob):
        assert torch.equal(a, b)
    _check_backward(w, g, *glob, c_oracle)


# (N, F, max bins, d): several sub-tiles and chunks a window; int16 and int32
# bin indices; 10% of x exactly on an edge, so rows on a window's first edge
# take the bin below from the row staged under the window
BIN_WINDOWS = [(20000, 5, 1024, 32), (9000, 2, 40000, 4), (12000, 3, 700, 62), (6000, 4, 48, 256)]


@pytest.mark.parametrize("shape", BIN_WINDOWS, ids=[f"{n}x{f}x{b}x{d}" for n, f, b, d in BIN_WINDOWS])
def test_bin_windows_backward(shape, tune, c_oracle):
    """Tables beyond LDS: the sorted path in windows of bins.  dx, dW, db at
    the fp32 bar of the float64 oracle, bitwise equal on a repeat, and within
    the same bar of the fallback kernels (another summation order)."""
    from piecewiselinearembeddings_optimized_amd import capi

    n, f, bmax, d = shape
    w = wide_case(n, f, bmax, d, seed=7 + bmax)
    pl = capi.backward_plan(n, f, bmax, d)
    print(f"bin windows {w.name} plan windows={pl['windows']} bins_per_window={pl['bins_per_window']} "
          f"chunks={pl['chunks']}", flush=True)
    assert pl["sorted"] == 1 and pl["windows"] > 1
    x, e, iw, nb, wt, _ = _inputs(w)
    _, idx = ops.forward(x, e, iw, nb, wt, torch.float32)
    g = np.random.default_rng(bmax).standard_normal((n, f, d)).astype(np.float32)
    got = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    again = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    torch.cuda.synchronize()
    for a, b in zip(got, again):
        assert torch.equal(a, b)
    _check_backward(w, g, *got, c_oracle)
    dx_only, _, _ = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, False, False)
    assert torch.equal(dx_only, got[0])
    tune("BWD_SIMPLE", 1)
    fb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    torch.cuda.synchronize()
    _check_backward(w, g, *fb, c_oracle)


def test_wide_tables_through_the_c_abi(c_oracle):
    """ple_forward_launch / ple_backward_launch take the wide shapes directly
    (no PLE_E_UNSUPPORTED), with int32 indices."""
    from piecewiselinearembeddings_optimized_amd import capi

    n, f, bmax, d = 2048, 4, 40000, 4
    w = wide_case(n, f, bmax, d, seed=77)
    x, e, iw, nb, wt, bt = _inputs(w)
    out = torch.empty((n, f, d), device=DEV)
    idx = torch.empty((n, f), device=DEV, dtype=torch.int32)
    L = capi.lib()
    s = torch.cuda.current_stream().cuda_stream
    rc = L.ple_forward_launch(x.data_ptr(), e.data_ptr(), iw.data_ptr(), nb.data_ptr(), wt.data_ptr(), None,
                              out.data_ptr(), idx.data_ptr(), n, f, bmax, d, 0, 0, s)
    assert rc == 0, capi.lib().ple_error_string(rc)
    torch.cuda.synchronize()
    mirror, midx = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight)
    np.testing.assert_array_equal(idx.cpu().numpy(), midx)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), mirror.view(np.uint32))
    g = torch.randn((n, f, d), device=DEV, generator=torch.Generator(DEV).manual_seed(1))
    ws_bytes = L.ple_backward_workspace_bytes(n, f, bmax, d)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    gx = torch.empty((n, f), device=DEV)
    gw = torch.empty((f, bmax, d), device=DEV)
    rc = L.ple_backward_launch(g.data_ptr(), x.data_ptr(), e.data_ptr(), iw.data_ptr(), nb.data_ptr(),
                               wt.data_ptr(), idx.data_ptr(), gx.data_ptr(), gw.data_ptr(), None, n, f, bmax, d,
                               0, 0, ws.data_ptr(), ws_bytes, s)
    assert rc == 0, capi.lib().ple_error_string(rc)
    torch.cuda.synchronize()
    _check_backward(w, g.cpu().numpy(), gx, gw, None, c_oracle)


@pytest.mark.parametrize("bmax", [8192, 40000])
def test_sampled_edge_search_special_values(bmax, c_oracle):
    """Edges beyond LDS: the wide kernel keeps every ES-th edge in LDS and
    finishes the bin search in global memory.  Every edge exactly (the sampled
    ones included), its float neighbours, midpoints, far outside both ends,
    +-inf and NaN: bin indices against searchsorted, outputs bit-exact against
    the C mirror, for the full feature and a ragged one (fewer real bins)."""
    rng = np.random.default_rng(bmax)
    f, d = 2, 4
    bins = [np.cumsum(rng.uniform(0.01, 1.0, bmax + 1)).astype(np.float32) - bmax * 0.25,
            np.cumsum(rng.uniform(0.01, 1.0, bmax // 3 + 1)).astype(np.float32)]
    edges, iw, nbins = workloads.pad_bins(bins)
    cols = []
    for e in bins:
        mids = ((e[:-1].astype(np.float64) + e[1:]) / 2).astype(np.float32)
        up = np.nextafter(e, np.float32(np.inf))
        dn = np.nextafter(e, np.float32(-np.inf))
        special = np.array([np.nan, np.inf, -np.inf, e[0] - 1e6, e[-1] + 1e6], np.float32)
        cols.append(np.concatenate([e, up, dn, mids, special]))
    n = max(c.size for c in cols)
    x = np.stack([np.resize(c, n) for c in cols], axis=1).astype(np.float32)
    wt = rng.uniform(-0.5, 0.5, (f, bmax, d)).astype(np.float32)
    w = workloads.Workload(f"sampled{bmax}", x, bins, edges, iw, nbins, wt, np.zeros((f, d), np.float32))
    print(f"sampled edge search {w.name} n={n}", flush=True)
    X, E, IW, NB, WT, _ = _inputs(w)
    out, idx = ops.forward(X, E, IW, NB, WT, torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), po.bin_indices(x, edges, nbins))
    mirror, _ = c_oracle.forward_f32(x, edges, iw, nbins, wt)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), mirror.view(np.uint32))


def test_module_on_wide_bins(c_oracle):
    """The module end to end on 450- to 600-bin features at d = 48: forward
    against its own CPU path (the dense upstream formulation) at the
    reference suite's tolerances; gradients, as they land in ``.grad``, at the
    fp32 bar of the float64 module oracle (hundreds of bins make the dense
    CPU path's own fp32 sums too coarse for the reference's fixed atol)."""
    import copy

    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings
    from tests.ple_cases import FORWARD_ATOL, FORWARD_RTOL

    torch.manual_seed(0)
    bins = [torch.sort(torch.randn(601) * 2).values, torch.sort(torch.rand(450) * 10).values,
            torch.linspace(-1, 1, 600)]
    for version, act in (("A", True), ("B", False)):
        cpu = CudaPiecewiseLinearEmbeddings(bins, 48, activation=act, version=version)
        gpu = copy.deepcopy(cpu).to(DEV)
        x = torch.randn(256, 3) * 2
        xg = x.to(DEV).requires_grad_(True)
        with torch.no_grad():
            oc = cpu(x)
        og = gpu(xg)
        torch.testing.assert_close(og.detach().cpu(), oc, rtol=FORWARD_RTOL, atol=FORWARD_ATOL)
        gr = torch.randn_like(oc)
        og.backward(gr.to(DEV))
        torch.cuda.synchronize()
        tables = tuple(t.cpu().numpy() for t in (gpu._cuda_bin_edges, gpu._cuda_inv_bin_widths, gpu._cuda_n_bins))
        wt = gpu.linear.weight.detach().cpu().numpy()
        xn = x.numpy()
        out = og.detach().cpu().numpy()
        passm = (out > 0) | np.isnan(out) if act else None     # ReLU passed where its output is not 0
        lin0 = None
        if version == "B":
            lin0 = (gpu.linear0.weight.detach().cpu().numpy(), gpu.linear0.bias.detach().cpu().numpy())
        ref = po.module_backward(gr.numpy(), xn, tables, wt, po.bin_indices(xn, tables[0], tables[2]),
                                 pass_mask=passm, has_bias=version == "A", linear0=lin0)
        pairs = [("dx", xg.grad, "dx"), ("dW", gpu.linear.weight.grad, "dw")]
        if version == "A":
            pairs.append(("db", gpu.linear.bias.grad, "db"))
        else:
            pairs += [("d lin_w", gpu.linear0.weight.grad, "dlw"), ("d lin_b", gpu.linear0.bias.grad, "dlb")]
        for name, got, key in pairs:
            _report(f"{version} {name}", *close_scaled(got.cpu().numpy(), ref[key], ref[key + "_abs"], FP32_RTOL,
                                                       FP32_ATOL))


@pytest.mark.parametrize("version", ["A", "B"])
def test_module_empty_batch_with_relu(version):
    """An empty batch through the module with ReLU: zero parameter gradients
    and an empty dx (the reference's result), not an error."""
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings

    bins = [torch.linspace(-1, 1, 9), torch.linspace(0, 3, 5)]
    m = CudaPiecewiseLinearEmbeddings(bins, 8, activation=True, version=version).to(DEV)
    x = torch.randn(4, 2, device=DEV)[:0].requires_grad_(True)
    out = m(x)
    assert out.shape == (0, 2, 8)
    out.sum().backward()
    assert x.grad is not None and x.grad.shape == (0, 2)
    for p in m.parameters():
        assert p.grad is not None and torch.count_nonzero(p.grad) == 0
