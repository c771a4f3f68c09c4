"""GPU parity through the C ABI (``include/ple_hip.h``) called with ctypes.

The same kernels the torch operators reach, driven here through the plain
pointer interface a non-torch caller binds: forward bit-exact against the C
mirror of the reference arithmetic with bin indices exact, backward within
the fp32 bar against the float64 oracle, and bitwise equal to the operator
path on the same inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ple_oracle as po
from piecewiselinearembeddings_optimized_amd import workloads
from tests.ple_cases import BF16_RTOL, FP32_ATOL, FP32_RTOL, close_scaled

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
REDUCED = {0: None, 1: 4096, 2: 2048, 3: 16384, 4: 1024}
IDX_DTYPE = {1: torch.uint8, 2: torch.int16, 4: torch.int32}
QUANT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


@pytest.fixture(scope="module")
def capi():
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd as pkg  # noqa: F401  (registers the ops)
    from piecewiselinearembeddings_optimized_amd import capi as c

    assert c.lib().ple_abi_version() >> 16 == 1
    return c


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _report(name, ok, worst):
    print(f"  {name}: worst error / allowance = {worst:.3g}", flush=True)
    assert ok, f"{name} outside tolerance (worst ratio {worst:.3g})"


@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4])
def test_c_abi_forward_matches_oracle(cfg, capi, c_oracle):
    w = workloads.make(cfg, REDUCED[cfg])
    n, f, bmax, d = w.shape
    print(f"C ABI forward {w.name} shape={w.shape} quant={w.quant}", flush=True)
    x, e, iw, nb, wt = _t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight)
    qd = QUANT[w.quant]
    out = torch.empty((n, f, d), dtype=qd, device=DEV)
    idx = torch.empty((n, f), dtype=IDX_DTYPE[capi.lib().ple_bin_index_bytes(bmax)], device=DEV)
    capi.forward(x, e, iw, nb, wt, None, out, idx, qd)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), po.bin_indices(w.x, w.edges, w.n_bins))
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant=w.quant)
    got = out.float().cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), mirror.view(np.uint32))
    ref, _, s = po.forward(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant=w.quant, return_abs=True)
    rtol, atol = (FP32_RTOL, FP32_ATOL) if w.quant == "f32" else (BF16_RTOL, 0.0)
    _report("out vs fp64", *close_scaled(got, ref, s, rtol, atol))


@pytest.mark.parametrize("cfg", [0, 1, 2, 3])
def test_c_abi_forward_bias_and_backward_match_oracle_and_operator(cfg, capi, c_oracle):
    w = workloads.make(cfg, REDUCED[cfg])
    n, f, bmax, d = w.shape
    print(f"C ABI forward+bias / backward {w.name} shape={w.shape}", flush=True)
    x, e, iw, nb, wt, bt = (_t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight), _t(w.bias))
    out = torch.empty((n, f, d), dtype=torch.float32, device=DEV)
    idx = torch.empty((n, f), dtype=IDX_DTYPE[capi.lib().ple_bin_index_bytes(bmax)], device=DEV)
    capi.forward(x, e, iw, nb, wt, bt, out, idx, torch.float32)
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, bias=w.bias)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), mirror.view(np.uint32))

    g = np.random.default_rng(300 + cfg).standard_normal((n, f, d), dtype=np.float32)
    gd = _t(g)
    gx = torch.empty((n, f), dtype=torch.float32, device=DEV)
    gw = torch.empty((f, bmax, d), dtype=torch.float32, device=DEV)
    gb = torch.empty((f, d), dtype=torch.float32, device=DEV)
    capi.backward(gd, x, e, iw, nb, wt, idx, gx, gw, gb, torch.float32)
    torch.cuda.synchronize()
    ref = c_oracle.backward_f64(g, w.x, w.edges, w.inv_widths, w.n_bins, w.weight,
                                po.bin_indices(w.x, w.edges, w.n_bins), quant="f32")
    _report("dx", *close_scaled(gx.cpu().numpy(), ref["dx"], ref["dx_abs"], FP32_RTOL, FP32_ATOL))
    _report("dW", *close_scaled(gw.cpu().numpy(), ref["dw"], ref["dw_abs"], FP32_RTOL, FP32_ATOL))
    _report("db", *close_scaled(gb.cpu().numpy(), ref["db"], ref["db_abs"], FP32_RTOL, FP32_ATOL))

    # the operator path runs the same kernels: bitwise equal results
    ops = torch.ops.rtdl_num_embeddings_cuda
    ox, ow, ob = ops.backward_with_bias(gd, x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    for a, b in ((gx, ox), (gw, ow), (gb, ob)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_c_abi_partial_gradients(capi, c_oracle):
    """Each gradient pointer may be NULL; the others are unchanged."""
    w = workloads.make(2, 1024)
    n, f, bmax, d = w.shape
    x, e, iw, nb, wt = _t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight)
    out = torch.empty((n, f, d), dtype=torch.float32, device=DEV)
    idx = torch.empty((n, f), dtype=torch.uint8, device=DEV)
    capi.forward(x, e, iw, nb, wt, None, out, idx, torch.float32)
    g = _t(np.random.default_rng(5).standard_normal((n, f, d), dtype=np.float32))
    full = [torch.empty((n, f), device=DEV), torch.empty((f, bmax, d), device=DEV), torch.empty((f, d), device=DEV)]
    capi.backward(g, x, e, iw, nb, wt, idx, *full, torch.float32)
    for keep in range(3):
        part = [None, None, None]
        part[keep] = torch.full_like(full[keep], float("nan"))
        capi.backward(g, x, e, iw, nb, wt, idx, *part, torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(part[keep].view(torch.int32), full[keep].view(torch.int32))


def test_c_abi_rejects_before_launch_on_device(capi):
    """Argument errors come back as codes with nothing launched."""
    w = workloads.make(0)
    n, f, bmax, d = w.shape
    x, e, iw, nb, wt, bt = (_t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight), _t(w.bias))
    idx = torch.empty((n, f), dtype=torch.uint8, device=DEV)
    out16 = torch.empty((n, f, d), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(capi.PleError) as ei:      # bias with a bf16 output: unsupported pairing
        capi.forward(x, e, iw, nb, wt, bt, out16, idx, torch.bfloat16)
    assert ei.value.code == -7
    out32 = torch.empty((n, f, d), dtype=torch.float32, device=DEV)
    capi.forward(x, e, iw, nb, wt, None, out32, idx, torch.float32)
    g = torch.randn((n, f, d), device=DEV)
    gw = torch.empty((f, bmax, d), device=DEV)
    small = torch.empty(16, dtype=torch.uint8, device=DEV)
    # (one chunk here: dW from the gradient kernel, no workspace needed)
    assert capi.workspace_bytes(n, f, bmax, d) == 0
    capi.backward(g, x, e, iw, nb, wt, idx, None, gw, None, torch.float32, workspace=small)
    # several chunks: partials in the workspace
    w2 = workloads.make(0, 4096)
    n2 = w2.shape[0]
    x2 = _t(w2.x)
    idx2 = torch.empty((n2, f), dtype=torch.uint8, device=DEV)
    capi.forward(x2, e, iw, nb, wt, None, torch.empty((n2, f, d), device=DEV), idx2, torch.float32)
    assert capi.workspace_bytes(n2, f, bmax, d) > 16
    with pytest.raises(capi.PleError) as ei:      # workspace too small
        capi.backward(torch.randn((n2, f, d), device=DEV), x2, e, iw, nb, wt, idx2, None, gw, None, torch.float32,
                      workspace=small)
    assert ei.value.code == -6
    with pytest.raises(capi.PleError) as ei:      # bf16 gradient with fp32 quantisation
        capi.backward(g.to(torch.bfloat16), x, e, iw, nb, wt, idx, None, gw, None, torch.float32)
    assert ei.value.code == -7
    torch.cuda.synchronize()


def test_kernel_timing_counts_launches(capi):
    """ple_timing_*: each forward and backward launch within the slots records
    one event pair around its main kernel (sorted path and fallback path);
    launches past the slots and after ple_timing_stop record nothing, and the
    results are unchanged by the timing."""
    w = workloads.make(1, 2048)
    n, f, bmax, d = w.shape
    x, e, iw, nb, wt = _t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight)
    out = torch.empty((n, f, d), device=DEV)
    idx = torch.empty((n, f), dtype=torch.uint8, device=DEV)
    g = torch.randn((n, f, d), device=DEV, generator=torch.Generator(DEV).manual_seed(3))
    grads = [torch.empty((n, f), device=DEV), torch.empty_like(wt), torch.empty((f, d), device=DEV)]
    capi.forward(x, e, iw, nb, wt, None, out, idx, torch.float32)
    capi.backward(g, x, e, iw, nb, wt, idx, *grads, torch.float32)
    torch.cuda.synchronize()
    ref = [t.clone() for t in grads]
    try:
        capi.timing_start(2)
        for _ in range(3):      # the third launch of each finds no slot left
            capi.forward(x, e, iw, nb, wt, None, out, idx, torch.float32)
            capi.backward(g, x, e, iw, nb, wt, idx, *grads, torch.float32)
        capi.set_tuning("BWD_SIMPLE", 1)     # the fallback kernels are timed as one span
        capi.timing_start(1)
        capi.backward(g, x, e, iw, nb, wt, idx, *grads, torch.float32)
        torch.cuda.synchronize()
        ms_b, cnt_b = capi.timing_read(capi.TIMER_BACKWARD)
        assert cnt_b == 1 and ms_b > 0.0
        capi.set_tuning("BWD_SIMPLE", 0)
        capi.timing_start(2)
        capi.forward(x, e, iw, nb, wt, None, out, idx, torch.float32)
        capi.backward(g, x, e, iw, nb, wt, idx, *grads, torch.float32)
        capi.timing_stop()
        capi.forward(x, e, iw, nb, wt, None, out, idx, torch.float32)
        torch.cuda.synchronize()
        for which in (capi.TIMER_FORWARD, capi.TIMER_BACKWARD):
            ms, cnt = capi.timing_read(which)
            print(f"  timer {which}: {cnt} launches, {ms:.4f} ms", flush=True)
            assert cnt == 1 and 0.0 < ms < 100.0
    finally:
        capi.set_tuning("BWD_SIMPLE", 0)
        capi.timing_start(0)
    for got, want in zip(grads, ref):
        assert torch.equal(got, want)
