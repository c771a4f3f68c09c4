"""The backward entry point that allocates nothing (ple_backward_launch_noalloc).

It runs the same kernels as ple_backward_launch with its workspace in a
static device array, so its results must equal ple_backward_launch's bit for
bit -- checked through the C ABI on two calls in a row, the second with a
smaller input (the array keeps the first call's contents), plus the fp32 bar
of the float64 oracle, and the rejection of sizes beyond the array.
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
SCRATCH_LIMIT = -9


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _run(w, g, quant_code, noalloc):
    import piecewiselinearembeddings_optimized_amd  # noqa: F401
    from piecewiselinearembeddings_optimized_amd import capi

    L = capi.lib()
    n, f, bmax, d = w.shape
    x, e, iw, nb, wt = _t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight)
    qdt = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}[quant_code]
    _, idx = torch.ops.rtdl_num_embeddings_cuda.forward(x, e, iw, nb, wt, qdt)
    gt = _t(g).to(qdt)
    gx = torch.empty((n, f), device=DEV)
    gw = torch.empty((f, bmax, d), device=DEV)
    gb = torch.empty((f, d), device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    args = (gt.data_ptr(), x.data_ptr(), e.data_ptr(), iw.data_ptr(), nb.data_ptr(), wt.data_ptr(), idx.data_ptr(),
            gx.data_ptr(), gw.data_ptr(), gb.data_ptr(), n, f, bmax, d, quant_code, quant_code)
    if noalloc:
        rc = L.ple_backward_launch_noalloc(*args, s)
    else:
        need = L.ple_backward_workspace_bytes(n, f, bmax, d)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
        rc = L.ple_backward_launch(*args, ws.data_ptr(), need, s)
    assert rc == 0, L.ple_error_string(rc)
    torch.cuda.synchronize()
    return gx, gw, gb


@pytest.mark.parametrize("quant_code", [0, 2])
def test_noalloc_backward_matches_workspace_backward(quant_code, c_oracle):
    # first call: c1's recipe at 8192 samples (about 26 MiB of workspace);
    # second: a smaller input (c0) reusing the array the first call left behind
    for cfg, n in ((1, 8192), (0, None)):
        w = workloads.make(cfg, n)
        nn, f, bmax, d = w.shape
        print(f"noalloc backward {w.name} shape={w.shape} quant={quant_code}", flush=True)
        g = np.random.default_rng(cfg + 10 * quant_code).standard_normal((nn, f, d)).astype(np.float32)
        ref = _run(w, g, quant_code, noalloc=False)
        got = _run(w, g, quant_code, noalloc=True)
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
        quant = {0: "f32", 2: "bf16"}[quant_code]
        g_seen = po.quantize(g, quant) if quant != "f32" else g
        oracle = c_oracle.backward_f64(g_seen, w.x, w.edges, w.inv_widths, w.n_bins, w.weight,
                                       po.bin_indices(w.x, w.edges, w.n_bins), quant=quant)
        for name, t, key in (("dx", got[0], "dx"), ("dW", got[1], "dw"), ("db", got[2], "db")):
            ok, worst = close_scaled(t.cpu().numpy(), oracle[key], oracle[key + "_abs"], FP32_RTOL, FP32_ATOL)
            print(f"  {name}: worst error / allowance = {worst:.3g}", flush=True)
            assert ok, name


def test_noalloc_rejects_sizes_beyond_its_scratch():
    from piecewiselinearembeddings_optimized_amd import capi

    L = capi.lib()
    # tables beyond LDS: the fallback's histogram cells live in the workspace,
    # F * B * 2 D floats = 128 MiB
    n, f, bmax, d = 1024, 64, 4096, 64
    assert L.ple_backward_workspace_bytes(n, f, bmax, d) > 64 << 20
    dummy = 256
    rc = L.ple_backward_launch_noalloc(*([dummy] * 7), dummy, dummy, dummy, n, f, bmax, d, 0, 0, None)
    assert rc == SCRATCH_LIMIT
    assert b"static scratch" in L.ple_error_string(rc)


def test_noalloc_single_chunk_plan_needs_no_scratch(c_oracle):
    """A plan of one chunk (more feature groups than resident workgroups)
    writes dW / db from the gradient kernel: no workspace at all, so the
    no-allocation entry point takes it however large the tables, with results
    equal to the workspace path bit for bit."""
    from piecewiselinearembeddings_optimized_amd import capi

    n, f, bmax, d = 1024, 8192, 48, 32
    assert capi.workspace_bytes(n, f, bmax, d) == 0
    rng = np.random.default_rng(3)
    bins = [np.sort(rng.standard_normal(bmax + 1)).astype(np.float32) for _ in range(f)]
    edges, iw, nbins = workloads.pad_bins(bins)
    x = rng.standard_normal((n, f)).astype(np.float32)
    wt = rng.uniform(-0.5, 0.5, (f, bmax, d)).astype(np.float32)
    w = workloads.Workload("single_chunk", x, bins, edges, iw, nbins, wt, np.zeros((f, d), np.float32))
    g = rng.standard_normal((n, f, d)).astype(np.float32)
    print(f"noalloc single-chunk plan shape={w.shape}", flush=True)
    ref = _run(w, g, 0, noalloc=False)
    got = _run(w, g, 0, noalloc=True)
    for a, b in zip(ref, got):
        assert torch.equal(a, b)


def test_noalloc_backward_under_graph_capture():
    """The no-allocation backward captured in a HIP graph (torch.cuda.graph)
    after one eager call (which looks up the scratch address): every replay,
    with eager work and synchronisations between them, gives the eager
    results bit for bit."""
    import piecewiselinearembeddings_optimized_amd  # noqa: F401
    from piecewiselinearembeddings_optimized_amd import capi

    L = capi.lib()
    w = workloads.make(1, 4096)
    n, f, bmax, d = w.shape
    assert 0 < L.ple_backward_workspace_bytes(n, f, bmax, d) <= 64 << 20
    x, e, iw, nb, wt = _t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight)
    _, idx = torch.ops.rtdl_num_embeddings_cuda.forward(x, e, iw, nb, wt, torch.float32)
    g = torch.randn((n, f, d), device=DEV, generator=torch.Generator(DEV).manual_seed(4))
    gx = torch.empty((n, f), device=DEV)
    gw = torch.empty((f, bmax, d), device=DEV)
    gb = torch.empty((f, d), device=DEV)
    print(f"noalloc backward under graph capture shape={w.shape}", flush=True)

    def launch(stream):
        rc = L.ple_backward_launch_noalloc(g.data_ptr(), x.data_ptr(), e.data_ptr(), iw.data_ptr(), nb.data_ptr(),
                                           wt.data_ptr(), idx.data_ptr(), gx.data_ptr(), gw.data_ptr(), gb.data_ptr(),
                                           n, f, bmax, d, 0, 0, stream)
        assert rc == 0, L.ple_error_string(rc)

    launch(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = (gx.clone(), gw.clone(), gb.clone())
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            launch(side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        for t in (gx, gw, gb):
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip((gx, gw, gb), eager):
            assert torch.equal(a, b), f"replay {rep}"
        # eager work between the replays
        launch(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
