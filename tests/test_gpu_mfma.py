"""GPU parity for the matrix-core backward (16-bit gradients in their own dtype).

A bf16 / fp16 gradient whose quantisation dtype is its own takes
``ple_bwd_mfma_kernel`` (rows of 8, 16, 24 or 32 columns, at most 96 bins, at
most 8 chunks): bucket and weighted histograms as products of one-hot
matrices with the gradient on the 32x32x16 matrix instructions, workgroups
of up to four adjacent features loading each step of samples together, dx
per sample from the pre-scaled weight rows (reference arithmetic:
``csrc/backward_cuda.cu`` dx ``:380-490``, histograms and suffix
``:170-336,889-923``, the gradient rounded through the output dtype
``:197-199,446-457``).  Checked here against the quantisation-aware float64
oracle at the fp32 bar (``|err| <= 1e-6 + 1e-5 * sum|terms|``), bitwise on a
repeat, against the sorted path on the same inputs (another summation order,
the same bar), with one chunk (dW written by the kernel) and with many (chunk
partials and the finalize kernel), feature groups cut short by F, x on
edges, ragged bins, single-bin features, batches that end inside a block and
inside a step, and the knob that forces the kernel past 8 chunks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.test_gpu_wide_tables import QT, _check_backward, _inputs, wide_case

pytestmark = pytest.mark.gpu

ops = None


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    global ops
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    ops = torch.ops.rtdl_num_embeddings_cuda
    yield


# (N, F, max bins, d): one to three 32-bin tiles, rows of 8 to 32 columns,
# groups of 2 and 4 features (and a last group cut short), batches ending
# inside a block, one chunk and up to 8
SHAPES = [
    (1000, 3, 48, 24), (4099, 2, 96, 32), (2048, 5, 33, 8), (777, 4, 1, 8), (2048, 8, 96, 24),
    (4096, 2, 64, 16), (2000, 6, 80, 16), (1500, 7, 17, 24),
]


@pytest.mark.parametrize("quant", ["bf16", "f16"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{n}x{f}x{b}x{d}" for n, f, b, d in SHAPES])
def test_mfma_backward(shape, quant, tune, c_oracle):
    from piecewiselinearembeddings_optimized_amd import capi

    n, f, bmax, d = shape
    qt = QT[quant]
    pl = capi.backward_plan(n, f, bmax, d, grad_dtype=qt)
    w = wide_case(n, f, bmax, d, seed=sum(shape) + (quant == "f16"))
    print(f"mfma backward {w.name} {quant} chunks={pl['chunks']}", flush=True)
    assert pl["matrix_cores"] == 1
    x, e, iw, nb, wt, _ = _inputs(w)
    _, idx = ops.forward(x, e, iw, nb, wt, qt)
    g_h = torch.from_numpy(np.random.default_rng(n + d).standard_normal((n, f, d), dtype=np.float32)).to(qt)
    g = g_h.to("cuda:0")
    gx, gw = ops.backward(g, x, e, iw, nb, wt, idx, True, True)
    gx2, gw2 = ops.backward(g, x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2)
    _check_backward(w, g_h.float().numpy(), gx, gw, None, c_oracle, quant=quant)
    # each gradient alone, and the fused-bias operator's db
    gx3, _ = ops.backward(g, x, e, iw, nb, wt, idx, True, False)
    _, gw3 = ops.backward(g, x, e, iw, nb, wt, idx, False, True)
    assert torch.equal(gx, gx3) and torch.equal(gw, gw3)
    bx, bw, bb = ops.backward_with_bias(g, x, e, iw, nb, wt, idx, qt, True, True, True)
    assert torch.equal(bx, gx) and torch.equal(bw, gw)
    _check_backward(w, g_h.float().numpy(), None, None, bb, c_oracle, quant=quant)
    # the sorted path on the same inputs
    tune("BWD_MFMA", 1)
    assert capi.backward_plan(n, f, bmax, d, grad_dtype=qt)["matrix_cores"] == 0
    sx, sw = ops.backward(g, x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    _check_backward(w, g_h.float().numpy(), sx, sw, None, c_oracle, quant=quant)


def test_mfma_backward_through_the_c_abi(c_oracle):
    """ple_backward_launch with a bf16 gradient of c4's row width and bin
    count, through ctypes: 32 groups of four features, 8 chunks (chunk
    partials in the caller's workspace)."""
    from piecewiselinearembeddings_optimized_amd import capi

    n, f, bmax, d = 2048, 128, 96, 24
    pl = capi.backward_plan(n, f, bmax, d, grad_dtype=torch.bfloat16)
    assert pl["matrix_cores"] == 1 and pl["chunks"] > 1 and pl["workspace_bytes"] > 0
    assert pl["features_per_group"] == 4
    w = wide_case(n, f, bmax, d, seed=5)
    x, e, iw, nb, wt, _ = _inputs(w)
    _, idx = ops.forward(x, e, iw, nb, wt, torch.bfloat16)
    g = torch.randn((n, f, d), device="cuda:0", generator=torch.Generator("cuda:0").manual_seed(2)).to(torch.bfloat16)
    L = capi.lib()
    ws = torch.empty(pl["workspace_bytes"], dtype=torch.uint8, device="cuda:0")
    gx = torch.empty((n, f), device="cuda:0")
    gw = torch.empty((f, bmax, d), device="cuda:0")
    gb = torch.empty((f, d), device="cuda:0")
    rc = L.ple_backward_launch(g.data_ptr(), x.data_ptr(), e.data_ptr(), iw.data_ptr(), nb.data_ptr(), wt.data_ptr(),
                               idx.data_ptr(), gx.data_ptr(), gw.data_ptr(), gb.data_ptr(), n, f, bmax, d, 2, 2,
                               ws.data_ptr(), pl["workspace_bytes"], torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.ple_error_string(rc)
    torch.cuda.synchronize()
    _check_backward(w, g.float().cpu().numpy(), gx, gw, gb, c_oracle, quant="bf16")


def test_mfma_backward_forced_past_eight_chunks(tune, c_oracle):
    """PLE_TUNE_BWD_MFMA = 2: the matrix-core kernel where the planner would
    take the sorted path (32 chunks of a two-feature group)."""
    from piecewiselinearembeddings_optimized_amd import capi

    n, f, bmax, d = 16384, 2, 64, 16
    assert capi.backward_plan(n, f, bmax, d, grad_dtype=torch.bfloat16)["matrix_cores"] == 0
    tune("BWD_MFMA", 2)
    pl = capi.backward_plan(n, f, bmax, d, grad_dtype=torch.bfloat16)
    assert pl["matrix_cores"] == 1 and pl["chunks"] > 8
    w = wide_case(n, f, bmax, d, seed=11)
    x, e, iw, nb, wt, _ = _inputs(w)
    _, idx = ops.forward(x, e, iw, nb, wt, torch.bfloat16)
    g_h = torch.from_numpy(np.random.default_rng(3).standard_normal((n, f, d), dtype=np.float32)).to(torch.bfloat16)
    gx, gw = ops.backward(g_h.to("cuda:0"), x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    _check_backward(w, g_h.float().numpy(), gx, gw, None, c_oracle, quant="bf16")


def test_mfma_backward_misaligned_bin_indices(c_oracle):
    """Bin indices at an odd address (a view one byte into a larger buffer,
    through the C ABI): the kernel reads the aligned word that holds each byte
    and shifts by the byte's place, so the results equal those from an
    aligned copy bit for bit (F = 5: a sample's bytes straddle words)."""
    from piecewiselinearembeddings_optimized_amd import capi

    n, f, bmax, d = 1024, 5, 48, 16
    pl = capi.backward_plan(n, f, bmax, d, grad_dtype=torch.bfloat16)
    assert pl["matrix_cores"] == 1
    w = wide_case(n, f, bmax, d, seed=21)
    x, e, iw, nb, wt, _ = _inputs(w)
    _, idx = ops.forward(x, e, iw, nb, wt, torch.bfloat16)
    raw = torch.zeros(n * f + 8, dtype=torch.uint8, device="cuda:0")
    raw[1:1 + n * f] = idx.reshape(-1)
    g = torch.randn((n, f, d), device="cuda:0", generator=torch.Generator("cuda:0").manual_seed(4)).to(torch.bfloat16)
    L = capi.lib()
    ws = torch.empty(max(pl["workspace_bytes"], 1), dtype=torch.uint8, device="cuda:0")
    outs = []
    for ptr in (idx.data_ptr(), raw.data_ptr() + 1):
        gx = torch.empty((n, f), device="cuda:0")
        gw = torch.empty((f, bmax, d), device="cuda:0")
        gb = torch.empty((f, d), device="cuda:0")
        rc = L.ple_backward_launch(g.data_ptr(), x.data_ptr(), e.data_ptr(), iw.data_ptr(), nb.data_ptr(),
                                   wt.data_ptr(), ptr, gx.data_ptr(), gw.data_ptr(), gb.data_ptr(), n, f, bmax, d,
                                   2, 2, ws.data_ptr(), pl["workspace_bytes"], torch.cuda.current_stream().cuda_stream)
        assert rc == 0, L.ple_error_string(rc)
        outs.append((gx, gw, gb))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    _check_backward(w, g.float().cpu().numpy(), outs[1][0], outs[1][1], outs[1][2], c_oracle, quant="bf16")


def _same_class(a, b):
    """Same NaN / +inf / -inf positions, and the finite values at the fp32 bar
    of their magnitude."""
    a, b = a.float().cpu(), b.float().cpu()
    assert torch.equal(torch.isnan(a), torch.isnan(b))
    assert torch.equal(torch.isposinf(a), torch.isposinf(b)) and torch.equal(torch.isneginf(a), torch.isneginf(b))
    fin = torch.isfinite(a)
    scale = b[fin].abs().max().clamp_min(1e-30) if fin.any() else torch.tensor(1.0)
    assert torch.allclose(a[fin], b[fin], rtol=1e-5, atol=1e-5 * float(scale))


@pytest.mark.parametrize("quant", ["bf16", "f16"])
def test_mfma_backward_non_finite_gradients(quant, tune):
    """inf, -inf and NaN in the gradient stay in their own bin's cells (as
    the sorted path sums them): dx, dW and db have the sorted path's NaN /
    inf pattern, and its finite values."""
    from piecewiselinearembeddings_optimized_amd import capi

    n, f, bmax, d = 2048, 8, 96, 24
    qt = QT[quant]
    assert capi.backward_plan(n, f, bmax, d, grad_dtype=qt)["matrix_cores"] == 1
    w = wide_case(n, f, bmax, d, seed=31)
    x, e, iw, nb, wt, _ = _inputs(w)
    _, idx = ops.forward(x, e, iw, nb, wt, qt)
    g = torch.randn((n, f, d), device="cuda:0", generator=torch.Generator("cuda:0").manual_seed(9)).to(qt)
    for (s, ff, c), v in (((5, 3, 7), float("inf")), ((100, 3, 2), float("-inf")), ((700, 6, 20), float("nan")),
                          ((701, 6, 20), float("inf")), ((1500, 0, 0), float("inf")), ((1501, 0, 0), float("-inf")),
                          ((2047, 7, 23), float("nan"))):
        g[s, ff, c] = v
    gx, gw = ops.backward(g, x, e, iw, nb, wt, idx, True, True)
    _, _, gb = ops.backward_with_bias(g, x, e, iw, nb, wt, idx, qt, False, False, True)
    tune("BWD_MFMA", 1)
    sx, sw = ops.backward(g, x, e, iw, nb, wt, idx, True, True)
    _, _, sb = ops.backward_with_bias(g, x, e, iw, nb, wt, idx, qt, False, False, True)
    torch.cuda.synchronize()
    for got, ref in ((gx, sx), (gw, sw), (gb, sb)):
        _same_class(got, ref)
    assert not torch.isfinite(gw).all() and torch.isfinite(gw[1]).all()   # feature 1 holds no non-finite value
