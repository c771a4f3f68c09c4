"""GPU parity for embedding rows wider than 64 columns.

The reference operators take any d_embedding (``csrc/forward_cuda.cu:764-766``
checks only D > 0; the forward tiles D in 16/32 columns, ``:447-455``; the dx
kernel loops over any D, ``csrc/backward_cuda.cu:437-441``); only the
reference module asserts d <= 64 (``src/rtdl_num_embeddings_cuda/module.py:47-49``).
Here rows of more than 64 lanes' columns are cut into column chunks in the
forward, the backward's sorted path takes 32- and 64-lane groups, and wider
rows (or tables beyond its LDS) the fallback kernels, whose histogram runs in
blocks of 64 columns.

Forward: bin indices exact, outputs bit-exact against the C mirror of the
reference arithmetic (``oracle/ple_oracle.c``).  Backward: dx, dW, db within
the fp32 bar (``|err| <= 1e-6 + 1e-5 * sum|terms|``) of the float64 oracle, and
the fallback kernels agree with the sorted path to the same bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.test_gpu_wide_tables import IDX_DTYPE, QT, _check_backward, _inputs, _t, wide_case

pytestmark = pytest.mark.gpu

ops = None


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    global ops
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    ops = torch.ops.rtdl_num_embeddings_cuda
    yield


# (N, F, max bins, d): the widths named for this path (48 bins), then a row of
# several column chunks, and a wide table whose rows are chunked too
WIDE_ROWS = [
    (2048, 4, 48, 65), (2048, 4, 48, 96), (2048, 4, 48, 128), (2048, 4, 48, 256),
    (1024, 3, 40, 1000), (1024, 2, 700, 260),
]


@pytest.mark.parametrize("shape", WIDE_ROWS, ids=[f"{n}x{f}x{b}x{d}" for n, f, b, d in WIDE_ROWS])
def test_wide_rows_forward_and_backward(shape, c_oracle):
    n, f, bmax, d = shape
    w = wide_case(n, f, bmax, d, seed=sum(shape))
    print(f"wide rows {w.name}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, idx = ops.forward(x, e, iw, nb, wt, torch.float32)
    torch.cuda.synchronize()
    mirror, midx = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), midx.astype(np.int64))
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), mirror.view(np.uint32))
    outb, _ = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    mirror_b, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, bias=w.bias)
    np.testing.assert_array_equal(outb.cpu().numpy().view(np.uint32), mirror_b.view(np.uint32))

    g = np.random.default_rng(sum(shape) + 1).standard_normal((n, f, d)).astype(np.float32)
    gx, gw, gb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    torch.cuda.synchronize()
    _check_backward(w, g, gx, gw, gb, c_oracle)
    gx2, gw2 = ops.backward(_t(g), x, e, iw, nb, wt, idx, True, True)
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2)
    gx3, _, _ = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, False, False)
    _, gw3, gb3 = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, False, True, True)
    assert torch.equal(gx, gx3) and torch.equal(gw, gw3) and torch.equal(gb, gb3)


@pytest.mark.parametrize("quant,d", [("bf16", 96), ("f16", 128), ("bf16", 512)])
def test_wide_rows_16bit(quant, d, c_oracle):
    """16-bit outputs (eight a lane) and gradients: forward bits against the C
    mirror, backward at the fp32 bar of the quantisation-aware oracle."""
    n, f, bmax = 1024, 3, 48
    w = wide_case(n, f, bmax, d, seed=d)
    print(f"wide rows {w.name} {quant}", flush=True)
    x, e, iw, nb, wt, _ = _inputs(w)
    out, idx = ops.forward(x, e, iw, nb, wt, QT[quant])
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant=quant)
    np.testing.assert_array_equal(out.float().cpu().numpy().view(np.uint32), mirror.view(np.uint32))
    g_h = torch.from_numpy(np.random.default_rng(d + 1).standard_normal((n, f, d), dtype=np.float32)).to(QT[quant])
    gx, gw = ops.backward(g_h.to("cuda:0"), x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    _check_backward(w, g_h.float().numpy(), gx, gw, None, c_oracle, quant=quant)


@pytest.mark.parametrize("d", [96, 200])
def test_wide_rows_fallback_kernels(d, c_oracle):
    """The fallback backward (histogram in blocks of 64 columns, cells in LDS
    or in global memory) against the oracle and the sorted path."""
    from piecewiselinearembeddings_optimized_amd import capi

    n, f, bmax = 1536, 3, 48
    w = wide_case(n, f, bmax, d, seed=3 * d)
    print(f"wide rows fallback {w.name}", flush=True)
    x, e, iw, nb, wt, _ = _inputs(w)
    _, idx = ops.forward(x, e, iw, nb, wt, torch.float32)
    g = np.random.default_rng(d).standard_normal((n, f, d)).astype(np.float32)
    gx, gw, gb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    for glob in (0, 1):
        capi.set_tuning("BWD_SIMPLE", 1)
        capi.set_tuning("BWD_SIMPLE_GLOBAL", glob)
        try:
            fx, fw, fb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
            torch.cuda.synchronize()
        finally:
            capi.set_tuning("BWD_SIMPLE", 0)
            capi.set_tuning("BWD_SIMPLE_GLOBAL", 0)
        _check_backward(w, g, fx, fw, fb, c_oracle)
    torch.cuda.synchronize()
    _check_backward(w, g, gx, gw, gb, c_oracle)


def test_wide_rows_module_epilogues_rejected():
    """The fused module tails with ReLU or linear0 keep the module's d <= 64:
    wider rows are refused before any launch (the module never asks)."""
    n, f, bmax, d = 256, 2, 16, 80
    w = wide_case(n, f, bmax, d, seed=1)
    x, e, iw, nb, wt, bt = _inputs(w)
    with pytest.raises(RuntimeError):
        ops.forward_epilogue(x, e, iw, nb, wt, bt, None, None, True, True, torch.float32)
    lw = torch.zeros((f, d), device="cuda:0")
    with pytest.raises(RuntimeError):
        ops.forward_epilogue(x, e, iw, nb, wt, None, lw, lw, False, False, torch.float32)
    out, idx = ops.forward(x, e, iw, nb, wt, torch.float32)
    assert out.shape == (n, f, d) and idx.dtype == IDX_DTYPE[1]
