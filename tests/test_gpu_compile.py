"""Operator-registration and ``torch.compile`` checks on the GPU.

The reference module promises first-order autograd and
``torch.compile(fullgraph=True)`` support (reference ``module.py:30-37``), which
rests on the operator schemas, the fake kernels (reference ``_meta.py:14-188``)
and the autograd registration (reference ``_autograd.py:92-96``).  These tests
run ``torch.library.opcheck`` (schema, fake-tensor, autograd-registration and
AOT-dispatch checks) on every operator and compile the module with
``fullgraph=True, dynamic=True``, comparing against eager execution.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from piecewiselinearembeddings_optimized_amd import workloads
from tests.ple_cases import init_parameters_, make_bins, sample_features

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ops = None


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    global ops
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    ops = torch.ops.rtdl_num_embeddings_cuda
    yield


def _inputs(n=96):
    w = workloads.make(0, n)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    return w, t(w.x), t(w.edges), t(w.inv_widths), t(w.n_bins), t(w.weight), t(w.bias)


OUT_DTYPES = pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16, torch.float16],
                                     ids=["f32", "bf16", "f16"])


@OUT_DTYPES
def test_opcheck_forward(out_dtype):
    w, x, e, iw, nb, wt, bt = _inputs()
    x.requires_grad_(True)
    wt.requires_grad_(True)
    torch.library.opcheck(ops.forward.default, (x, e, iw, nb, wt, out_dtype))


@OUT_DTYPES
def test_opcheck_forward_with_bias(out_dtype):
    w, x, e, iw, nb, wt, bt = _inputs()
    x.requires_grad_(True)
    wt.requires_grad_(True)
    bt.requires_grad_(True)
    torch.library.opcheck(ops.forward_with_bias.default, (x, e, iw, nb, wt, bt, out_dtype))


@OUT_DTYPES
def test_opcheck_backward(out_dtype):
    w, x, e, iw, nb, wt, bt = _inputs()
    _, idx = ops.forward(x, e, iw, nb, wt, out_dtype)
    n, f, _, d = w.shape
    g = torch.randn((n, f, d), device=DEV, generator=torch.Generator(DEV).manual_seed(5)).to(out_dtype)
    for want_x, want_w in ((True, True), (True, False), (False, True)):
        torch.library.opcheck(ops.backward.default, (g, x, e, iw, nb, wt, idx, want_x, want_w))


@OUT_DTYPES
def test_opcheck_backward_with_bias(out_dtype):
    w, x, e, iw, nb, wt, bt = _inputs()
    _, idx = ops.forward(x, e, iw, nb, wt, out_dtype)
    n, f, _, d = w.shape
    g = torch.randn((n, f, d), device=DEV, generator=torch.Generator(DEV).manual_seed(6))
    torch.library.opcheck(ops.backward_with_bias.default, (g, x, e, iw, nb, wt, idx, out_dtype, True, True, True))


@pytest.mark.parametrize("version,activation", [("A", False), ("A", True), ("B", False), ("B", True)])
def test_compile_fullgraph_dynamic_matches_eager(version, activation):
    """fullgraph + dynamic shapes through AOTAutograd (fake kernels and the
    autograd formula traced), two batch sizes, forward and backward."""
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings

    torch._dynamo.reset()
    bins = make_bins("ragged")
    eager = CudaPiecewiseLinearEmbeddings(bins, 16, activation=activation, version=version)
    init_parameters_(eager, seed=3)
    eager = eager.to(DEV)
    comp_mod = copy.deepcopy(eager)
    compiled = torch.compile(comp_mod, fullgraph=True, dynamic=True, backend="aot_eager")
    for batch, seed in ((64, 11), (96, 12)):
        x = sample_features(bins, batch_size=batch, seed=seed).to(DEV)
        xe = x.clone().requires_grad_(True)
        xc = x.clone().requires_grad_(True)
        oe = eager(xe)
        oc = compiled(xc)
        assert oc.shape == oe.shape and oc.dtype == oe.dtype
        torch.testing.assert_close(oc, oe, rtol=1e-6, atol=1e-6)
        g = torch.randn_like(oe)
        oe.backward(g)
        oc.backward(g)
        torch.testing.assert_close(xc.grad, xe.grad, rtol=1e-6, atol=1e-6)
        for (name, pe), (_, pc) in zip(eager.named_parameters(), comp_mod.named_parameters()):
            torch.testing.assert_close(pc.grad, pe.grad, rtol=1e-6, atol=1e-6, msg=name)
            pe.grad = None
            pc.grad = None


def test_compile_inductor_under_autocast():
    """Inductor (generated kernels around the custom ops) under bf16 autocast:
    the output dtype and values follow eager."""
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings

    torch._dynamo.reset()
    bins = make_bins("equal")
    eager = CudaPiecewiseLinearEmbeddings(bins, 8, activation=True, version="B")
    init_parameters_(eager, seed=4)
    eager = eager.to(DEV)
    compiled = torch.compile(copy.deepcopy(eager), fullgraph=True)
    x = sample_features(bins, batch_size=64, seed=21).to(DEV)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        oe = eager(x)
        oc = compiled(x)
    assert oc.dtype == oe.dtype
    torch.testing.assert_close(oc.float(), oe.float(), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("version,relu", [("A", False), ("A", True), ("B", False), ("B", True)])
def test_opcheck_forward_epilogue(version, relu):
    w, x, e, iw, nb, wt, bt = _inputs()
    f, d = wt.shape[0], wt.shape[2]
    x.requires_grad_(True)
    wt.requires_grad_(True)
    if version == "A":
        bias, lw, lb = bt.requires_grad_(True), None, None
    else:
        gen = torch.Generator(DEV).manual_seed(3)
        bias = None
        lw = torch.randn((f, d), device=DEV, generator=gen).requires_grad_(True)
        lb = torch.randn((f, d), device=DEV, generator=gen).requires_grad_(True)
    torch.library.opcheck(ops.forward_epilogue.default, (x, e, iw, nb, wt, bias, lw, lb, relu, True, torch.bfloat16))


@pytest.mark.parametrize("version,relu", [("A", True), ("B", True)])
def test_opcheck_backward_epilogue(version, relu):
    w, x, e, iw, nb, wt, bt = _inputs()
    n, f, _, d = w.shape
    gen = torch.Generator(DEV).manual_seed(4)
    lw = torch.randn((f, d), device=DEV, generator=gen) if version == "B" else None
    lb = torch.randn((f, d), device=DEV, generator=gen) if version == "B" else None
    _, idx, mask = ops.forward_epilogue(x, e, iw, nb, wt, bt if version == "A" else None, lw, lb, relu, True,
                                        torch.float32)
    g = torch.randn((n, f, d), device=DEV, generator=gen)
    a = version == "A"
    torch.library.opcheck(ops.backward_epilogue.default,
                          (g, x, e, iw, nb, wt, idx, mask, lw, relu, torch.float32, True, True, a, not a, not a))
