"""GPU parity of the fused module tail (``forward_epilogue`` / ``backward_epilogue``).

The reference module runs its tail -- version A's ``x_ple + bias`` and ReLU,
version B's ReLU and ``linear0(x)`` residual (reference ``module.py:230-248``)
-- as separate PyTorch ops; here it is fused into the kernels.

Forward: bin indices exact; version A outputs and every ReLU pass bit exact
against the C mirror of the reference arithmetic followed by the same fp32
operations in NumPy; version B outputs within two fp32 roundings of the
float64 value (the residual is one fma, then one add).  Backward: dx, dW, the
bias gradient and linear0's gradients within the fp32 bar
(``|err| <= 1e-6 + 1e-5 * sum|terms|``) of the float64 oracle
(``oracle.ple_oracle.module_backward``), which is pinned against torch
autograd of the dense module in ``tests/test_oracle.py``.
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
QT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
REDUCED = {0: None, 1: 2048, 2: 2048, 3: 8192}
KINDS = [("A", False), ("A", True), ("B", False), ("B", True)]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    global ops
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    ops = torch.ops.rtdl_num_embeddings_cuda
    yield


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _setup(cfg, seed=0):
    w = workloads.make(cfg, REDUCED[cfg])
    n, f, bmax, d = w.shape
    rng = np.random.default_rng(100 + seed)
    w0 = rng.uniform(-0.3, 0.3, size=(f, d)).astype(np.float32)
    b0 = rng.uniform(-0.3, 0.3, size=(f, d)).astype(np.float32)
    g = rng.standard_normal((n, f, d)).astype(np.float32)
    return w, w0, b0, g


def _run_forward(w, w0, b0, version, relu, quant, save_mask=True):
    x, e, iw, nb, wt = _t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight)
    bias = _t(w.bias) if version == "A" else None
    lw, lb = (_t(w0), _t(b0)) if version == "B" else (None, None)
    out, idx, mask = ops.forward_epilogue(x, e, iw, nb, wt, bias, lw, lb, relu, save_mask, QT[quant])
    torch.cuda.synchronize()
    return (x, e, iw, nb, wt, lw), out, idx, mask


def _expected_forward(w, w0, b0, version, relu, quant, c_oracle):
    """fp32 ops after the C mirror's exactly rounded x_ple (A), float64 (B)."""
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant=quant)
    if version == "A":
        v = (mirror + w.bias[None]).astype(np.float32)            # one fp32 add, like the store
        passm = po.relu_pass(v)
        out = np.where(passm, v, np.float32(0.0)) if relu else v
        return out.astype(np.float32), None, passm
    passm = po.relu_pass(mirror)
    a = np.where(passm, mirror, np.float32(0.0)) if relu else mirror
    lin = b0[None].astype(np.float64) + w0[None].astype(np.float64) * w.x.astype(np.float64)[..., None]
    exp = lin + a.astype(np.float64)
    return exp, np.abs(lin) + np.abs(a), passm


@pytest.mark.parametrize("cfg,quant", [(0, "f32"), (1, "f32"), (2, "f32"), (0, "bf16"), (1, "bf16"), (0, "f16")])
@pytest.mark.parametrize("version,relu", KINDS)
def test_forward_epilogue_matches_mirror(cfg, quant, version, relu, c_oracle):
    w, w0, b0, _ = _setup(cfg)
    print(f"forward_epilogue {w.name} shape={w.shape} quant={quant} version={version} relu={relu}", flush=True)
    _, out, idx, mask = _run_forward(w, w0, b0, version, relu, quant)
    assert out.dtype == torch.float32
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), po.bin_indices(w.x, w.edges, w.n_bins))
    exp, abs_terms, passm = _expected_forward(w, w0, b0, version, relu, quant, c_oracle)
    got = out.cpu().numpy()
    if version == "A":
        np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))
    else:
        # one fma (lin) and one add: two fp32 roundings of values bounded by abs_terms
        ok, worst = close_scaled(got, exp, abs_terms, 2.0 ** -22, 0.0)
        print(f"  out vs fp64: worst error / allowance = {worst:.3g}", flush=True)
        assert ok
    if relu:
        assert mask.shape == (w.shape[0], w.shape[1], (w.shape[3] + 31) // 32) and mask.dtype == torch.int32
        np.testing.assert_array_equal(mask.cpu().numpy(), po.pack_pass_bits(passm))
    else:
        assert mask.numel() == 0


def _check_backward(w, w0, b0, g, version, relu, quant, mask, grads):
    gx, gw, gb, glw, glb = grads
    idx = po.bin_indices(w.x, w.edges, w.n_bins)
    passm = po.unpack_pass_bits(mask.cpu().numpy(), w.shape[3]) if relu else None
    ref = po.module_backward(g, w.x, (w.edges, w.inv_widths, w.n_bins), w.weight, idx, pass_mask=passm,
                             has_bias=version == "A", linear0=(w0, b0) if version == "B" else None, quant=quant)
    pairs = [("dx", gx, "dx"), ("dW", gw, "dw")]
    pairs += [("db", gb, "db")] if version == "A" else [("d lin_w", glw, "dlw"), ("d lin_b", glb, "dlb")]
    for name, got, key in pairs:
        ok, worst = close_scaled(got.cpu().numpy(), ref[key], ref[key + "_abs"], FP32_RTOL, FP32_ATOL)
        print(f"  {name}: worst error / allowance = {worst:.3g}", flush=True)
        assert ok, name


@pytest.mark.parametrize("cfg,quant", [(0, "f32"), (1, "f32"), (2, "f32"), (0, "bf16"), (1, "bf16"), (0, "f16")])
@pytest.mark.parametrize("version,relu", KINDS)
def test_backward_epilogue_matches_oracle(cfg, quant, version, relu):
    w, w0, b0, g = _setup(cfg, seed=1)
    print(f"backward_epilogue {w.name} shape={w.shape} quant={quant} version={version} relu={relu}", flush=True)
    (x, e, iw, nb, wt, lw), _, idx, mask = _run_forward(w, w0, b0, version, relu, quant)
    a = version == "A"
    grads = ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, mask, lw, relu, QT[quant],
                                  True, True, a, not a, not a)
    torch.cuda.synchronize()
    for t, want in zip(grads[2:], (a, not a, not a)):
        assert (t.numel() > 0) == want
    _check_backward(w, w0, b0, g, version, relu, quant, mask, grads)


def _setup_shape(n, f, bmax, d, seed):
    """Random edges (ragged bin counts), x with exact edge hits, and the
    linear0 parameters and gradient of `_setup`, at any shape."""
    rng = np.random.default_rng(seed)
    bins = []
    for j in range(f):
        nb = bmax if j == 0 else int(rng.integers(1, bmax + 1))
        bins.append(np.cumsum(rng.uniform(0.05, 1.0, nb + 1)).astype(np.float32) - np.float32(nb * 0.25))
    edges, iw, nbins = workloads.pad_bins(bins)
    x = (rng.standard_normal((n, f)) * 3).astype(np.float32)
    for j, e in enumerate(bins):
        hit = rng.random(n) < 0.1
        x[hit, j] = e[rng.integers(0, e.size, int(hit.sum()))]
    wt = rng.uniform(-0.5, 0.5, (f, bmax, d)).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, (f, d)).astype(np.float32)
    w = workloads.Workload(f"rand{n}x{f}x{bmax}x{d}", x, bins, edges, iw, nbins, wt, b)
    w0 = rng.uniform(-0.3, 0.3, size=(f, d)).astype(np.float32)
    b0 = rng.uniform(-0.3, 0.3, size=(f, d)).astype(np.float32)
    g = rng.standard_normal((n, f, d)).astype(np.float32)
    return w, w0, b0, g


# Embedding widths whose lane groups differ from the configs': two-lane groups
# (d = 8, 4 columns a lane), a group of four with one idle lane (12), one
# column a lane in 16-, 32- and 64-lane groups (15, 23, 47), two columns a
# lane (30, 38), and ReLU masks of two words where a quad of lanes holds both
# active and idle lanes (40, 44).
@pytest.mark.parametrize("d,quant", [(8, "f32"), (12, "f32"), (15, "f32"), (23, "f32"), (30, "f32"), (40, "f32"),
                                     (44, "f32"), (38, "f32"), (47, "f32"), (15, "bf16"), (30, "bf16"),
                                     (44, "bf16")])
@pytest.mark.parametrize("version,relu", [("A", True), ("B", True), ("B", False)])
def test_backward_epilogue_lane_group_widths(d, quant, version, relu):
    w, w0, b0, g = _setup_shape(1500, 7, 40, d, seed=d)
    print(f"backward_epilogue {w.name} quant={quant} version={version} relu={relu}", flush=True)
    (x, e, iw, nb, wt, lw), _, idx, mask = _run_forward(w, w0, b0, version, relu, quant)
    a = version == "A"
    grads = ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, mask, lw, relu, QT[quant],
                                  True, True, a, not a, not a)
    torch.cuda.synchronize()
    _check_backward(w, w0, b0, g, version, relu, quant, mask, grads)


@pytest.mark.parametrize("version,relu", [("A", True), ("B", True), ("B", False)])
def test_fallback_backward_epilogue_matches_oracle(version, relu, tune):
    """The shapes that leave the sorted path (the BWD_SIMPLE knob forces it)."""
    tune("BWD_SIMPLE", 1)
    w, w0, b0, g = _setup(0, seed=2)
    (x, e, iw, nb, wt, lw), _, idx, mask = _run_forward(w, w0, b0, version, relu, "f32")
    a = version == "A"
    grads = ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, mask, lw, relu, torch.float32,
                                  True, True, a, not a, not a)
    torch.cuda.synchronize()
    _check_backward(w, w0, b0, g, version, relu, "f32", mask, grads)


@pytest.mark.parametrize("version,relu", KINDS)
def test_partial_gradients_match_full(version, relu):
    """Each gradient alone equals the same gradient from the full launch."""
    w, w0, b0, g = _setup(1, seed=3)
    (x, e, iw, nb, wt, lw), _, idx, mask = _run_forward(w, w0, b0, version, relu, "f32")
    a = version == "A"
    flags = [True, True, a, not a, not a]
    full = ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, mask, lw, relu, torch.float32, *flags)
    for i, on in enumerate(flags):
        if not on:
            continue
        only = [j == i for j in range(5)]
        part = ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, mask, lw, relu, torch.float32, *only)
        assert torch.equal(part[i], full[i]), i


def test_backward_epilogue_is_deterministic():
    w, w0, b0, g = _setup(3, seed=4)
    (x, e, iw, nb, wt, lw), _, idx, mask = _run_forward(w, w0, b0, "B", True, "f32")
    runs = [ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, mask, lw, True, torch.float32,
                                  True, True, False, True, True) for _ in range(2)]
    for a_, b_ in zip(*runs):
        assert torch.equal(a_, b_)


@pytest.mark.parametrize("version,relu", KINDS)
@pytest.mark.parametrize("amp", [None, torch.bfloat16])
def test_module_fused_matches_unfused_ops(version, relu, amp):
    """The module's fused path against the reference's op sequence on the GPU
    (``forward`` + PyTorch tail), forward and every gradient."""
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings
    from tests.ple_cases import init_parameters_, make_bins, sample_features

    bins = make_bins("ragged")
    m = CudaPiecewiseLinearEmbeddings(bins, 24, activation=relu, version=version)
    init_parameters_(m, seed=7)
    if version == "B":
        torch.nn.init.uniform_(m.linear.weight, -0.5, 0.5)   # version B starts at zero
    m = m.to(DEV)
    x = sample_features(bins, batch_size=300, seed=8).to(DEV)
    g = torch.randn((300, len(bins), 24), device=DEV, generator=torch.Generator(DEV).manual_seed(9))

    def unfused(xx):
        out_dtype = amp if amp is not None else torch.float32
        x_ple, _ = ops.forward(xx, m._cuda_bin_edges, m._cuda_inv_bin_widths, m._cuda_n_bins, m.linear.weight,
                               out_dtype)
        if m.linear.bias is not None:
            x_ple = x_ple + m.linear.bias
        if m.activation is not None:
            x_ple = m.activation(x_ple)
        return x_ple if m.linear0 is None else m.linear0(xx) + x_ple

    results = []
    for fn in (m, unfused):
        xx = x.clone().requires_grad_(True)
        for p in m.parameters():
            p.grad = None
        if amp is None:
            out = fn(xx)
        else:
            with torch.autocast(device_type="cuda", dtype=amp):
                out = fn(xx)
        out.backward(g.to(out.dtype))
        results.append([out.detach().float(), xx.grad] + [p.grad.clone() for p in m.parameters()])
    assert results[0][0].dtype == results[1][0].dtype
    for got, exp in zip(*results):
        torch.testing.assert_close(got, exp, rtol=1e-5, atol=1e-5)


def test_relu_without_saved_mask_cannot_be_differentiated():
    w, w0, b0, _ = _setup(0)
    x, e, iw, nb, wt = _t(w.x).requires_grad_(True), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight)
    out, _, mask = ops.forward_epilogue(x, e, iw, nb, wt, _t(w.bias), None, None, True, False, torch.float32)
    assert mask.numel() == 0
    with pytest.raises(RuntimeError, match="save_mask=False"):
        out.sum().backward()


def test_epilogue_argument_errors():
    w, w0, b0, g = _setup(0)
    x, e, iw, nb, wt = _t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight)
    with pytest.raises(RuntimeError, match="exactly one of bias and lin_weight"):
        ops.forward_epilogue(x, e, iw, nb, wt, _t(w.bias), _t(w0), _t(b0), False, True, torch.float32)
    with pytest.raises(RuntimeError, match="exactly one of bias and lin_weight"):
        ops.forward_epilogue(x, e, iw, nb, wt, None, None, None, True, True, torch.float32)
    with pytest.raises(RuntimeError, match="lin_bias must be given"):
        ops.forward_epilogue(x, e, iw, nb, wt, None, _t(w0), None, False, True, torch.float32)
    _, idx, mask = ops.forward_epilogue(x, e, iw, nb, wt, None, _t(w0), _t(b0), True, True, torch.float32)
    with pytest.raises(RuntimeError, match="no bias gradient with lin_weight"):
        ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, mask, _t(w0), True, torch.float32,
                              True, True, True, True, True)
    with pytest.raises(RuntimeError, match="relu_mask must be"):
        ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, mask[:, :1].contiguous().view(-1), _t(w0), True,
                              torch.float32, True, True, False, True, True)


def test_c_abi_epilogue_matches_operators():
    """ctypes calls of the epilogue entry points give the operators' bits, and
    the argument checks return their codes before any launch."""
    from piecewiselinearembeddings_optimized_amd import capi

    w, w0, b0, g = _setup(1, seed=5)
    n, f, bmax, d = w.shape
    (x, e, iw, nb, wt, lw), out_op, idx_op, mask_op = _run_forward(w, w0, b0, "B", True, "bf16")
    lb = _t(b0)
    out = torch.empty_like(out_op)
    idx = torch.empty_like(idx_op)
    mask = torch.empty_like(mask_op)
    epi = capi.epilogue(lin_weight=lw, lin_bias=lb, relu=True, relu_mask=mask)
    capi.forward_epilogue(x, e, iw, nb, wt, epi, out, idx, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(out, out_op) and torch.equal(idx, idx_op) and torch.equal(mask, mask_op)
    gx, gw, glw, glb = (torch.empty_like(x), torch.empty_like(wt), torch.empty((f, d), device=DEV),
                        torch.empty((f, d), device=DEV))
    capi.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, epi, gx, gw, None, glw, glb, torch.bfloat16)
    ref = ops.backward_epilogue(_t(g), x, e, iw, nb, wt, idx_op, mask_op, lw, True, torch.bfloat16,
                                True, True, False, True, True)
    torch.cuda.synchronize()
    for a_, b_ in zip((gx, gw, glw, glb), (ref[0], ref[1], ref[3], ref[4])):
        assert torch.equal(a_, b_)
    both = capi.epilogue(bias=_t(w.bias), lin_weight=lw, lin_bias=lb)
    with pytest.raises(capi.PleError) as ei:
        capi.forward_epilogue(x, e, iw, nb, wt, both, out, idx, torch.float32)
    assert ei.value.code == -7
    no_mask = capi.epilogue(lin_weight=lw, lin_bias=lb, relu=True)
    with pytest.raises(capi.PleError) as ei:
        capi.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, no_mask, gx, None, None, None, None, torch.float32)
    assert ei.value.code == -1
    with pytest.raises(capi.PleError) as ei:
        capi.backward_epilogue(_t(g), x, e, iw, nb, wt, idx, epi, gx, None, glw, None, None, torch.float32)
    assert ei.value.code == -7
