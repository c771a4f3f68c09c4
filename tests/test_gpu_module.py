"""Module-level parity on the GPU, mirroring the reference's
``tests/test_correctness.py``: the same bin sets, input sampler, parameter
initialisation, grid (version x activation x seed x d) and tolerances.

The expected values come from the same module evaluated on the CPU, whose
path is the dense upstream formulation (addcmul -> clamps -> per-feature
matmul -> bias), i.e. what the reference compares against.
"""

from __future__ import annotations

import copy

import pytest
import torch

from tests.ple_cases import (
    AMP_FORWARD_ATOL, AMP_FORWARD_RTOL, AMP_GRAD_ATOL, AMP_GRAD_RTOL, BIN_CASE_NAMES,
    D_EMBEDDING_VALUES, FORWARD_ATOL, FORWARD_RTOL, GRAD_ATOL, GRAD_RTOL, SEED_VALUES,
    init_parameters_, make_bins, sample_features,
)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "HIP device required"
    yield


def _modules(case_name, d, activation, version, seed):
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings

    bins = make_bins(case_name)
    cpu = CudaPiecewiseLinearEmbeddings(bins, d, activation=activation, version=version)
    init_parameters_(cpu, seed=seed)
    gpu = copy.deepcopy(cpu).to("cuda")
    assert set(dict(gpu.named_parameters())) == set(dict(cpu.named_parameters()))
    return bins, cpu, gpu


GRID = pytest.mark.parametrize(
    "case_name,version,activation,seed,d",
    [
        (c, v, a, s, d)
        for c in BIN_CASE_NAMES for v in ("A", "B") for a in (False, True)
        for s in SEED_VALUES for d in D_EMBEDDING_VALUES
    ],
)


@GRID
def test_forward_matches_cpu_module(case_name, version, activation, seed, d):
    bins, cpu, gpu = _modules(case_name, d, activation, version, seed)
    x = sample_features(bins, batch_size=128, seed=seed + 1000)
    with torch.no_grad():
        expected = cpu(x)
        actual = gpu(x.cuda())
    assert actual.shape == (128, len(bins), d)
    assert actual.dtype == expected.dtype
    assert gpu.get_output_shape() == cpu.get_output_shape()
    torch.testing.assert_close(actual.cpu(), expected, rtol=FORWARD_RTOL, atol=FORWARD_ATOL)


@GRID
def test_backward_matches_cpu_module(case_name, version, activation, seed, d):
    bins, cpu, gpu = _modules(case_name, d, activation, version, seed)
    xb = sample_features(bins, batch_size=128, seed=seed + 2000)
    xc = xb.clone().requires_grad_(True)
    xg = xb.cuda().requires_grad_(True)
    oc, og = cpu(xc), gpu(xg)
    torch.manual_seed(seed + 3000)
    g = torch.randn_like(oc)
    oc.backward(g)
    og.backward(g.cuda())
    torch.testing.assert_close(xg.grad.cpu(), xc.grad, rtol=GRAD_RTOL, atol=GRAD_ATOL)
    torch.testing.assert_close(gpu.linear.weight.grad.cpu(), cpu.linear.weight.grad, rtol=GRAD_RTOL, atol=GRAD_ATOL)
    if version == "A":
        torch.testing.assert_close(gpu.linear.bias.grad.cpu(), cpu.linear.bias.grad, rtol=GRAD_RTOL, atol=GRAD_ATOL)
    else:
        assert gpu.linear.bias is None
        _check_linear0_grads(gpu, xb, g, GRAD_RTOL, GRAD_ATOL)


def _check_linear0_grads(gpu, x, g, rtol, atol):
    """linear0 (x_linear = b0 + w0 * x) is plain PyTorch on both sides; its
    gradients are sums over the batch, so they are checked against float64
    with the tolerance scaled by the sum of |terms| (a CPU and a GPU fp32 sum
    of 128 terms may differ by more than rtol * |sum| under cancellation)."""
    gd, xd = g.double(), x.double()
    terms_w = gd * xd[..., None]
    dw0, dw0_abs = terms_w.sum(0), terms_w.abs().sum(0)
    db0, db0_abs = gd.sum(0), gd.abs().sum(0)
    for got, exp, s in ((gpu.linear0.weight.grad, dw0, dw0_abs), (gpu.linear0.bias.grad, db0, db0_abs)):
        err = (got.cpu().double() - exp).abs()
        assert bool((err <= atol + rtol * s).all()), float((err / (atol + rtol * s)).max())


def _amp_reference(cpu, x, dtype=torch.bfloat16):
    """The reference module under ``dtype`` autocast, evaluated on the CPU: PLE
    branch rounded through ``dtype`` (encoding and weights), fp32
    accumulation, ``dtype`` result, then the fp32 bias / residual."""
    enc = cpu.impl(x)
    x_ple = (enc.to(dtype).float().transpose(0, 1) @ cpu.linear.weight.to(dtype).float())
    x_ple = x_ple.transpose(0, 1).to(dtype)
    out = x_ple.float() + cpu.linear.bias if cpu.linear.bias is not None else x_ple
    if cpu.activation is not None:
        out = cpu.activation(out)
    if cpu.linear0 is not None:
        out = cpu.linear0(x) + out
    return out


AMP_DTYPES = pytest.mark.parametrize("amp_dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])


@AMP_DTYPES
@GRID
def test_forward_amp_matches(case_name, version, activation, seed, d, amp_dtype):
    bins, cpu, gpu = _modules(case_name, d, activation, version, seed)
    x = sample_features(bins, batch_size=128, seed=seed + 4000)
    with torch.no_grad():
        expected = _amp_reference(cpu, x, amp_dtype)
        with torch.autocast(device_type="cuda", dtype=amp_dtype):
            actual = gpu(x.cuda())
    assert actual.dtype == expected.dtype
    torch.testing.assert_close(actual.float().cpu(), expected.float(), rtol=AMP_FORWARD_RTOL, atol=AMP_FORWARD_ATOL)


@AMP_DTYPES
@GRID
def test_backward_amp_matches(case_name, version, activation, seed, d, amp_dtype):
    bins, cpu, gpu = _modules(case_name, d, activation, version, seed)
    xb = sample_features(bins, batch_size=128, seed=seed + 5000)
    xc = xb.clone().requires_grad_(True)
    xg = xb.cuda().requires_grad_(True)
    oc = _amp_reference(cpu, xc, amp_dtype)
    with torch.autocast(device_type="cuda", dtype=amp_dtype):
        og = gpu(xg)
    torch.manual_seed(seed + 6000)
    g = torch.randn(oc.shape, dtype=torch.float32).to(oc.dtype)
    oc.backward(g)
    og.backward(g.to(og.dtype).cuda())
    assert xg.grad.dtype == torch.float32
    torch.testing.assert_close(xg.grad.cpu(), xc.grad, rtol=AMP_GRAD_RTOL, atol=AMP_GRAD_ATOL)
    torch.testing.assert_close(gpu.linear.weight.grad.cpu(), cpu.linear.weight.grad, rtol=AMP_GRAD_RTOL, atol=AMP_GRAD_ATOL)
    if version == "A":
        torch.testing.assert_close(gpu.linear.bias.grad.cpu(), cpu.linear.bias.grad, rtol=AMP_GRAD_RTOL, atol=AMP_GRAD_ATOL)
    else:
        _check_linear0_grads(gpu, xb, g.float(), AMP_GRAD_RTOL, AMP_GRAD_ATOL)


def test_module_errors_on_gpu():
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings

    m = CudaPiecewiseLinearEmbeddings(make_bins("equal"), 8, activation=False, version="A").cuda()
    with pytest.raises(TypeError):
        m(torch.zeros(4, 3, device="cuda", dtype=torch.float64))
    with pytest.raises(ValueError):
        m(torch.zeros(3, 4, device="cuda").t())
    with pytest.raises(ValueError):
        m(torch.zeros(4, 2, device="cuda"))
    with pytest.raises(ValueError):
        m(torch.zeros(4, 3, 1, device="cuda"))


@pytest.mark.parametrize("version,activation", [("A", True), ("B", False), ("B", True)])
def test_module_on_computed_bins(version, activation, c_oracle):
    """compute_bins (quantile edges with duplicate collapse: discrete and
    two-valued features give ragged and single-bin features) -> module on the
    GPU, evaluated on the very samples the bins came from (so x sits exactly
    on edges, the minimum and maximum included).  The forward is checked
    against the CPU module; the gradients against the float64 closed form
    with the fp32 ReLU decisions of the C mirror: at x == e_0 the dense CPU
    formulation's addcmul rounding turns an exact 0 into +-1e-9, which a ReLU
    then passes or blocks (upstream's rounding, "parity unpinned"), while the
    reference kernel's arithmetic, like this one's, gives exactly 0."""
    import numpy as np

    from oracle import ple_oracle as po
    from piecewiselinearembeddings_optimized_amd import bin_tables, compute_bins
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings
    from tests.ple_cases import FP32_ATOL, FP32_RTOL, close_scaled

    rng = np.random.default_rng(17)
    n = 4000
    cols = [rng.standard_normal(n), rng.lognormal(0, 1, n), rng.poisson(3.0, n).astype(float),
            np.where(rng.random(n) < 0.8, -1.0, 2.0), rng.uniform(-5, 5, n)]
    X = torch.tensor(np.stack(cols, 1), dtype=torch.float32)
    with pytest.warns(UserWarning):
        bins = compute_bins(X, n_bins=32)
    assert len({b.numel() for b in bins}) > 1 and min(b.numel() for b in bins) == 2
    cpu = CudaPiecewiseLinearEmbeddings(bins, 16, activation=activation, version=version)
    init_parameters_(cpu, seed=5)
    if version == "B":
        torch.nn.init.uniform_(cpu.linear.weight, -0.5, 0.5)
    gpu = copy.deepcopy(cpu).to("cuda")
    order = torch.argsort(X[:, 1])                     # includes feature 1's minimum and maximum
    xb = torch.cat([X[order[:4]], X[order[-4:]], X[:120]])
    xg = xb.cuda().requires_grad_(True)
    og = gpu(xg)
    with torch.no_grad():
        oc = cpu(xb)
    torch.testing.assert_close(og.detach().cpu(), oc, rtol=FORWARD_RTOL, atol=FORWARD_ATOL)
    g = torch.randn(og.shape, generator=torch.Generator().manual_seed(6))
    og.backward(g.cuda())

    edges, iw, nb = (t.numpy() for t in bin_tables(bins))
    w = cpu.linear.weight.detach().numpy()
    bias = None if cpu.linear.bias is None else cpu.linear.bias.detach().numpy()
    x_np = xb.numpy()
    pre32, idx = c_oracle.forward_f32(x_np, edges, iw, nb, w, bias=bias)   # the kernel's fp32 pre-activation
    lin = None if version == "A" else (cpu.linear0.weight.detach().numpy(), cpu.linear0.bias.detach().numpy())
    ref = po.module_backward(g.numpy(), x_np, (edges, iw, nb), w, idx.astype(np.int64),
                             pass_mask=po.relu_pass(pre32) if activation else None,
                             has_bias=version == "A", linear0=lin)
    got = {"dx": xg.grad, "dw": gpu.linear.weight.grad}
    if version == "A":
        got["db"] = gpu.linear.bias.grad
    else:
        got["dlw"], got["dlb"] = gpu.linear0.weight.grad, gpu.linear0.bias.grad
    for key, t in got.items():
        ok, worst = close_scaled(t.cpu().numpy(), ref[key], ref[key + "_abs"], FP32_RTOL, FP32_ATOL)
        assert ok, (key, worst)
