"""GPU parity of the HIP kernels against the CPU oracle (run with ``-m gpu``).

Forward: bin indices bit-exact against the oracle; float outputs bit-exact
against the C mirror of the reference arithmetic (``oracle/ple_oracle.c``),
and within the fp32 (1e-5 rel / 1e-6 abs) or bf16 (1e-2 rel) bar against the
float64 closed form, the relative part scaled by the sum of |terms|.

Backward: dx, dW, db within the same bar against the float64 oracle, and
bitwise reproducible run to run.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ple_oracle as po
from piecewiselinearembeddings_optimized_amd import workloads
from tests.ple_cases import BF16_RTOL, FP32_ATOL, FP32_RTOL, close_scaled, normwise_rel

pytestmark = pytest.mark.gpu

ops = None
DEV = "cuda:0"

# reduced sample counts: the float64 oracle finishes in seconds
REDUCED = {0: None, 1: 8192, 2: 4096, 3: 32768, 4: 2048}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    global ops
    assert torch.cuda.is_available(), "HIP device required"
    import piecewiselinearembeddings_optimized_amd  # noqa: F401  (registers the ops)

    ops = torch.ops.rtdl_num_embeddings_cuda
    yield


def _t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t if dtype is None else t.to(dtype)


def _inputs(w):
    return _t(w.x), _t(w.edges), _t(w.inv_widths), _t(w.n_bins), _t(w.weight), _t(w.bias)


def _grad(shape, seed):
    rng = np.random.default_rng(seed)
    return rng.standard_normal(shape, dtype=np.float32)


def _report(name, ok, worst):
    print(f"  {name}: worst error / allowance = {worst:.3g}", flush=True)
    assert ok, f"{name} outside tolerance (worst ratio {worst:.3g})"


QUANT_TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4])
def test_forward_matches_oracle(cfg, c_oracle):
    w = workloads.make(cfg, REDUCED[cfg])
    print(f"forward {w.name} shape={w.shape} quant={w.quant}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, idx = ops.forward(x, e, iw, nb, wt, QUANT_TORCH[w.quant])
    torch.cuda.synchronize()
    idx_ref = po.bin_indices(w.x, w.edges, w.n_bins)
    assert idx.dtype == {1: torch.uint8, 2: torch.int16, 4: torch.int32}[po.bin_index_dtype(w.shape[2]).itemsize]
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), idx_ref)
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant=w.quant)
    got = out.float().cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), mirror.view(np.uint32))
    ref, _, s = po.forward(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant=w.quant, return_abs=True)
    if w.quant == "f32":
        _report("out vs fp64", *close_scaled(got, ref, s, FP32_RTOL, FP32_ATOL))
    else:
        _report("out vs fp64 (bf16 bar)", *close_scaled(got, ref, s, BF16_RTOL, 0.0))
        # against the unrounded fp32 math: relative error of the tensor
        ref32, _ = po.forward(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant="f32")
        rel = normwise_rel(got, ref32)
        print(f"  out vs unrounded fp64: normwise relative error {rel:.3g}", flush=True)
        assert rel <= BF16_RTOL


@pytest.mark.parametrize("cfg", [0, 1, 2])
def test_forward_float16_matches_oracle(cfg, c_oracle):
    """fp16 output (the autocast-fp16 path): the fraction, the weights and the
    result round through IEEE half; bit-exact against the C mirror."""
    w = workloads.make(cfg, REDUCED[cfg])
    print(f"forward f16 {w.name} shape={w.shape}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, idx = ops.forward(x, e, iw, nb, wt, torch.float16)
    assert out.dtype == torch.float16
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), po.bin_indices(w.x, w.edges, w.n_bins))
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant="f16")
    got = out.float().cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), mirror.view(np.uint32))
    ref, _, s = po.forward(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant="f16", return_abs=True)
    # half's subnormal quantum (2^-24) bounds the rounding error near zero
    _report("out vs fp64 (f16 rounding, bf16 bar)", *close_scaled(got, ref, s, BF16_RTOL, 2.0 ** -24))
    ref32, _ = po.forward(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant="f32")
    rel = normwise_rel(got, ref32)
    print(f"  out vs unrounded fp64: normwise relative error {rel:.3g}", flush=True)
    assert rel <= 1e-3   # half keeps 11 significant bits


@pytest.mark.parametrize("cfg,dtype", [(1, torch.float16), (4, torch.bfloat16)])
def test_forward_16bit_store_widths_agree(cfg, dtype, tune):
    """16-bit outputs store 8 per lane when D allows (16-byte stores) or 4 per
    lane (the FWD_VEC knob forces it): the same bits either way."""
    w = workloads.make(cfg, REDUCED[cfg])
    print(f"forward store widths {w.name} {dtype}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out8, idx8 = ops.forward(x, e, iw, nb, wt, dtype)
    tune("FWD_VEC", 4)
    out4, idx4 = ops.forward(x, e, iw, nb, wt, dtype)
    tune("FWD_VEC", 0)
    assert torch.equal(idx8, idx4)
    assert torch.equal(out8.view(torch.int16), out4.view(torch.int16))


@pytest.mark.parametrize("cfg", [0, 1, 3, 4])
def test_forward_workgroup_sizes_agree(cfg, tune):
    """256- and 512-thread forward workgroups (the FWD_FB knob; the planner picks
    512 for large tables and narrow rows) give the same bits."""
    w = workloads.make(cfg, REDUCED[cfg])
    print(f"forward workgroup sizes {w.name}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    dtype = torch.bfloat16 if w.quant == "bf16" else torch.float32
    outs = []
    for fb in (256, 512):
        tune("FWD_FB", fb)
        outs.append(ops.forward(x, e, iw, nb, wt, dtype))
    tune("FWD_FB", 0)
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))


@pytest.mark.parametrize("cfg", [0, 1, 2])
def test_backward_float16_grad_matches_oracle(cfg, c_oracle):
    """fp16 gradient with fp16 quantisation (the backward of the autocast-fp16
    forward): dx / dW against the fp16-aware float64 oracle at the fp32 bar."""
    w = workloads.make(cfg, REDUCED[cfg])
    n, f, bmax, d = w.shape
    print(f"backward f16 {w.name} shape={w.shape}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    _, idx = ops.forward(x, e, iw, nb, wt, torch.float16)
    g_h = torch.from_numpy(_grad((n, f, d), 300 + cfg)).to(torch.float16)
    gx, gw = ops.backward(g_h.to(DEV), x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    _check_backward(w, "f16", g_h.float().numpy(), gx, gw, None, c_oracle)


@pytest.mark.parametrize("cfg", [0, 1, 2, 3])
def test_forward_with_bias_matches_oracle(cfg, c_oracle):
    w = workloads.make(cfg, REDUCED[cfg])
    print(f"forward_with_bias {w.name} shape={w.shape}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, _ = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, bias=w.bias)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), mirror.view(np.uint32))
    ref, _, s = po.forward(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, bias=w.bias, return_abs=True)
    _report("out+bias vs fp64", *close_scaled(got, ref, s, FP32_RTOL, FP32_ATOL))


def _check_backward(w, quant, g, gx, gw, gb, c_oracle, grad_bias_source=None):
    idx = po.bin_indices(w.x, w.edges, w.n_bins)
    ref = c_oracle.backward_f64(g, w.x, w.edges, w.inv_widths, w.n_bins, w.weight, idx, quant=quant,
                                grad_bias_source=grad_bias_source)
    if gx is not None:
        _report("dx", *close_scaled(gx.cpu().numpy(), ref["dx"], ref["dx_abs"], FP32_RTOL, FP32_ATOL))
    if gw is not None:
        _report("dW", *close_scaled(gw.cpu().numpy(), ref["dw"], ref["dw_abs"], FP32_RTOL, FP32_ATOL))
    if gb is not None:
        _report("db", *close_scaled(gb.cpu().numpy(), ref["db"], ref["db_abs"], FP32_RTOL, FP32_ATOL))


@pytest.mark.parametrize("cfg", [0, 1, 2, 3])
def test_backward_with_bias_matches_oracle(cfg, c_oracle):
    w = workloads.make(cfg, REDUCED[cfg])
    print(f"backward_with_bias {w.name} shape={w.shape}", flush=True)
    n, f, bmax, d = w.shape
    x, e, iw, nb, wt, bt = _inputs(w)
    _, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    g = _grad((n, f, d), 100 + cfg)
    gx, gw, gb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    torch.cuda.synchronize()
    _check_backward(w, "f32", g, gx, gw, gb, c_oracle)


def test_backward_bf16_grad_matches_oracle(c_oracle):
    w = workloads.make(4, REDUCED[4])
    n, f, bmax, d = w.shape
    print(f"backward bf16 {w.name} shape={w.shape}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    _, idx = ops.forward(x, e, iw, nb, wt, torch.bfloat16)
    g32 = _grad((n, f, d), 104)
    g_bf = torch.from_numpy(g32).to(torch.bfloat16)
    gx, gw = ops.backward(g_bf.to(DEV), x, e, iw, nb, wt, idx, True, True)
    g_seen = g_bf.float().numpy()
    _check_backward(w, "bf16", g_seen, gx, gw, None, c_oracle)
    # against the unrounded fp32 math at the bf16 bar
    idx_np = po.bin_indices(w.x, w.edges, w.n_bins)
    ref = c_oracle.backward_f64(g32, w.x, w.edges, w.inv_widths, w.n_bins, w.weight, idx_np, quant="f32")
    for name, got, key in (("dW", gw, "dw"), ("dx", gx, "dx")):
        rel = normwise_rel(got.cpu().numpy(), ref[key])
        print(f"  {name} vs unrounded fp32 math: normwise relative error {rel:.3g}", flush=True)
        assert rel <= BF16_RTOL


def test_autocast_style_backward_rounds_grad_but_not_bias_grad(c_oracle):
    """quant=bf16 with an fp32 gradient: dx/dW see bf16(g), db sees g."""
    w = workloads.make(0)
    n, f, bmax, d = w.shape
    x, e, iw, nb, wt, bt = _inputs(w)
    _, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.bfloat16)
    g = _grad((n, f, d), 7)
    gx, gw, gb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.bfloat16, True, True, True)
    gq = po.quantize(g, "bf16")
    _check_backward(w, "bf16", gq, gx, gw, gb, c_oracle, grad_bias_source=g)


def test_backward_is_deterministic():
    w = workloads.make(3, 65536)
    n, f, bmax, d = w.shape
    print(f"determinism {w.name} shape={w.shape}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    _, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    g = torch.randn((n, f, d), device=DEV, generator=torch.Generator(DEV).manual_seed(3))
    r1 = ops.backward_with_bias(g, x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    r2 = ops.backward_with_bias(g, x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)


def test_bin_indices_and_outputs_for_special_values(c_oracle):
    w = workloads.make(0)
    x = w.x.copy()
    x[0, :] = np.nan
    x[1, :] = np.inf
    x[2, :] = -np.inf
    x[3, :] = w.edges[np.arange(x.shape[1]), w.n_bins]        # last edge exactly
    x[4, :] = w.edges[:, 0]                                   # first edge exactly
    x[5, :] = 1e30
    xt, e, iw, nb, wt, bt = _inputs(w)
    xt = _t(x)
    out, idx = ops.forward(xt, e, iw, nb, wt, torch.float32)
    mirror, midx = c_oracle.forward_f32(x, w.edges, w.inv_widths, w.n_bins, w.weight)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int32), midx)
    got = out.cpu().numpy()
    same = (got.view(np.uint32) == mirror.view(np.uint32)) | (np.isnan(got) & np.isnan(mirror))
    assert same.all()
    assert (idx[0].cpu().numpy() == w.n_bins - 1).all()       # NaN -> last bin


def _random_case(n, f, bmax, d, seed, ragged=True):
    """Random edges (ragged bin counts up to bmax), x with exact edge hits and
    out-of-range values, weights and bias."""
    rng = np.random.default_rng(seed)
    bins = []
    for j in range(f):
        nb = int(rng.integers(1, bmax + 1)) if ragged else bmax
        if j == 0:
            nb = bmax
        e = np.cumsum(rng.uniform(0.05, 1.0, nb + 1)).astype(np.float32) - np.float32(nb * 0.25)
        bins.append(e)
    edges, iw, nbins = workloads.pad_bins(bins)
    x = (rng.standard_normal((n, f)) * 3).astype(np.float32)
    for j, e in enumerate(bins):
        hit = rng.random(n) < 0.1
        x[hit, j] = e[rng.integers(0, e.size, int(hit.sum()))]
    w = rng.uniform(-0.5, 0.5, (f, edges.shape[1] - 1, d)).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, (f, d)).astype(np.float32)
    return workloads.Workload(f"rand{n}x{f}x{bmax}x{d}", x, bins, edges, iw, nbins, w, b)


SHAPES = [
    (1, 1, 1, 1), (7, 3, 5, 10), (129, 5, 7, 15), (1000, 9, 48, 20), (333, 1, 300, 16),
    (2500, 17, 64, 64), (513, 6, 256, 24), (64, 33, 2, 3), (1025, 4, 130, 2), (700, 2, 1000, 8),
    # finalize without an LDS table (B * 2 * 8 * 4 bytes > 160 KiB) over several chunks summed first
    (3000, 2, 3000, 4),
    # even widths that are not multiples of 4: two columns a lane (lane groups of 4, 8 and 16)
    (500, 4, 9, 6), (900, 5, 33, 10), (1200, 6, 64, 14), (640, 3, 50, 18), (410, 2, 17, 26), (777, 3, 20, 30),
    # odd widths: one column a lane in 16- and 32-lane groups
    (600, 3, 25, 23), (450, 2, 70, 31), (350, 4, 12, 9),
    # wider ones: two columns a lane in 32-lane groups, one column a lane in 64-lane groups
    (700, 3, 30, 38), (400, 3, 15, 62), (500, 2, 20, 47),
    # the forward's 512-thread plans of rows up to 24 columns with up to 8 features a group
    (2048, 128, 48, 24), (2048, 128, 48, 12),
    # gradient rows ending inside a 128-byte line in lane groups that would stream them (plain-load twins)
    (1500, 5, 40, 28), (900, 3, 40, 48), (700, 4, 33, 36),
    # forward segments (a feature group's outputs of a sample) ending off 64-byte boundaries: plain stores
    (800, 6, 30, 44),
]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{n}x{f}x{b}x{d}" for n, f, b, d in SHAPES])
def test_shape_sweep_forward_and_backward(shape, c_oracle):
    n, f, bmax, d = shape
    w = _random_case(n, f, bmax, d, seed=sum(shape))
    print(f"shape sweep {w.name}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    mirror, midx = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, bias=w.bias)
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int32), midx)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), mirror.view(np.uint32))
    g = _grad((n, f, d), 5)
    gx, gw, gb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    _check_backward(w, "f32", g, gx, gw, gb, c_oracle)
    # dx alone and dW alone give the same values as together
    gx2, _, _ = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, False, False)
    _, gw2, gb2 = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, False, True, True)
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2) and torch.equal(gb, gb2)


@pytest.mark.parametrize("d", [10, 30])
@pytest.mark.parametrize("quant", ["bf16", "f16"])
def test_two_column_lanes_16bit(d, quant, c_oracle):
    """16-bit outputs and gradients at even widths that are not multiples of
    4 (two columns a lane: 4-byte stores and loads): forward bit-exact against
    the C mirror, backward against the quantisation-aware float64 oracle."""
    n, f, bmax = 1500, 5, 40
    w = _random_case(n, f, bmax, d, seed=d + 7)
    print(f"two-column lanes {w.name} {quant}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, idx = ops.forward(x, e, iw, nb, wt, QUANT_TORCH[quant])
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), po.bin_indices(w.x, w.edges, w.n_bins))
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant=quant)
    np.testing.assert_array_equal(out.float().cpu().numpy().view(np.uint32), mirror.view(np.uint32))
    g_h = torch.from_numpy(_grad((n, f, d), d)).to(QUANT_TORCH[quant])
    gx, gw = ops.backward(g_h.to(DEV), x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    _check_backward(w, quant, g_h.float().numpy(), gx, gw, None, c_oracle)


@pytest.mark.parametrize("d", [8, 16, 40, 64])
@pytest.mark.parametrize("quant", ["bf16", "f16"])
def test_eight_column_lanes_16bit(d, quant, c_oracle, tune):
    """16-bit gradients with D a multiple of 8: eight columns a lane, rows kept
    packed in registers (lane groups of 2, 2, 8 and 8 lanes), with rows on
    their bins' left edges among them; against the quantisation-aware float64
    oracle, as is the four-column form of the same call (knob BWD_VEC=4)."""
    n, f, bmax = 1300, 3, 37
    w = _random_case(n, f, bmax, d, seed=d + 101)
    print(f"eight-column lanes {w.name} {quant}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, idx = ops.forward(x, e, iw, nb, wt, QUANT_TORCH[quant])
    g_h = torch.from_numpy(_grad((n, f, d), d + 3)).to(QUANT_TORCH[quant])
    gx, gw = ops.backward(g_h.to(DEV), x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    _check_backward(w, quant, g_h.float().numpy(), gx, gw, None, c_oracle)
    tune("BWD_VEC", 4)
    gx4, gw4 = ops.backward(g_h.to(DEV), x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    _check_backward(w, quant, g_h.float().numpy(), gx4, gw4, None, c_oracle)


@pytest.mark.parametrize("d", [44, 48, 56])
@pytest.mark.parametrize("quant", ["bf16", "f16"])
def test_16bit_rows_ending_inside_a_line(d, quant, c_oracle):
    """16-bit gradient rows of 88, 96 and 112 bytes in lane groups that stream
    whole-line rows (four columns a lane in 16-lane groups at d = 44, eight
    columns a lane in 8-lane groups at d = 48 and 56): the launcher's
    plain-load twins, against the quantisation-aware float64 oracle.  The
    forward's segments end off 64-byte boundaries at d = 44 and 56 (plain
    stores) and on them at d = 48: bit-exact against the C mirror."""
    n, f, bmax = 1100, 3, 29
    w = _random_case(n, f, bmax, d, seed=d + 301)
    print(f"16-bit rows inside a line {w.name} {quant}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    out, idx = ops.forward(x, e, iw, nb, wt, QUANT_TORCH[quant])
    mirror, _ = c_oracle.forward_f32(w.x, w.edges, w.inv_widths, w.n_bins, w.weight, quant=quant)
    np.testing.assert_array_equal(out.float().cpu().numpy().view(np.uint32), mirror.view(np.uint32))
    g_h = torch.from_numpy(_grad((n, f, d), d + 5)).to(QUANT_TORCH[quant])
    gx, gw = ops.backward(g_h.to(DEV), x, e, iw, nb, wt, idx, True, True)
    torch.cuda.synchronize()
    _check_backward(w, quant, g_h.float().numpy(), gx, gw, None, c_oracle)


@pytest.mark.parametrize("d", [10, 30])
def test_two_column_lanes_match_one_column_lanes(d, c_oracle, tune):
    """The one-column-a-lane forms (knobs FWD_VEC=1, BWD_VEC=1) at the same
    even widths: forward bits equal, backward within the fp32 bar of the oracle."""
    w = _random_case(1100, 3, 30, d, seed=d + 11)
    x, e, iw, nb, wt, bt = _inputs(w)
    g = _grad((1100, 3, d), d + 1)
    out2, _ = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    tune("FWD_VEC", 1)
    tune("BWD_VEC", 1)
    out1, idx1 = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    gx, gw, gb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx1, torch.float32, True, True, True)
    torch.cuda.synchronize()
    assert torch.equal(out1.view(torch.int32), out2.view(torch.int32))
    _check_backward(w, "f32", g, gx, gw, gb, c_oracle)


@pytest.mark.parametrize("quant", ["f32", "bf16"])
def test_single_chunk_plan_writes_dw_db_in_kernel(quant, c_oracle, tune):
    """Plans with one chunk of samples (one feature a workgroup over 600
    features, or a batch of one sub-tile) take dW and db from the gradient
    kernel's own histogram, with no partials and no finalize kernel; a plan
    of several chunks (knob BWD_WG_PER_CU=8) takes the two-kernel route.
    Both against the float64 oracle (bf16: an fp32 gradient rounded for
    dx/dW, db from the unrounded gradient), every output element written
    (the buffers start as NaN), padding weight slots exactly zero."""
    from piecewiselinearembeddings_optimized_amd import capi

    qt = QUANT_TORCH[quant]
    for n, f in ((3000, 600), (700, 9)):
        bmax, d = 20, 8
        w = _random_case(n, f, bmax, d, seed=n + f)
        print(f"single-chunk plan {w.name} n={n} f={f} {quant}", flush=True)
        x, e, iw, nb, wt, bt = _inputs(w)
        _, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, qt)
        g = _grad((n, f, d), n)
        gd = _t(g)
        tune("BWD_FS", 1)
        for wg in (0, 8):
            tune("BWD_WG_PER_CU", wg)
            gx = torch.full((n, f), float("nan"), device=DEV)
            gw = torch.full(tuple(wt.shape), float("nan"), device=DEV)
            gb = torch.full((f, d), float("nan"), device=DEV)
            capi.backward(gd, x, e, iw, nb, wt, idx, gx, gw, gb, qt)
            torch.cuda.synchronize()
            gq = po.quantize(g, quant) if quant != "f32" else g
            _check_backward(w, quant, gq, gx, gw, gb, c_oracle, grad_bias_source=g if quant != "f32" else None)
            for j in range(f):   # the last bin sits in slot bmax-1; slots n-1 .. bmax-2 are padding
                assert torch.count_nonzero(gw[j, max(int(w.n_bins[j]), 1) - 1:bmax - 1]) == 0
            if n <= 1024:   # one sub-tile: one chunk whatever the knob
                break
        tune("BWD_WG_PER_CU", 0)


@pytest.mark.parametrize("cfg", [0, 1, 2, 3])
def test_fallback_backward_path_matches_oracle(cfg, c_oracle, tune):
    """The simple (non-fused) backward kernels, forced by the BWD_SIMPLE knob."""
    tune("BWD_SIMPLE", 1)
    w = workloads.make(cfg, min(REDUCED[cfg] or 4096, 4096))
    n, f, bmax, d = w.shape
    print(f"fallback backward {w.name} shape={w.shape}", flush=True)
    x, e, iw, nb, wt, bt = _inputs(w)
    _, idx = ops.forward_with_bias(x, e, iw, nb, wt, bt, torch.float32)
    g = _grad((n, f, d), 200 + cfg)
    gx, gw, gb = ops.backward_with_bias(_t(g), x, e, iw, nb, wt, idx, torch.float32, True, True, True)
    _check_backward(w, "f32", g, gx, gw, gb, c_oracle)


def test_empty_batch():
    w = workloads.make(0)
    x, e, iw, nb, wt, bt = _inputs(w)
    x0 = x[:0].contiguous()
    out, idx = ops.forward_with_bias(x0, e, iw, nb, wt, bt, torch.float32)
    assert out.shape == (0, x.shape[1], wt.shape[2]) and idx.shape == (0, x.shape[1])
    g = torch.zeros((0, x.shape[1], wt.shape[2]), device=DEV)
    gx, gw, gb = ops.backward_with_bias(g, x0, e, iw, nb, wt, idx, torch.float32, True, True, True)
    assert gx.shape == (0, x.shape[1])
    assert torch.count_nonzero(gw) == 0 and torch.count_nonzero(gb) == 0
