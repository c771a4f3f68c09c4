"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check uses an independent route to the answer -- np.searchsorted, the
dense upstream formulation, torch autograd, finite differences, exact
rational arithmetic, torch/NumPy dtype conversions, closed forms of special
cases -- chosen so that a dropped term, a wrong bin or edge index, a
transposed operand or a wrong rounding step fails at least one of them.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import ple_oracle as po
from tests.ple_cases import BIN_CASE_NAMES, make_bins, sample_features, with_edge_hits


def _case(case_name, d, seed, n=128, edge_hits=True):
    bins_t = make_bins(case_name)
    x = sample_features(bins_t, batch_size=n, seed=seed + 1000)
    if edge_hits:
        x = with_edge_hits(x, bins_t)
    bins = [b.numpy() for b in bins_t]
    edges, iw, nb = po.pad_bins(bins)
    rng = np.random.default_rng(seed)
    f, bmax = edges.shape[0], edges.shape[1] - 1
    w = rng.uniform(-0.5, 0.5, size=(f, bmax, d)).astype(np.float32)
    b = rng.uniform(-0.3, 0.3, size=(f, d)).astype(np.float32)
    g = rng.standard_normal((n, f, d)).astype(np.float32)
    return bins, x.numpy(), edges, iw, nb, w, b, g


def _dense_w(w, nb):
    """Zero the weight rows that no bin maps to (the dense form multiplies
    them by a phantom 0 component; the closed form never reads them)."""
    w = w.copy()
    bmax = w.shape[1]
    for f, n in enumerate(nb):
        w[f, n - 1: bmax - 1] = 0.0
    return w


# ---------------------------------------------------------------------------
# bin index
# ---------------------------------------------------------------------------

def test_bin_index_matches_brute_force_count():
    rng = np.random.default_rng(0)
    for case in BIN_CASE_NAMES:
        bins = [b.numpy() for b in make_bins(case)]
        edges, _, nb = po.pad_bins(bins)
        pts = np.concatenate([
            rng.normal(0, 5, 500).astype(np.float32),
            np.concatenate(bins).astype(np.float32),
            np.array([np.nan, np.inf, -np.inf, 1e30, -1e30], dtype=np.float32),
        ])
        x = np.repeat(pts[:, None], len(bins), axis=1)
        idx = po.bin_indices(x, edges, nb)
        for f, e in enumerate(bins):
            n = len(e) - 1
            for i, v in enumerate(pts):
                if np.isnan(v):
                    expect = n - 1           # every "v < e" is false
                else:
                    cnt = sum(1 for t in e if not (v < t))   # upper bound
                    expect = min(max(cnt - 1, 0), n - 1)
                assert idx[i, f] == expect, (case, f, v)


def test_bin_index_dtype_thresholds():
    assert po.bin_index_dtype(1) == np.uint8
    assert po.bin_index_dtype(256) == np.uint8
    assert po.bin_index_dtype(257) == np.int16
    assert po.bin_index_dtype(32768) == np.int16
    assert po.bin_index_dtype(32769) == np.int32


# ---------------------------------------------------------------------------
# forward: closed form vs dense upstream formulation
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case_name", BIN_CASE_NAMES)
@pytest.mark.parametrize("d", (10, 15, 20))
@pytest.mark.parametrize("seed", (42, 0, 1))
def test_closed_form_forward_equals_dense(case_name, d, seed):
    bins, x, edges, iw, nb, w, b, _ = _case(case_name, d, seed)
    closed, idx = po.forward(x, edges, iw, nb, w, bias=b)
    dense = po.dense_forward(x, bins, _dense_w(w, nb), bias=b)
    # closed form uses the fp32 inverse width, the dense form 1 / width in fp64
    np.testing.assert_allclose(closed, dense, rtol=2e-6, atol=2e-6)


def test_padded_weight_rows_do_not_matter():
    bins, x, edges, iw, nb, w, b, _ = _case("ragged", 12, 3)
    w2 = w.copy()
    for f, n in enumerate(nb):
        w2[f, n - 1: w.shape[1] - 1] = 1e6
    a, _ = po.forward(x, edges, iw, nb, w, bias=b)
    c, _ = po.forward(x, edges, iw, nb, w2, bias=b)
    np.testing.assert_array_equal(a, c)


def test_single_bin_feature_is_affine():
    bins, x, edges, iw, nb, w, b, _ = _case("single_bin", 9, 5)
    out, _ = po.forward(x, edges, iw, nb, w, bias=b)
    f = 1                                      # the single-bin feature
    x64 = x[:, f].astype(np.float64)
    expect = ((x64 - edges[f, 0]) * np.float64(iw[f, 0]))[:, None] * w[f, -1][None].astype(np.float64) + b[f]
    np.testing.assert_allclose(out[:, f], expect, rtol=1e-6, atol=1e-6)


def test_all_single_bin_module_is_affine_and_unclamped():
    bins, x, edges, iw, nb, w, b, _ = _case("all_single_bin", 7, 6)
    out, _ = po.forward(x, edges, iw, nb, w, bias=b)
    x64 = x.astype(np.float64)
    frac = (x64 - edges[:, 0][None]) * iw[:, 0][None].astype(np.float64)
    expect = frac[..., None] * w[:, 0][None].astype(np.float64) + b[None]
    np.testing.assert_allclose(out, expect, rtol=1e-6, atol=1e-6)
    # values far outside the range extrapolate on both sides
    assert (frac < -0.5).any() and (frac > 1.5).any()


def test_forward_is_continuous_across_internal_edges():
    bins, _, edges, iw, nb, w, b, _ = _case("ragged", 8, 7)
    for f, e in enumerate(bins):
        for k in range(1, len(e) - 1):
            at = np.float32(e[k])
            below = np.nextafter(at, np.float32(-np.inf))
            x = np.zeros((2, len(bins)), dtype=np.float32)
            x[0, f], x[1, f] = below, at
            out, idx = po.forward(x, edges, iw, nb, w, bias=b)
            assert idx[0, f] == k - 1 and idx[1, f] == k
            np.testing.assert_allclose(out[0, f], out[1, f], rtol=0, atol=1e-5)


# ---------------------------------------------------------------------------
# backward: closed form vs dense Jacobian vs torch autograd vs differences
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case_name", BIN_CASE_NAMES)
@pytest.mark.parametrize("d", (10, 15, 20))
def test_closed_form_backward_equals_dense_jacobian(case_name, d):
    bins, x, edges, iw, nb, w, b, g = _case(case_name, d, 11)
    _, idx = po.forward(x, edges, iw, nb, w, bias=b)
    cf = po.backward(g, x, edges, iw, nb, w, idx)
    dn = po.dense_backward(g, x, bins, _dense_w(w, nb))
    np.testing.assert_allclose(cf["dx"], dn["dx"], rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(cf["dw"], dn["dw"], rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(cf["db"], dn["db"], rtol=1e-12, atol=1e-12)


def _torch_dense_forward(x, bins, w, b):
    """Upstream dense forward written with torch ops (float64), for autograd."""
    left, width, single = po.dense_layout(bins)
    left_t = torch.tensor(np.nan_to_num(left), dtype=torch.float64)
    width_t = torch.tensor(np.nan_to_num(width, nan=1.0), dtype=torch.float64)
    phantom = torch.tensor(np.isnan(width))
    raw = (x[:, :, None] - left_t[None]) / width_t[None]
    bmax = left.shape[1]
    if bmax > 1:
        first = raw[..., :1].clamp_max(1.0)
        mid = raw[..., 1:-1].clamp(0.0, 1.0)
        last = raw[..., -1:]
        last = torch.where(torch.tensor(single)[None, :, None], last, last.clamp_min(0.0))
        enc = torch.cat([first, mid, last], dim=-1)
    else:
        enc = raw
    enc = torch.where(phantom[None], torch.zeros_like(enc), enc)
    return torch.einsum("nfb,fbd->nfd", enc, w) + b


@pytest.mark.parametrize("case_name", BIN_CASE_NAMES)
def test_dense_jacobian_equals_torch_autograd(case_name):
    bins, x, edges, iw, nb, w, b, g = _case(case_name, 13, 21)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(_dense_w(w, nb), dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    out = _torch_dense_forward(xt, bins, wt, bt)
    out.backward(torch.tensor(g, dtype=torch.float64))
    dn = po.dense_backward(g, x, bins, _dense_w(w, nb))
    np.testing.assert_allclose(dn["dx"], xt.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dn["dw"], wt.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dn["db"], bt.grad.numpy(), rtol=1e-12, atol=1e-12)
    # and the closed form against autograd directly (exact edge hits included)
    _, idx = po.forward(x, edges, iw, nb, w, bias=b)
    cf = po.backward(g, x, edges, iw, nb, w, idx)
    np.testing.assert_allclose(cf["dx"], xt.grad.numpy(), rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(cf["dw"], wt.grad.numpy(), rtol=2e-6, atol=2e-6)


def test_edge_hit_gets_both_neighbouring_terms():
    bins, _, edges, iw, nb, w, b, _ = _case("equal", 5, 2)
    f, k = 0, 2
    x = np.zeros((1, len(bins)), dtype=np.float32)
    x[0, f] = edges[f, k]
    g = np.ones((1, len(bins), 5), dtype=np.float32)
    _, idx = po.forward(x, edges, iw, nb, w, bias=b)
    assert idx[0, f] == k
    dx = po.backward(g, x, edges, iw, nb, w, idx)["dx"][0, f]
    expect = w[f, k].astype(np.float64).sum() * iw[f, k] + w[f, k - 1].astype(np.float64).sum() * iw[f, k - 1]
    np.testing.assert_allclose(dx, expect, rtol=1e-12)


def test_dx_matches_central_differences_away_from_edges():
    bins, x, edges, iw, nb, w, b, g = _case("ragged", 6, 9, edge_hits=False)
    allp = np.concatenate(bins)
    keep = np.all(np.abs(x[:, :, None] - allp[None, None, :]) > 1e-2, axis=2)
    x = x.astype(np.float64)
    _, idx = po.forward(x.astype(np.float32), edges, iw, nb, w, bias=b)
    dx = po.backward(g, x.astype(np.float32), edges, iw, nb, w, idx)["dx"]

    def f64_forward(xx):
        # closed form in float64 throughout (fp64 frac)
        out = np.zeros(xx.shape + (w.shape[2],))
        for ff in range(xx.shape[1]):
            n = nb[ff]
            e = edges[ff, : n + 1].astype(np.float64)
            k = np.clip(np.searchsorted(e, xx[:, ff], side="right") - 1, 0, n - 1)
            frac = (xx[:, ff] - e[k]) / (e[k + 1] - e[k])
            cum = np.concatenate([np.zeros((1, w.shape[2])), np.cumsum(w[ff, : n - 1].astype(np.float64), 0)])
            p = np.where(k == n - 1, w.shape[1] - 1, k)
            out[:, ff] = cum[k] + frac[:, None] * w[ff, p].astype(np.float64)
        return out

    h = 1e-6
    fd = np.zeros_like(x)
    for ff in range(x.shape[1]):
        xp, xm = x.copy(), x.copy()
        xp[:, ff] += h
        xm[:, ff] -= h
        fd[:, ff] = ((f64_forward(xp)[:, ff] - f64_forward(xm)[:, ff]) / (2 * h) * g[:, ff]).sum(-1)
    np.testing.assert_allclose(dx[keep], fd[keep], rtol=1e-4, atol=1e-5)


def test_dw_padded_slots_are_zero_and_db_is_sum():
    bins, x, edges, iw, nb, w, b, g = _case("ragged", 4, 8)
    _, idx = po.forward(x, edges, iw, nb, w, bias=b)
    r = po.backward(g, x, edges, iw, nb, w, idx)
    for f, n in enumerate(nb):
        assert np.all(r["dw"][f, n - 1: w.shape[1] - 1] == 0.0)
    np.testing.assert_allclose(r["db"], g.astype(np.float64).sum(0), rtol=1e-12)
    # the first real bin collects the gradient of every sample
    # (its component is 1 or frac for every x): dW row 0 == sum over n of enc_0 * g
    enc, _, _ = po.dense_encoding(x, bins)
    np.testing.assert_allclose(r["dw"][:, 0], np.einsum("nf,nfd->fd", enc[:, :, 0], g), rtol=2e-6, atol=2e-6)


# ---------------------------------------------------------------------------
# quantisation helpers against library conversions
# ---------------------------------------------------------------------------

def _special_values():
    rng = np.random.default_rng(5)
    v = np.concatenate([
        rng.standard_normal(5000).astype(np.float32),
        (rng.standard_normal(2000) * 1e-6).astype(np.float32),
        (rng.standard_normal(2000) * 1e4).astype(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e-8, 6e-8, 3e-5, 6.1e-5, 1e38,
                  np.inf, -np.inf, 1.00390625, 1.01171875, 3.0e-39], dtype=np.float32),
    ])
    # exact bf16 ties (lower half == 0x8000) with even and odd kept bit
    ties = (np.arange(1000, dtype=np.uint32) << 16 | 0x8000).astype(np.uint32) + np.uint32(0x3F800000)
    return np.concatenate([v, ties.view(np.float32)])


def test_bf16_rounding_matches_torch():
    v = _special_values()
    ours = po.quantize(v, "bf16")
    ref = torch.from_numpy(v).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(ours.view(np.uint32), ref.view(np.uint32))
    nan = po.quantize(np.array([np.nan], dtype=np.float32), "bf16")
    assert np.isnan(nan).all()


def test_f16_rounding_matches_numpy():
    v = _special_values()
    with np.errstate(over="ignore"):
        ref = v.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(po.quantize(v, "f16"), ref)


# ---------------------------------------------------------------------------
# the C restatement against the NumPy one and against exact arithmetic
# ---------------------------------------------------------------------------

def test_c_quantize_matches_library(c_oracle):
    v = _special_values()
    for q in ("bf16", "f16"):
        c = np.array([c_oracle.quantize_scalar(float(t), q) for t in v], dtype=np.float32)
        np.testing.assert_array_equal(c, po.quantize(v, q))


def _round_to_f32(exact: Fraction) -> np.float32:
    c = np.float32(float(exact))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        err = abs(Fraction(float(cand)) - exact)
        key = (err, int(np.array(cand, dtype=np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return np.float32(best[1])


@pytest.mark.parametrize("quant", ("f32", "bf16"))
def test_c_forward_mirror_is_exactly_rounded(c_oracle, quant):
    bins, x, edges, iw, nb, w, b, _ = _case("ragged", 6, 4, n=64)
    out, idx = c_oracle.forward_f32(x, edges, iw, nb, w, bias=None, quant=quant)
    np.testing.assert_array_equal(idx, po.bin_indices(x, edges, nb))
    qw = po.quantize(w, quant)
    frac = po.fractions(x, edges, iw, idx.astype(np.int64))
    qf = po.quantize(frac, quant)
    for f in range(x.shape[1]):
        n = nb[f]
        pref = np.zeros((n, w.shape[2]), dtype=np.float32)
        acc = np.zeros(w.shape[2], dtype=np.float32)
        for k in range(n):
            pref[k] = acc
            p = w.shape[1] - 1 if k == n - 1 else k
            acc = (acc + qw[f, p]).astype(np.float32)
        for i in range(x.shape[0]):
            k = idx[i, f]
            p = w.shape[1] - 1 if k == n - 1 else k
            for j in range(w.shape[2]):
                exact = Fraction(float(qf[i, f])) * Fraction(float(qw[f, p, j])) + Fraction(float(pref[k, j]))
                r = _round_to_f32(exact)
                r = po.quantize(np.array([r], dtype=np.float32), quant)[0]
                assert out[i, f, j].view(np.uint32) == np.float32(r).view(np.uint32), (f, i, j)


def test_c_forward_matches_numpy_oracle(c_oracle):
    for case in BIN_CASE_NAMES:
        bins, x, edges, iw, nb, w, b, _ = _case(case, 15, 42)
        out, idx = c_oracle.forward_f32(x, edges, iw, nb, w, bias=b)
        ref, ridx, s = po.forward(x, edges, iw, nb, w, bias=b, return_abs=True)
        np.testing.assert_array_equal(idx, ridx)
        assert np.all(np.abs(out - ref) <= 1e-6 * s + 1e-7)


def test_c_backward_matches_numpy_oracle(c_oracle):
    for case in BIN_CASE_NAMES:
        for quant in ("f32", "bf16"):
            bins, x, edges, iw, nb, w, b, g = _case(case, 15, 42)
            _, idx = po.forward(x, edges, iw, nb, w, bias=b)
            ref = po.backward(g, x, edges, iw, nb, w, idx, quant=quant)
            got = c_oracle.backward_f64(g, x, edges, iw, nb, w, idx, quant=quant)
            for key in ("dx", "dw", "db", "dx_abs", "dw_abs", "db_abs"):
                np.testing.assert_allclose(got[key], ref[key], rtol=1e-10, atol=1e-12, err_msg=key)


# ---------------------------------------------------------------------------
# module tail (bias / ReLU / version-B linear0): closed form vs torch autograd
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case_name", BIN_CASE_NAMES)
@pytest.mark.parametrize("version,relu", [("A", False), ("A", True), ("B", False), ("B", True)])
def test_module_tail_matches_torch_autograd(case_name, version, relu):
    bins, x, edges, iw, nb, w, b, g = _case(case_name, 12, 31)
    rng = np.random.default_rng(5)
    f, d = w.shape[0], w.shape[2]
    w0 = rng.uniform(-0.4, 0.4, size=(f, d)).astype(np.float32)
    b0 = rng.uniform(-0.4, 0.4, size=(f, d)).astype(np.float32)
    tables = (edges, iw, nb)
    lin = (w0, b0) if version == "B" else None
    bias = b if version == "A" else None
    out, idx, pre = po.module_forward(x, tables, w, bias=bias, linear0=lin, activation=relu)
    passm = po.relu_pass(pre) if relu else None
    r = po.module_backward(g, x, tables, w, idx, pass_mask=passm, has_bias=version == "A", linear0=lin)

    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(_dense_w(w, nb), dtype=torch.float64, requires_grad=True)
    zero = torch.zeros((f, d), dtype=torch.float64)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True) if version == "A" else zero
    v = _torch_dense_forward(xt, bins, wt, bt)
    a = torch.relu(v) if relu else v
    if version == "B":
        w0t = torch.tensor(w0, dtype=torch.float64, requires_grad=True)
        b0t = torch.tensor(b0, dtype=torch.float64, requires_grad=True)
        a = torch.addcmul(b0t, w0t, xt[..., None]) + a
    a.backward(torch.tensor(g, dtype=torch.float64))
    np.testing.assert_allclose(out, a.detach().numpy(), rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(r["dx"], xt.grad.numpy(), rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(r["dw"], wt.grad.numpy(), rtol=2e-6, atol=2e-6)
    if version == "A":
        np.testing.assert_allclose(r["db"], bt.grad.numpy(), rtol=1e-12, atol=1e-12)
        assert "dlw" not in r
    else:
        assert "db" not in r
        np.testing.assert_allclose(r["dlw"], w0t.grad.numpy(), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(r["dlb"], b0t.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_pass_bits_pack_and_unpack():
    rng = np.random.default_rng(3)
    for d in (1, 10, 31, 32, 33, 64):
        passm = rng.random((5, 3, d)) < 0.5
        words = po.pack_pass_bits(passm)
        assert words.dtype == np.int32 and words.shape == (5, 3, (d + 31) // 32)
        np.testing.assert_array_equal(po.unpack_pass_bits(words, d), passm)
        # bit j of the row sits at bit j % 32 of word j // 32
        j = d - 1
        np.testing.assert_array_equal((words.view(np.uint32)[..., j // 32] >> (j % 32)) & 1, passm[..., j])
    assert po.relu_pass(np.array([np.nan, -0.0, 0.0, 1e-30, -1e-30])).tolist() == [True, False, False, True, False]


# ---------------------------------------------------------------------------
# dense encoding output: closed form vs the upstream dense formulation
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case_name", BIN_CASE_NAMES)
def test_encoding_closed_form_equals_dense(case_name):
    bins, x, edges, iw, nb, w, b, g = _case(case_name, 4, 41)
    enc, passm, width = po.dense_encoding(x, bins)
    real = ~np.isnan(width)                                  # [F, Bmax] real slots, in slot order
    dense = np.concatenate([enc[:, f, real[f]] for f in range(len(bins))], axis=1)
    closed = po.encoding_closed_form(x, edges, iw, nb)
    assert closed.shape == (x.shape[0], int(nb.sum()))
    np.testing.assert_allclose(closed, dense, rtol=1e-6, atol=1e-6)
    # the fp32 evaluation differs from the float64 one by the two roundings only
    c32 = po.encoding_closed_form(x, edges, iw, nb, dtype=np.float32)
    np.testing.assert_allclose(c32, closed, rtol=3e-7, atol=1e-7)


@pytest.mark.parametrize("case_name", BIN_CASE_NAMES)
def test_encoding_backward_equals_torch_autograd_of_dense(case_name):
    bins, x, edges, iw, nb, w, b, _ = _case(case_name, 4, 43)
    total = int(nb.sum())
    g = np.random.default_rng(7).standard_normal((x.shape[0], total))
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    eye = np.zeros((len(bins), edges.shape[1] - 1, total))
    offs = po.encoding_offsets(nb)
    _, width, _ = po.dense_layout(bins)
    for f in range(len(bins)):
        slots = np.flatnonzero(~np.isnan(width[f]))
        eye[f, slots, offs[f] + np.arange(len(slots))] = 1.0
    # the dense encoding, then a fixed 0/1 map that drops phantom slots and flattens
    left, width_t, single = po.dense_layout(bins)
    lt = torch.tensor(np.nan_to_num(left))
    wt = torch.tensor(np.nan_to_num(width_t, nan=1.0))
    raw = (xt[:, :, None] - lt[None]) / wt[None]
    bmax = left.shape[1]
    if bmax > 1:
        first = raw[..., :1].clamp_max(1.0)
        mid = raw[..., 1:-1].clamp(0.0, 1.0)
        last = raw[..., -1:]
        last = torch.where(torch.tensor(single)[None, :, None], last, last.clamp_min(0.0))
        enc = torch.cat([first, mid, last], dim=-1)
    else:
        enc = raw
    flat = torch.einsum("nfb,fbt->nt", enc, torch.tensor(eye))
    flat.backward(torch.tensor(g))
    dx, _ = po.encoding_backward(g, x, edges, iw, nb)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=2e-6, atol=2e-6)
