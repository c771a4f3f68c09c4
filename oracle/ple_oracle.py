"""CPU oracle for the fused piecewise-linear-embedding (PLE) path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this file;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker.

Everything here is a from-scratch NumPy restatement, computed in float64 unless
a function says otherwise.  Two independent formulations are kept on purpose:

* the *closed form* the fused operator evaluates (bin search, prefix of
  weights, one interpolated bin) -- ``bin_indices``, ``forward``,
  ``backward``;
* the *dense* upstream formulation (``rtdl_num_embeddings==0.0.12``,
  ``_PiecewiseLinearEncodingImpl`` + ``_NLinear``): an explicit [N, F, Bmax]
  encoding with first/middle/last clamps, then a per-feature matrix product --
  ``dense_encoding``, ``dense_forward``, ``dense_backward``.

The tests pin the closed form against the dense form on small inputs
(including exact edge hits, ragged and single-bin features), against
``np.searchsorted`` and against torch autograd of the dense form, so that a
dropped term, a wrong bin index or a transposed operand fails one of them.

Reference files followed (paths relative to the reference checkout):

* ``csrc/common.cuh:27-63``   right-sided bin search, clamp, NaN -> last bin
* ``csrc/common.cuh:66-78``   logical -> physical bin (last real bin lives at
  slot ``Bmax - 1``)
* ``csrc/common.cuh:81-96``   quantisation round trip through the output dtype
* ``csrc/forward_cuda.cu:135-178,208-283``  prefix of quantised weights and
  ``fma(q(frac), q(W[phys(k)]), prefix[k])``
* ``csrc/backward_cuda.cu:380-490``  dx with the internal-boundary double term
* ``csrc/backward_cuda.cu:170-336,889-923``  bucket / weighted histograms and
  the suffix over bins that produces dW
* ``src/rtdl_num_embeddings_cuda/module.py:58-131``  padded edges (+inf),
  inverse widths (``torch.reciprocal`` of the fp32 difference, 0-padded),
  ``n_bins`` int32
* ``src/rtdl_num_embeddings_cuda/module.py:230-248``  bias / ReLU / version-B
  epilogue
"""

from __future__ import annotations

import numpy as np

QUANT_KINDS = ("f32", "f16", "bf16")


# ----------------------------------------------------------------------------
# dtype helpers
# ----------------------------------------------------------------------------


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest, ties to even) and back.

    Restates the float -> bfloat16 conversion the reference uses through
    ``static_cast<c10::BFloat16>`` (``common.cuh:81-88``): add ``0x7FFF`` plus
    the lowest kept bit, truncate the low 16 bits; NaN stays NaN.
    """
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    bias = ((u >> 16) & 1) + 0x7FFF
    r = ((u + bias) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.float32(np.nan)
    return out


def quantize(a: np.ndarray, kind: str) -> np.ndarray:
    """Round-trip float32 values through the quantisation dtype.

    ``common.cuh:81-96``: ``quantize_to_float<output_t>`` -- identity for
    float32, a round trip through ``half`` / ``bfloat16`` otherwise.
    """
    a = np.asarray(a, dtype=np.float32)
    if kind == "f32":
        return a
    if kind == "f16":
        return a.astype(np.float16).astype(np.float32)
    if kind == "bf16":
        return bf16_round(a)
    raise ValueError(f"unknown quantisation kind {kind!r}")


def bin_index_dtype(max_n_bins: int) -> np.dtype:
    """``_meta.py:14-19``: uint8 up to 256 bins, int16 up to 32768, else int32."""
    if max_n_bins <= 256:
        return np.dtype(np.uint8)
    if max_n_bins <= 32768:
        return np.dtype(np.int16)
    return np.dtype(np.int32)


# ----------------------------------------------------------------------------
# bin tables (module.py:58-131)
# ----------------------------------------------------------------------------


def pad_bins(bins: list[np.ndarray]):
    """Build ``(bin_edges, inv_bin_widths, n_bins)`` from per-feature edges.

    ``module.py:74-131``: edges padded with +inf to ``[F, Bmax + 1]``; inverse
    widths = fp32 reciprocal of the fp32 edge difference, 0-padded to
    ``[F, Bmax]``; ``n_bins`` int32.
    """
    n_bins = np.array([len(e) - 1 for e in bins], dtype=np.int32)
    max_n_bins = int(n_bins.max())
    n_features = len(bins)
    edges = np.full((n_features, max_n_bins + 1), np.inf, dtype=np.float32)
    inv_w = np.zeros((n_features, max_n_bins), dtype=np.float32)
    for f, e in enumerate(bins):
        e32 = np.asarray(e, dtype=np.float32)
        edges[f, : e32.size] = e32
        width = (e32[1:] - e32[:-1]).astype(np.float32)
        with np.errstate(divide="ignore"):
            inv_w[f, : e32.size - 1] = (np.float32(1.0) / width).astype(np.float32)
    return edges, inv_w, n_bins


def physical_bin(k: np.ndarray, n_real: np.ndarray | int, max_n_bins: int) -> np.ndarray:
    """``common.cuh:66-78``: last real bin -> slot ``Bmax - 1``, others identity."""
    k = np.asarray(k)
    return np.where(k == np.asarray(n_real) - 1, max_n_bins - 1, k)


# ----------------------------------------------------------------------------
# closed form (what the fused operator computes)
# ----------------------------------------------------------------------------


def bin_indices(x: np.ndarray, bin_edges: np.ndarray, n_bins: np.ndarray) -> np.ndarray:
    """Logical bin per (sample, feature), int64 ``[N, F]``.

    ``common.cuh:27-63``: ``searchsorted(edges[:n + 1], v, right) - 1`` clamped
    to ``[0, n - 1]``.  NumPy orders NaN after every number, so a NaN query
    lands past the last edge and clamps to the last bin, as in the reference.
    """
    x = np.asarray(x, dtype=np.float32)
    n, f_count = x.shape
    out = np.empty((n, f_count), dtype=np.int64)
    for f in range(f_count):
        nf = int(n_bins[f])
        e = bin_edges[f, : nf + 1]
        k = np.searchsorted(e, x[:, f], side="right") - 1
        out[:, f] = np.clip(k, 0, nf - 1)
    return out


def fractions(x, bin_edges, inv_bin_widths, idx) -> np.ndarray:
    """fp32 position inside the bin, ``(x - e_k) * iw_k`` (``forward_cuda.cu:223-225``).

    Evaluated in float32 exactly as the kernel does (no fused multiply-add is
    possible in this expression), so quantised modes round the same value.
    """
    x = np.asarray(x, dtype=np.float32)
    f_idx = np.arange(x.shape[1])[None, :]
    e = bin_edges[f_idx, idx].astype(np.float32)
    iw = inv_bin_widths[f_idx, idx].astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        return ((x - e).astype(np.float32) * iw).astype(np.float32)


def prefix_table(weight: np.ndarray, n_bins: np.ndarray, quant: str = "f32") -> np.ndarray:
    """float64 ``cumW[f, k, :] = sum_{j<k} q(W[f, phys(j), :])`` for logical k.

    ``forward_cuda.cu:135-178``.  Rows ``k >= n_f`` are unused and left 0.
    """
    f_count, max_n_bins, d = weight.shape
    qw = quantize(weight, quant).astype(np.float64)
    cum = np.zeros((f_count, max_n_bins, d), dtype=np.float64)
    for f in range(f_count):
        nf = int(n_bins[f])
        # j < k <= nf - 1, so phys(j) == j for every prefix term.
        if nf > 1:
            cum[f, 1:nf] = np.cumsum(qw[f, : nf - 1], axis=0)
    return cum


def forward(x, bin_edges, inv_bin_widths, n_bins, weight, bias=None, quant="f32",
            return_abs=False):
    """Closed-form forward in float64.

    ``out[n, f] = sum_{j<k} q(W[f, j]) + q(frac) * q(W[f, phys(k)]) (+ b[f])``
    with ``k`` from :func:`bin_indices` (``forward_cuda.cu:97-131,188-285``).
    The first bin is unclamped below and the last bin unclamped above because
    ``k`` clamps while ``frac`` does not.  ``bias`` is added after the
    quantised term, as ``module.py:238-239`` adds it to ``x_ple``.

    Returns ``(out, idx)`` or, with ``return_abs``, ``(out, idx, abs_sum)``
    where ``abs_sum`` bounds the magnitude of the summed terms (used to scale
    the relative tolerance of a differently ordered fp32 sum).
    """
    x = np.asarray(x, dtype=np.float32)
    f_count, max_n_bins, d = weight.shape
    idx = bin_indices(x, bin_edges, n_bins)
    frac = fractions(x, bin_edges, inv_bin_widths, idx)
    qf = quantize(frac, quant).astype(np.float64)
    qw = quantize(weight, quant).astype(np.float64)
    cum = prefix_table(weight, n_bins, quant)
    f_idx = np.arange(f_count)[None, :]
    phys = physical_bin(idx, n_bins[None, :], max_n_bins)
    w_k = qw[f_idx, phys]                       # [N, F, d]
    cum_k = cum[f_idx, idx]                     # [N, F, d]
    with np.errstate(invalid="ignore", over="ignore"):
        out = cum_k + qf[..., None] * w_k
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float64)[None]
    if not return_abs:
        return out, idx
    abs_cum = np.zeros_like(cum)
    for f in range(f_count):
        nf = int(n_bins[f])
        if nf > 1:
            abs_cum[f, 1:nf] = np.cumsum(np.abs(qw[f, : nf - 1]), axis=0)
    with np.errstate(invalid="ignore", over="ignore"):
        abs_sum = abs_cum[f_idx, idx] + np.abs(qf[..., None] * w_k)
    if bias is not None:
        abs_sum = abs_sum + np.abs(np.asarray(bias, dtype=np.float64))[None]
    return out, idx, abs_sum


def backward(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, idx, quant="f32",
             grad_bias_source=None):
    """Closed-form backward in float64.  Returns a dict.

    * ``dx[n, f] = iw_k * <g, q(W[f, phys(k)])>`` plus, when ``k > 0`` and
      ``x == e_k`` exactly, ``iw_{k-1} * <g, q(W[f, k-1])>``
      (``backward_cuda.cu:380-490``).
    * ``dW[f, phys(k)] = sum_{bin=k} q(frac) g + sum_{bin>k} g``; padded slots
      stay 0 (``backward_cuda.cu:170-336,889-923``).
    * ``db[f] = sum_n g`` (autograd of ``x_ple + bias``, ``module.py:238-239``),
      taken from ``grad_bias_source`` when given (the unquantised gradient in
      autocast mode), else from ``grad_output``.

    ``grad_output`` is used as given (already in the dtype the operator sees);
    ``q`` rounds ``frac`` and ``W`` through ``quant`` like the forward.  Each
    result comes with an ``*_abs`` companion: the sum of absolute values of its
    terms, which scales the tolerance of an fp32 reduction.
    """
    g = np.asarray(grad_output, dtype=np.float64)
    x = np.asarray(x, dtype=np.float32)
    n, f_count = x.shape
    _, max_n_bins, d = weight.shape
    idx = np.asarray(idx, dtype=np.int64)
    frac = fractions(x, bin_edges, inv_bin_widths, idx)
    qf = quantize(frac, quant).astype(np.float64)
    qw = quantize(weight, quant).astype(np.float64)
    f_idx = np.arange(f_count)[None, :]
    phys = physical_bin(idx, n_bins[None, :], max_n_bins)
    iw_k = inv_bin_widths[f_idx, idx].astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        t = g * qw[f_idx, phys]
        dx = t.sum(-1) * iw_k
        dx_abs = np.abs(t).sum(-1) * np.abs(iw_k)
        e_k = bin_edges[f_idx, idx]
        boundary = (idx > 0) & (x == e_k)
        if boundary.any():
            km1 = np.maximum(idx - 1, 0)
            iw_p = inv_bin_widths[f_idx, km1].astype(np.float64)
            t2 = g * qw[f_idx, km1]
            dx = dx + np.where(boundary, t2.sum(-1) * iw_p, 0.0)
            dx_abs = dx_abs + np.where(boundary, np.abs(t2).sum(-1) * np.abs(iw_p), 0.0)

    bucket = np.zeros((f_count, max_n_bins, d))
    weighted = np.zeros((f_count, max_n_bins, d))
    bucket_abs = np.zeros((f_count, max_n_bins, d))
    weighted_abs = np.zeros((f_count, max_n_bins, d))
    for f in range(f_count):
        np.add.at(bucket[f], idx[:, f], g[:, f])
        np.add.at(bucket_abs[f], idx[:, f], np.abs(g[:, f]))
        wg = qf[:, f, None] * g[:, f]
        np.add.at(weighted[f], idx[:, f], wg)
        np.add.at(weighted_abs[f], idx[:, f], np.abs(wg))
    dw = np.zeros((f_count, max_n_bins, d))
    dw_abs = np.zeros((f_count, max_n_bins, d))
    for f in range(f_count):
        nf = int(n_bins[f])
        future = np.zeros(d)
        future_abs = np.zeros(d)
        for k in range(nf - 1, -1, -1):
            p = max_n_bins - 1 if k == nf - 1 else k
            dw[f, p] = weighted[f, k] + future
            dw_abs[f, p] = weighted_abs[f, k] + future_abs
            future = future + bucket[f, k]
            future_abs = future_abs + bucket_abs[f, k]
    gb = g if grad_bias_source is None else np.asarray(grad_bias_source, dtype=np.float64)
    db = gb.sum(0)
    db_abs = np.abs(gb).sum(0)
    return {
        "dx": dx, "dx_abs": dx_abs,
        "dw": dw, "dw_abs": dw_abs,
        "db": db, "db_abs": db_abs,
        "bucket": bucket, "weighted": weighted,
    }


# ----------------------------------------------------------------------------
# dense upstream formulation (rtdl_num_embeddings==0.0.12, restated)
# ----------------------------------------------------------------------------


def dense_layout(bins: list[np.ndarray]):
    """Per-component slope/offset/role tables of the upstream dense encoding.

    Upstream ``_PiecewiseLinearEncodingImpl`` keeps, per feature, ``Bmax``
    components: the first ``n_f - 1`` real bins at slots ``0 .. n_f - 2``, the
    last real bin at slot ``Bmax - 1``, zero (phantom) components between.
    Returns float64 ``left[F, Bmax]``, ``width[F, Bmax]`` (NaN for phantom
    slots) and ``single[F]`` (feature has exactly one bin).
    """
    n_bins = [len(e) - 1 for e in bins]
    max_n_bins = max(n_bins)
    f_count = len(bins)
    left = np.full((f_count, max_n_bins), np.nan)
    width = np.full((f_count, max_n_bins), np.nan)
    for f, e in enumerate(bins):
        e64 = np.asarray(e, dtype=np.float32).astype(np.float64)
        nf = n_bins[f]
        for k in range(nf):
            p = max_n_bins - 1 if k == nf - 1 else k
            left[f, p] = e64[k]
            width[f, p] = e64[k + 1] - e64[k]
    single = np.array([nf == 1 for nf in n_bins])
    return left, width, single


def dense_encoding(x: np.ndarray, bins: list[np.ndarray]):
    """Upstream dense encoding in float64.  Returns ``(enc, pass_mask, width)``.

    Component value ``(x - left) / width``; slot 0 is clamped above at 1, middle
    slots to ``[0, 1]``, slot ``Bmax - 1`` below at 0 (not at all for a
    single-bin feature); with ``Bmax == 1`` nothing is clamped.  Phantom slots
    are 0.  ``pass_mask`` marks where the clamp lets the gradient through
    (torch's clamp backward is inclusive at both bounds).
    """
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    left, width, single = dense_layout(bins)
    f_count, max_n_bins = left.shape
    with np.errstate(invalid="ignore", divide="ignore"):
        raw = (x[:, :, None] - left[None]) / width[None]
    enc = raw.copy()
    passm = np.ones_like(raw, dtype=bool)
    if max_n_bins > 1:
        lo = np.full(max_n_bins, 0.0)
        hi = np.full(max_n_bins, 1.0)
        lo[0] = -np.inf
        hi[-1] = np.inf
        lo_b = np.broadcast_to(lo, raw.shape).copy()
        hi_b = np.broadcast_to(hi, raw.shape).copy()
        # single-bin features: the last slot is not clamped at all
        lo_b[:, single, -1] = -np.inf
        enc = np.minimum(np.maximum(raw, lo_b), hi_b)
        passm = (raw >= lo_b) & (raw <= hi_b)
    phantom = np.isnan(width)[None].repeat(x.shape[0], 0)
    enc = np.where(phantom, 0.0, enc)
    passm = np.where(phantom, False, passm)
    return enc, passm, width


def dense_forward(x, bins, weight, bias=None):
    """Upstream dense forward in float64: ``enc @ W (+ b)`` per feature."""
    enc, _, _ = dense_encoding(x, bins)
    out = np.einsum("nfb,fbd->nfd", enc, np.asarray(weight, dtype=np.float64))
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float64)[None]
    return out


def dense_backward(grad_output, x, bins, weight):
    """Explicit Jacobian of :func:`dense_forward` in float64.

    ``dW = sum_n enc^T g``, ``db = sum_n g``,
    ``dx = sum_b <g, W_b> / width_b * pass_b``.
    """
    g = np.asarray(grad_output, dtype=np.float64)
    enc, passm, width = dense_encoding(x, bins)
    w64 = np.asarray(weight, dtype=np.float64)
    dw = np.einsum("nfb,nfd->fbd", enc, g)
    denc = np.einsum("nfd,fbd->nfb", g, w64)
    with np.errstate(invalid="ignore", divide="ignore"):
        inv = np.where(np.isnan(width), 0.0, 1.0 / width)
    dx = (denc * inv[None] * passm).sum(-1)
    db = g.sum(0)
    return {"dx": dx, "dw": dw, "db": db}


# ----------------------------------------------------------------------------
# module-level epilogue (module.py:230-248)
# ----------------------------------------------------------------------------


def module_forward(x, bins_tables, weight, bias=None, linear0=None, activation=False,
                   quant="f32"):
    """Module output in float64: PLE branch (+bias), ReLU, version-B residual.

    ``linear0 = (w0[F, d], b0[F, d])`` gives ``x_linear = b0 + w0 * x``
    (upstream ``LinearEmbeddings``).  Returns ``(out, idx, pre_activation)``.
    """
    edges, iw, n_bins = bins_tables
    pre, idx = forward(x, edges, iw, n_bins, weight, bias=bias, quant=quant)
    out = np.maximum(pre, 0.0) if activation else pre
    if linear0 is not None:
        w0, b0 = linear0
        x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
        out = out + (np.asarray(b0, np.float64)[None] + np.asarray(w0, np.float64)[None] * x64[..., None])
    return out, idx, pre


def relu_pass(pre: np.ndarray) -> np.ndarray:
    """Where torch.relu passes its input's gradient: ``not (v <= 0)`` (NaN passes)."""
    with np.errstate(invalid="ignore"):
        return ~(np.asarray(pre) <= 0)


def pack_pass_bits(passm: np.ndarray) -> np.ndarray:
    """[N, F, D] bool -> int32 [N, F, ceil(D / 32)]: bit j % 32 of word j // 32."""
    n, f, d = passm.shape
    words = (d + 31) // 32
    out = np.zeros((n, f, words), dtype=np.uint32)
    for j in range(d):
        out[:, :, j // 32] |= passm[:, :, j].astype(np.uint32) << np.uint32(j % 32)
    return out.view(np.int32)


def unpack_pass_bits(words: np.ndarray, d: int) -> np.ndarray:
    w = np.asarray(words).view(np.uint32)
    return np.stack([((w[:, :, j // 32] >> np.uint32(j % 32)) & 1).astype(bool) for j in range(d)], axis=-1)


def module_backward(grad_output, x, bins_tables, weight, idx, pass_mask=None, has_bias=True, linear0=None,
                    quant="f32"):
    """Gradients of :func:`module_forward` in float64 (``module.py:230-248``).

    ``g_v = g * pass`` behind a ReLU; the PLE branch sees ``q(g_v)`` (fp32 then
    ``quant``, as autograd casts the gradient to ``x_ple``'s dtype) and
    :func:`backward` gives dx / dW; version A's bias gradient is ``sum_n g_v``;
    version B adds ``dx += <g, w0>``, ``d w0 = sum_n g x``, ``d b0 = sum_n g``.
    Every result has an ``*_abs`` companion (sum of |terms|).
    """
    edges, iw, n_bins = bins_tables
    g = np.asarray(grad_output, dtype=np.float64)
    gv = g if pass_mask is None else np.where(pass_mask, g, 0.0)
    gq = quantize(gv.astype(np.float32), quant)
    r = backward(gq, x, edges, iw, n_bins, weight, idx, quant=quant, grad_bias_source=gv)
    if linear0 is None:
        if not has_bias:
            del r["db"], r["db_abs"]
        return r
    del r["db"], r["db_abs"]
    w0, _b0 = linear0
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
    t = g * np.asarray(w0, dtype=np.float64)[None]
    r["dx"] = r["dx"] + t.sum(-1)
    r["dx_abs"] = r["dx_abs"] + np.abs(t).sum(-1)
    gx = g * x64[..., None]
    r["dlw"], r["dlw_abs"] = gx.sum(0), np.abs(gx).sum(0)
    r["dlb"], r["dlb_abs"] = g.sum(0), np.abs(g).sum(0)
    return r


# ----------------------------------------------------------------------------
# dense encoding output (upstream PiecewiseLinearEncoding), closed form
# ----------------------------------------------------------------------------


def encoding_offsets(n_bins) -> np.ndarray:
    nb = np.asarray(n_bins, dtype=np.int64)
    return np.concatenate([[0], np.cumsum(nb)[:-1]]).astype(np.int64)


def encoding_closed_form(x, bin_edges, inv_bin_widths, n_bins, dtype=np.float64):
    """``[N, sum n_f]``: per feature ``1`` below the active bin, ``frac`` at it,
    ``0`` above; NaN x gives NaN components.  ``dtype=np.float32`` evaluates
    ``frac = (x - e_b) * iw_b`` with two fp32 roundings, the kernel's
    arithmetic; float64 gives the exact value of the same expression."""
    x = np.asarray(x, dtype=np.float32)
    n, f_count = x.shape
    idx = bin_indices(x, bin_edges, n_bins)
    f_idx = np.arange(f_count)[None, :]
    with np.errstate(invalid="ignore", over="ignore"):
        if dtype == np.float32:
            frac = (x - bin_edges[f_idx, idx]).astype(np.float32) * inv_bin_widths[f_idx, idx]
        else:
            frac = (x.astype(np.float64) - bin_edges[f_idx, idx].astype(np.float64)) * \
                inv_bin_widths[f_idx, idx].astype(np.float64)
    offs = encoding_offsets(n_bins)
    total = int(np.sum(n_bins))
    out = np.zeros((n, total), dtype=dtype)
    for f in range(f_count):
        nf = int(n_bins[f])
        k = np.arange(nf)[None, :]
        b = idx[:, f:f + 1]
        val = np.where(k < b, 1.0, np.where(k == b, frac[:, f:f + 1], 0.0))
        val = np.where(np.isnan(x[:, f:f + 1]), np.nan, val)
        out[:, offs[f]:offs[f] + nf] = val
    return out


def encoding_backward(grad_output, x, bin_edges, inv_bin_widths, n_bins):
    """``dx[n, f] = g[off_f + b] iw_b (+ g[off_f + b - 1] iw_{b-1} if b > 0 and
    x == e_b)`` in float64, with the sum of |terms|."""
    g = np.asarray(grad_output, dtype=np.float64)
    x = np.asarray(x, dtype=np.float32)
    n, f_count = x.shape
    idx = bin_indices(x, bin_edges, n_bins)
    offs = encoding_offsets(n_bins)
    rows = np.arange(n)
    dx = np.zeros((n, f_count))
    dx_abs = np.zeros((n, f_count))
    for f in range(f_count):
        b = idx[:, f]
        t = g[rows, offs[f] + b] * inv_bin_widths[f, b].astype(np.float64)
        edge = (b > 0) & (x[:, f] == bin_edges[f, b])
        bm = np.maximum(b - 1, 0)
        t2 = np.where(edge, g[rows, offs[f] + bm] * inv_bin_widths[f, bm].astype(np.float64), 0.0)
        dx[:, f] = t + t2
        dx_abs[:, f] = np.abs(t) + np.abs(t2)
    return dx, dx_abs
