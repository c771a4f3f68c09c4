"""Bin-edge preparation (``compute_bins``, ``bin_tables``) on the CPU.

``compute_bins`` restates upstream ``rtdl_num_embeddings.compute_bins``
(``rtdl_num_embeddings==0.0.12``, not installed here): the reference holds no
vectors for it, so it is pinned against independent routes -- NumPy quantiles
with ``np.unique`` for the quantile bins, a separately fitted scikit-learn tree
read through another field (split nodes are the ones with ``feature >= 0``)
for the tree bins -- and against the properties the algorithm fixes (edges
start at the minimum and end at the maximum, are strictly increasing, repeated
quantiles collapse).  Upstream's exact error texts are "parity unpinned".
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ple_oracle as po
from piecewiselinearembeddings_optimized_amd.bins import bin_tables, check_bins, compute_bins


def _mixed(n=6000, seed=0):
    rng = np.random.default_rng(seed)
    cols = [
        rng.standard_normal(n),
        rng.lognormal(0.0, 1.0, n),
        rng.uniform(-5, 5, n),
        rng.poisson(3.0, n).astype(np.float64),       # discrete: quantiles repeat
        np.where(rng.random(n) < 0.9, 0.0, 1.0),      # two values: one bin
    ]
    return torch.tensor(np.stack(cols, 1), dtype=torch.float32)


def test_quantile_bins_match_numpy_quantiles():
    X = _mixed()
    with pytest.warns(UserWarning, match="Feature 4 has just two bin edges"):
        bins = compute_bins(X, n_bins=48)
    assert len(bins) == X.shape[1]
    for j, b in enumerate(bins):
        col = X[:, j].numpy().astype(np.float64)
        ref = np.unique(np.quantile(col, np.linspace(0.0, 1.0, 49)).astype(np.float32))
        assert b.dtype == torch.float32 and b.ndim == 1
        assert b.numel() == ref.size, j
        np.testing.assert_allclose(b.numpy(), ref, rtol=2e-6, atol=1e-6)
        assert float(b[0]) == float(col.min()) and float(b[-1]) == float(col.max())
        assert bool((b[1:] > b[:-1]).all())
    # continuous columns keep all 48 bins; the discrete ones collapse
    assert [b.numel() - 1 for b in bins[:3]] == [48, 48, 48]
    assert bins[3].numel() - 1 < 48
    assert bins[4].tolist() == [0.0, 1.0]


def test_quantile_bins_of_integers_are_exact():
    X = torch.tensor(np.random.default_rng(1).poisson(3.0, (4000, 2)), dtype=torch.float32)
    for j, b in enumerate(compute_bins(X, n_bins=16)):
        ref = np.unique(np.quantile(X[:, j].numpy().astype(np.float64), np.linspace(0, 1, 17)))
        np.testing.assert_array_equal(b.numpy(), ref.astype(np.float32))


@pytest.mark.parametrize("regression", [True, False])
def test_tree_bins_are_min_max_and_split_thresholds(regression):
    from sklearn.tree import DecisionTreeClassifier, DecisionTreeRegressor

    rng = np.random.default_rng(2)
    X = torch.tensor(rng.standard_normal((3000, 3)), dtype=torch.float32)
    signal = np.sin(3 * X[:, 0].numpy()) + X[:, 1].numpy() ** 2
    y = torch.tensor(signal if regression else (signal > np.median(signal)).astype(np.int64))
    kw = {"random_state": 0, "min_samples_leaf": 20}
    bins = compute_bins(X, n_bins=12, tree_kwargs=kw, y=y, regression=regression)
    est = DecisionTreeRegressor if regression else DecisionTreeClassifier
    for j, b in enumerate(bins):
        col = X[:, j].numpy()
        t = est(max_leaf_nodes=12, **kw).fit(col.reshape(-1, 1), y.numpy()).tree_
        thresholds = t.threshold[t.feature >= 0]
        ref = torch.as_tensor([float(col.min()), float(col.max())] + [float(v) for v in thresholds]).unique()
        assert torch.equal(b, ref.to(torch.float32)), j
        assert b.numel() - 1 <= 12 and b.numel() >= 2
        assert bool((b[1:] > b[:-1]).all())


def test_compute_bins_argument_errors():
    X = _mixed(200)[:, :3]
    with pytest.raises(ValueError, match="two dimensions"):
        compute_bins(X[:, 0])
    with pytest.raises(ValueError, match="at least two rows"):
        compute_bins(X[:1], n_bins=2)
    with pytest.raises(ValueError, match="nan/inf"):
        Xn = X.clone()
        Xn[3, 1] = float("nan")
        compute_bins(Xn)
    with pytest.raises(ValueError, match="two distinct values"):
        Xc = X.clone()
        Xc[:, 2] = 1.5
        compute_bins(Xc)
    with pytest.raises(ValueError, match="n_bins must be more than 1"):
        compute_bins(X, n_bins=1)
    with pytest.raises(ValueError, match="n_bins must be more than 1"):
        compute_bins(X, n_bins=200)
    with pytest.raises(ValueError, match="If tree_kwargs is None"):
        compute_bins(X, y=torch.zeros(200))
    with pytest.raises(ValueError, match="y and regression must not be None"):
        compute_bins(X, tree_kwargs={})
    with pytest.raises(ValueError, match="max_leaf_nodes"):
        compute_bins(X, tree_kwargs={"max_leaf_nodes": 3}, y=torch.zeros(200), regression=True)
    with pytest.raises(ValueError, match="len\\(y\\)"):
        compute_bins(X, tree_kwargs={}, y=torch.zeros(100), regression=True)


def test_check_bins_rejects_bad_edges():
    with pytest.raises(ValueError, match="must not be empty"):
        check_bins([])
    with pytest.raises(ValueError, match="at least two bin edges"):
        check_bins([torch.tensor([1.0])])
    with pytest.raises(ValueError, match="strictly increasing"):
        check_bins([torch.tensor([0.0, 1.0, 1.0])])
    with pytest.raises(ValueError, match="nan/inf"):
        check_bins([torch.tensor([0.0, float("inf")])])


def test_bin_tables_match_oracle_and_module_buffers():
    from piecewiselinearembeddings_optimized_amd import CudaPiecewiseLinearEmbeddings

    X = _mixed(3000, seed=4)[:, :4]
    bins = compute_bins(X, n_bins=24)
    edges, inv_w, nb = bin_tables(bins)
    e_ref, iw_ref, nb_ref = po.pad_bins([b.numpy() for b in bins])
    np.testing.assert_array_equal(edges.numpy(), e_ref)
    np.testing.assert_array_equal(inv_w.numpy().view(np.uint32), iw_ref.view(np.uint32))
    np.testing.assert_array_equal(nb.numpy(), nb_ref)
    m = CudaPiecewiseLinearEmbeddings(bins, 8, activation=False, version="B")
    assert torch.equal(m._cuda_bin_edges, edges)
    assert torch.equal(m._cuda_inv_bin_widths, inv_w)
    assert torch.equal(m._cuda_n_bins, nb)
