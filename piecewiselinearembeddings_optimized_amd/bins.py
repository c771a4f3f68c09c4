"""Bin-edge preparation: the step that produces ``bins`` for the module, and
the padded per-feature tables the kernels read.

``compute_bins`` restates the published algorithm of the upstream
``rtdl_num_embeddings.compute_bins`` (package ``rtdl_num_embeddings==0.0.12``,
pinned by the reference's ``requirements.txt:1`` / ``pyproject.toml:17``; the
reference calls it from ``tests/test_ple_cuda_benchmark.py`` and feeds its
output to ``CudaPiecewiseLinearEmbeddings``).  That package is not part of the
reference checkout and is not installed here, so this is a restatement of its
documented behaviour, not a copy:

* quantile bins (``tree_kwargs=None``): per column, ``torch.quantile`` at
  ``linspace(0, 1, n_bins + 1)``, then ``unique`` -- repeated quantiles
  (discrete or heavy-tailed features) collapse, leaving fewer bins, down to
  one;
* tree bins (``tree_kwargs`` given): per column, a scikit-learn decision tree
  (regressor or classifier, ``max_leaf_nodes=n_bins``) is fitted to ``y``; the
  edges are the column's min and max plus every split threshold, ``unique``;
* both end with the upstream validation of bins (``check_bins``).

``bin_tables`` builds ``(bin_edges, inv_bin_widths, n_bins)`` exactly as the
reference module's constructor does (``module.py:74-131``): edges padded with
+inf to ``[F, Bmax + 1]``, inverse widths as ``torch.reciprocal`` of the fp32
edge difference padded with 0 to ``[F, Bmax]``, ``n_bins`` int32.
"""

from __future__ import annotations

import warnings
from typing import Any

import torch
from torch import Tensor

__all__ = ["bin_tables", "check_bins", "compute_bins"]


def check_bins(bins: list[Tensor]) -> None:
    """Validate per-feature bin edges (upstream ``_check_bins``)."""
    if not bins:
        raise ValueError("The list of bins must not be empty")
    for i, feature_bins in enumerate(bins):
        if not isinstance(feature_bins, Tensor):
            raise ValueError(f"bins must be a list of PyTorch tensors; bins[{i}] is {type(feature_bins)}")
        if feature_bins.ndim != 1:
            raise ValueError(f"Each item of the bin list must have exactly one dimension; bins[{i}].ndim={feature_bins.ndim}")
        if len(feature_bins) < 2:
            raise ValueError(f"All features must have at least two bin edges; len(bins[{i}])={len(feature_bins)}")
        if not feature_bins.isfinite().all():
            raise ValueError(f"Bin edges must not contain nan/inf/-inf; this is not true for feature {i}")
        if (feature_bins[:-1] >= feature_bins[1:]).any():
            raise ValueError(f"Bin edges must be sorted (strictly increasing); this is not true for feature {i}")
        if len(feature_bins) == 2:
            warnings.warn(
                f"Feature {i} has just two bin edges, i.e. a single bin; its piecewise-linear encoding "
                "is the same as min-max scaling"
            )


# torch.quantile refuses inputs longer than this (upstream warns about it)
_QUANTILE_MAX_ROWS = 2**24


def _check_x(X: Tensor, n_bins: int) -> None:
    if not isinstance(X, Tensor):
        raise ValueError(f"X must be a PyTorch tensor, however: type(X)={type(X)}")
    if X.ndim != 2:
        raise ValueError(f"X must have exactly two dimensions, however: X.ndim={X.ndim}")
    if X.shape[0] < 2:
        raise ValueError(f"X must have at least two rows, however: X.shape[0]={X.shape[0]}")
    if X.shape[1] < 1:
        raise ValueError(f"X must have at least one column, however: X.shape[1]={X.shape[1]}")
    if not bool(X.isfinite().all()):
        raise ValueError("X must not contain nan/inf/-inf.")
    if bool((X == X[0]).all(dim=0).any()):
        raise ValueError(
            "All columns of X must have at least two distinct values."
            " However, X contains columns with just one distinct value."
        )
    if n_bins <= 1 or n_bins >= len(X):
        raise ValueError(f"n_bins must be more than 1, but less than len(X), however: n_bins={n_bins}, len(X)={len(X)}")


def compute_bins(
    X: Tensor,
    n_bins: int = 48,
    *,
    tree_kwargs: dict[str, Any] | None = None,
    y: Tensor | None = None,
    regression: bool | None = None,
    verbose: bool = False,
) -> list[Tensor]:
    """Per-feature bin edges for ``CudaPiecewiseLinearEmbeddings``.

    ``X`` is ``[n_objects, n_features]`` (any device); the result is a list of
    ``n_features`` strictly increasing 1-D tensors with at least two edges
    each, on ``X``'s device and dtype.  See the module docstring for the two
    algorithms.
    """
    _check_x(X, n_bins)
    if tree_kwargs is None:
        if y is not None or regression is not None or verbose:
            raise ValueError(
                "If tree_kwargs is None, then y must be None, regression must be None and verbose must be False"
            )
        if len(X) > _QUANTILE_MAX_ROWS:
            warnings.warn(
                f"Computing quantile-based bins for more than {_QUANTILE_MAX_ROWS} objects may fail in"
                " torch.quantile; subsample the data (e.g. X = X[:2**24]) to avoid it."
            )
        levels = torch.linspace(0.0, 1.0, n_bins + 1, dtype=X.dtype, device=X.device)
        quantiles = torch.quantile(X, levels, dim=0)           # [n_bins + 1, n_features]
        bins = [column.unique() for column in quantiles.T]
        check_bins(bins)
        return bins

    try:
        from sklearn import tree as sklearn_tree
    except ImportError as e:  # pragma: no cover - scikit-learn is present in this image
        raise RuntimeError("tree-based bins need scikit-learn") from e
    if y is None or regression is None:
        raise ValueError("If tree_kwargs is not None, then y and regression must not be None")
    if y.ndim != 1:
        raise ValueError(f"y must have exactly one dimension, however: y.ndim={y.ndim}")
    if len(y) != len(X):
        raise ValueError(f"len(y) must be equal to len(X), however: len(y)={len(y)}, len(X)={len(X)}")
    if "max_leaf_nodes" in tree_kwargs:
        raise ValueError('tree_kwargs must not contain the key "max_leaf_nodes" (it is set to n_bins).')
    if X.device.type != "cpu" or y.device.type != "cpu":
        warnings.warn(
            "Computing tree-based bins converts the inputs to NumPy arrays; the tensors are not on the CPU,"
            " so the conversion has some overhead.",
            UserWarning,
        )
    columns = X.detach().cpu().numpy().T
    target = y.detach().cpu().numpy()
    estimator = sklearn_tree.DecisionTreeRegressor if regression else sklearn_tree.DecisionTreeClassifier
    if verbose:
        try:
            from tqdm import tqdm

            columns_iter = tqdm(columns)
        except ImportError as e:
            raise ImportError("If verbose is True, tqdm must be installed") from e
    else:
        columns_iter = columns
    bins = []
    for column in columns_iter:
        fitted = estimator(max_leaf_nodes=n_bins, **tree_kwargs).fit(column.reshape(-1, 1), target).tree_
        edges = [float(column.min()), float(column.max())]
        # split nodes are the ones whose children differ (leaves have -1 / -1)
        split = fitted.children_left != fitted.children_right
        edges.extend(float(t) for t in fitted.threshold[split])
        bins.append(torch.as_tensor(edges).unique())
    check_bins(bins)
    return [b.to(device=X.device, dtype=X.dtype) for b in bins]


def bin_tables(bins: list[Tensor], device: torch.device | str | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """``(bin_edges fp32 [F, Bmax + 1], inv_bin_widths fp32 [F, Bmax], n_bins int32 [F])``.

    Same construction as the reference module (``module.py:74-131``): the
    fp32 edges of feature f fill ``bin_edges[f, :n_f + 1]`` and +inf the rest;
    ``inv_bin_widths[f, :n_f] = reciprocal(e[1:] - e[:-1])`` in fp32 and 0 the
    rest.
    """
    n_bins_list = [int(e.numel() - 1) for e in bins]
    max_n_bins = max(n_bins_list)
    device = bins[0].device if device is None else torch.device(device)
    n_features = len(bins)
    edges = torch.full((n_features, max_n_bins + 1), torch.inf, dtype=torch.float32, device=device)
    inv_w = torch.zeros((n_features, max_n_bins), dtype=torch.float32, device=device)
    for i, e in enumerate(bins):
        e32 = e.to(device=device, dtype=torch.float32)
        edges[i, : e32.numel()].copy_(e32)
        inv_w[i, : e32.numel() - 1].copy_(torch.reciprocal(e32[1:] - e32[:-1]))
    n_bins = torch.tensor(n_bins_list, dtype=torch.int32, device=device)
    return edges, inv_w, n_bins
