"""Pins of the exact-KNN oracle (oracle/knn_oracle.py) on the CPU.

The oracle restates the ordering of tests/testthat/helper-knn.R:5-38 of the
reference (per-row order of the squared distances, ties by index, the row
itself excluded or at distance 0).  It is checked here against an
independent implementation (scipy's cKDTree), against a pure-Python brute
force on inputs with duplicates and exact lattice ties, and against the
invariants any exact KNN has.
"""

from __future__ import annotations

import numpy as np
import pytest
from scipy.spatial import cKDTree

from oracle import knn_oracle


def _lattice(n, d, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, 3, size=(n, d)).astype(np.float64)


@pytest.mark.parametrize("n,d,k", [(500, 7, 10), (1200, 50, 30), (300, 1, 5)])
def test_matches_kdtree_on_tie_free_data(n, d, k):
    rng = np.random.default_rng(n + d)
    x = rng.normal(size=(n, d))
    idx, dist = knn_oracle.exact_knn(x, k)
    tree_d, tree_i = cKDTree(x).query(x, k=k + 1)
    assert np.all(tree_i[:, 0] == np.arange(n))  # the point itself first (no duplicates)
    np.testing.assert_array_equal(idx, tree_i[:, 1:])
    np.testing.assert_allclose(dist, tree_d[:, 1:], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("exclude_self", [True, False])
@pytest.mark.parametrize("n,d,k,seed", [(40, 3, 7, 1), (57, 2, 12, 2), (25, 5, 24, 3)])
def test_matches_brute_force_with_ties(n, d, k, seed, exclude_self):
    x = _lattice(n, d, seed)  # few distinct distances: many exact ties, some duplicate rows
    if k > n - (1 if exclude_self else 0):
        k = n - (1 if exclude_self else 0)
    idx, dist = knn_oracle.exact_knn(x, k, exclude_self=exclude_self, margin=2)
    bi, bd = knn_oracle.brute_force_knn(x, k, exclude_self=exclude_self)
    np.testing.assert_array_equal(idx, bi)
    np.testing.assert_allclose(dist, bd, rtol=0, atol=1e-12)


def test_duplicates_order_by_index_and_self_handling():
    x = np.zeros((6, 2))
    x[3:] = 1.0
    idx, dist = knn_oracle.exact_knn(x, 2, exclude_self=True)
    np.testing.assert_array_equal(idx[0], [1, 2])
    np.testing.assert_array_equal(idx[4], [3, 5])
    assert np.all(dist == 0.0)
    idx, _ = knn_oracle.exact_knn(x, 2, exclude_self=False)
    np.testing.assert_array_equal(idx[1], [0, 1])  # itself competes at distance 0, ties by index
    np.testing.assert_array_equal(idx[5], [3, 4])


def test_invariants_on_clustered_data():
    rng = np.random.default_rng(9)
    centres = rng.normal(scale=20.0, size=(8, 16))
    x = centres[rng.integers(0, 8, size=2000)] + rng.normal(size=(2000, 16))
    k = 15
    idx, dist = knn_oracle.exact_knn(x, k)
    assert np.all(idx != np.arange(2000)[:, None])
    assert np.all(np.diff(dist, axis=1) >= 0)
    # the distances are those of the listed rows
    d_direct = np.sqrt(((x[idx] - x[:, None, :]) ** 2).sum(-1))
    np.testing.assert_allclose(dist, d_direct, rtol=1e-12)
    # translation invariance (a large offset exercises the centring)
    idx2, dist2 = knn_oracle.exact_knn(x + 1e4, k)
    np.testing.assert_array_equal(idx2, idx)
    np.testing.assert_allclose(dist2, dist, rtol=1e-9)
    # no unlisted point is closer than the k-th (checked by brute force on a sample)
    for i in range(0, 2000, 97):
        d_all = np.sqrt(((x - x[i]) ** 2).sum(1))
        d_all[i] = np.inf
        assert np.sum(d_all < dist[i, -1] * (1 - 1e-12)) <= k - 1


def test_reference_layout():
    idx = np.array([[1, 2], [0, 2], [0, 1]])
    dist = np.array([[1.0, 2.0], [1.0, 3.0], [2.0, 3.0]])
    li, ld = knn_oracle.to_reference_layout(idx, dist)
    assert li.dtype == np.int32 and ld.dtype == np.float32
    # neighbour j of point i at j * n + i, 1-based
    assert li.ravel()[1 * 3 + 0] == 3 and li.ravel()[0 * 3 + 2] == 1
    assert ld.ravel()[1 * 3 + 1] == 3.0


def test_rejects_bad_k():
    x = np.zeros((4, 2))
    with pytest.raises(ValueError):
        knn_oracle.exact_knn(x, 4, exclude_self=True)
    with pytest.raises(ValueError):
        knn_oracle.exact_knn(x, 0)


def test_query_knn_matches_kdtree_and_brute_force():
    rng = np.random.default_rng(31)
    ref = rng.normal(size=(800, 9))
    qry = rng.normal(size=(150, 9))
    idx, dist = knn_oracle.exact_query_knn(ref, qry, 12)
    tree_d, tree_i = cKDTree(ref).query(qry, k=12)
    np.testing.assert_array_equal(idx, tree_i)
    np.testing.assert_allclose(dist, tree_d, rtol=1e-12, atol=1e-12)
    # lattice ties: query rows that coincide with reference rows, ties by index
    lat = rng.integers(0, 3, size=(60, 3)).astype(np.float64)
    q = lat[:10] + 0.0
    qi, qd = knn_oracle.exact_query_knn(lat, q, 8, margin=2)
    for i in range(10):
        d2 = ((lat - q[i]) ** 2).sum(1)
        order = sorted(range(60), key=lambda j: (d2[j], j))[:8]
        np.testing.assert_array_equal(qi[i], order)
        np.testing.assert_allclose(qd[i], np.sqrt(d2[order]), atol=1e-12)


@pytest.mark.parametrize("metric", ["cosine", "correlation"])
def test_metric_distances_match_scipy(metric):
    from scipy.spatial.distance import cdist

    rng = np.random.default_rng(41)
    x = (rng.normal(size=(300, 17)) + rng.uniform(-2, 2, size=(1, 17))).astype(np.float32)
    idx, dist = knn_oracle.metric_knn(x, 12, metric)
    full = cdist(x.astype(np.float64), x.astype(np.float64), metric=metric)  # 1 - cos, computed independently
    np.fill_diagonal(full, np.inf)
    want_i = np.argsort(full, axis=1, kind="stable")[:, :12]
    np.testing.assert_allclose(dist, np.take_along_axis(full, want_i, 1), rtol=0, atol=2e-6)
    # the order may differ from scipy's only where two distances agree to fp32 rounding
    differ = idx != want_i
    if differ.any():
        r, c = np.nonzero(differ)
        np.testing.assert_allclose(full[r, idx[r, c]], full[r, want_i[r, c]], atol=2e-6)
    q = (rng.normal(size=(40, 17))).astype(np.float32)
    qi, qd = knn_oracle.metric_knn(x, 5, metric, query=q)
    qfull = cdist(q.astype(np.float64), x.astype(np.float64), metric=metric)
    np.testing.assert_allclose(qd, np.sort(qfull, axis=1)[:, :5], atol=2e-6)


def test_normalize_rows_invariants():
    rng = np.random.default_rng(42)
    x = rng.normal(size=(200, 9)).astype(np.float32) * rng.uniform(0.1, 100, size=(200, 1)).astype(np.float32)
    x[5] = 0.0          # a zero row stays zero
    x[6] = 3.25         # a constant row: zero after centring
    xc = knn_oracle.normalize_rows(x, center=False)
    xr = knn_oracle.normalize_rows(x, center=True)
    norms = np.linalg.norm(xc.astype(np.float64), axis=1)
    assert np.all(xc[5] == 0) and np.all(xr[6] == 0)
    keep = np.ones(200, bool)
    keep[5] = False
    np.testing.assert_allclose(norms[keep], 1.0, atol=1e-6)
    keep[6] = False
    np.testing.assert_allclose(np.linalg.norm(xr[keep].astype(np.float64), axis=1), 1.0, atol=1e-6)
    np.testing.assert_allclose(xr[keep].astype(np.float64).mean(axis=1), 0.0, atol=1e-6)
    # a row's direction, not its scale, is what is kept
    np.testing.assert_allclose(knn_oracle.normalize_rows(4.0 * x[:3], False), xc[:3], atol=1e-7)
