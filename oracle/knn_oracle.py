"""CPU oracle for exact Euclidean k-nearest neighbours.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product path never loads it.

What it restates.  The reference's tests define exact KNN as a dense
squared-distance matrix whose rows are ordered with R's stable ``order``, so
that ties keep the lower index first, with the point itself either set to
+Inf (self excluded) or 0 (tests/testthat/helper-knn.R:5-38,
tests/testthat/test-native-knn.R:1-11).  The reference's GPU route hands the
same ordering to a third-party brute force (FAISS GPU ``bfKnn`` / cuVS,
src/native_knn_cuda_impl.cpp:549, :704, not vendored) and finishes it in
src/embedding_cuda_kernels.cpp:1412-1464: k + 1 searched, the point itself
dropped by index, ``sqrt(max(d2, 0))`` as float32, 1-based int32 indices in a
column-major query-by-k layout.

This oracle keeps the ordering of helper-knn.R but computes each squared
distance from the difference of the two rows in fp64 (sum of (x_i - y_i)^2),
which is exact to ~1e-16 relative, instead of R's expansion
|x|^2 + |y|^2 - 2 x.y, whose cancellation can reorder near-ties.  Candidates
are preselected with the fp64 expansion on centred rows and kept only when a
bound on that expansion's error proves that no unselected point can enter the
first k; rows that fail the bound are ordered from the full direct distances.

Pins (tests/test_knn_oracle.py): scipy's cKDTree on tie-free data, a
pure-Python brute force (sorted by (d2, index)) on tiny inputs with
duplicates and lattice ties, and the invariants of the result; the same for
the query-to-reference search (exact_query_knn).

Cosine and correlation (normalize_rows, metric_knn): the reference
normalises each fp32 row to unit length, centring it first for correlation
(src/native_knn_common.h:50-67), searches by Euclidean distance and reports
half the squared distance, 1 - cos (:119-128).  Pinned against scipy's
``cdist`` cosine and correlation distances, which compute 1 - cos on their
own, and by the invariants of unit rows.
"""

from __future__ import annotations

import numpy as np


def _direct_d2(xd: np.ndarray, q: int, cols: np.ndarray) -> np.ndarray:
    diff = xd[cols] - xd[q]
    return np.einsum("ij,ij->i", diff, diff)


def exact_knn(x, k: int, exclude_self: bool = True, chunk: int = 512, margin: int = 16):
    """Exact KNN of every row of ``x`` (n x d) among the rows of ``x``.

    Returns ``(indices, distances)``, each (n, k): 0-based int64 indices and
    fp64 distances, ascending by (distance, index).  With ``exclude_self`` the
    row itself never appears (helper-knn.R's ``diag(d2) <- Inf``); without it,
    it competes at distance 0 like any duplicate.
    """
    x = np.asarray(x)
    if x.ndim != 2:
        raise ValueError("x must be a matrix")
    n, d = x.shape
    k = int(k)
    if k < 1 or k > n - (1 if exclude_self else 0):
        raise ValueError("k must be between 1 and the number of candidate rows")
    xd = x.astype(np.float64)
    xc = xd - xd.mean(axis=0)
    sq = np.einsum("ij,ij->i", xc, xc)
    sq_max = float(sq.max()) if n else 0.0
    m = min(n, k + margin + (1 if exclude_self else 0))
    idx = np.empty((n, k), np.int64)
    dist = np.empty((n, k), np.float64)
    # |expansion - exact| <= (d + 4) 2^-52 (|q|^2 + |r|^2) for fp64 dot
    # products of d terms, doubled for safety
    eps_unit = 2.0 * (d + 4) * 2.0 ** -52
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        d2 = sq[s:e, None] + sq[None, :] - 2.0 * (xc[s:e] @ xc.T)
        if exclude_self:
            d2[np.arange(e - s), np.arange(s, e)] = np.inf
        if m < n:
            part = np.argpartition(d2, m - 1, axis=1)[:, :m]
        else:
            part = np.broadcast_to(np.arange(n), (e - s, n))
        for r in range(e - s):
            q = s + r
            cols = part[r]
            if exclude_self:
                cols = cols[cols != q]
            exact = _direct_d2(xd, q, cols)
            order = np.lexsort((cols, exact))
            cols, exact = cols[order], exact[order]
            if m < n:
                # the (m)-th expanded value bounds every unselected point from below
                rest = np.partition(d2[r], m - 1)[m - 1]
                eps = eps_unit * (sq[q] + sq_max)
                if not rest - eps > exact[k - 1]:
                    allc = np.arange(n)
                    if exclude_self:
                        allc = allc[allc != q]
                    full = _direct_d2(xd, q, allc)
                    order = np.lexsort((allc, full))
                    cols, exact = allc[order], full[order]
            idx[q] = cols[:k]
            dist[q] = np.sqrt(exact[:k])
    return idx, dist


def exact_query_knn(reference, query, k: int, chunk: int = 512, margin: int = 16):
    """Exact KNN of every row of ``query`` among the rows of ``reference``
    (the query-to-reference search of tests/testthat/helper-knn.R:5-38 with
    a separate ``query``): 0-based int64 reference indices and fp64
    distances, (n_query, k), ascending by (distance, index)."""
    ref = np.asarray(reference, dtype=np.float64)
    qry = np.asarray(query, dtype=np.float64)
    if ref.ndim != 2 or qry.ndim != 2 or ref.shape[1] != qry.shape[1]:
        raise ValueError("reference and query must be matrices with the same columns")
    n, d = ref.shape
    k = int(k)
    if k < 1 or k > n:
        raise ValueError("k must be between 1 and the number of reference rows")
    mu = ref.mean(axis=0)
    rc, qc = ref - mu, qry - mu
    sr = np.einsum("ij,ij->i", rc, rc)
    sq = np.einsum("ij,ij->i", qc, qc)
    m = min(n, k + margin)
    eps_unit = 2.0 * (d + 4) * 2.0 ** -52
    idx = np.empty((qry.shape[0], k), np.int64)
    dist = np.empty((qry.shape[0], k), np.float64)
    for s in range(0, qry.shape[0], chunk):
        e = min(qry.shape[0], s + chunk)
        d2 = sq[s:e, None] + sr[None, :] - 2.0 * (qc[s:e] @ rc.T)
        part = np.argpartition(d2, m - 1, axis=1)[:, :m] if m < n else np.broadcast_to(np.arange(n), (e - s, n))
        for r in range(e - s):
            q = s + r
            cols = np.asarray(part[r])
            diff = ref[cols] - qry[q]
            exact = np.einsum("ij,ij->i", diff, diff)
            order = np.lexsort((cols, exact))
            cols, exact = cols[order], exact[order]
            if m < n:
                rest = np.partition(d2[r], m - 1)[m - 1]
                if not rest - eps_unit * (sq[q] + sr.max()) > exact[k - 1]:
                    diff = ref - qry[q]
                    full = np.einsum("ij,ij->i", diff, diff)
                    allc = np.arange(n)
                    order = np.lexsort((allc, full))
                    cols, exact = allc[order], full[order]
            idx[q] = cols[:k]
            dist[q] = np.sqrt(exact[:k])
    return idx, dist


def brute_force_knn(x, k: int, exclude_self: bool = True):
    """Pure-Python restatement for tiny inputs: for each row, all other rows
    (or all rows) sorted by (squared distance, index)."""
    rows = [[float(v) for v in r] for r in np.asarray(x, dtype=np.float64)]
    n = len(rows)
    idx, dist = [], []
    for i in range(n):
        cand = []
        for j in range(n):
            if exclude_self and j == i:
                continue
            d2 = sum((a - b) * (a - b) for a, b in zip(rows[i], rows[j]))
            cand.append((d2, j))
        cand.sort()
        idx.append([j for _, j in cand[:k]])
        dist.append([d2 ** 0.5 for d2, _ in cand[:k]])
    return np.asarray(idx, np.int64), np.asarray(dist, np.float64)


def to_reference_layout(indices: np.ndarray, distances: np.ndarray):
    """The reference's device layout (src/embedding_cuda_kernels.cpp:1447-1449):
    column-major n x k, 1-based int32 indices and float32 distances, returned
    as (k, n) C-order arrays whose bytes are that layout."""
    return (np.ascontiguousarray((indices + 1).T, dtype=np.int32),
            np.ascontiguousarray(distances.T, dtype=np.float32))


def normalize_rows(x, center: bool):
    """Rows of ``x`` (cast to fp32) normalised as src/native_knn_common.h:50-67
    does it: mean = sequential fp64 sum / d (centre only), v = fl32(x - mean),
    s = sequential fp64 sum of v^2, and when s > 0 each v times
    fl32(1 / sqrt(s)) in fp32; a row with s = 0 is left as it is."""
    x32 = np.asarray(x, dtype=np.float32)
    x64 = x32.astype(np.float64)
    n, d = x32.shape
    mean = np.cumsum(x64, axis=1)[:, -1] / max(1, d) if center else np.zeros(n)  # cumsum sums in order
    v = (x64 - mean[:, None]).astype(np.float32)
    sq = np.cumsum(v.astype(np.float64) ** 2, axis=1)[:, -1]  # squares of fp32 values are exact in fp64
    inv = np.ones(n, np.float32)
    pos = sq > 0
    inv[pos] = (1.0 / np.sqrt(sq[pos])).astype(np.float32)
    return np.where(pos[:, None], v * inv[:, None], v).astype(np.float32)


def metric_knn(x, k: int, metric: str, exclude_self: bool = True, query=None):
    """Exact KNN under "euclidean", "cosine" or "correlation": indices as
    exact_knn / exact_query_knn of the (normalised) rows, distances sqrt(d2)
    for euclidean and d2 / 2 = 1 - cos otherwise."""
    if metric == "euclidean":
        return exact_knn(x, k, exclude_self=exclude_self) if query is None else exact_query_knn(x, query, k)
    center = {"cosine": False, "correlation": True}[metric]
    xn = normalize_rows(x, center)
    if query is None:
        idx, dist = exact_knn(xn, k, exclude_self=exclude_self)
    else:
        idx, dist = exact_query_knn(xn, normalize_rows(query, center), k)
    return idx, 0.5 * dist * dist
