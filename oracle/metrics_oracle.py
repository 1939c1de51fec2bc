"""CPU oracle for the exact rank-based structure metrics.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker.  The product
path never loads it.

Restates exact_structure_metrics_cpp (src/embedding_utils.cpp:1582-1752) of
the reference in numpy: squared distances in both spaces summed over the
columns in order (each square rounded, no fused multiply-add: the same fp64
values as the reference), every row's other rows ranked by (d2, index), and
for each k the shared-neighbour count, trustworthiness and continuity
penalties and neighbour rank error, normalised as the reference does.

Pins (tests/test_metrics_oracle.py): a pure-Python restatement on tiny
inputs, closed forms (a layout equal to the data gives trustworthiness =
continuity = preservation = 1 and rank error 0; a layout that reverses the
order of points on a line), and invariance under a common translation or
rotation of the layout.
"""

from __future__ import annotations

import numpy as np


def _sq_dists(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    n, p = x.shape
    d2 = np.zeros((n, n))
    for c in range(p):  # in column order, as the reference
        delta = x[:, c][:, None] - x[:, c][None, :]
        d2 = d2 + delta * delta
    return d2


def _orders(d2: np.ndarray) -> np.ndarray:
    n = d2.shape[0]
    out = np.empty((n, n - 1), np.int64)
    idx = np.arange(n)
    for i in range(n):
        others = idx[idx != i]
        out[i] = others[np.lexsort((others, d2[i, others]))]
    return out


def exact_structure_metrics(high, low, ks):
    """Returns an (len(ks), 4) array: trustworthiness, continuity,
    knn_preservation, mean_neighbor_rank_error."""
    high = np.asarray(high, dtype=np.float64)
    low = np.asarray(low, dtype=np.float64)
    n = high.shape[0]
    if low.shape[0] != n:
        raise ValueError("high and low must have the same row count")
    if n < 3:
        raise ValueError("at least three observations are required")
    ks = [int(k) for k in ks]
    for k in ks:
        if k < 1 or k >= n or 2 * n - 3 * k - 1 <= 0:
            raise ValueError("each k must satisfy 1 <= k < (2 * n - 1) / 3")
    ho = _orders(_sq_dists(high))
    lo = _orders(_sq_dists(low))
    hr = np.empty((n, n), np.int64)
    lr = np.empty((n, n), np.int64)
    rows = np.arange(n)[:, None]
    hr[rows, ho] = np.arange(1, n)[None, :]
    lr[rows, lo] = np.arange(1, n)[None, :]
    out = np.empty((len(ks), 4))
    for q, k in enumerate(ks):
        in_high = hr[rows, lo[:, :k]]          # high rank of each low neighbour
        in_low = lr[rows, ho[:, :k]]           # low rank of each high neighbour
        shared = float((in_high <= k).sum())
        trust = float(np.where(in_high > k, in_high - k, 0).sum())
        cont = float(np.where(in_low > k, in_low - k, 0).sum())
        rerr = float(np.abs(in_high - np.arange(1, k + 1)[None, :]).sum())
        norm = 2.0 / (n * k * (2.0 * n - 3.0 * k - 1.0))
        out[q] = [min(1.0, max(0.0, 1.0 - norm * trust)), min(1.0, max(0.0, 1.0 - norm * cont)),
                  shared / (n * k), rerr / (n * k)]
    return out


def brute_force_metrics(high, low, k):
    """Pure-Python restatement for tiny inputs (one k)."""
    high = [[float(v) for v in r] for r in np.asarray(high, dtype=np.float64)]
    low = [[float(v) for v in r] for r in np.asarray(low, dtype=np.float64)]
    n = len(high)

    def d2(rows, i, j):
        s = 0.0
        for a, b in zip(rows[i], rows[j]):
            s += (a - b) * (a - b)
        return s

    shared = trust = cont = rerr = 0.0
    for i in range(n):
        others = [j for j in range(n) if j != i]
        ho = sorted(others, key=lambda j: (d2(high, i, j), j))
        lo = sorted(others, key=lambda j: (d2(low, i, j), j))
        hrank = {j: r + 1 for r, j in enumerate(ho)}
        lrank = {j: r + 1 for r, j in enumerate(lo)}
        for r in range(k):
            a = hrank[lo[r]]
            b = lrank[ho[r]]
            shared += a <= k
            trust += a - k if a > k else 0
            cont += b - k if b > k else 0
            rerr += abs(a - (r + 1))
    norm = 2.0 / (n * k * (2.0 * n - 3.0 * k - 1.0))
    return [min(1.0, max(0.0, 1.0 - norm * trust)), min(1.0, max(0.0, 1.0 - norm * cont)),
            shared / (n * k), rerr / (n * k)]
