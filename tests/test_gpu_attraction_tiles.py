"""Tiled attraction on the GPU (P regrouped per (row block, column tile) into
runs of 16-bit slot words and values, attraction_tiles_hip.hip) against a
direct fp64 sum over the device's own P, and against the row-parallel CSR
kernel.

The attraction alone is read from two gradients at one layout: the repulsion
does not depend on the exaggeration, so (g(e1) - g(e2)) / (e1 - e2) is
sum_j p_ij q_ij (y_i - y_j) (src/tsne_neighbors.cpp:985-1012).

Tolerance: relative L2 <= 1e-5 (fp32 sums in another order; the hardware
reciprocal is within 1 ulp).  The cases cover many tiles per row block, rows
whose parts in one tile are far longer than a lane's group of 8 slots, rows
of one or two entries, sparse runs whose rows lie more than 7 apart (bridge
slots), and sizes that are not multiples of the tile shape, each in both
tile shapes (1024 rows x 4096 columns and 2048 x 2048, the one picked from
2**19 points; FASTEMBEDR_HIP_TILE_SHAPE forces either).
"""

import sys

import numpy as np
import pytest

from fastembedr_amd import _lib
from tests.helpers import rel_l2, small_problem

pytestmark = pytest.mark.gpu

TOL = 1e-5
SHAPES = {"1": (1024, 4096), "2": (2048, 2048)}


@pytest.fixture(params=sorted(SHAPES), ids=lambda k: "x".join(map(str, SHAPES[k])))
def shape(request, monkeypatch):
    monkeypatch.setenv("FASTEMBEDR_HIP_TILE_SHAPE", request.param)
    return SHAPES[request.param]


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def attraction_numpy(row_ptr, col, val, y):
    n = len(row_ptr) - 1
    rows = np.repeat(np.arange(n), np.diff(row_ptr))
    d = y[rows].astype(np.float64) - y[col].astype(np.float64)
    w = val.astype(np.float64) / (1.0 + (d * d).sum(1))
    out = np.zeros((n, 2))
    np.add.at(out, rows, w[:, None] * d)
    return out


def attraction_device(s, e1=12.0, e2=4.0):
    g1 = s.gradient(e1, _lib.REPULSION_EXACT).astype(np.float64)
    g2 = s.gradient(e2, _lib.REPULSION_EXACT).astype(np.float64)
    return (g1 - g2) / (e1 - e2)


def ring_knn(n, k):
    """Neighbours i+1 .. i+k (wrapping), 1-based, column-major: every row's
    entries fall in one or two column tiles, in parts far longer than a piece."""
    idx = (np.arange(n)[:, None] + np.arange(1, k + 1)[None, :]) % n + 1
    dist = np.broadcast_to(np.arange(1, k + 1, dtype=np.float32) * 0.1, (n, k))
    return np.asfortranarray(idx.astype(np.int32)), np.asfortranarray(dist.astype(np.float32))


def _check(hip, idx, dist, perplexity, y, label, shape):
    tile_rows, tile_cols = shape
    with hip.TsneSession(idx, dist, perplexity=perplexity, index_offset=1) as s:
        s.set_state(y)
        att = attraction_device(s)
        row_ptr, col, val = s.csr()
        info = s.attraction_info()
        tiles = info["tiles"]
    n = y.shape[0]
    # slots: every entry, the bridges between entries more than 7 rows apart
    # within a run (at most (rows - 1) // 7 per run) and each run's padding to 8
    assert info["slots"] % 8 == 0
    assert len(col) <= info["slots"] <= len(col) + ((tile_rows - 1) // 7 + 7) * info["tiles"]
    ref = attraction_numpy(row_ptr, col, val, y)
    rows = np.repeat(np.arange(n), np.diff(row_ptr))
    want_tiles = len(np.unique((rows // tile_rows).astype(np.int64) * (1 << 20) + col // tile_cols))
    err = rel_l2(att, ref)
    _say(f"  {label} {tile_rows}x{tile_cols}: n={n} nnz={len(col)} tiles={tiles} relL2={err:.2e}")
    assert tiles == want_tiles
    assert err <= TOL
    return att


@pytest.fixture(scope="module")
def mixture20k():
    x, labels, idx, dist = small_problem(n=20000, dim=6, k=30, components=5, seed=8)
    y = (np.random.default_rng(2).standard_normal((20000, 2)) * 10).astype(np.float32)
    return idx, dist, y


def test_tiled_attraction_matches_direct_sum(hip, mixture20k, shape):
    _say(f"case: tiled attraction, mixture n=20000 k=30, tiles {shape}")
    idx, dist, y = mixture20k
    _check(hip, idx, dist, 10.0, y, "mixture", shape)


def test_tiled_attraction_short_rows(hip, shape):
    _say(f"case: tiled attraction, mixture n=13001 k=3 (pieces of 1 to 6 entries), tiles {shape}")
    n = 13001
    x, labels, idx, dist = small_problem(n=n, dim=6, k=3, components=5, seed=8)
    y = (np.random.default_rng(5).standard_normal((n, 2)) * 10).astype(np.float32)
    _check(hip, idx, dist, 1.0, y, "short rows", shape)


def test_tiled_attraction_long_parts(hip, shape):
    _say(f"case: tiled attraction, ring neighbours (parts of up to 60 entries), tiles {shape}")
    n, k = 9000, 60
    idx, dist = ring_knn(n, k)
    rng = np.random.default_rng(3)
    y = (rng.standard_normal((n, 2)) * 3).astype(np.float32)
    _check(hip, idx, dist, 20.0, y, "ring", shape)


def scattered_knn(n, k, seed):
    """k neighbours drawn uniformly from all rows: each (row block, column
    tile) run holds few entries, so its rows are often more than 7 apart and
    the slot layout needs bridge slots (and row gaps up to a whole block)."""
    rng = np.random.default_rng(seed)
    idx = np.empty((n, k), np.int32)
    for i in range(n):
        c = rng.choice(n - 1, size=k, replace=False)
        idx[i] = c + (c >= i) + 1
    dist = np.sort(rng.uniform(0.5, 2.0, size=(n, k)), axis=1).astype(np.float32)
    return np.asfortranarray(idx), np.asfortranarray(dist)


def test_tiled_attraction_sparse_runs(hip, shape):
    _say(f"case: tiled attraction, scattered neighbours n=60000 k=3 (sparse runs, bridge slots), tiles {shape}")
    n = 60000
    idx, dist = scattered_knn(n, 3, 11)
    y = (np.random.default_rng(6).standard_normal((n, 2)) * 5).astype(np.float32)
    _check(hip, idx, dist, 1.0, y, "scattered", shape)


def test_tiled_matches_row_parallel(hip, mixture20k, shape, monkeypatch):
    _say(f"case: tiled vs row-parallel attraction, tiles {shape}")
    idx, dist, y = mixture20k
    with hip.TsneSession(idx, dist, perplexity=10.0, index_offset=1) as s:
        s.set_state(y)
        tiled = attraction_device(s)
    monkeypatch.setenv("FASTEMBEDR_HIP_ATTRACT_TILED", "0")
    with hip.TsneSession(idx, dist, perplexity=10.0, index_offset=1) as s:
        s.set_state(y)
        rowpar = attraction_device(s)
        assert s.attraction_info()["tiles"] == -1
    err = rel_l2(tiled, rowpar)
    _say(f"  relL2 tiled vs row-parallel {err:.2e}")
    assert err <= TOL
