"""Pins for the oracle's FIt-SNE interpolation grid (an extension: the
reference's native code has only the bilinear grid).

* Lagrange basis: scipy.interpolate.lagrange on the same nodes, partition of
  unity, exact reproduction of polynomials of degree < order, and the
  cardinal property L_j(t_l) = delta_jl;
* convolution: the zero-padded fp64 FFT against the O(nodes^4) direct node sum;
* geometry: box count max(min_intervals, ceil(span / ints_per_unit)) with the
  node cap, lower corner at the smallest coordinate;
* gradient and normaliser: convergence to the exact O(n^2) closed form (dense
  numpy) as the boxes shrink, with the error falling at the rate of an
  order-3 interpolant.
"""

import math

import numpy as np
import pytest
from scipy.interpolate import lagrange

from tests.helpers import csr_to_dense, exact_gradient_numpy, rel_l2, small_problem


@pytest.mark.parametrize("order", [2, 3, 4, 5])
def test_lagrange_basis(oracle_mod, order):
    nodes = (np.arange(order) + 0.5) / order
    rng = np.random.default_rng(order)
    for u in rng.uniform(0.0, 1.0, size=9):
        w = oracle_mod.lagrange_weights(u, order)
        ref = np.array([lagrange(nodes, np.eye(order)[j])(u) for j in range(order)])
        np.testing.assert_allclose(w, ref, rtol=1e-9, atol=1e-12)
        assert abs(w.sum() - 1.0) < 1e-12
        for deg in range(order):
            assert abs((w * nodes**deg).sum() - u**deg) < 1e-12
    for l, t in enumerate(nodes):
        np.testing.assert_allclose(oracle_mod.lagrange_weights(t, order), np.eye(order)[l], atol=1e-14)


def _problem(n=500, scale=6.0, seed=3):
    x, _, idx, dist = small_problem(n=n, dim=6, k=20, components=4, seed=seed)
    P = __import__("oracle.oracle", fromlist=["OracleP"]).OracleP.build(idx, dist, 8.0, threads=2)
    from fastembedr_amd import synthetic

    y = synthetic.pca_init(x)
    y = (y / np.abs(y).max() * scale).astype(np.float32)
    return P, y


def test_fft_convolution_matches_direct_node_sum(oracle_mod):
    P, y = _problem(n=300, scale=4.0)
    for min_int in (6, 11):
        g_fft, geo, z_fft = P.lagrange_gradient(y, 1.0, order=3, min_intervals=min_int)
        g_dir, geo_d, z_dir = P.lagrange_gradient(y, 1.0, order=3, min_intervals=min_int, direct=True)
        assert geo == geo_d
        assert rel_l2(g_fft, g_dir) < 1e-6
        assert abs(z_fft - z_dir) / z_dir < 1e-12


def test_geometry(oracle_mod):
    P, y = _problem(n=300, scale=40.0)
    lo = float(y.min())
    span = float(y.max()) - lo
    _, geo, _ = P.lagrange_gradient(y, 1.0, order=3, min_intervals=50)
    assert geo["boxes"] == max(50, math.ceil(span)) and geo["nodes"] == 3 * geo["boxes"]
    assert geo["lo"] == lo and abs(geo["box_w"] * geo["boxes"] - span) < 1e-9 * span
    _, geo, _ = P.lagrange_gradient(y, 1.0, order=3, min_intervals=10, ints_per_unit=0.5)
    assert geo["boxes"] == max(10, math.ceil(span / 0.5))
    _, geo, _ = P.lagrange_gradient(y * 50.0, 1.0, order=3, min_intervals=50)
    assert geo["boxes"] == 2048 // 3  # node cap: FFT length 2 * nodes <= 4096


def test_gradient_converges_to_exact(oracle_mod):
    P, y = _problem(n=500, scale=6.0)
    dense = csr_to_dense(*P.csr(), P.n)
    for ex in (1.0, 12.0):
        g_ex = exact_gradient_numpy(y, dense, ex)
        d = y.astype(np.float64)[:, None, :] - y.astype(np.float64)[None, :, :]
        q = 1.0 / (1.0 + (d * d).sum(-1))
        np.fill_diagonal(q, 0.0)
        z_ex = q.sum()
        errs, zerrs = [], []
        for boxes in (8, 16, 32, 64):
            g, geo, z = P.lagrange_gradient(y, ex, order=3, min_intervals=boxes, ints_per_unit=1e6)
            assert geo["boxes"] == boxes
            errs.append(rel_l2(g, g_ex))
            zerrs.append(abs(z - z_ex) / z_ex)
        # third-order interpolation: each halving of the box width cuts the
        # error about eightfold
        assert all(b < a / 4.0 for a, b in zip(errs, errs[1:])), errs
        assert all(b < a / 4.0 for a, b in zip(zerrs, zerrs[1:])), zerrs
        assert errs[-1] < 5e-4 and zerrs[-1] < 5e-5, (errs, zerrs)
