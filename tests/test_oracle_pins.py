"""Pins for the CPU oracle (oracle/tsne_oracle.cpp) that do not retype its code.

* perplexity search: row sums, row entropy at the target (the stopping rule),
  a float64 bisection solved to machine precision, and scikit-learn's
  independent implementation of the same search;
* symmetrisation: the closed form P = (C + C^T) / (2 * total) with scipy.sparse;
* grid convolution: numpy.fft on the zero-padded charge grids;
* grid repulsion: convergence to the exact O(n^2) gradient as the grid refines;
  its fp64 instantiation against a numpy float64 statement of the whole
  bilinear-grid gradient (geometry, spread, numpy.fft, read-back, attraction);
* exact gradient and KL: dense closed forms;
* update: elementwise closed form including the sign(0) == 0 first step.
"""

import math

import numpy as np
import pytest
import scipy.sparse as sp

from tests.helpers import csr_to_dense, exact_gradient_numpy, rel_l2, small_problem


def _entropy(p):
    p = p.astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = np.where(p > 0, p * np.log(p), 0.0)
    return -t.sum(axis=1)


def test_row_search_invariants_and_fp64_bisection(oracle_mod):
    rng = np.random.default_rng(11)
    n, k, perp = 400, 40, 12.0
    d = np.sort(rng.gamma(4.0, 1.0, size=(n, k)).astype(np.float32), axis=1)
    p, beta, steps = oracle_mod.conditional_p(d, perp)
    assert np.all(steps < 200)
    np.testing.assert_allclose(p.sum(axis=1), 1.0, atol=2e-6)
    # stopping rule: |H - log(perp)| < 1e-5 in fp32 arithmetic -> ~1e-4 in fp64
    np.testing.assert_allclose(_entropy(p), math.log(perp), atol=2e-4)
    # fp64 bisection to machine precision
    sq = d.astype(np.float64) ** 2
    for i in range(0, n, 37):
        lo, hi = 1e-12, 1e6
        for _ in range(200):
            b = math.sqrt(lo * hi)
            w = np.exp(-b * (sq[i] - sq[i].min()))
            q = w / w.sum()
            h = -(q * np.log(np.maximum(q, 1e-300))).sum()
            if h > math.log(perp):
                lo = b
            else:
                hi = b
        assert abs(beta[i] - b) / b < 2e-3, (i, beta[i], b)
        np.testing.assert_allclose(p[i], q, rtol=2e-3, atol=1e-7)
    # monotone in distance
    assert np.all(np.diff(p, axis=1) <= 1e-12)


def test_row_search_matches_sklearn(oracle_mod):
    from sklearn.manifold._utils import _binary_search_perplexity

    rng = np.random.default_rng(5)
    n, k, perp = 300, 30, 9.0
    d = np.sort(rng.gamma(3.0, 1.0, size=(n, k)).astype(np.float32), axis=1)
    p, _, _ = oracle_mod.conditional_p(d, perp)
    ref = _binary_search_perplexity((d.astype(np.float32) ** 2).astype(np.float32), perp, 0)
    assert rel_l2(p, ref) < 5e-4


@pytest.mark.parametrize("one_based", [True, False])
@pytest.mark.parametrize("with_self", [False, True])
def test_symmetrisation_closed_form(oracle_mod, one_based, with_self):
    x, _, idx, dist = small_problem(n=300, k=15, one_based=one_based)
    if with_self:
        base = 1 if one_based else 0
        idx = np.asfortranarray(np.concatenate([np.arange(300)[:, None] + base, idx[:, :-1]], axis=1))
        dist = np.asfortranarray(np.concatenate([np.zeros((300, 1), np.float32), dist[:, :-1]], axis=1))
    n, k = idx.shape
    P = oracle_mod.OracleP.build(idx, dist, perplexity=4.0)
    rp, col, val = P.csr()
    pc, _, _ = oracle_mod.conditional_p(dist, 4.0)
    base = 1 if (idx.min() >= 1 and idx.max() <= n) else 0
    rows = np.repeat(np.arange(n), k)
    cols = (idx - base).reshape(-1)
    vals = pc.reshape(-1).astype(np.float64)
    keep = rows != cols
    total = vals[keep].sum()
    c = sp.coo_matrix((vals[keep], (rows[keep], cols[keep])), shape=(n, n)).tocsr()
    s = (c + c.T).tocoo()
    expect = np.zeros((n, n), np.float64)
    expect[s.row, s.col] = (s.data.astype(np.float32) * np.float32(0.5 / total)).astype(np.float64)
    got = csr_to_dense(rp, col, val, n)
    np.testing.assert_array_equal(got, expect)
    assert np.all(np.diag(got) == 0)
    assert abs(got.sum() - 1.0) < 1e-5
    np.testing.assert_array_equal(got, got.T)
    for i in range(n):
        assert np.all(np.diff(col[rp[i]:rp[i + 1]]) > 0)


def test_symmetrisation_errors(oracle_mod):
    _, _, idx, dist = small_problem(n=100, k=8)
    bad = idx.copy()
    bad[3, 2] = 500
    with pytest.raises(ValueError, match="out of range"):
        oracle_mod.OracleP.build(bad, dist, 2.0)
    badd = dist.copy()
    badd[4, 1] = -1.0
    with pytest.raises(ValueError, match="finite and non-negative"):
        oracle_mod.OracleP.build(idx, badd, 2.0)


def _numpy_fields(y, geom, g):
    lo_x, lo_y, h, inv_h = [float(v) for v in geom]
    ux = np.clip((y[:, 0] - lo_x) * inv_h, 0, g - 1)
    uy = np.clip((y[:, 1] - lo_y) * inv_h, 0, g - 1)
    x0 = np.clip(np.floor(ux).astype(int), 0, g - 2)
    y0 = np.clip(np.floor(uy).astype(int), 0, g - 2)
    tx, ty = ux - x0, uy - y0
    mass = np.zeros((3, g, g))
    for wy, dy in ((1 - ty, 0), (ty, 1)):
        for wx, dx in ((1 - tx, 0), (tx, 1)):
            w = wy * wx
            for c, v in enumerate((np.ones(len(y)), y[:, 0].astype(np.float64), y[:, 1].astype(np.float64))):
                np.add.at(mass[c], (y0 + dy, x0 + dx), w * v)
    f = 2 * g
    off = np.arange(-(g - 1), g)
    dxx, dyy = np.meshgrid(off * h, off * h)
    k1 = 1.0 / (1.0 + dxx * dxx + dyy * dyy)
    K1 = np.zeros((f, f))
    K2 = np.zeros((f, f))
    K1[np.ix_(off % f, off % f)] = k1
    K2[np.ix_(off % f, off % f)] = k1 * k1

    def conv(m, K):
        A = np.zeros((f, f))
        A[:g, :g] = m
        return np.real(np.fft.ifft2(np.fft.fft2(A) * np.fft.fft2(K)))[:g, :g]

    return np.stack([conv(mass[0], K1), conv(mass[0], K2), conv(mass[1], K2), conv(mass[2], K2)])


@pytest.mark.parametrize("grid", [32, 64])
def test_grid_fields_match_numpy_fft(oracle_mod, grid):
    x, _, idx, dist = small_problem(n=500, k=20)
    P = oracle_mod.OracleP.build(idx, dist, 6.0)
    rng = np.random.default_rng(2)
    y = (rng.standard_normal((500, 2)) * 3).astype(np.float32)
    geom, fields = P.grid_fields(y, grid_size=grid)
    ref = _numpy_fields(y, geom, grid)
    for c in range(4):
        assert rel_l2(fields[c], ref[c]) < 2e-5, c


def _numpy_bilinear(field, ux, uy, g):
    x0 = np.clip(np.floor(ux).astype(int), 0, g - 2)
    y0 = np.clip(np.floor(uy).astype(int), 0, g - 2)
    tx, ty = ux - x0, uy - y0
    return ((1 - tx) * (1 - ty) * field[y0, x0] + tx * (1 - ty) * field[y0, x0 + 1]
            + (1 - tx) * ty * field[y0 + 1, x0] + tx * ty * field[y0 + 1, x0 + 1])


@pytest.mark.parametrize("grid", [32, 128])
def test_fp64_grid_gradient_matches_numpy_closed_form(oracle_mod, grid):
    """The fp64 bilinear-grid gradient (the yardstick for both fp32 sides)
    against numpy in float64: the geometry, bilinear spread, numpy.fft
    convolution, bilinear read-back, normalisation by sum(q) - n and the
    dense attraction closed form."""
    n = 500
    x, _, idx, dist = small_problem(n=n, k=20)
    P = oracle_mod.OracleP.build(idx, dist, 6.0)
    rp, col, val = P.csr()
    dense = csr_to_dense(rp, col, val, n)
    rng = np.random.default_rng(12)
    y = (rng.standard_normal((n, 2)) * 7).astype(np.float32)
    y64 = y.astype(np.float64)
    lo, hi = y64.min(0), y64.max(0)
    span = float(max(hi - lo))
    half = 0.55 * span + 1e-3
    c = 0.5 * (lo + hi)
    h = 2 * half / (grid - 1)
    geom = (c[0] - half, c[1] - half, h, 1.0 / h)
    q, q2, xq2, yq2 = _numpy_fields(y64, geom, grid)
    ux = np.clip((y64[:, 0] - geom[0]) / h, 0, grid - 1)
    uy = np.clip((y64[:, 1] - geom[1]) / h, 0, grid - 1)
    z = _numpy_bilinear(q, ux, uy, grid).sum() - n
    a = _numpy_bilinear(q2, ux, uy, grid)
    rep = -np.stack([y64[:, 0] * a - _numpy_bilinear(xq2, ux, uy, grid),
                     y64[:, 1] * a - _numpy_bilinear(yq2, ux, uy, grid)], 1) / z
    d = y64[:, None, :] - y64[None, :, :]
    qq = 1.0 / (1.0 + (d * d).sum(-1))
    for ex in (1.0, 12.0):
        want = rep + ex * ((dense * qq)[:, :, None] * d).sum(1)
        got = P.gradient_grid_f64(y, ex, grid_size=grid, threads=3)
        assert got.dtype == np.float64
        assert rel_l2(got, want) < 1e-10
        # and the fp32 path is the same algorithm, to fp32 rounding
        assert rel_l2(P.gradient(y, ex, grid_size=grid, threads=3), got) < 1e-4


def test_exact_gradient_closed_form(oracle_mod):
    x, _, idx, dist = small_problem(n=250, k=15)
    P = oracle_mod.OracleP.build(idx, dist, 4.0)
    rp, col, val = P.csr()
    dense = csr_to_dense(rp, col, val, 250)
    rng = np.random.default_rng(9)
    y = (rng.standard_normal((250, 2)) * 2).astype(np.float32)
    for ex in (1.0, 12.0):
        g = P.gradient(y, ex, method=oracle_mod.METHOD_EXACT, threads=3)
        assert rel_l2(g, exact_gradient_numpy(y, dense, ex)) < 1e-5


def test_grid_gradient_converges_to_exact(oracle_mod):
    x, _, idx, dist = small_problem(n=400, k=15)
    P = oracle_mod.OracleP.build(idx, dist, 4.0)
    rng = np.random.default_rng(4)
    y = (rng.standard_normal((400, 2)) * 4).astype(np.float32)
    exact = P.gradient(y, 1.0, method=oracle_mod.METHOD_EXACT)
    errs = [rel_l2(P.gradient(y, 1.0, grid_size=g), exact) for g in (32, 128, 512)]
    assert errs[0] > errs[1] > errs[2]
    assert errs[2] < 2e-3, errs


def test_kl_closed_form(oracle_mod):
    x, _, idx, dist = small_problem(n=200, k=12)
    P = oracle_mod.OracleP.build(idx, dist, 3.0)
    rp, col, val = P.csr()
    rng = np.random.default_rng(1)
    y = rng.standard_normal((200, 2)).astype(np.float32)
    kl, rows = P.kl(y, threads=2, row_costs=True)
    dense = csr_to_dense(rp, col, val, 200)
    d = y[:, None, :].astype(np.float64) - y[None, :, :]
    q = 1.0 / (1.0 + (d * d).sum(-1))
    np.fill_diagonal(q, 0)
    q /= q.sum()
    mask = dense > 0
    ref = (dense[mask] * np.log((dense[mask] + 1e-9) / (q[mask] + 1e-9))).sum()
    assert abs(kl - ref) / abs(ref) < 1e-6
    assert abs(rows.sum() - kl) < 1e-9


def test_update_closed_form(oracle_mod):
    rng = np.random.default_rng(8)
    n = 1000
    y = rng.standard_normal((n, 2)).astype(np.float32)
    upd = np.zeros((n, 2), np.float32)
    upd[: n // 2] = rng.standard_normal((n // 2, 2)).astype(np.float32)
    gains = np.ones((n, 2), np.float32)
    gains[::3] = 0.005
    grad = rng.standard_normal((n, 2)).astype(np.float32)
    grad[::7, 0] = 0.0
    lr, mom, mg, ms = np.float32(50.0), np.float32(0.5), np.float32(0.01), np.float32(5.0)
    # closed form in float32
    sgn = lambda v: np.sign(v).astype(np.float32)
    g2 = np.where(sgn(upd) != sgn(grad), gains + np.float32(0.2), gains * np.float32(0.8) + mg).astype(np.float32)
    g2 = np.maximum(g2, mg)
    u2 = (mom * upd - lr * g2 * grad).astype(np.float32)
    ns = (u2[:, 0] * u2[:, 0] + u2[:, 1] * u2[:, 1]).astype(np.float32)
    scale = np.where(ns > ms * ms, ms / np.sqrt(np.maximum(ns, np.float32(np.finfo(np.float32).tiny))), 1.0)
    u2 = (u2 * scale[:, None].astype(np.float32)).astype(np.float32)
    y2 = (y + u2).astype(np.float32)
    yy, uu, gg = y.copy(), upd.copy(), gains.copy()
    oracle_mod.update(yy, uu, gg, grad, lr, mom, mg, ms, threads=2)
    np.testing.assert_array_equal(gg, g2)
    np.testing.assert_allclose(uu, u2, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(yy, y2, rtol=1e-6, atol=1e-6)
    # first step from rest: sign(0) == 0 differs from sign(grad) -> gains 1.2
    yy, uu, gg = y.copy(), np.zeros_like(upd), np.ones_like(gains)
    oracle_mod.update(yy, uu, gg, grad, lr, mom, mg, ms)
    nz = grad != 0
    np.testing.assert_array_equal(gg[nz], np.float32(1.2))
    np.testing.assert_array_equal(gg[~nz], np.float32(0.81))


def test_zero_mean(oracle_mod):
    rng = np.random.default_rng(0)
    y = (rng.standard_normal((777, 2)) + 5).astype(np.float32)
    ref = (y - y.astype(np.float64).mean(axis=0).astype(np.float32)).astype(np.float32)
    oracle_mod.zero_mean(y)
    np.testing.assert_array_equal(y, ref)


def test_optimizer_reduces_kl(oracle_mod):
    x, labels, idx, dist = small_problem(n=600, k=30)
    P = oracle_mod.OracleP.build(idx, dist, 10.0, threads=2)
    y0 = oracle_mod.random_init(600, 42)
    y, costs, its = P.optimize(y0, 50, 100, 12.0, 1.0, 600 / 12.0, False, 0.5, 0.8, threads=2,
                               record_costs=True)
    assert list(its) == [50, 100, 150]
    assert costs[-1] < costs[0]
    assert np.all(np.isfinite(y))
    assert abs(float(y.astype(np.float64).mean())) < 1e-3
