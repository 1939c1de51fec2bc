"""Pins of the transform oracle (oracle/transform_oracle.cpp) against known
answers, closed forms and independent restatements (CPU only)."""

import math

import numpy as np
import pytest

from oracle import oracle


def _problem(n_ref=300, nq=40, k=15, seed=0):
    rng = np.random.default_rng(seed)
    ref = rng.normal(size=(n_ref, 2))
    idx = rng.integers(1, n_ref + 1, size=(nq, k)).astype(np.int32)
    dist = np.sort(rng.exponential(size=(nq, k)), axis=1)
    return ref, idx, dist


def test_xorshift32_known_answer():
    # Marsaglia, "Xorshift RNGs" (J. Stat. Softw. 8(14), 2003): the (13, 17, 5)
    # generator started at y = 2463534242 first returns 723471715.
    assert int(oracle.xorshift32(2463534242, 1)[0]) == 723471715


def test_hash_never_returns_zero_and_iteration_seed_wraps():
    assert oracle.hash32(0) == 0x6D2B79F5
    assert oracle.transform_iteration_seed(7, 0) == 7 + 65537
    assert oracle.transform_iteration_seed(-(2 ** 31), 2) == 5489 + 3 * 65537  # NA seed
    big = oracle.transform_iteration_seed(2 ** 31 - 1, 0)  # wraps like 32-bit arithmetic
    assert big == ((2 ** 31 - 1 + 65537) & 0xFFFFFFFF) - 2 ** 32


def test_conditional_p_invariants():
    _, _, dist = _problem(nq=60, k=20)
    perp = 5.0
    p = oracle.transform_conditional_p(dist, perp)
    np.testing.assert_allclose(p.sum(axis=1), 1.0, rtol=0, atol=1e-12)
    # the stopping rule: |H(p) - log(perplexity)| < 1e-5, H in nats
    h = -(p * np.log(np.where(p > 0, p, 1))).sum(axis=1)
    assert np.abs(h - math.log(perp)).max() < 2e-5
    # monotone in distance (distances are sorted per row)
    assert np.all(np.diff(p, axis=1) <= 1e-15)


def test_exact_gradient_closed_form():
    ref, idx, dist = _problem(n_ref=200, nq=30, k=12)
    p = oracle.transform_conditional_p(dist, 4.0)
    y = np.random.default_rng(3).normal(size=(30, 2))
    ex = 1.5
    g = oracle.transform_gradient(ref, idx, p, y, ex, n_negatives=256, exact_threshold=4096, iter_seed=11)
    d = y[:, None, :] - ref[None, :, :]                       # (nq, n_ref, 2)
    q = 1.0 / (1.0 + (d ** 2).sum(-1))
    rep = -((q ** 2)[..., None] * d).sum(1) / (q.sum(1)[:, None] + np.finfo(float).tiny)
    dn = y[:, None, :] - ref[idx - 1]                         # (nq, k, 2)
    qn = 1.0 / (1.0 + (dn ** 2).sum(-1))
    att = ex * ((p * qn)[..., None] * dn).sum(1)
    np.testing.assert_allclose(g, rep + att, rtol=1e-12, atol=1e-15)


def test_sampled_repulsion_is_a_ratio_estimate_of_the_exact_one():
    ref, idx, dist = _problem(n_ref=2000, nq=8, k=10, seed=5)
    p = np.zeros((8, 10))  # repulsion only
    y = np.random.default_rng(6).normal(size=(8, 2)) * 0.5
    exact = oracle.transform_gradient(ref, idx, p, y, 1.0, 4096, 4096, 1)
    acc = np.zeros_like(exact)
    draws = 400
    for s in range(draws):
        acc += oracle.transform_gradient(ref, idx, p, y, 1.0, 64, 16, 1000 + s)
    rel = np.linalg.norm(acc / draws - exact) / np.linalg.norm(exact)
    assert rel < 0.05, rel


def test_sampling_is_uniform_over_the_reference():
    # multiply-shift of xorshift32 outputs: counts per index are uniform
    out = oracle.xorshift32(oracle.hash32(12345), 200000).astype(np.uint64)
    n = 97
    counts = np.bincount(((out * np.uint64(n)) >> np.uint64(32)).astype(np.int64), minlength=n)
    chi2 = ((counts - counts.mean()) ** 2 / counts.mean()).sum()
    assert chi2 < 200  # 96 degrees of freedom


def test_median_and_weighted_init():
    ref, idx, dist = _problem(n_ref=150, nq=25, k=14)
    med = oracle.transform_init(ref, idx, dist, oracle.INIT_MEDIAN)
    np.testing.assert_array_equal(med, np.median(ref[idx - 1], axis=1))
    w = 1.0 / (np.maximum(dist, 0) + 1e-6)
    want = (w[..., None] * ref[idx - 1]).sum(1) / (w.sum(1)[:, None] + np.finfo(float).tiny)
    np.testing.assert_allclose(oracle.transform_init(ref, idx, dist, oracle.INIT_WEIGHTED), want, rtol=1e-14)
    # odd k: the middle value itself
    med_odd = oracle.transform_init(ref, idx[:, :13], dist[:, :13], oracle.INIT_MEDIAN)
    np.testing.assert_array_equal(med_odd, np.median(ref[idx[:, :13] - 1], axis=1))


def _libstdcxx_normal_pair(state_seed: int, sd: float):
    """normal_distribution<double> (Marsaglia polar, as libstdc++ implements
    it) fed by mt19937(state_seed); returns the first two values."""
    bg = np.random.MT19937()
    bg._legacy_seeding(state_seed)  # init_genrand: the std::mt19937 seeding

    def canonical():
        a, b = (float(v) for v in bg.random_raw(2))
        return (a + b * 2.0 ** 32) / 2.0 ** 64

    while True:
        x = 2.0 * canonical() - 1.0
        yv = 2.0 * canonical() - 1.0
        r2 = x * x + yv * yv
        if r2 <= 1.0 and r2 != 0.0:
            break
    mult = math.sqrt(-2.0 * math.log(r2) / r2)
    return yv * mult * sd, x * mult * sd


def test_random_init_follows_mt19937_and_polar_normal():
    ref, idx, dist = _problem(n_ref=50, nq=6, k=5)
    seed = 401
    y = oracle.transform_init(ref, idx, dist, oracle.INIT_RANDOM, seed=seed)
    for i in range(6):
        s = oracle.hash32(seed ^ (((i + 1) * 0x9E3779B9) & 0xFFFFFFFF))
        assert tuple(y[i]) == _libstdcxx_normal_pair(s, 1e-4)


def test_update_closed_form():
    rng = np.random.default_rng(9)
    n = 400
    y = rng.normal(size=(n, 2))
    upd = rng.normal(size=(n, 2)) * 0.1
    upd[:20] = 0.0
    gains = rng.uniform(0.005, 2.0, size=(n, 2))
    grad = rng.normal(size=(n, 2))
    grad[20:30] = 0.0
    lr, mom, gmax, smax = 0.1, 0.8, 0.25, 0.05
    g = grad.copy()
    gn = np.sqrt((g ** 2).sum(1))
    clip = gn ** 2 > gmax ** 2
    g[clip] *= (gmax / (gn[clip] + 1e-12))[:, None]
    same = np.sign(upd) == np.sign(g)
    w = np.where(same, gains * 0.8 + 0.01, gains + 0.2)
    w = np.maximum(w, 0.01)
    u = mom * upd - lr * w * g
    un = np.sqrt((u ** 2).sum(1))
    sc = un ** 2 > smax ** 2
    u[sc] *= (smax / (un[sc] + 1e-12))[:, None]
    y2, upd2, gains2, grad2 = y.copy(), upd.copy(), gains.copy(), grad.copy()
    oracle.transform_update(y2, upd2, gains2, grad2, lr, mom, gmax, smax)
    np.testing.assert_allclose(gains2, w, rtol=1e-15)
    np.testing.assert_allclose(upd2, u, rtol=1e-13, atol=1e-16)
    np.testing.assert_allclose(y2, y + u, rtol=1e-13, atol=1e-16)


def test_run_is_thread_invariant_and_composes_gradient_and_update():
    ref, idx, dist = _problem(n_ref=300, nq=40, k=15)
    kw = dict(perplexity=4.0, n_iter=5, n_negatives=10, exact_threshold=8, seed=406)
    a, exact = oracle.transform_run(ref, idx, dist, threads=1, **kw)
    b, _ = oracle.transform_run(ref, idx, dist, threads=4, **kw)
    assert not exact
    np.testing.assert_array_equal(a, b)
    # one iteration = gradient at the median init + update
    y0 = oracle.transform_init(ref, idx, dist, oracle.INIT_MEDIAN)
    one, _ = oracle.transform_run(ref, idx, dist, perplexity=4.0, n_iter=1, n_negatives=10, exact_threshold=8,
                                  seed=406, exaggeration=1.5)
    p = oracle.transform_conditional_p(dist, 4.0)
    g = oracle.transform_gradient(ref, idx, p, y0, 1.5, 10, 8, oracle.transform_iteration_seed(406, 0))
    y, u, w = y0.copy(), np.zeros_like(y0), np.ones_like(y0)
    oracle.transform_update(y, u, w, g, 0.1, 0.8, 0.25, float("inf"))
    np.testing.assert_array_equal(one, y)


def test_run_rejects_bad_input():
    ref, idx, dist = _problem()
    bad = idx.copy()
    bad[0, 0] = 10 ** 6
    with pytest.raises(ValueError, match="out of range"):
        oracle.transform_run(ref, bad, dist, n_iter=1)
    dneg = dist.copy()
    dneg[1, 1] = -1.0
    with pytest.raises(ValueError, match="finite and non-negative"):
        oracle.transform_run(ref, idx, dneg, n_iter=1)


# ---------------------------------------------------------------------------
# Reference-grid repulsion (config 3's precomputed reference grid)
# ---------------------------------------------------------------------------
def _grid_problem(n_ref=600, nq=150, k=12, seed=3):
    rng = np.random.default_rng(seed)
    centers = rng.normal(0, 6, size=(5, 2))
    lab = rng.integers(0, 5, size=n_ref)
    ref = centers[lab] + rng.normal(0, 1.0, size=(n_ref, 2))
    yq = ref[rng.integers(0, n_ref, size=nq)] + rng.normal(0, 0.5, size=(nq, 2))
    d2 = ((yq[:, None, :] - ref[None, :, :]) ** 2).sum(-1)
    idx = np.argsort(d2, axis=1)[:, :k]
    dist = np.sqrt(np.take_along_axis(d2, idx, axis=1))
    return ref, (idx + 1).astype(np.int32), dist, yq


def test_grid_node_fields_are_the_direct_sums(oracle_mod):
    """Z = sum_j q, F = sum_j q^2 (node - r_j) at every node, q = 1/(1+d^2),
    nodes at lo + (a + 1/2) h."""
    ref, idx, dist, yq = _grid_problem(n_ref=300, nq=40)
    geo, f = oracle_mod.transform_grid_fields(ref, yq, min_intervals=8, ints_in_interval=100.0)
    m = geo["nodes"]
    assert geo["boxes"] == 8 and m == 24
    h = geo["box_w"] / 3.0
    nodes = geo["lo"] + (np.arange(m) + 0.5) * h
    nx, ny = np.meshgrid(nodes, nodes)  # ny varies along axis 0: node (a, b) at f[b, a]
    dx = nx[..., None] - ref[:, 0]
    dy = ny[..., None] - ref[:, 1]
    q = 1.0 / (1.0 + dx * dx + dy * dy)
    np.testing.assert_allclose(f[..., 0], q.sum(-1), rtol=1e-12)
    np.testing.assert_allclose(f[..., 1], (q * q * dx).sum(-1), rtol=1e-11, atol=1e-14)
    np.testing.assert_allclose(f[..., 2], (q * q * dy).sum(-1), rtol=1e-11, atol=1e-14)
    # the square covers the reference and the queries with a margin
    lo, hi = geo["lo"], geo["lo"] + geo["boxes"] * geo["box_w"]
    allpts = np.vstack([ref, yq])
    assert lo < allpts.min() - 0.99 and hi > allpts.max() + 0.99


def test_grid_gradient_converges_to_the_exact_mode(oracle_mod):
    """Order-3 interpolation: the error against the exact mode's gradient
    falls about eightfold per halving of the box width."""
    ref, idx, dist, yq = _grid_problem()
    p = oracle_mod.transform_conditional_p(dist, 5.0)
    exact = oracle_mod.transform_gradient(ref, idx, p, yq, 1.0, 10 ** 6, 10 ** 6, 0)
    errs = []
    for ints in (2.0, 1.0, 0.5, 0.25):
        g, outside = oracle_mod.transform_grid_gradient(ref, idx, p, yq, 1.0, min_intervals=1, ints_in_interval=ints)
        assert outside == 0
        errs.append(float(np.linalg.norm(g - exact) / np.linalg.norm(exact)))
    assert all(b < a / 4.0 for a, b in zip(errs, errs[1:])), errs
    # two boxes per unit (the HIP grid transform's default): ~0.15 %
    assert errs[2] < 2e-3 and errs[3] < 3e-4, errs
    # the repulsion alone (exaggeration 0 leaves the attraction out)
    rep_exact = oracle_mod.transform_gradient(ref, idx, p, yq, 0.0, 10 ** 6, 10 ** 6, 0)
    rep_grid, _ = oracle_mod.transform_grid_gradient(ref, idx, p, yq, 0.0, min_intervals=1, ints_in_interval=0.25)
    assert np.linalg.norm(rep_grid - rep_exact) / np.linalg.norm(rep_exact) < 3e-4


def test_grid_queries_outside_take_the_exact_sums(oracle_mod):
    ref, idx, dist, yq = _grid_problem()
    p = oracle_mod.transform_conditional_p(dist, 5.0)
    far = yq + np.array([400.0, -350.0])
    g, outside = oracle_mod.transform_grid_gradient(ref, idx, p, far, 1.0, geometry_y=yq)
    assert outside == far.shape[0]
    exact = oracle_mod.transform_gradient(ref, idx, p, far, 1.0, 10 ** 6, 10 ** 6, 0)
    np.testing.assert_array_equal(g, exact)


def test_grid_run_approaches_the_exact_run(oracle_mod):
    ref, idx, dist, yq = _grid_problem()
    kw = dict(perplexity=5.0, n_iter=40, learning_rate=0.1, exaggeration=1.0, seed=4)
    y_exact, exact = oracle_mod.transform_run(ref, idx, dist, n_negatives=10 ** 6, exact_threshold=10 ** 6, **kw)
    assert exact
    y_grid, st = oracle_mod.transform_grid_run(ref, idx, dist, ints_in_interval=0.25, min_intervals=1, **kw)
    assert st["exact_evaluations"] == 0 and st["nodes"] == 3 * st["boxes"]
    scale = np.abs(y_exact).max()
    # the gradient error (~2e-4 at this box width) carried through 40 steps
    assert np.abs(y_grid - y_exact).max() < 1e-3 * scale
