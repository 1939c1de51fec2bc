"""FIt-SNE interpolation grid on the GPU against the oracle (through the C ABI).

The reference's native backends have only the bilinear grid; this mode is an
extension that the benchmark configurations ask for (3 interpolation points
per interval, at least 50 intervals).  Its checker is the oracle's fp64
restatement (gradient_lagrange), itself pinned against the exact O(n^2)
gradient and a direct node sum in tests/test_oracle_lagrange.py.

Tolerances:
  gradient from the same y        relative L2 error <= 1e-3 (fp32 FFTs and
                                  float atomics against an fp64 oracle)
  box count and node count        identical to the oracle's
  final KL divergence             within 1 % of the oracle's
"""

import sys

import numpy as np
import pytest

from fastembedr_amd import _lib, synthetic
from tests.helpers import rel_l2, small_problem

pytestmark = pytest.mark.gpu

GRAD_TOL = 1e-3
LAGRANGE = _lib.REPULSION_LAGRANGE


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def prob():
    x, labels, idx, dist = small_problem(n=3000, dim=20, k=45, components=6, seed=21)
    return x, idx, dist, synthetic.pca_init(x)


def _with_span(y0, span):
    y = y0 - y0.mean(axis=0)
    return (y * (span / float(y.max() - y.min()))).astype(np.float32)


# span -> boxes -> nodes -> FFT length (the smallest 2^a or 3 * 2^a >= 2 nodes,
# at least 64): 8/min 10 -> 10 -> 30 -> 64; 15/min 10 -> 15 -> 45 -> 96;
# 30/min 10 -> 30 -> 90 -> 192; 30 -> 50 -> 150 -> 384; 80 -> 240 -> 512;
# 120 -> 360 -> 768; 250 -> 750 -> 1536; 300 -> 900 -> 2048;
# 400 -> 1200 -> 3072; 700 -> capped 682 -> 2046 -> 4096
@pytest.mark.parametrize("span,min_int,ex,fft", [(8.0, 10, 12.0, 64), (15.0, 10, 12.0, 96), (30.0, 10, 1.0, 192),
                                                 (30.0, 50, 1.0, 384), (80.0, 50, 1.0, 512), (120.0, 50, 1.0, 768),
                                                 (250.0, 50, 1.0, 1536), (300.0, 50, 1.0, 2048),
                                                 (400.0, 50, 1.0, 3072), (700.0, 50, 1.0, 4096)])
def test_interp_gradient_matches_oracle(hip, oracle_mod, prob, span, min_int, ex, fft):
    x, idx, dist, y0 = prob
    y = _with_span(y0, span)
    _say(f"case: interpolation-grid gradient, span {span}, min_intervals {min_int}, exaggeration {ex}")
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        s.set_repulsion(LAGRANGE, 3, min_int, 1.0)
        s.set_state(y)
        g = s.gradient(ex, LAGRANGE)
        info = s.interp_info()
        P = oracle_mod.OracleP.wrap(*s.csr())
    g0, geo, _ = P.lagrange_gradient(y, ex, order=3, min_intervals=min_int, threads=8)
    err = rel_l2(g, g0)
    _say(f"  boxes {info['boxes']} nodes {info['nodes']} fft {info['fft_len']}: relL2 {err:.2e}")
    assert (info["boxes"], info["nodes"]) == (geo["boxes"], geo["nodes"])
    assert info["fft_len"] == fft >= 2 * info["nodes"]
    assert err <= GRAD_TOL


def test_interp_gradient_settings(hip, oracle_mod, prob):
    """ints_in_interval and min_num_intervals reach the device geometry."""
    x, idx, dist, y0 = prob
    y = _with_span(y0, 40.0)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        P = oracle_mod.OracleP.wrap(*s.csr())
        s.set_state(y)
        for min_int, ipu in ((20, 0.5), (100, 1.0), (5, 4.0)):
            s.set_repulsion(LAGRANGE, 3, min_int, ipu)
            g = s.gradient(1.0, LAGRANGE)
            info = s.interp_info()
            g0, geo, _ = P.lagrange_gradient(y, 1.0, order=3, min_intervals=min_int, ints_per_unit=ipu, threads=8)
            _say(f"  min_intervals {min_int} ints_in_interval {ipu}: boxes {info['boxes']} relL2 {rel_l2(g, g0):.2e}")
            assert info["boxes"] == geo["boxes"]
            assert rel_l2(g, g0) <= GRAD_TOL


def test_interp_settings_errors(hip, prob):
    x, idx, dist, y0 = prob
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        for args in ((LAGRANGE, 4, 50, 1.0), (LAGRANGE, 3, 0, 1.0), (LAGRANGE, 3, 50, 0.0),
                     (_lib.REPULSION_EXACT, 3, 50, 1.0)):
            with pytest.raises(_lib.HipBackendError):
                s.set_repulsion(*args)


@pytest.mark.parametrize("phase", ["early", "normal"])
def test_interp_each_iteration_matches_oracle(hip, oracle_mod, prob, phase):
    """One device iteration (interpolation-grid gradient, update, centring)
    against one oracle iteration from the device's own state, at every step."""
    x, idx, dist, y0 = prob
    n = x.shape[0]
    ex, mom = (12.0, 0.5) if phase == "early" else (1.0, 0.8)
    _say(f"case: interpolation-grid per-iteration parity ({phase} phase)")
    start = _with_span(y0, 2.0 if phase == "early" else 60.0)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        P = oracle_mod.OracleP.wrap(*s.csr())
        s.set_repulsion(LAGRANGE, 3, 50, 1.0)
        s.set_state(start)
        s.center()
        worst = 0.0
        for t in range(6):
            y, u, g = s.get_state()
            s.run(1, ex, mom, n / 12.0, 0.01, 5.0)
            y1, u1, g1 = s.get_state()
            yr, ur, gr = y.copy(), u.copy(), g.copy()
            grad, _, _ = P.lagrange_gradient(yr, ex, order=3, min_intervals=50, threads=8)
            oracle_mod.update(yr, ur, gr, grad, n / 12.0, mom)
            oracle_mod.zero_mean(yr)
            err = rel_l2(y1 - y, yr - y)
            worst = max(worst, err)
            assert err <= GRAD_TOL, (t, err)
        _say(f"  worst per-step relL2 {worst:.2e}")


@pytest.mark.parametrize("clip", [5.0, 0.0])
def test_interp_fft_length_follows_growing_span(hip, prob, clip):
    """A run whose span grows across an FFT-length threshold (342 boxes:
    1026 nodes need length 3072 instead of 2048; 513 would need 4096).  The
    host picks each iteration's FFT length from a lagged box count and the
    step-clip bound, or waits for the current count without the clip; the
    device flags any length too small for its node count, and sync() reports
    the flag."""
    x, idx, dist, y0 = prob
    n = x.shape[0]
    _say(f"case: growing span, max_step_norm {clip}")
    # weak attraction and a large step: repulsion pushes the layout outwards
    lr = 100.0 * n if clip > 0 else 30.0 * n
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        s.set_repulsion(LAGRANGE, 3, 50, 1.0)
        s.set_state(_with_span(y0, 330.0))
        s.center()
        s.run(12, 0.05, 0.5, lr, 0.01, clip)
        s.sync()
        info = s.interp_info()
        y = s.y
    _say(f"  after 12 iterations: span {float(np.ptp(y)):.1f}, boxes {info['boxes']} fft {info['fft_len']}")
    assert np.all(np.isfinite(y))
    assert 342 <= info["boxes"] <= 512 and info["fft_len"] == 3072


def _drifting(y0, span):
    """A layout with a long right tail in x and a long lower tail in y, and an
    update that moves the bulk by (-3.4, 3.4) while the largest x moves +5 in
    x and the smallest y moves -5 in y: the mean moves, so the centred extremes
    move by up to 2 max_step_norm each and the two-axis span grows ~17 boxes
    per iteration (against the 10 that a one-axis bound of 2 max_step_norm
    allows)."""
    y = (y0 - y0.mean(axis=0)).astype(np.float64)
    y[:, 0] += 0.6 * np.abs(y[:, 0])
    y[:, 1] -= 0.6 * np.abs(y[:, 1])
    y -= y.mean(axis=0)
    y = (y * (span / float(y.max() - y.min()))).astype(np.float32)
    u = np.tile(np.array([-3.4, 3.4], np.float32), (len(y), 1))
    u[np.argmax(y[:, 0])] = (5.0, 0.0)
    u[np.argmin(y[:, 1])] = (0.0, -5.0)
    return y, u


def test_interp_fft_length_bound_holds_for_drifting_layout(hip, prob):
    """The lagged FFT-length bound with a drifting layout: from 300 boxes the
    span reaches ~351 boxes (1053 nodes, FFT length 3072) after 3 iterations
    and ~500 after twelve.
    Twelve iterations in one call must raise no device flag and agree with the
    same twelve taken one call at a time (exact FFT length each time)."""
    x, idx, dist, y0 = prob
    _say("case: drifting layout, lagged FFT length")
    start, u0 = _drifting(y0, 300.0)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        s.set_repulsion(LAGRANGE, 3, 50, 1.0)
        s.set_state(start, u0)
        s.run(12, 1.0, 1.0, 1.0, 0.01, 5.0)
        s.sync()
        info = s.interp_info()
        y_lag = s.y
        s.set_state(start, u0)
        for _ in range(12):
            s.run(1, 1.0, 1.0, 1.0, 0.01, 5.0)
        s.sync()
        y_one = s.y
    err = rel_l2(y_lag - start, y_one - start)
    _say(f"  boxes {info['boxes']} fft {info['fft_len']}: displacement relL2 {err:.2e}")
    assert np.all(np.isfinite(y_lag))
    assert info["boxes"] >= 342 and info["fft_len"] >= max(3072, 2 * info["nodes"])
    assert err <= 1e-4


def test_interp_lagged_fft_length_agrees_with_exact(hip, prob):
    """Twelve iterations in one call (the FFT length comes from the lagged
    bound: 330 boxes known, up to 348 allowed, so length 3072) against the
    same twelve taken one call at a time (each call reads the current count:
    990 nodes, length 2048).  The padding differs, the convolution does not:
    the layouts agree to rounding."""
    x, idx, dist, y0 = prob
    n = x.shape[0]
    _say("case: lagged vs exact FFT length")
    start = _with_span(y0, 330.0)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        s.set_repulsion(LAGRANGE, 3, 50, 1.0)
        s.set_state(start)
        s.center()
        s.run(12, 1.0, 0.8, n / 12.0, 0.01, 5.0)
        lag_fft = s.interp_info()["fft_len"]
        y_lag = s.y
        s.set_state(start)
        s.center()
        for _ in range(12):
            s.run(1, 1.0, 0.8, n / 12.0, 0.01, 5.0)
        one_fft = s.interp_info()["fft_len"]
        y_one = s.y
    err = rel_l2(y_lag - start, y_one - start)
    _say(f"  fft lagged {lag_fft}, stepwise {one_fft}: displacement relL2 {err:.2e}")
    assert (lag_fft, one_fft) == (3072, 2048)
    assert err <= 1e-4


def test_interp_end_to_end_kl(hip, oracle_mod, prob):
    """Full schedule (250 early-exaggeration + 500 iterations) with the
    interpolation grid from the same PCA initialisation as the oracle's
    interpolation-grid run; final exact KL within 1 %."""
    x, idx, dist, y0 = prob
    n = x.shape[0]
    _say("case: interpolation grid end to end, n=3000")
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        P = oracle_mod.OracleP.wrap(*s.csr())
        s.set_repulsion(LAGRANGE, 3, 50, 1.0)
        s.set_state(y0)
        s.center()
        s.run(250, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        s.run(500, 1.0, 0.8, n / 12.0, 0.01, 5.0)
        y_hip = s.y
        info = s.interp_info()
    y_cpu, _, _ = P.optimize(y0, 250, 500, 12.0, 1.0, n / 12.0, False, 0.5, 0.8,
                             method=oracle_mod.METHOD_LAGRANGE, threads=8)
    kl_hip = P.kl(y_hip, threads=8)
    kl_cpu = P.kl(y_cpu, threads=8)
    _say(f"  boxes {info['boxes']}: KL hip={kl_hip:.5f} oracle={kl_cpu:.5f}")
    assert np.all(np.isfinite(y_hip))
    assert abs(kl_hip - kl_cpu) <= 0.01 * kl_cpu


def test_opentsne_knn_interpolation_grid(hip, oracle_mod, prob):
    """The API mirror's interpolation_grid option runs the same schedule on
    the FIt-SNE grid: the layout equals a session run with the same settings
    from the same initialisation (a few iterations: longer runs diverge by
    the amplified reordering of float atomics, as two session runs do), and
    the result is labelled as such."""
    x, idx, dist, y0 = prob
    n = x.shape[0]
    _say("case: opentsne_knn with interpolation_grid")
    y0 = _with_span(y0, 20.0)
    res = hip.opentsne_knn(idx, dist, n_neighbors=45, perplexity=15.0, Y_init=y0, early_exaggeration_iter=3,
                           n_iter=2, initial_momentum=0.5, interpolation_grid={"min_num_intervals": 40})
    assert res.config["repulsion"] == "fitsne_interpolation_grid_hip"
    assert res.config["interpolation_grid"] == {"n_interpolation_points": 3, "min_num_intervals": 40,
                                                "ints_in_interval": 1.0}
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        s.set_repulsion(LAGRANGE, 3, 40, 1.0)
        s.set_state(y0)
        s.center()
        y_start = s.y
        s.run(3, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        s.run(2, 1.0, 0.8, n / 12.0, 0.01, 5.0)
        y = s.y
    err = rel_l2(res.layout - y_start, y - y_start)
    _say(f"  API vs session displacement relL2 {err:.2e}")
    assert err <= 1e-4
    with pytest.raises(ValueError):
        hip.opentsne_knn(idx, dist, n_neighbors=45, perplexity=15.0, interpolation_grid={"order": 3})


def _relabel(idx, dist, y, order):
    """The same problem with point order[j] renamed j: KNN rows and their
    1-based indices, and the layout."""
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    idx_new = np.asfortranarray((inv[np.asarray(idx)[order] - 1] + 1).astype(np.int32))
    dist_new = np.asfortranarray(np.asarray(dist)[order])
    return idx_new, dist_new, np.ascontiguousarray(y[order])


@pytest.mark.parametrize("n_keep", [3000, 2945])
def test_interp_spread_independent_of_point_order(hip, oracle_mod, prob, n_keep):
    """The spread sums each wave's runs of points that share a box, so run
    structure must not matter: the same points in random order (runs of about
    one point), in box order (runs of up to 64), and with a ragged last wave
    (2945 = 46 * 64 + 1 points) give the oracle's gradient; a layout with every
    point on one spot (one box, one run per wave) stays finite and matches."""
    x, idx, dist, y0 = prob
    if n_keep < idx.shape[0]:
        small = small_problem(n=n_keep, dim=20, k=45, components=6, seed=21)
        x, idx, dist = small[0], small[2], small[3]
        y0 = synthetic.pca_init(x)
    y = _with_span(y0, 60.0)
    n = y.shape[0]
    rng = np.random.default_rng(7)
    boxes = np.floor((y - y.min(0)) / 1.0).astype(np.int64)
    orders = {"random": rng.permutation(n), "box": np.lexsort((boxes[:, 0], boxes[:, 1]))}
    _say(f"case: interpolation-grid spread under point orders, n {n}")
    for name, order in orders.items():
        idx_o, dist_o, y_o = _relabel(idx, dist, y, order)
        with hip.TsneSession(idx_o, dist_o, perplexity=15.0, index_offset=1) as s:
            s.set_repulsion(LAGRANGE, 3, 50, 1.0)
            s.set_state(y_o)
            g = s.gradient(1.0, LAGRANGE)
            P = oracle_mod.OracleP.wrap(*s.csr())
        g0, _, _ = P.lagrange_gradient(y_o, 1.0, order=3, min_intervals=50, threads=8)
        err = rel_l2(g, g0)
        _say(f"  {name} order: relL2 {err:.2e}")
        assert err <= GRAD_TOL
    # every point on one spot, plus one far away: one box holds all but one
    y1 = np.zeros_like(y)
    y1[-1] = (30.0, -20.0)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        s.set_repulsion(LAGRANGE, 3, 50, 1.0)
        s.set_state(y1)
        g = s.gradient(1.0, LAGRANGE)
        P = oracle_mod.OracleP.wrap(*s.csr())
    g0, _, _ = P.lagrange_gradient(y1, 1.0, order=3, min_intervals=50, threads=8)
    err = rel_l2(g, g0)
    _say(f"  one crowded box: relL2 {err:.2e}")
    assert np.all(np.isfinite(g)) and err <= GRAD_TOL


@pytest.mark.parametrize("dense", ["0", "0.001"])
def test_interp_spread_table_sizes(hip, oracle_mod, prob, monkeypatch, dense):
    """The spread's two LDS tables give the oracle's gradient:
    FASTEMBEDR_HIP_SPREAD_DENSE=0 forces the 256-slot table, 0.001 the 64-slot
    one, whatever the density.  Gradient probes at 30, 7.5 and 0.8 points per
    box (a fresh spread order: few boxes per wave of 64 points in the first,
    more than eight in the last, where the grouping keeps the order and the
    small table overflows into its straggler path), then 40 iterations of
    run() checked step by step, so that the order ages while the grid drifts
    away from the lattice it was made on (the case the grouping is for)."""
    x, idx, dist, y0 = prob
    monkeypatch.setenv("FASTEMBEDR_HIP_SPREAD_DENSE", dense)
    n = x.shape[0]
    for span, min_int in ((8.0, 10), (20.0, 10), (60.0, 50)):
        y = _with_span(y0, span)
        _say(f"case: spread table (dense threshold {dense}), gradient at span {span}")
        with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
            s.set_repulsion(LAGRANGE, 3, min_int, 1.0)
            s.set_state(y)
            g = s.gradient(1.0, LAGRANGE)
            P = oracle_mod.OracleP.wrap(*s.csr())
        g0, _, _ = P.lagrange_gradient(y, 1.0, order=3, min_intervals=min_int, threads=8)
        err = rel_l2(g, g0)
        _say(f"  relL2 {err:.2e}")
        assert np.all(np.isfinite(g)) and err <= GRAD_TOL
    _say(f"case: spread table (dense threshold {dense}), 40 iterations step by step")
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        P = oracle_mod.OracleP.wrap(*s.csr())
        s.set_repulsion(LAGRANGE, 3, 10, 1.0)
        s.set_state(_with_span(y0, 8.0))
        s.center()
        worst = 0.0
        for t in range(40):
            y, u, g = s.get_state()
            s.run(1, 1.0, 0.8, n / 12.0, 0.01, 5.0)
            y1, _, _ = s.get_state()
            yr, ur, gr = y.copy(), u.copy(), g.copy()
            grad, _, _ = P.lagrange_gradient(yr, 1.0, order=3, min_intervals=10, threads=8)
            oracle_mod.update(yr, ur, gr, grad, n / 12.0, 0.8)
            oracle_mod.zero_mean(yr)
            err = rel_l2(y1 - y, yr - y)
            worst = max(worst, err)
            assert err <= GRAD_TOL, (t, err)
        _say(f"  worst per-step relL2 {worst:.2e}")
