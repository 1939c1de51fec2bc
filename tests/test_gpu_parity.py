"""HIP backend vs the CPU oracle on identical seeded inputs (through the C ABI).

Tolerances:
  P (conditional and symmetric)   relative L2 error <= 1e-5, identical sparsity
  gradient from the same y        relative L2 error <= 1e-3 (float atomics and
                                  parallel sums reorder fp32 additions)
  final KL divergence             within 1 % of the oracle's
  15-NN preservation              within 0.01 of the oracle's
"""

import ctypes as C
import sys

import numpy as np
import pytest

from fastembedr_amd import _lib, synthetic
from tests.helpers import DeviceArray, knn_preservation, rel_l2, small_problem

pytestmark = pytest.mark.gpu

P_TOL = 1e-5
GRAD_TOL = 1e-3


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def mid_problem():
    x, labels, idx, dist = small_problem(n=3000, dim=20, k=45, components=6, seed=21)
    return x, idx, dist


@pytest.fixture(scope="module")
def config0():
    spec = synthetic.CONFIGS[0]
    x, labels = synthetic.gaussian_mixture(spec, seed=1)
    idx, dist = synthetic.exact_knn_numpy(x, 90)
    idx_r, dist_r = synthetic.to_r_layout(idx, dist, one_based=True)
    return x, idx_r, dist_r, synthetic.pca_init(x)


def test_conditional_p_matches_oracle(hip, oracle_mod, mid_problem):
    _say("case: conditional P, n=3000 k=45 perplexity=15")
    x, idx, dist = mid_problem
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        pc = s.conditional_p()
    ref, _, steps = oracle_mod.conditional_p(dist, 15.0)
    assert rel_l2(pc, ref) <= P_TOL
    same = np.mean(pc == ref)
    _say(f"bit-identical conditional entries: {same:.4f}")
    assert same > 0.5


@pytest.mark.parametrize("n,k,perp", [(3000, 45, 15.0), (10000, 90, 30.0)])
def test_symmetric_p_matches_oracle(hip, oracle_mod, n, k, perp):
    _say(f"case: symmetric P n={n} k={k}")
    x, _, idx, dist = small_problem(n=n, dim=30, k=k, components=8, seed=n)
    with hip.TsneSession(idx, dist, perplexity=perp, index_offset=1) as s:
        rp, col, val = s.csr()
        build_ms = s.p_build_ms
    _say(f"P build {build_ms:.2f} ms, nnz {col.size}")
    P = oracle_mod.OracleP.build(idx, dist, perp, threads=4)
    rp0, col0, val0 = P.csr()
    np.testing.assert_array_equal(rp, rp0)
    np.testing.assert_array_equal(col, col0)
    assert rel_l2(val, val0) <= P_TOL
    assert abs(float(val.astype(np.float64).sum()) - 1.0) < 1e-5


def test_p_with_self_columns_and_zero_based(hip, oracle_mod):
    _say("case: P with a self column, 0-based indices")
    x, _, idx, dist = small_problem(n=800, k=20, one_based=False)
    idx2 = np.asfortranarray(np.concatenate([np.arange(800)[:, None], idx[:, :-1]], axis=1).astype(np.int32))
    dist2 = np.asfortranarray(np.concatenate([np.zeros((800, 1), np.float32), dist[:, :-1]], axis=1))
    with hip.TsneSession(idx2, dist2, perplexity=5.0, index_offset=0) as s:
        rp, col, val = s.csr()
    P = oracle_mod.OracleP.build(idx2, dist2, 5.0)
    rp0, col0, val0 = P.csr()
    np.testing.assert_array_equal(rp, rp0)
    np.testing.assert_array_equal(col, col0)
    assert rel_l2(val, val0) <= P_TOL


def test_p_single_neighbor_and_duplicates(hip, oracle_mod):
    _say("case: P with k=1 and with a duplicated neighbour")
    x, _, idx, dist = small_problem(n=300, k=6)
    for i2, d2, perp in ((idx[:, :1], dist[:, :1], 0.5), (idx, dist, 1.5)):
        i2 = np.asfortranarray(i2.copy())
        d2 = np.asfortranarray(d2.copy())
        if i2.shape[1] > 1:
            i2[::5, 1] = i2[::5, 0]
            d2[::5, 1] = d2[::5, 0]
        with hip.TsneSession(i2, d2, perplexity=perp, index_offset=1) as s:
            rp, col, val = s.csr()
        rp0, col0, val0 = oracle_mod.OracleP.build(i2, d2, perp).csr()
        np.testing.assert_array_equal(col, col0)
        assert rel_l2(val, val0) <= P_TOL


def test_p_input_errors(hip):
    _say("case: P input validation")
    x, _, idx, dist = small_problem(n=200, k=8)
    bad = idx.copy()
    bad[7, 3] = 10_000
    with pytest.raises(_lib.HipBackendError, match="out of range"):
        hip.TsneSession(bad, dist, perplexity=2.0, index_offset=1)
    badd = dist.copy()
    badd[9, 1] = np.nan
    with pytest.raises(_lib.HipBackendError, match="finite and non-negative"):
        hip.TsneSession(idx, badd, perplexity=2.0, index_offset=1)
    with pytest.raises(_lib.HipBackendError, match="at most 256"):
        hip.TsneSession(np.ones((300, 257), np.int32), np.ones((300, 257), np.float32), perplexity=2.0)


@pytest.mark.parametrize("grid", [0, 32, 128, 512, 1024])
def test_gradient_matches_oracle(hip, oracle_mod, mid_problem, grid):
    _say(f"case: gradient grid={grid}")
    x, idx, dist = mid_problem
    rng = np.random.default_rng(grid + 1)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1, grid_size=grid) as s:
        P = oracle_mod.OracleP.wrap(*s.csr())
        for scale, ex in ((1e-4, 12.0), (2.0, 12.0), (25.0, 1.0)):
            y = (rng.standard_normal((3000, 2)) * scale).astype(np.float32)
            s.set_state(y)
            g = s.gradient(ex)
            ref = P.gradient(y, ex, grid_size=grid if grid else 0, threads=4)
            err = rel_l2(g, ref)
            _say(f"  scale={scale} ex={ex} relL2={err:.2e}")
            assert err <= GRAD_TOL


def test_exact_gradient_matches_oracle(hip, oracle_mod, mid_problem):
    _say("case: exact gradient")
    x, idx, dist = mid_problem
    rng = np.random.default_rng(3)
    y = (rng.standard_normal((3000, 2)) * 5).astype(np.float32)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        P = oracle_mod.OracleP.wrap(*s.csr())
        s.set_state(y)
        g = s.gradient(4.0, repulsion=_lib.REPULSION_EXACT)
    ref = P.gradient(y, 4.0, method=oracle_mod.METHOD_EXACT, threads=4)
    assert rel_l2(g, ref) <= 1e-5


@pytest.mark.parametrize("phase", ["early", "normal"])
def test_each_iteration_matches_oracle(hip, oracle_mod, mid_problem, phase):
    """Per-iteration parity: from the device's own state (y, update, gains) at
    every step, one oracle iteration (gradient, update, centring) and one
    device iteration agree; the step taken (y_{t+1} - y_t) to the gradient
    tolerance, and the gains exactly except where a gradient component sits
    at rounding level."""
    x, idx, dist = mid_problem
    n = x.shape[0]
    ex, mom = (12.0, 0.5) if phase == "early" else (1.0, 0.8)
    _say(f"case: per-iteration parity ({phase} phase)")
    y0 = synthetic.pca_init(x) * (1.0 if phase == "early" else 3e4)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        P = oracle_mod.OracleP.wrap(*s.csr())
        s.set_state(y0)
        s.center()
        if phase == "normal":
            s.run(30, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        worst = 0.0
        for t in range(12):
            y, u, g = s.get_state()
            s.run(1, ex, mom, n / 12.0, 0.01, 5.0)
            y1, u1, g1 = s.get_state()
            yr, ur, gr = y.copy(), u.copy(), g.copy()
            grad = P.gradient(yr, ex, threads=4)
            oracle_mod.update(yr, ur, gr, grad, n / 12.0, mom)
            oracle_mod.zero_mean(yr)
            err = rel_l2(y1 - y, yr - y)
            worst = max(worst, err)
            assert err <= GRAD_TOL, (t, err)
            assert np.mean(g1 != gr) <= 1e-3, t
        _say(f"  worst per-step relL2 {worst:.2e}")


def test_free_run_divergence_is_rounding_level(hip, oracle_mod, mid_problem):
    """Twenty free-running iterations from the same initialisation.  The
    iteration amplifies rounding (sign-driven gains, early exaggeration), so
    the yardstick is the oracle against itself: the same run started from a
    layout perturbed by about four ulps.  The device run may not diverge from
    the oracle by more than a small multiple of that."""
    x, idx, dist = mid_problem
    n = x.shape[0]
    _say("case: 20 free-running iterations")
    y0 = synthetic.pca_init(x)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        P = oracle_mod.OracleP.wrap(*s.csr())
        s.set_state(y0)
        s.center()
        s.run(20, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        y20 = s.y
    args = (20, 0, 12.0, 1.0, n / 12.0, False, 0.5, 0.8)
    yo, _, _ = P.optimize(y0, *args, threads=4)
    rng = np.random.default_rng(0)
    y0p = (y0 * (1.0 + 4.8e-7 * rng.standard_normal(y0.shape))).astype(np.float32)
    yp, _, _ = P.optimize(y0p, *args, threads=4)
    err = rel_l2(y20, yo)
    ref = rel_l2(yp, yo)
    _say(f"  20 iterations relL2 hip-vs-oracle={err:.2e}, oracle-vs-perturbed-oracle={ref:.2e}")
    assert err <= max(5.0 * ref, 1e-4)


def test_kl_matches_oracle(hip, oracle_mod, mid_problem):
    _say("case: exact KL on the device")
    x, idx, dist = mid_problem
    rng = np.random.default_rng(12)
    y = (rng.standard_normal((3000, 2)) * 3).astype(np.float32)
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        s.set_state(y)
        kl = s.kl()
        kl2, rows = s.kl_rows()
        P = oracle_mod.OracleP.wrap(*s.csr())
        # after iterations the session works in its own (renumbered) order
        s.run(30, 12.0, 0.5, 3000 / 12.0)
        s.sync()
        y_run = s.y
        assert s.attraction_info()["renumbers"] >= 1
        kl_run, rows_run = s.kl_rows()
    ref, ref_rows = P.kl(y, threads=4, row_costs=True)
    assert abs(kl - ref) <= 1e-6 * abs(ref)
    assert kl2 == kl
    # each row's term (the reference's per-row `costs`), in the caller's numbering
    assert np.abs(rows - ref_rows).max() <= 1e-6 * np.abs(ref_rows).max()
    assert abs(float(rows.sum()) - kl) <= 1e-9 * abs(kl)
    ref_run, ref_rows_run = P.kl(y_run, threads=4, row_costs=True)
    assert abs(kl_run - ref_run) <= 1e-6 * abs(ref_run)
    assert np.abs(rows_run - ref_rows_run).max() <= 1e-6 * np.abs(ref_rows_run).max()


def _one_shot(fn_name, idx, dist, init, n_early, n_norm, device=False, shape=None):
    lib = _lib.load()
    n, k = shape if device else idx.shape
    out = np.empty((n, 2), np.float32)
    fn = getattr(lib, fn_name)
    rc = fn(C.c_void_p(idx) if device else C.c_void_p(idx.ctypes.data),
            C.c_void_p(dist) if device else C.c_void_p(dist.ctypes.data),
            C.c_void_p(init.ctypes.data) if init is not None else None, int(init is not None), n, k, 2, 30.0,
            n_early, n_norm, 12.0, 1.0, n / 12.0, 0, 0.5, 0.8, 0.01, 5.0, 1, 1, C.c_void_p(out.ctypes.data))
    _lib.check(rc, fn_name)
    return out


def test_end_to_end_config0_kl_and_knn_preservation(hip, oracle_mod, config0):
    """Config 0 (10,000 x 50, k=90, perplexity 30, 250 + 500 iterations),
    one-shot C ABI vs the oracle's full run from the same PCA init."""
    x, idx, dist, y0 = config0
    n = x.shape[0]
    _say("case: config 0 end to end (one-shot ABI)")
    y_hip = _one_shot("fastembedr_hip_opentsne_fft_from_knn_float", idx, dist, y0, 250, 500)
    P = oracle_mod.OracleP.build(idx, dist, 30.0, threads=8)
    y_cpu, _, _ = P.optimize(y0, 250, 500, 12.0, 1.0, n / 12.0, False, 0.5, 0.8, threads=8)
    kl_hip = P.kl(y_hip, threads=8)
    kl_cpu = P.kl(y_cpu, threads=8)
    pres_hip = knn_preservation(x, y_hip, 15)
    pres_cpu = knn_preservation(x, y_cpu, 15)
    _say(f"  KL hip={kl_hip:.5f} cpu={kl_cpu:.5f}; 15-NN hip={pres_hip:.4f} cpu={pres_cpu:.4f}")
    assert np.all(np.isfinite(y_hip))
    assert abs(kl_hip - kl_cpu) <= 0.01 * kl_cpu
    assert abs(pres_hip - pres_cpu) <= 0.01


def test_one_shot_variants_agree(hip, mid_problem):
    """double-distance and device-KNN entry points give the float entry's result."""
    _say("case: one-shot variants")
    x, idx, dist = mid_problem
    y0 = synthetic.pca_init(x)
    a = _one_shot("fastembedr_hip_opentsne_fft_from_knn_float", idx, dist, y0, 5, 5)
    b = _one_shot("fastembedr_hip_opentsne_fft_from_knn", idx, np.asfortranarray(dist, np.float64), y0, 5, 5)
    di = DeviceArray(np.asfortranarray(idx, np.int32).T)  # (k, n) C-order bytes == (n, k) column-major
    dd = DeviceArray(np.asfortranarray(dist, np.float32).T)
    try:
        c = _one_shot("fastembedr_hip_opentsne_fft_from_device_knn_float", di.address, dd.address, y0, 5, 5,
                      device=True, shape=idx.shape)
    finally:
        di.free()
        dd.free()
    assert rel_l2(b, a) <= GRAD_TOL
    assert rel_l2(c, a) <= GRAD_TOL


def test_random_init_matches_reference_generator(hip, oracle_mod):
    lib = _lib.load()
    y = np.empty((1000, 2), np.float32)
    _lib.check(lib.fastembedr_hip_random_init(1000, 42, C.c_void_p(y.ctypes.data)), "random_init")
    np.testing.assert_array_equal(y, oracle_mod.random_init(1000, 42))


def test_opentsne_knn_api(hip):
    _say("case: opentsne_knn API mirror")
    x, _, idx, dist = small_problem(n=1200, k=40, seed=8)
    res = hip.opentsne_knn(idx, dist, n_neighbors=30, perplexity=10.0, early_exaggeration_iter=30, n_iter=40,
                           seed=3)
    assert res.layout.shape == (1200, 2) and np.all(np.isfinite(res.layout))
    assert res.config["backend"] == "hip"
    assert res.config["optimizer"] == "opentsne_fitsne_fft_grid_native_hip"
    assert res.config["repulsion"] == "fft_grid_hip"
    assert res.config["learning_rate"] == "auto_opt_sne_n_over_early_exaggeration"
    assert res.config["learning_rate_early"] == res.config["learning_rate_normal"] == 1200 / 12.0
    rec = hip.opentsne_knn({"indices": idx, "distances": dist}, n_neighbors=30, perplexity=10.0,
                           early_exaggeration_iter=30, n_iter=40, seed=3, record_costs=True)
    assert list(rec.itercost_iterations) == [50, 70]
    assert np.all(np.isfinite(rec.itercosts))
    assert rec.costs.shape == (1200,)
    assert abs(float(rec.costs.sum()) - rec.itercosts[-1]) <= 1e-9 * abs(rec.itercosts[-1])
    assert res.costs.size == 0


@pytest.mark.parametrize("every", [1, 4])
def test_sampled_kernel_timing(hip, mid_problem, every):
    """set_timing(only=..., every=E) brackets the named kernel on every E-th
    iteration of run() only: 10 iterations time ceil(10 / E) attraction
    launches, with positive durations, and no other kernel; both the timed
    and an untimed run from the same state end with finite layouts (their
    difference is not a check: float atomics reorder sums run to run, and
    early exaggeration amplifies that to ~4e-3 over 15 iterations)."""
    x, idx, dist = mid_problem
    n = x.shape[0]
    y0 = synthetic.pca_init(x)
    _say(f"case: sampled timing of the attraction, every {every}")
    layouts = []
    for timed in (True, False):
        with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
            s.set_state(y0)
            s.run(5, 12.0, 0.5, n / 12.0, 0.01, 5.0)
            s.sync()
            if timed:
                s.set_timing(True, only="attract", every=every)
            s.run(10, 12.0, 0.5, n / 12.0, 0.01, 5.0)
            s.sync()
            if timed:
                t = s.timing()
                s.set_timing(False)
                cnt, tot = t["attract"]
                assert cnt == -(-10 // every), t
                assert tot > 0.0
                assert all(c == 0 for name, (c, _) in t.items() if name != "attract"), t
            layouts.append(s.y)
    assert all(np.all(np.isfinite(y)) for y in layouts)


def test_repulsion_span_timing(hip, mid_problem):
    """set_timing(only="repulsion") runs the iterations in sequence and
    brackets the repulsion step's kernels with one pair of events: one span
    per iteration, no kernel timed on its own, and each span longer than the
    largest of the step's kernels timed one by one and within twice their
    sum plus 50 us (the span also holds the short gaps between them)."""
    x, idx, dist = mid_problem
    n = x.shape[0]
    y0 = synthetic.pca_init(x)
    _say("case: repulsion span timing")
    with hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1) as s:
        s.set_state(y0)
        s.run(5, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        s.set_timing(True)
        s.run(10, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        s.sync()
        each = s.timing()
        s.set_timing(True, only="repulsion")
        s.run(10, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        s.sync()
        span = s.timing()
        s.set_timing(False)
        assert np.all(np.isfinite(s.y))
    cnt, tot = span["repulsion"]
    assert cnt == 10, span
    assert all(c == 0 for name, (c, _) in span.items() if name != "repulsion"), span
    assert each["repulsion"][0] == 0, each
    rep = [name for name in each if name.startswith("interp_") or name in (
        "bin_count", "bin_plan", "bin_scatter", "spread", "kernel_rows", "kernel_cols", "charge_rows", "conv_cols",
        "inverse_rows")]
    per = {name: each[name][1] / 10 for name in rep if each[name][0]}
    _say(f"  span {tot / cnt:.4f} ms, kernels one by one {sum(per.values()):.4f} ms ({per})")
    assert max(per.values()) < tot / cnt < 2.0 * sum(per.values()) + 0.05
