"""HIP fixed-reference transform vs the CPU oracle (through the C ABI).

Both sides compute in fp64 in the reference's operation order; the only
differences come from the device's exp/log in the perplexity search (last-bit
differences of the conditional probabilities).  Tolerances:
  conditional P, gradient         relative error <= 1e-12
  median initialisation           bit-identical; weighted relative <= 1e-14
  whole run (layout)              max abs difference <= 1e-9 x layout scale
"""

import ctypes as C
import sys

import numpy as np
import pytest

from fastembedr_amd import _lib
from tests.helpers import query_problem

pytestmark = pytest.mark.gpu

TIGHT = 1e-12


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def qp():
    return query_problem()


def _probe(ref, idx, dist, perplexity, y=None, ex=1.0, n_neg=256, thr=4096, iter_seed=0, init=0):
    lib = _lib.load()
    nq, k = idx.shape
    ref_cm = np.asfortranarray(ref, np.float64)
    idx_cm = np.asfortranarray(idx, np.int32)
    dist_cm = np.asfortranarray(dist, np.float64)
    p = np.empty((nq, k), np.float64)
    g = np.empty((nq, 2), np.float64)
    y0 = np.empty((nq, 2), np.float64)
    yy = None if y is None else np.ascontiguousarray(y, np.float64)
    rc = lib.fastembedr_hip_transform_probe(
        ref_cm.ctypes.data_as(C.c_void_p), ref.shape[0], idx_cm.ctypes.data_as(C.c_void_p),
        dist_cm.ctypes.data_as(C.c_void_p), nq, k, float(perplexity),
        None if yy is None else yy.ctypes.data_as(C.c_void_p), float(ex), int(n_neg), int(thr), int(iter_seed),
        int(init), p.ctypes.data_as(C.c_void_p), g.ctypes.data_as(C.c_void_p), y0.ctypes.data_as(C.c_void_p))
    _lib.check(rc, "transform probe")
    return p, g, y0


def _rel(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def test_transform_p_and_init_match_oracle(hip, oracle_mod, qp):
    _say("case: transform P + median/weighted init, n_ref=3000 nq=1200 k=30")
    ref, idx, dist = qp
    p, _, med = _probe(ref, idx, dist, 5.0, init=0)
    p_ref = oracle_mod.transform_conditional_p(dist, 5.0)
    assert np.abs(p - p_ref).max() <= TIGHT * np.abs(p_ref).max()
    _say(f"bit-identical P entries: {np.mean(p == p_ref):.4f}")
    np.testing.assert_array_equal(med, oracle_mod.transform_init(ref, idx, dist, oracle_mod.INIT_MEDIAN))
    _, _, wt = _probe(ref, idx, dist, 5.0, init=1)
    np.testing.assert_allclose(wt, oracle_mod.transform_init(ref, idx, dist, oracle_mod.INIT_WEIGHTED), rtol=1e-14)


@pytest.mark.parametrize("k", [1, 2, 5, 8, 13, 16, 30, 33, 64, 65])
def test_median_init_all_lane_widths(hip, oracle_mod, k):
    """The median initialisation at every lane width of its kernel (8, 16, 32
    and 64 lanes per query) and past it (k = 65, one thread per query), with
    tied coordinates (references on a half-unit lattice) and repeated
    neighbours; bit-identical to the oracle."""
    _say(f"case: median init, k={k}, tied coordinates")
    rng = np.random.default_rng(100 + k)
    n_ref, nq = 400, 333
    ref = np.round(rng.normal(0.0, 3.0, (n_ref, 2)) * 2.0) / 2.0
    idx = rng.integers(1, n_ref + 1, (nq, k)).astype(np.int32)
    dist = np.sort(rng.uniform(0.1, 2.0, (nq, k)), axis=1)
    _, _, med = _probe(ref, idx, dist, 0.5, init=0)
    np.testing.assert_array_equal(med, oracle_mod.transform_init(ref, idx, dist, oracle_mod.INIT_MEDIAN))


@pytest.mark.parametrize("mode", ["sampled", "exact"])
def test_transform_gradient_matches_oracle(hip, oracle_mod, qp, mode):
    _say(f"case: transform gradient ({mode})")
    ref, idx, dist = qp
    thr = 100 if mode == "sampled" else 4096
    y = oracle_mod.transform_init(ref, idx, dist, oracle_mod.INIT_MEDIAN)
    y = y + np.random.default_rng(2).normal(0, 0.3, size=y.shape)
    p, g, _ = _probe(ref, idx, dist, 5.0, y=y, ex=1.5, n_neg=256, thr=thr, iter_seed=4 + 65537)
    p_ref = oracle_mod.transform_conditional_p(dist, 5.0)
    g_ref = oracle_mod.transform_gradient(ref, idx, p_ref, y, 1.5, 256, thr, 4 + 65537)
    r = _rel(g, g_ref)
    _say(f"gradient relative error {r:.3e}, bit-identical {np.mean(g == g_ref):.4f}")
    assert r <= TIGHT


def _run(ref, idx, dist, **kw):
    from fastembedr_amd import transform_tsne

    res = transform_tsne(ref, knn={"indices": idx, "distances": dist}, **kw)
    return res.layout, res.config


@pytest.mark.parametrize("case", ["sampled", "exact", "random_init_early", "weighted_clipped"])
def test_transform_run_matches_oracle(hip, oracle_mod, qp, case):
    ref, idx, dist = qp
    kw = dict(perplexity=5.0, n_iter=60, learning_rate=0.1, exaggeration=1.0, seed=17)
    okw = dict(perplexity=5.0, n_iter=60, learning_rate=0.1, exaggeration=1.0, seed=17)
    if case == "sampled":
        kw.update(exact_repulsion_threshold=100, n_negatives=256)
        okw.update(exact_threshold=100, n_negatives=256)
    elif case == "exact":
        kw.update(exact_repulsion_threshold=4096)
        okw.update(exact_threshold=4096, n_negatives=3000)
    elif case == "random_init_early":
        kw.update(initialization="random", early_exaggeration_iter=10, early_exaggeration=4.0,
                  initial_momentum=0.5, exact_repulsion_threshold=100, n_negatives=64)
        okw.update(initialization=oracle_mod.INIT_RANDOM, early_exaggeration_iter=10, early_exaggeration=4.0,
                   initial_momentum=0.5, exact_threshold=100, n_negatives=64)
    else:
        kw.update(initialization="weighted", max_step_norm=0.05, max_grad_norm=0.1, exact_repulsion_threshold=100,
                  n_negatives=128)
        okw.update(initialization=oracle_mod.INIT_WEIGHTED, max_step_norm=0.05, max_grad_norm=0.1,
                   exact_threshold=100, n_negatives=128)
    _say(f"case: transform run {case}")
    y, cfg = _run(ref, idx, dist, **kw)
    y_ref, exact = oracle_mod.transform_run(ref, idx, dist, threads=8, **okw)
    assert cfg["repulsion"] == ("exact_reference" if exact else "sampled_reference")
    scale = np.abs(y_ref).max()
    dev = np.abs(y - y_ref).max()
    _say(f"max |dy| = {dev:.3e} (scale {scale:.2f}); bit-identical rows {np.mean(np.all(y == y_ref, axis=1)):.4f}")
    assert dev <= 1e-9 * scale


def test_transform_is_deterministic(hip, qp):
    ref, idx, dist = qp
    a, _ = _run(ref, idx, dist, n_iter=20, exact_repulsion_threshold=100, seed=3)
    b, _ = _run(ref, idx, dist, n_iter=20, exact_repulsion_threshold=100, seed=3)
    np.testing.assert_array_equal(a, b)


def test_transform_api_rules_and_labels(hip, qp):
    ref, idx, dist = qp
    y, cfg = _run(ref[:500], np.minimum(idx, 500), dist, n_iter=2)
    assert cfg["repulsion"] == "exact_reference" and cfg["n_negatives"] == 500  # n_ref <= 4096
    y, cfg = _run(ref, idx, dist, n_iter=2, exact_repulsion_threshold=1000)
    assert cfg["repulsion"] == "sampled_reference" and cfg["n_negatives"] == 256
    assert cfg["optimizer"] == "opentsne_style_fixed_reference_transform"
    assert cfg["affinities"] == "precomputed_query_conditional"
    assert cfg["affinity_storage"] == "flat_row_major_double"
    assert y.shape == (idx.shape[0], 2) and np.all(np.isfinite(y))


def test_transform_input_errors(hip, qp):
    ref, idx, dist = qp
    bad = idx.copy()
    bad[3, 2] = 10 ** 6
    with pytest.raises(_lib.HipBackendError, match="out of range"):
        _run(ref, bad, dist, n_iter=1)
    dneg = dist.copy()
    dneg[0, 0] = -1.0
    with pytest.raises(_lib.HipBackendError, match="finite and non-negative"):
        _run(ref, idx, dneg, n_iter=1)
    with pytest.raises(ValueError, match="two-dimensional"):
        _run(np.zeros((10, 3)), idx, dist, n_iter=1)


# ---------------------------------------------------------------------------
# Reference-grid repulsion (fastembedr_hip_transform_tsne_grid), against the
# oracle's fp64 restatement of the same algorithm (itself pinned against the
# exact mode and brute-force node sums in tests/test_transform_oracle.py).
# ---------------------------------------------------------------------------
def _grid_probe(ref, idx, dist, y, geometry_y=None, ex=1.0, min_int=50, ints=0.5):
    lib = _lib.load()
    nq, k = idx.shape
    ref_cm = np.asfortranarray(ref, np.float64)
    idx_cm = np.asfortranarray(idx, np.int32)
    dist_cm = np.asfortranarray(dist, np.float64)
    yy = np.ascontiguousarray(y, np.float64)
    gy = None if geometry_y is None else np.ascontiguousarray(geometry_y, np.float64)
    g = np.empty((nq, 2), np.float64)
    stats = (C.c_longlong * 3)()
    rc = lib.fastembedr_hip_transform_grid_probe(
        ref_cm.ctypes.data_as(C.c_void_p), ref.shape[0], idx_cm.ctypes.data_as(C.c_void_p),
        dist_cm.ctypes.data_as(C.c_void_p), nq, k, 5.0, yy.ctypes.data_as(C.c_void_p),
        None if gy is None else gy.ctypes.data_as(C.c_void_p), 0 if gy is None else gy.shape[0], float(ex), 3,
        int(min_int), float(ints), g.ctypes.data_as(C.c_void_p), stats)
    _lib.check(rc, "transform grid probe")
    return g, [int(v) for v in stats]


def test_transform_grid_gradient_matches_oracle(hip, oracle_mod, qp):
    _say("case: reference-grid transform gradient, n_ref=3000 nq=1200 k=30")
    ref, idx, dist = qp
    y = oracle_mod.transform_init(ref, idx, dist, oracle_mod.INIT_MEDIAN)
    y = y + np.random.default_rng(2).normal(0, 0.3, size=y.shape)
    p_ref = oracle_mod.transform_conditional_p(dist, 5.0)
    g, st = _grid_probe(ref, idx, dist, y, ex=1.5)
    g_ref, outside = oracle_mod.transform_grid_gradient(ref, idx, p_ref, y, 1.5, min_intervals=50,
                                                        ints_in_interval=0.5)
    geo, _ = oracle_mod.transform_grid_fields(ref, y, 50, 0.5, fields=False)
    r = _rel(g, g_ref)
    _say(f"  grid {st[0]} boxes / {st[1]} nodes; relative error {r:.3e}, bit-identical {np.mean(g == g_ref):.4f}")
    assert (st[0], st[1], st[2]) == (geo["boxes"], geo["nodes"], outside) == (geo["boxes"], geo["nodes"], 0)
    assert r <= TIGHT
    # queries outside the grid take the exact sums
    far = y + np.array([500.0, -300.0])
    g_far, st_far = _grid_probe(ref, idx, dist, far, geometry_y=y, ex=1.5)
    g_far_ref, outside_far = oracle_mod.transform_grid_gradient(ref, idx, p_ref, far, 1.5, min_intervals=50,
                                                                ints_in_interval=0.5, geometry_y=y)
    assert st_far[2] == outside_far == far.shape[0]
    assert _rel(g_far, g_far_ref) <= TIGHT


# off_grid: a learning rate at which queries leave the grid (33 exact-sum
# query-iterations in the oracle), so the run's wave-wide exact sums are
# checked too.  (At 10, 2612 of them, the counts still agree but the
# trajectories are chaotic: summation-order rounding grows to O(1).)
@pytest.mark.parametrize("case", ["median", "weighted_early", "off_grid"])
def test_transform_grid_run_matches_oracle(hip, oracle_mod, qp, case):
    ref, idx, dist = qp
    lr = 2.0 if case == "off_grid" else 0.1
    kw = dict(perplexity=5.0, n_iter=60, learning_rate=lr, exaggeration=1.0, seed=17)
    okw = dict(kw)
    if case == "weighted_early":
        kw.update(initialization="weighted", early_exaggeration_iter=10, early_exaggeration=4.0, initial_momentum=0.5)
        okw.update(initialization=oracle_mod.INIT_WEIGHTED, early_exaggeration_iter=10, early_exaggeration=4.0,
                   initial_momentum=0.5)
    _say(f"case: reference-grid transform run ({case})")
    res = hip.transform_tsne(ref, knn={"indices": idx, "distances": dist}, reference_grid={}, **kw)
    y_ref, st = oracle_mod.transform_grid_run(ref, idx, dist, min_intervals=50, ints_in_interval=0.5, threads=8,
                                              **okw)
    cfg = res.config["reference_grid"]
    assert res.config["repulsion"] == "reference_grid_interpolation"
    assert (cfg["boxes_per_axis"], cfg["nodes_per_axis"], cfg["exact_evaluations"]) == \
        (st["boxes"], st["nodes"], st["exact_evaluations"])
    assert (st["exact_evaluations"] > 0) == (case == "off_grid")
    y = np.asarray(res.layout)
    scale = np.abs(y_ref).max()
    dev = np.abs(y - y_ref).max()
    _say(f"  max |dy| = {dev:.3e} (scale {scale:.2f}); bit-identical rows {np.mean(np.all(y == y_ref, axis=1)):.4f}; "
         f"exact-sum query-iterations {st['exact_evaluations']}")
    assert dev <= 1e-9 * scale
