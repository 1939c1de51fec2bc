"""Parity at the benchmark configurations' full sizes (BASELINE.json configs
1 and 3; configs 2 and 4 are in tests/test_gpu_config2.py and
tests/test_gpu_config4.py), HIP path vs the CPU oracle on identical inputs,
through the C ABI.

Every configuration's KNN comes from the library's exact GPU search (itself
checked against the oracle's KNN in tests/test_gpu_knn.py); the HIP path and
the oracle are then fed the same KNN bytes.

Gates:
  P                       identical row pointers and columns; values within
                          1e-5 relative L2 of the oracle's
  final KL                within 1 % of the oracle's full run
  15-NN preservation      within 0.01 of the oracle's full run (2000-row
                          sample)
  transform (config 3)    max |dy| <= 1e-9 x layout scale (fp64 on both sides)
"""

import os
import sys

import numpy as np
import pytest

from fastembedr_amd import _lib, synthetic
from tests.helpers import knn_preservation, rel_l2

pytestmark = pytest.mark.gpu

P_TOL = 1e-5
GRAD_TOL = 1e-3
LAGRANGE = _lib.REPULSION_LAGRANGE
SCHED = synthetic.SCHEDULE
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _gpu_knn(hip, x, k):
    """Exact KNN on the GPU; host copy (n, k), 1-based, plus the device result."""
    knn = hip.exact_knn(np.ascontiguousarray(x, np.float32), k, keep_device=True)
    host = knn.to_host()
    return knn, np.asarray(host.indices, np.int32), np.asarray(host.distances, np.float32)


def _schedule(s, n, upto, start=0):
    """Runs iterations [start, upto) of the two-phase schedule on session s."""
    ee = SCHED["early_exaggeration_iter"]
    lr = n / 12.0
    early = max(0, min(upto, ee) - start)
    if early:
        s.run(early, SCHED["early_exaggeration"], SCHED["initial_momentum"], lr, SCHED["min_gain"],
              SCHED["max_step_norm"])
    late = upto - max(start, ee)
    if late > 0:
        s.run(late, SCHED["exaggeration"], SCHED["final_momentum"], lr, SCHED["min_gain"], SCHED["max_step_norm"])


def _check_p(s, P, label):
    rp, col, val = s.csr()
    rp0, col0, val0 = P.csr()
    np.testing.assert_array_equal(rp, rp0)
    np.testing.assert_array_equal(col, col0)
    err = rel_l2(val, val0)
    _say(f"  {label}: nnz {col.size}, P values relL2 {err:.2e}")
    assert err <= P_TOL
    assert abs(float(val.astype(np.float64).sum()) - 1.0) < 1e-5


# ---------------------------------------------------------------------------
# config 1: 70,000 x 50, the headline parity case
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def config1(hip, oracle_mod):
    spec = synthetic.CONFIGS[1]
    x, _ = synthetic.gaussian_mixture(spec, seed=1)
    knn, idx, dist = _gpu_knn(hip, x, SCHED["k"])
    del knn
    P = oracle_mod.OracleP.build(idx, dist, SCHED["perplexity"], threads=THREADS)
    return {"x": x, "idx": idx, "dist": dist, "y0": synthetic.pca_init(x), "P": P, "layouts": {}}


@pytest.mark.parametrize("repulsion", ["grid", "interp"])
def test_config1_end_to_end_kl_and_knn_preservation(hip, oracle_mod, config1, repulsion):
    """750 iterations from the same PCA init on both sides; the bilinear grid
    through the reference-shaped one-shot call, the FIt-SNE grid through the
    session."""
    x, idx, dist, y0, P = (config1[k] for k in ("x", "idx", "dist", "y0", "P"))
    n = x.shape[0]
    lr = n / 12.0
    _say(f"case: config 1 end to end, n={n}, {repulsion}")
    if repulsion == "grid":
        y_hip = hip.opentsne_knn(idx, dist, n_neighbors=SCHED["k"], perplexity=SCHED["perplexity"], Y_init=y0,
                                 early_exaggeration_iter=SCHED["early_exaggeration_iter"], n_iter=SCHED["n_iter"],
                                 initial_momentum=SCHED["initial_momentum"], learning_rate=lr).layout
        method = oracle_mod.METHOD_GRID
    else:
        with hip.TsneSession(idx, dist, perplexity=SCHED["perplexity"], index_offset=1) as s:
            _check_p(s, P, "config 1")
            s.set_repulsion(LAGRANGE, 3, SCHED["min_intervals"], SCHED["ints_in_interval"])
            s.set_state(y0)
            s.center()
            _schedule(s, n, 750)
            s.sync()
            y_hip = s.y
        method = oracle_mod.METHOD_LAGRANGE
    y_hip = np.asarray(y_hip, np.float32)
    y_cpu, _, _ = P.optimize(y0, SCHED["early_exaggeration_iter"], SCHED["n_iter"], SCHED["early_exaggeration"],
                             SCHED["exaggeration"], lr, False, SCHED["initial_momentum"], SCHED["final_momentum"],
                             method=method, threads=THREADS)
    kl_hip, kl_cpu = P.kl(y_hip, threads=THREADS), P.kl(y_cpu, threads=THREADS)
    pres_hip, pres_cpu = knn_preservation(x, y_hip, 15), knn_preservation(x, y_cpu, 15)
    _say(f"  KL hip={kl_hip:.5f} cpu={kl_cpu:.5f}; 15-NN hip={pres_hip:.4f} cpu={pres_cpu:.4f}")
    assert np.all(np.isfinite(y_hip))
    assert abs(kl_hip - kl_cpu) <= 0.01 * kl_cpu
    assert abs(pres_hip - pres_cpu) <= 0.01
    config1["layouts"][repulsion] = y_hip


# ---------------------------------------------------------------------------
# config 3: 100,000 queries against the fixed config-1 embedding
# ---------------------------------------------------------------------------
def test_config3_transform_full_size(hip, oracle_mod, config1):
    """The first 30 iterations of config 3 (perplexity 5, k = 30, learning
    rate 0.1, exaggeration 1, 256 sampled negatives) at full size: 100,000
    queries against the 70,000-point config-1 embedding."""
    ref = config1["layouts"].get("interp")
    if ref is None:
        ref = config1["layouts"].get("grid")
    assert ref is not None, "the config-1 tests provide the reference layout"
    spec = synthetic.CONFIGS[1]
    xq = synthetic.mixture_queries(spec, 100_000)
    qknn = hip.exact_query_knn(np.ascontiguousarray(config1["x"], np.float32), xq, 30)
    idx, dist = np.asarray(qknn.indices, np.int32), np.asarray(qknn.distances, np.float64)
    ref64 = np.asarray(ref, np.float64)
    _say(f"case: config 3 transform, {xq.shape[0]} queries x {ref64.shape[0]} references, k=30")
    kw = dict(perplexity=5.0, n_iter=30, learning_rate=0.1, exaggeration=1.0, seed=4)
    res = hip.transform_tsne(ref64, knn={"indices": idx, "distances": dist}, n_negatives=256, **kw)
    y_ref, exact = oracle_mod.transform_run(ref64, idx, dist, n_negatives=256, exact_threshold=4096,
                                            threads=THREADS, **kw)
    assert not exact and res.config["repulsion"] == "sampled_reference"
    y = np.asarray(res.layout)
    scale = np.abs(y_ref).max()
    dev = np.abs(y - y_ref).max()
    _say(f"  max |dy| = {dev:.3e} (scale {scale:.2f}); bit-identical rows {np.mean(np.all(y == y_ref, axis=1)):.4f}")
    assert dev <= 1e-9 * scale
    # the configuration's own design: the reference grid precomputed once,
    # the whole 250-iteration schedule
    kw["n_iter"] = 250
    _say("  reference-grid mode, 250 iterations")
    res = hip.transform_tsne(ref64, knn={"indices": idx, "distances": dist}, reference_grid={}, **kw)
    y_ref, st = oracle_mod.transform_grid_run(ref64, idx, dist, min_intervals=50, ints_in_interval=0.5,
                                              threads=THREADS, **kw)
    cfg = res.config["reference_grid"]
    y = np.asarray(res.layout)
    dev = np.abs(y - y_ref).max()
    scale = np.abs(y_ref).max()
    _say(f"  grid {cfg['boxes_per_axis']} boxes, {cfg['nodes_per_axis']} nodes, {cfg['exact_evaluations']} exact "
         f"evaluations; max |dy| = {dev:.3e} (scale {scale:.2f})")
    assert (cfg["boxes_per_axis"], cfg["nodes_per_axis"], cfg["exact_evaluations"]) == \
        (st["boxes"], st["nodes"], st["exact_evaluations"])
    assert dev <= 1e-9 * scale
