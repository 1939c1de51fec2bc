"""Replayed iterations (FASTEMBEDR_HIP_GRAPH_CAPTURE) against eager launches.

run() captures one iteration's launches on its three streams into a graph and
replays it; the kernels and their order are the same as the eager path's, so
a replayed run must agree with an eager one as closely as two eager runs
agree with each other (the float atomics of the binning make two eager runs
differ by rounding).  The switch is read when a session is created: unset or
empty is on, "0"/"false"/"FALSE"/"no"/"NO" is off, as for the reference's
FASTEMBEDR_CUDA_GRAPH_CAPTURE (src/embedding_cuda_kernels.cpp:170-178).

Checked per repulsion (bilinear grid, interpolation grid):
  * the replayed run took most iterations from graphs (graph_info);
  * the displacement from the start differs from an eager run's by at most
    4 x (eager vs eager) + 1e-6, relative L2, over 40 iterations that cross
    an early-exaggeration -> normal switch (two graph keys);
  * with a growing span (the interpolation grid's FFT length changes between
    keys, and the host learns box counts through the device-indexed ring) the
    final exact KL agrees with the eager run's within 0.5 %;
  * the switch's off values turn capture off.
"""

import os
import sys

import numpy as np
import pytest

from fastembedr_amd import _lib, synthetic
from tests.helpers import rel_l2, small_problem

pytestmark = pytest.mark.gpu

ENV = "FASTEMBEDR_HIP_GRAPH_CAPTURE"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def prob():
    x, labels, idx, dist = small_problem(n=3000, dim=20, k=45, components=6, seed=21)
    return x, idx, dist, synthetic.pca_init(x)


def _session(hip, idx, dist, capture):
    old = os.environ.get(ENV)
    if capture is None:
        os.environ.pop(ENV, None)
    else:
        os.environ[ENV] = capture
    try:
        return hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1)
    finally:
        if old is None:
            os.environ.pop(ENV, None)
        else:
            os.environ[ENV] = old


def _schedule(hip, idx, dist, y0, repulsion, capture, early, normal):
    n = y0.shape[0]
    with _session(hip, idx, dist, capture) as s:
        if repulsion == _lib.REPULSION_LAGRANGE:
            s.set_repulsion(repulsion, 3, 50, 1.0)
        s.set_state(y0)
        s.center()
        start = s.y
        s.run(early, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        s.run(normal, 1.0, 0.8, n / 12.0, 0.01, 5.0)
        return start, s.y, s.kl(), s.graph_info()


@pytest.mark.parametrize("repulsion", [_lib.REPULSION_GRID, _lib.REPULSION_LAGRANGE], ids=["bilinear", "interp"])
def test_replayed_iterations_match_eager(hip, prob, repulsion):
    x, idx, dist, y0 = prob
    _say(f"case: graph replay vs eager, repulsion {repulsion}, 20 + 20 iterations")
    start, y_e1, _, info_e = _schedule(hip, idx, dist, y0, repulsion, "0", 20, 20)
    _, y_e2, _, _ = _schedule(hip, idx, dist, y0, repulsion, "0", 20, 20)
    _, y_g, _, info_g = _schedule(hip, idx, dist, y0, repulsion, None, 20, 20)
    assert not info_e["enabled"] and info_e["launches"] == 0
    assert info_g["enabled"] and info_g["captures"] >= 2 and info_g["launches"] >= 30, info_g
    base = rel_l2(y_e2 - start, y_e1 - start)
    err = rel_l2(y_g - start, y_e1 - start)
    _say(f"  eager vs eager {base:.2e}, graph vs eager {err:.2e}, {info_g}")
    assert np.all(np.isfinite(y_g))
    assert err <= 4.0 * base + 1e-6


def test_replayed_growing_span_kl(hip, prob):
    """150 + 150 iterations from a small span: the interpolation grid grows
    through several FFT lengths (several graph keys, LRU reuse)."""
    x, idx, dist, y0 = prob
    y0 = (y0 - y0.mean(axis=0)) * (4.0 / float(np.ptp(y0)))
    _say("case: graph replay vs eager, interpolation grid, growing span, 150 + 150 iterations")
    _, y_e, kl_e, _ = _schedule(hip, idx, dist, y0.astype(np.float32), _lib.REPULSION_LAGRANGE, "no", 150, 150)
    _, y_g, kl_g, info = _schedule(hip, idx, dist, y0.astype(np.float32), _lib.REPULSION_LAGRANGE, "", 150, 150)
    _say(f"  KL eager {kl_e:.5f}, graph {kl_g:.5f}, {info}")
    assert info["launches"] >= 250, info
    assert np.all(np.isfinite(y_g))
    assert abs(kl_g - kl_e) <= 0.005 * kl_e


@pytest.mark.parametrize("value,enabled", [("0", False), ("false", False), ("FALSE", False), ("no", False),
                                           ("NO", False), ("", True), ("1", True), ("yes", True)])
def test_capture_switch_values(hip, prob, value, enabled):
    x, idx, dist, y0 = prob
    with _session(hip, idx, dist, value) as s:
        assert s.graph_info()["enabled"] is enabled
