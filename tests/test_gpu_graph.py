"""Replayed iterations (FASTEMBEDR_HIP_GRAPH_CAPTURE) against eager launches.

run() captures one iteration's launches on the main stream alone into a graph
and replays it; the kernels and their order are the eager path's without the
side streams.  The switch is read when a session is created: unset, empty and
"0"/"false"/"FALSE"/"no"/"NO" are off, anything else on (the reference's
FASTEMBEDR_CUDA_GRAPH_CAPTURE, src/embedding_cuda_kernels.cpp:170-178, takes
the same off values but is on when unset).

Float atomics (the attraction's row sums, the binning's order) make two eager
runs differ by rounding, which t-SNE's early-exaggeration phase amplifies
over tens of iterations; so the layouts are compared one iteration at a time
and whole runs by their KL divergence.  Checked per repulsion (bilinear grid,
interpolation grid):
  * one replayed iteration (the third from the same state: eager, captured,
    replayed) equals one eager iteration from that state: displacement
    relative L2 <= max(5e-5, 4 x (eager vs eager)) (the bilinear spreading's
    LDS float atomics alone give about 1.6e-5);
  * 60 + 60 iterations, most replayed (graph_info), end at an exact KL within
    1 % of the eager run's (independent eager runs of this problem spread
    over 0.8 % of KL: 2.8119 to 2.8343 in 16 runs on MI355X);
  * with a growing span (the interpolation grid's FFT length changes between
    graph keys, and the host learns box counts from the device-indexed ring)
    the final KL agrees within 1 %;
  * the switch's off values (and unset) turn capture off;
  * the arrangements of the eager overlapped iteration (the attraction on
    the stream of the previous update with the chain beside it and the
    update right behind the attraction, the default; the same with the
    update after the chain on the chain's stream,
    FASTEMBEDR_HIP_UPDATE_ON_CHAIN=1; and the attraction beside the chain
    with a helper launch, FASTEMBEDR_HIP_ATTRACT_MAIN=0) end within 1 % of
    the single-stream replayed run's KL;
  * a closed session gives its device memory back, replayed or not (graphs
    with parallel branches, once launched, held their side-branch kernels'
    allocations past hipFree until a device-wide synchronisation: 4.7 GB
    per session at config 2, piling up over sessions).
"""

import ctypes as C

import os
import sys

import numpy as np
import pytest

from fastembedr_amd import _lib, synthetic
from tests.helpers import rel_l2, small_problem

pytestmark = pytest.mark.gpu

ENV = "FASTEMBEDR_HIP_GRAPH_CAPTURE"
KL_TOL = 0.01


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def prob():
    x, labels, idx, dist = small_problem(n=3000, dim=20, k=45, components=6, seed=21)
    return x, idx, dist, synthetic.pca_init(x)


def _session(hip, idx, dist, capture, extra=None):
    settings = {ENV: capture, **(extra or {})}
    old = {k: os.environ.get(k) for k in settings}
    for k, v in settings.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v
    try:
        return hip.TsneSession(idx, dist, perplexity=15.0, index_offset=1)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _schedule(hip, idx, dist, y0, repulsion, capture, early, normal, extra=None):
    n = y0.shape[0]
    with _session(hip, idx, dist, capture, extra) as s:
        if repulsion == _lib.REPULSION_LAGRANGE:
            s.set_repulsion(repulsion, 3, 50, 1.0)
        s.set_state(y0)
        s.center()
        start = s.y
        s.run(early, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        s.run(normal, 1.0, 0.8, n / 12.0, 0.01, 5.0)
        return start, s.y, s.kl(), s.graph_info()


@pytest.mark.parametrize("repulsion", [_lib.REPULSION_GRID, _lib.REPULSION_LAGRANGE], ids=["bilinear", "interp"])
def test_replayed_iteration_matches_eager(hip, prob, repulsion):
    x, idx, dist, y0 = prob
    n = y0.shape[0]
    _say(f"case: one replayed iteration vs one eager iteration, repulsion {repulsion}")

    def one(s):
        if repulsion == _lib.REPULSION_LAGRANGE:
            s.set_repulsion(repulsion, 3, 50, 1.0)
        s.set_state(y0)
        s.center()
        start = s.y
        s.run(1, 12.0, 0.5, n / 12.0, 0.01, 5.0)
        return start, s.y

    with _session(hip, idx, dist, "1") as s:
        for _ in range(3):  # eager (first sight of the key), captured and replayed, replayed
            start, y_g = one(s)
        info = s.graph_info()
    with _session(hip, idx, dist, "0") as s:
        start_e, y_e1 = one(s)
        _, y_e2 = one(s)
    np.testing.assert_array_equal(start, start_e)
    base = rel_l2(y_e2 - start, y_e1 - start)
    err = rel_l2(y_g - start, y_e1 - start)
    _say(f"  eager vs eager {base:.2e}, replayed vs eager {err:.2e}, {info}")
    assert info["captures"] == 1 and info["launches"] == 2, info
    assert err <= max(5e-5, 4.0 * base)


@pytest.mark.parametrize("repulsion", [_lib.REPULSION_GRID, _lib.REPULSION_LAGRANGE], ids=["bilinear", "interp"])
def test_replayed_schedule_kl(hip, prob, repulsion):
    x, idx, dist, y0 = prob
    _say(f"case: graph replay vs eager, repulsion {repulsion}, 60 + 60 iterations")
    _, y_e, kl_e, info_e = _schedule(hip, idx, dist, y0, repulsion, "0", 60, 60)
    _, y_g, kl_g, info_g = _schedule(hip, idx, dist, y0, repulsion, "1", 60, 60)
    _say(f"  KL eager {kl_e:.5f}, graph {kl_g:.5f}, {info_g}")
    assert not info_e["enabled"] and info_e["launches"] == 0
    assert info_g["enabled"] and info_g["launches"] >= 100, info_g
    assert np.all(np.isfinite(y_g))
    assert abs(kl_g - kl_e) <= KL_TOL * kl_e


@pytest.mark.parametrize("arrangement,on_chain", [("1", "0"), ("1", "1"), ("0", "0")],
                         ids=["attraction_main", "attraction_main_update_on_chain", "attraction_beside"])
def test_overlap_arrangements_kl(hip, prob, arrangement, on_chain):
    x, idx, dist, y0 = prob
    extra = {"FASTEMBEDR_HIP_ATTRACT_MAIN": arrangement, "FASTEMBEDR_HIP_UPDATE_ON_CHAIN": on_chain}
    _say(f"case: {extra}, eager vs replayed, interpolation grid, 60 + 60 iterations")
    _, y_e, kl_e, info_e = _schedule(hip, idx, dist, y0, _lib.REPULSION_LAGRANGE, None, 60, 60, extra)
    _, y_g, kl_g, info = _schedule(hip, idx, dist, y0, _lib.REPULSION_LAGRANGE, "1", 60, 60)
    _say(f"  KL eager {kl_e:.5f}, graph {kl_g:.5f}, {info}")
    assert not info_e["enabled"] and info_e["launches"] == 0, info_e
    assert info["launches"] >= 100, info
    assert np.all(np.isfinite(y_g)) and np.all(np.isfinite(y_e))
    assert abs(kl_g - kl_e) <= KL_TOL * kl_e


def test_replayed_growing_span_kl(hip, prob):
    """150 + 150 iterations from a small span: the interpolation grid grows
    through several FFT lengths (several graph keys, LRU reuse)."""
    x, idx, dist, y0 = prob
    y0 = (y0 - y0.mean(axis=0)) * (4.0 / float(np.ptp(y0)))
    _say("case: graph replay vs eager, interpolation grid, growing span, 150 + 150 iterations")
    _, y_e, kl_e, _ = _schedule(hip, idx, dist, y0.astype(np.float32), _lib.REPULSION_LAGRANGE, "no", 150, 150)
    _, y_g, kl_g, info = _schedule(hip, idx, dist, y0.astype(np.float32), _lib.REPULSION_LAGRANGE, "yes", 150, 150)
    _say(f"  KL eager {kl_e:.5f}, graph {kl_g:.5f}, {info}")
    assert info["launches"] >= 250, info
    assert np.all(np.isfinite(y_g))
    assert abs(kl_g - kl_e) <= KL_TOL * kl_e


@pytest.mark.parametrize("value,enabled", [(None, False), ("", False), ("0", False), ("false", False),
                                           ("FALSE", False), ("no", False), ("NO", False), ("1", True),
                                           ("yes", True)])
def test_capture_switch_values(hip, prob, value, enabled):
    x, idx, dist, y0 = prob
    with _session(hip, idx, dist, value) as s:
        assert s.graph_info()["enabled"] is enabled


def _free_bytes() -> int:
    """Free device memory as a caller sees it after close() (no device-wide
    synchronisation first: deferred releases count as lost)."""
    hip_rt = C.CDLL("libamdhip64.so.7")
    free_b, total_b = C.c_size_t(), C.c_size_t()
    assert hip_rt.hipMemGetInfo(C.byref(free_b), C.byref(total_b)) == 0
    return free_b.value


@pytest.mark.parametrize("capture", ["0", "1"], ids=["eager", "replayed"])
def test_closed_session_returns_memory(hip, capture):
    """Seven 200,000-point sessions of config 2's mixture (perplexity 30,
    k = 90; about 2.6 GB of device buffers each), one after another, each
    run for 30 iterations and closed.  The first two absorb the runtime's
    one-time pools (54 and 40 MiB in a fresh process).  After a close the
    runtime sometimes keeps the closed session's blocks for a while (free
    memory then reads at the in-session level, and the next session's
    identical requests reuse them), so a reading may sit anywhere between
    the in-session level and a full return (here: two of five readings at the
    in-session level, alternating with full returns, and once 870 MB of a
    session's 2.7 GB held); a leak instead lowers every later reading.  The
    check: the highest of the last three readings is within 64 MiB of the
    second warm-up session's reading (memory comes back), and no reading
    after the warm-up falls more than 64 MiB below the in-session level.
    Graphs with parallel branches lost 1.4 GB per session here; a steady leak
    of more than about 22 MiB per session fails."""
    n, k = 200_000, 90
    x, _ = synthetic.gaussian_mixture(synthetic.CONFIGS[2], seed=1, n=n)
    knn = hip.exact_knn(np.ascontiguousarray(x, np.float32), k, keep_device=True)
    y0 = synthetic.pca_init(x)
    _say(f"case: device memory after close, n {n}, capture {capture}")

    def one():
        settings = {ENV: capture}
        old = {key: os.environ.get(key) for key in settings}
        os.environ.update(settings)
        try:
            s = hip.TsneSession(perplexity=30.0, index_offset=1, n=n, k=k,
                                device_pointers=(knn.indices_ptr, knn.distances_ptr))
        finally:
            for key, v in old.items():
                if v is None:
                    os.environ.pop(key, None)
                else:
                    os.environ[key] = v
        with s:
            s.set_repulsion(_lib.REPULSION_LAGRANGE, 3, 50, 1.0)
            s.set_state(y0)
            s.center()
            s.run(30, 12.0, 0.5, n / 12.0, 0.01, 5.0)
            s.sync()
            used = _free_bytes()
            info = s.graph_info()
        return used, info

    start = _free_bytes()
    during, after = [], []
    for _ in range(7):
        used, info = one()
        during.append(used)
        after.append(_free_bytes())
        assert (info["launches"] >= 20) if capture == "1" else (info["launches"] == 0), info
    mib = lambda v: f"{v / 2**20:.0f}"
    _say(f"  free at start {mib(start)} MiB, in sessions {[mib(v) for v in during]}, "
         f"after them {[mib(v) for v in after]}, {info}")
    footprint = start - during[0]  # one session's buffers
    assert footprint > 256 * 2**20
    slack = 64 * 2**20
    in_session = min(during)
    assert max(after[-3:]) >= after[1] - slack, (after, during)
    assert min(after[2:]) >= in_session - slack, (after, during)
