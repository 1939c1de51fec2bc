"""Allocation-free transform (fastembedr_hip_transform_tsne_noalloc) against the
allocating entry point (fastembedr_hip_transform_tsne) on the same inputs,
through the C ABI.

Both run the same fp64 kernels in the same order, so the layouts must be
bit-identical.  The allocation-free call keeps its work buffers in one static
device array that every call shares: two calls in a row, the second with a
smaller input (fewer queries, a smaller reference, fewer neighbours, another
repulsion mode), check that nothing of the first call leaks into the second.
"""

import ctypes as C
import sys

import numpy as np
import pytest

from fastembedr_amd import _lib
from tests.helpers import DeviceArray, query_problem

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _params(**kw):
    p = dict(y_init=None, init=0, perplexity=5.0, n_iter=40, early_iter=0, lr=0.1, early_ex=4.0, ex=1.0, m0=0.5,
             m1=0.8, gmax=0.25, smax=float("inf"), n_neg=256, thr=4096, seed=7)
    p.update(kw)
    return p


def _host_call(ref, idx, dist, p):
    lib = _lib.load()
    nq, k = idx.shape
    ref_cm = np.asfortranarray(ref, np.float64)
    idx_cm = np.asfortranarray(idx, np.int32)
    dist_cm = np.asfortranarray(dist, np.float64)
    y0 = None if p["y_init"] is None else np.asfortranarray(p["y_init"], np.float64)
    out = np.empty((nq, 2), np.float64, order="F")
    exact = C.c_int(-1)
    rc = lib.fastembedr_hip_transform_tsne(
        ref_cm.ctypes.data_as(C.c_void_p), ref.shape[0], idx_cm.ctypes.data_as(C.c_void_p),
        dist_cm.ctypes.data_as(C.c_void_p), nq, k, None if y0 is None else y0.ctypes.data_as(C.c_void_p), p["init"],
        p["perplexity"], p["n_iter"], p["early_iter"], p["lr"], p["early_ex"], p["ex"], p["m0"], p["m1"], p["gmax"],
        p["smax"], p["n_neg"], p["thr"], p["seed"], out.ctypes.data_as(C.c_void_p), C.byref(exact))
    _lib.check(rc, "fastembedr_hip_transform_tsne")
    return out, exact.value


def _noalloc_call(ref, idx, dist, p):
    """The allocation-free entry point on device copies of the same arrays
    (column-major, as the ABI lays them out); returns (rc, layout, exact)."""
    lib = _lib.load()
    nq, k = idx.shape
    bufs = [DeviceArray(np.asfortranarray(ref, np.float64).ravel(order="F")),
            DeviceArray(np.asfortranarray(idx, np.int32).ravel(order="F")),
            DeviceArray(np.asfortranarray(dist, np.float64).ravel(order="F")),
            DeviceArray(np.zeros(2 * nq, np.float64))]
    y0 = None
    if p["y_init"] is not None:
        y0 = DeviceArray(np.asfortranarray(p["y_init"], np.float64).ravel(order="F"))
        bufs.append(y0)
    try:
        exact = C.c_int(-1)
        rc = lib.fastembedr_hip_transform_tsne_noalloc(
            C.c_void_p(bufs[0].address), ref.shape[0], C.c_void_p(bufs[1].address), C.c_void_p(bufs[2].address),
            nq, k, None if y0 is None else C.c_void_p(y0.address), p["init"], p["perplexity"], p["n_iter"],
            p["early_iter"], p["lr"], p["early_ex"], p["ex"], p["m0"], p["m1"], p["gmax"], p["smax"], p["n_neg"],
            p["thr"], p["seed"], C.c_void_p(bufs[3].address), C.byref(exact))
        out = bufs[3].to_host(np.float64, (nq, 2), order="F") if rc == 0 else None
        return rc, out, exact.value
    finally:
        for b in bufs:
            b.free()


def test_noalloc_transform_matches_allocating_call_twice(hip):
    """Two calls in a row, the second smaller, each against the allocating call."""
    ref, idx, dist = query_problem(n_ref=3000, nq=1200, k=30, seed=11)
    p1 = _params(early_iter=10, thr=100)  # sampled repulsion, median init, early phase
    _say("case: allocation-free transform, call 1: n_ref=3000 nq=1200 k=30 sampled, median init")
    want, ex_want = _host_call(ref, idx, dist, p1)
    rc, got, ex_got = _noalloc_call(ref, idx, dist, p1)
    _lib.check(rc, "fastembedr_hip_transform_tsne_noalloc")
    assert ex_got == ex_want == 0
    np.testing.assert_array_equal(got, want)

    ref2, idx2, dist2 = query_problem(n_ref=900, nq=400, k=12, seed=5)
    p2 = _params(init=1, n_iter=25, gmax=0.1, smax=0.05, seed=3)  # exact repulsion (n_ref <= 4096), weighted init
    _say("case: allocation-free transform, call 2: n_ref=900 nq=400 k=12 exact, weighted init")
    want2, ex_want2 = _host_call(ref2, idx2, dist2, p2)
    rc, got2, ex_got2 = _noalloc_call(ref2, idx2, dist2, p2)
    _lib.check(rc, "fastembedr_hip_transform_tsne_noalloc")
    assert ex_got2 == ex_want2 == 1
    np.testing.assert_array_equal(got2, want2)


def test_noalloc_transform_with_given_init_and_zero_based(hip):
    ref, idx, dist = query_problem(n_ref=2000, nq=700, k=20, seed=9)
    idx0 = idx - 1  # 0-based indices are detected as in the allocating call
    y0 = np.random.default_rng(1).normal(0, 2.0, size=(idx.shape[0], 2))
    p = _params(y_init=y0, n_iter=15, thr=500, n_neg=64)
    _say("case: allocation-free transform with y_init and 0-based indices")
    want, _ = _host_call(ref, idx0, dist, p)
    rc, got, _ = _noalloc_call(ref, idx0, dist, p)
    _lib.check(rc, "fastembedr_hip_transform_tsne_noalloc")
    np.testing.assert_array_equal(got, want)


def test_noalloc_transform_refusals(hip):
    """Inputs the static buffer cannot hold, the host-drawn random
    initialisation without y_init, and the allocating call's input checks."""
    ref, idx, dist = query_problem(n_ref=500, nq=200, k=10, seed=2)
    lib = _lib.load()
    big = 1 << 17
    rc = lib.fastembedr_hip_transform_tsne_noalloc(C.c_void_p(1), 10, C.c_void_p(1), C.c_void_p(1), big + 1, 8,
                                                   None, 0, 5.0, 1, 0, 0.1, 4.0, 1.0, 0.5, 0.8, 0.25, 0.0, 256, 4096,
                                                   1, C.c_void_p(1), None)
    assert rc == 1 and b"static work buffer" in lib.fastembedr_hip_embedding_last_error()
    rc, _, _ = _noalloc_call(ref, idx, dist, _params(init=2))
    assert rc == 1 and b"pass y_init" in lib.fastembedr_hip_embedding_last_error()
    bad = idx.copy()
    bad[3, 2] = 10 ** 6
    rc, _, _ = _noalloc_call(ref, bad, dist, _params(n_iter=1))
    assert rc == 1 and b"out of range" in lib.fastembedr_hip_embedding_last_error()
    dneg = dist.copy()
    dneg[0, 0] = -1.0
    rc, _, _ = _noalloc_call(ref, idx, dneg, _params(n_iter=1))
    assert rc == 1 and b"finite and non-negative" in lib.fastembedr_hip_embedding_last_error()
    # both errors in one input: the earlier entry in column-major order names
    # the error, in both calls (the allocating call scans the entries in order)
    nq = idx.shape[0]
    for (bi, bj), (di, dj) in (((3, 2), (0, 0)), ((0, 0), (5, 3)), ((7, 1), (7, 1)), ((150, 0), (2, 1))):
        both_i, both_d = idx.copy(), dist.copy()
        both_i[bi, bj] = 10 ** 6
        both_d[di, dj] = np.nan
        want_msg = b"out of range" if bj * nq + bi <= dj * nq + di else b"finite and non-negative"
        with pytest.raises(RuntimeError) as err:
            _host_call(ref, both_i, both_d, _params(n_iter=1))
        assert want_msg.decode() in str(err.value)
        rc, _, _ = _noalloc_call(ref, both_i, both_d, _params(n_iter=1))
        assert rc == 1 and want_msg in lib.fastembedr_hip_embedding_last_error()
    # after refusals the shared buffer still gives the allocating call's result
    want, _ = _host_call(ref, idx, dist, _params(n_iter=5))
    rc, got, _ = _noalloc_call(ref, idx, dist, _params(n_iter=5))
    _lib.check(rc, "fastembedr_hip_transform_tsne_noalloc")
    np.testing.assert_array_equal(got, want)
