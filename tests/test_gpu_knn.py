"""Exact KNN on the GPU (knn_hip.hip through fastembedr_hip_knn_exact)
against the CPU oracle (oracle/knn_oracle.py, the ordering of the reference's
tests/testthat/helper-knn.R:5-38).

The bar: indices identical to the oracle's (ties by index included),
distances within 2e-6 relative (fp32 square roots of fp64 squared
distances).  Cases: row- and column-major input, self excluded or not, odd
and small d, d above 64, d above 128 (scanned in a projection: low-rank
data up to d = 784 and isotropic data), k = n - 1, sizes off the tile shapes, lattice data
with duplicates and long runs of exact ties (which take the rerun path with a
larger candidate set), device input and device-resident output, the
reference's argument errors, and a large input checked on sampled rows
against a direct CPU computation.
"""

import sys

import numpy as np
import pytest

from fastembedr_amd import _lib
from oracle import knn_oracle

pytestmark = pytest.mark.gpu

DIST_RTOL = 2e-6


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check(res, x, k, exclude_self=True):
    ref_i, ref_d = knn_oracle.exact_knn(x, k, exclude_self=exclude_self)
    got_i = np.asarray(res.indices)
    got_d = np.asarray(res.distances)
    assert got_i.shape == (x.shape[0], k) and got_i.dtype == np.int32
    assert got_d.dtype == np.float32
    bad = np.nonzero((got_i - 1 != ref_i).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {got_i[bad[0]] - 1} vs {ref_i[bad[0]]}"
    np.testing.assert_allclose(got_d, ref_d, rtol=DIST_RTOL, atol=1e-30)


def _gauss(n, d, seed, scale=1.0, offset=0.0):
    rng = np.random.default_rng(seed)
    return (rng.normal(size=(n, d)) * scale + offset).astype(np.float32)


@pytest.mark.parametrize("n,d,k", [(3000, 10, 15), (1000, 2, 30), (777, 7, 5), (5, 3, 3), (130, 1, 12)])
def test_matches_oracle(hip, n, d, k):
    _say(f"case: exact KNN n={n} d={d} k={k}")
    x = _gauss(n, d, seed=n + d)
    _check(hip.exact_knn(x, k), x, k)


def test_column_major_input_and_offset_data(hip):
    _say("case: column-major input with a large common offset")
    x = _gauss(2500, 12, seed=5, scale=0.5, offset=300.0)  # centring keeps the expansion accurate
    res_c = hip.exact_knn(np.asfortranarray(x), 20)
    res_r = hip.exact_knn(np.ascontiguousarray(x), 20)
    np.testing.assert_array_equal(res_c.indices, res_r.indices)
    np.testing.assert_array_equal(res_c.distances, res_r.distances)
    _check(res_c, x, 20)


def test_self_included(hip):
    _say("case: exclude_self = False")
    x = _gauss(1500, 9, seed=11)
    res = hip.exact_knn(x, 10, exclude_self=False)
    _check(res, x, 10, exclude_self=False)
    assert np.all(res.indices[:, 0] == np.arange(1, 1501))


@pytest.mark.parametrize("n,d,k", [(2000, 100, 25), (900, 65, 40), (600, 128, 8)])
def test_wide_rows(hip, n, d, k):
    _say(f"case: wide rows n={n} d={d} k={k}")
    x = _gauss(n, d, seed=d)
    _check(hip.exact_knn(x, k), x, k)


def _low_rank(n, d, rank, seed, noise=0.05, components=8):
    """Rows on a few clusters of a rank-`rank` subspace of R^d plus small
    isotropic noise: the spectrum of image or expression data, whose leading
    principal directions carry most of the variance."""
    rng = np.random.default_rng(seed)
    basis = np.linalg.qr(rng.normal(size=(d, rank)))[0]
    centres = rng.normal(scale=4.0, size=(components, rank))
    z = centres[rng.integers(0, components, size=n)] + rng.normal(size=(n, rank))
    return (z @ basis.T + rng.normal(scale=noise, size=(n, d)) + 3.0).astype(np.float32)


@pytest.mark.parametrize("n,d,k,rank", [(3000, 300, 20, 24), (1500, 784, 30, 60), (5000, 784, 90, 50),
                                        (1000, 129, 10, 129)])
def test_rows_wider_than_the_scan(hip, n, d, k, rank):
    # d > 128: the scan runs on the projection on 128 leading directions (a
    # lower bound of every distance); the ranking is exact in full width.
    # rank = d is isotropic data, where the projection keeps most but not
    # all of the variance and rows take the rerun path.
    _say(f"case: exact KNN of rows wider than the scan n={n} d={d} k={k} rank={rank}")
    x = _low_rank(n, d, rank, seed=d) if rank < d else _gauss(n, d, seed=d)
    res = hip.exact_knn(x, k)
    _say(f"  stats {res.stats}")
    _check(res, x, k)
    res_c = hip.exact_knn(np.asfortranarray(x), k, exclude_self=False)
    _check(res_c, x, k, exclude_self=False)


def test_wide_isotropic_rows(hip):
    # 200 isotropic dimensions: the 128 leading directions keep ~64 % of the
    # spread, too little to certify k = 60 within the largest candidate set;
    # those rows are ranked by a full pass over the references instead.
    _say("case: exact KNN of isotropic rows n=3000 d=200 k=60 (full pass for uncertified rows)")
    x = _gauss(3000, 200, seed=3)
    res = hip.exact_knn(x, 60)
    _say(f"  stats {res.stats}")
    assert res.stats["rerun_rows"] > 0
    _check(res, x, 60)


def test_wide_isotropic_rows_beyond_the_full_pass_budget_are_refused(hip):
    # 20000 x 600 isotropic rows: no candidate set certifies them and a full
    # pass for each (2.4e11 row-reference-dimension steps) exceeds the time
    # budget, so the search refuses instead of returning an unproven result.
    _say("case: exact KNN of isotropic rows n=20000 d=600 k=30 (refused)")
    with pytest.raises(_lib.HipBackendError, match="reduce the dimension"):
        hip.exact_knn(_gauss(20000, 600, seed=5), 30)
    x = _gauss(400, 9, seed=4)
    _check(hip.exact_knn(x, 5), x, 5)  # the library still works afterwards


def test_query_rows_wider_than_the_scan(hip):
    _say("case: query KNN of rows wider than the scan n_ref=2000 n_q=400 d=512 k=15")
    x = _low_rank(2400, 512, 40, seed=3)
    ref, qry = x[:2000], x[2000:]
    _check_query(hip.exact_query_knn(ref, qry, 15), ref, qry, 15)


@pytest.mark.parametrize("metric", ["cosine", "correlation"])
@pytest.mark.parametrize("n,d,k", [(2500, 20, 15), (800, 300, 10)])
def test_cosine_and_correlation(hip, metric, n, d, k):
    # rows normalised on the device in the reference's operation order
    # (bit-identical to the oracle's), then the exact search; distances are
    # 1 - cos = d^2 / 2.  Row scales vary over four orders of magnitude, a
    # zero row and (for correlation) a constant row are included.
    _say(f"case: exact KNN metric={metric} n={n} d={d} k={k}")
    rng = np.random.default_rng(n + d)
    x = (rng.normal(size=(n, d)) + rng.uniform(-1, 1, size=(1, d))).astype(np.float32)
    x *= rng.uniform(0.01, 100.0, size=(n, 1)).astype(np.float32)
    x[7] = 0.0
    x[8] = 2.5
    ref_i, ref_d = knn_oracle.metric_knn(x, k, metric)
    for layout in (np.ascontiguousarray, np.asfortranarray):
        res = hip.precompute_knn(layout(x), k=k, metric=metric)
        assert res.metric == metric
        got_i = np.asarray(res.indices) - 1
        bad = np.nonzero((got_i != ref_i).any(axis=1))[0]
        assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}"
        np.testing.assert_allclose(np.asarray(res.distances), ref_d, rtol=DIST_RTOL, atol=1e-7)
    q = (rng.normal(size=(200, d))).astype(np.float32)
    qi, qd = knn_oracle.metric_knn(x, k, metric, query=q)
    qres = hip.precompute_query_knn(x, q, k=k, metric=metric)
    np.testing.assert_array_equal(np.asarray(qres.indices) - 1, qi)
    np.testing.assert_allclose(np.asarray(qres.distances), qd, rtol=DIST_RTOL, atol=1e-7)


def test_metric_errors(hip):
    _say("case: KNN metric errors")
    x = _gauss(50, 4, seed=1)
    with pytest.raises(ValueError, match="CUDA-only"):
        hip.precompute_knn(x, k=3, metric="inner_product")
    with pytest.raises(ValueError, match="must be one of"):
        hip.exact_knn(x, 3, metric="manhattan")
    lib = _lib.load()
    idx = np.empty((3, 50), np.int32)
    dist = np.empty((3, 50), np.float32)
    assert lib.fastembedr_hip_knn_exact_metric(x.ctypes.data, 50, 4, 0, 3, 1, 7, 0, idx.ctypes.data,
                                               dist.ctypes.data, 0, None) == 1
    assert "metric" in _lib.last_error()


def test_k_is_n_minus_one(hip):
    _say("case: k = n - 1")
    x = _gauss(70, 4, seed=2)
    res = hip.exact_knn(x, 69)
    _check(res, x, 69)
    for i in range(70):
        assert sorted(res.indices[i] - 1) == [j for j in range(70) if j != i]


def test_max_k(hip):
    _say("case: k = 256")
    x = _gauss(4000, 16, seed=3)
    _check(hip.exact_knn(x, 256), x, 256)


@pytest.mark.parametrize("exclude_self", [True, False])
def test_lattice_ties_and_duplicates(hip, exclude_self):
    _say(f"case: lattice ties exclude_self={exclude_self}")
    rng = np.random.default_rng(21)
    x = rng.integers(0, 3, size=(2000, 6)).astype(np.float32)  # 729 distinct points, integer d2
    res = hip.exact_knn(x, 20, exclude_self=exclude_self)
    _check(res, x, 20, exclude_self=exclude_self)
    _say(f"  stats {res.stats}")


def test_rerun_path_is_taken_and_exact(hip):
    _say("case: long tie runs force reruns")
    rng = np.random.default_rng(22)
    # 8 distinct points, ~375 copies each: the first candidate set (192) ends
    # inside the run of zero distances, so no row is certified until the
    # candidate set outgrows the run
    x = rng.integers(0, 2, size=(3000, 3)).astype(np.float32)
    res = hip.exact_knn(x, 60)
    _say(f"  stats {res.stats}")
    assert res.stats["passes"] >= 2 and res.stats["rerun_rows"] > 0
    _check(res, x, 60)


def test_device_input_and_output(hip):
    from fastembedr_amd.device import DeviceMatrix

    _say("case: device input, device-resident result")
    x = _gauss(3000, 20, seed=8)
    host = hip.exact_knn(x, 12)
    dm = DeviceMatrix.from_host(x)
    dev = hip.precompute_knn(dm, k=12, keep_device=True)
    assert dev.result_residency == "hip"
    assert dev.device_indices.shape == (12, 3000)
    back = dev.to_host()
    np.testing.assert_array_equal(back.indices, host.indices)
    np.testing.assert_array_equal(back.distances, host.distances)
    # column-major device input gives the same result
    dev2 = hip.exact_knn(DeviceMatrix.from_host(x, col_major=True), 12)
    np.testing.assert_array_equal(dev2.indices, host.indices)
    np.testing.assert_array_equal(dev2.distances, host.distances)


def test_device_knn_feeds_opentsne(hip):
    """The device-resident result builds the same P as its host copy, and
    opentsne_knn takes it directly (a few iterations agree within the
    gradient tolerance: float atomics reorder sums from run to run)."""
    from fastembedr_amd import synthetic
    from tests.helpers import rel_l2

    _say("case: device-resident KNN into the t-SNE session and opentsne_knn")
    spec = synthetic.MixtureSpec(n=3000, dim=10, components=5, mean_sd=4.0)
    x, _ = synthetic.gaussian_mixture(spec, seed=3)
    x = x.astype(np.float32)
    host = hip.precompute_knn(x, k=30)
    dev = hip.precompute_knn(x, k=30, keep_device=True)
    with hip.TsneSession(host.indices, host.distances, perplexity=10.0, index_offset=1) as sh, \
            hip.TsneSession(perplexity=10.0, index_offset=1, n=dev.n, k=dev.k,
                            device_pointers=(dev.indices_ptr, dev.distances_ptr)) as sd:
        for a, b in zip(sh.csr(), sd.csr()):
            np.testing.assert_array_equal(a, b)
    y0 = synthetic.pca_init(x)
    a = hip.opentsne_knn(host, perplexity=10.0, Y_init=y0, early_exaggeration_iter=5, n_iter=5)
    b = hip.opentsne_knn(dev, perplexity=10.0, Y_init=y0, early_exaggeration_iter=5, n_iter=5)
    assert b.config["knn_residency"] == "hip" and a.config["knn_residency"] == "host"
    assert rel_l2(b.layout, a.layout) <= 1e-3


def test_errors(hip):
    _say("case: argument errors")
    x = _gauss(10, 4, seed=1)
    with pytest.raises(ValueError, match="between 1 and nrow"):
        hip.precompute_knn(x, k=10)
    with pytest.raises(_lib.HipBackendError, match="k exceeds"):
        hip.exact_knn(x, 10, exclude_self=True)
    with pytest.raises(_lib.HipBackendError, match="dimensions"):
        hip.exact_knn(_gauss(20, 16385, seed=2), 5)
    with pytest.raises(_lib.HipBackendError, match="k up to"):
        hip.exact_knn(_gauss(400, 3, seed=2), 257)
    bad = _gauss(300, 5, seed=4)
    bad[17, 2] = np.nan
    with pytest.raises(_lib.HipBackendError, match="non-finite"):
        hip.exact_knn(bad, 5)
    lib = _lib.load()
    assert lib.fastembedr_hip_knn_exact(None, 10, 4, 0, 3, 1, 0, None, None, 0, None) == 1
    # the library still works after the errors
    _check(hip.exact_knn(x, 3), x, 3)


def test_large_input_sampled_rows(hip):
    """200k points of a 20-component mixture in 50 dimensions, k = 90 (the
    benchmark's shape at a fifth of its size): sampled rows against a direct
    fp64 computation over all points."""
    from fastembedr_amd import synthetic

    _say("case: 200k x 50, k = 90, sampled rows")
    spec = synthetic.MixtureSpec(n=200_000, dim=50, components=20, mean_sd=4.0)
    x, _ = synthetic.gaussian_mixture(spec, seed=5)
    x = np.ascontiguousarray(x, dtype=np.float32)
    res = hip.exact_knn(x, 90)
    _say(f"  elapsed {res.elapsed_sec:.3f} s, stats {res.stats}")
    xd = x.astype(np.float64)
    rows = np.random.default_rng(0).choice(x.shape[0], 64, replace=False)
    for i in rows:
        d2 = ((xd - xd[i]) ** 2).sum(1)
        d2[i] = np.inf
        order = np.lexsort((np.arange(x.shape[0]), d2))[:90]
        np.testing.assert_array_equal(res.indices[i] - 1, order)
        np.testing.assert_allclose(res.distances[i], np.sqrt(d2[order]), rtol=DIST_RTOL)


# ---- query-to-reference search (fastembedr_hip_knn_query) ----------------------------


def _check_query(res, ref, qry, k):
    ref_i, ref_d = knn_oracle.exact_query_knn(ref, qry, k)
    got_i = np.asarray(res.indices)
    assert got_i.shape == (qry.shape[0], k) and got_i.dtype == np.int32
    bad = np.nonzero((got_i - 1 != ref_i).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {got_i[bad[0]] - 1} vs {ref_i[bad[0]]}"
    np.testing.assert_allclose(np.asarray(res.distances), ref_d, rtol=DIST_RTOL, atol=1e-30)


@pytest.mark.parametrize("n_ref,n_q,d,k", [(3000, 500, 10, 15), (700, 1300, 3, 30), (40, 17, 5, 40),
                                           (2000, 300, 77, 12)])
def test_query_matches_oracle(hip, n_ref, n_q, d, k):
    _say(f"case: query KNN n_ref={n_ref} n_q={n_q} d={d} k={k}")
    ref = _gauss(n_ref, d, seed=n_ref)
    qry = _gauss(n_q, d, seed=n_q + 1) * 1.1 + 0.2
    _check_query(hip.precompute_query_knn(ref, qry, k=k), ref, qry, k)


def test_query_layouts_ties_and_device(hip):
    from fastembedr_amd.device import DeviceMatrix

    _say("case: query KNN column-major, queries on reference rows, device buffers")
    rng = np.random.default_rng(41)
    ref = rng.integers(0, 3, size=(1500, 4)).astype(np.float32)  # duplicates and exact ties
    qry = np.concatenate([ref[:200], rng.integers(0, 3, size=(100, 4)).astype(np.float32)])
    res = hip.exact_query_knn(ref, qry, 25)
    _check_query(res, ref, qry, 25)
    res_cm = hip.exact_query_knn(np.asfortranarray(ref), np.asfortranarray(qry), 25)
    np.testing.assert_array_equal(res_cm.indices, res.indices)
    dev = hip.exact_query_knn(DeviceMatrix.from_host(ref), DeviceMatrix.from_host(qry), 25, keep_device=True)
    back = dev.to_host()
    np.testing.assert_array_equal(back.indices, res.indices)
    np.testing.assert_array_equal(back.distances, res.distances)


def test_query_config3_shape(hip):
    """Query-to-reference search at the transform configuration's shape, scaled
    down (reference 20k x 50 from a 10-component mixture, 5k queries from the
    same mixture, k = 30)."""
    from fastembedr_amd import synthetic

    _say("case: query KNN 20k refs x 5k queries x 50 dims, k = 30")
    spec = synthetic.MixtureSpec(n=25_000, dim=50, components=10, mean_sd=4.0)
    x, _ = synthetic.gaussian_mixture(spec, seed=12)
    x = x.astype(np.float32)
    ref, qry = x[:20_000], x[20_000:]
    res = hip.exact_query_knn(ref, qry, 30)
    _say(f"  elapsed {res.elapsed_sec:.3f} s, stats {res.stats}")
    _check_query(res, ref, qry, 30)


def test_query_errors(hip):
    _say("case: query KNN argument errors")
    ref = _gauss(20, 4, seed=1)
    with pytest.raises(ValueError, match="between 1 and nrow"):
        hip.precompute_query_knn(ref, ref[:3], k=21)
    with pytest.raises(ValueError, match="same number of columns"):
        hip.exact_query_knn(ref, _gauss(5, 3, seed=2), 3)
    with pytest.raises(_lib.HipBackendError, match="k exceeds"):
        hip.exact_query_knn(ref, ref[:3], 21)
    _check_query(hip.exact_query_knn(ref, ref[:3], 20), ref, ref[:3], 20)
