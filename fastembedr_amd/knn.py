"""Host-side mirror of the reference's native exact KNN for the HIP backend.

``precompute_knn()`` follows R/native_knn.R:237-331 of tkcaccia/fastEmbedR
(argument meaning, the ``1 <= k <= n - 1`` rule and its message, self always
excluded, the result's fields) for the Euclidean, cosine and correlation metrics.  Where the reference
routes CUDA to a FAISS GPU brute force below 100,000 rows and to cuVS
IVF-Flat above (R/native_knn.R:99-126), this build runs one exact search for
every size: fastembedr_hip_knn_exact, an MFMA brute force whose results are
re-ranked in fp64 and certified exact (recall 1 by construction).  Its device
result has the layout of the reference's device-resident KNN
(src/native_knn_cuda_impl.cpp:427-466: column-major query-by-k, 1-based int32
indices, float32 distances) and feeds ``opentsne_knn()`` without a host copy.
"""

from __future__ import annotations

import ctypes as C
import sys
import time
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .device import DeviceBuffer, DeviceMatrix

MAX_DIM = 16384  # kKnnMaxInputDim in csrc/knn_device.h (rows wider than 128 are scanned in a projection)
MAX_K = 256     # kKnnMaxK in csrc/knn_device.h
ENGINE = "native_hip_exact_mfma_l2"


@dataclass
class KnnResult:
    """Neighbours of every row, ascending by (distance, index).

    Host residency: ``indices`` (n, k) int32, 1-based, and ``distances``
    (n, k) float32.  Device residency ("hip"): ``device_indices`` and
    ``device_distances`` are DeviceBuffers of shape (k, n), whose bytes are
    the reference's column-major n x k layout; they live as long as this
    object.
    """

    n: int
    k: int
    indices: np.ndarray | None = None
    distances: np.ndarray | None = None
    device_indices: DeviceBuffer | None = None
    device_distances: DeviceBuffer | None = None
    metric: str = "euclidean"
    exclude_self: bool = True
    backend_requested: str = "hip"
    execution_backend: str = "hip"
    engine: str = ENGINE
    elapsed_sec: float = float("nan")
    result_residency: str = "host"
    index_base: int = 1
    layout: str = "column_major_query_by_k"
    n_reference: int | None = None  # query-to-reference results: rows of the reference
    stats: dict = field(default_factory=dict)

    @property
    def indices_ptr(self) -> int:
        return self.device_indices.address

    @property
    def distances_ptr(self) -> int:
        return self.device_distances.address

    def to_host(self) -> "KnnResult":
        """A host-resident copy (R/native_knn.R:39-59, fastembedr_gpu_knn_to_host)."""
        if self.result_residency == "host":
            return self
        idx = self.device_indices.to_host().T.copy()
        dist = self.device_distances.to_host().T.copy()
        return KnnResult(self.n, self.k, idx, dist, metric=self.metric, exclude_self=self.exclude_self,
                         backend_requested=self.backend_requested, execution_backend=self.execution_backend,
                         engine=self.engine, elapsed_sec=self.elapsed_sec, result_residency="host",
                         stats=dict(self.stats))

    def __getitem__(self, key):  # dict-style access, as R's list fields
        if key in ("indices", "distances") and self.result_residency != "host":
            return getattr(self.to_host(), key)
        return getattr(self, key)

    def keys(self):
        return ("indices", "distances")


def _prepare(data):
    """Returns (pointer, n, d, col_major, on_device, keepalive)."""
    if isinstance(data, DeviceMatrix):
        return data.address, data.n, data.d, int(data.col_major), 1, data
    torch = sys.modules.get("torch")  # never imported here: see device.py
    if torch is not None and isinstance(data, torch.Tensor):
        data = data.detach().to("cpu", torch.float32).numpy()
    x = np.asarray(data)
    if x.ndim != 2:
        raise ValueError("`data` must be a matrix with observations in rows.")
    if not np.issubdtype(x.dtype, np.number) or np.issubdtype(x.dtype, np.complexfloating):
        raise ValueError("`data` must be numeric.")
    if x.dtype == np.float32 and x.flags.f_contiguous and not x.flags.c_contiguous:
        return x.ctypes.data, x.shape[0], x.shape[1], 1, 0, x
    x = np.ascontiguousarray(x, dtype=np.float32)
    return x.ctypes.data, x.shape[0], x.shape[1], 0, 0, x


def _metric_code(metric) -> tuple[str, int]:
    """The reference's metric argument (match.arg: the first of a vector) and
    its code; "inner_product" is CUDA-only in the reference and refused."""
    if isinstance(metric, (list, tuple)):
        metric = metric[0]
    name = str(metric)
    if name == "inner_product":
        raise ValueError("Native HIP KNN does not support this metric; raw inner product is CUDA-only "
                         "in the reference.")
    if name not in _lib.KNN_METRICS:
        raise ValueError("`metric` must be one of \"euclidean\", \"cosine\", \"correlation\", \"inner_product\".")
    return name, _lib.KNN_METRICS[name]


def exact_knn(data, k: int, exclude_self: bool = True, keep_device: bool = False,
              metric: str = "euclidean") -> KnnResult:
    """Exact KNN of the rows of ``data`` among themselves: Euclidean, or
    cosine / correlation (rows normalised, centred first for correlation, as
    the reference does; distances 1 - cos).

    ``data`` is an (n, d) array (float32 is used as is, row- or column-major;
    other numeric types are converted) or a DeviceMatrix already on the GPU.
    With ``exclude_self`` the row itself never appears; without it, it
    competes at distance 0 like any duplicate.  Raises HipBackendError for
    inputs the kernels do not take (d > 16384, k > 256, k beyond the candidate
    count, non-finite values).
    """
    metric, code = _metric_code(metric)
    ptr, n, d, col_major, on_device, keep = _prepare(data)
    k = int(k)
    lib = _lib.load()
    if not lib.fastembedr_hip_available():
        raise _lib.HipBackendUnavailable(
            "Native HIP KNN was requested, but no gfx950 device is visible. No CPU fallback is used.")
    stats = (C.c_longlong * 5)()
    t0 = time.perf_counter()
    if keep_device:
        if not 1 <= k <= MAX_K:
            raise _lib.HipBackendError(f"HIP exact KNN failed: exact KNN supports k up to {MAX_K}")
        dev_idx = DeviceBuffer((k, n), np.int32)
        dev_dist = DeviceBuffer((k, n), np.float32)
        rc = lib.fastembedr_hip_knn_exact_metric(C.c_void_p(ptr), n, d, col_major, k, int(bool(exclude_self)), code,
                                                 on_device, C.c_void_p(dev_idx.address),
                                                 C.c_void_p(dev_dist.address), 1, stats)
        _lib.check(rc, "HIP exact KNN")
        res = KnnResult(n, k, device_indices=dev_idx, device_distances=dev_dist, result_residency="hip")
    else:
        idx = np.empty((max(k, 0), n), np.int32)
        dist = np.empty((max(k, 0), n), np.float32)
        rc = lib.fastembedr_hip_knn_exact_metric(C.c_void_p(ptr), n, d, col_major, k, int(bool(exclude_self)), code,
                                                 on_device, C.c_void_p(idx.ctypes.data),
                                                 C.c_void_p(dist.ctypes.data), 0, stats)
        _lib.check(rc, "HIP exact KNN")
        res = KnnResult(n, k, indices=idx.T, distances=dist.T)
    del keep
    res.elapsed_sec = time.perf_counter() - t0
    res.exclude_self = bool(exclude_self)
    res.metric = metric
    res.stats = dict(rerun_rows=int(stats[0]), passes=int(stats[1]), candidates=int(stats[2]),
                     tiles_staged=int(stats[3]), tiles_computed=int(stats[4]))
    return res


def _prepare_pair(reference, query):
    """Both matrices in one layout and residency: (ref_ptr, n_ref, q_ptr, n_q, d, col_major, on_device, keep)."""
    if isinstance(reference, DeviceMatrix) or isinstance(query, DeviceMatrix):
        if not (isinstance(reference, DeviceMatrix) and isinstance(query, DeviceMatrix)):
            raise ValueError("`reference` and `query` must both be host arrays or both DeviceMatrix objects.")
        if reference.col_major != query.col_major:
            raise ValueError("device `reference` and `query` must share one layout.")
        if reference.d != query.d:
            raise ValueError("`reference` and `query` must have the same number of columns.")
        return (reference.address, reference.n, query.address, query.n, reference.d, int(reference.col_major), 1,
                (reference, query))
    rp, nr, dr, rcm, _, rkeep = _prepare(reference)
    qp, nq, dq, qcm, _, qkeep = _prepare(query)
    if dr != dq:
        raise ValueError("`reference` and `query` must have the same number of columns.")
    if rcm != qcm:  # one layout for both: row-major copies
        rkeep = np.ascontiguousarray(np.asarray(rkeep), dtype=np.float32)
        qkeep = np.ascontiguousarray(np.asarray(qkeep), dtype=np.float32)
        rp, qp, rcm = rkeep.ctypes.data, qkeep.ctypes.data, 0
    return rp, nr, qp, nq, dr, rcm, 0, (rkeep, qkeep)


def exact_query_knn(reference, query, k: int, keep_device: bool = False, metric: str = "euclidean") -> KnnResult:
    """Exact KNN of every row of ``query`` among the rows of ``reference``
    (fastembedr_hip_knn_query_metric), Euclidean or cosine / correlation as
    exact_knn.  Indices are 1-based rows of ``reference``; the result has one
    row per query."""
    metric, code = _metric_code(metric)
    rp, nr, qp, nq, d, col_major, on_device, keep = _prepare_pair(reference, query)
    k = int(k)
    lib = _lib.load()
    if not lib.fastembedr_hip_available():
        raise _lib.HipBackendUnavailable(
            "Native HIP KNN was requested, but no gfx950 device is visible. No CPU fallback is used.")
    stats = (C.c_longlong * 5)()
    t0 = time.perf_counter()
    if keep_device:
        if not 1 <= k <= MAX_K:
            raise _lib.HipBackendError(f"HIP exact query KNN failed: exact KNN supports k up to {MAX_K}")
        dev_idx = DeviceBuffer((k, nq), np.int32)
        dev_dist = DeviceBuffer((k, nq), np.float32)
        rc = lib.fastembedr_hip_knn_query_metric(C.c_void_p(rp), nr, C.c_void_p(qp), nq, d, col_major, k, code,
                                                 on_device, C.c_void_p(dev_idx.address),
                                                 C.c_void_p(dev_dist.address), 1, stats)
        _lib.check(rc, "HIP exact query KNN")
        res = KnnResult(nq, k, device_indices=dev_idx, device_distances=dev_dist, result_residency="hip")
    else:
        idx = np.empty((max(k, 0), nq), np.int32)
        dist = np.empty((max(k, 0), nq), np.float32)
        rc = lib.fastembedr_hip_knn_query_metric(C.c_void_p(rp), nr, C.c_void_p(qp), nq, d, col_major, k, code,
                                                 on_device, C.c_void_p(idx.ctypes.data),
                                                 C.c_void_p(dist.ctypes.data), 0, stats)
        _lib.check(rc, "HIP exact query KNN")
        res = KnnResult(nq, k, indices=idx.T, distances=dist.T)
    del keep
    res.elapsed_sec = time.perf_counter() - t0
    res.exclude_self = False
    res.metric = metric
    res.stats = dict(rerun_rows=int(stats[0]), passes=int(stats[1]), candidates=int(stats[2]),
                     tiles_staged=int(stats[3]), tiles_computed=int(stats[4]))
    return res


def precompute_query_knn(reference, query, k: int = 30, metric: str = "euclidean", backend: str = "hip",
                         n_cores=None, keep_device: bool = False) -> KnnResult:
    """Nearest reference rows of every query row (R's
    ``precompute_query_knn()``, R/native_knn.R:333-416): one-based indices
    into ``reference``, self not excluded.  Metrics "euclidean", "cosine" and
    "correlation" on the HIP backend."""
    if str(backend).lower() != "hip":
        raise ValueError(f'backend "{backend}" is not part of this build; only backend = "hip" is provided. '
                         "No CPU fallback is used for HIP-labelled runs.")
    metric, _ = _metric_code(metric)
    n_ref = reference.n if isinstance(reference, DeviceMatrix) else len(reference)
    try:
        k_int = int(k)
        ok = float(k) == k_int
    except (TypeError, ValueError):
        ok = False
    if not ok or k_int < 1 or k_int > n_ref:
        raise ValueError("`k` must be one integer between 1 and nrow(reference).")
    res = exact_query_knn(reference, query, k_int, keep_device=keep_device, metric=metric)
    res.n_reference = n_ref
    res.backend_requested = "hip"
    return res


def precompute_knn(data, k: int = 30, metric: str = "euclidean", backend: str = "hip", n_cores=None,
                   keep_device: bool = False) -> KnnResult:
    """Nearest neighbours of every observation, itself excluded (R's
    ``precompute_knn()``, R/native_knn.R:237-331).

    Metrics "euclidean", "cosine" and "correlation" on ``backend = "hip"``
    ("inner_product" is CUDA-only in the reference and refused); ``n_cores``
    is accepted and ignored, as by the reference's GPU
    backends.  ``keep_device=True`` leaves the result on the GPU, as the
    reference's CUDA route does.
    """
    if str(backend).lower() != "hip":
        raise ValueError(f'backend "{backend}" is not part of this build; only backend = "hip" is provided. '
                         "No CPU fallback is used for HIP-labelled runs.")
    metric, _ = _metric_code(metric)
    n = data.n if isinstance(data, DeviceMatrix) else len(data)
    try:
        k_int = int(k)
        ok = float(k) == k_int
    except (TypeError, ValueError):
        ok = False
    if not ok or k_int < 1 or k_int >= n:
        raise ValueError("`k` must be one integer between 1 and nrow(data) - 1.")
    res = exact_knn(data, k_int, exclude_self=True, keep_device=keep_device, metric=metric)
    res.backend_requested = "hip"
    return res
