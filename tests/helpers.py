"""Shared numpy restatements and fixtures for the tests (closed forms used to
pin the oracle, and small seeded KNN problems)."""

from __future__ import annotations

import numpy as np

from fastembedr_amd import synthetic


def small_problem(n=600, dim=8, k=24, components=4, seed=3, one_based=True):
    spec = synthetic.MixtureSpec(n=n, dim=dim, components=components, mean_sd=4.0)
    x, labels = synthetic.gaussian_mixture(spec, seed=seed)
    idx, dist = synthetic.exact_knn_numpy(x, k)
    idx_r, dist_r = synthetic.to_r_layout(idx, dist, one_based=one_based)
    return x, labels, idx_r, dist_r


def query_problem(n_ref=3000, nq=1200, k=30, seed=11):
    """A fixed-reference transform problem: a reference layout (a 2-D
    embedding stand-in: cluster centres plus noise), 20-D mixture data, and
    each query's exact k nearest reference rows (1-based, fp64 distances)."""
    spec = synthetic.MixtureSpec(n=n_ref + nq, dim=20, components=8, mean_sd=4.0)
    x, labels = synthetic.gaussian_mixture(spec, seed=seed)
    rng = np.random.default_rng(seed)
    centers = rng.normal(0, 8, size=(8, 2))
    layout = centers[labels[:n_ref]] + rng.normal(0, 1.0, size=(n_ref, 2))
    xr, xq = x[:n_ref].astype(np.float64), x[n_ref:].astype(np.float64)
    d2 = (xq ** 2).sum(1)[:, None] - 2 * xq @ xr.T + (xr ** 2).sum(1)[None, :]
    idx = np.argsort(d2, axis=1)[:, :k]
    dist = np.sqrt(np.maximum(np.take_along_axis(d2, idx, axis=1), 0))
    return layout, (idx + 1).astype(np.int32), dist


class DeviceArray:
    """A host array copied into device memory with the HIP runtime that the
    backend library already loaded (no second runtime in the process)."""

    def __init__(self, host: np.ndarray):
        import ctypes as C

        from fastembedr_amd import _lib

        _lib.load()
        self._hip = C.CDLL("libamdhip64.so.7")
        self._hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self._hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self._hip.hipFree.argtypes = [C.c_void_p]
        host = np.ascontiguousarray(host)
        self.nbytes = host.nbytes
        self.ptr = C.c_void_p()
        if self._hip.hipMalloc(C.byref(self.ptr), self.nbytes) != 0:
            raise RuntimeError("hipMalloc failed")
        if self._hip.hipMemcpy(self.ptr, C.c_void_p(host.ctypes.data), self.nbytes, 1) != 0:
            raise RuntimeError("hipMemcpy failed")

    @property
    def address(self) -> int:
        return int(self.ptr.value)

    def to_host(self, dtype, shape, order="C") -> np.ndarray:
        """The first prod(shape) elements, copied back to a new host array."""
        import ctypes as C

        out = np.empty(shape, dtype=dtype, order=order)
        if out.nbytes > self.nbytes:
            raise ValueError("read beyond the device buffer")
        if self._hip.hipMemcpy(C.c_void_p(out.ctypes.data), self.ptr, out.nbytes, 2) != 0:
            raise RuntimeError("hipMemcpy failed")
        return out

    def free(self):
        if self.ptr:
            self._hip.hipFree(self.ptr)
            self.ptr = None


def csr_to_dense(row_ptr, col, val, n):
    m = np.zeros((n, n), np.float64)
    for i in range(n):
        s, e = row_ptr[i], row_ptr[i + 1]
        m[i, col[s:e]] += val[s:e]
    return m


def exact_gradient_numpy(y, p_dense, ex):
    """openTSNE-convention gradient: ex * sum_j p_ij q_ij (yi - yj) - sum_j q_ij^2 (yi - yj) / Z."""
    y = y.astype(np.float64)
    d = y[:, None, :] - y[None, :, :]
    r2 = (d * d).sum(-1)
    q = 1.0 / (1.0 + r2)
    np.fill_diagonal(q, 0.0)
    z = q.sum()
    rep = -((q * q)[:, :, None] * d).sum(1) / z
    att = ex * ((p_dense * q)[:, :, None] * d).sum(1)
    return rep + att


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def knn_preservation(x_high, y_low, k=15, sample=2000, seed=4):
    """Share of each sampled point's k nearest low-dimensional neighbours that
    are among its k nearest high-dimensional ones, within the sample; ties
    broken by index (src/embedding_utils.cpp:1582-1752, knn_preservation)."""
    n = x_high.shape[0]
    rng = np.random.default_rng(seed)
    keep = np.sort(rng.choice(n, size=min(sample, n), replace=False))
    xh = x_high[keep].astype(np.float64)
    yl = y_low[keep].astype(np.float64)
    m = keep.size

    def ranks(z):
        sq = (z * z).sum(1)
        d = sq[:, None] + sq[None, :] - 2 * z @ z.T
        np.fill_diagonal(d, np.inf)
        order = np.lexsort((np.broadcast_to(np.arange(m), (m, m)), d), axis=1)
        return order

    oh = ranks(xh)[:, :k]
    ol = ranks(yl)[:, :k]
    shared = sum(len(np.intersect1d(oh[i], ol[i], assume_unique=True)) for i in range(m))
    return shared / (m * k)
