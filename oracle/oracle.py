"""ctypes view of the CPU oracle (oracle/tsne_oracle.cpp, oracle/transform_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product path never loads it.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libtsne_oracle.so"

METHOD_GRID = 0
METHOD_EXACT = 1
METHOD_LAGRANGE = 2

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        build()
    lib = C.CDLL(str(LIB))
    P, I, F, D = C.c_void_p, C.c_int, C.c_float, C.c_double
    sig = {
        "tsne_oracle_last_error": (C.c_char_p, []),
        "tsne_oracle_policy_grid_size": (I, [I]),
        "tsne_oracle_conditional_p": (I, [P, I, I, D, P, P, P]),
        "tsne_oracle_build_p": (P, [P, P, I, I, D, I]),
        "tsne_oracle_wrap_p": (P, [P, P, P, I]),
        "tsne_oracle_p_nnz": (C.c_longlong, [P]),
        "tsne_oracle_p_copy": (None, [P, P, P, P]),
        "tsne_oracle_p_free": (None, [P]),
        "tsne_oracle_gradient": (I, [P, P, I, F, I, I, I, I, I, P]),
        "tsne_oracle_gradient_grid_f64": (I, [P, P, I, F, I, I, P]),
        "tsne_oracle_grid_fields": (I, [P, P, I, I, I, P, P]),
        "tsne_oracle_lagrange_gradient": (I, [P, P, I, F, I, I, F, I, I, P, P, P]),
        "tsne_oracle_lagrange_weights": (None, [D, I, P]),
        "tsne_oracle_update": (None, [P, P, P, P, I, F, F, F, F, I]),
        "tsne_oracle_zero_mean": (None, [P, I]),
        "tsne_oracle_kl": (D, [P, P, I, I, P]),
        "tsne_oracle_optimize": (I, [P, P, I, I, I, D, D, D, I, D, D, D, D, I, I, I, I, P, P]),
        "tsne_oracle_random_init": (None, [P, I, C.c_uint]),
        "transform_oracle_last_error": (C.c_char_p, []),
        "transform_oracle_offset": (I, [P, I, I, I]),
        "transform_oracle_conditional_p": (None, [P, I, I, D, I, P]),
        "transform_oracle_init": (None, [P, I, P, P, I, I, I, I, I, P]),
        "transform_oracle_gradient": (None, [P, I, P, P, I, I, P, D, I, I, I, I, P]),
        "transform_oracle_update": (None, [P, P, P, P, I, D, D, D, D]),
        "transform_oracle_run": (I, [P, I, P, P, I, I, P, I, D, I, I, D, D, D, D, D, D, D, I, I, I, I, P]),
        "transform_oracle_grid_fields": (I, [P, I, P, I, I, D, I, P, P]),
        "transform_oracle_grid_gradient": (C.c_longlong, [P, I, P, P, I, I, P, P, I, D, I, D, I, P]),
        "transform_oracle_grid_run": (I, [P, I, P, P, I, I, P, I, D, I, I, D, D, D, D, D, D, D, I, I, D, I, P, P]),
        "transform_oracle_iteration_seed": (I, [I, I]),
        "transform_oracle_hash32": (C.c_uint, [C.c_uint]),
        "transform_oracle_xorshift": (None, [C.c_uint, I, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _err() -> str:
    return load().tsne_oracle_last_error().decode()


def policy_grid_size(n: int) -> int:
    return int(load().tsne_oracle_policy_grid_size(n))


def conditional_p(distances: np.ndarray, perplexity: float):
    """Row search only: (p (n, k) float32, beta (n,), steps (n,))."""
    d = np.asfortranarray(distances, dtype=np.float32)
    n, k = d.shape
    p = np.empty((n, k), np.float32, order="F")
    beta = np.empty(n, np.float32)
    steps = np.empty(n, np.int32)
    load().tsne_oracle_conditional_p(_p(d), n, k, float(perplexity), _p(p), _p(beta), _p(steps))
    return p, beta, steps


class OracleP:
    """Symmetric CSR P built (or wrapped) on the CPU."""

    def __init__(self, handle, n: int):
        self.h = C.c_void_p(handle)
        self.n = n

    @classmethod
    def build(cls, indices: np.ndarray, distances: np.ndarray, perplexity: float, threads: int = 1) -> "OracleP":
        idx = np.asfortranarray(indices, dtype=np.int32)
        dist = np.asfortranarray(distances, dtype=np.float32)
        n, k = idx.shape
        h = load().tsne_oracle_build_p(_p(idx), _p(dist), n, k, float(perplexity), int(threads))
        if not h:
            raise ValueError(_err())
        return cls(h, n)

    @classmethod
    def wrap(cls, row_ptr, col, val) -> "OracleP":
        rp = np.ascontiguousarray(row_ptr, np.int32)
        cc = np.ascontiguousarray(col, np.int32)
        vv = np.ascontiguousarray(val, np.float32)
        n = rp.size - 1
        return cls(load().tsne_oracle_wrap_p(_p(rp), _p(cc), _p(vv), n), n)

    def __del__(self):
        try:
            if self.h:
                load().tsne_oracle_p_free(self.h)
                self.h = C.c_void_p()
        except Exception:
            pass

    @property
    def nnz(self) -> int:
        return int(load().tsne_oracle_p_nnz(self.h))

    def csr(self):
        nnz = self.nnz
        rp = np.empty(self.n + 1, np.int32)
        col = np.empty(nnz, np.int32)
        val = np.empty(nnz, np.float32)
        load().tsne_oracle_p_copy(self.h, _p(rp), _p(col), _p(val))
        return rp, col, val

    def gradient(self, y: np.ndarray, exaggeration: float = 1.0, method: int = METHOD_GRID, grid_size: int = 0,
                 threads: int = 1, lagrange_order: int = 3, min_intervals: int = 50) -> np.ndarray:
        y = np.ascontiguousarray(y, np.float32).reshape(self.n, 2)
        g = np.empty((self.n, 2), np.float32)
        rc = load().tsne_oracle_gradient(self.h, _p(y), self.n, float(exaggeration), int(method), int(grid_size),
                                         int(lagrange_order), int(min_intervals), int(threads), _p(g))
        if rc != 0:
            raise ValueError(_err())
        return g

    def gradient_grid_f64(self, y: np.ndarray, exaggeration: float = 1.0, grid_size: int = 0,
                          threads: int = 1) -> np.ndarray:
        """The bilinear grid gradient (method METHOD_GRID) with every step in
        fp64: the same algorithm as the reference's fp32 path, evaluated with
        fp64 rounding, so that each fp32 side's own error can be read off."""
        y = np.ascontiguousarray(y, np.float32).reshape(self.n, 2)
        g = np.empty((self.n, 2), np.float64)
        rc = load().tsne_oracle_gradient_grid_f64(self.h, _p(y), self.n, float(exaggeration), int(grid_size),
                                                  int(threads), _p(g))
        if rc != 0:
            raise ValueError(_err())
        return g

    def lagrange_gradient(self, y: np.ndarray, exaggeration: float = 1.0, order: int = 3, min_intervals: int = 50,
                          ints_per_unit: float = 1.0, direct: bool = False, threads: int = 1):
        """FIt-SNE interpolation-grid gradient (an extension: the reference has
        only the bilinear grid).  Returns (grad, geometry, z) with geometry =
        {"boxes", "nodes", "lo", "box_w"}."""
        y = np.ascontiguousarray(y, np.float32).reshape(self.n, 2)
        g = np.empty((self.n, 2), np.float32)
        geo = np.zeros(4, np.float64)
        z = np.zeros(1, np.float64)
        rc = load().tsne_oracle_lagrange_gradient(self.h, _p(y), self.n, float(exaggeration), int(order),
                                                  int(min_intervals), float(ints_per_unit), int(bool(direct)),
                                                  int(threads), _p(g), _p(geo), _p(z))
        if rc != 0:
            raise ValueError(_err())
        geometry = {"boxes": int(geo[0]), "nodes": int(geo[1]), "lo": float(geo[2]), "box_w": float(geo[3])}
        return g, geometry, float(z[0])

    def grid_fields(self, y: np.ndarray, grid_size: int = 0, threads: int = 1):
        """(geometry (lo_x, lo_y, h, 1/h), fields (4, g, g): q, q2, xq2, yq2)."""
        y = np.ascontiguousarray(y, np.float32).reshape(self.n, 2)
        geom = np.empty(4, np.float32)
        g = int(load().tsne_oracle_grid_fields(self.h, _p(y), self.n, int(grid_size), int(threads), _p(geom), None))
        fields = np.empty((4, g, g), np.float32)
        load().tsne_oracle_grid_fields(self.h, _p(y), self.n, int(grid_size), int(threads), _p(geom), _p(fields))
        return geom, fields

    def kl(self, y: np.ndarray, threads: int = 1, row_costs: bool = False):
        y = np.ascontiguousarray(y, np.float32).reshape(self.n, 2)
        rc = np.empty(self.n, np.float64) if row_costs else None
        v = float(load().tsne_oracle_kl(self.h, _p(y), self.n, int(threads), _p(rc)))
        return (v, rc) if row_costs else v

    def optimize(self, y0: np.ndarray, early_iter: int, n_iter: int, early_ex: float, ex: float,
                 learning_rate: float, learning_rate_auto: bool, m0: float, m1: float, min_gain: float = 0.01,
                 max_step_norm: float = 5.0, method: int = METHOD_GRID, grid_size: int = 0, threads: int = 1,
                 record_costs: bool = False):
        y = np.array(y0, dtype=np.float32, copy=True).reshape(self.n, 2)
        total = early_iter + n_iter
        cap = max(1, -(-total // 50))
        costs = np.zeros(cap, np.float64)
        its = np.zeros(cap, np.int32)
        rec = load().tsne_oracle_optimize(self.h, _p(y), self.n, int(early_iter), int(n_iter), float(early_ex),
                                          float(ex), float(learning_rate), int(bool(learning_rate_auto)), float(m0),
                                          float(m1), float(min_gain), float(max_step_norm), int(method),
                                          int(grid_size), int(threads), int(bool(record_costs)), _p(costs), _p(its))
        if rec < 0:
            raise ValueError(_err())
        return y, costs[:rec], its[:rec]


def update(y, upd, gains, grad, lr, momentum, min_gain=0.01, max_step_norm=5.0, threads=1):
    """In-place update of float32 arrays (n, 2)."""
    n = y.shape[0]
    load().tsne_oracle_update(_p(y), _p(upd), _p(gains), _p(grad), n, float(lr), float(momentum), float(min_gain),
                              float(max_step_norm), int(threads))


def lagrange_weights(u: float, order: int) -> np.ndarray:
    w = np.empty(order, np.float64)
    load().tsne_oracle_lagrange_weights(float(u), int(order), _p(w))
    return w


def zero_mean(y):
    load().tsne_oracle_zero_mean(_p(y), y.shape[0])


def random_init(n: int, seed: int) -> np.ndarray:
    y = np.empty((n, 2), np.float32)
    load().tsne_oracle_random_init(_p(y), n, int(seed) & 0xFFFFFFFF)
    return y


# ---------------------------------------------------------------------------
# Fixed-reference transform (transform_oracle.cpp).  Layouts as R hands them
# over: reference (n_ref, 2), indices / distances (nq, k), column-major
# internally; y arrays (nq, 2) row-major float64.
# ---------------------------------------------------------------------------
INIT_MEDIAN, INIT_WEIGHTED, INIT_RANDOM = 0, 1, 2


def _f64_cm(a):
    return np.asfortranarray(a, dtype=np.float64)


def transform_offset(indices, n_ref: int) -> int:
    idx = np.asfortranarray(indices, dtype=np.int32)
    return int(load().transform_oracle_offset(_p(idx), idx.shape[0], idx.shape[1], int(n_ref)))


def transform_conditional_p(distances, perplexity: float, threads: int = 1) -> np.ndarray:
    d = _f64_cm(distances)
    nq, k = d.shape
    p = np.empty((nq, k), np.float64)
    load().transform_oracle_conditional_p(_p(d), nq, k, float(perplexity), int(threads), _p(p))
    return p


def transform_init(reference, indices, distances, mode: int = INIT_MEDIAN, seed: int = 4, threads: int = 1):
    ref = _f64_cm(reference)
    idx = np.asfortranarray(indices, dtype=np.int32)
    d = _f64_cm(distances)
    nq, k = idx.shape
    y = np.empty((nq, 2), np.float64)
    load().transform_oracle_init(_p(ref), ref.shape[0], _p(idx), _p(d), nq, k, int(mode), int(seed), int(threads),
                                 _p(y))
    return y


def transform_gradient(reference, indices, p, y, exaggeration: float, n_negatives: int, exact_threshold: int,
                       iter_seed: int, threads: int = 1) -> np.ndarray:
    ref = _f64_cm(reference)
    idx = np.asfortranarray(indices, dtype=np.int32)
    pp = np.ascontiguousarray(p, np.float64)
    yy = np.ascontiguousarray(y, np.float64)
    nq, k = idx.shape
    g = np.empty((nq, 2), np.float64)
    load().transform_oracle_gradient(_p(ref), ref.shape[0], _p(idx), _p(pp), nq, k, _p(yy), float(exaggeration),
                                     int(n_negatives), int(exact_threshold), int(iter_seed), int(threads), _p(g))
    return g


def transform_update(y, upd, gains, grad, lr, momentum, max_grad_norm, max_step_norm):
    """In place on float64 (nq, 2) arrays; grad is clipped in place."""
    load().transform_oracle_update(_p(y), _p(upd), _p(gains), _p(grad), y.shape[0], float(lr), float(momentum),
                                   float(max_grad_norm), float(max_step_norm))


def transform_run(reference, indices, distances, y_init=None, initialization: int = INIT_MEDIAN,
                  perplexity: float = 5.0, n_iter: int = 250, early_exaggeration_iter: int = 0,
                  learning_rate: float = 0.1, early_exaggeration: float = 4.0, exaggeration: float = 1.5,
                  initial_momentum: float = 0.8, final_momentum: float = 0.8, max_grad_norm: float = 0.25,
                  max_step_norm: float = float("inf"), n_negatives: int = 256, exact_threshold: int = 4096,
                  seed: int = 4, threads: int = 1):
    """Returns (layout (nq, 2) float64, exact_repulsion bool)."""
    ref = _f64_cm(reference)
    idx = np.asfortranarray(indices, dtype=np.int32)
    d = _f64_cm(distances)
    nq, k = idx.shape
    init = None if y_init is None else _f64_cm(y_init)
    out = np.empty((nq, 2), np.float64, order="F")
    rc = load().transform_oracle_run(_p(ref), ref.shape[0], _p(idx), _p(d), nq, k, _p(init), int(initialization),
                                     float(perplexity), int(n_iter), int(early_exaggeration_iter),
                                     float(learning_rate), float(early_exaggeration), float(exaggeration),
                                     float(initial_momentum), float(final_momentum), float(max_grad_norm),
                                     float(max_step_norm), int(n_negatives), int(exact_threshold), int(seed),
                                     int(threads), _p(out))
    if rc < 0:
        raise ValueError(load().transform_oracle_last_error().decode())
    return np.ascontiguousarray(out), bool(rc)


def transform_grid_fields(reference, y, min_intervals: int = 50, ints_in_interval: float = 1.0,
                          threads: int = 1, fields: bool = True):
    """Reference-grid geometry around the reference and the query layout y
    (nq, 2): ({"lo", "box_w", "boxes", "nodes"}, node fields (nodes, nodes,
    3) = (Z, Fx, Fy) or None)."""
    ref = _f64_cm(reference)
    yy = np.ascontiguousarray(y, np.float64).reshape(-1, 2)
    geo = np.zeros(4, np.float64)
    m_guess = None
    rc = load().transform_oracle_grid_fields(_p(ref), ref.shape[0], _p(yy), yy.shape[0], int(min_intervals),
                                             float(ints_in_interval), int(threads), _p(geo), None)
    if rc < 0:
        raise ValueError(load().transform_oracle_last_error().decode())
    m_guess = int(geo[3])
    f = None
    if fields:
        f = np.empty((m_guess, m_guess, 3), np.float64)
        load().transform_oracle_grid_fields(_p(ref), ref.shape[0], _p(yy), yy.shape[0], int(min_intervals),
                                            float(ints_in_interval), int(threads), _p(geo), _p(f))
    return {"lo": float(geo[0]), "box_w": float(geo[1]), "boxes": int(geo[2]), "nodes": int(geo[3])}, f


def transform_grid_gradient(reference, indices, p, y, exaggeration: float, min_intervals: int = 50,
                            ints_in_interval: float = 1.0, threads: int = 1, geometry_y=None):
    """Gradient at y with the reference-grid repulsion, the grid built around
    the reference and geometry_y (default: y): (grad (nq, 2), queries that
    took the exact sums)."""
    ref = _f64_cm(reference)
    idx = np.asfortranarray(indices, dtype=np.int32)
    pp = np.ascontiguousarray(p, np.float64)
    yy = np.ascontiguousarray(y, np.float64)
    gy = yy if geometry_y is None else np.ascontiguousarray(geometry_y, np.float64).reshape(-1, 2)
    nq, k = idx.shape
    g = np.empty((nq, 2), np.float64)
    out = load().transform_oracle_grid_gradient(_p(ref), ref.shape[0], _p(idx), _p(pp), nq, k, _p(yy), _p(gy),
                                                gy.shape[0], float(exaggeration), int(min_intervals),
                                                float(ints_in_interval), int(threads), _p(g))
    if out < 0:
        raise ValueError(load().transform_oracle_last_error().decode())
    return g, int(out)


def transform_grid_run(reference, indices, distances, y_init=None, initialization: int = INIT_MEDIAN,
                       perplexity: float = 5.0, n_iter: int = 250, early_exaggeration_iter: int = 0,
                       learning_rate: float = 0.1, early_exaggeration: float = 4.0, exaggeration: float = 1.5,
                       initial_momentum: float = 0.8, final_momentum: float = 0.8, max_grad_norm: float = 0.25,
                       max_step_norm: float = float("inf"), seed: int = 4, min_intervals: int = 50,
                       ints_in_interval: float = 1.0, threads: int = 1):
    """Whole transform with the reference-grid repulsion: (layout (nq, 2),
    {"boxes", "nodes", "exact_evaluations"})."""
    ref = _f64_cm(reference)
    idx = np.asfortranarray(indices, dtype=np.int32)
    d = _f64_cm(distances)
    nq, k = idx.shape
    init = None if y_init is None else _f64_cm(y_init)
    out = np.empty((nq, 2), np.float64, order="F")
    stats = np.zeros(3, np.int64)
    rc = load().transform_oracle_grid_run(_p(ref), ref.shape[0], _p(idx), _p(d), nq, k, _p(init),
                                          int(initialization), float(perplexity), int(n_iter),
                                          int(early_exaggeration_iter), float(learning_rate),
                                          float(early_exaggeration), float(exaggeration), float(initial_momentum),
                                          float(final_momentum), float(max_grad_norm), float(max_step_norm),
                                          int(seed), int(min_intervals), float(ints_in_interval), int(threads),
                                          _p(out), _p(stats))
    if rc < 0:
        raise ValueError(load().transform_oracle_last_error().decode())
    return np.ascontiguousarray(out), {"boxes": int(stats[0]), "nodes": int(stats[1]),
                                       "exact_evaluations": int(stats[2])}


def transform_iteration_seed(seed: int, it: int) -> int:
    return int(load().transform_oracle_iteration_seed(int(seed), int(it)))


def hash32(v: int) -> int:
    return int(load().transform_oracle_hash32(int(v) & 0xFFFFFFFF))


def xorshift32(state: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint32)
    load().transform_oracle_xorshift(int(state) & 0xFFFFFFFF, int(count), _p(out))
    return out
