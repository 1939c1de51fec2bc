"""Python view of the session ABI (fastembedr_hip_tsne_*).

A ``TsneSession`` owns P and the optimiser state in HBM.  Host arrays follow
the ABI layouts: KNN column-major n x k, layouts row-major n x 2.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib


def _ptr(a: np.ndarray | None) -> C.c_void_p | None:
    return None if a is None else C.c_void_p(a.ctypes.data)


class TsneSession:
    """P construction + iteration control on one device.

    ``indices`` / ``distances`` are numpy arrays of shape (n, k) (any memory
    order; they are passed column-major as the ABI requires), or, with
    ``device_pointers=(idx_ptr, dist_ptr)``, raw device addresses of
    column-major int32 / float32 buffers.
    """

    def __init__(self, indices=None, distances=None, perplexity: float = 30.0, index_offset: int = 0,
                 grid_size: int = 0, n: int | None = None, k: int | None = None,
                 device_pointers: tuple[int, int] | None = None):
        lib = _lib.load()
        self._lib = lib
        self._h = C.c_void_p()
        if device_pointers is not None:
            if n is None or k is None:
                raise ValueError("n and k are required with device pointers")
            idx_p, dist_p = (C.c_void_p(int(device_pointers[0])), C.c_void_p(int(device_pointers[1])))
            on_device = 1
            self.n, self.k = int(n), int(k)
        else:
            idx = np.asfortranarray(indices, dtype=np.int32)
            dist = np.asfortranarray(distances, dtype=np.float32)
            if idx.shape != dist.shape or idx.ndim != 2:
                raise ValueError("KNN `indices` and `distances` must have the same dimensions.")
            self.n, self.k = idx.shape
            self._keep = (idx, dist)
            idx_p, dist_p = _ptr(idx), _ptr(dist)
            on_device = 0
        rc = lib.fastembedr_hip_tsne_create(idx_p, dist_p, self.n, self.k, float(perplexity), int(index_offset),
                                            on_device, int(grid_size), C.byref(self._h))
        _lib.check(rc, "fastembedr_hip_tsne_create")
        self._keep = None

    # -- lifetime -----------------------------------------------------------
    def close(self) -> None:
        if self._h:
            self._lib.fastembedr_hip_tsne_destroy(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- P ------------------------------------------------------------------
    @property
    def nnz(self) -> int:
        v = C.c_longlong()
        _lib.check(self._lib.fastembedr_hip_tsne_p_nnz(self._h, C.byref(v)), "p_nnz")
        return int(v.value)

    @property
    def grid_size(self) -> int:
        v = C.c_int()
        _lib.check(self._lib.fastembedr_hip_tsne_grid_size(self._h, C.byref(v)), "grid_size")
        return int(v.value)

    @property
    def p_build_ms(self) -> float:
        v = C.c_double()
        _lib.check(self._lib.fastembedr_hip_tsne_p_build_ms(self._h, C.byref(v)), "p_build_ms")
        return float(v.value)

    def csr(self) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        nnz = self.nnz
        row_ptr = np.empty(self.n + 1, np.int32)
        col = np.empty(nnz, np.int32)
        val = np.empty(nnz, np.float32)
        _lib.check(self._lib.fastembedr_hip_tsne_copy_p(self._h, _ptr(row_ptr), _ptr(col), _ptr(val)), "copy_p")
        return row_ptr, col, val

    def conditional_p(self) -> np.ndarray:
        """p_{j|i} as an (n, k) array."""
        out = np.empty((self.n, self.k), np.float32, order="F")
        _lib.check(self._lib.fastembedr_hip_tsne_copy_conditional_p(self._h, _ptr(out)), "copy_conditional_p")
        return out

    # -- state --------------------------------------------------------------
    def set_state(self, y, update=None, gains=None) -> None:
        y = np.ascontiguousarray(y, dtype=np.float32).reshape(self.n, 2)
        u = None if update is None else np.ascontiguousarray(update, dtype=np.float32).reshape(self.n, 2)
        g = None if gains is None else np.ascontiguousarray(gains, dtype=np.float32).reshape(self.n, 2)
        _lib.check(self._lib.fastembedr_hip_tsne_set_state(self._h, _ptr(y), _ptr(u), _ptr(g)), "set_state")

    def get_state(self) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        y = np.empty((self.n, 2), np.float32)
        u = np.empty((self.n, 2), np.float32)
        g = np.empty((self.n, 2), np.float32)
        _lib.check(self._lib.fastembedr_hip_tsne_get_state(self._h, _ptr(y), _ptr(u), _ptr(g)), "get_state")
        return y, u, g

    @property
    def y(self) -> np.ndarray:
        y = np.empty((self.n, 2), np.float32)
        _lib.check(self._lib.fastembedr_hip_tsne_get_state(self._h, _ptr(y), None, None), "get_state")
        return y

    # -- iteration ----------------------------------------------------------
    def gradient(self, exaggeration: float = 1.0, repulsion: int = _lib.REPULSION_GRID) -> np.ndarray:
        out = np.empty((self.n, 2), np.float32)
        _lib.check(self._lib.fastembedr_hip_tsne_gradient(self._h, float(exaggeration), int(repulsion), _ptr(out)),
                   "gradient")
        return out

    def set_repulsion(self, repulsion: int = _lib.REPULSION_GRID, n_interpolation_points: int = 3,
                      min_num_intervals: int = 50, ints_in_interval: float = 1.0) -> None:
        """Repulsion used by run(): REPULSION_GRID (the reference's bilinear
        grid) or REPULSION_LAGRANGE (the FIt-SNE interpolation grid with
        openTSNE's settings)."""
        _lib.check(self._lib.fastembedr_hip_tsne_set_repulsion(self._h, int(repulsion), int(n_interpolation_points),
                                                               int(min_num_intervals), float(ints_in_interval)),
                   "set_repulsion")

    def interp_info(self) -> dict:
        """Interpolation-grid geometry at the current layout and the FFT
        length of its last iteration."""
        b, m, f = C.c_int(), C.c_int(), C.c_int()
        w = C.c_float()
        z = C.c_double()
        _lib.check(self._lib.fastembedr_hip_tsne_interp_info(self._h, C.byref(b), C.byref(m), C.byref(f),
                                                             C.byref(w), C.byref(z)), "interp_info")
        return {"boxes": b.value, "nodes": m.value, "fft_len": f.value, "box_w": w.value, "z": z.value}

    def attraction_info(self) -> dict:
        """Tiles of the attraction's regrouped P in the current numbering and
        the number of renumberings so far."""
        t = C.c_longlong()
        r = C.c_int()
        _lib.check(self._lib.fastembedr_hip_tsne_attraction_info(self._h, C.byref(t), C.byref(r)), "attraction_info")
        s = C.c_longlong()
        _lib.check(self._lib.fastembedr_hip_tsne_attraction_slots(self._h, C.byref(s)), "attraction_slots")
        return {"tiles": int(t.value), "renumbers": int(r.value), "slots": int(s.value)}

    def graph_info(self) -> dict:
        """Iterations of run() replayed from captured graphs, graphs captured,
        and whether capture is on for this session."""
        n, c, e = C.c_longlong(), C.c_int(), C.c_int()
        _lib.check(self._lib.fastembedr_hip_tsne_graph_info(self._h, C.byref(n), C.byref(c), C.byref(e)),
                   "graph_info")
        return {"launches": int(n.value), "captures": int(c.value), "enabled": bool(e.value)}

    def center(self) -> None:
        _lib.check(self._lib.fastembedr_hip_tsne_center(self._h), "center")

    def run(self, n_iter: int, exaggeration: float, momentum: float, learning_rate: float,
            min_gain: float = 0.01, max_step_norm: float = 5.0) -> None:
        _lib.check(self._lib.fastembedr_hip_tsne_run(self._h, int(n_iter), float(exaggeration), float(momentum),
                                                     float(learning_rate), float(min_gain), float(max_step_norm)),
                   "run")

    def sync(self) -> None:
        _lib.check(self._lib.fastembedr_hip_tsne_sync(self._h), "sync")

    def kl(self) -> float:
        v = C.c_double()
        _lib.check(self._lib.fastembedr_hip_tsne_kl(self._h, C.byref(v)), "kl")
        return float(v.value)

    def kl_rows(self) -> tuple[float, np.ndarray]:
        """Exact KL and each row's term (the reference's per-row `costs`)."""
        v = C.c_double()
        rows = np.empty(self.n, np.float64)
        _lib.check(self._lib.fastembedr_hip_tsne_kl_rows(self._h, C.byref(v), _ptr(rows)), "kl_rows")
        return float(v.value), rows

    # -- timing -------------------------------------------------------------
    def set_timing(self, enabled: bool, only: str | None = None, every: int = 1) -> None:
        """Per-kernel HIP-event timing of run(); `only` names the one kernel
        to time (the others then run without events), on every `every`-th
        iteration."""
        mode = int(bool(enabled))
        if enabled and only is not None:
            names = [self._lib.fastembedr_hip_tsne_kernel_name(i).decode()
                     for i in range(self._lib.fastembedr_hip_tsne_kernel_count())]
            if not 1 <= every < 32768:
                raise ValueError("every must be in [1, 32767]")
            mode = 2 + names.index(only) + (every << 16)
        _lib.check(self._lib.fastembedr_hip_tsne_set_timing(self._h, mode), "set_timing")

    def timing(self) -> dict[str, tuple[int, float]]:
        """{kernel name: (launches timed, summed ms)}."""
        m = self._lib.fastembedr_hip_tsne_kernel_count()
        launches = (C.c_longlong * m)()
        total = (C.c_double * m)()
        _lib.check(self._lib.fastembedr_hip_tsne_timing_stats(self._h, m, launches, total), "timing_stats")
        out = {}
        for i in range(m):
            name = self._lib.fastembedr_hip_tsne_kernel_name(i).decode()
            out[name] = (int(launches[i]), float(total[i]))
        return out
