"""Host-side mirror of the reference's openTSNE KNN entry point for the HIP backend.

``opentsne_knn()`` follows R/fast_knn_tsne.R:39-187 and the dispatch in
R/tsne_affinity_dispatch.R:37-396 of tkcaccia/fastEmbedR: KNN coercion and
self-neighbour stripping, the neighbour/perplexity policy, the "auto"
parameter resolution (opt-SNE learning rate n / 12 in both phases,
exaggeration 12, max_step_norm 5), then a call of the C ABI.  Only the
``backend="hip"`` route exists here; there is no CPU fallback.
"""

from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .session import TsneSession

OPTIMIZER_LABEL = "opentsne_fitsne_fft_grid_native_hip"
REPULSION_LABEL = "fft_grid_hip"
INTERP_REPULSION_LABEL = "fitsne_interpolation_grid_hip"
PROBABILITIES_LABEL = "symmetric_sparse_knn_hip_float32"


# ---------------------------------------------------------------------------
# Policy (src/tsne_neighbors.cpp:1573-1618, R/tsne_control.R)
# ---------------------------------------------------------------------------
def tsne_auto_parameters(n: int, k: int, perplexity: float | None = None) -> dict:
    """Mirror of tsne_auto_parameters_cpp (src/tsne_neighbors.cpp:1573-1618)."""
    if n < 2:
        raise ValueError("`n` must be at least 2.")
    if k < 1:
        raise ValueError("`k` must be positive.")
    missing = perplexity is None or not math.isfinite(perplexity) or perplexity <= 0
    max_n = max(1, (n - 1) // 3)
    max_k = max(1, k // 3)
    resolved = float(min(30, min(max_n, max_k))) if missing else float(perplexity)
    max_resolved = min(max_n, max_k) if perplexity is None else max_n
    resolved = max(1.0, min(resolved, float(max_resolved)))
    early = 12.0
    needed_k = max(1, min(n - 1, int(math.ceil(resolved))))
    return dict(perplexity=resolved, n_neighbors=needed_k, early_exaggeration=early, exaggeration=1.0,
                learning_rate=n / early, early_exaggeration_iter=250, n_iter=500, auto_kld_stop=False,
                auto_iter_end=5000.0,
                rule="opt_sne_learning_rate_fixed_iterations_no_expensive_kld_polling")


def opentsne_neighbor_policy(n: int, perplexity: float | None = None, available: int | None = None) -> dict:
    """Mirror of opentsne_neighbor_policy (R/tsne_control.R:28-68)."""
    if n < 2:
        raise ValueError("`data` must contain at least two rows.")
    max_perplexity = (n - 1) // 3
    if available is not None and available < 1:
        raise ValueError("The supplied KNN object has no usable non-self neighbor columns.")
    if perplexity is None:
        nn = max(1, min(15, n - 1))
        if available is not None:
            nn = min(nn, available)
        return dict(perplexity=None, n_neighbors=int(nn))
    perplexity = float(perplexity)
    if not math.isfinite(perplexity) or perplexity <= 0:
        raise ValueError("`perplexity` must be a positive finite number.")
    if perplexity > max_perplexity:
        raise ValueError("`perplexity` must be no larger than floor((nrow(data) - 1) / 3).")
    nn = max(1, min(n - 1, int(math.ceil(perplexity))))
    if available is not None and nn > available:
        raise ValueError("The supplied KNN object has fewer non-self columns than `ceiling(perplexity)`.")
    return dict(perplexity=perplexity, n_neighbors=int(nn))


def knn_index_offset(indices: np.ndarray) -> int:
    """1 iff every index lies in [1, n] (src/embedding_cuda_impl.cpp:890-902)."""
    n = indices.shape[0]
    return 1 if (indices.min() >= 1 and indices.max() <= n) else 0


def strip_self_neighbors(indices: np.ndarray, distances: np.ndarray, float32: bool = True):
    """Drops a self column (R/knn_input.R:108-166, src/embedding_utils.cpp:1025-1130).

    Returns (indices, distances, has_self).  A self entry is the row's own
    index at distance <= tolerance; when every row has one, it is removed.
    """
    n, k = indices.shape
    if k < 1:
        return indices, distances, False
    tol = max(math.sqrt(np.finfo(np.float32).eps), 1e-6) if float32 else max(math.sqrt(np.finfo(np.float64).eps), 1e-12)
    expected = np.arange(n) + knn_index_offset(indices)
    if np.all((indices[:, 0] == expected) & (distances[:, 0] <= tol)):
        return indices[:, 1:], distances[:, 1:], True
    mask = (indices == expected[:, None]) & (distances <= tol)
    if not np.all(mask.any(axis=1)):
        return indices, distances, False
    if k == 1:
        return indices[:, :0], distances[:, :0], True
    first = mask.argmax(axis=1)
    keep = np.ones((n, k), bool)
    keep[np.arange(n), first] = False
    return indices[keep].reshape(n, k - 1), distances[keep].reshape(n, k - 1), True


def normalize_negative_gradient_method(method: str) -> str:
    """R/tsne_control.R:174-197 aliases; the HIP route supports FFT only
    (as the CUDA route, src/embedding_cuda_impl.cpp:2110-2122)."""
    m = str(method).lower().replace("-", "_")
    if m in ("bh", "barnes_hut", "barnes"):
        raise ValueError('`negative_gradient_method = "bh"` has been removed from fastEmbedR.')
    if m in ("sampled", "negative_sampling", "sample"):
        raise ValueError('`negative_gradient_method = "sampled"` is not part of the standard GPU openTSNE path '
                         "because it changes the optimization mathematics.")
    aliases = {"auto": "fft", "fft": "fft", "interpolation": "fft", "fitsne": "fft", "fit_sne": "fft",
               "exact": "exact", "pair": "exact", "pair_symmetric": "exact"}
    if m not in aliases:
        raise ValueError('`negative_gradient_method` must be one of `"auto"`, `"exact"`, or `"fft"`.')
    if aliases[m] != "fft":
        raise ValueError('HIP openTSNE supports `negative_gradient_method = "fft"` only.')
    return "fft"


@dataclass
class OpenTsneResult:
    """Layout plus the fields the reference attaches as attributes."""

    layout: np.ndarray
    config: dict
    itercosts: np.ndarray = field(default_factory=lambda: np.zeros(0))
    itercost_iterations: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    # per-row KL terms of the final layout when costs are recorded
    # (src/tsne_neighbors.cpp:1816-1823), else empty
    costs: np.ndarray = field(default_factory=lambda: np.zeros(0))


def _is_device_knn(knn) -> bool:
    """A device-resident KNN result (R/native_knn.R:17-37: the layout fields
    plus "cuda" residency; here "hip")."""
    return getattr(knn, "result_residency", None) == "hip" and getattr(knn, "device_indices", None) is not None


def _coerce_knn(indices, distances):
    if distances is None:
        if isinstance(indices, dict) and "indices" in indices and "distances" in indices:
            distances = indices["distances"]
            indices = indices["indices"]
        elif getattr(indices, "indices", None) is not None and getattr(indices, "distances", None) is not None:
            distances = indices.distances
            indices = indices.indices
        else:
            raise ValueError("`distances` is required unless `indices` is a mapping containing "
                             "`indices` and `distances`.")
    idx = np.asarray(indices)
    dist = np.asarray(distances)
    if idx.shape != dist.shape or idx.ndim != 2:
        raise ValueError("KNN `indices` and `distances` must have the same dimensions.")
    if idx.shape[0] < 2 or idx.shape[1] < 1:
        raise ValueError("KNN input must have at least two rows and one neighbor column.")
    if not np.issubdtype(idx.dtype, np.integer):
        idx = idx.astype(np.int64)
    return idx, dist


def opentsne_knn(indices, distances=None, n_neighbors: int | None = None, perplexity: float | None = None,
                 n_components: int = 2, Y_init=None, seed: int = 4, verbose: bool = False, backend: str = "hip",
                 learning_rate="auto", early_exaggeration_iter: int | None = None, early_exaggeration="auto",
                 n_iter: int | None = None, exaggeration: float | None = None, initial_momentum: float = 0.8,
                 final_momentum: float = 0.8, min_gain: float = 0.01, max_step_norm="auto",
                 negative_gradient_method: str = "auto", record_costs: bool = False,
                 auto_config: bool = True, interpolation_grid: dict | None = None) -> OpenTsneResult:
    """openTSNE-style t-SNE from precomputed KNN on the HIP backend.

    Arguments have the meaning of R's ``opentsne_knn()``.  ``Y_init=None``
    uses the reference CPU backend's own initialisation, mt19937(seed)
    normals with sd 1e-4 (R's ``rnorm`` stream cannot be reproduced here).

    The repulsion is the reference's bilinear grid for every FFT method
    string, as in the reference (src/tsne_neighbors.cpp:354-390).
    ``interpolation_grid`` (an extension with no R counterpart) selects the
    FIt-SNE interpolation grid instead; it is a dict of openTSNE's settings,
    ``n_interpolation_points`` (3), ``min_num_intervals`` (50) and
    ``ints_in_interval`` (1.0), any of which may be omitted.
    """
    if str(backend).lower() != "hip":
        raise ValueError(f'backend "{backend}" is not part of this build; only backend = "hip" is provided. '
                         "No CPU fallback is used for HIP-labelled runs.")
    if not _lib.available():
        raise _lib.HipBackendUnavailable(
            "Native HIP openTSNE optimizer was requested, but it is not available in this build. "
            "No CPU fallback is used for HIP-labelled runs.")
    if n_components != 2:
        raise ValueError("HIP openTSNE FFT-grid currently supports exactly two output components.")
    method = normalize_negative_gradient_method(negative_gradient_method)
    interp = None
    if interpolation_grid is not None:
        unknown = set(interpolation_grid) - {"n_interpolation_points", "min_num_intervals", "ints_in_interval"}
        if unknown:
            raise ValueError(f"unknown interpolation_grid settings: {sorted(unknown)}")
        interp = (int(interpolation_grid.get("n_interpolation_points", 3)),
                  int(interpolation_grid.get("min_num_intervals", 50)),
                  float(interpolation_grid.get("ints_in_interval", 1.0)))

    device_knn = indices if distances is None and _is_device_knn(indices) else None
    if device_knn is not None:
        # device-resident, self excluded, 1-based (the reference's GPU KNN contract)
        if not getattr(device_knn, "exclude_self", True):
            raise ValueError("A device-resident KNN object must exclude self neighbours.")
        n, available = int(device_knn.n), int(device_knn.k)
        if n < 2:
            raise ValueError("KNN input must have at least two rows and one neighbor column.")
    else:
        idx0, dist0 = _coerce_knn(indices, distances)
        float32_input = dist0.dtype == np.float32
        idx_s, dist_s, has_self = strip_self_neighbors(idx0, dist0, float32=float32_input)
        n = idx_s.shape[0]
        available = idx_s.shape[1]
    if available < 1:
        raise ValueError("KNN input must contain at least one non-self neighbor.")
    policy = opentsne_neighbor_policy(n, perplexity, available)
    if n_neighbors is None:
        n_neighbors = policy["n_neighbors"]
    n_neighbors = int(n_neighbors)
    if n_neighbors < 1 or n_neighbors >= n:
        raise ValueError("`n_neighbors` must be a positive integer smaller than the number of rows.")
    if n_neighbors > available:
        raise ValueError("`n_neighbors` is larger than the supplied KNN width.")
    if perplexity is None:
        perplexity = policy["perplexity"]
    if device_knn is None:
        idx_m = idx_s[:, :n_neighbors]
        dist_m = dist_s[:, :n_neighbors]
    k = n_neighbors

    # "auto" resolution (R/tsne_control.R:70-130, 249-283; R/tsne_affinity_dispatch.R:190-217)
    auto = tsne_auto_parameters(n, k, perplexity) if auto_config else dict(
        perplexity=perplexity if perplexity is not None else float(max(1, min(30, (n - 1) // 3, k // 3))),
        early_exaggeration_iter=250, n_iter=500, learning_rate=float("nan"))
    perplexity = float(auto["perplexity"]) if perplexity is None else float(perplexity)
    if early_exaggeration_iter is None:
        early_exaggeration_iter = int(auto["early_exaggeration_iter"])
    if n_iter is None:
        n_iter = int(auto["n_iter"])
    if early_exaggeration_iter < 0 or n_iter < 0:
        raise ValueError("iteration counts must be non-negative.")
    if early_exaggeration_iter + n_iter < 1:
        raise ValueError("At least one optimization iteration is required.")
    if n - 1 < 3 * perplexity:
        raise ValueError("perplexity is too large for the number of samples.")
    if initial_momentum < 0 or final_momentum < 0:
        raise ValueError("momentum values must be non-negative.")
    normal_ex = 1.0 if exaggeration is None else float(exaggeration)
    if isinstance(early_exaggeration, str) and early_exaggeration.lower() == "auto":
        early_ex = 12.0 if exaggeration is None else max(12.0, normal_ex)
    else:
        early_ex = float(early_exaggeration)
    if not (early_ex > 0 and normal_ex > 0):
        raise ValueError("exaggeration values must be positive.")
    lr_auto = isinstance(learning_rate, str) and learning_rate.lower() == "auto"
    opt_sne_lr = bool(auto_config) and lr_auto
    if opt_sne_lr and math.isfinite(auto["learning_rate"]) and auto["learning_rate"] > 0:
        lr_auto, lr_value = False, float(auto["learning_rate"])
    elif lr_auto:
        lr_value = 1.0
    else:
        lr_value = float(learning_rate)
        if not (lr_value > 0):
            raise ValueError('`learning_rate` must be a positive number or "auto".')
    if not (min_gain > 0):
        raise ValueError("`min_gain` must be a positive number.")
    if isinstance(max_step_norm, str) and max_step_norm.lower() == "auto":
        step = 5.0
    elif max_step_norm is None or (isinstance(max_step_norm, float) and math.isnan(max_step_norm)):
        step = float("nan")
    else:
        step = float(max_step_norm)
        if not (step > 0):
            raise ValueError("`max_step_norm` must be NULL/NA or a positive number.")

    init = None
    if Y_init is not None:
        init = np.ascontiguousarray(Y_init, dtype=np.float32)
        if init.shape != (n, 2):
            raise ValueError("incorrect format for `Y_init`.")

    if device_knn is None:
        offset = knn_index_offset(idx_m)
        idx_c = np.asfortranarray(idx_m, dtype=np.int32)
    else:
        # column-major n x k: the first n_neighbors columns are a prefix of the buffers
        offset = int(getattr(device_knn, "index_base", 1))
    out = np.empty((n, 2), np.float32)
    itercosts = np.zeros(0)
    iters = np.zeros(0, np.int32)
    row_costs = np.zeros(0)
    lr_early = n / early_ex if lr_auto else lr_value
    lr_normal = n / normal_ex if lr_auto else lr_value
    if record_costs or verbose or interp is not None:
        # Session route: same kernels, with the exact KL every 50 iterations
        # when costs are recorded, and the interpolation grid when asked for.
        if device_knn is None:
            sess = TsneSession(idx_c, np.asfortranarray(dist_m, dtype=np.float32), perplexity=perplexity,
                               index_offset=offset)
        else:
            sess = TsneSession(perplexity=perplexity, index_offset=offset, n=n, k=k,
                               device_pointers=(device_knn.indices_ptr, device_knn.distances_ptr))
        try:
            if interp is not None:
                sess.set_repulsion(_lib.REPULSION_LAGRANGE, *interp)
            if init is None:
                init = np.empty((n, 2), np.float32)
                _lib.check(_lib.load().fastembedr_hip_random_init(n, int(seed) & 0xFFFFFFFF,
                                                                  C.c_void_p(init.ctypes.data)), "random_init")
            sess.set_state(init)
            sess.center()
            costs, its = [], []
            total = early_exaggeration_iter + n_iter
            done = 0
            for count, ex, mom, lr in ((early_exaggeration_iter, early_ex, initial_momentum, lr_early),
                                       (n_iter, normal_ex, final_momentum, lr_normal)):
                left = count
                while left > 0:
                    to_next = 50 - (done % 50)
                    step_n = min(left, to_next)
                    sess.run(step_n, ex, mom, lr, min_gain, step)
                    done += step_n
                    left -= step_n
                    if (record_costs or verbose) and (done % 50 == 0 or done == total):
                        costs.append(sess.kl())
                        its.append(done)
                        if verbose:
                            print(f"Iteration {done}: error is {costs[-1]}")
            out = sess.y
            itercosts = np.asarray(costs)
            iters = np.asarray(its, np.int32)
            if record_costs:
                _, row_costs = sess.kl_rows()
        finally:
            sess.close()
    else:
        lib = _lib.load()
        if device_knn is not None:
            idx_p, dist_p = C.c_void_p(device_knn.indices_ptr), C.c_void_p(device_knn.distances_ptr)
            fn = lib.fastembedr_hip_opentsne_fft_from_device_knn_float
        elif dist_m.dtype == np.float64:
            dist_c = np.asfortranarray(dist_m, dtype=np.float64)
            idx_p, dist_p = C.c_void_p(idx_c.ctypes.data), C.c_void_p(dist_c.ctypes.data)
            fn = lib.fastembedr_hip_opentsne_fft_from_knn
        else:
            dist_c = np.asfortranarray(dist_m, dtype=np.float32)
            idx_p, dist_p = C.c_void_p(idx_c.ctypes.data), C.c_void_p(dist_c.ctypes.data)
            fn = lib.fastembedr_hip_opentsne_fft_from_knn_float
        init_p = None if init is None else C.c_void_p(init.ctypes.data)
        rc = fn(idx_p, dist_p, init_p, int(init is not None), n,
                k, 2, float(perplexity), int(early_exaggeration_iter), int(n_iter), float(early_ex),
                float(normal_ex), float(lr_value), int(lr_auto), float(initial_momentum), float(final_momentum),
                float(min_gain), float(step), int(seed) & 0xFFFFFFFF, offset, C.c_void_p(out.ctypes.data))
        _lib.check(rc, "HIP openTSNE FFT-grid")

    config = dict(
        method="opentsne", backend="hip", n=n, n_neighbors=k, perplexity=perplexity,
        early_exaggeration_iter=int(early_exaggeration_iter), n_iter=int(n_iter),
        max_iter=int(early_exaggeration_iter + n_iter),
        learning_rate=("auto_opt_sne_n_over_early_exaggeration" if opt_sne_lr else ("auto" if lr_auto else lr_value)),
        learning_rate_early=lr_early, learning_rate_normal=lr_normal, early_exaggeration=early_ex,
        exaggeration=normal_ex, initial_momentum=initial_momentum, final_momentum=final_momentum,
        min_gain=min_gain, max_step_norm=step, initialization="user" if Y_init is not None else "random_normal",
        negative_gradient_method=method, auto_config=bool(auto_config), optimizer=OPTIMIZER_LABEL,
        repulsion=REPULSION_LABEL if interp is None else INTERP_REPULSION_LABEL,
        interpolation_grid=None if interp is None else dict(
            n_interpolation_points=interp[0], min_num_intervals=interp[1], ints_in_interval=interp[2]),
        precision="float32", probabilities=PROBABILITIES_LABEL,
        input_had_self=False if device_knn is not None else has_self,
        knn_residency="hip" if device_knn is not None else "host", record_costs=bool(record_costs or verbose),
        provenance="openTSNE_style_native_hip_symmetric_knn_gpu_probability_optimizer",
    )
    return OpenTsneResult(layout=out.astype(np.float64), config=config, itercosts=itercosts,
                          itercost_iterations=iters, costs=row_costs)
