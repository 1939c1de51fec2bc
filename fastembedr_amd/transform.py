"""Host-side mirror of the reference's fixed-reference t-SNE transform for the
HIP backend.

``transform_tsne()`` follows R/transform_tsne.R:57-315 of tkcaccia/fastEmbedR
(argument meaning, defaults, the n_negatives rule and the result labels) and
R/transform_embedding.R:77-111 (KNN coercion), then calls the C ABI entry
fastembedr_hip_transform_tsne, whose numerics follow transform_tsne_cpp
(src/tsne_neighbors.cpp:1859-2109).  Only precomputed query KNN is accepted
(the reference's own native query-KNN search is outside this build), and only
two-dimensional reference layouts, as in the reference's GPU branches.
"""

from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field

import numpy as np

from . import _lib

INITIALIZATIONS = {"median": 0, "weighted": 1, "random": 2}
NA_SEED = -(2 ** 31)  # R's NA_integer_


@dataclass
class TransformResult:
    layout: np.ndarray                      # (n_query, 2) float64
    config: dict = field(default_factory=dict)

    def __array__(self, dtype=None, copy=None):
        return self.layout if dtype is None else self.layout.astype(dtype)


def _coerce_query_knn(knn, n_reference: int, k: int | None):
    """R/transform_embedding.R:77-111: `knn` with `indices` and `distances`
    of one shape; the first k columns are used."""
    if isinstance(knn, dict):
        indices, distances = knn.get("indices"), knn.get("distances")
    else:
        indices, distances = getattr(knn, "indices", None), getattr(knn, "distances", None)
    if indices is None or distances is None:
        raise ValueError("`knn` must contain `indices` and `distances`.")
    idx = np.asarray(indices)
    dist = np.asarray(distances, dtype=np.float64)
    if idx.ndim != 2 or idx.shape != dist.shape:
        raise ValueError("KNN `indices` and `distances` must have the same dimensions.")
    if idx.shape[0] < 1 or idx.shape[1] < 1:
        raise ValueError("`knn` must have at least one row and one neighbor column.")
    if k is not None:
        k = int(k)
        if k < 1:
            raise ValueError("`k` must be NULL or a positive integer.")
        if k > idx.shape[1]:
            raise ValueError("`k` cannot be larger than the available reference count.")
        idx, dist = idx[:, :k], dist[:, :k]
    return np.asfortranarray(idx, dtype=np.int32), np.asfortranarray(dist)


def transform_tsne(reference_layout, knn=None, reference_data=None, new_data=None, k: int | None = None,
                   perplexity: float = 5.0, initialization: str = "median", Y_init=None, n_iter: int = 250,
                   early_exaggeration_iter: int = 0, learning_rate: float = 0.1, early_exaggeration: float = 4.0,
                   exaggeration: float = 1.5, initial_momentum: float = 0.8, final_momentum: float = 0.8,
                   max_grad_norm: float = 0.25, max_step_norm: float = math.inf, n_negatives: int | None = None,
                   exact_repulsion_threshold: int = 4096, seed: int | None = 4,
                   backend: str = "hip", reference_grid: dict | None = None) -> TransformResult:
    """Places new points against a fixed two-dimensional reference layout.

    ``reference_grid`` (an extension with no R counterpart) replaces the
    reference's exact / sampled repulsion by the reference's repulsion fields
    precomputed once on an interpolation grid and interpolated at each query
    (fastembedr_hip_transform_tsne_grid); a dict of ``n_interpolation_points``
    (3), ``min_num_intervals`` (50) and ``ints_in_interval`` (0.5: two boxes
    per unit of span), any of which may be omitted.  ``n_negatives`` and
    ``exact_repulsion_threshold`` do not apply then."""
    if str(backend).lower() != "hip":
        raise ValueError(f'backend "{backend}" is not part of this build; only backend = "hip" is provided. '
                         "No CPU fallback is used for HIP-labelled runs.")
    if knn is None:
        raise ValueError("This build takes precomputed query neighbours: supply `knn` "
                         "(`reference_data` / `new_data` need the package's native query KNN search).")
    ref = np.asarray(reference_layout, dtype=np.float64)
    if ref.ndim != 2 or ref.shape[0] < 1:
        raise ValueError("`reference_layout` must be a non-empty matrix.")
    if ref.shape[1] != 2:
        raise ValueError("HIP t-SNE transform currently supports only two-dimensional reference layouts.")
    if initialization not in INITIALIZATIONS:
        raise ValueError("`initialization` must be 'median', 'weighted', or 'random'.")
    perplexity = float(perplexity)
    if not (math.isfinite(perplexity) and perplexity > 0):
        raise ValueError("`perplexity` must be a positive number.")
    n_ref = ref.shape[0]
    idx, dist = _coerce_query_knn(knn, n_ref, k)
    n_query, kk = idx.shape
    n_iter, early_exaggeration_iter = int(n_iter), int(early_exaggeration_iter)
    if n_iter < 0 or early_exaggeration_iter < 0 or n_iter + early_exaggeration_iter < 1:
        raise ValueError("Transform iteration counts must be non-negative and sum to at least one.")
    exact_repulsion_threshold = int(exact_repulsion_threshold)
    if n_negatives is None:
        n_negatives = n_ref if n_ref <= exact_repulsion_threshold else min(256, n_ref)
    n_negatives = int(n_negatives)
    if n_negatives < 1:
        raise ValueError("`n_negatives` must be NULL or a positive integer.")
    init = None
    if Y_init is not None:
        init = np.asfortranarray(Y_init, dtype=np.float64)
        if init.shape != (n_query, 2):
            raise ValueError("`Y_init` must have one row per query and the same columns as `reference_layout`.")
    if not _lib.available():
        raise _lib.HipBackendUnavailable(
            "Native HIP t-SNE transform was requested, but it is not available in this build. "
            "No CPU fallback is used for HIP-labelled runs.")
    seed_i = NA_SEED if seed is None else int(seed)
    ref_cm = np.asfortranarray(ref)
    out = np.empty((n_query, 2), np.float64, order="F")
    exact = C.c_int(0)
    lib = _lib.load()
    if reference_grid is not None:
        return _transform_grid(lib, ref_cm, idx, dist, init, initialization, perplexity, n_iter,
                               early_exaggeration_iter, learning_rate, early_exaggeration, exaggeration,
                               initial_momentum, final_momentum, max_grad_norm, max_step_norm, seed, seed_i,
                               reference_grid, out)
    rc = lib.fastembedr_hip_transform_tsne(
        ref_cm.ctypes.data_as(C.c_void_p), n_ref, idx.ctypes.data_as(C.c_void_p), dist.ctypes.data_as(C.c_void_p),
        n_query, kk, None if init is None else init.ctypes.data_as(C.c_void_p), INITIALIZATIONS[initialization],
        perplexity, n_iter, early_exaggeration_iter, float(learning_rate), float(early_exaggeration),
        float(exaggeration), float(initial_momentum), float(final_momentum), float(max_grad_norm),
        float(max_step_norm), n_negatives, exact_repulsion_threshold, seed_i, out.ctypes.data_as(C.c_void_p),
        C.byref(exact))
    _lib.check(rc, "HIP t-SNE transform")
    n_neg_used = min(n_negatives, n_ref)
    config = dict(
        method="transform_tsne", backend="hip", n_reference=n_ref, n_query=n_query, k=kk, perplexity=perplexity,
        n_iter=n_iter, early_exaggeration_iter=early_exaggeration_iter, learning_rate=float(learning_rate),
        early_exaggeration=float(early_exaggeration), exaggeration=float(exaggeration),
        initial_momentum=float(initial_momentum), final_momentum=float(final_momentum),
        max_grad_norm=float(max_grad_norm), max_step_norm=float(max_step_norm), n_negatives=n_neg_used,
        exact_repulsion_threshold=exact_repulsion_threshold, initialization=initialization,
        optimizer="opentsne_style_fixed_reference_transform",
        repulsion="exact_reference" if exact.value else "sampled_reference",
        affinities="precomputed_query_conditional", affinity_storage="flat_row_major_double",
        transform_batch_size=n_query, transform_batches=1, seed=seed,
        transform="opentsne_style_fixed_reference")
    return TransformResult(np.ascontiguousarray(out), config)


GRID_DEFAULTS = {"n_interpolation_points": 3, "min_num_intervals": 50, "ints_in_interval": 0.5}


def _transform_grid(lib, ref_cm, idx, dist, init, initialization, perplexity, n_iter, early_exaggeration_iter,
                    learning_rate, early_exaggeration, exaggeration, initial_momentum, final_momentum,
                    max_grad_norm, max_step_norm, seed, seed_i, settings, out) -> TransformResult:
    unknown = set(settings) - set(GRID_DEFAULTS)
    if unknown:
        raise ValueError(f"unknown reference_grid settings: {sorted(unknown)}")
    grid = {**GRID_DEFAULTS, **settings}
    n_ref = ref_cm.shape[0]
    n_query, kk = idx.shape
    stats = (C.c_longlong * 3)()
    rc = lib.fastembedr_hip_transform_tsne_grid(
        ref_cm.ctypes.data_as(C.c_void_p), n_ref, idx.ctypes.data_as(C.c_void_p), dist.ctypes.data_as(C.c_void_p),
        n_query, kk, None if init is None else init.ctypes.data_as(C.c_void_p), INITIALIZATIONS[initialization],
        perplexity, n_iter, early_exaggeration_iter, float(learning_rate), float(early_exaggeration),
        float(exaggeration), float(initial_momentum), float(final_momentum), float(max_grad_norm),
        float(max_step_norm), seed_i, int(grid["n_interpolation_points"]), int(grid["min_num_intervals"]),
        float(grid["ints_in_interval"]), out.ctypes.data_as(C.c_void_p), stats)
    _lib.check(rc, "HIP t-SNE transform (reference grid)")
    config = dict(
        method="transform_tsne", backend="hip", n_reference=n_ref, n_query=n_query, k=kk, perplexity=perplexity,
        n_iter=n_iter, early_exaggeration_iter=early_exaggeration_iter, learning_rate=float(learning_rate),
        early_exaggeration=float(early_exaggeration), exaggeration=float(exaggeration),
        initial_momentum=float(initial_momentum), final_momentum=float(final_momentum),
        max_grad_norm=float(max_grad_norm), max_step_norm=float(max_step_norm), initialization=initialization,
        optimizer="opentsne_style_fixed_reference_transform", repulsion="reference_grid_interpolation",
        reference_grid=dict(grid, boxes_per_axis=int(stats[0]), nodes_per_axis=int(stats[1]),
                            exact_evaluations=int(stats[2])),
        affinities="precomputed_query_conditional", affinity_storage="flat_row_major_double",
        transform_batch_size=n_query, transform_batches=1, seed=seed,
        transform="opentsne_style_fixed_reference")
    return TransformResult(np.ascontiguousarray(out), config)
