"""Exact rank-based structure metrics on the GPU: the reference's
``exact_structure_metrics_cpp`` (src/embedding_utils.cpp:1582-1752), which
R's ``evaluate_embedding()`` applies to a row sample of at most 5000 rows
(R/evaluate_embedding.R:483-500), through fastembedr_hip_structure_metrics."""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

COLUMNS = ("trustworthiness", "continuity", "knn_preservation", "mean_neighbor_rank_error")


def exact_structure_metrics(high, low, k=(15,)) -> dict:
    """Metrics of layout ``low`` (n x p_low) against data ``high`` (n x
    p_high) for each requested k; returns {column: np.ndarray over k} plus
    ``k``.  Same validation and messages as the reference."""
    h = np.asfortranarray(high, dtype=np.float64)
    lo = np.asfortranarray(low, dtype=np.float64)
    if h.ndim != 2 or lo.ndim != 2:
        raise ValueError("high and low must be matrices")
    if h.shape[0] != lo.shape[0]:
        raise ValueError("high and low must have the same row count")
    ks = np.ascontiguousarray(np.atleast_1d(k), dtype=np.int32)
    out = np.empty((ks.size, 4), np.float64, order="F")
    lib = _lib.load()
    rc = lib.fastembedr_hip_structure_metrics(C.c_void_p(h.ctypes.data), h.shape[0], h.shape[1],
                                              C.c_void_p(lo.ctypes.data), lo.shape[1], C.c_void_p(ks.ctypes.data),
                                              ks.size, C.c_void_p(out.ctypes.data))
    _lib.check(rc, "HIP exact structure metrics")
    res = {name: out[:, j].copy() for j, name in enumerate(COLUMNS)}
    res["k"] = ks.copy()
    return res
