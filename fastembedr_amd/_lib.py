"""ctypes binding of the C ABI declared in include/fastembedr_hip.h.

The shared library is built in-tree by ``python -m fastembedr_amd.build``.
There is no fallback: if the library is missing or cannot be loaded, every
entry point raises ``HipBackendUnavailable``.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libfastembedr_hip.so"

# Every symbol declared in include/fastembedr_hip.h: (name, restype, argtypes).
_P = C.c_void_p
_I = C.c_int
_F = C.c_float
_IP = C.POINTER(C.c_int)
_FP = C.POINTER(C.c_float)
_DP = C.POINTER(C.c_double)
_LLP = C.POINTER(C.c_longlong)

_ONE_SHOT_ARGS = [_P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _F, _F, _F, _I, _F, _F, _F, _F, C.c_uint, _I, _P]

SIGNATURES = {
    "fastembedr_hip_embedding_last_error": (C.c_char_p, []),
    "fastembedr_hip_available": (C.c_bool, []),
    "fastembedr_hip_opentsne_fft_from_knn_float": (_I, _ONE_SHOT_ARGS),
    "fastembedr_hip_opentsne_fft_from_knn": (_I, _ONE_SHOT_ARGS),
    "fastembedr_hip_opentsne_fft_from_device_knn_float": (_I, _ONE_SHOT_ARGS),
    "fastembedr_hip_tsne_create": (_I, [_P, _P, _I, _I, _F, _I, _I, _I, C.POINTER(_P)]),
    "fastembedr_hip_tsne_destroy": (None, [_P]),
    "fastembedr_hip_tsne_p_nnz": (_I, [_P, _LLP]),
    "fastembedr_hip_tsne_copy_p": (_I, [_P, _P, _P, _P]),
    "fastembedr_hip_tsne_copy_conditional_p": (_I, [_P, _P]),
    "fastembedr_hip_tsne_grid_size": (_I, [_P, _IP]),
    "fastembedr_hip_tsne_set_state": (_I, [_P, _P, _P, _P]),
    "fastembedr_hip_tsne_get_state": (_I, [_P, _P, _P, _P]),
    "fastembedr_hip_tsne_gradient": (_I, [_P, _F, _I, _P]),
    "fastembedr_hip_tsne_center": (_I, [_P]),
    "fastembedr_hip_tsne_run": (_I, [_P, _I, _F, _F, _F, _F, _F]),
    "fastembedr_hip_tsne_sync": (_I, [_P]),
    "fastembedr_hip_tsne_kl": (_I, [_P, _DP]),
    "fastembedr_hip_tsne_kl_rows": (_I, [_P, _DP, _P]),
    "fastembedr_hip_tsne_set_repulsion": (_I, [_P, _I, _I, _I, _F]),
    "fastembedr_hip_tsne_interp_info": (_I, [_P, _IP, _IP, _IP, _FP, _DP]),
    "fastembedr_hip_tsne_attraction_info": (_I, [_P, _LLP, _IP]),
    "fastembedr_hip_tsne_graph_info": (_I, [_P, _LLP, _IP, _IP]),
    "fastembedr_hip_tsne_attraction_slots": (_I, [_P, _LLP]),
    "fastembedr_hip_tsne_set_timing": (_I, [_P, _I]),
    "fastembedr_hip_tsne_timing_stats": (_I, [_P, _I, _LLP, _DP]),
    "fastembedr_hip_tsne_kernel_name": (C.c_char_p, [_I]),
    "fastembedr_hip_tsne_kernel_count": (_I, []),
    "fastembedr_hip_tsne_p_build_ms": (_I, [_P, _DP]),
    "fastembedr_hip_random_init": (_I, [_I, C.c_uint, _P]),
    "fastembedr_hip_transform_tsne": (_I, [_P, _I, _P, _P, _I, _I, _P, _I, C.c_double, _I, _I, C.c_double,
                                           C.c_double, C.c_double, C.c_double, C.c_double, C.c_double,
                                           C.c_double, _I, _I, _I, _P, _IP]),
    "fastembedr_hip_transform_tsne_grid": (_I, [_P, _I, _P, _P, _I, _I, _P, _I, C.c_double, _I, _I, C.c_double,
                                                C.c_double, C.c_double, C.c_double, C.c_double, C.c_double,
                                                C.c_double, _I, _I, _I, C.c_double, _P, _LLP]),
    "fastembedr_hip_transform_grid_probe": (_I, [_P, _I, _P, _P, _I, _I, C.c_double, _P, _P, _I, C.c_double, _I,
                                                 _I, C.c_double, _P, _LLP]),
    "fastembedr_hip_transform_tsne_noalloc": (_I, [_P, _I, _P, _P, _I, _I, _P, _I, C.c_double, _I, _I, C.c_double,
                                                   C.c_double, C.c_double, C.c_double, C.c_double, C.c_double,
                                                   C.c_double, _I, _I, _I, _P, _IP]),
    "fastembedr_hip_transform_probe": (_I, [_P, _I, _P, _P, _I, _I, C.c_double, _P, C.c_double, _I, _I, _I, _I,
                                            _P, _P, _P]),
    "fastembedr_hip_knn_exact": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _LLP]),
    "fastembedr_hip_knn_query": (_I, [_P, _I, _P, _I, _I, _I, _I, _I, _P, _P, _I, _LLP]),
    "fastembedr_hip_knn_exact_metric": (_I, [_P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I, _LLP]),
    "fastembedr_hip_knn_query_metric": (_I, [_P, _I, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _LLP]),
    "fastembedr_hip_structure_metrics": (_I, [_P, _I, _I, _P, _I, _P, _I, _P]),
}

REPULSION_GRID = 0
REPULSION_EXACT = 1
REPULSION_LAGRANGE = 2
KNN_METRICS = {"euclidean": 0, "cosine": 1, "correlation": 2}  # FASTEMBEDR_HIP_KNN_*


class HipBackendUnavailable(RuntimeError):
    """Raised when the HIP library is missing, fails to load, or finds no gfx950 device."""


class HipBackendError(RuntimeError):
    """An entry point returned 1; the message is the library's last error."""


_lib = None


def load(path: Path | str | None = None) -> C.CDLL:
    """Loads the library once and attaches the declared signatures."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise HipBackendUnavailable(
            f"HIP backend library not found at {p}; build it with `python -m fastembedr_amd.build`. "
            "No CPU fallback is used for HIP-labelled runs."
        )
    try:
        lib = C.CDLL(str(p))
    except OSError as exc:  # pragma: no cover - depends on the host
        raise HipBackendUnavailable(f"cannot load {p}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    msg = load().fastembedr_hip_embedding_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise HipBackendError(f"{what} failed: {last_error()}")


def available() -> bool:
    try:
        return bool(load().fastembedr_hip_available())
    except HipBackendUnavailable:
        return False
