"""Device buffers owned through the HIP runtime that the backend library links.

The torch wheel in this image bundles its own HIP runtime; a second runtime
in the process must not share device pointers with the library's.  Buffers
that the library reads or writes in place (device-resident KNN results,
device input matrices) are therefore allocated here, with the library's own
runtime (the ``libamdhip64.so.7`` that ``libfastembedr_hip.so`` already
loaded), and freed when the Python object is collected.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

_H2D, _D2H = 1, 2
_hip = None


def _runtime() -> C.CDLL:
    global _hip
    if _hip is None:
        _lib.load()  # the library's runtime is loaded first; this opens the same one
        hip = C.CDLL("libamdhip64.so.7")
        hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        hip.hipMalloc.restype = C.c_int
        hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        hip.hipMemcpy.restype = C.c_int
        hip.hipFree.argtypes = [C.c_void_p]
        hip.hipFree.restype = C.c_int
        _hip = hip
    return _hip


class DeviceBuffer:
    """A C-order device array of ``shape`` and ``dtype`` (owned, freed on
    ``free()`` or collection)."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self._ptr = C.c_void_p()
        hip = _runtime()
        rc = hip.hipMalloc(C.byref(self._ptr), max(self.nbytes, 1))
        if rc != 0:
            raise _lib.HipBackendError(f"hipMalloc({self.nbytes} bytes) failed with HIP error {rc}")

    @classmethod
    def from_host(cls, host: np.ndarray) -> "DeviceBuffer":
        host = np.ascontiguousarray(host)
        buf = cls(host.shape, host.dtype)
        if buf.nbytes:
            rc = _runtime().hipMemcpy(buf._ptr, C.c_void_p(host.ctypes.data), buf.nbytes, _H2D)
            if rc != 0:
                raise _lib.HipBackendError(f"hipMemcpy (host to device) failed with HIP error {rc}")
        return buf

    @property
    def address(self) -> int:
        if not self._ptr:
            raise _lib.HipBackendError("device buffer already freed")
        return int(self._ptr.value)

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            rc = _runtime().hipMemcpy(C.c_void_p(out.ctypes.data), C.c_void_p(self.address), self.nbytes, _D2H)
            if rc != 0:
                raise _lib.HipBackendError(f"hipMemcpy (device to host) failed with HIP error {rc}")
        return out

    def free(self) -> None:
        if self._ptr:
            _runtime().hipFree(self._ptr)
            self._ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:  # pragma: no cover - interpreter shutdown
            pass


class DeviceMatrix(DeviceBuffer):
    """An (n, d) float32 matrix on the device, row-major (C order) or, with
    ``col_major``, column-major: the layouts the exact KNN entry reads."""

    def __init__(self, n: int, d: int, col_major: bool = False):
        super().__init__((d, n) if col_major else (n, d), np.float32)
        self.n, self.d, self.col_major = int(n), int(d), bool(col_major)

    @classmethod
    def from_host(cls, x: np.ndarray, col_major: bool = False) -> "DeviceMatrix":
        x = np.asarray(x, dtype=np.float32)
        if x.ndim != 2:
            raise ValueError("a device matrix must be two-dimensional")
        m = cls(x.shape[0], x.shape[1], col_major)
        host = np.ascontiguousarray(x.T if col_major else x)
        if m.nbytes:
            rc = _runtime().hipMemcpy(m._ptr, C.c_void_p(host.ctypes.data), m.nbytes, _H2D)
            if rc != 0:
                raise _lib.HipBackendError(f"hipMemcpy (host to device) failed with HIP error {rc}")
        return m
