"""Minimal ctypes access to the HIP runtime that libmans_hip.so links.

Device buffers, streams and events for the device-pointer entry points of the
C ABI, without a second HIP runtime in the process (torch ships its own copy
of libamdhip64, and two copies in one process do not share the device).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import lib

_hip = None

H2D, D2H, D2D = 1, 2, 3


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        lib()  # loads libamdhip64.so.7 as a dependency first, so this resolves to it
        H = C.CDLL("libamdhip64.so.7")
        H.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        H.hipFree.argtypes = [C.c_void_p]
        H.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        H.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        H.hipDeviceSynchronize.argtypes = []
        H.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        H.hipStreamDestroy.argtypes = [C.c_void_p]
        H.hipStreamSynchronize.argtypes = [C.c_void_p]
        H.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        H.hipEventDestroy.argtypes = [C.c_void_p]
        H.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        H.hipEventSynchronize.argtypes = [C.c_void_p]
        H.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        H.hipSetDevice.argtypes = [C.c_int]
        _hip = H
    return _hip


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed with hipError {rc}")


class DeviceArray:
    """A device allocation with numpy-shaped upload/download."""

    def __init__(self, shape, dtype):
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        _ok(hip().hipMalloc(C.byref(p), max(self.nbytes, 256)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            _ok(hip().hipMemcpy(d.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            _ok(hip().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def offset(self, elements: int) -> int:
        return self.ptr + elements * self.dtype.itemsize

    def copy_from(self, other: "DeviceArray") -> None:
        """Device-to-device copy of min(nbytes) bytes (a plain copy kernel)."""
        _ok(hip().hipMemcpy(self.ptr, other.ptr, min(self.nbytes, other.nbytes), D2D),
            "hipMemcpy D2D")

    def free(self) -> None:
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = C.c_void_p()
        _ok(hip().hipStreamCreate(C.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self) -> None:
        _ok(hip().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            hip().hipStreamDestroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        e = C.c_void_p()
        _ok(hip().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream | None = None) -> None:
        _ok(hip().hipEventRecord(self.handle, stream.handle if stream else None), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        _ok(hip().hipEventSynchronize(end.handle), "hipEventSynchronize")
        ms = C.c_float()
        _ok(hip().hipEventElapsedTime(C.byref(ms), self.handle, end.handle), "hipEventElapsedTime")
        return ms.value


def synchronize() -> None:
    _ok(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
