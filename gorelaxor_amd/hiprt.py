"""Device buffers and events over the HIP runtime libgrx.so links against.

Tests and the benchmark use these instead of torch: torch ships its own copy
of the HIP runtime, and a process that loads two copies gets two runtimes
that do not see each other's devices.  This module resolves
libamdhip64.so.7 after libgrx.so is loaded, so it is the very same runtime.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

_hip = None


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        _lib.lib()  # libgrx.so first: its libamdhip64.so.7 is the one reused below
        H = C.CDLL("libamdhip64.so.7")
        H.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        H.hipFree.argtypes = [C.c_void_p]
        H.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        H.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        H.hipDeviceSynchronize.argtypes = []
        H.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        H.hipEventDestroy.argtypes = [C.c_void_p]
        H.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        H.hipEventSynchronize.argtypes = [C.c_void_p]
        H.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        H.hipGetErrorString.restype = C.c_char_p
        H.hipGetErrorString.argtypes = [C.c_int]
        _hip = H
    return _hip


def _check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(rc).decode()}")


H2D, D2H, D2D = 1, 2, 3


class DeviceBuffer:
    """nbytes of device memory; data_ptr() for the C ABI's device pointers."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(hip().hipMalloc(C.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def data_ptr(self) -> int:
        return self.ptr

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check(hip().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        _check(hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def copy_from(self, other: "DeviceBuffer", nbytes: int | None = None) -> None:
        n = min(self.nbytes, other.nbytes) if nbytes is None else nbytes
        _check(hip().hipMemcpy(self.ptr, other.ptr, n, D2D), "hipMemcpy D2D")

    def zero(self) -> None:
        _check(hip().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def free(self) -> None:
        if self.ptr:
            _check(hip().hipFree(self.ptr), "hipFree")
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    """A HIP event recorded on a given stream (the library context's)."""

    def __init__(self):
        e = C.c_void_p()
        _check(hip().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.ev = e.value

    def record(self, stream: int) -> None:
        _check(hip().hipEventRecord(self.ev, stream), "hipEventRecord")

    def synchronize(self) -> None:
        _check(hip().hipEventSynchronize(self.ev), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        _check(hip().hipEventElapsedTime(C.byref(ms), self.ev, end.ev), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            hip().hipEventDestroy(self.ev)
        except Exception:
            pass


def mem_free() -> int:
    """Free device memory in bytes (hipMemGetInfo)."""
    free, total = C.c_size_t(), C.c_size_t()
    _check(hip().hipMemGetInfo(C.byref(free), C.byref(total)), "hipMemGetInfo")
    return free.value


def synchronize() -> None:
    _check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
