"""Device buffers and events through the HIP runtime the library links
(/opt/rocm/lib/libamdhip64.so.7), via ctypes.

PyTorch bundles a different HIP runtime build; loading both into one process
leaves one of them without devices, so GPU tests and the benchmark use this
module for device memory, copies and event timing instead of torch.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_RUNTIME = os.environ.get("FAH_HIP_RUNTIME", "/opt/rocm/lib/libamdhip64.so.7")
_hip = None

H2D, D2H, D2D = 1, 2, 3


def runtime() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        lib = ctypes.CDLL(_RUNTIME, mode=ctypes.RTLD_GLOBAL)
        vp = ctypes.c_void_p
        sig = {
            "hipMalloc": (ctypes.c_int, [ctypes.POINTER(vp), ctypes.c_size_t]),
            "hipFree": (ctypes.c_int, [vp]),
            "hipMemcpy": (ctypes.c_int, [vp, vp, ctypes.c_size_t, ctypes.c_int]),
            "hipMemset": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_size_t]),
            "hipDeviceSynchronize": (ctypes.c_int, []),
            "hipGetErrorString": (ctypes.c_char_p, [ctypes.c_int]),
            "hipEventCreate": (ctypes.c_int, [ctypes.POINTER(vp)]),
            "hipEventDestroy": (ctypes.c_int, [vp]),
            "hipEventRecord": (ctypes.c_int, [vp, vp]),
            "hipEventSynchronize": (ctypes.c_int, [vp]),
            "hipEventElapsedTime": (ctypes.c_int, [ctypes.POINTER(ctypes.c_float), vp, vp]),
            "hipStreamSynchronize": (ctypes.c_int, [vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _hip = lib
    return _hip


def _check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"{what}: {runtime().hipGetErrorString(rc).decode()}")


class DeviceArray:
    """A typed device allocation (hipMalloc) with numpy copies in and out."""

    def __init__(self, shape, dtype):
        self.shape = tuple(np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        _check(runtime().hipMalloc(ctypes.byref(p), max(self.nbytes, 16)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        _check(runtime().hipMemcpy(self.ptr, a.ctypes.data, self.nbytes, H2D), "hipMemcpy H2D")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _check(runtime().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def fill_zero(self):
        _check(runtime().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def free(self):
        if self.ptr:
            runtime().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        _check(runtime().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: int):
        _check(runtime().hipEventRecord(self.handle, stream), "hipEventRecord")

    def synchronize(self):
        _check(runtime().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _check(runtime().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                runtime().hipEventDestroy(self.handle)
        except Exception:
            pass


def synchronize():
    _check(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")
