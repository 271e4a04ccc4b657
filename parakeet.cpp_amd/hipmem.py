"""Device buffers for callers that hand the decoder HBM-resident inputs.

Binds hipMalloc / hipMemcpy / hipFree / hipDeviceSynchronize from the same
libamdhip64 that libparakeet_hip.so links, so pointers stay within one HIP
runtime instance.
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np

_hip = None
H2D, D2H, D2D = 1, 2, 3


def hip():
    global _hip
    if _hip is None:
        L = C.CDLL("libamdhip64.so.7")
        L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        L.hipFree.argtypes = [C.c_void_p]
        L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        L.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        L.hipGetErrorString.restype = C.c_char_p
        _hip = L
    return _hip


def _check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(rc).decode()}")


class DeviceArray:
    def __init__(self, nbytes: int):
        self.nbytes = max(int(nbytes), 1)
        p = C.c_void_p()
        _check(hip().hipMalloc(C.byref(p), self.nbytes), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray):
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        _check(hip().hipMemcpy(d.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return d

    def to_numpy(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        _check(hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        _check(hip().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        # No HIP call while the interpreter shuts down: the runtime (and a
        # profiler's preloaded library) may already be torn down by then.
        # Callers free their buffers explicitly; a buffer left to the garbage
        # collector at exit is reclaimed with the process.
        if sys.is_finalizing():
            return
        try:
            self.free()
        except Exception:
            pass


def synchronize():
    _check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
