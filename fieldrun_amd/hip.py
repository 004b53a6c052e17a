"""Minimal HIP runtime access (device buffers, events) through ctypes.

Uses the HIP runtime libfrq.so itself is linked against (resolved by its
SONAME after libfrq.so is loaded), so buffers, streams and events are the
library's own.  Used by bench.py for inputs resident in HBM and for event
timing on the stream the kernels run on.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import lib as _frq  # noqa: F401  (loads libfrq.so and its runtime first)

_hip = C.CDLL("libamdhip64.so.7")
_P, _S = C.c_void_p, C.c_size_t
for _name, _res, _args in [
    ("hipMalloc", C.c_int, [C.POINTER(C.c_void_p), _S]),
    ("hipFree", C.c_int, [_P]),
    ("hipMemcpy", C.c_int, [_P, _P, _S, C.c_int]),
    ("hipMemset", C.c_int, [_P, C.c_int, _S]),
    ("hipDeviceSynchronize", C.c_int, []),
    ("hipStreamSynchronize", C.c_int, [_P]),
    ("hipEventCreate", C.c_int, [C.POINTER(C.c_void_p)]),
    ("hipEventDestroy", C.c_int, [_P]),
    ("hipEventRecord", C.c_int, [_P, _P]),
    ("hipEventSynchronize", C.c_int, [_P]),
    ("hipEventElapsedTime", C.c_int, [C.POINTER(C.c_float), _P, _P]),
    ("hipGetErrorString", C.c_char_p, [C.c_int]),
    ("hipMemGetInfo", C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
]:
    _f = getattr(_hip, _name)
    _f.restype = _res
    _f.argtypes = _args

H2D, D2H, D2D = 1, 2, 3


def _chk(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"{what}: {_hip.hipGetErrorString(rc).decode()}")


class DeviceArray:
    """A device allocation holding a C-contiguous array of a fixed dtype."""

    def __init__(self, shape, dtype):
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        _chk(_hip.hipMalloc(C.byref(p), max(self.nbytes, 256)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            _chk(_hip.hipMemcpy(d.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            _chk(_hip.hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        _chk(_hip.hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def free(self):
        if self.ptr:
            _hip.hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        p = C.c_void_p()
        _chk(_hip.hipEventCreate(C.byref(p)), "hipEventCreate")
        self.h = p.value

    def record(self, stream):
        _chk(_hip.hipEventRecord(self.h, stream), "hipEventRecord")

    def synchronize(self):
        _chk(_hip.hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        _chk(_hip.hipEventElapsedTime(C.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            _hip.hipEventDestroy(self.h)
        except Exception:
            pass


def synchronize():
    _chk(_hip.hipDeviceSynchronize(), "hipDeviceSynchronize")


def copy_d2d(dst: int, src: int, nbytes: int):
    """Device-to-device copy (the runtime's blit kernel), synchronous."""
    _chk(_hip.hipMemcpy(dst, src, nbytes, D2D), "hipMemcpy D2D")


def mem_info():
    """(free, total) bytes of the current device."""
    f, t = C.c_size_t(), C.c_size_t()
    _chk(_hip.hipMemGetInfo(C.byref(f), C.byref(t)), "hipMemGetInfo")
    return f.value, t.value
