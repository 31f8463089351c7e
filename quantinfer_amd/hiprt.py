"""Minimal ctypes plumbing over the HIP runtime that libqi_hip.so links
(device buffers, streams, events) for Python callers such as tests and
bench.py. It binds the libamdhip64.so.7 already loaded by libqi_hip.so, so
both share one runtime.

(PyTorch wheels bundle their own libamdhip64; a process that uses torch's
GPU support together with libqi_hip.so must import torch before loading
libqi_hip.so so that the library binds torch's already-loaded runtime.)
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import lib as _qi_lib

_hip = None


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _qi_lib()  # loads libamdhip64.so.7 as a dependency first
        h = ctypes.CDLL("libamdhip64.so.7")
        vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        h.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        h.hipFree.argtypes = [vp]
        h.hipMemcpy.argtypes = [vp, vp, sz, i32]
        h.hipMemcpyAsync.argtypes = [vp, vp, sz, i32, vp]
        h.hipMemset.argtypes = [vp, i32, sz]
        h.hipDeviceSynchronize.argtypes = []
        h.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
        h.hipStreamDestroy.argtypes = [vp]
        h.hipStreamSynchronize.argtypes = [vp]
        h.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        h.hipEventDestroy.argtypes = [vp]
        h.hipEventRecord.argtypes = [vp, vp]
        h.hipEventSynchronize.argtypes = [vp]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        h.hipGetErrorString.argtypes = [i32]
        h.hipGetErrorString.restype = ctypes.c_char_p
        _hip = h
    return _hip


H2D, D2H, D2D = 1, 2, 3


def _ok(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(err).decode()}")


class DeviceBuffer:
    def __init__(self, nbytes: int):
        p = ctypes.c_void_p()
        _ok(hip().hipMalloc(ctypes.byref(p), max(nbytes, 1)), "hipMalloc")
        self.ptr = p.value
        self.nbytes = nbytes

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        _ok(hip().hipMemcpy(b.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return b

    def to_array(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _ok(hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self) -> None:
        _ok(hip().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def copy_from(self, src: "DeviceBuffer", nbytes: int, stream: "Stream") -> None:
        """Device-to-device copy on `stream` (the HIP runtime's copy kernel)."""
        _ok(hip().hipMemcpyAsync(self.ptr, src.ptr, nbytes, D2D, stream.handle), "hipMemcpyAsync D2D")

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
        s = ctypes.c_void_p()
        _ok(hip().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self) -> None:
        _ok(hip().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            hip().hipStreamDestroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        _ok(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream) -> None:
        _ok(hip().hipEventRecord(self.handle, stream.handle), "hipEventRecord")

    def elapsed_ms(self, later: "Event") -> float:
        _ok(hip().hipEventSynchronize(later.handle), "hipEventSynchronize")
        ms = ctypes.c_float()
        _ok(hip().hipEventElapsedTime(ctypes.byref(ms), self.handle, later.handle),
            "hipEventElapsedTime")
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            hip().hipEventDestroy(self.handle)
            self.handle = None


def synchronize() -> None:
    _ok(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
