"""Minimal ctypes binding of the HIP runtime libswin2sr_hip.so links against.

Device buffers, copies, synchronisation and events for callers that hold
inputs in HBM (the throughput harness, the device-resident tests). It binds
the SAME libamdhip64 the library uses (/opt/rocm/lib), so buffers and streams
are shared with it directly; torch is not needed (and its bundled HIP runtime
is a different copy, which must not be mixed into this process).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
_hip = None

H2D, D2H, D2D = 1, 2, 3


def rt():
    global _hip
    if _hip is None:
        h = C.CDLL(os.path.join(_ROCM, "lib", "libamdhip64.so"), mode=C.RTLD_GLOBAL)
        vp, sz = C.c_void_p, C.c_size_t
        for name, args in {
            "hipMalloc": [C.POINTER(vp), sz], "hipFree": [vp],
            "hipMemcpy": [vp, vp, sz, C.c_int], "hipMemset": [vp, C.c_int, sz],
            "hipMemcpyAsync": [vp, vp, sz, C.c_int, vp],
            "hipDeviceSynchronize": [], "hipStreamSynchronize": [vp],
            "hipEventCreate": [C.POINTER(vp)], "hipEventDestroy": [vp],
            "hipEventRecord": [vp, vp], "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [C.POINTER(C.c_float), vp, vp],
            "hipGetErrorString": [C.c_int],
        }.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = C.c_char_p if name == "hipGetErrorString" else C.c_int
        _hip = h
    return _hip


def _chk(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed: {rt().hipGetErrorString(rc).decode()}")


class DeviceBuffer:
    """A hipMalloc'd float32 buffer of `n` elements."""

    def __init__(self, n: int):
        self.n = int(n)
        p = C.c_void_p()
        _chk(rt().hipMalloc(C.byref(p), max(self.n, 1) * 4), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = cls(a.size)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=np.float32)
        assert a.size <= self.n
        _chk(rt().hipMemcpy(C.c_void_p(self.ptr), a.ctypes.data_as(C.c_void_p), a.size * 4, H2D),
             "hipMemcpy H2D")

    def download(self, shape=None) -> np.ndarray:
        out = np.empty(self.n, np.float32)
        _chk(rt().hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr), self.n * 4, D2H),
             "hipMemcpy D2H")
        return out.reshape(shape) if shape is not None else out

    def free(self):
        if self.ptr:
            rt().hipFree(C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def copy_device(dst: int, src: int, nbytes: int):
    """Device-to-device hipMemcpy of `nbytes` (the runtime's plain copy kernel)."""
    _chk(rt().hipMemcpy(C.c_void_p(dst), C.c_void_p(src), nbytes, D2D), "hipMemcpy D2D")


def copy_device_async(dst: int, src: int, nbytes: int, stream: int = 0):
    """Device-to-device hipMemcpyAsync of `nbytes`, ordered on `stream`."""
    _chk(rt().hipMemcpyAsync(C.c_void_p(dst), C.c_void_p(src), nbytes, D2D, C.c_void_p(stream)),
         "hipMemcpyAsync D2D")


def synchronize():
    _chk(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")


def stream_synchronize(stream: int):
    _chk(rt().hipStreamSynchronize(C.c_void_p(stream)), "hipStreamSynchronize")


class Event:
    def __init__(self):
        e = C.c_void_p()
        _chk(rt().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.e = e.value

    def record(self, stream: int):
        _chk(rt().hipEventRecord(C.c_void_p(self.e), C.c_void_p(stream)), "hipEventRecord")

    def synchronize(self):
        _chk(rt().hipEventSynchronize(C.c_void_p(self.e)), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        _chk(rt().hipEventElapsedTime(C.byref(ms), C.c_void_p(self.e), C.c_void_p(end.e)),
             "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            rt().hipEventDestroy(C.c_void_p(self.e))
        except Exception:
            pass
