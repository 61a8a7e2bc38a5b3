"""Minimal ctypes access to the HIP runtime that libchatnet_hip links.

Device buffers, copies and events for callers that hand device pointers to
chatnet_matmul (tests, bench).  It binds libamdhip64.so.7 after loading
libchatnet_hip.so, so both share one runtime instance; a second HIP runtime in
the same process (for example the one bundled with a torch wheel) cannot see
the device once the first has claimed it, so nothing here goes through torch.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native

H2D, D2H, D2D = 1, 2, 3
_rt = None


def rt() -> ctypes.CDLL:
    global _rt
    if _rt is None:
        _native.hip_lib()  # resolve the runtime through the product library first
        L = ctypes.CDLL("libamdhip64.so.7")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        sig = {
            "hipMalloc": [ctypes.POINTER(vp), sz],
            "hipFree": [vp],
            "hipMemcpy": [vp, vp, sz, ctypes.c_int],
            "hipMemset": [vp, ctypes.c_int, sz],
            "hipDeviceSynchronize": [],
            "hipGetDeviceCount": [ctypes.POINTER(ctypes.c_int)],
            "hipEventCreate": [ctypes.POINTER(vp)],
            "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
            "hipEventDestroy": [vp],
            "hipGetErrorString": [ctypes.c_int],
            "hipStreamCreate": [ctypes.POINTER(vp)],
            "hipStreamDestroy": [vp],
            "hipStreamSynchronize": [vp],
            "hipStreamBeginCapture": [vp, ctypes.c_int],
            "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
            "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, vp, sz],
            "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp],
            "hipGraphDestroy": [vp],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "hipGetErrorString" else ctypes.c_int
        _rt = L
    return _rt


def _ok(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what}: {rt().hipGetErrorString(err).decode()}")


def device_count() -> int:
    n = ctypes.c_int(0)
    err = rt().hipGetDeviceCount(ctypes.byref(n))
    return n.value if err == 0 else 0


def synchronize() -> None:
    _ok(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceBuffer:
    """An owned device allocation."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _ok(rt().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), f"hipMalloc({nbytes})")
        self.ptr = int(p.value)

    @classmethod
    def from_numpy(cls, arr: np.ndarray, pad: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        b = cls(a.nbytes + pad)
        if pad:
            _ok(rt().hipMemset(b.ptr, 0, b.nbytes), "hipMemset")
        _ok(rt().hipMemcpy(b.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return b

    def to_numpy(self, dtype, count: int, offset_bytes: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        _ok(rt().hipMemcpy(out.ctypes.data, self.ptr + offset_bytes, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def fill(self, byte: int) -> None:
        _ok(rt().hipMemset(self.ptr, byte, self.nbytes), "hipMemset")

    def copy_from(self, src: "DeviceBuffer", nbytes: int, dst_offset: int = 0, src_offset: int = 0) -> None:
        _ok(rt().hipMemcpy(self.ptr + dst_offset, src.ptr + src_offset, nbytes, D2D), "hipMemcpy D2D")

    def free(self) -> None:
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A non-default stream (default priority)."""

    def __init__(self):
        s = ctypes.c_void_p()
        _ok(rt().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.h = s.value

    def synchronize(self) -> None:
        _ok(rt().hipStreamSynchronize(self.h), "hipStreamSynchronize")

    def __del__(self):
        try:
            rt().hipStreamDestroy(self.h)
        except Exception:
            pass


class Graph:
    """Captures the work issued on a stream by `fn()` into a replayable graph."""

    def __init__(self, stream: Stream, fn):
        _ok(rt().hipStreamBeginCapture(stream.h, 0), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = ctypes.c_void_p()
            _ok(rt().hipStreamEndCapture(stream.h, ctypes.byref(g)), "hipStreamEndCapture")
        e = ctypes.c_void_p()
        _ok(rt().hipGraphInstantiate(ctypes.byref(e), g, None, None, 0), "hipGraphInstantiate")
        rt().hipGraphDestroy(g)
        self.exec = e.value
        self.stream = stream

    def launch(self) -> None:
        _ok(rt().hipGraphLaunch(self.exec, self.stream.h), "hipGraphLaunch")

    def __del__(self):
        try:
            rt().hipGraphExecDestroy(self.exec)
        except Exception:
            pass


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        _ok(rt().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.h = e.value

    def record(self, stream: int = 0) -> None:
        _ok(rt().hipEventRecord(self.h, stream or None), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        _ok(rt().hipEventSynchronize(end.h), "hipEventSynchronize")
        ms = ctypes.c_float()
        _ok(rt().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            rt().hipEventDestroy(self.h)
        except Exception:
            pass
