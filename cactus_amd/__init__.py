"""cactus_amd -- MI355X (gfx950) kernel layer for Cactus's quantized graph ops.

The hot path lives in native code: HIP kernels behind the C ABI of
include/cactus_hip.h (libcactus_hip.so) and the C++ graph/engine layer of
include/cactus_engine.h (libcactus_engine.so).  This package only loads
those libraries and moves numpy arrays in and out of device memory.
"""
from __future__ import annotations

import ctypes

import numpy as np

from ._native import NativeError, check, engine, hip

__all__ = ["NativeError", "check", "hip", "engine", "DeviceBuffer", "call", "device_count",
           "Stream", "Event"]


def call(name: str, *args) -> None:
    """Call a C-ABI entry point and raise NativeError on a non-zero status."""
    lib = hip()
    check(getattr(lib, name)(*args), lib)


def device_count() -> int:
    n = ctypes.c_int(0)
    check(hip().cactus_hip_device_count(ctypes.byref(n)))
    return n.value


class DeviceBuffer:
    """Owning handle of one device allocation."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        call("cactus_hip_malloc", ctypes.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, arr: np.ndarray, stream=None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        if arr.nbytes:
            call("cactus_hip_memcpy_h2d", buf.ptr, arr.ctypes.data, arr.nbytes, stream)
        return buf

    def upload(self, arr: np.ndarray, stream=None) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        if arr.nbytes:
            call("cactus_hip_memcpy_h2d", self.ptr, arr.ctypes.data, arr.nbytes, stream)

    def to_numpy(self, dtype, shape, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        if out.nbytes:
            call("cactus_hip_memcpy_d2h", out.ctypes.data, self.ptr, out.nbytes, stream)
        return out

    def free(self) -> None:
        if self.ptr:
            hip().cactus_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        call("cactus_hip_stream_create", ctypes.byref(p))
        self.handle = p.value

    def sync(self) -> None:
        call("cactus_hip_stream_sync", self.handle)

    def __del__(self):
        try:
            if self.handle:
                hip().cactus_hip_stream_destroy(self.handle)
        except Exception:
            pass


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        call("cactus_hip_event_create", ctypes.byref(p))
        self.handle = p.value

    def record(self, stream=None) -> None:
        call("cactus_hip_event_record", self.handle,
             stream.handle if isinstance(stream, Stream) else stream)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        call("cactus_hip_event_elapsed_ms", self.handle, end.handle, ctypes.byref(ms))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                hip().cactus_hip_event_destroy(self.handle)
        except Exception:
            pass
