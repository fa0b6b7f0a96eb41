"""Device memory, streams and events over the C-ABI plumbing entry points.

Host data is numpy; a :class:`DeviceBuffer` is a typed view of one device
allocation.  Nothing here computes: it only moves bytes for the kernels.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import call


class DeviceBuffer:
    """One device allocation with a numpy dtype and shape."""

    def __init__(self, shape, dtype, *, zero: bool = False):
        _lib.init()
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        call("ouro_malloc", C.byref(p), max(self.nbytes, 16))
        self._ptr = p.value
        if zero:
            self.zero()

    @classmethod
    def from_host(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.shape, arr.dtype)
        buf.upload(arr)
        return buf

    @property
    def ptr(self) -> int:
        if self._ptr is None:
            raise ValueError("DeviceBuffer already freed")
        return self._ptr

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"upload of {arr.nbytes} B into {self.nbytes} B buffer")
        call("ouro_memcpy_htod", self.ptr, arr.ctypes.data, self.nbytes)

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        call("ouro_memcpy_dtoh", out.ctypes.data, self.ptr, self.nbytes)
        return out

    def zero(self, stream=None) -> None:
        call("ouro_memset", self.ptr, 0, self.nbytes, stream)

    def free(self) -> None:
        if self._ptr is not None:
            call("ouro_free", self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            if getattr(self, "_ptr", None) is not None and _lib._LIB is not None:
                _lib.lib().ouro_free(self._ptr)
                self._ptr = None
        except Exception:
            pass


def synchronize(stream=None) -> None:
    call("ouro_stream_synchronize", stream)


class Stream:
    def __init__(self):
        _lib.init()
        p = C.c_void_p()
        call("ouro_stream_create", C.byref(p))
        self.handle = p.value

    def synchronize(self) -> None:
        call("ouro_stream_synchronize", self.handle)

    def __del__(self):
        try:
            if self.handle is not None and _lib._LIB is not None:
                _lib.lib().ouro_stream_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Event:
    """HIP event recorded on a given stream (the stream the kernels run on)."""

    def __init__(self):
        _lib.init()
        p = C.c_void_p()
        call("ouro_event_create", C.byref(p))
        self.handle = p.value

    def record(self, stream=None) -> None:
        call("ouro_event_record", self.handle, stream)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        call("ouro_event_elapsed_ms", C.byref(ms), self.handle, end.handle)
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle is not None and _lib._LIB is not None:
                _lib.lib().ouro_event_destroy(self.handle)
                self.handle = None
        except Exception:
            pass
