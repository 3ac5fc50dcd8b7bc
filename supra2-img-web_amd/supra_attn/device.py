"""Device buffers, a stream and events over the C ABI helpers.

A small Python counterpart of the runtime pieces the operator's callers use in
app/gpu/device.js: `Tensor` (41-55: a device buffer plus a shape), `GPU.empty` / `fromArray`
(144-176), `read` (178-191) and `sync` (255-259). Data is numpy on the host.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_void_p

import numpy as np

from . import _lib


class Buffer:
    """One device allocation holding a numpy-typed array of `shape`."""

    def __init__(self, dev: "Device", shape, dtype=np.float32):
        self.dev = dev
        self.shape = tuple(int(s) for s in np.atleast_1d(np.asarray(shape, dtype=np.int64)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        ptr = c_void_p()
        _lib.check(_lib.load().sa_malloc(ctypes.byref(ptr), self.nbytes))
        self.ptr = ptr.value

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def upload(self, arr) -> "Buffer":
        a = np.ascontiguousarray(arr, dtype=self.dtype)
        if a.nbytes != self.nbytes:
            raise ValueError(f"upload of {a.nbytes} bytes into a {self.nbytes}-byte buffer")
        _lib.check(_lib.load().sa_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, self.dev.stream))
        return self

    def read(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _lib.check(_lib.load().sa_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes, self.dev.stream))
        return out

    def fill_bytes(self, value: int) -> "Buffer":
        _lib.check(_lib.load().sa_memset(self.ptr, value, self.nbytes, self.dev.stream))
        return self

    def release(self) -> None:
        if self.ptr:
            self.dev.sync()
            _lib.check(_lib.load().sa_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr:
                _lib.load().sa_free(self.ptr)
        except Exception:
            pass


class Event:
    def __init__(self):
        ev = c_void_p()
        _lib.check(_lib.load().sa_event_create(ctypes.byref(ev)))
        self.ev = ev.value

    def record(self, stream) -> None:
        _lib.check(_lib.load().sa_event_record(self.ev, stream))

    def elapsed_ms(self, stop: "Event") -> float:
        ms = c_float(0.0)
        _lib.check(_lib.load().sa_event_elapsed_ms(ctypes.byref(ms), self.ev, stop.ev))
        return float(ms.value)

    def __del__(self):
        try:
            _lib.load().sa_event_destroy(self.ev)
        except Exception:
            pass


class Device:
    """Device 0 (or `index`) with one non-blocking stream at the default priority."""

    def __init__(self, index: int = 0):
        lib = _lib.load()
        n = _lib.device_count()
        if n < 1:
            raise RuntimeError("no HIP device visible: " + lib.sa_last_error().decode())
        _lib.check(lib.sa_set_device(index))
        s = c_void_p()
        _lib.check(lib.sa_stream_create(ctypes.byref(s)))
        self.stream = s.value

    def empty(self, shape, dtype=np.float32) -> Buffer:
        return Buffer(self, shape, dtype)

    def from_array(self, arr, dtype=None) -> Buffer:
        a = np.asarray(arr)
        buf = Buffer(self, a.shape, dtype or a.dtype)
        return buf.upload(a)

    def sync(self) -> None:
        _lib.check(_lib.load().sa_stream_sync(self.stream))

    def attention(self, args: _lib.AttnArgs) -> None:
        _lib.attention(args, self.stream)

    def linear(self, args: _lib.LinearArgs) -> None:
        _lib.linear(args, self.stream)
