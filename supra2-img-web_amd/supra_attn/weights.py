"""Safetensors weights into device memory: the Python mirror of app/weights.js over the C ABI of
include/supra_weights.h.

- `SafeTensors.open(path)` / `SafeTensors.from_bytes(buf)`: SafeTensors.open (weights.js:40-47);
  `has`, `info` (:56-64), `metadata`.
- `st.resident(dev)`: the file's whole data section in device memory, copied once (bulk DMA
  through pinned staging); every decode below reads from it.
- `st.f32(dev, name)`: toF32 (:28-37, :66-70) on the device, into a new float32 buffer.
- `st.rows(dev, name, ids)`: rows (:73-83), the embedding gather, on the device.
- `upload_vector`, `upload_linear`, `upload_conv3`: uploadVector / uploadLinear / uploadConv3
  (:85-118), returning device buffers ({"kind": "f32", "N", "K", "buf", "bias"} for the layers).

The reference decodes on the CPU and returns Float32Arrays; here results stay on the device (read
them back with `Buffer.read()`).
"""

from __future__ import annotations

import ctypes
from ctypes import c_void_p

import numpy as np

from . import _lib
from .device import Buffer, Device

DTYPE_NAMES = {v: k for k, v in _lib.SA_DT.items()}


class PinnedBuffer:
    """Pinned host memory (hipHostMalloc) for staged uploads."""

    def __init__(self, nbytes: int):
        ptr = c_void_p()
        _lib.check(_lib.load().sa_malloc_host(ctypes.byref(ptr), nbytes))
        self.ptr = ptr.value
        self.nbytes = nbytes

    def release(self) -> None:
        if self.ptr:
            _lib.check(_lib.load().sa_free_host(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr:
                _lib.load().sa_free_host(self.ptr)
        except Exception:
            pass


class SafeTensors:
    """An opened safetensors file (or in-memory buffer): header on the host, data section copied to a
    device on first use."""

    def __init__(self, handle: int, keepalive=None):
        self._h = handle
        self._keep = keepalive
        self._resident: dict[int, Buffer] = {}

    @classmethod
    def open(cls, path: str) -> "SafeTensors":
        h = c_void_p()
        _lib.check(_lib.load().sa_st_open(str(path).encode(), ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def from_bytes(cls, buf) -> "SafeTensors":
        arr = np.frombuffer(buf, dtype=np.uint8)
        h = c_void_p()
        _lib.check(_lib.load().sa_st_open_memory(arr.ctypes.data, arr.size, ctypes.byref(h)))
        return cls(h.value, keepalive=arr)

    def close(self) -> None:
        for b in self._resident.values():
            b.release()
        self._resident.clear()
        if self._h:
            _lib.load().sa_st_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            if self._h:
                _lib.load().sa_st_close(self._h)
        except Exception:
            pass

    # ---- header (host only) ----
    def names(self) -> list[str]:
        lib = _lib.load()
        return [lib.sa_st_name(self._h, i).decode() for i in range(lib.sa_st_count(self._h))]

    def has(self, name: str) -> bool:
        t = _lib.StTensor()
        return _lib.load().sa_st_info(self._h, name.encode(), ctypes.byref(t)) == _lib.SA_OK

    def raw_info(self, name: str) -> _lib.StTensor:
        t = _lib.StTensor()
        _lib.check(_lib.load().sa_st_info(self._h, name.encode(), ctypes.byref(t)))
        return t

    def info(self, name: str) -> dict:
        """The header entry, as app/weights.js:60-64 returns it."""
        t = self.raw_info(name)
        return {"dtype": t.dtype_name.decode(), "shape": [int(t.shape[i]) for i in range(t.ndim)],
                "data_offsets": [int(t.begin), int(t.end)]}

    @property
    def metadata(self) -> dict:
        lib = _lib.load()
        keys = [lib.sa_st_metadata_key(self._h, i).decode() for i in range(lib.sa_st_metadata_count(self._h))]
        return {k: lib.sa_st_metadata_value(self._h, k.encode()).decode() for k in keys}

    @property
    def data_bytes(self) -> int:
        return int(_lib.load().sa_st_data_bytes(self._h))

    # ---- device side ----
    def resident(self, dev: Device, staging: PinnedBuffer | None = None, staging_bytes: int = 64 << 20) -> Buffer:
        """The data section in device memory (copied on the first call for `dev`)."""
        key = id(dev)
        if key not in self._resident:
            n = self.data_bytes
            buf = dev.empty([max(n, 1)], np.uint8)
            own = None
            if staging is None and n > 0:
                own = staging = PinnedBuffer(max(2 << 20, min(staging_bytes, 2 * n)))
            try:
                _lib.check(_lib.load().sa_st_upload(self._h, 0, n, buf.ptr, staging.ptr if staging else None,
                                                    staging.nbytes if staging else 0, dev.stream))
            finally:
                if own is not None:
                    own.release()
            self._resident[key] = buf
        return self._resident[key]

    def _src(self, dev: Device, t: _lib.StTensor) -> int:
        return self.resident(dev).ptr + int(t.begin)

    def f32(self, dev: Device, name: str, out: Buffer | None = None, out_offset: int = 0) -> Buffer:
        """toF32 of tensor `name` into a new float32 buffer shaped like it (or into `out` at element
        `out_offset`)."""
        t = self.raw_info(name)
        shape = [int(t.shape[i]) for i in range(t.ndim)] or [1]
        if out is None:
            out = dev.empty(shape, np.float32)
        elif out_offset + int(t.numel) > out.size:
            raise ValueError(f"{name}: {t.numel} elements do not fit at offset {out_offset} of {out.size}")
        _lib.check(_lib.load().sa_to_f32(self._src(dev, t), t.dtype, t.numel, out.ptr + 4 * out_offset, dev.stream))
        return out

    def rows(self, dev: Device, name: str, ids) -> Buffer:
        """rows(): the rows `ids` of the 2-D table `name`, as a [len(ids), dim] float32 buffer."""
        t = self.raw_info(name)
        if t.ndim != 2:
            raise ValueError(f"{name} is not a 2-D table")
        ids_h = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        dim = int(t.shape[1])
        out = dev.empty([ids_h.size, dim], np.float32)
        if ids_h.size:
            ids_d = dev.from_array(ids_h)
            _lib.check(_lib.load().sa_rows_f32(self._src(dev, t), t.dtype, int(t.shape[0]), dim, ids_d.ptr, ids_h.size,
                                               out.ptr, dev.stream))
            dev.sync()
            ids_d.release()
        return out


def upload_vector(dev: Device, st: SafeTensors, name: str) -> Buffer:
    return st.f32(dev, name)


def upload_linear(dev: Device, st: SafeTensors, base: str) -> dict:
    """Linear layer "<base>weight" [N, K] (+ "<base>bias"), K the product of the trailing dims."""
    w = st.info(base + "weight")
    N = w["shape"][0]
    K = int(np.prod(w["shape"][1:], dtype=np.int64))
    bias = upload_vector(dev, st, base + "bias") if st.has(base + "bias") else None
    return {"kind": "f32", "N": N, "K": K, "buf": st.f32(dev, base + "weight"), "bias": bias}


def upload_conv3(dev: Device, st: SafeTensors, base: str, cin_pad: int = 0) -> dict:
    """3x3 conv "<base>weight" [cout, cin, 3, 3] -> [cout, 3, 3, cin_pad] float32 (+ bias)."""
    t = st.raw_info(base + "weight")
    if t.ndim != 4 or t.shape[2] != 3 or t.shape[3] != 3:
        raise ValueError(f"{base}: expected a 3x3 conv")
    cout, cin = int(t.shape[0]), int(t.shape[1])
    cp = cin_pad or cin
    out = dev.empty([cout, 3, 3, cp], np.float32)
    _lib.check(_lib.load().sa_conv3_pack_f32(st._src(dev, t), t.dtype, cout, cin, cp, out.ptr, dev.stream))
    bias = upload_vector(dev, st, base + "bias") if st.has(base + "bias") else None
    return {"kind": "f32", "N": cout, "K": 9 * cp, "buf": out, "bias": bias}
