"""Stage a workload `Call` on the device and run it through sa_attention_f32."""

from __future__ import annotations

import numpy as np

from . import _lib
from .device import Device
from .workloads import Call


class Staged:
    """Device-resident buffers of one call plus its ready-to-launch sa_attn_args.

    With per-sequence key lengths, the host copy of the lengths goes along too (key_len_host), so
    the library schedules the sequences (balanced by key blocks), as the DiT caller does; host_key_len=False
    leaves it out (the launch-order schedule)."""

    def __init__(self, dev: Device, call: Call, out_fill: float | None = None, host_key_len: bool = True):
        self.dev = dev
        self.call = call
        self.bufs = []
        self.key_len_host = None
        q = self._put(call.q)
        k = q if call.same_qkv else self._put(call.k)
        v = q if call.same_qkv else (k if call.v is call.k else self._put(call.v))
        self.out = dev.empty(call.out_shape)
        self.bufs.append(self.out)
        if out_fill is not None:
            self.out.upload(np.full(call.out_shape, out_fill, dtype=np.float32))
        a = dict(call.args)
        kw = dict(B=call.B, H=call.H, D=call.D, Lq=call.Lq, Lk=call.Lk, q=q.ptr, k=k.ptr, v=v.ptr,
                  o=self.out.ptr, scale=call.scale, bias_mode=call.bias_mode, mask_mode=call.mask_mode)
        kw.update(a)
        if call.bias is not None:
            kw["bias"] = self._put(call.bias).ptr
        if call.lut is not None:
            kw["bucket_lut"] = self._put(np.asarray(call.lut, dtype=np.int32)).ptr
            kw["num_buckets"] = int(call.bias.shape[0])
        if call.key_len is not None:
            kl = np.ascontiguousarray(call.key_len, dtype=np.int32)
            kw["key_len"] = self._put(kl).ptr
            if host_key_len:
                self.key_len_host = kl  # kept alive: the library reads it during each call
                kw["key_len_host"] = kl.ctypes.data
        if call.key_mask is not None:
            km = np.asarray(call.key_mask, dtype=np.uint8)
            kw["key_mask"] = self._put(km).ptr
            kw.setdefault("smask", km.shape[-1])
        self.args = _lib.AttnArgs(**kw)
        ws_bytes = _lib.workspace_bytes(self.args)
        if ws_bytes > 0:  # scratch for the calls that merge partial results (wide heads)
            ws = dev.empty(((ws_bytes + 3) // 4,))
            self.bufs.append(ws)
            self.args.workspace = ws.ptr
            self.args.workspace_bytes = ws_bytes

    def _put(self, arr):
        buf = self.dev.from_array(np.ascontiguousarray(arr))
        self.bufs.append(buf)
        return buf

    def launch(self) -> None:
        self.dev.attention(self.args)

    def run(self) -> np.ndarray:
        self.launch()
        self.dev.sync()
        return self.out.read()

    @property
    def kernel(self) -> str:
        return _lib.kernel_name(self.args)

    def release(self) -> None:
        for b in self.bufs:
            b.release()
        self.bufs = []


class StagedLinear:
    """Device-resident buffers of one linear call plus its ready-to-launch sa_linear_args."""

    def __init__(self, dev: Device, call):
        self.dev = dev
        self.call = call
        self.bufs = []
        x = self._put(call.x)
        w = self._put(call.w)
        self.y = self._put(call.y0)
        kw = dict(M=call.M, N=call.N, K=call.K, x=x.ptr, x_off=call.x_off, ldx=call.ldx, w=w.ptr, ldw=call.ldw,
                  alpha=call.alpha, act=call.act, epilogue=call.epi, y=self.y.ptr, y_off=call.y_off, ldy=call.ldy,
                  gate_off=call.gate_off)
        if call.bias is not None:
            kw["bias"] = self._put(call.bias).ptr
        if call.gate is not None:
            kw["gate"] = self._put(call.gate).ptr
        self.args = _lib.LinearArgs(**kw)

    def _put(self, arr):
        buf = self.dev.from_array(np.ascontiguousarray(arr))
        self.bufs.append(buf)
        return buf

    def reset(self) -> None:
        """Restore the initial output (the residual epilogues accumulate into it)."""
        self.y.upload(self.call.y0)

    def launch(self) -> None:
        self.dev.linear(self.args)

    def run(self) -> np.ndarray:
        self.launch()
        self.dev.sync()
        return self.y.read()

    @property
    def kernel(self) -> str:
        return _lib.linear_kernel_name(self.args)

    def release(self) -> None:
        for b in self.bufs:
            b.release()
        self.bufs = []


class StagedVae:
    """Device-resident buffers of one VAE mid-block attention call, its workspace and args."""

    def __init__(self, dev: Device, call, in_place: bool = False):
        self.dev = dev
        self.call = call
        self.bufs = []
        put = self._put
        self.x = put(call.x)
        self.out = self.x if in_place else dev.empty(call.x.shape)
        if not in_place:
            self.bufs.append(self.out)
        kw = dict(HW=call.HW, C=call.C, groups=call.groups, eps=call.eps, x=self.x.ptr, gamma=put(call.gamma).ptr,
                  beta=put(call.beta).ptr, wqkv=put(call.wqkv).ptr, wo=put(call.wo).ptr, out=self.out.ptr)
        if call.bqkv is not None:
            kw["bqkv"] = put(call.bqkv).ptr
        if call.bo is not None:
            kw["bo"] = put(call.bo).ptr
        self.args = _lib.VaeAttnArgs(**kw)
        n = _lib.vae_workspace_bytes(self.args)
        ws = dev.empty(((n + 3) // 4,))
        self.bufs.append(ws)
        self.args.workspace = ws.ptr
        self.args.workspace_bytes = n

    def _put(self, arr):
        buf = self.dev.from_array(np.ascontiguousarray(arr))
        self.bufs.append(buf)
        return buf

    @property
    def kernel(self) -> str:
        return "groupnorm + linear + attention + linear"

    def reset(self) -> None:
        """Restore x (an in-place call overwrites it)."""
        self.x.upload(self.call.x)

    def launch(self) -> None:
        _lib.vae_attention(self.args, self.dev.stream)

    def run(self) -> np.ndarray:
        self.launch()
        self.dev.sync()
        return self.out.read()

    def release(self) -> None:
        for b in self.bufs:
            b.release()
        self.bufs = []
