"""Parameterised attention calls for the parity tests (seeded, small enough for the oracle)."""

from __future__ import annotations

import math

import numpy as np

from supra_attn import _lib
from supra_attn.workloads import Call


def make_call(B=1, H=2, D=64, Lq=64, Lk=64, *, seed=0, scale=None, packed=False, pad_cols=0, q_off=0,
              o_off=0, ldo_pad=0, bias_mode=_lib.SA_BIAS_NONE, mask_mode=_lib.SA_MASK_NONE, key_len=None,
              key_mask_p=0.7, num_buckets=32, max_distance=128, bias_std=0.5, dense_bias_batched=False,
              name=None) -> Call:
    """A call with q/k/v either packed in one buffer (the DiT layout) or separate, optional
    extra columns per row (pad_cols), offsets, and any bias/mask mode."""
    from oracle import t5_bucket  # the LUT is checked separately; tests use the oracle's LUT here

    rng = np.random.default_rng(seed)
    hd = H * D
    if packed:
        ld = 3 * hd + pad_cols
        buf = rng.standard_normal(q_off + B * max(Lq, Lk) * ld, dtype=np.float32)
        q = k = v = buf
        args = dict(q_off=q_off, k_off=q_off + hd, v_off=q_off + 2 * hd, ldq=ld, ldk=ld, ldv=ld,
                    sq=max(Lq, Lk) * ld, sk=max(Lq, Lk) * ld, sv=max(Lq, Lk) * ld)
    else:
        ld = hd + pad_cols
        q = rng.standard_normal(q_off + B * Lq * ld, dtype=np.float32)
        k = rng.standard_normal(B * Lk * ld, dtype=np.float32)
        v = rng.standard_normal(B * Lk * ld, dtype=np.float32)
        args = dict(q_off=q_off, ldq=ld, ldk=ld, ldv=ld, sq=Lq * ld, sk=Lk * ld, sv=Lk * ld)
    ldo = hd + ldo_pad
    args.update(o_off=o_off, ldo=ldo, so=Lq * ldo)
    call = Call(name=name or f"B{B}H{H}D{D}q{Lq}k{Lk}", B=B, H=H, D=D, Lq=Lq, Lk=Lk, q=q, k=k, v=v,
                out_shape=(o_off + B * Lq * ldo,), args=args,
                scale=(1.0 / math.sqrt(D)) if scale is None else scale, same_qkv=packed)
    if bias_mode == _lib.SA_BIAS_DENSE:
        nb = B if dense_bias_batched else 1
        call.bias = (rng.standard_normal((nb, H, Lq, Lk), dtype=np.float32) * np.float32(bias_std))
        call.args["sbias"] = H * Lq * Lk if dense_bias_batched else 0
        call.bias_mode = bias_mode
    elif bias_mode == _lib.SA_BIAS_RELPOS:
        call.bias = rng.standard_normal((num_buckets, H), dtype=np.float32) * np.float32(bias_std)
        call.lut = t5_bucket.bucket_lut(Lq, Lk, True, num_buckets, max_distance)
        call.bias_mode = bias_mode
    if mask_mode == _lib.SA_MASK_KEY_LEN:
        call.key_len = (np.asarray(key_len, dtype=np.int32) if key_len is not None
                        else rng.integers(0, Lk + 1, size=B, dtype=np.int32))
        call.mask_mode = mask_mode
    elif mask_mode == _lib.SA_MASK_KEY_MASK:
        call.key_mask = (rng.random((B, Lk)) < key_mask_p).astype(np.uint8)
        call.args["smask"] = Lk
        call.mask_mode = mask_mode
    return call
