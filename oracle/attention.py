"""CPU oracle for the fused attention operator.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or, for the CPU baseline, as the thing timed on the
host). The product path never calls it.

Two restatements of the operator's semantics:

1. `attention_fp64`: brute force in float64 NumPy, the ground truth of the closed-form checks.
2. `attention_torch_fp32`: the PyTorch fp32 CPU path the parity bar is defined against:
   - no bias: F.scaled_dot_product_attention with a boolean key mask (True = attend), the
     formulation of tools/reference.py:72-79 (q.view(B, N, H, -1).transpose(1, 2), output
     transpose(1, 2).reshape(B, N, C)) and of its padded cross-attention, tools/reference.py:159-171;
   - with a bias: HF T5 eager attention (transformers modeling_t5.py:144-172): matmul(q, k^T) *
     scaling + position_bias + additive mask (0 / finfo(float32).min), softmax, matmul with v.

Semantics shared by both (the operator contract of app/gpu/ops.js:103-149 plus the mask/bias
extension):
  element (b, h, i, d) of Q is q[q_off + b*sq + i*ldq + h*D + d] (likewise K, V, O), the score is
  scale * (Q K^T) + bias, keys outside the mask are excluded, and a query row with no attended key
  yields zeros. (SDPA's convention; HF's additive finfo.min would give mean(V) there instead, and
  the WGSL kernel of app/gpu/kernels.js:193 NaN.)

Bias layouts: dense [H, Lq, Lk] (app/models/t5.js:55-65, added as in app/gpu/kernels.js:34), or the
relative-position form table[bucket(j - i), h] expanded by `dense_relpos_bias`.
"""

from __future__ import annotations

import numpy as np


def heads(buf: np.ndarray, *, B: int, L: int, H: int, D: int, off: int = 0, ld: int, sb: int = 0) -> np.ndarray:
    """Gather the strided view [B, H, L, D] of a flat buffer (the ops.js addressing with batch
    strides): element (b, h, i, d) = buf[off + b*sb + i*ld + h*D + d]."""
    flat = np.asarray(buf).reshape(-1)
    b = np.arange(B)[:, None, None, None]
    h = np.arange(H)[None, :, None, None]
    i = np.arange(L)[None, None, :, None]
    d = np.arange(D)[None, None, None, :]
    return flat[off + b * sb + i * ld + h * D + d]


def place(out_buf: np.ndarray, O: np.ndarray, *, off: int = 0, ld: int, sb: int = 0) -> np.ndarray:
    """Scatter O [B, Lq, H, D] into a copy of the flat output buffer with the same addressing."""
    res = np.array(out_buf, copy=True).reshape(-1)
    B, Lq, H, D = O.shape
    b = np.arange(B)[:, None, None, None]
    i = np.arange(Lq)[None, :, None, None]
    h = np.arange(H)[None, None, :, None]
    d = np.arange(D)[None, None, None, :]
    res[off + b * sb + i * ld + h * D + d] = O
    return res.reshape(np.shape(out_buf))


def key_valid(B: int, Lk: int, key_len=None, key_mask=None) -> np.ndarray | None:
    """Boolean [B, Lk] of attended keys (None = all). key_len: keys j < key_len[b] attend;
    key_mask: nonzero attends (tools/reference.py:78 passes mask.bool())."""
    if key_len is None and key_mask is None:
        return None
    valid = np.ones((B, Lk), dtype=bool)
    if key_len is not None:
        kl = np.clip(np.asarray(key_len, dtype=np.int64).reshape(B), 0, Lk)
        valid &= np.arange(Lk)[None, :] < kl[:, None]
    if key_mask is not None:
        valid &= np.asarray(key_mask).reshape(B, -1)[:, :Lk] != 0
    return valid


def dense_relpos_bias(table: np.ndarray, lut: np.ndarray, H: int, Lq: int, Lk: int) -> np.ndarray:
    """[H, Lq, Lk] bias with element (h, i, j) = table[lut[j - i + Lq - 1], h]: the gather of
    app/models/t5.js:55-65 (out[(h*L + i)*L + j] = relBias[bucket(j - i)*H + h]) and of HF
    T5Attention.compute_bias (relative_position = memory - context = j - i)."""
    i = np.arange(Lq)[:, None]
    j = np.arange(Lk)[None, :]
    buckets = np.asarray(lut)[j - i + Lq - 1]
    return np.ascontiguousarray(np.asarray(table)[buckets, :].transpose(2, 0, 1))


def attention_fp64(Q: np.ndarray, K: np.ndarray, V: np.ndarray, *, scale: float, bias: np.ndarray | None = None,
                   valid: np.ndarray | None = None) -> np.ndarray:
    """Exact (float64) attention. Q [B, H, Lq, D], K/V [B, H, Lk, D], bias broadcastable to
    [B, H, Lq, Lk], valid [B, Lk] bool. Returns O [B, Lq, H, D] float64."""
    Q = np.asarray(Q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    S = np.matmul(Q, np.swapaxes(K, -1, -2)) * float(scale)
    if bias is not None:
        S = S + np.asarray(bias, dtype=np.float64)
    if valid is not None:
        S = np.where(valid[:, None, None, :], S, -np.inf)
    m = S.max(axis=-1, keepdims=True)
    any_valid = np.isfinite(m)
    m = np.where(any_valid, m, 0.0)
    P = np.exp(S - m)
    den = P.sum(axis=-1, keepdims=True)
    P = np.where(any_valid, P / np.where(den > 0, den, 1.0), 0.0)
    O = np.matmul(P, V)
    return np.ascontiguousarray(O.transpose(0, 2, 1, 3))


def attention_torch_fp32(Q, K, V, *, scale: float, bias=None, valid=None, threads: int | None = None) -> np.ndarray:
    """The PyTorch fp32 CPU path (see module docstring). Inputs as for attention_fp64 (numpy);
    returns O [B, Lq, H, D] float32."""
    import torch
    import torch.nn.functional as F

    if threads is not None:
        torch.set_num_threads(threads)
    q = torch.from_numpy(np.ascontiguousarray(Q, dtype=np.float32))
    k = torch.from_numpy(np.ascontiguousarray(K, dtype=np.float32))
    v = torch.from_numpy(np.ascontiguousarray(V, dtype=np.float32))
    vt = None if valid is None else torch.from_numpy(np.ascontiguousarray(valid))
    with torch.no_grad():
        if bias is None:
            mask = None if vt is None else vt[:, None, None, :]
            o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=float(scale))
        else:
            w = torch.matmul(q, k.transpose(2, 3)) * float(scale)
            w = w + torch.from_numpy(np.ascontiguousarray(bias, dtype=np.float32))
            if vt is not None:
                add = torch.zeros(vt.shape, dtype=torch.float32)
                add[~vt] = torch.finfo(torch.float32).min
                w = w + add[:, None, None, :]
            w = torch.softmax(w, dim=-1)
            o = torch.matmul(w, v)
        if vt is not None:
            # rows with no attended key are zero (SDPA's convention, adopted by the operator)
            none = ~vt.any(dim=-1)
            if bool(none.any()):
                o[none] = 0.0
        return o.transpose(1, 2).contiguous().numpy()


def gather_call(call):
    """(Q, K, V, bias, valid) of a workload-like object with the sa_attn_args field names
    (B, H, D, Lq, Lk, q, k, v, args{q_off, ldq, sq, ...}, bias_mode, bias, lut, key_len, key_mask)."""
    a = call.args
    B, H, D, Lq, Lk = call.B, call.H, call.D, call.Lq, call.Lk
    Q = heads(call.q, B=B, L=Lq, H=H, D=D, off=a.get("q_off", 0), ld=a["ldq"], sb=a.get("sq", 0))
    K = heads(call.k, B=B, L=Lk, H=H, D=D, off=a.get("k_off", 0), ld=a["ldk"], sb=a.get("sk", 0))
    V = heads(call.v, B=B, L=Lk, H=H, D=D, off=a.get("v_off", 0), ld=a["ldv"], sb=a.get("sv", 0))
    bias = None
    if call.bias_mode == 1:  # dense [B?, H, Lq, Lk]
        bias = np.asarray(call.bias).reshape(-1, H, Lq, Lk)
    elif call.bias_mode == 2:  # relative-position table + bucket LUT
        bias = dense_relpos_bias(call.bias, call.lut, H, Lq, Lk)[None]
    valid = key_valid(B, Lk, call.key_len, call.key_mask)
    return Q, K, V, bias, valid


def reference_fp64(call) -> np.ndarray:
    Q, K, V, bias, valid = gather_call(call)
    return attention_fp64(Q, K, V, scale=call.scale, bias=bias, valid=valid)


def reference_torch(call, threads: int | None = None) -> np.ndarray:
    Q, K, V, bias, valid = gather_call(call)
    return attention_torch_fp32(Q, K, V, scale=call.scale, bias=bias, valid=valid, threads=threads)


def output_view(out: np.ndarray, call) -> np.ndarray:
    """O [B, Lq, H, D] read back from an output buffer written by the operator."""
    a = call.args
    hd = call.H * call.D
    ldo = a.get("ldo", 0) or hd
    O = heads(out, B=call.B, L=call.Lq, H=call.H, D=call.D, off=a.get("o_off", 0), ld=ldo, sb=a.get("so", 0))
    return O.transpose(0, 2, 1, 3)


def errors(got: np.ndarray, ref: np.ndarray) -> dict:
    """The parity metrics: relative L2 (tools/check.js:31-44) and normwise max relative error
    max|got - ref| / max|ref|."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    d = g - r
    den = float(np.sqrt((r * r).sum()))
    mx = float(np.abs(r).max()) if r.size else 0.0
    return {
        "rel_l2": float(np.sqrt((d * d).sum())) / max(den, 1e-30),
        "max_rel": float(np.abs(d).max()) / max(mx, 1e-30) if d.size else 0.0,
        "max_abs": float(np.abs(d).max()) if d.size else 0.0,
        "finite": bool(np.isfinite(g).all()),
    }


# ---- the tools/reference.py formulation on the callers' packed layouts (CPU baseline leg)


def reference_py_attention(q, k, v, heads: int, mask=None):
    """tools/reference.py:72-79 on torch tensors q [B, N, C], k/v [B, M, C], mask [B, M] or None."""
    import torch.nn.functional as F

    B, N, C = q.shape
    M = k.shape[1]
    q = q.view(B, N, heads, -1).transpose(1, 2)
    k = k.view(B, M, heads, -1).transpose(1, 2)
    v = v.view(B, M, heads, -1).transpose(1, 2)
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=None if mask is None else mask.bool()[:, None, None, :])
    return o.transpose(1, 2).reshape(B, N, C)


def cpu_dit_self(call):
    """DiT self-attention as tools/reference.py:96-97 runs it: qkv.view(B, -1, 3, dim) split into
    q, k, v, all heads of the batch in one call. Returns [B, N, dim]."""
    import torch

    dim = call.H * call.D
    with torch.no_grad():
        qkv = torch.from_numpy(call.q).view(call.B, -1, 3, dim)
        return reference_py_attention(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], call.H)


def cpu_dit_cross(call):
    """DiT cross-attention as tools/reference.py:98-100 runs it on contexts padded to a common
    length with a key mask (tools/reference.py:159-171). Returns [B, N, dim]."""
    import torch

    dim = call.H * call.D
    with torch.no_grad():
        q = torch.from_numpy(call.q).view(call.B, -1, dim)
        kv = torch.from_numpy(call.k).view(call.B, -1, 2, dim)
        mask = torch.arange(call.Lk)[None, :] < torch.from_numpy(call.key_len.astype("int64"))[:, None]
        return reference_py_attention(q, kv[:, :, 0], kv[:, :, 1], call.H, mask)
