"""CPU oracle for the SD-VAE mid-block attention (sa_vae_attention_f32).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker. The product path never calls it.

Semantics restated (app/models/vae.js:77-94, i.e. diffusers Attention with a group norm and the
residual connection, AttnProcessor2_0), over an NHWC image x [HW, C]:

  n     = GroupNorm(x; groups, eps, gamma, beta)   per group of C/groups channels, mean and biased
          variance over all pixels and the group's channels (app/gpu/kernels.js:117-162)
  q|k|v = n Wqkv^T + bqkv                          Wqkv [3C, C]: the q, k, v weights stacked
  a     = softmax(q k^T / sqrt(C)) v               one head of dim C (vae.js:86, default scale)
  out   = x + a Wo^T + bo                          (vae.js:88-90)

Two restatements: `block_fp64` (NumPy float64) and `block_torch_fp32` (PyTorch CPU float32:
F.group_norm, F.linear, F.scaled_dot_product_attention), which the parity bar is defined against.
"""

from __future__ import annotations

import numpy as np


def groupnorm_fp64(x, gamma, beta, groups: int, eps: float) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    HW, C = x.shape
    g = x.reshape(HW, groups, C // groups)
    mean = g.mean(axis=(0, 2), keepdims=True)
    var = ((g - mean) ** 2).mean(axis=(0, 2), keepdims=True)
    n = ((g - mean) / np.sqrt(var + eps)).reshape(HW, C)
    return n * np.asarray(gamma, dtype=np.float64)[None, :] + np.asarray(beta, dtype=np.float64)[None, :]


def block_fp64(x, gamma, beta, wqkv, bqkv, wo, bo, groups: int = 32, eps: float = 1e-6) -> np.ndarray:
    x64 = np.asarray(x, dtype=np.float64)
    HW, C = x64.shape
    n = groupnorm_fp64(x64, gamma, beta, groups, eps)
    qkv = n @ np.asarray(wqkv, dtype=np.float64).T
    if bqkv is not None:
        qkv = qkv + np.asarray(bqkv, dtype=np.float64)[None, :]
    q, k, v = qkv[:, :C], qkv[:, C:2 * C], qkv[:, 2 * C:]
    s = (q @ k.T) / np.sqrt(C)
    s = s - s.max(axis=1, keepdims=True)
    p = np.exp(s)
    a = (p / p.sum(axis=1, keepdims=True)) @ v
    o = a @ np.asarray(wo, dtype=np.float64).T
    if bo is not None:
        o = o + np.asarray(bo, dtype=np.float64)[None, :]
    return (x64 + o).astype(np.float32)


def block_torch_fp32(x, gamma, beta, wqkv, bqkv, wo, bo, groups: int = 32, eps: float = 1e-6) -> np.ndarray:
    import torch
    import torch.nn.functional as F

    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    xt = t(x)
    HW, C = xt.shape
    n = F.group_norm(xt.t().reshape(1, C, HW), groups, t(gamma), t(beta), eps).reshape(C, HW).t()
    qkv = F.linear(n, t(wqkv), t(bqkv))
    q, k, v = (qkv[:, i * C:(i + 1) * C].reshape(1, 1, HW, C) for i in range(3))
    a = F.scaled_dot_product_attention(q, k, v).reshape(HW, C)
    return (xt + F.linear(a, t(wo), t(bo))).numpy()
