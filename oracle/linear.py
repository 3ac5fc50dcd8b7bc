"""CPU oracle for the linear layer (sa_linear_f32).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or, for the CPU baseline, as the thing timed on the
host). The product path never calls it.

Semantics restated (app/gpu/ops.js:35-43 `linear`, app/gpu/gemm.js:116-137 `matmulShader` with A mode
"rows", B format "f32"):

  X[m][k] = x[x_off + m*ldx + k],  W[n][k] = w[n*ldw + k]   (PyTorch [out, in] layout)
  r[m][n] = act(alpha * sum_k X[m][k] W[n][k] + bias[n])   (gemm.js:126-130, alpha at :205)
  epilogue (gemm.js:131): Y = r | Y += r | Y += gate[gate_off + n] * r,  Y[m][n] = y[y_off + m*ldy + n]

Activations (gemm.js:21-36): gelu = 0.5 x (1 + erf(x / sqrt 2)); gelu_tanh = 0.5 x (1 + tanh(sqrt(2/pi)
(x + 0.044715 x^3))), PyTorch GELU(approximate="tanh"); silu = x / (1 + exp(-x)). The reference's
WGSL evaluates erf with the Abramowitz-Stegun 7.1.26 polynomial (|error| < 1.5e-7); the oracle and
the kernel use erf itself, as PyTorch does.

Two restatements: `linear_fp64` (NumPy float64, the ground truth of the closed-form checks) and
`linear_torch_fp32` (PyTorch CPU float32: torch.mm, F.gelu / F.silu), which the parity bar is
defined against.
"""

from __future__ import annotations

import math

import numpy as np

ACT_NONE, ACT_GELU, ACT_GELU_TANH, ACT_SILU = 0, 1, 2, 3
EPI_STORE, EPI_RESID, EPI_RESID_GATE = 0, 1, 2
ACT_NAMES = {"none": ACT_NONE, "gelu": ACT_GELU, "gelu_tanh": ACT_GELU_TANH, "silu": ACT_SILU}

_erf = np.vectorize(math.erf, otypes=[np.float64])


def act_fp64(v: np.ndarray, act: int) -> np.ndarray:
    v = np.asarray(v, dtype=np.float64)
    if act == ACT_GELU:
        return 0.5 * v * (1.0 + _erf(v / math.sqrt(2.0)))
    if act == ACT_GELU_TANH:
        return 0.5 * v * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (v + 0.044715 * v ** 3)))
    if act == ACT_SILU:
        return v / (1.0 + np.exp(-v))
    return v


def operands(x, w, *, M, N, K, x_off=0, ldx=0, ldw=0):
    """Gather X [M, K] and W [N, K] from flat buffers with the sa_linear_args addressing."""
    ldx = ldx or K
    ldw = ldw or K
    xf, wf = np.asarray(x).reshape(-1), np.asarray(w).reshape(-1)
    X = xf[x_off + np.arange(M)[:, None] * ldx + np.arange(K)[None, :]]
    W = wf[np.arange(N)[:, None] * ldw + np.arange(K)[None, :]]
    return X, W


def _out_index(M, N, y_off, ldy):
    return y_off + np.arange(M)[:, None] * ldy + np.arange(N)[None, :]


def linear_fp64(x, w, y0, *, M, N, K, bias=None, gate=None, gate_off=0, alpha=1.0, act=ACT_NONE, epi=EPI_STORE,
                x_off=0, ldx=0, ldw=0, y_off=0, ldy=0) -> np.ndarray:
    """The whole flat output buffer after the call (float64 arithmetic, float32 result)."""
    X, W = operands(x, w, M=M, N=N, K=K, x_off=x_off, ldx=ldx, ldw=ldw)
    r = alpha * (X.astype(np.float64) @ W.astype(np.float64).T)
    if bias is not None:
        r = r + np.asarray(bias, dtype=np.float64)[None, :N]
    r = act_fp64(r, act)
    y = np.array(y0, dtype=np.float64, copy=True).reshape(-1)
    idx = _out_index(M, N, y_off, ldy or N)
    if epi == EPI_STORE:
        y[idx] = r
    elif epi == EPI_RESID:
        y[idx] = y[idx] + r
    else:
        g = np.asarray(gate, dtype=np.float64).reshape(-1)[gate_off + np.arange(N)]
        y[idx] = y[idx] + g[None, :] * r
    return y.astype(np.float32).reshape(np.shape(y0))


def linear_torch_fp32(x, w, y0, *, M, N, K, bias=None, gate=None, gate_off=0, alpha=1.0, act=ACT_NONE,
                      epi=EPI_STORE, x_off=0, ldx=0, ldw=0, y_off=0, ldy=0) -> np.ndarray:
    """The PyTorch fp32 CPU formulation: torch.mm, alpha, + bias, F.gelu / F.silu, epilogue."""
    import torch
    import torch.nn.functional as F

    X, W = operands(x, w, M=M, N=N, K=K, x_off=x_off, ldx=ldx, ldw=ldw)
    r = torch.mm(torch.from_numpy(np.ascontiguousarray(X, dtype=np.float32)),
                 torch.from_numpy(np.ascontiguousarray(W, dtype=np.float32)).t())
    if alpha != 1.0:
        r = r * alpha
    if bias is not None:
        r = r + torch.from_numpy(np.asarray(bias, dtype=np.float32)[:N])
    if act == ACT_GELU:
        r = F.gelu(r)
    elif act == ACT_GELU_TANH:
        r = F.gelu(r, approximate="tanh")
    elif act == ACT_SILU:
        r = F.silu(r)
    r = r.numpy()
    y = np.array(y0, dtype=np.float32, copy=True).reshape(-1)
    idx = _out_index(M, N, y_off, ldy or N)
    if epi == EPI_STORE:
        y[idx] = r
    elif epi == EPI_RESID:
        y[idx] = y[idx] + r
    else:
        g = np.asarray(gate, dtype=np.float32).reshape(-1)[gate_off + np.arange(N)]
        y[idx] = y[idx] + g[None, :] * r
    return y.reshape(np.shape(y0))


def errors(got: np.ndarray, ref: np.ndarray) -> dict:
    """rel-L2 and normwise max relative error of the written region (same bar as attention)."""
    g = np.asarray(got, dtype=np.float64).reshape(-1)
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    d = g - r
    nr = float(np.linalg.norm(r))
    mr = float(np.max(np.abs(r))) if r.size else 0.0
    return {
        "finite": bool(np.isfinite(g).all()),
        "rel_l2": float(np.linalg.norm(d)) / nr if nr > 0 else float(np.linalg.norm(d)),
        "max_rel": float(np.max(np.abs(d))) / mr if mr > 0 else float(np.max(np.abs(d), initial=0.0)),
    }
