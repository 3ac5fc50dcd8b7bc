"""Seeded synthetic inputs for the linear layers either side of attention in the DiT block.

The shapes and epilogues follow app/models/dit.js:165-192 with R = B*256 rows (dim 576, MLP 2304):

- qkv   h [R, 576] -> [R, 1728] + bias                         (dit.js:167)
- proj  a [R, 576] -> x [R, 576] += gate * (a W^T + b)         (dit.js:175, AdaLN-Zero gate)
- q     h [R, 576] -> [R, 576] + bias                          (dit.js:178)
- cproj c [R, 576] -> x [R, 576] += c W^T + b                  (dit.js:187)
- fc1   h [R, 576] -> gelu_tanh(h W^T + b) [R, 2304]           (dit.js:191)
- fc2   f [R, 2304] -> x [R, 576] += gate * (f W^T + b)        (dit.js:193)

and the per-prompt context projection kv [L, 576] -> [L, 1152] (dit.js:141). Weights ~ N(0, 1/K)
(unit-variance outputs), activations and the residual stream ~ N(0, 1), biases ~ N(0, 0.1^2),
gates ~ N(0, 1). FLOPs count 2*M*N*K (app/gpu/ops.js:24).

Also the SD-VAE mid-block attention as one call (`vae_block`, app/models/vae.js:77-94): GroupNorm,
the q/k/v projections, one-head attention, the output projection and the residual.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib

DIT_DIM, DIT_MLP, DIT_TOKENS = 576, 2304, 256


@dataclass
class LinearCall:
    """Host buffers and arguments of one linear call (fields as in sa_linear_args)."""

    name: str
    M: int
    N: int
    K: int
    x: np.ndarray              # flat buffer holding X at x_off with row stride ldx
    w: np.ndarray              # [N, ldw]
    y0: np.ndarray             # initial output buffer (read by the residual epilogues)
    bias: np.ndarray | None = None
    gate: np.ndarray | None = None
    gate_off: int = 0
    alpha: float = 1.0
    act: int = _lib.SA_ACT_NONE
    epi: int = _lib.SA_EPI_STORE
    x_off: int = 0
    ldx: int = 0
    ldw: int = 0
    y_off: int = 0
    ldy: int = 0

    def flops(self) -> int:
        return 2 * self.M * self.N * self.K

    def algorithmic_bytes(self) -> int:
        """x and W read once, y written once (and read once for a residual), bias and gate once."""
        y = self.M * self.N * (2 if self.epi != _lib.SA_EPI_STORE else 1)
        extra = (self.N if self.bias is not None else 0) + (self.N if self.epi == _lib.SA_EPI_RESID_GATE else 0)
        return 4 * (self.M * self.K + self.N * self.K + y + extra)

    def oracle_kwargs(self) -> dict:
        return dict(M=self.M, N=self.N, K=self.K, bias=self.bias, gate=self.gate, gate_off=self.gate_off,
                    alpha=self.alpha, act=self.act, epi=self.epi, x_off=self.x_off, ldx=self.ldx, ldw=self.ldw,
                    y_off=self.y_off, ldy=self.ldy)


def make_linear(name: str, M: int, N: int, K: int, *, seed: int = 0, bias: bool = True, act: int = _lib.SA_ACT_NONE,
                epi: int = _lib.SA_EPI_STORE, alpha: float = 1.0, x_off: int = 0, ldx: int = 0, ldw: int = 0,
                y_off: int = 0, ldy: int = 0, gate_off: int = 0) -> LinearCall:
    rng = np.random.default_rng(seed)
    ldx_ = ldx or K
    ldw_ = ldw or K
    ldy_ = ldy or N
    x = rng.standard_normal(x_off + (M - 1) * ldx_ + K, dtype=np.float32)
    w = (rng.standard_normal((N, ldw_), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    y0 = rng.standard_normal(y_off + (M - 1) * ldy_ + N, dtype=np.float32)
    b = (rng.standard_normal(N, dtype=np.float32) * np.float32(0.1)) if bias else None
    g = rng.standard_normal(gate_off + N, dtype=np.float32) if epi == _lib.SA_EPI_RESID_GATE else None
    return LinearCall(name=name, M=M, N=N, K=K, x=x, w=w, y0=y0, bias=b, gate=g, gate_off=gate_off, alpha=alpha,
                      act=act, epi=epi, x_off=x_off, ldx=ldx, ldw=ldw, y_off=y_off, ldy=ldy)


def dit_block_linears(B: int = 64, seed: int = 20) -> list[LinearCall]:
    """The six per-block linears of the DiT forward at batch B (R = B*256 rows)."""
    R = B * DIT_TOKENS
    D, F = DIT_DIM, DIT_MLP
    gate, resid = _lib.SA_EPI_RESID_GATE, _lib.SA_EPI_RESID
    return [
        make_linear("qkv", R, 3 * D, D, seed=seed),
        make_linear("proj", R, D, D, seed=seed + 1, epi=gate, gate_off=2 * D),
        make_linear("q", R, D, D, seed=seed + 2),
        make_linear("cproj", R, D, D, seed=seed + 3, epi=resid),
        make_linear("fc1", R, F, D, seed=seed + 4, act=_lib.SA_ACT_GELU_TANH),
        make_linear("fc2", R, D, F, seed=seed + 5, epi=gate, gate_off=5 * D),
    ]


def context_kv(L: int = 77, seed: int = 26) -> LinearCall:
    """Per-prompt cross-attention keys/values of one block (dit.js:141): [L, 576] -> [L, 1152]."""
    return make_linear("ctx_kv", L, 2 * DIT_DIM, DIT_DIM, seed=seed)


@dataclass
class VaeBlockCall:
    """Host buffers of one VAE mid-block attention call (fields as in sa_vae_attn_args)."""

    name: str
    HW: int
    C: int
    groups: int
    eps: float
    x: np.ndarray      # [HW, C]
    gamma: np.ndarray  # [C]
    beta: np.ndarray
    wqkv: np.ndarray   # [3C, C]
    bqkv: np.ndarray | None
    wo: np.ndarray     # [C, C]
    bo: np.ndarray | None

    def flops(self) -> int:
        """Projections 2*HW*C*(3C + C) plus attention 4*C*HW^2 (app/gpu/ops.js:24, 116)."""
        return 2 * self.HW * self.C * 4 * self.C + 4 * self.C * self.HW * self.HW

    def algorithmic_bytes(self) -> int:
        """x read, out written, the weights and vectors read once."""
        return 4 * (2 * self.HW * self.C + 4 * self.C * self.C + 6 * self.C)

    def oracle_args(self) -> tuple:
        return (self.x, self.gamma, self.beta, self.wqkv, self.bqkv, self.wo, self.bo)


def vae_block(HW: int = 1024, C: int = 512, groups: int = 32, seed: int = 30, bias: bool = True) -> VaeBlockCall:
    """The SD-VAE mid-block attention (app/models/vae.js:77-94) at a 32x32 latent: x ~ N(0, 1),
    GroupNorm affine ~ (1 + 0.1 N, 0.1 N), projections ~ N(0, 1/C), biases ~ 0.1 N."""
    rng = np.random.default_rng(seed)
    f = lambda *shape, s=1.0: (rng.standard_normal(shape, dtype=np.float32) * np.float32(s)).astype(np.float32)
    return VaeBlockCall(name=f"vae_block_{HW}x{C}", HW=HW, C=C, groups=groups, eps=1e-6, x=f(HW, C),
                        gamma=(1 + f(C, s=0.1)).astype(np.float32), beta=f(C, s=0.1), wqkv=f(3 * C, C, s=C ** -0.5),
                        bqkv=f(3 * C, s=0.1) if bias else None, wo=f(C, C, s=C ** -0.5),
                        bo=f(C, s=0.1) if bias else None)
