"""Seeded synthetic inputs for the attention workloads, in the layouts the reference callers use.

Each workload is a set of host (numpy) buffers plus the call description that `sa_attention_f32`
takes. The layouts follow the call sites:

- DiT self-attention (app/models/dit.js:167-172): one packed qkv buffer [B*256, 1728] with q, k, v
  at columns 0, 576, 1152; output [B*256, 576].
- DiT cross-attention (app/models/dit.js:179-185): q [B*256, 576]; per-sequence k|v rows
  [Lk_max, 1152] (k at column 0, v at 576), padded to Lk_max with a per-sequence key length.
- T5 encoder self-attention (app/models/t5.js:73-80): q, k, v [L, 768], scale 1, relative-position
  bias from a [32, 12] table; the last 40 keys are masked with a boolean key mask.
- SD-VAE mid-block attention (app/models/vae.js:77-94): one head, D = C = 512 over 32x32 = 1024
  tokens of GroupNorm(32)-normalised activations, q/k/v from seeded projections.

FLOPs count 4*D per attended (query, key) pair, the convention of app/gpu/ops.js:116.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import _lib

DIT_TOKENS, DIT_DIM, DIT_HEADS, DIT_HEAD_DIM, DIT_BLOCKS = 256, 576, 9, 64, 14
T5_LEN, T5_DIM, T5_HEADS, T5_BUCKETS, T5_MAX_DIST = 128, 768, 12, 32, 128
VAE_HW, VAE_C, VAE_GROUPS = 1024, 512, 32


@dataclass
class Call:
    """Host buffers and arguments of one attention call (fields as in sa_attn_args)."""

    name: str
    B: int
    H: int
    D: int
    Lq: int
    Lk: int
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    out_shape: tuple
    args: dict = field(default_factory=dict)
    scale: float = 1.0
    bias_mode: int = _lib.SA_BIAS_NONE
    bias: np.ndarray | None = None        # dense [B?, H, Lq, Lk] or relpos table [nb, H]
    lut: np.ndarray | None = None         # relpos bucket LUT (int32)
    mask_mode: int = _lib.SA_MASK_NONE
    key_len: np.ndarray | None = None     # int32 [B]
    key_mask: np.ndarray | None = None    # uint8 [B, Lk]
    same_qkv: bool = False                # q, k, v are one buffer

    def valid_pairs(self) -> int:
        if self.mask_mode == _lib.SA_MASK_KEY_LEN:
            return int(np.clip(self.key_len, 0, self.Lk).sum()) * self.H * self.Lq
        if self.mask_mode == _lib.SA_MASK_KEY_MASK:
            return int((self.key_mask[:, : self.Lk] != 0).sum()) * self.H * self.Lq
        return self.B * self.H * self.Lq * self.Lk

    def flops(self) -> int:
        return 4 * self.D * self.valid_pairs()

    def algorithmic_bytes(self) -> int:
        """Q read + O written once, K and V rows of attended keys read once, plus masks/bias."""
        hd = self.H * self.D
        qo = 2 * self.B * self.Lq * hd * 4
        if self.mask_mode == _lib.SA_MASK_KEY_LEN:
            keys = int(np.clip(self.key_len, 0, self.Lk).sum())
        elif self.mask_mode == _lib.SA_MASK_KEY_MASK:
            keys = int((self.key_mask[:, : self.Lk] != 0).sum())
        else:
            keys = self.B * self.Lk
        extra = 0
        if self.key_len is not None:
            extra += self.key_len.nbytes
        if self.key_mask is not None:
            extra += self.key_mask.nbytes
        if self.bias is not None:
            extra += self.bias.nbytes
        if self.lut is not None:
            extra += self.lut.nbytes
        return qo + 2 * keys * hd * 4 + extra


def _normal(rng, shape, std=1.0):
    x = rng.standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    return x


def dit_self(B: int = 2, seed: int = 0, rng=None, qkv=None) -> Call:
    D3 = 3 * DIT_DIM
    if qkv is None:
        qkv = _normal(rng or np.random.default_rng(seed), (B * DIT_TOKENS, D3))
    return Call(
        name=f"dit_self_b{B}", B=B, H=DIT_HEADS, D=DIT_HEAD_DIM, Lq=DIT_TOKENS, Lk=DIT_TOKENS,
        q=qkv, k=qkv, v=qkv, same_qkv=True, out_shape=(B * DIT_TOKENS, DIT_DIM),
        args=dict(q_off=0, k_off=DIT_DIM, v_off=2 * DIT_DIM, ldq=D3, ldk=D3, ldv=D3, ldo=DIT_DIM,
                  sq=DIT_TOKENS * D3, sk=DIT_TOKENS * D3, sv=DIT_TOKENS * D3, so=DIT_TOKENS * DIT_DIM),
        scale=1.0 / math.sqrt(DIT_HEAD_DIM),
    )


def dit_cross(B: int = 2, key_len=(77, 1), Lk_max: int = 128, seed: int = 1, rng=None, q=None, kv=None) -> Call:
    if q is None or kv is None:
        rng = rng or np.random.default_rng(seed)
        q = _normal(rng, (B * DIT_TOKENS, DIT_DIM))
        kv = _normal(rng, (B * Lk_max, 2 * DIT_DIM))
    kl = np.asarray(key_len, dtype=np.int32)
    assert kl.shape == (B,)
    return Call(
        name=f"dit_cross_b{B}", B=B, H=DIT_HEADS, D=DIT_HEAD_DIM, Lq=DIT_TOKENS, Lk=Lk_max,
        q=q, k=kv, v=kv, out_shape=(B * DIT_TOKENS, DIT_DIM),
        args=dict(q_off=0, k_off=0, v_off=DIT_DIM, ldq=DIT_DIM, ldk=2 * DIT_DIM, ldv=2 * DIT_DIM, ldo=DIT_DIM,
                  sq=DIT_TOKENS * DIT_DIM, sk=Lk_max * 2 * DIT_DIM, sv=Lk_max * 2 * DIT_DIM,
                  so=DIT_TOKENS * DIT_DIM),
        scale=1.0 / math.sqrt(DIT_HEAD_DIM), mask_mode=_lib.SA_MASK_KEY_LEN, key_len=kl,
    )


def t5_self(L: int = T5_LEN, masked_tail: int = 40, seed: int = 2, rng=None, lut=None) -> Call:
    """T5-base encoder self-attention. `lut` is the bucket LUT for (L, L); by default it comes from
    the library's sa_t5_bucket_lut."""
    rng = rng or np.random.default_rng(seed)
    q = _normal(rng, (L, T5_DIM))
    k = _normal(rng, (L, T5_DIM))
    v = _normal(rng, (L, T5_DIM))
    table = _normal(rng, (T5_BUCKETS, T5_HEADS), std=0.5)
    mask = np.ones((1, L), dtype=np.uint8)
    if masked_tail:
        mask[0, L - masked_tail:] = 0
    if lut is None:
        lut = _lib.bucket_lut(L, L, T5_BUCKETS, T5_MAX_DIST, True)
    return Call(
        name="t5_self", B=1, H=T5_HEADS, D=T5_DIM // T5_HEADS, Lq=L, Lk=L, q=q, k=k, v=v,
        out_shape=(L, T5_DIM), args=dict(ldq=T5_DIM, ldk=T5_DIM, ldv=T5_DIM, ldo=T5_DIM),
        scale=1.0, bias_mode=_lib.SA_BIAS_RELPOS, bias=table, lut=np.asarray(lut, dtype=np.int32),
        mask_mode=_lib.SA_MASK_KEY_MASK, key_mask=mask,
    )


def vae_mid(seed: int = 3, rng=None, hw: int = VAE_HW) -> Call:
    rng = rng or np.random.default_rng(seed)
    C = VAE_C
    x = _normal(rng, (hw, C))
    # GroupNorm(32 groups, eps 1e-6, gamma 1, beta 0) over the NHWC image [pixels, C]
    g = x.reshape(hw, VAE_GROUPS, C // VAE_GROUPS).astype(np.float64)
    mu = g.mean(axis=(0, 2), keepdims=True)
    var = g.var(axis=(0, 2), keepdims=True)
    xn = ((g - mu) / np.sqrt(var + 1e-6)).reshape(hw, C).astype(np.float32)
    std = 1.0 / math.sqrt(C)
    wq, wk, wv = (_normal(rng, (C, C), std=std) for _ in range(3))
    q = xn @ wq.T
    k = xn @ wk.T
    v = xn @ wv.T
    return Call(
        name="vae_mid", B=1, H=1, D=C, Lq=hw, Lk=hw, q=np.ascontiguousarray(q, dtype=np.float32),
        k=np.ascontiguousarray(k, dtype=np.float32), v=np.ascontiguousarray(v, dtype=np.float32),
        out_shape=(hw, C), args=dict(ldq=C, ldk=C, ldv=C, ldo=C), scale=1.0 / math.sqrt(C),
    )


SWEEP_BATCH, SWEEP_STEPS, SWEEP_LK = 64, 50, 128


def sweep_key_lengths(seed: int = 4, B: int = SWEEP_BATCH) -> np.ndarray:
    """Cross-attention key lengths ~ U{1..128}, drawn once per run (a fixed prompt per sequence)."""
    return np.random.default_rng([seed, 999]).integers(1, SWEEP_LK + 1, size=B, dtype=np.int32)


class SweepData:
    """Inputs of the batch-B DiT throughput sweep: per-block self-attention qkv, cross-attention q
    and k|v, and the fixed per-sequence key lengths.

    Each tensor kind comes from one seeded N(0,1) pool; block i reads the window starting at
    element i*4099, so the 14 blocks have distinct contents and addresses (no call replays a
    cache-hot buffer) while the host generates only about one block's worth of normals."""

    SHIFT = 4099

    def __init__(self, seed: int = 4, B: int = SWEEP_BATCH, blocks: int = DIT_BLOCKS):
        rng = np.random.default_rng([seed, 0])
        self.B, self.blocks, self.seed = B, blocks, seed
        self.n_self = B * DIT_TOKENS * 3 * DIT_DIM
        self.n_q = B * DIT_TOKENS * DIT_DIM
        self.n_kv = B * SWEEP_LK * 2 * DIT_DIM
        extra = (blocks - 1) * self.SHIFT
        self.self_pool = rng.standard_normal(self.n_self + extra, dtype=np.float32)
        self.q_pool = rng.standard_normal(self.n_q + extra, dtype=np.float32)
        self.kv_pool = rng.standard_normal(self.n_kv + extra, dtype=np.float32)
        self.key_len = sweep_key_lengths(seed, B)

    def block(self, i: int) -> tuple[Call, Call]:
        o = i * self.SHIFT
        s = dit_self(B=self.B, qkv=self.self_pool[o:o + self.n_self].reshape(self.B * DIT_TOKENS, 3 * DIT_DIM))
        c = dit_cross(B=self.B, key_len=self.key_len, Lk_max=SWEEP_LK,
                      q=self.q_pool[o:o + self.n_q].reshape(self.B * DIT_TOKENS, DIT_DIM),
                      kv=self.kv_pool[o:o + self.n_kv].reshape(self.B * SWEEP_LK, 2 * DIT_DIM))
        s.name = f"sweep_self_blk{i}"
        c.name = f"sweep_cross_blk{i}"
        return s, c


def sweep_block(block: int, seed: int = 4, B: int = SWEEP_BATCH) -> tuple[Call, Call]:
    """Self- and cross-attention inputs of one DiT block of the sweep."""
    return SweepData(seed, B, blocks=block + 1).block(block)


CONFIGS = {
    "dit_self_b2": lambda: dit_self(B=2, seed=0),
    "dit_cross_b2": lambda: dit_cross(B=2, seed=1),
    "t5_self": lambda: t5_self(seed=2),
    "vae_mid": lambda: vae_mid(seed=3),
}
