"""One attention call per compiled flash-kernel and small-launch-kernel variant <kernel, D, key_split, bias, mask>.

Each call has the shape real callers give that variant (T5 batches with the relative-position
bias, DiT-sized batches, head dim 128 with every bias and mask), ragged Lq and Lk (not multiples
of 32), and enough keys that every splitting wave runs at least two loop steps, so the second LDS
stage of the K/V, relative-bias and key-mask staging is read and the softmax reference is carried
across blocks. The kernel choice is the library's own (sa_attention_plan); the shapes below are
picked so that it lands on the wanted variant, which tests assert.
"""

from __future__ import annotations

import ctypes

import numpy as np

from supra_attn import _lib
from cases import make_call

TOL = 1e-5
SENTINEL = np.float32(-12345.5)

# (kernel, D, key_split) -> (B, H, Lq, Lk): every B >= 8 (the scheduled key-length variant needs it),
# and ceil(Lk / 32) >= 2 * key_split: at least two steps (two blocks) for the last splitting wave.
FLASH, SMALL, SMALL16 = _lib.SA_KERNEL_FLASH, _lib.SA_KERNEL_FLASH_SMALL, _lib.SA_KERNEL_FLASH_SMALL16
SHAPES = {
    (FLASH, 64, 1): (48, 12, 123, 123),   # T5-like batch of prompts (48 x 12 heads, 4 query tiles of 128)
    (FLASH, 64, 2): (16, 12, 200, 150),
    (FLASH, 128, 1): (32, 8, 250, 100),   # head dim 128 (the reference's fused gate admits it, ops.js:112)
    (FLASH, 128, 2): (8, 2, 100, 150),
    (SMALL, 64, 4): (8, 4, 200, 250),     # 224 groups of 32 queries (416 of 16), 8 key blocks: two per wave
    (SMALL16, 64, 4): (8, 4, 100, 250),   # 224 groups of 16 queries, 8 key blocks: two per wave
}
# the 16-query kernel's packed key-length variant: 280 groups of 16 queries, more than the 256 CUs,
# until the empty and the 5-key sequence take 2 waves per group (250 workgroups)
SMALL16_PACKED = (8, 5, 100, 250)
KERNEL_NAMES = {FLASH: "flash", SMALL: "small", SMALL16: "small16"}

MASK_NAMES = {0: "none", 1: "key_len", 2: "key_mask", 3: "key_len_scheduled"}
BIAS_NAMES = {0: "none", 1: "dense", 2: "relpos"}


def key_lengths(rng, B: int, Lk: int, split: int) -> np.ndarray:
    """Mostly long sequences (two steps or more per splitting wave), plus a ragged short one, a
    zero and a full one; not sorted, so the sequence schedule is not the identity."""
    lo = 32 * (2 * split - 1) + 1  # last splitting wave still gets two blocks
    kl = rng.integers(min(lo, Lk), Lk + 1, size=B).astype(np.int32)
    kl[1] = Lk
    kl[2] = 0
    kl[3] = 5
    return kl


def call_for(kernel: int, D: int, split: int, bias: int, mask: int, seed: int = 0):
    """(call, host_key_len) for the variant; host_key_len says whether the host copy of the key
    lengths goes with the call (it selects the scheduled variant)."""
    B, H, Lq, Lk = SMALL16_PACKED if (kernel, mask) == (SMALL16, 3) else SHAPES[(kernel, D, split)]
    seed = seed + 10000 * kernel + 1000 * D + 100 * split + 10 * bias + mask
    rng = np.random.default_rng(seed)
    mask_mode = {0: _lib.SA_MASK_NONE, 1: _lib.SA_MASK_KEY_LEN, 2: _lib.SA_MASK_KEY_MASK,
                 3: _lib.SA_MASK_KEY_LEN}[mask]
    kl = key_lengths(rng, B, Lk, split) if mask_mode == _lib.SA_MASK_KEY_LEN else None
    # T5 calls carry no 1/sqrt(d) scaling (t5.js:80); the others the ops.js default. T5 heads are 64
    # wide: at D = 128, scale 1 and unit-normal q, k the logits have a standard deviation of 11, where
    # the fp32 oracle itself is 7.5e-6 (normwise max) from float64, so those cases take 1/sqrt(D).
    scale = 1.0 if bias == _lib.SA_BIAS_RELPOS and D == 64 else None
    call = make_call(B=B, H=H, D=D, Lq=Lq, Lk=Lk, seed=seed, scale=scale, packed=(D == 64 and bias == 0),
                     bias_mode=bias, mask_mode=mask_mode, key_len=kl,
                     dense_bias_batched=(bias == _lib.SA_BIAS_DENSE and split == 1),
                     name=f"{KERNEL_NAMES[kernel]}_d{D}_s{split}_{BIAS_NAMES[bias]}_{MASK_NAMES[mask]}")
    if mask_mode == _lib.SA_MASK_KEY_MASK:
        call.key_mask[0, :] = 0  # a sequence with no attended key: zeros
    return call, mask == 3


# wide kernels: (D, mask) -> (B, H, Lq, Lk), ragged; split into key chunks (merged by a second kernel)
# or not, both per head dim
WIDE = _lib.SA_KERNEL_WIDE
WIDE_SHAPES = {
    (256, 0): (2, 3, 70, 300),    # 18 query groups: 10 key chunks
    (256, 1): (32, 4, 100, 90),   # 512 query groups: one chunk each
    (256, 2): (2, 2, 33, 257),    # 8 query groups: 9 key chunks
    (512, 0): (1, 1, 129, 250),   # 5 query groups: 2 chunks of one round
    (512, 1): (16, 1, 500, 300),  # 256 query groups: one chunk of 3 rounds
    (512, 2): (2, 1, 200, 333),   # 14 query groups: 3 chunks
}


def wide_variants() -> list[tuple]:
    """(kernel, D, key_split, bias, mask) of every compiled wide-kernel variant."""
    return [(v.kernel, v.head_dim, v.key_split, v.bias_mode, v.mask_variant) for v in _lib.variants()
            if v.kernel == WIDE]


def wide_call_for(kernel: int, D: int, split: int, bias: int, mask: int, seed: int = 0):
    """The call for a wide variant: key lengths with 0, 1 and a full sequence where there are
    enough sequences, a key mask with one sequence fully masked, dense biases shared or per
    sequence."""
    B, H, Lq, Lk = WIDE_SHAPES[(D, mask)]
    seed = seed + 20000 + D + 10 * bias + mask
    rng = np.random.default_rng(seed)
    mask_mode = {0: _lib.SA_MASK_NONE, 1: _lib.SA_MASK_KEY_LEN, 2: _lib.SA_MASK_KEY_MASK}[mask]
    kl = None
    if mask_mode == _lib.SA_MASK_KEY_LEN:
        kl = rng.integers(0, Lk + 1, size=B).astype(np.int32)
        kl[:3] = [0, 1, Lk]
    call = make_call(B=B, H=H, D=D, Lq=Lq, Lk=Lk, seed=seed, bias_mode=bias, mask_mode=mask_mode, key_len=kl,
                     key_mask_p=0.6, dense_bias_batched=(bias == _lib.SA_BIAS_DENSE and B > 1 and mask != 1),
                     name=f"wide_d{D}_{BIAS_NAMES[bias]}_{MASK_NAMES[mask]}")
    if mask_mode == _lib.SA_MASK_KEY_MASK:
        call.key_mask[0, :] = 0
    return call


def fake_args(call, host_key_len: bool) -> _lib.AttnArgs:
    """sa_attn_args for `call` with distinct, 16-byte aligned made-up device addresses: enough for
    the host-only plan query (which compares addresses but never dereferences them)."""
    base = [0x7F0000000000]

    def addr(nbytes):
        a = base[0]
        base[0] += (int(nbytes) + 4095) // 4096 * 4096 + 4096
        return a

    q = addr(call.q.nbytes)
    k = q if call.same_qkv else addr(call.k.nbytes)
    v = q if call.same_qkv else addr(call.v.nbytes)
    kw = dict(B=call.B, H=call.H, D=call.D, Lq=call.Lq, Lk=call.Lk, q=q, k=k, v=v,
              o=addr(4 * int(np.prod(call.out_shape))), scale=call.scale, bias_mode=call.bias_mode,
              mask_mode=call.mask_mode)
    kw.update(call.args)
    keep = []
    if call.bias is not None:
        kw["bias"] = addr(call.bias.nbytes)
    if call.lut is not None:
        kw["bucket_lut"] = addr(4 * len(call.lut))
        kw["num_buckets"] = int(call.bias.shape[0])
    if call.key_len is not None:
        kw["key_len"] = addr(call.key_len.nbytes)
        if host_key_len:
            kl = np.ascontiguousarray(call.key_len, dtype=np.int32)
            keep.append(kl)
            kw["key_len_host"] = kl.ctypes.data
    if call.key_mask is not None:
        kw["key_mask"] = addr(call.key_mask.nbytes)
        kw.setdefault("smask", call.key_mask.shape[-1])
    args = _lib.AttnArgs(**kw)
    args._keep = keep  # the host key lengths must outlive the query
    return args


def flash_variants() -> list[tuple]:
    """(kernel, D, key_split, bias, mask) of every compiled flash and small-launch variant."""
    return [(v.kernel, v.head_dim, v.key_split, v.bias_mode, v.mask_variant) for v in _lib.variants()
            if v.kernel in (FLASH, SMALL, SMALL16)]


def variant_id(v) -> str:
    return "%s_d%d_s%d_b%d_m%d" % ((KERNEL_NAMES[v[0]],) + tuple(v[1:]))


def steps_per_wave(call, split: int) -> tuple:
    """Key blocks of the first and of the last splitting wave for the longest sequence (blocks of
    32 keys dealt round robin)."""
    if call.key_len is not None:
        kv = int(np.clip(call.key_len, 0, call.Lk).max())
    else:
        kv = call.Lk
    nblk = (kv + 31) // 32
    return (nblk + split - 1) // split, (nblk - (split - 1) + split - 1) // split


def check_call(dev, call, host, variant, poison_padding=False, host_copy=None):
    """Runs `call` on the GPU (host_key_len = host) after checking that the library picks `variant`;
    the output against the PyTorch fp32 CPU path and the float64 brute force (both <= 1e-5,
    relative L2 and normwise max), zero rows for sequences with no attended key, and nothing
    written outside the output rows. poison_padding: the references are taken first, then every K
    and V row past a sequence's key length is filled with NaN and Inf (separate K and V arrays).
    host_copy: a host copy of the key lengths that differs from the device's (a stale one)."""
    from oracle import attention as orc
    from supra_attn.runner import Staged

    ref = orc.reference_torch(call)
    ref64 = orc.reference_fp64(call)
    if poison_padding:
        ld = call.args["ldk"]
        k = call.k.reshape(call.B, call.Lk, ld).copy()
        v = call.v.reshape(call.B, call.Lk, ld).copy()
        for b, n in enumerate(np.clip(call.key_len, 0, call.Lk)):
            k[b, n:] = np.nan
            v[b, n:] = np.where(np.arange(ld) % 2 == 0, np.inf, np.nan).astype(np.float32)
        call.k, call.v = k.reshape(-1), v.reshape(-1)
    print(f"[case] {call.name} B={call.B} H={call.H} D={call.D} Lq={call.Lq} Lk={call.Lk}", flush=True)
    st = Staged(dev, call, out_fill=SENTINEL, host_key_len=host)
    try:
        if host_copy is not None:
            st.key_len_host = np.ascontiguousarray(host_copy, dtype=np.int32)
            st.args.key_len_host = st.key_len_host.ctypes.data
        assert _lib.plan(st.args).variant() == variant
        out = st.run()
    finally:
        st.release()
    got = orc.output_view(out, call)
    e = orc.errors(got, ref)
    assert e["finite"], call.name
    assert e["rel_l2"] <= TOL and e["max_rel"] <= TOL, f"{call.name} vs torch fp32: {e}"
    e64 = orc.errors(got, ref64)
    assert e64["rel_l2"] <= TOL and e64["max_rel"] <= TOL, f"{call.name} vs fp64: {e64}"
    # rows of a sequence with no attended key are zeros
    if call.key_len is not None:
        empty = np.asarray(call.key_len) == 0
        assert (got[empty] == 0).all()
    if call.key_mask is not None:
        empty = ~(np.asarray(call.key_mask) != 0).any(axis=1)
        assert (got[empty] == 0).all()
    # nothing written outside the output rows
    ldo = call.args.get("ldo", 0) or call.H * call.D
    written = np.zeros(out.size, dtype=bool)
    idx = orc.heads(np.arange(out.size), B=call.B, L=call.Lq, H=call.H, D=call.D, off=call.args.get("o_off", 0),
                    ld=ldo, sb=call.args.get("so", 0))
    written[idx.reshape(-1)] = True
    assert (out.reshape(-1)[~written] == SENTINEL).all()
