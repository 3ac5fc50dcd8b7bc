"""Packed sequences of the 16-query small-launch kernel (flash_small16.hip, MASK_KEY_LEN_ORDERED).

A sequence of at most two key blocks (32 keys each) keeps waves of its workgroups idle. Where a
launch has more 16-query groups than the 256 CUs, the host copy of the key lengths lets the library
give such sequences 2 waves per group, then (if that is not enough) those of at most one block 1
wave, shortest first, only until the launch fits one workgroup per CU: a workgroup holding several
groups costs more than one group per CU. The batch-2 guided DiT cross call (keys 77 and 1,
app/models/dit.js:184) takes 144 + 72 workgroups in place of 288 and runs on this kernel.

Host tests (no GPU): the plan against that rule, and the kernel's workgroup decode (restated below
from flash_small16_kernel's prologue) against the plan's grid: every (sequence, head, 16-query
group) of the call is covered once, by exactly its waves, and no workgroup decodes to a sequence or
head outside the call, which is what keeps the kernel's loads in bounds. GPU tests: parity of packed
launches (<= 1e-5 against the PyTorch fp32 CPU path and the float64 brute force) with ragged query
counts, every bias mode, empty sequences and sequences of 1, 2 and more blocks.
"""

from __future__ import annotations

import numpy as np
import pytest

from supra_attn import _lib
from cases import make_call
from variant_cases import SMALL, SMALL16, check_call

PACKED = _lib.SA_MASK_VARIANT_KEY_LEN_SCHEDULED
MAX_PACKED = 16  # sequences: 2 bits each in the kernel arguments


def packing(key_len, H, Lq, Lk, cus=256):
    """Log2 of the waves per 16-query group of each sequence under the rule above (None: no packing)."""
    B = len(key_len)
    q_groups = -(-Lq // 16)
    nblk = (np.clip(np.asarray(key_len), 0, Lk) + 31) // 32
    if B > MAX_PACKED or B * H * q_groups <= cus:
        return None
    lw = [2] * B

    def grid():
        return sum(H * -(-q_groups // (4 >> w)) for w in lw)

    order = sorted(range(B), key=lambda s: nblk[s])  # stable: shortest first, then batch order
    for most, w in ((2, 1), (1, 0)):
        for s in order:
            if nblk[s] > most or grid() <= cus:
                break
            lw[s] = w
        if grid() <= cus:
            break
    return lw if min(lw) < 2 else None


def args_for(key_len, H, Lq, Lk, host=True, bias_mode=_lib.SA_BIAS_NONE):
    B = len(key_len)
    kl = np.ascontiguousarray(key_len, dtype=np.int32)
    hd = H * 64
    kw = dict(B=B, H=H, D=64, Lq=Lq, Lk=Lk, q=1 << 20, k=1 << 34, v=1 << 38, o=1 << 42, ldq=hd, ldk=hd, ldv=hd,
              ldo=hd, sq=Lq * hd, sk=Lk * hd, sv=Lk * hd, so=Lq * hd, scale=0.125, mask_mode=_lib.SA_MASK_KEY_LEN,
              key_len=1 << 46, key_len_host=kl.ctypes.data if host else None, bias_mode=bias_mode)
    if bias_mode == _lib.SA_BIAS_RELPOS:
        kw.update(bias=1 << 45, bucket_lut=1 << 44, num_buckets=32)
    a = _lib.AttnArgs(**kw)
    a._keep = kl
    return a


def decode(tile, code, H, q_groups):
    """Workgroup `tile` of a packed launch -> (sequence, head, first group, log2 waves per group),
    as flash_small16_kernel's prologue computes it."""
    b = 0
    while True:
        lw = min((code >> (2 * b)) & 3, 2)
        per_head = (q_groups + (4 >> lw) - 1) >> (2 - lw)
        if tile < H * per_head or b == MAX_PACKED - 1:
            break
        tile -= H * per_head
        b += 1
    h = tile // per_head
    return b, h, (tile - h * per_head) << (2 - lw), lw


def test_guided_dit_cross_batch2_is_packed():
    p = _lib.plan(args_for([77, 1], H=9, Lq=256, Lk=128))
    assert (p.kernel, p.mask_variant, p.workgroups) == (SMALL16, PACKED, 9 * 16 + 9 * 8)
    # without the host copy nothing is known of the lengths: 288 groups of 16 exceed one per CU
    p = _lib.plan(args_for([77, 1], H=9, Lq=256, Lk=128, host=False))
    assert (p.kernel, p.mask_variant) == (SMALL, _lib.SA_MASK_KEY_LEN)


def test_packing_only_as_far_as_needed():
    # a launch that fits one workgroup per CU as it is: no packing (the per-sample unconditioned call)
    p = _lib.plan(args_for([1], H=9, Lq=256, Lk=128))
    assert (p.kernel, p.mask_variant, p.workgroups) == (SMALL16, _lib.SA_MASK_KEY_LEN, 144)
    # every sequence longer than two blocks: nothing to pack, the 32-query kernel
    p = _lib.plan(args_for([77, 100], H=9, Lq=256, Lk=128))
    assert (p.kernel, p.mask_variant) == (SMALL, _lib.SA_MASK_KEY_LEN)
    # more sequences than the kernel arguments code: no packing
    p = _lib.plan(args_for([1] * 17, H=2, Lq=100, Lk=128))
    assert p.mask_variant == _lib.SA_MASK_KEY_LEN and p.workgroups == 17 * 2 * 7
    # 16 one-block sequences, 416 groups: 14 of them at 2 waves per group make 248 workgroups
    p = _lib.plan(args_for([1] * 16, H=2, Lq=200, Lk=128))
    assert (p.kernel, p.mask_variant, p.workgroups) == (SMALL16, PACKED, 14 * 2 * 7 + 2 * 2 * 13)
    assert packing([1] * 16, 2, 200, 128) == [1] * 14 + [2] * 2
    # 2 waves per group for both short sequences is not enough (324 of 468): then 1 wave, 252
    p = _lib.plan(args_for([1, 20, 128], H=12, Lq=200, Lk=128))
    assert (p.kernel, p.mask_variant, p.workgroups) == (SMALL16, PACKED, 2 * 12 * 4 + 12 * 13)
    assert packing([1, 20, 128], 12, 200, 128) == [0, 0, 2]


def test_grid_and_decode_cover_every_group_once():
    rng = np.random.default_rng(2024)
    checked = 0
    for _ in range(1500):
        B = int(rng.integers(1, MAX_PACKED + 1))
        H = int(rng.integers(1, 13))
        Lq = int(rng.integers(1, 300))
        Lk = int(rng.integers(33, 200))
        kl = rng.integers(-5, Lk + 40, size=B)
        short = rng.random(B) < 0.5
        kl[short] = rng.integers(-2, 65, size=int(short.sum()))
        p = _lib.plan(args_for(kl, H, Lq, Lk))
        if p.kernel != SMALL16:
            continue
        q_groups = -(-Lq // 16)
        lws = packing(kl, H, Lq, Lk)
        if p.mask_variant != PACKED:
            assert lws is None and p.workgroups == B * H * q_groups <= 256
            continue
        assert lws is not None and p.workgroups <= 256 < B * H * q_groups
        code = sum(int(lw) << (2 * s) for s, lw in enumerate(lws))
        want = sum(H * -(-q_groups // (4 >> int(lw))) for lw in lws)
        assert p.workgroups == want
        seen = {}
        for tile in range(p.workgroups):
            b, h, g0, lw = decode(tile, code, H, q_groups)
            assert 0 <= b < B and 0 <= h < H and lw == lws[b]
            for wave in range(4):
                gq = g0 + (wave >> lw)
                if gq < q_groups:
                    seen.setdefault((b, h, gq), []).append(wave & ((1 << lw) - 1))
        assert len(seen) == B * H * q_groups
        for (b, _, _), ranks in seen.items():
            assert sorted(ranks) == list(range(1 << int(lws[b])))
        checked += 1
    assert checked >= 100


# (name, B, H, Lq, Lk, key lengths, log2 waves per group the rule gives): 2 and 1 waves per group,
# unpacked sequences beside them, empty and one-key sequences, ragged query counts (groups past the
# last query inside a packed workgroup)
PACKED_CASES = [
    ("dit_cross_b2", 2, 9, 256, 128, [77, 1], [2, 1]),
    ("mixed_lq100", 8, 6, 100, 150, [0, 1, 32, 33, 64, 65, 150, 17], [1, 1, 1, 1, 2, 2, 2, 1]),
    ("three_lq200", 3, 12, 200, 128, [1, 20, 128], [0, 0, 2]),
    ("sixteen_lq20", 16, 9, 20, 96, [5, 0, 96, 40, 31, 64, 70, 1, 2, 33, 90, 12, 63, 96, 0, 30],
     [1, 1, 2, 2, 1, 2, 2, 2, 2, 2, 2, 2, 2, 2, 1, 2]),
]


@pytest.mark.parametrize("case", PACKED_CASES, ids=[c[0] for c in PACKED_CASES])
def test_parity_cases_are_packed(case):
    name, B, H, Lq, Lk, kl, lws = case
    assert packing(kl, H, Lq, Lk) == lws
    p = _lib.plan(args_for(kl, H, Lq, Lk))
    q_groups = -(-Lq // 16)
    assert (p.kernel, p.mask_variant) == (SMALL16, PACKED)
    assert p.workgroups == sum(H * -(-q_groups // (4 >> lw)) for lw in lws)


@pytest.mark.gpu
@pytest.mark.parametrize("bias", [_lib.SA_BIAS_NONE, _lib.SA_BIAS_DENSE, _lib.SA_BIAS_RELPOS],
                         ids=["none", "dense", "relpos"])
@pytest.mark.parametrize("case", PACKED_CASES, ids=[c[0] for c in PACKED_CASES])
def test_packed_parity(dev, case, bias):
    """With NaN and Inf in every K and V row past a sequence's length (a wave's first block reads
    them before the length is known), against the attention over the valid keys alone."""
    name, B, H, Lq, Lk, kl, _ = case
    call = make_call(B=B, H=H, D=64, Lq=Lq, Lk=Lk, seed=300 + 7 * bias + len(name), bias_mode=bias,
                     mask_mode=_lib.SA_MASK_KEY_LEN, key_len=np.asarray(kl, dtype=np.int32),
                     dense_bias_batched=(B <= 8), name=f"packed_{name}_b{bias}")
    check_call(dev, call, True, (SMALL16, 64, 4, bias, PACKED), poison_padding=True)


# (name, B, H, Lq, Lk, device key lengths, host copy): the host copy calls long sequences short, so
# they are packed anyway and a wave runs several key blocks: 1 wave per group over 4 blocks (two
# loop iterations with both operand sets), 2 waves per group over 2 blocks each
STALE_CASES = [
    ("one_wave_4_blocks", 3, 12, 200, 128, [128, 100, 77], [1, 20, 128]),
    ("two_waves_2_blocks", 3, 9, 256, 128, [128, 128, 5], [1, 1, 128]),
]


@pytest.mark.parametrize("case", STALE_CASES, ids=[c[0] for c in STALE_CASES])
def test_stale_cases_are_packed(case):
    name, B, H, Lq, Lk, kl, host = case
    p = _lib.plan(args_for(host, H, Lq, Lk))
    assert (p.kernel, p.mask_variant) == (SMALL16, PACKED) and min(packing(host, H, Lq, Lk)) < 2


@pytest.mark.gpu
@pytest.mark.parametrize("case", STALE_CASES, ids=[c[0] for c in STALE_CASES])
def test_stale_host_copy_costs_speed_not_results(dev, case):
    """The kernel takes its key lengths from the device, so a wrong host copy only shapes the launch."""
    name, B, H, Lq, Lk, kl, host = case
    call = make_call(B=B, H=H, D=64, Lq=Lq, Lk=Lk, seed=400 + B, mask_mode=_lib.SA_MASK_KEY_LEN,
                     key_len=np.asarray(kl, dtype=np.int32), name=f"stale_{name}")
    check_call(dev, call, True, (SMALL16, 64, 4, _lib.SA_BIAS_NONE, PACKED), poison_padding=True, host_copy=host)
