"""Randomised parity sweep over the C ABI's argument space (GPU), to the same bar as the fixed cases:
relative L2 and normwise max relative error <= 1e-5 against the PyTorch fp32 CPU path and float64,
with every output element outside the written rows left untouched.

The draws are seeded, so the cases are the same on every run. Attention calls cover every kernel
(flash MFMA at head dims 64/128 with and without key splits, the wide-head kernel at 256/512, the
generic kernel at other head dims and unaligned rows), packed and separate q/k/v, padded rows,
element offsets, output row padding, scales of either sign, dense and relative-position biases,
per-sequence key lengths (zero included) and boolean key masks. Linear calls cover the 64 x 64 MFMA
tile and the generic kernel (the large-grid tiles are exercised at full scale in test_linear_gpu.py),
ragged M/N/K, strides and offsets on every operand, alpha, the four activations and the three
epilogues. A second seeded draw adds wide-head calls with dense biases and key lengths or masks, and
head-dim-64 small launches whose short sequences pack (with the host copy of the key lengths). Sizes
keep the float64 oracle to a few seconds in total.
"""

from __future__ import annotations

import numpy as np
import pytest

from supra_attn import _lib
from supra_attn.linear_workloads import make_linear
from cases import make_call
from test_linear_gpu import run_checked as run_linear
from test_parity_gpu import run_checked as run_attention

pytestmark = pytest.mark.gpu

OPS_BUDGET = 12_000_000  # B*H*Lq*Lk*D per attention case


def _attention_cases(seed: int, n: int) -> list[dict]:
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        kind = rng.choice(["flash64", "flash128", "wide", "generic"], p=[0.4, 0.2, 0.15, 0.25])
        D = {"flash64": 64, "flash128": 128}.get(kind)
        if kind == "wide":
            D = int(rng.choice([256, 512]))
        elif kind == "generic":
            D = int(rng.choice([1, 8, 32, 48, 80, 96, 200]))
        B = int(rng.integers(1, 5))
        H = int(rng.integers(1, 5 if D <= 128 else 3))
        Lq = int(rng.integers(1, 300))
        Lk = int(rng.integers(1, 300))
        while B * H * Lq * Lk * D > OPS_BUDGET:
            if Lq >= Lk:
                Lq = max(1, Lq // 2)
            else:
                Lk = max(1, Lk // 2)
        kw = dict(B=B, H=H, D=D, Lq=Lq, Lk=Lk, seed=1000 + i, packed=bool(rng.random() < 0.3),
                  pad_cols=int(rng.choice([0, 0, 4, 8, 3])), q_off=int(rng.choice([0, 0, 4, 12, 1])),
                  o_off=int(rng.choice([0, 0, 8, 5])), ldo_pad=int(rng.choice([0, 0, 4, 7])))
        if rng.random() < 0.3:
            # multiples of the default 1/sqrt(D), up to the T5 call's 1 at D = 64 (logits of std 8):
            # beyond that the float32 logits alone carry more than the 1e-5 bar
            kw["scale"] = float(rng.choice([1.0, -0.7, 2.5, 8.0, 0.02])) / float(np.sqrt(D))
        if D <= 128 and rng.random() < 0.35:
            kw["bias_mode"] = int(rng.choice([_lib.SA_BIAS_DENSE, _lib.SA_BIAS_RELPOS]))
            kw["dense_bias_batched"] = bool(rng.random() < 0.5)
        r = rng.random()
        if r < 0.3:
            kw["mask_mode"] = _lib.SA_MASK_KEY_LEN
            kw["key_len"] = [int(x) for x in rng.integers(0, Lk + 1, size=B)]
        elif r < 0.5:
            kw["mask_mode"] = _lib.SA_MASK_KEY_MASK
            kw["key_mask_p"] = float(rng.choice([0.1, 0.5, 0.9]))
        kw["name"] = (f"rand{i}_B{B}H{H}D{D}q{Lq}k{Lk}_b{kw.get('bias_mode', 0)}m{kw.get('mask_mode', 0)}"
                      f"_pad{kw['pad_cols']}_qoff{kw['q_off']}{'_packed' if kw['packed'] else ''}")
        cases.append(kw)
    return cases


def _linear_cases(seed: int, n: int) -> list[dict]:
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        M = int(rng.integers(1, 600))
        N = int(rng.integers(1, 700))
        K = int(rng.choice([8, 24, 64, 96, 576, 1032, 36, 50]))  # K % 8 != 0 -> generic kernel
        kw = dict(seed=2000 + i, act=int(rng.integers(0, 4)), epi=int(rng.integers(0, 3)),
                  bias=bool(rng.random() < 0.8))
        if rng.random() < 0.4:
            kw.update(x_off=int(rng.choice([0, 4, 1])), ldx=K + int(rng.choice([0, 4, 12, 3])),
                      ldw=K + int(rng.choice([0, 8, 5])), y_off=int(rng.choice([0, 3, 16])),
                      ldy=N + int(rng.choice([0, 1, 32])))
        if kw["epi"] == _lib.SA_EPI_RESID_GATE:
            kw["gate_off"] = int(rng.integers(0, 64))
        if rng.random() < 0.3:
            kw["alpha"] = float(rng.choice([0.5, -1.0, 2.0]))
        cases.append(dict(name=f"lrand{i}_M{M}N{N}K{K}_a{kw['act']}e{kw['epi']}", M=M, N=N, K=K, kw=kw))
    return cases


def _wide_and_packed_cases(seed: int, n: int) -> list[dict]:
    """Half wide-head calls (D 256 / 512) with dense biases and either mask kind, half head-dim-64 small
    launches whose key lengths (many of at most 64 keys, with the host copy) pack their sequences."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        if i % 2 == 0:
            D = int(rng.choice([256, 512]))
            B, H = int(rng.integers(1, 4)), int(rng.integers(1, 3))
            Lq, Lk = int(rng.integers(1, 300)), int(rng.integers(1, 300))
            while B * H * Lq * Lk * D > OPS_BUDGET:
                Lq, Lk = max(1, Lq // 2), max(1, Lk // 2)
            kw = dict(B=B, H=H, D=D, Lq=Lq, Lk=Lk, seed=3000 + i, pad_cols=int(rng.choice([0, 4, 8])),
                      o_off=int(rng.choice([0, 8])), ldo_pad=int(rng.choice([0, 4])))
            if rng.random() < 0.7:
                kw["bias_mode"] = _lib.SA_BIAS_DENSE
                kw["dense_bias_batched"] = bool(rng.random() < 0.5)
            r = rng.random()
            if r < 0.4:
                kw["mask_mode"] = _lib.SA_MASK_KEY_LEN
                kw["key_len"] = [int(x) for x in rng.integers(0, Lk + 1, size=B)]
            elif r < 0.8:
                kw["mask_mode"] = _lib.SA_MASK_KEY_MASK
                kw["key_mask_p"] = float(rng.choice([0.1, 0.5, 0.9]))
        else:
            B = int(rng.integers(2, 17))
            H = int(rng.integers(1, max(2, min(13, 128 // B + 1))))
            Lk = int(rng.integers(96, 200))
            # more 16-query groups than the 256 CUs, at most 256 groups of 32 (the small-launch range):
            # with a = 256 // (B * H), exactly Lq in [16a + 1, 32a]
            a = 256 // (B * H)
            Lq = int(rng.integers(16 * a + 1, 32 * a + 1))
            kl = rng.integers(0, 65, size=B)
            long_ = rng.random(B) < 0.4
            kl[long_] = rng.integers(65, Lk + 1, size=int(long_.sum()))
            kw = dict(B=B, H=H, D=64, Lq=Lq, Lk=Lk, seed=3000 + i, mask_mode=_lib.SA_MASK_KEY_LEN,
                      key_len=[int(x) for x in kl], bias_mode=int(rng.choice([0, 1, 2])))
            if kw["bias_mode"] == _lib.SA_BIAS_RELPOS:
                kw["scale"] = 1.0 / 8.0
        kw["name"] = (f"rand_wp{i}_B{kw['B']}H{kw['H']}D{kw['D']}q{kw['Lq']}k{kw['Lk']}"
                      f"_b{kw.get('bias_mode', 0)}m{kw.get('mask_mode', 0)}")
        cases.append(kw)
    return cases


def _wide_round_cases(seed: int, n: int) -> list[dict]:
    """Wide-head calls whose query groups fill one round of workgroups (256 at head dim 512, 512 at
    256) and part of another: the plan runs the whole round unsplit and splits the groups past it
    into key chunks, or splits every group alike. Ragged Lq and Lk, dense biases, both mask kinds."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice([256, 512]))
        slots = 256 if D == 512 else 512
        B, H = int(rng.integers(1, 4)), int(rng.integers(1, 10))
        per = -(-slots // (B * H))  # 32-query groups per (sequence, head) that just pass one round
        Lq = 32 * int(rng.integers(per, per + max(2, per // 4) + 1)) - int(rng.integers(0, 32))
        Lq = max(Lq, 32 * (per - 1) + 1)
        Lk = int(rng.integers(33, 400))
        kw = dict(B=B, H=H, D=D, Lq=Lq, Lk=Lk, seed=4000 + i, o_off=int(rng.choice([0, 8])),
                  pad_cols=int(rng.choice([0, 4])))
        if rng.random() < 0.5:
            kw["bias_mode"] = _lib.SA_BIAS_DENSE
            kw["dense_bias_batched"] = bool(rng.random() < 0.5)
        r = rng.random()
        if r < 0.4:
            kw["mask_mode"] = _lib.SA_MASK_KEY_LEN
            kw["key_len"] = [int(x) for x in rng.integers(0, Lk + 1, size=B)]
        elif r < 0.8:
            kw["mask_mode"] = _lib.SA_MASK_KEY_MASK
            kw["key_mask_p"] = float(rng.choice([0.1, 0.5, 0.9]))
        kw["name"] = (f"rand_wr{i}_B{B}H{H}D{D}q{Lq}k{Lk}_b{kw.get('bias_mode', 0)}m{kw.get('mask_mode', 0)}")
        cases.append(kw)
    return cases


ATTENTION = _attention_cases(seed=2026, n=40)
WIDE_PACKED = _wide_and_packed_cases(seed=2028, n=24)
WIDE_ROUNDS = _wide_round_cases(seed=2029, n=8)
LINEAR = _linear_cases(seed=2027, n=24)


@pytest.mark.parametrize("case", ATTENTION, ids=[c["name"] for c in ATTENTION])
def test_random_attention(dev, case):
    kw = dict(case)
    key_len = kw.pop("key_len", None)
    call = make_call(key_len=key_len, **kw)
    run_attention(dev, call, check_fp64=call.B * call.H * call.Lq * call.Lk * call.D <= 4_000_000)


def test_draw_reaches_every_kernel():
    """The seeded draw exercises each kernel family (the library's own selection, host only)."""
    fake = 0x7F0000000000
    names = set()
    for case in ATTENTION:
        kw = dict(case)
        key_len = kw.pop("key_len", None)
        call = make_call(key_len=key_len, **kw)
        a = dict(call.args)
        args = _lib.AttnArgs(B=call.B, H=call.H, D=call.D, Lq=call.Lq, Lk=call.Lk, q=fake, k=fake + (1 << 34),
                             v=fake + (2 << 34), o=fake + (3 << 34), scale=call.scale, bias_mode=call.bias_mode,
                             bias=fake + (4 << 34), bucket_lut=fake + (5 << 34), num_buckets=32,
                             mask_mode=call.mask_mode, key_len=fake + (6 << 34), key_mask=fake + (7 << 34), **a)
        names.add(_lib.kernel_name(args).split("_split")[0])
    assert {"flash_mfma_d64", "flash_mfma_d128", "generic"} <= names, names
    assert any(n.startswith("wide") for n in names) and any(n.startswith("flash_small") for n in names), names


@pytest.mark.parametrize("case", WIDE_PACKED, ids=[c["name"] for c in WIDE_PACKED])
def test_random_wide_and_packed(dev, case):
    kw = dict(case)
    key_len = kw.pop("key_len", None)
    call = make_call(key_len=key_len, **kw)
    run_attention(dev, call, check_fp64=call.B * call.H * call.Lq * call.Lk * call.D <= 4_000_000)


def test_wide_and_packed_draw_reaches_its_variants():
    """The second draw reaches the wide kernels with a dense bias under both mask kinds and the packed
    small-launch variant (host only, with the host copy of the key lengths as the GPU run passes it)."""
    from variant_cases import fake_args

    variants = set()
    for case in WIDE_PACKED:
        kw = dict(case)
        key_len = kw.pop("key_len", None)
        call = make_call(key_len=key_len, **kw)
        variants.add(_lib.plan(fake_args(call, True)).variant())
    wide = {(v[1], v[3], v[4]) for v in variants if v[0] == _lib.SA_KERNEL_WIDE}
    assert {(d, _lib.SA_BIAS_DENSE, _lib.SA_MASK_KEY_LEN) for d in (256, 512)} & wide, wide
    assert {(d, _lib.SA_BIAS_DENSE, _lib.SA_MASK_KEY_MASK) for d in (256, 512)} & wide, wide
    packed = [v for v in variants if v[0] == _lib.SA_KERNEL_FLASH_SMALL16 and v[4] == 3]
    assert len({v[3] for v in packed}) >= 2, variants


@pytest.mark.parametrize("case", WIDE_ROUNDS, ids=[c["name"] for c in WIDE_ROUNDS])
def test_random_wide_past_one_round(dev, case):
    kw = dict(case)
    key_len = kw.pop("key_len", None)
    run_attention(dev, make_call(key_len=key_len, **kw), check_fp64=False)


def test_wide_round_draw_reaches_split_tails():
    """The third draw reaches plans that split only the groups past the whole round, at both head
    dims, with a dense bias, key lengths and a key mask among them (host only)."""
    from variant_cases import fake_args

    tails = []
    for case in WIDE_ROUNDS:
        kw = dict(case)
        key_len = kw.pop("key_len", None)
        call = make_call(key_len=key_len, **kw)
        p = _lib.plan(fake_args(call, False))
        assert p.kernel == _lib.SA_KERNEL_WIDE, call.name
        if p.tail_kernel == _lib.SA_KERNEL_WIDE:
            tails.append((call.D, call.bias_mode, call.mask_mode))
    assert {d for d, _, _ in tails} == {256, 512}, tails
    assert {m for _, _, m in tails} >= {_lib.SA_MASK_KEY_LEN, _lib.SA_MASK_KEY_MASK}, tails
    assert any(b == _lib.SA_BIAS_DENSE for _, b, _ in tails), tails


@pytest.mark.parametrize("case", LINEAR, ids=[c["name"] for c in LINEAR])
def test_random_linear(dev, case):
    call = make_linear(case["name"], case["M"], case["N"], case["K"], **case["kw"])
    run_linear(dev, call)
