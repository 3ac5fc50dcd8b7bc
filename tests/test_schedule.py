"""The host sequence schedule (sa_attn_args.key_len_host) as sa_attention_plan reports it (no GPU).

The library orders the sequences of a key-length call before launching the flash kernel: longest
first by key blocks, balanced over the 8 L2 domains (domain x takes the ranks [x*B/8, (x+1)*B/8)),
then a bounded search per domain against a model of how the hardware deals workgroups to CUs.
These tests read the order back through the revision-2 plan fields and check what must hold of it
whatever the search finds: a permutation, equal work per domain, the model's heaviest CU no worse
than the plain round-robin deal (and at the bound for the benchmark's sweep), the documented
fallbacks exactly, and no schedule where none is used. The GPU tests check that the order never
changes a result (tests/test_schedule_gpu.py)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from supra_attn import _lib, workloads

CUS = 256  # the plan query's CU count without a GPU (the MI355X value)


def plan_for(key_len, H=9, Lq=256, Lk=128, host=True) -> _lib.AttnPlan:
    B = len(key_len)
    kl = np.ascontiguousarray(key_len, dtype=np.int32)
    hd = H * 64
    a = _lib.AttnArgs(B=B, H=H, D=64, Lq=Lq, Lk=Lk, q=1 << 20, k=1 << 34, v=1 << 38, o=1 << 42, ldq=hd, ldk=hd, ldv=hd,
                      ldo=hd, sq=Lq * hd, sk=Lk * hd, sv=Lk * hd, so=Lq * hd, scale=0.125,
                      mask_mode=_lib.SA_MASK_KEY_LEN, key_len=1 << 46, key_len_host=kl.ctypes.data if host else None)
    a._keep = kl
    return _lib.plan(a)


def blocks(key_len, Lk=128):
    return (np.clip(np.asarray(key_len), 0, Lk) + 31) // 32


def longest_first(key_len, Lk=128):
    nb = blocks(key_len, Lk)
    return sorted(range(len(nb)), key=lambda i: -nb[i])  # Python's sort is stable


def heaviest_cu(order, nb, units, C=CUS // 8):
    """The dispatch model, per L2 domain: local workgroup j of the first residency (4 per CU) on CU
    j % C, each later one on the CU with the fewest key blocks so far; returns the heaviest CU's."""
    B = len(order)
    per = B // 8
    worst = 0
    for x in range(8):
        load = np.zeros(C, dtype=np.int64)
        j = 0
        for r in range(x * per, (x + 1) * per):
            for _ in range(units):
                c = j % C if j < 4 * C else int(np.argmin(load))
                load[c] += nb[order[r]]
                j += 1
        worst = max(worst, int(load.max()))
    return worst


def test_sweep_schedule_is_balanced():
    kl = workloads.sweep_key_lengths()
    p = plan_for(kl)
    assert p.mask_variant == _lib.SA_MASK_VARIANT_KEY_LEN_SCHEDULED
    assert p.order_n == 64
    order = list(p.sequence_order[:64])
    assert sorted(order) == list(range(64))
    assert all(v == 0 for v in p.sequence_order[64:])
    nb = blocks(kl)
    sums = [int(sum(nb[order[r]] for r in range(8 * x, 8 * x + 8))) for x in range(8)]
    assert max(sums) - min(sums) <= 1, sums
    units = 9 * 2  # heads x 128-query tiles per sequence
    lf = longest_first(kl)
    round_robin = [None] * 64
    for j, i in enumerate(lf):
        round_robin[(j % 8) * 8 + j // 8] = i
    total = int(nb.sum()) * units
    bound = -(-total // CUS)
    got = heaviest_cu(order, nb, units)
    assert got <= heaviest_cu(round_robin, nb, units)
    assert got == bound == 12


@pytest.mark.parametrize("B", [16, 24, 40, 64, 72])
def test_searched_schedules(B):
    rng = np.random.default_rng(B)
    kl = rng.integers(0, 129, size=B)
    p = plan_for(kl)
    order = list(p.sequence_order[:p.order_n])
    assert p.order_n == B and sorted(order) == list(range(B))
    nb = blocks(kl)
    per = B // 8
    lf = longest_first(kl)
    round_robin = [None] * B
    for j, i in enumerate(lf):
        round_robin[(j % 8) * per + j // 8] = i
    assert heaviest_cu(order, nb, 18) <= heaviest_cu(round_robin, nb, 18)
    # every domain gets B/8 sequences, and the domains' key blocks come out within one sequence's
    sums = [int(sum(nb[order[r]] for r in range(per * x, per * (x + 1)))) for x in range(8)]
    assert max(sums) - min(sums) <= int(nb.max())


def test_fallbacks_are_longest_first():
    rng = np.random.default_rng(7)
    # B not a multiple of 8: plain longest first (stable)
    kl = rng.integers(0, 129, size=13)
    assert list(plan_for(kl).sequence_order[:13]) == longest_first(kl)
    # one sequence per domain: nothing to search, the round-robin deal is the longest-first order
    kl = rng.integers(0, 129, size=8)
    kl[0] = 1
    assert list(plan_for(kl).sequence_order[:8]) == longest_first(kl)
    # 32 sequences of 18 units per domain: one pass of the search exceeds its budget, so the
    # longest-first order is dealt round-robin over the domains
    kl = rng.integers(0, 129, size=256)
    lf = longest_first(kl)
    want = [None] * 256
    for j, i in enumerate(lf):
        want[(j % 8) * 32 + j // 8] = i
    assert list(plan_for(kl).sequence_order[:256]) == want


def test_lengths_outside_the_key_range_schedule_as_clamped():
    rng = np.random.default_rng(11)
    kl = rng.integers(-50, 300, size=64)
    a = list(plan_for(kl).sequence_order[:64])
    b = list(plan_for(np.clip(kl, 0, 128)).sequence_order[:64])
    assert a == b and sorted(a) == list(range(64))


def test_no_schedule_where_none_is_used():
    rng = np.random.default_rng(5)
    kl = rng.integers(1, 129, size=64)
    p = plan_for(kl, host=False)  # no host copy
    assert p.order_n == 0 and p.mask_variant == _lib.SA_MASK_KEY_LEN
    assert all(v == 0 for v in p.sequence_order)
    assert plan_for(rng.integers(1, 129, size=7)).order_n == 0  # below 8 sequences
    # equal lengths: the schedule is the identity, so the plain key-length kernel runs
    p = plan_for(np.full(64, 77))
    assert p.order_n == 0 and p.mask_variant == _lib.SA_MASK_KEY_LEN


def test_cached_schedules_repeat():
    rng = np.random.default_rng(9)
    sets = [rng.integers(0, 129, size=64) for _ in range(6)]
    first = [list(plan_for(kl).sequence_order[:64]) for kl in sets]  # more sets than the cache holds
    again = [list(plan_for(kl).sequence_order[:64]) for kl in reversed(sets)]
    assert first == list(reversed(again))


def test_plan_revision_1_is_accepted_and_not_overrun():
    """A revision-1 sa_attn_plan (ending at tail_workgroups) still works; nothing past it is written."""
    v1 = _lib.AttnPlan.order_n.offset
    buf = (ctypes.c_uint8 * ctypes.sizeof(_lib.AttnPlan))(*([0xAB] * ctypes.sizeof(_lib.AttnPlan)))
    plan = _lib.AttnPlan.from_buffer(buf)
    plan.struct_size = v1
    kl = np.ascontiguousarray(workloads.sweep_key_lengths(), dtype=np.int32)
    hd = 9 * 64
    a = _lib.AttnArgs(B=64, H=9, D=64, Lq=256, Lk=128, q=1 << 20, k=1 << 34, v=1 << 38, o=1 << 42, ldq=hd, ldk=hd,
                      ldv=hd, ldo=hd, sq=256 * hd, sk=128 * hd, sv=128 * hd, so=256 * hd, scale=0.125,
                      mask_mode=_lib.SA_MASK_KEY_LEN, key_len=1 << 46, key_len_host=kl.ctypes.data)
    assert _lib.load().sa_attention_plan(ctypes.byref(a), ctypes.byref(plan)) == _lib.SA_OK
    assert plan.kernel == _lib.SA_KERNEL_FLASH and plan.struct_size == v1
    assert bytes(buf[v1:]) == b"\xab" * (len(buf) - v1)
    vplan = _lib.AttnPlan.from_buffer(buf)
    buf[v1:] = [0xAB] * (len(buf) - v1)
    vplan.struct_size = v1
    assert _lib.load().sa_attention_variant(0, ctypes.byref(vplan)) == _lib.SA_OK
    assert bytes(buf[v1:]) == b"\xab" * (len(buf) - v1)
