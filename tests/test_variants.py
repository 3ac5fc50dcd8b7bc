"""Host-only: the variant cases reach every compiled flash-kernel variant, each with at least two
loop steps for every splitting wave and ragged query and key lengths (sa_attention_plan, no GPU)."""

from __future__ import annotations

import pytest

from supra_attn import _lib
from variant_cases import (SMALL, SMALL16, WIDE_SHAPES, call_for, fake_args, flash_variants, steps_per_wave,
                           variant_id, wide_call_for, wide_variants)


def test_every_compiled_variant_is_enumerated_once():
    vs = _lib.variants()
    flash = flash_variants()
    assert len(flash) == len(set(flash))
    assert sum(v[0] == _lib.SA_KERNEL_FLASH for v in flash) == 48  # D 64, 128 x splits 1, 2 x 3 biases x 4 masks
    assert sum(v[0] == SMALL for v in flash) == 9                  # 4 waves x 3 biases x 3 masks
    assert sum(v[0] == SMALL16 for v in flash) == 12               # 16-query groups: 3 masks + packed key lengths
    assert sum(v.kernel == _lib.SA_KERNEL_WIDE for v in vs) == 12  # D 256, 512 x 2 biases x 3 masks
    assert sum(v.kernel == _lib.SA_KERNEL_GENERIC for v in vs) == 1
    assert all(v.name for v in vs)


@pytest.mark.parametrize("variant", flash_variants(), ids=variant_id)
def test_case_selects_its_variant(variant):
    kernel, D, split, bias, mask = variant
    call, host = call_for(*variant)
    plan = _lib.plan(fake_args(call, host))
    assert plan.variant() == variant, call.name
    assert plan.keys_per_step == 32 * split
    first, last = steps_per_wave(call, split)
    assert last >= 2, call.name
    assert call.Lq % 32 != 0 and call.Lk % 32 != 0, "lengths must be ragged"
    assert plan.workgroups > 0 and plan.workspace_bytes == 0


def test_plan_of_the_wide_and_generic_kernels():
    vae = _lib.AttnArgs(B=1, H=1, D=512, Lq=1024, Lk=1024, q=0x7F0000000000, k=0x7F0001000000, v=0x7F0002000000,
                        o=0x7F0003000000, ldq=512, ldk=512, ldv=512, scale=0.0442)
    p = _lib.plan(vae)
    assert p.kernel == _lib.SA_KERNEL_WIDE and p.head_dim == 512 and p.key_chunks >= 2
    assert p.workspace_bytes == _lib.workspace_bytes(vae) > 0
    assert p.workgroups == 32 * p.key_chunks
    gen = _lib.AttnArgs(B=1, H=2, D=48, Lq=10, Lk=10, q=0x7F0000000000, k=0x7F0001000000, v=0x7F0002000000,
                        o=0x7F0003000000, ldq=96, ldk=96, ldv=96, scale=0.1)
    p = _lib.plan(gen)
    assert (p.kernel, p.head_dim, p.name) == (_lib.SA_KERNEL_GENERIC, 48, b"generic")


def test_plan_rejects_like_the_call():
    bad = _lib.AttnArgs(B=0, H=1, D=64, Lq=1, Lk=1, q=16, k=16, v=16, o=4096, ldq=64, ldk=64, ldv=64, scale=1.0)
    out = _lib.AttnPlan()
    import ctypes

    assert _lib.load().sa_attention_plan(ctypes.byref(bad), ctypes.byref(out)) == _lib.SA_ERR_INVALID
    assert _lib.load().sa_last_status() == _lib.SA_ERR_INVALID
    small = _lib.AttnPlan()
    small.struct_size = 8
    good = _lib.AttnArgs(B=1, H=1, D=64, Lq=1, Lk=1, q=16, k=16, v=16, o=4096, ldq=64, ldk=64, ldv=64, scale=1.0)
    assert _lib.load().sa_attention_plan(ctypes.byref(good), ctypes.byref(small)) == _lib.SA_ERR_INVALID


@pytest.mark.parametrize("variant", wide_variants(), ids=lambda v: "wide_d%d_b%d_m%d" % (v[1], v[3], v[4]))
def test_wide_case_selects_its_variant(variant):
    call = wide_call_for(*variant)
    plan = _lib.plan(fake_args(call, False))
    assert plan.variant() == variant, call.name
    assert call.Lq % 32 != 0 and call.Lk % 32 != 0, "lengths must be ragged"
    # the key-chunk split (merge kernel, workspace) and the single-chunk path both run for each head dim
    assert (plan.key_chunks > 1) == (plan.workspace_bytes > 0)


def test_wide_cases_cover_split_and_unsplit():
    chunks = {}
    for v in wide_variants():
        plan = _lib.plan(fake_args(wide_call_for(*v), False))
        chunks.setdefault(v[1], set()).add(plan.key_chunks > 1)
    assert chunks == {256: {True, False}, 512: {True, False}}
    assert len(WIDE_SHAPES) == 6
