"""Host-only: the variant cases reach every compiled flash-kernel variant, each with at least two
loop steps for every splitting wave and ragged query and key lengths (sa_attention_plan, no GPU)."""

from __future__ import annotations

import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

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


def wide_plan(B, H, D, Lq, Lk):
    a = _lib.AttnArgs(B=B, H=H, D=D, Lq=Lq, Lk=Lk, q=0x7F0000000000, k=0x7F4000000000, v=0x7F8000000000,
                      o=0x7FC000000000, ldq=H * D, ldk=H * D, ldv=H * D, sq=Lq * H * D, sk=Lk * H * D,
                      sv=Lk * H * D, so=Lq * H * D, scale=D ** -0.5)
    return _lib.plan(a)


@pytest.mark.parametrize("D,B,H,L,chunks,keys", [
    (512, 1, 1, 1024, 8, 128),    # the VAE call: 32 groups x 8 chunks of one round, 256 workgroups
    (512, 2, 1, 1024, 4, 256),    # 64 groups x 4 chunks
    (512, 1, 8, 1024, 1, 1024),   # 256 groups fill the CUs unsplit
    (512, 1, 1, 2304, 3, 768),    # 216 workgroups in one round, not 4 chunks = 288 in two
    (512, 1, 1, 1536, 4, 384),    # 192 workgroups of 12 blocks, not 6 chunks = 288 of 8 blocks
    (512, 1, 1, 4096, 2, 2048),
    (512, 1, 1, 5120, 3, 1792),   # two rounds of 56 blocks beat one round of 160 (1 chunk) or two of 80
    (256, 1, 1, 1024, 16, 64),    # two workgroups per CU: 512 slots
    (256, 1, 1, 2304, 7, 352),    # 504 workgroups, not 8 chunks = 576 in two rounds
    (256, 1, 1, 9216, 3, 3072),   # 864 workgroups of 96 blocks in two rounds
    (256, 1, 1, 16352, 1, 16352), # 511 groups fill the 512 slots unsplit (2 chunks: two rounds)
])
def test_wide_key_chunks_minimise_the_rounds(D, B, H, L, chunks, keys):
    p = wide_plan(B, H, D, L, L)
    assert (p.kernel, p.head_dim) == (_lib.SA_KERNEL_WIDE, D)
    assert (p.key_chunks, p.keys_per_step, p.tail_kernel) == (chunks, keys, 0)
    groups = B * H * ((L + 31) // 32)
    assert p.workgroups == groups * chunks
    rec = (32 * D + 64) * 4
    assert p.workspace_bytes == (groups * chunks * rec if chunks > 1 else 0)


@pytest.mark.parametrize("D,B,H,L,whole,tail_chunks", [
    (512, 1, 1, 9216, 256, 8),    # 288 groups: 256 unsplit, then 32 in 8 chunks of 36 blocks
    (512, 1, 9, 1024, 256, 8),    # 9 heads of the VAE size: 288 groups likewise, chunks of 4 blocks
    (512, 1, 1, 8448, 256, 14),   # 8 groups past the round, 14 chunks of 20 blocks
    (512, 2, 9, 512, 256, 4),     # the 32 groups past the round span two heads of the second sequence
    (256, 1, 17, 1024, 512, 16),  # 544 groups for 512 slots
])
def test_wide_groups_past_whole_rounds_are_split_alone(D, B, H, L, whole, tail_chunks):
    """Groups that fill whole rounds and a few more: the whole rounds run unsplit (the main
    launch) and only the groups past them are split into key chunks (a second launch and the
    merge), instead of a second round of whole groups."""
    p = wide_plan(B, H, D, L, L)
    groups = B * H * ((L + 31) // 32)
    unit = 128 if D == 512 else 32
    assert (p.kernel, p.key_chunks, p.keys_per_step) == (_lib.SA_KERNEL_WIDE, 1, -(-L // unit) * unit)
    assert p.workgroups == whole and (p.tail_kernel, p.tail_key_split) == (_lib.SA_KERNEL_WIDE, tail_chunks)
    assert p.tail_workgroups == (groups - whole) * tail_chunks
    assert p.workspace_bytes == (groups - whole) * tail_chunks * (32 * D + 64) * 4


@settings(max_examples=300, deadline=None)
@given(D=st.sampled_from([256, 512]), B=st.integers(1, 4), H=st.integers(1, 16), Lq=st.integers(1, 20000),
       Lk=st.integers(1, 20000))
def test_every_wide_plan_fits_the_allocation_free_scratch(D, B, H, Lq, Lk):
    """Whatever the shape, the key chunks cover the keys in whole rounds of the kernel, at most 16 of
    them, the launches cover every query group once, and the merge records fit the allocation-free
    entry point's scratch (so that entry point takes every wide-head call the workspace entry point
    takes)."""
    p = wide_plan(B, H, D, Lq, Lk)
    unit = 128 if D == 512 else 32
    groups = B * H * ((Lq + 31) // 32)
    assert 1 <= p.key_chunks <= 16 and p.keys_per_step % unit == 0
    assert p.key_chunks == -(-Lk // p.keys_per_step) and (p.key_chunks - 1) * p.keys_per_step < Lk
    assert p.workspace_bytes <= _lib.SA_NOALLOC_SCRATCH_BYTES
    if p.tail_kernel:  # whole rounds of unsplit groups, then the groups past them in chunks
        slots = 256 if D == 512 else 512
        assert p.tail_kernel == _lib.SA_KERNEL_WIDE and p.key_chunks == 1 and 2 <= p.tail_key_split <= 16
        assert p.workgroups == groups // slots * slots and 0 < groups - p.workgroups < slots
        assert p.tail_workgroups == (groups - p.workgroups) * p.tail_key_split
        assert p.workspace_bytes == p.tail_workgroups * (32 * D + 64) * 4
    else:
        assert p.workgroups == groups * p.key_chunks
        assert (p.workspace_bytes > 0) == (p.key_chunks > 1)
