"""The balanced sequence schedule (sa_attn_args.key_len_host, GPU).

A host copy of the per-sequence key lengths lets the library order the sequences so that the L2
domains and their CUs get even shares of key blocks (longest first, balanced over the domains, then a
bounded swap search per domain). It changes only which workgroup runs which sequence, so the output
must be bit-identical with the host copy, without it, and with a stale (wrong) host copy - the
kernel reads the device key lengths for the arithmetic - and must match the oracle at the usual
bar. Cases: the sweep's batch-64 cross-attention (searched), batch 24 (also a multiple of 8), batch
128 with two query tiles (16 sequences per domain), batch 58 with ragged queries (1044 units over
unequal L2 domains, plain longest-first order), batch 13 (plain longest-first order) and batch 2
(below the batch the schedule is used for; there the host copy may instead pack a short sequence
into the 16-query small-launch kernel, which runs other arithmetic: that case is held to the
oracle's bar, not to bits)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as orc
from supra_attn import _lib, workloads
from supra_attn.runner import Staged
from cases import make_call

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _calls():
    yield "sweep_cross_b64", workloads.SweepData(blocks=1).block(0)[1]
    for B, H, Lq, seed in ((24, 9, 256, 31), (128, 2, 128, 34), (58, 9, 250, 35), (13, 9, 256, 32), (2, 9, 256, 33)):
        rng = np.random.default_rng(seed)
        key_len = [int(x) for x in rng.integers(0, 129, size=B)]  # zero-length sequences included
        key_len[0] = 128
        yield f"B{B}", make_call(B=B, H=H, D=64, Lq=Lq, Lk=128, seed=seed, mask_mode=_lib.SA_MASK_KEY_LEN,
                                 key_len=key_len)


CALLS = list(_calls())


def _packed(variant) -> bool:
    """The 16-query small-launch kernel with sequences packed by their host key lengths."""
    return variant[0] == _lib.SA_KERNEL_FLASH_SMALL16 and variant[4] == _lib.SA_MASK_VARIANT_KEY_LEN_SCHEDULED


@pytest.mark.parametrize("name,call", CALLS, ids=[c[0] for c in CALLS])
def test_schedule_is_bitwise_neutral(dev, name, call):
    """Bit for bit wherever the host copy only orders the flash kernel's sequences. A small launch
    whose host copy packs short sequences (flash_small16.hip) runs other arithmetic than the same call
    without it (another kernel, or fewer waves per 16-query group): those runs match the oracle at the
    usual bar instead."""
    print(f"[schedule case] {name} B={call.B} Lq={call.Lq} kernel=", end="", flush=True)
    outs, plans = {}, {}
    for mode in ("host", "none", "stale"):
        st = Staged(dev, call, out_fill=np.nan, host_key_len=mode != "none")
        try:
            if mode == "stale":  # a wrong host copy: reversed lengths, so the order is wrong too
                st.key_len_host = np.ascontiguousarray(st.key_len_host[::-1])
                st.args.key_len_host = st.key_len_host.ctypes.data
            plans[mode] = _lib.plan(st.args).variant()
            if mode == "host":
                print(st.kernel, flush=True)
            outs[mode] = st.run()
        finally:
            st.release()
    ref = orc.reference_torch(call)
    for mode in ("none", "stale"):
        same_arithmetic = plans[mode][:4] == plans["host"][:4] and not _packed(plans[mode]) and not _packed(plans["host"])
        if same_arithmetic:
            np.testing.assert_array_equal(outs[mode].view(np.uint32), outs["host"].view(np.uint32), err_msg=mode)
        else:
            e = orc.errors(orc.output_view(outs[mode], call), ref)
            assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, (mode, plans[mode], e)
    e = orc.errors(orc.output_view(outs["host"], call), ref)
    assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, e


RANDOM_BATCHES = [8, 16, 40, 57, 72, 96, 99, 200, 255, 256]


@pytest.mark.parametrize("B", RANDOM_BATCHES)
def test_schedule_random_batches(dev, B):
    """The schedule over batch sizes that exercise every path of its construction (18 units of 128
    queries per sequence): one sequence per L2 domain (B = 8, no swaps), the bounded swap search
    (16-72), a search too large for its budget (the round-robin deal of the longest-first order,
    96-256), batches that 8 does not divide (57, 99: dealt over the domains' rank ranges and searched;
    255: dealt, beyond the search budget), with random lengths including zero and full ones:
    bit-identical to the launch-order run and within the usual bar of the oracle."""
    rng = np.random.default_rng(100 + B)
    key_len = rng.integers(0, 129, size=B).astype(np.int32)
    key_len[0], key_len[-1] = 0, 128
    call = make_call(B=B, H=9, D=64, Lq=256, Lk=128, seed=B, mask_mode=_lib.SA_MASK_KEY_LEN, key_len=key_len)
    print(f"[schedule random] B={B}", flush=True)
    outs = {}
    for mode in ("host", "none"):
        st = Staged(dev, call, out_fill=np.nan, host_key_len=mode == "host")
        try:
            outs[mode] = st.run()
        finally:
            st.release()
    np.testing.assert_array_equal(outs["none"].view(np.uint32), outs["host"].view(np.uint32))
    e = orc.errors(orc.output_view(outs["host"], call), orc.reference_torch(call))
    assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, e
