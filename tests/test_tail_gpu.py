"""GPU parity of flash launches whose last round holds few units: more units (128-query tiles) than
the 4-per-CU kernel holds at once, with few enough left over for one workgroup per CU of the
small-launch kernel (32-query groups) or of the 2-way key-split flash kernel (64-query units). The
first launch covers the leading units; the rest go to a second launch, or, after a single round, run
as 64-query units inside it, on its first workgroups after their own units. Every output row is
checked against the PyTorch fp32 CPU path and the float64 brute force (1e-5)."""

from __future__ import annotations

import numpy as np
import pytest

from cases import make_call
from oracle import attention as orc
from supra_attn import _lib
from supra_attn.runner import Staged

pytestmark = pytest.mark.gpu

TOL = 1e-5
SENTINEL = np.float32(-12345.5)


def tail_units(call) -> int:
    cus = 256  # MI355X
    tiles = call.B * call.H * ((call.Lq + 127) // 128)
    rest = tiles % (4 * cus)
    return rest if tiles > 4 * cus and 2 * rest <= cus else 0


@pytest.mark.parametrize("B,Lq,Lk", [
    (57, 256, 256),   # 1026 units: a tail of two (small-launch kernel)
    (60, 256, 256),   # 1080 units: a tail of 56 (224 small workgroups)
    (60, 250, 250),   # ragged
    (57, 200, 230),   # 7 groups of 32 per (b, h): the tail starts inside a head
    (64, 256, 256),   # the batch-64 DiT call: 128 left, 2-way key-split units folded into the round
    (61, 200, 230),   # 74 left, folded split units, ragged 64-query units
    (118, 256, 250),  # two rounds and 76 left: a second launch of the split kernel
])
def test_tail_launch_parity(dev, B, Lq, Lk):
    call = make_call(B=B, H=9, D=64, Lq=Lq, Lk=Lk, seed=B * 7 + Lq, packed=(Lq == Lk), name=f"tail_B{B}_q{Lq}_k{Lk}")
    print(f"[case] {call.name}", flush=True)
    st = Staged(dev, call, out_fill=SENTINEL)
    try:
        plan = _lib.plan(st.args)
        assert plan.kernel == _lib.SA_KERNEL_FLASH
        n_tail = tail_units(call)
        assert n_tail > 0
        assert plan.workgroups == B * 9 * ((Lq + 127) // 128) - n_tail
        small = 4 * n_tail <= 256
        assert (plan.tail_kernel, plan.tail_key_split) == ((_lib.SA_KERNEL_FLASH_SMALL, 4) if small
                                                           else (_lib.SA_KERNEL_FLASH, 2))
        tiles = B * 9 * ((Lq + 127) // 128)
        assert plan.tail_folded == (0 if small or tiles >= 2 * 1024 else 1)
        out = st.run()
    finally:
        st.release()
    got = orc.output_view(out, call)
    e = orc.errors(got, orc.reference_torch(call))
    assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, f"{call.name} vs torch fp32: {e}"
    e64 = orc.errors(got, orc.reference_fp64(call))
    assert e64["rel_l2"] <= TOL and e64["max_rel"] <= TOL, f"{call.name} vs fp64: {e64}"
    ldo = call.args.get("ldo", 0) or call.H * call.D
    written = np.zeros(out.size, dtype=bool)
    idx = orc.heads(np.arange(out.size), B=call.B, L=call.Lq, H=call.H, D=call.D, off=call.args.get("o_off", 0),
                    ld=ldo, sb=call.args.get("so", 0))
    written[idx.reshape(-1)] = True
    assert (out.reshape(-1)[~written] == SENTINEL).all()


def _fold_draw(seed: int, n: int) -> list[dict]:
    """Seeded calls whose units fill one round and part of a second that folds into it (more than 64
    and at most 128 of them past the 1024 slots): any batch, head count and ragged lengths, packed or
    separate q/k/v, padded rows and element offsets."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        B, H = int(rng.integers(1, 130)), int(rng.integers(1, 17))
        Lq, Lk = int(rng.integers(129, 700)), int(rng.integers(33, 400))
        tiles = B * H * ((Lq + 127) // 128)
        if not 1024 + 64 < tiles <= 1024 + 128 or B * H * Lq * Lk > 60_000_000:
            continue
        out.append(dict(B=B, H=H, D=64, Lq=Lq, Lk=Lk, seed=5000 + len(out), packed=bool(rng.random() < 0.5),
                        pad_cols=int(rng.choice([0, 4, 8])), q_off=int(rng.choice([0, 4, 12])),
                        o_off=int(rng.choice([0, 8])), ldo_pad=int(rng.choice([0, 4])),
                        name=f"fold_B{B}H{H}q{Lq}k{Lk}"))
    return out


FOLD_DRAW = _fold_draw(seed=2031, n=6)


@pytest.mark.parametrize("case", FOLD_DRAW, ids=[c["name"] for c in FOLD_DRAW])
def test_folded_launch_random_shapes(dev, case):
    call = make_call(**case)
    print(f"[case] {call.name}", flush=True)
    st = Staged(dev, call, out_fill=SENTINEL)
    try:
        plan = _lib.plan(st.args)
        assert (plan.kernel, plan.tail_folded) == (_lib.SA_KERNEL_FLASH, 1), call.name
        out = st.run()
    finally:
        st.release()
    e = orc.errors(orc.output_view(out, call), orc.reference_torch(call))
    assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, f"{call.name}: {e}"
    ldo = call.args.get("ldo", 0) or call.H * call.D
    written = np.zeros(out.size, dtype=bool)
    idx = orc.heads(np.arange(out.size), B=call.B, L=call.Lq, H=call.H, D=call.D, off=call.args.get("o_off", 0),
                    ld=ldo, sb=call.args.get("so", 0))
    written[idx.reshape(-1)] = True
    assert (out.reshape(-1)[~written] == SENTINEL).all()
