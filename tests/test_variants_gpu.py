"""GPU parity of every compiled flash and small-launch kernel variant <kernel, D, key_split, bias, mask>, each at a shape
that real callers give it, with ragged lengths and at least two loop steps per splitting wave,
against the PyTorch fp32 CPU path and the float64 brute force (both <= 1e-5, relative L2 and
normwise max). The cases come from variant_cases.py; test_variants.py shows on the host that they
reach every compiled variant."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as orc
from supra_attn import _lib
from supra_attn.runner import Staged
from cases import make_call
from variant_cases import call_for, flash_variants, variant_id

pytestmark = pytest.mark.gpu

TOL = 1e-5
SENTINEL = np.float32(-12345.5)


@pytest.mark.parametrize("variant", flash_variants(), ids=variant_id)
def test_variant_parity(dev, variant):
    call, host = call_for(*variant)
    check_call(dev, call, host, variant)


@pytest.mark.parametrize("kernel,Lq", [(_lib.SA_KERNEL_FLASH_SMALL, 200), (_lib.SA_KERNEL_FLASH_SMALL16, 100)],
                         ids=["small", "small16"])
@pytest.mark.parametrize("bias,batched,mask", [
    (_lib.SA_BIAS_DENSE, False, _lib.SA_MASK_NONE),
    (_lib.SA_BIAS_DENSE, True, _lib.SA_MASK_KEY_MASK),
    (_lib.SA_BIAS_NONE, False, _lib.SA_MASK_KEY_MASK),
], ids=["dense", "dense_batched_keymask", "keymask"])
def test_small_kernel_aligned_operand_rows(dev, kernel, Lq, bias, batched, mask):
    """Lk = 252: every dense-bias and key-mask row starts 16 (4) bytes aligned, so the small-launch
    kernels read whole blocks of them with vector loads and the last, partial block (keys 224..251)
    element by element; Lk = 250 in the variant cases covers the misaligned rows."""
    call = make_call(B=8, H=4, D=64, Lq=Lq, Lk=252, seed=77 + bias + 3 * mask, bias_mode=bias, mask_mode=mask,
                     dense_bias_batched=batched, name=f"small_aligned_k{kernel}_b{bias}_m{mask}")
    if call.key_mask is not None:
        call.key_mask[0, :] = 0
        call.key_mask[1, 3] = 1  # a row whose only attended key sits inside a vector-loaded run
        call.key_mask[1, :3] = 0
        call.key_mask[1, 4:] = 0
    check_call(dev, call, False, (kernel, 64, 4, bias, 2 if mask else 0))


def check_call(dev, call, host, variant):
    print(f"[case] {call.name} B={call.B} H={call.H} D={call.D} Lq={call.Lq} Lk={call.Lk}", flush=True)
    st = Staged(dev, call, out_fill=SENTINEL, host_key_len=host)
    try:
        assert _lib.plan(st.args).variant() == variant
        out = st.run()
    finally:
        st.release()
    got = orc.output_view(out, call)
    e = orc.errors(got, orc.reference_torch(call))
    assert e["finite"], call.name
    assert e["rel_l2"] <= TOL and e["max_rel"] <= TOL, f"{call.name} vs torch fp32: {e}"
    e64 = orc.errors(got, orc.reference_fp64(call))
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
