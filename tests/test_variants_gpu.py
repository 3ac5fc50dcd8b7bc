"""GPU parity of every compiled flash and small-launch kernel variant <kernel, D, key_split, bias, mask>, each at a shape
that real callers give it, with ragged lengths and at least two loop steps per splitting wave,
against the PyTorch fp32 CPU path and the float64 brute force (both <= 1e-5, relative L2 and
normwise max). The cases come from variant_cases.py; test_variants.py shows on the host that they
reach every compiled variant."""

from __future__ import annotations

import pytest

from supra_attn import _lib
from cases import make_call
from variant_cases import call_for, check_call, flash_variants, variant_id, wide_call_for, wide_variants

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("variant", flash_variants(), ids=variant_id)
def test_variant_parity(dev, variant):
    """Key-length cases with separate K and V arrays also carry NaN and Inf in every row past a
    sequence's length: no row past it may reach the output."""
    call, host = call_for(*variant)
    check_call(dev, call, host, variant, poison_padding=call.key_len is not None and not call.same_qkv)


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


@pytest.mark.parametrize("variant", wide_variants(), ids=lambda v: "wide_d%d_b%d_m%d" % (v[1], v[3], v[4]))
def test_wide_variant_parity(dev, variant):
    """Every wide-kernel variant <D, bias, mask>: split into key chunks or not, ragged lengths; key-length
    cases carry NaN and Inf in every K and V row past a sequence's length."""
    call = wide_call_for(*variant)
    check_call(dev, call, False, variant, poison_padding=call.key_len is not None)
