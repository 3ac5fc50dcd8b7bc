"""The C ABI boundary on the CPU: the library loads, exports every symbol include/supra_attn.h
declares, lays out sa_attn_args as the Python mirror does, and rejects invalid calls before any
launch (no GPU needed: validation never touches the pointers it is given)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from oracle import t5_bucket as tb
from supra_attn import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "supra_attn.h")
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include"))) if h.endswith(".h")]
FAKE = 0x7F0000000000  # a device-looking address; validation only compares addresses

# The tests that pass made-up addresses to the launching entry points (sa_attention_f32,
# sa_linear_f32, sa_vae_attention_f32) to show that validation rejects a call before any launch run
# only where no device is visible: on a GPU host a validation regression would launch a kernel on
# those addresses. The host-only queries (sa_attention_plan, *_kernel_name, *_workspace_bytes) are
# exercised everywhere.
launches_fake_addresses = pytest.mark.skipif(_lib.device_count() > 0,
                                             reason="made-up device addresses: run on a host without a GPU")


def header_functions() -> list[str]:
    text = "\n".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(sa_\w+)\s*\(", text, flags=re.M)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert sorted(_lib.SIGNATURES) == names, "ctypes bindings drift from the header"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (sa_\w+)", out))
    assert exported == set(names), f"exported but undeclared: {exported - set(names)}"


def test_version_and_constants():
    lib = _lib.load()
    assert lib.sa_version() == 5
    text = open(HEADER).read()
    text += open(os.path.join(ROOT, "include", "supra_linear.h")).read()
    weights = open(os.path.join(ROOT, "include", "supra_weights.h")).read()
    for dt, code in _lib.SA_DT.items():
        m = re.search(rf"#define SA_DT_{dt} (\d+)", weights)
        assert m and int(m.group(1)) == code, dt
    assert re.search(rf"#define SA_ST_MAX_DIMS {_lib.SA_ST_MAX_DIMS}\b", weights)
    for name in ("SA_OK", "SA_ERR_INVALID", "SA_ERR_UNSUPPORTED", "SA_ERR_HIP", "SA_ERR_ALIAS", "SA_ERR_NOT_FOUND",
                 "SA_ERR_IO", "SA_ERR_FORMAT", "SA_BIAS_NONE",
                 "SA_BIAS_DENSE", "SA_BIAS_RELPOS", "SA_MASK_NONE", "SA_MASK_KEY_LEN", "SA_MASK_KEY_MASK",
                 "SA_ACT_NONE", "SA_ACT_GELU", "SA_ACT_GELU_TANH", "SA_ACT_SILU", "SA_EPI_STORE", "SA_EPI_RESID",
                 "SA_EPI_RESID_GATE"):
        m = re.search(rf"#define {name} \(?(-?\d+)\)?", text)
        assert m and int(m.group(1)) == getattr(_lib, name), name


@pytest.mark.parametrize("cls,ctype,header", [(_lib.AttnArgs, "sa_attn_args", "supra_attn.h"),
                                              (_lib.LinearArgs, "sa_linear_args", "supra_linear.h"),
                                              (_lib.VaeAttnArgs, "sa_vae_attn_args", "supra_vae.h"),
                                              (_lib.StTensor, "sa_st_tensor", "supra_weights.h"),
                                              (_lib.AttnPlan, "sa_attn_plan", "supra_attn.h")])
def test_struct_layout_matches_c(tmp_path, cls, ctype, header):
    fields = [f[0] for f in cls._fields_]
    src = tmp_path / "layout.c"
    body = "\n".join(f'  printf("{f} %zu\\n", offsetof({ctype}, {f}));' for f in fields)
    src.write_text(f'#include <stdio.h>\n#include <stddef.h>\n#include "{header}"\nint main(void) {{\n'
                   f'  printf("sizeof %zu\\n", sizeof({ctype}));\n{body}\n  return 0;\n}}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{os.path.dirname(HEADER)}", str(src), "-o", str(exe)], check=True)
    lines = dict(ln.split() for ln in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    assert int(lines["sizeof"]) == ctypes.sizeof(cls)
    for f in fields:
        assert int(lines[f]) == getattr(cls, f).offset, f


def good_args(**over):
    kw = dict(B=2, H=9, D=64, Lq=256, Lk=256, q=FAKE, k=FAKE, v=FAKE, o=FAKE + (1 << 32), q_off=0, k_off=576,
              v_off=1152, ldq=1728, ldk=1728, ldv=1728, ldo=576, sq=256 * 1728, sk=256 * 1728, sv=256 * 1728,
              so=256 * 576, scale=0.125)
    kw.update(over)
    return _lib.AttnArgs(**kw)


def rc_of(args):
    return _lib.load().sa_attention_f32(ctypes.byref(args), None)


def test_valid_call_selects_mfma_kernel():
    assert _lib.kernel_name(good_args()) == "flash_small_d64"
    assert _lib.kernel_name(good_args(B=64, o=FAKE + (1 << 36), sq=256 * 1728)) == "flash_mfma_d64"
    assert _lib.kernel_name(good_args(B=16, o=FAKE + (1 << 36))) == "flash_mfma_d64_split2"
    assert _lib.kernel_name(good_args(D=128, H=4, ldo=512, so=256 * 512)) == "flash_mfma_d128_split2"


def big(B, Lq=256, **over):
    return good_args(B=B, Lq=Lq, sq=Lq * 1728, so=Lq * 576, o=FAKE + (1 << 36), **over)


SMALL, FLASH = _lib.SA_KERNEL_FLASH_SMALL, _lib.SA_KERNEL_FLASH


@pytest.mark.parametrize("B,Lq,tail_units,tail_kernel,tail_split,tail_wg,folded", [
    (56, 256, 0, 0, 0, 0, 0),          # 1008 units: one round on 256 CUs
    (57, 256, 2, SMALL, 4, 8, 0),      # 1026: a round of 1024, two left: 8 groups of 32 queries
    (60, 256, 56, SMALL, 4, 224, 0),   # 1080: 56 left, 224 groups
    (61, 256, 74, FLASH, 2, 148, 1),   # 1098: 74 left, 296 groups would not fit: 148 units of 64 queries,
                                       # folded into the first 148 workgroups of the round
    (64, 256, 128, FLASH, 2, 256, 1),  # the batch-64 DiT call: 128 left, 256 units of 64, one per CU, folded
    (71, 256, 0, 0, 0, 0, 0),          # 1278: 254 left would need more than one workgroup per CU: one launch
    (114, 256, 4, SMALL, 4, 16, 0),    # 2052: two whole rounds and four left
    (118, 256, 76, FLASH, 2, 152, 0),  # 2124: two whole rounds and 76 left: a second launch, not folded
    (57, 200, 2, SMALL, 4, 7, 0),      # 7 groups of 32 per head: the tail is one whole head of 2 units
    (61, 200, 74, FLASH, 2, 148, 1),   # 4 units of 64 per head (the last one 8 queries)
])
def test_plan_reports_the_tail_launch(B, Lq, tail_units, tail_kernel, tail_split, tail_wg, folded):
    """The batch-B, 9-head self-attention call on 256 CUs (the count without a device): the units past
    the last whole round of 1024 run at one workgroup per CU, in a second launch, or, after a single
    round, as 64-query units folded into the round's first workgroups."""
    plan = _lib.plan(big(B, Lq))
    assert plan.kernel == _lib.SA_KERNEL_FLASH and plan.name == b"flash_mfma_d64"
    assert plan.workgroups == B * 9 * ((Lq + 127) // 128) - tail_units
    assert (plan.tail_kernel, plan.tail_key_split, plan.tail_workgroups) == (tail_kernel, tail_split, tail_wg)
    assert plan.tail_folded == folded


@pytest.mark.parametrize("over", [
    dict(bias_mode=1, bias=FAKE + (3 << 36)),                 # a dense bias
    dict(mask_mode=2, key_mask=FAKE + (3 << 36), smask=256),  # a key mask
    dict(Lk=32, sk=32 * 1728, sv=32 * 1728),                  # one key block
    dict(mask_mode=1, key_len=FAKE + (3 << 36)),              # key lengths: the result may not depend on
])                                                            # whether the schedule's host copy comes along
def test_no_tail_launch_outside_the_plain_variants(over):
    for B in (60, 64):  # a small-launch tail, a folded one
        plan = _lib.plan(big(B, **over))
        assert plan.kernel == _lib.SA_KERNEL_FLASH and plan.tail_kernel == 0 and plan.tail_folded == 0


def test_generic_kernel_for_row_strides_beyond_32bit_copy_offsets():
    big = 1 << 22  # 128 rows of this stride no longer fit a 31-bit byte offset
    far = FAKE + (1 << 40)  # an output beyond the long k/v extents
    assert _lib.kernel_name(good_args(ldk=big - 4, ldv=big - 4, sk=256 * big, sv=256 * big, o=far)) == "flash_small_d64"
    assert _lib.kernel_name(good_args(ldk=big, ldv=1728, sk=256 * big, o=far)) == "generic"
    assert _lib.kernel_name(good_args(ldv=big, sv=256 * big, o=far)) == "generic"


def test_generic_kernel_for_other_head_dims_and_unaligned_rows():
    assert _lib.kernel_name(good_args(D=32, ldo=288, so=256 * 288)) == "generic"
    assert _lib.kernel_name(good_args(q_off=1)) == "generic"
    assert _lib.kernel_name(good_args(ldq=1729, ldk=1729, ldv=1729)) == "generic"
    assert _lib.kernel_name(good_args(q=FAKE + 4, k=FAKE + 4, v=FAKE + 4)) == "generic"
    vae = _lib.AttnArgs(B=1, H=1, D=512, Lq=1024, Lk=1024, q=FAKE, k=FAKE + (1 << 24), v=FAKE + (2 << 24),
                        o=FAKE + (3 << 24), ldq=512, ldk=512, ldv=512, scale=0.0442)
    assert _lib.kernel_name(vae) == "wide_mfma_d512"
    wide = dict(D=512, H=2, ldq=4096, ldk=4096, ldv=4096, ldo=1024, so=256 * 1024)
    # a dense bias and a key mask fuse into the wide kernels; the relative-position gather does not
    assert _lib.kernel_name(good_args(**wide, bias_mode=1, bias=FAKE + (2 << 32))) == "wide_mfma_d512"
    assert _lib.kernel_name(good_args(**wide, mask_mode=2, key_mask=FAKE + (2 << 32))) == "wide_mfma_d512"
    assert _lib.kernel_name(good_args(**wide, bias_mode=2, bias=FAKE + (2 << 32), bucket_lut=FAKE + (3 << 32),
                                      num_buckets=32)) == "generic"
    # the wide kernels take 32-bit strides: a batch stride past 2^31 - 1 elements takes the generic kernel
    far = dict(wide, so=1 << 31, o=FAKE + (1 << 44))
    assert _lib.kernel_name(good_args(**far)) == "generic"
    assert _lib.kernel_name(good_args(**dict(far, so=(1 << 31) - 1024))) == "wide_mfma_d512"


@pytest.mark.parametrize("over,code", [
    (dict(struct_size=8), _lib.SA_ERR_INVALID),
    (dict(B=0), _lib.SA_ERR_INVALID),
    (dict(H=0), _lib.SA_ERR_INVALID),
    (dict(Lq=0), _lib.SA_ERR_INVALID),
    (dict(Lk=0), _lib.SA_ERR_INVALID),
    (dict(q=0), _lib.SA_ERR_INVALID),
    (dict(o=0), _lib.SA_ERR_INVALID),
    (dict(scale=float("nan")), _lib.SA_ERR_INVALID),
    (dict(scale=float("inf")), _lib.SA_ERR_INVALID),
    (dict(q_off=-4), _lib.SA_ERR_INVALID),
    (dict(ldq=500), _lib.SA_ERR_INVALID),
    (dict(ldo=100), _lib.SA_ERR_INVALID),
    (dict(so=100), _lib.SA_ERR_INVALID),
    (dict(sq=-1), _lib.SA_ERR_INVALID),
    (dict(k_off=1 << 40), _lib.SA_ERR_INVALID),
    (dict(ldv=1 << 41), _lib.SA_ERR_INVALID),
    (dict(sk=1 << 40), _lib.SA_ERR_INVALID),
    (dict(o=FAKE + 4096), _lib.SA_ERR_ALIAS),
    (dict(bias_mode=1), _lib.SA_ERR_INVALID),
    (dict(bias_mode=2, bias=FAKE + (2 << 32)), _lib.SA_ERR_INVALID),
    (dict(bias_mode=2, bias=FAKE + (2 << 32), bucket_lut=FAKE + (3 << 32)), _lib.SA_ERR_INVALID),
    (dict(bias_mode=7), _lib.SA_ERR_INVALID),
    (dict(mask_mode=1), _lib.SA_ERR_INVALID),
    (dict(mask_mode=2), _lib.SA_ERR_INVALID),
    (dict(mask_mode=2, key_mask=FAKE + (2 << 32), smask=100), _lib.SA_ERR_INVALID),
    (dict(mask_mode=9), _lib.SA_ERR_INVALID),
    (dict(D=2048, ldq=1 << 16, ldk=1 << 16, ldv=1 << 16, ldo=1 << 16, so=256 << 16), _lib.SA_ERR_UNSUPPORTED),
])
def test_plan_reports_the_rejection(over, code):
    """The host-only plan query runs the same validation as the call and returns its status."""
    args = good_args(**over)
    if "struct_size" in over:
        args.struct_size = over["struct_size"]
    plan = _lib.AttnPlan()
    lib = _lib.load()
    assert lib.sa_attention_plan(ctypes.byref(args), ctypes.byref(plan)) == code
    assert lib.sa_last_status() == code
    assert lib.sa_attention_kernel_name(ctypes.byref(args)) is None
    assert lib.sa_last_status() == code


O = FAKE + (1 << 36)  # the output of the overlap cases below; q/k/v stay at FAKE


@pytest.mark.parametrize("over", [
    dict(bias_mode=1, bias=O + 1024),                                     # dense bias inside o
    dict(bias_mode=1, bias=O - 4 * 9 * 256 * 256 + 4),                    # dense bias ending inside o
    dict(bias_mode=1, bias=O - 4 * 9 * 256 * 256 - 1024, sbias=9 * 256 * 256),  # second batch's bias inside o
    dict(bias_mode=2, bias=O + 64, bucket_lut=FAKE + (3 << 36), num_buckets=32),   # relpos table
    dict(bias_mode=2, bias=FAKE + (3 << 36), bucket_lut=O + 64, num_buckets=32),   # bucket LUT
    dict(mask_mode=1, key_len=O + 4),                                     # key lengths
    dict(mask_mode=2, key_mask=O + 100),                                  # key mask
    dict(mask_mode=2, key_mask=O - 256 - 10, smask=256),                  # the second sequence's mask row
])
def test_output_overlapping_any_read_operand_is_an_alias(over):
    args = good_args(o=O, **over)
    plan = _lib.AttnPlan()
    assert _lib.load().sa_attention_plan(ctypes.byref(args), ctypes.byref(plan)) == _lib.SA_ERR_ALIAS
    assert b"overlaps" in _lib.load().sa_last_error()
    # the same operands clear of o are accepted
    moved = {k: (v + (1 << 38) if k in ("bias", "bucket_lut", "key_len", "key_mask") else v) for k, v in over.items()}
    assert _lib.plan(good_args(o=O, **moved)).name


@pytest.mark.parametrize("over,code", [
    (dict(struct_size=8), _lib.SA_ERR_INVALID),
    (dict(B=0), _lib.SA_ERR_INVALID),
    (dict(H=0), _lib.SA_ERR_INVALID),
    (dict(Lq=0), _lib.SA_ERR_INVALID),
    (dict(Lk=0), _lib.SA_ERR_INVALID),
    (dict(q=0), _lib.SA_ERR_INVALID),
    (dict(o=0), _lib.SA_ERR_INVALID),
    (dict(scale=float("nan")), _lib.SA_ERR_INVALID),
    (dict(scale=float("inf")), _lib.SA_ERR_INVALID),
    (dict(q_off=-4), _lib.SA_ERR_INVALID),
    (dict(ldq=500), _lib.SA_ERR_INVALID),
    (dict(ldo=100), _lib.SA_ERR_INVALID),
    (dict(so=100), _lib.SA_ERR_INVALID),
    (dict(sq=-1), _lib.SA_ERR_INVALID),
    (dict(k_off=1 << 40), _lib.SA_ERR_INVALID),
    (dict(ldv=1 << 41), _lib.SA_ERR_INVALID),
    (dict(sk=1 << 40), _lib.SA_ERR_INVALID),
    (dict(o=FAKE + 4096), _lib.SA_ERR_ALIAS),
    (dict(bias_mode=1), _lib.SA_ERR_INVALID),
    (dict(bias_mode=2, bias=FAKE + (2 << 32)), _lib.SA_ERR_INVALID),
    (dict(bias_mode=2, bias=FAKE + (2 << 32), bucket_lut=FAKE + (3 << 32)), _lib.SA_ERR_INVALID),
    (dict(bias_mode=7), _lib.SA_ERR_INVALID),
    (dict(mask_mode=1), _lib.SA_ERR_INVALID),
    (dict(mask_mode=2), _lib.SA_ERR_INVALID),
    (dict(mask_mode=2, key_mask=FAKE + (2 << 32), smask=100), _lib.SA_ERR_INVALID),
    (dict(mask_mode=9), _lib.SA_ERR_INVALID),
    (dict(D=2048, ldq=1 << 16, ldk=1 << 16, ldv=1 << 16, ldo=1 << 16, so=256 << 16), _lib.SA_ERR_UNSUPPORTED),
])
@launches_fake_addresses
def test_invalid_calls_are_rejected_before_launch(over, code):
    args = good_args(**over)
    if "struct_size" in over:
        args.struct_size = over["struct_size"]
    assert rc_of(args) == code
    msg = _lib.load().sa_last_error().decode()
    assert msg, "an error must carry a message"
    assert _lib.load().sa_attention_kernel_name(ctypes.byref(args)) is None


def test_revision2_struct_size_is_accepted():
    """Callers built against revision 2 (the struct ending at workspace_bytes) keep working; the
    revision-3 field (key_len_host) is then treated as absent."""
    v2 = _lib.AttnArgs.key_len_host.offset
    assert v2 + ctypes.sizeof(ctypes.c_void_p) == ctypes.sizeof(_lib.AttnArgs)
    for over in (dict(), dict(mask_mode=_lib.SA_MASK_KEY_LEN, key_len=FAKE + (5 << 32))):
        args = good_args(**over)
        full = _lib.kernel_name(args)
        args.struct_size = v2
        args.key_len_host = 1  # past the revision-2 struct: must not be read
        assert _lib.kernel_name(args) == full
    args = good_args()
    args.struct_size = v2 + 4
    assert _lib.load().sa_attention_kernel_name(ctypes.byref(args)) is None


@launches_fake_addresses
def test_extents_that_overflow_are_rejected():
    """Offsets and strides below the 2^40 limit can still multiply past int64 with a large batch or
    row count: the extent arithmetic is checked, and such calls fail with a message that says so."""
    lib = _lib.load()
    big = (1 << 40) - 1
    args = good_args(B=1 << 30, sq=big, sk=big, sv=big, so=big)
    assert rc_of(args) == _lib.SA_ERR_INVALID
    assert b"overflows" in lib.sa_last_error()
    largs = lin_args(M=(1 << 31) - 1, ldx=big, ldy=big)
    assert lib.sa_linear_f32(ctypes.byref(largs), None) == _lib.SA_ERR_INVALID
    assert b"overflows" in lib.sa_last_error()


@launches_fake_addresses
def test_null_args_pointer():
    lib = _lib.load()
    assert lib.sa_attention_f32(None, None) == _lib.SA_ERR_INVALID
    assert b"NULL" in lib.sa_last_error()


@launches_fake_addresses
def test_error_message_clears_on_success():
    lib = _lib.load()
    assert rc_of(good_args(B=0)) == _lib.SA_ERR_INVALID
    assert _lib.kernel_name(good_args()) == "flash_small_d64"
    assert lib.sa_last_error() == b""


@pytest.mark.parametrize("Lq,Lk", [(1, 1), (128, 128), (7, 300), (300, 7)])
@pytest.mark.parametrize("bidirectional", [True, False])
def test_bucket_lut_matches_oracle(Lq, Lk, bidirectional):
    got = _lib.bucket_lut(Lq, Lk, 32, 128, bidirectional)
    np.testing.assert_array_equal(got, tb.bucket_lut(Lq, Lk, bidirectional))


def test_bucket_lut_other_bucket_counts():
    for nb, md in ((16, 64), (64, 256), (8, 20)):
        got = _lib.bucket_lut(50, 60, nb, md, True)
        np.testing.assert_array_equal(got, tb.bucket_lut(50, 60, True, nb, md))


def test_bucket_lut_rejects_bad_arguments():
    lib = _lib.load()
    out = (ctypes.c_int32 * 8)()
    assert lib.sa_t5_bucket_lut(0, 4, 32, 128, 1, out) == _lib.SA_ERR_INVALID
    assert lib.sa_t5_bucket_lut(4, 4, 2, 128, 1, out) == _lib.SA_ERR_INVALID
    assert lib.sa_t5_bucket_lut(4, 4, 32, 4, 1, out) == _lib.SA_ERR_INVALID
    assert lib.sa_t5_bucket_lut(4, 4, 32, 128, 1, None) == _lib.SA_ERR_INVALID


def test_device_helpers_reject_null_pointers():
    lib = _lib.load()
    assert lib.sa_malloc(None, 16) == _lib.SA_ERR_INVALID
    assert lib.sa_memcpy_h2d(None, None, 16, None) == _lib.SA_ERR_INVALID
    assert lib.sa_memcpy_d2h(None, None, 16, None) == _lib.SA_ERR_INVALID
    assert lib.sa_memcpy_d2d(None, None, 16, None) == _lib.SA_ERR_INVALID
    assert lib.sa_event_elapsed_ms(None, None, None) == _lib.SA_ERR_INVALID
    assert lib.sa_t5_position_bias(None, None, 32, 12, 4, 4, None, None) == _lib.SA_ERR_INVALID
    assert lib.sa_memcpy_h2d(None, None, 0, None) == _lib.SA_OK  # zero bytes is a no-op
    assert lib.sa_free(None) == _lib.SA_OK


def vae_args(**over):
    kw = dict(B=1, H=1, D=512, Lq=1024, Lk=1024, q=FAKE, k=FAKE + (1 << 24), v=FAKE + (2 << 24), o=FAKE + (3 << 24),
              ldq=512, ldk=512, ldv=512, scale=0.0442)
    kw.update(over)
    return _lib.AttnArgs(**kw)


def test_workspace_size_query():
    # flash and generic kernels need none; the wide-head kernel needs one partial record per key chunk
    assert _lib.workspace_bytes(good_args()) == 0
    assert _lib.workspace_bytes(good_args(D=32, ldo=288, so=256 * 288)) == 0
    need = _lib.workspace_bytes(vae_args())
    assert need > 0 and need % 16 == 0
    assert need < 64 << 20
    with pytest.raises(_lib.SaError) as e:
        _lib.workspace_bytes(good_args(B=0))
    assert e.value.code == _lib.SA_ERR_INVALID


@pytest.mark.parametrize("over,code,text", [
    (dict(), _lib.SA_ERR_INVALID, "workspace of"),
    (dict(workspace=FAKE + (8 << 24)), _lib.SA_ERR_INVALID, "workspace of"),
    (dict(workspace=FAKE + (8 << 24), workspace_bytes="need-1"), _lib.SA_ERR_INVALID, "workspace of"),
    (dict(workspace=FAKE + (8 << 24) + 4, workspace_bytes="need"), _lib.SA_ERR_INVALID, "aligned"),
    (dict(workspace=FAKE + (3 << 24) - 64, workspace_bytes="need"), _lib.SA_ERR_ALIAS, "overlaps"),
    (dict(workspace=FAKE + (1 << 24) + 4096, workspace_bytes="need"), _lib.SA_ERR_ALIAS, "overlaps"),
])
@launches_fake_addresses
def test_workspace_is_checked_before_launch(over, code, text):
    need = _lib.workspace_bytes(vae_args())
    over = {k: (need - 1 if v == "need-1" else need if v == "need" else v) for k, v in over.items()}
    assert rc_of(vae_args(**over)) == code
    assert text in _lib.load().sa_last_error().decode()


def lin_args(**over):
    M, N, K = over.pop("M", 512), over.pop("N", 1728), over.pop("K", 576)
    kw = dict(M=M, N=N, K=K, x=FAKE, w=FAKE + (1 << 30), y=FAKE + (2 << 30), bias=FAKE + (3 << 30))
    kw.update(over)
    return _lib.LinearArgs(**kw)


def test_linear_kernel_choice():
    # DiT layers at batch 64 (16384 rows): 64 x 192 or 128 x 192 tiles while the grid fills the chip; grids of fewer
    # 64 x 64 tiles than 1.25 per CU: 32 x 32 tiles with the k split over the workgroup's waves; under 2 per CU:
    # 32 x 64 tiles, k split in two; else 64 x 64
    assert _lib.linear_kernel_name(lin_args(M=16384, N=1728, K=576)) == "linear_mfma_64x192"       # qkv
    assert _lib.linear_kernel_name(lin_args(M=16384, N=2304, K=576)) == "linear_mfma_128x192"      # fc1
    assert _lib.linear_kernel_name(lin_args(M=16384, N=576, K=576)) == "linear_mfma_64x192"        # proj, q, cproj
    assert _lib.linear_kernel_name(lin_args(M=16384, N=576, K=2304)) == "linear_mfma_64x192"       # fc2
    assert _lib.linear_kernel_name(lin_args(M=512, N=1728, K=576)) == "linear_mfma_32x32_ksplit"   # batch 2
    assert _lib.linear_kernel_name(lin_args(M=512, N=2304, K=576)) == "linear_mfma_32x32_ksplit"   # batch-2 fc1
    assert _lib.linear_kernel_name(lin_args(M=1024, N=512, K=512)) == "linear_mfma_32x32_ksplit"   # VAE output
    assert _lib.linear_kernel_name(lin_args(M=4096, N=600, K=576)) == "linear_mfma_64x64"
    assert _lib.linear_kernel_name(lin_args(M=77, N=1152, K=576)) == "linear_mfma_32x32_ksplit"  # small call
    assert _lib.linear_kernel_name(lin_args(M=1024, N=1536, K=512)) == "linear_mfma_32x64_ksplit"  # VAE q|k|v
    assert _lib.linear_kernel_name(lin_args(M=2000, N=1024, K=512)) == "linear_mfma_64x64"  # 512 tiles
    assert _lib.linear_kernel_name(lin_args(K=36)) == "linear_generic"            # K % 8 != 0
    assert _lib.linear_kernel_name(lin_args(x_off=1)) == "linear_generic"         # unaligned rows
    assert _lib.linear_kernel_name(lin_args(x=FAKE + 4)) == "linear_generic"
    assert _lib.linear_kernel_name(lin_args(ldw=578)) == "linear_generic"
    # the MFMA kernels take 32-bit row strides: row offsets of a 128-row x tile past 2^31 bytes take the
    # generic kernel (which keeps 64-bit strides)
    assert _lib.linear_kernel_name(lin_args(ldx=1 << 22, M=64)) == "linear_generic"
    assert _lib.linear_kernel_name(lin_args(ldy=1 << 22, M=64, y=FAKE + (1 << 44))) == "linear_generic"


@pytest.mark.parametrize("over,code", [
    (dict(struct_size=8), _lib.SA_ERR_INVALID),
    (dict(M=0), _lib.SA_ERR_INVALID),
    (dict(N=-1), _lib.SA_ERR_INVALID),
    (dict(K=0), _lib.SA_ERR_INVALID),
    (dict(x=0), _lib.SA_ERR_INVALID),
    (dict(y=0), _lib.SA_ERR_INVALID),
    (dict(ldx=100), _lib.SA_ERR_INVALID),
    (dict(ldw=100), _lib.SA_ERR_INVALID),
    (dict(ldy=100), _lib.SA_ERR_INVALID),
    (dict(x_off=-4), _lib.SA_ERR_INVALID),
    (dict(y_off=1 << 40), _lib.SA_ERR_INVALID),
    (dict(ldw=1 << 40), _lib.SA_ERR_INVALID),
    (dict(alpha=float("nan")), _lib.SA_ERR_INVALID),
    (dict(act=9), _lib.SA_ERR_INVALID),
    (dict(epilogue=3), _lib.SA_ERR_INVALID),
    (dict(epilogue=2), _lib.SA_ERR_INVALID),                       # gated residual without a gate
    (dict(y=FAKE + 4096), _lib.SA_ERR_ALIAS),                      # y inside x
    (dict(y=FAKE + (1 << 30) + 64), _lib.SA_ERR_ALIAS),            # y inside w
    (dict(bias=FAKE + (2 << 30) + 128), _lib.SA_ERR_ALIAS),        # bias inside y
    (dict(epilogue=2, gate=FAKE + (2 << 30), gate_off=8), _lib.SA_ERR_ALIAS),
    (dict(M=2000000, K=36, w=FAKE + (1 << 40), y=FAKE + (2 << 40), bias=0), _lib.SA_ERR_UNSUPPORTED),
])
@launches_fake_addresses
def test_invalid_linear_calls_are_rejected(over, code):
    args = lin_args(**over)
    if "struct_size" in over:
        args.struct_size = over["struct_size"]
    assert _lib.load().sa_linear_f32(ctypes.byref(args), None) == code
    assert _lib.load().sa_last_error().decode()
    assert _lib.load().sa_linear_kernel_name(ctypes.byref(args)) is None


def vae_block_args(**over):
    kw = dict(HW=1024, C=512, x=FAKE, gamma=FAKE + (1 << 30), beta=FAKE + (1 << 30) + 4096, wqkv=FAKE + (2 << 30),
              wo=FAKE + (3 << 30), out=FAKE + (4 << 30), workspace=FAKE + (5 << 30))
    kw["workspace_bytes"] = _lib.vae_workspace_bytes(_lib.VaeAttnArgs(**kw))
    kw.update(over)
    return _lib.VaeAttnArgs(**kw)


def test_vae_workspace_size():
    # normalized image + q|k|v + attention output (5 * HW * C floats) + the wide-head merge scratch
    n = _lib.vae_workspace_bytes(vae_block_args())
    assert n >= 5 * 1024 * 512 * 4 + _lib.workspace_bytes(_lib.AttnArgs(
        B=1, H=1, D=512, Lq=1024, Lk=1024, q=FAKE, k=FAKE + 2048, v=FAKE + 4096, o=FAKE + (1 << 30),
        ldq=1536, ldk=1536, ldv=1536, scale=0.044))


@launches_fake_addresses
def test_vae_block_passes_on_the_rejecting_part_status():
    """A VAE block that one of its parts cannot run fails with that part's status, not a generic one:
    SA_ERR_UNSUPPORTED from the attention (head dim C = 2048 above the generic kernel's 1024) and from
    the q|k|v projection (K = C = 36, not a multiple of 8, over more rows than its generic kernel's
    grid); nothing launches either way (fake addresses)."""
    lib = _lib.load()
    for over in (dict(HW=64, C=2048, groups=32), dict(HW=1_100_000, C=36, groups=4)):
        kw = dict(HW=1024, C=512, x=FAKE, gamma=FAKE + (1 << 30), beta=FAKE + (1 << 30) + (1 << 20),
                  wqkv=FAKE + (2 << 30), wo=FAKE + (3 << 30), out=FAKE + (4 << 30), workspace=FAKE + (5 << 30))
        kw.update(over)
        probe = _lib.VaeAttnArgs(**kw)
        need = lib.sa_vae_attention_workspace_bytes(ctypes.byref(probe))
        if need < 0:  # the attention part already rejects the sizes
            assert need == _lib.SA_ERR_UNSUPPORTED
            kw["workspace_bytes"] = 1 << 30
        else:
            kw["workspace_bytes"] = need
        args = _lib.VaeAttnArgs(**kw)
        assert lib.sa_vae_attention_f32(ctypes.byref(args), None) == _lib.SA_ERR_UNSUPPORTED, over
        assert lib.sa_last_status() == _lib.SA_ERR_UNSUPPORTED
        assert lib.sa_last_error().decode()


@pytest.mark.parametrize("over,code", [
    (dict(struct_size=8), _lib.SA_ERR_INVALID),
    (dict(HW=0), _lib.SA_ERR_INVALID),
    (dict(groups=0), _lib.SA_ERR_INVALID),
    (dict(groups=7), _lib.SA_ERR_INVALID),                  # C % groups != 0
    (dict(eps=float("nan")), _lib.SA_ERR_INVALID),
    (dict(x=0), _lib.SA_ERR_INVALID),
    (dict(workspace=0), _lib.SA_ERR_INVALID),
    (dict(workspace_bytes=1024), _lib.SA_ERR_INVALID),
    (dict(workspace=FAKE + (5 << 30) + 4), _lib.SA_ERR_INVALID),   # unaligned
    (dict(out=FAKE + 64), _lib.SA_ERR_ALIAS),                      # partial overlap with x
    (dict(out=FAKE + (2 << 30)), _lib.SA_ERR_ALIAS),               # out over the weights
    (dict(workspace=FAKE + (4 << 30) + 1024), _lib.SA_ERR_ALIAS),  # workspace over out
])
@launches_fake_addresses
def test_invalid_vae_calls_are_rejected(over, code):
    args = vae_block_args(**over)
    if "struct_size" in over:
        args.struct_size = over["struct_size"]
    assert _lib.load().sa_vae_attention_f32(ctypes.byref(args), None) == code
    assert _lib.load().sa_last_error().decode()
