"""GPU parity: the HIP operator, called through the C ABI, against the CPU oracle.

The bar (the PyTorch fp32 CPU path, oracle.attention.attention_torch_fp32): relative L2 and
normwise max relative error both <= 1e-5; the fp64 brute force is checked with the same bound.
Output elements outside the written rows must keep their previous contents.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as orc
from supra_attn import _lib, workloads
from supra_attn.runner import Staged
from cases import make_call
from variant_cases import fake_args

pytestmark = pytest.mark.gpu

TOL = 1e-5
SENTINEL = np.float32(-12345.5)


def run_checked(dev, call, *, expect_kernel=None, tol=TOL, check_fp64=True):
    print(f"[case] {call.name} B={call.B} H={call.H} D={call.D} Lq={call.Lq} Lk={call.Lk} "
          f"bias={call.bias_mode} mask={call.mask_mode}", flush=True)
    st = Staged(dev, call, out_fill=SENTINEL)
    try:
        if expect_kernel is not None:
            assert st.kernel == expect_kernel
        out = st.run()
    finally:
        st.release()
    got = orc.output_view(out, call)
    ref = orc.reference_torch(call)
    e = orc.errors(got, ref)
    assert e["finite"], f"non-finite output for {call.name}"
    assert e["rel_l2"] <= tol and e["max_rel"] <= tol, f"{call.name} vs torch fp32: {e}"
    if check_fp64:
        e64 = orc.errors(got, orc.reference_fp64(call))
        assert e64["rel_l2"] <= tol and e64["max_rel"] <= tol, f"{call.name} vs fp64: {e64}"
    # untouched elements of the output buffer keep the sentinel
    written = np.zeros(out.size, dtype=bool)
    a = call.args
    ldo = a.get("ldo", 0) or call.H * call.D
    idx = orc.heads(np.arange(out.size), B=call.B, L=call.Lq, H=call.H, D=call.D, off=a.get("o_off", 0), ld=ldo,
                    sb=a.get("so", 0))
    written[idx.reshape(-1)] = True
    assert (out.reshape(-1)[~written] == SENTINEL).all(), "operator wrote outside its output rows"
    return e


# ---- the four single-call configs


def test_dit_self_b2(dev):
    call = workloads.dit_self(B=2, seed=0)
    run_checked(dev, call, expect_kernel="flash_small_d64")


def test_dit_cross_b2(dev):
    call = workloads.dit_cross(B=2, seed=1)
    run_checked(dev, call)


def test_t5_relpos_keymask(dev):
    call = workloads.t5_self(seed=2)
    run_checked(dev, call)


def test_vae_mid(dev):
    call = workloads.vae_mid(seed=3)
    run_checked(dev, call)


def test_sweep_block0(dev):
    s, c = workloads.sweep_block(0)
    run_checked(dev, s, expect_kernel="flash_mfma_d64", check_fp64=False)
    run_checked(dev, c, expect_kernel="flash_mfma_d64", check_fp64=False)


# ---- shapes, layouts and splits


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Lq,Lk", [(1, 1), (32, 32), (77, 45), (130, 257), (256, 31)])
def test_shapes(dev, D, Lq, Lk):
    run_checked(dev, make_call(B=2, H=3, D=D, Lq=Lq, Lk=Lk, seed=Lq * 1000 + Lk))


@pytest.mark.parametrize("B,H,Lq,Lk", [(1, 1, 64, 256), (4, 9, 256, 256), (64, 9, 256, 256), (8, 16, 512, 96)])
def test_split_modes(dev, B, H, Lq, Lk):
    """Work sizes that select each key-split variant of the MFMA kernel."""
    run_checked(dev, make_call(B=B, H=H, D=64, Lq=Lq, Lk=Lk, seed=B * H + Lk, packed=True), check_fp64=(B < 64))


def test_packed_offsets_padded_rows(dev):
    call = make_call(B=3, H=4, D=64, Lq=100, Lk=70, packed=True, pad_cols=8, q_off=12, o_off=20, ldo_pad=36, seed=7)
    run_checked(dev, call)


def test_scale_values(dev):
    for sc in (1.0, 0.01, 3.0, -0.5):
        run_checked(dev, make_call(B=1, H=2, D=64, Lq=40, Lk=90, scale=sc, seed=11))


# ---- masks and bias


def test_key_len_including_zero(dev):
    call = make_call(B=6, H=2, D=64, Lq=64, Lk=128, mask_mode=_lib.SA_MASK_KEY_LEN,
                     key_len=[0, 1, 31, 32, 33, 128], seed=3)
    run_checked(dev, call)


PADDING_CASES = [
    # (B, H, D, Lq, Lk, host copy of the lengths): the 4-per-CU flash kernel with and without the
    # schedule, both small-launch kernels, head dim 128, and the wide kernels
    (64, 9, 64, 256, 128, True),
    (64, 9, 64, 256, 128, False),
    (6, 2, 64, 64, 128, False),     # 48 groups of 16 queries: the 16-query small-launch kernel
    (6, 4, 64, 200, 128, True),     # 312 groups of 16: the short sequences packed, 2 waves per group
    (2, 9, 64, 256, 128, True),     # the batch-2 DiT cross shape, packed
    (8, 9, 64, 64, 128, False),     # 144 groups of 32 (288 of 16): the 32-query small-launch kernel
    (32, 8, 128, 256, 160, True),
    (2, 1, 512, 96, 300, False),
    (2, 2, 256, 64, 200, False),
]


@pytest.mark.parametrize("B,H,D,Lq,Lk,host", PADDING_CASES, ids=[f"B{c[0]}D{c[2]}k{c[4]}{'h' if c[5] else ''}"
                                                                 for c in PADDING_CASES])
def test_key_len_padding_is_never_used(dev, B, H, D, Lq, Lk, host):
    """Keys past a sequence's length may hold anything (the reference runs each sample at its own
    Lk, app/models/dit.js:182-185): with NaN and Inf in every K and V row past the length, the output
    equals the attention over the valid keys alone (the oracle on the original, finite inputs)."""
    rng = np.random.default_rng(B * 1000 + D + Lk)
    key_len = rng.integers(0, Lk + 1, size=B).astype(np.int32)
    key_len[: min(B, 5)] = [0, 1, 31, 33, Lk][: min(B, 5)]
    call = make_call(B=B, H=H, D=D, Lq=Lq, Lk=Lk, mask_mode=_lib.SA_MASK_KEY_LEN, key_len=key_len, seed=B + D)
    ref = orc.reference_torch(call)
    ld = call.args["ldk"]
    k = call.k.reshape(B, Lk, ld).copy()
    v = call.v.reshape(B, Lk, ld).copy()
    for b in range(B):
        k[b, key_len[b]:] = np.nan
        v[b, key_len[b]:] = np.where(np.arange(ld) % 2 == 0, np.inf, np.nan).astype(np.float32)
    call.k, call.v = k.reshape(-1), v.reshape(-1)
    print(f"[case] padding B={B} H={H} D={D} Lq={Lq} Lk={Lk} host={host}", flush=True)
    st = Staged(dev, call, out_fill=SENTINEL, host_key_len=host)
    try:
        print(f"  kernel {st.kernel}", flush=True)
        out = st.run()
    finally:
        st.release()
    e = orc.errors(orc.output_view(out, call), ref)
    assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, e


def test_key_mask_random_and_empty(dev):
    call = make_call(B=3, H=2, D=64, Lq=50, Lk=100, mask_mode=_lib.SA_MASK_KEY_MASK, seed=5)
    call.key_mask[1, :] = 0  # a sequence with no attended key -> zeros
    run_checked(dev, call)


@pytest.mark.parametrize("batched", [False, True])
def test_dense_bias(dev, batched):
    call = make_call(B=2, H=3, D=64, Lq=70, Lk=90, bias_mode=_lib.SA_BIAS_DENSE, dense_bias_batched=batched, seed=9)
    run_checked(dev, call)


@pytest.mark.parametrize("Lq,Lk", [(128, 128), (37, 200), (300, 20)])
def test_relpos_bias(dev, Lq, Lk):
    call = make_call(B=2, H=12, D=64, Lq=Lq, Lk=Lk, scale=1.0, bias_mode=_lib.SA_BIAS_RELPOS,
                     mask_mode=_lib.SA_MASK_KEY_LEN, key_len=[Lk, max(1, Lk - 40)], seed=Lq + Lk)
    run_checked(dev, call)


def test_relpos_matches_dense(dev):
    """The in-kernel relative-position gather equals passing its dense expansion."""
    c1 = make_call(B=1, H=12, D=64, Lq=128, Lk=128, scale=1.0, bias_mode=_lib.SA_BIAS_RELPOS, seed=21)
    c2 = make_call(B=1, H=12, D=64, Lq=128, Lk=128, scale=1.0, seed=21)
    c2.bias = orc.dense_relpos_bias(c1.bias, c1.lut, 12, 128, 128)[None]
    c2.bias_mode = _lib.SA_BIAS_DENSE
    o1 = Staged(dev, c1).run()
    o2 = Staged(dev, c2).run()
    assert orc.errors(o1, o2)["max_rel"] <= 1e-6


# ---- generic kernel (head dims / alignment outside the MFMA kernels)


@pytest.mark.parametrize("D", [1, 32, 80, 1000])
def test_generic_head_dims(dev, D):
    call = make_call(B=2, H=2, D=D, Lq=33, Lk=300, seed=D)
    name = _lib.kernel_name(Staged(dev, call).args)
    assert name == "generic"
    run_checked(dev, call)


# ---- wide-head kernel (D = 256 / 512: head dim split over waves, keys split over workgroups)


@pytest.mark.parametrize("D,B,H,Lq,Lk", [(512, 1, 1, 1024, 1024), (512, 1, 1, 33, 300), (256, 2, 3, 70, 200),
                                          (512, 2, 2, 64, 40), (256, 1, 1, 1, 1),
                                          # D = 512 in several rounds of four key blocks per workgroup: one
                                          # chunk per query group (3 rounds, the last with one wave's block
                                          # and a partial one), and 10 chunks of 2 rounds, the last chunk short
                                          (512, 8, 1, 1024, 300), (512, 1, 1, 64, 2500),
                                          # 2304 tokens: 3 chunks of 768 keys (D = 512), 7 of 352 (D = 256)
                                          (512, 1, 1, 2304, 2304), (256, 1, 1, 2304, 2304),
                                          # groups past whole rounds split alone: 256 + 32 in 8 chunks
                                          # (D = 512), 512 + 32 in 16 chunks, ragged (D = 256)
                                          (512, 1, 9, 1024, 1024), (256, 1, 17, 1000, 1000)])
def test_wide_shapes(dev, D, B, H, Lq, Lk):
    call = make_call(B=B, H=H, D=D, Lq=Lq, Lk=Lk, seed=D + Lq + Lk)
    assert _lib.kernel_name(Staged(dev, call).args) == f"wide_mfma_d{D}"
    run_checked(dev, call, check_fp64=Lq * Lk < 500000)


@pytest.mark.parametrize("bias_mode,mask_mode", [(_lib.SA_BIAS_NONE, _lib.SA_MASK_KEY_LEN),
                                                 (_lib.SA_BIAS_DENSE, _lib.SA_MASK_KEY_MASK)])
def test_wide_whole_rounds_then_split_groups(dev, bias_mode, mask_mode):
    """288 query groups (2 sequences x 9 heads x 500 queries, D = 512): the first 256 run unsplit,
    the last 32 (two heads of the second sequence) in key chunks, with key lengths or a key mask
    and a dense bias per sequence."""
    call = make_call(B=2, H=9, D=512, Lq=500, Lk=512, bias_mode=bias_mode, mask_mode=mask_mode,
                     key_len=[512, 300] if mask_mode == _lib.SA_MASK_KEY_LEN else None, dense_bias_batched=True,
                     seed=77 + mask_mode)
    p = _lib.plan(fake_args(call, False))
    assert (p.workgroups, p.tail_kernel, p.tail_workgroups) == (256, _lib.SA_KERNEL_WIDE, 32 * p.tail_key_split)
    run_checked(dev, call, check_fp64=False)


def test_wide_key_len_and_workspace_reuse(dev):
    """Key lengths (incl. 0 and ones that leave whole key chunks empty); back-to-back calls on one
    workspace that is refilled with NaN bytes before each call (no result may depend on what the
    workspace held), then a smaller call on the same, larger workspace."""
    call = make_call(B=4, H=1, D=512, Lq=96, Lk=512, mask_mode=_lib.SA_MASK_KEY_LEN, key_len=[0, 1, 100, 512], seed=8)
    st = Staged(dev, call)
    assert st.kernel == "wide_mfma_d512"
    ws = st.bufs[-1]
    assert st.args.workspace == ws.ptr and ws.nbytes >= st.args.workspace_bytes > 0
    ref = orc.reference_torch(call)
    for _ in range(3):
        ws.fill_bytes(0xFF)
        out = st.run()
        e = orc.errors(orc.output_view(out, call), ref)
        assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, e
    small = make_call(B=1, H=1, D=512, Lq=33, Lk=300, seed=9)
    s2 = Staged(dev, small)
    assert 0 < _lib.workspace_bytes(s2.args) <= ws.nbytes
    s2.args.workspace = ws.ptr
    s2.args.workspace_bytes = ws.nbytes
    ws.fill_bytes(0xFF)
    e = orc.errors(orc.output_view(s2.run(), small), orc.reference_torch(small))
    assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, e
    s2.release()
    st.release()


def test_wide_rounds_with_key_lengths(dev):
    """D = 512, one key chunk per query group (256 query groups fill the chip), so each workgroup takes
    its keys in rounds of four blocks with the reference moved between rounds; key lengths leave
    0, 1, 2 or 3 rounds, whole blocks and single keys."""
    lens = [0, 1, 31, 32, 33, 127, 128, 129, 200, 255, 256, 257, 299, 300, 64, 96]
    call = make_call(B=16, H=1, D=512, Lq=512, Lk=300, mask_mode=_lib.SA_MASK_KEY_LEN, key_len=lens, seed=21)
    st = Staged(dev, call)
    assert st.kernel == "wide_mfma_d512"
    assert _lib.plan(st.args).key_chunks == 1
    st.release()
    run_checked(dev, call, check_fp64=False)


def test_wide_large_batch_without_key_split(dev):
    call = make_call(B=16, H=4, D=256, Lq=128, Lk=96, seed=12)
    run_checked(dev, call, check_fp64=False)


def test_generic_unaligned(dev):
    call = make_call(B=2, H=3, D=64, Lq=40, Lk=50, pad_cols=1, seed=4, bias_mode=_lib.SA_BIAS_RELPOS,
                     mask_mode=_lib.SA_MASK_KEY_MASK)
    st = Staged(dev, call)
    assert st.kernel == "generic"
    run_checked(dev, call)


def test_position_bias_builder(dev):
    """sa_t5_position_bias writes the dense [H, Lq, Lk] bias of app/models/t5.js:55-65."""
    import ctypes

    rng = np.random.default_rng(0)
    H, Lq, Lk = 12, 50, 70
    table = rng.standard_normal((32, H), dtype=np.float32)
    lut = _lib.bucket_lut(Lq, Lk)
    tb = dev.from_array(table)
    lb = dev.from_array(lut)
    out = dev.empty((H, Lq, Lk))
    _lib.check(_lib.load().sa_t5_position_bias(tb.ptr, lb.ptr, 32, H, Lq, Lk, out.ptr, ctypes.c_void_p(dev.stream)))
    dev.sync()
    np.testing.assert_array_equal(out.read(), orc.dense_relpos_bias(table, lut, H, Lq, Lk))


@pytest.mark.parametrize("shape,kernel", [
    (dict(B=1, H=12, D=64, Lq=128, Lk=128), "flash_small16_d64"),        # small launch (96 groups of 16)
    (dict(B=3, H=12, D=64, Lq=128, Lk=128), "flash_small_d64"),          # small launch (144 groups of 32)
    (dict(B=4, H=12, D=64, Lq=256, Lk=100), "flash_mfma_d64_split2"),    # 384 groups: 2-way key split
    (dict(B=22, H=12, D=64, Lq=256, Lk=70), "flash_mfma_d64"),           # 2112 groups: single split
    (dict(B=2, H=4, D=128, Lq=100, Lk=90), "flash_mfma_d128_split2"),
    (dict(B=2, H=3, D=80, Lq=40, Lk=50), "generic"),
])
def test_out_of_range_buckets_clamp_alike_in_every_kernel(dev, shape, kernel):
    """A bucket LUT holding ids outside [0, num_buckets) (out of contract: sa_t5_bucket_lut never
    writes one) gives, in every kernel family, bit for bit the result of the LUT clamped into the
    table, and so does the dense builder."""
    import ctypes

    c1 = make_call(**shape, scale=1.0, bias_mode=_lib.SA_BIAS_RELPOS, num_buckets=8, seed=5)
    rng = np.random.default_rng(6)
    c1.lut = rng.integers(-20, 30, size=c1.lut.shape).astype(np.int32)
    c2 = make_call(**shape, scale=1.0, bias_mode=_lib.SA_BIAS_RELPOS, num_buckets=8, seed=5)
    c2.lut = np.clip(c1.lut, 0, 7).astype(np.int32)
    print(f"[case] clamp {kernel} {shape}", flush=True)
    s1, s2 = Staged(dev, c1), Staged(dev, c2)
    try:
        assert s1.kernel == s2.kernel == kernel
        o1, o2 = s1.run(), s2.run()
    finally:
        s1.release()
        s2.release()
    assert np.isfinite(o1).all()
    np.testing.assert_array_equal(o1, o2)
    H, Lq, Lk = shape["H"], shape["Lq"], shape["Lk"]
    tb = dev.from_array(c1.bias)
    outs = []
    for lut in (c1.lut, c2.lut):
        lb = dev.from_array(lut)
        out = dev.empty((H, Lq, Lk))
        _lib.check(_lib.load().sa_t5_position_bias(tb.ptr, lb.ptr, 8, H, Lq, Lk, out.ptr, ctypes.c_void_p(dev.stream)))
        dev.sync()
        outs.append(out.read())
    np.testing.assert_array_equal(outs[0], outs[1])


@pytest.mark.parametrize("D,Lq,Lk,bias,mask,batched", [
    (256, 70, 300, _lib.SA_BIAS_DENSE, _lib.SA_MASK_KEY_MASK, True),
    (512, 129, 250, _lib.SA_BIAS_DENSE, _lib.SA_MASK_KEY_MASK, False),
    (512, 33, 65, _lib.SA_BIAS_DENSE, _lib.SA_MASK_KEY_LEN, True),
    (256, 1, 257, _lib.SA_BIAS_DENSE, _lib.SA_MASK_NONE, False),
    (512, 100, 90, _lib.SA_BIAS_RELPOS, _lib.SA_MASK_KEY_MASK, False),
])
def test_wide_heads_with_a_bias(dev, D, Lq, Lk, bias, mask, batched):
    """A score bias at head dims 256 and 512 (which the reference's unfused chain serves at any head
    dim, app/gpu/ops.js:119-147): a dense bias runs on the wide kernels, the relative-position gather
    on the generic kernel; ragged Lq/Lk, key masks and key lengths, shared and per-sequence dense
    biases."""
    call = make_call(B=2, H=2, D=D, Lq=Lq, Lk=Lk, bias_mode=bias, mask_mode=mask, dense_bias_batched=batched,
                     key_mask_p=0.6, seed=D + Lq + Lk)
    run_checked(dev, call, expect_kernel=f"wide_mfma_d{D}" if bias == _lib.SA_BIAS_DENSE else "generic")
