"""Pins of the CPU oracle (oracle/attention.py, oracle/t5_bucket.py), CPU only.

The reference commits no operator-level golden vectors (its dumps need network-fetched weights), so
the oracle is pinned by:
- an independent library implementation: torch.nn.functional.scaled_dot_product_attention (plain
  and boolean-masked attention), transformers' T5Attention module (relative-position bias, additive
  key mask) and T5Attention._relative_position_bucket (bucket function);
- the closed forms and invariants the mathematics fixes (uniform scores give the mean of V, one key
  gives its value row, per-row shifts and key permutations change nothing, masked keys equal
  removed keys, linearity in V, the bucket thresholds 8, 12, 16, 23, 32, 46, 64, 91);
- the tools/reference.py formulation on the callers' packed layouts.
Each plausible mistake (transposed bias, dropped scale, wrong mask polarity, wrong head offset) is
planted in a copy of the oracle below and must be caught by one of these checks.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as orc
from oracle import t5_bucket as tb

RNG = np.random.default_rng(1234)


def rand(*shape, std=1.0):
    return (RNG.standard_normal(shape) * std).astype(np.float32)


# ---------------------------------------------------------------- library agreement


@pytest.mark.parametrize("B,H,Lq,Lk,D", [(2, 9, 256, 256, 64), (1, 1, 1024, 1024, 512), (3, 2, 17, 45, 32)])
def test_fp64_matches_torch_sdpa(B, H, Lq, Lk, D):
    Q, K, V = rand(B, H, Lq, D), rand(B, H, Lk, D), rand(B, H, Lk, D)
    scale = 1 / math.sqrt(D)
    got = orc.attention_fp64(Q, K, V, scale=scale)
    with torch.no_grad():
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(Q).double(), torch.from_numpy(K).double(), torch.from_numpy(V).double(), scale=scale)
    np.testing.assert_allclose(got, ref.numpy().transpose(0, 2, 1, 3), rtol=1e-10, atol=1e-12)
    e = orc.errors(orc.attention_torch_fp32(Q, K, V, scale=scale), got)
    assert e["rel_l2"] < 2e-6 and e["max_rel"] < 5e-6


def test_masked_fp64_matches_torch_sdpa_bool_mask():
    B, H, Lq, Lk, D = 3, 4, 20, 50, 64
    Q, K, V = rand(B, H, Lq, D), rand(B, H, Lk, D), rand(B, H, Lk, D)
    valid = RNG.random((B, Lk)) < 0.6
    valid[:, 0] = True
    got = orc.attention_fp64(Q, K, V, scale=0.125, valid=valid)
    with torch.no_grad():
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(Q).double(), torch.from_numpy(K).double(), torch.from_numpy(V).double(),
            attn_mask=torch.from_numpy(valid)[:, None, None, :], scale=0.125)
    np.testing.assert_allclose(got, ref.numpy().transpose(0, 2, 1, 3), rtol=1e-10, atol=1e-12)


def _hf_t5_attention(x, kv_w, table, valid):
    """transformers T5Attention (eager) with q/o projections set to identity and k/v projections
    kv_w = (Wk, Wv): its output is softmax(q k^T + bias + mask) v with q = x, k = x Wk^T, v = x Wv^T."""
    from transformers import T5Config
    from transformers.models.t5.modeling_t5 import T5Attention

    Lq, dm = x.shape
    H = table.shape[1]
    cfg = T5Config(d_model=dm, d_kv=dm // H, num_heads=H, relative_attention_num_buckets=table.shape[0],
                   relative_attention_max_distance=128, is_decoder=False)
    cfg._attn_implementation = "eager"
    att = T5Attention(cfg, has_relative_attention_bias=True).eval().double()
    with torch.no_grad():
        att.q.weight.copy_(torch.eye(dm))
        att.o.weight.copy_(torch.eye(dm))
        att.k.weight.copy_(torch.from_numpy(kv_w[0]))
        att.v.weight.copy_(torch.from_numpy(kv_w[1]))
        att.relative_attention_bias.weight.copy_(torch.from_numpy(table))
        mask = torch.zeros(1, 1, 1, Lq, dtype=torch.float64)
        mask[0, 0, 0, ~torch.from_numpy(valid[0])] = torch.finfo(torch.float64).min
        out = att(torch.from_numpy(x).double()[None], mask=mask)[0][0]
    return out.numpy()


def _t5_case(L=40, H=4, d=16, masked=7, seed=0):
    rng = np.random.default_rng(seed)
    dm = H * d
    x = rng.standard_normal((L, dm))
    wk = rng.standard_normal((dm, dm)) / math.sqrt(dm)
    wv = rng.standard_normal((dm, dm)) / math.sqrt(dm)
    table = rng.standard_normal((32, H)) * 2.0
    valid = np.ones((1, L), dtype=bool)
    valid[0, L - masked:] = False
    k = x @ wk.T
    v = x @ wv.T
    return x, k, v, (wk, wv), table, valid


def _oracle_t5(x, k, v, table, valid, H, bias_fn=None):
    L, dm = x.shape
    d = dm // H
    lut = tb.bucket_lut(L, L)
    bias = (bias_fn or orc.dense_relpos_bias)(table, lut, H, L, L)[None]
    Q = orc.heads(x, B=1, L=L, H=H, D=d, ld=dm)
    K = orc.heads(k, B=1, L=L, H=H, D=d, ld=dm)
    V = orc.heads(v, B=1, L=L, H=H, D=d, ld=dm)
    return orc.attention_fp64(Q, K, V, scale=1.0, bias=bias, valid=valid)[0].reshape(L, dm)


def test_t5_relpos_mask_matches_hf_t5attention():
    x, k, v, kv_w, table, valid = _t5_case()
    ref = _hf_t5_attention(x, kv_w, table, valid)
    got = _oracle_t5(x, k, v, table, valid, H=4)
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-11)
    # the fp32 torch path (HF eager formulation) agrees at fp32 precision
    d = 16
    Q = orc.heads(x.astype(np.float32), B=1, L=40, H=4, D=d, ld=64)
    K = orc.heads(k.astype(np.float32), B=1, L=40, H=4, D=d, ld=64)
    V = orc.heads(v.astype(np.float32), B=1, L=40, H=4, D=d, ld=64)
    bias = orc.dense_relpos_bias(table.astype(np.float32), tb.bucket_lut(40, 40), 4, 40, 40)[None]
    o32 = orc.attention_torch_fp32(Q, K, V, scale=1.0, bias=bias, valid=valid)[0].reshape(40, 64)
    assert orc.errors(o32, ref)["max_rel"] < 5e-6


# ---------------------------------------------------------------- closed forms and invariants


def test_uniform_scores_give_mean_of_values():
    Q = np.zeros((1, 2, 5, 8))
    K, V = rand(1, 2, 9, 8), rand(1, 2, 9, 8)
    out = orc.attention_fp64(Q, K, V, scale=0.3)
    mean = V.astype(np.float64).mean(axis=2)[:, None]
    np.testing.assert_allclose(out, np.broadcast_to(mean, out.shape), rtol=1e-12, atol=1e-12)


def test_single_key_returns_its_value_row():
    Q, K, V = rand(2, 3, 7, 16), rand(2, 3, 1, 16), rand(2, 3, 1, 16)
    out = orc.attention_fp64(Q, K, V, scale=5.0)
    np.testing.assert_allclose(out, np.broadcast_to(V.transpose(0, 2, 1, 3), out.shape), rtol=1e-12)


def test_dominant_key_is_selected():
    K = rand(1, 1, 6, 4)
    Q = 50.0 * K[:, :, 2:3, :]          # query aligned with key 2, huge scale
    V = rand(1, 1, 6, 4)
    out = orc.attention_fp64(Q, K, V, scale=10.0)
    np.testing.assert_allclose(out[0, 0, 0], V[0, 0, 2], rtol=1e-9)


def test_softmax_weights_sum_to_one_constant_values():
    Q, K = rand(2, 2, 11, 8), rand(2, 2, 13, 8)
    V = np.full((2, 2, 13, 8), 3.25)
    np.testing.assert_allclose(orc.attention_fp64(Q, K, V, scale=0.7), 3.25, rtol=1e-12)


def test_row_shift_and_key_permutation_invariance():
    Q, K, V = rand(1, 2, 6, 8), rand(1, 2, 10, 8), rand(1, 2, 10, 8)
    base = orc.attention_fp64(Q, K, V, scale=0.5)
    shift = np.broadcast_to(RNG.standard_normal((1, 2, 6, 1)) * 30, (1, 2, 6, 10))
    np.testing.assert_allclose(orc.attention_fp64(Q, K, V, scale=0.5, bias=shift), base, rtol=1e-10, atol=1e-12)
    perm = RNG.permutation(10)
    np.testing.assert_allclose(orc.attention_fp64(Q, K[:, :, perm], V[:, :, perm], scale=0.5), base, rtol=1e-10, atol=1e-12)


def test_masked_keys_equal_removed_keys_and_empty_rows_are_zero():
    Q, K, V = rand(2, 2, 5, 8), rand(2, 2, 12, 8), rand(2, 2, 12, 8)
    valid = np.zeros((2, 12), dtype=bool)
    valid[0, [1, 4, 5, 11]] = True   # sequence 1 has no attended key
    out = orc.attention_fp64(Q, K, V, scale=0.4, valid=valid)
    keep = [1, 4, 5, 11]
    ref0 = orc.attention_fp64(Q[:1], K[:1, :, keep], V[:1, :, keep], scale=0.4)
    np.testing.assert_allclose(out[:1], ref0, rtol=1e-12)
    assert np.all(out[1] == 0.0)
    assert np.all(orc.attention_torch_fp32(Q, K, V, scale=0.4, valid=valid)[1] == 0.0)


def test_linear_in_values():
    Q, K, V1, V2 = rand(1, 3, 4, 8), rand(1, 3, 9, 8), rand(1, 3, 9, 8), rand(1, 3, 9, 8)
    V1, V2 = V1.astype(np.float64), V2.astype(np.float64)
    a = orc.attention_fp64(Q, K, 2.0 * V1 - 3.0 * V2, scale=0.6)
    b = 2.0 * orc.attention_fp64(Q, K, V1, scale=0.6) - 3.0 * orc.attention_fp64(Q, K, V2, scale=0.6)
    np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


def test_strided_gather_matches_reference_py_layout():
    """heads()/output_view() address packed qkv exactly like tools/reference.py:96-97 views it."""
    from supra_attn import workloads

    call = workloads.dit_self(B=2, seed=5)
    Q, K, V, _, _ = orc.gather_call(call)
    qkv = torch.from_numpy(call.q).view(2, -1, 3, 576)
    for X, idx in ((Q, 0), (K, 1), (V, 2)):
        ref = qkv[:, :, idx].reshape(2, 256, 9, 64).permute(0, 2, 1, 3).numpy()
        np.testing.assert_array_equal(X, ref)
    o_py = orc.cpu_dit_self(call).numpy().reshape(2, 256, 9, 64)
    np.testing.assert_allclose(orc.reference_torch(call), o_py, rtol=0, atol=0)


def test_place_and_output_view_roundtrip():
    O = rand(2, 5, 3, 4)
    buf = np.full(200 + 2 * 70, -1.0, dtype=np.float32)
    placed = orc.place(buf, O, off=7, ld=13, sb=70)
    back = orc.heads(placed, B=2, L=5, H=3, D=4, off=7, ld=13, sb=70).transpose(0, 2, 1, 3)
    np.testing.assert_array_equal(back, O)
    assert (placed == -1.0).sum() == buf.size - O.size


# ---------------------------------------------------------------- T5 buckets


def test_bucket_thresholds_closed_form():
    assert tb.bucket_thresholds() == [8, 12, 16, 23, 32, 46, 64, 91]
    for k, n in enumerate(tb.bucket_thresholds()):
        assert tb.relative_bucket(n) == 16 + 8 + k and tb.relative_bucket(-n) == 8 + k
        assert tb.relative_bucket(n - 1) == 16 + 8 + k - 1
    assert [tb.relative_bucket(-r) for r in range(8)] == list(range(8))
    assert tb.relative_bucket(500) == 31 and tb.relative_bucket(-500) == 15


@pytest.mark.parametrize("bidirectional", [True, False])
def test_buckets_match_hf(bidirectional):
    from transformers.models.t5.modeling_t5 import T5Attention

    rel = torch.arange(-600, 601)
    hf = T5Attention._relative_position_bucket(rel, bidirectional=bidirectional, num_buckets=32, max_distance=128)
    ours = np.array([tb.relative_bucket(int(r), bidirectional) for r in rel])
    np.testing.assert_array_equal(ours, hf.numpy())


def test_bucket_lut_indexing():
    lut = tb.bucket_lut(5, 7)
    assert lut.shape == (11,)
    for i in range(5):
        for j in range(7):
            assert lut[j - i + 4] == tb.relative_bucket(j - i)


# ---------------------------------------------------------------- planted mistakes are caught


def test_transposed_bias_is_caught():
    x, k, v, kv_w, table, valid = _t5_case(seed=3)
    ref = _hf_t5_attention(x, kv_w, table, valid)

    def transposed(table_, lut, H, Lq, Lk):
        return orc.dense_relpos_bias(table_, lut, H, Lq, Lk).transpose(0, 2, 1)

    bad = _oracle_t5(x, k, v, table, valid, H=4, bias_fn=transposed)
    assert orc.errors(bad, ref)["max_rel"] > 1e-3


def test_wrong_mask_polarity_and_dropped_scale_are_caught():
    B, H, Lq, Lk, D = 1, 2, 8, 16, 8
    Q, K, V = rand(B, H, Lq, D), rand(B, H, Lk, D), rand(B, H, Lk, D)
    valid = RNG.random((B, Lk)) < 0.5
    valid[0, 0] = True
    with torch.no_grad():
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(Q).double(), torch.from_numpy(K).double(), torch.from_numpy(V).double(),
            attn_mask=torch.from_numpy(valid)[:, None, None, :], scale=0.3).numpy().transpose(0, 2, 1, 3)
    inv = ~valid
    inv[0, 0] = True
    assert orc.errors(orc.attention_fp64(Q, K, V, scale=0.3, valid=inv), ref)["max_rel"] > 1e-3
    assert orc.errors(orc.attention_fp64(Q, K, V, scale=1.0, valid=valid), ref)["max_rel"] > 1e-3


def test_wrong_head_offset_is_caught():
    from supra_attn import workloads

    call = workloads.dit_self(B=1, seed=6)
    good = orc.cpu_dit_self(call).numpy().reshape(1, 256, 9, 64)
    a = dict(call.args)
    a["k_off"] = a["q_off"]           # planted: K read from the Q columns
    call.args = a
    assert orc.errors(orc.reference_fp64(call), good)["max_rel"] > 1e-2
