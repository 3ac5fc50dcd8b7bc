"""Parity of the device-side weight loader (include/supra_weights.h) with the oracle, bit for bit:

- sa_to_f32 for every decoded dtype: all 65536 half and bfloat16 patterns, random and special
  values of the others, sources at every byte offset (element-aligned vector path, unaligned byte
  path) and destinations at 4-byte offsets (float4 and single-float stores), ragged lengths, and a
  large BF16 tensor;
- sa_rows_f32 (the T5 embedding gather) with repeated and out-of-range ids;
- sa_conv3_pack_f32 at the VAE shapes (conv_in padded 4 -> 8, 512 -> 512, a ragged channel count);
- whole files written by the `safetensors` library: bulk upload through pinned staging (several
  chunks) and without it, every tensor decoded, uploadLinear weights driving sa_linear_f32.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
from safetensors.numpy import save as st_save

from oracle import linear as ol
from oracle import weights as ow
from supra_attn import _lib
from supra_attn.linear_workloads import make_linear
from supra_attn.weights import PinnedBuffer, SafeTensors, upload_conv3, upload_linear, upload_vector

pytestmark = pytest.mark.gpu

NP_OF = {"F32": "<f4", "F16": "<f2", "BF16": "<u2", "F64": "<f8", "I64": "<i8", "I32": "<i4", "I16": "<i2",
         "I8": "i1", "U8": "u1", "BOOL": "u1"}


def _raw(dtype: str, n: int, seed: int) -> bytes:
    rng = np.random.default_rng(seed)
    if dtype in ("F16", "BF16"):
        return rng.integers(0, 65536, n, dtype=np.uint16).astype("<u2").tobytes()
    if dtype in ("F32", "F64"):
        x = rng.standard_normal(n) * np.exp2(rng.integers(-60, 60, n))
        specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -3.5e38, 1 + 2.0 ** -24], dtype=np.float64)
        x[: min(n, specials.size)] = specials[: min(n, specials.size)]
        with np.errstate(over="ignore"):
            return x.astype(NP_OF[dtype]).tobytes()
    info = np.iinfo(np.dtype(NP_OF[dtype]))
    if dtype == "BOOL":
        return rng.integers(0, 2, n, dtype=np.uint8).tobytes()
    return rng.integers(info.min, info.max, n, dtype=np.dtype(NP_OF[dtype]), endpoint=True).tobytes()


def _decode(dev, raw: bytes, dtype: str, n: int, src_off: int = 0, dst_off: int = 0) -> np.ndarray:
    src = dev.empty([src_off + len(raw) + 16], np.uint8)
    host = np.zeros(src.size, np.uint8)
    host[src_off:src_off + len(raw)] = np.frombuffer(raw, np.uint8)
    src.upload(host)
    dst = dev.empty([dst_off + n + 8], np.float32).fill_bytes(0xAB)
    _lib.check(_lib.load().sa_to_f32(src.ptr + src_off, _lib.SA_DT[dtype], n, dst.ptr + 4 * dst_off, dev.stream))
    out = dst.read()
    guard = np.full(1, 0xABABABAB, np.uint32).view(np.float32)[0]
    assert np.all(out[:dst_off].view(np.uint32) == guard.view(np.uint32)), "wrote before dst"
    assert np.all(out[dst_off + n:].view(np.uint32) == guard.view(np.uint32)), "wrote past dst + n"
    src.release()
    dst.release()
    return out[dst_off:dst_off + n]


def _bits_equal(got: np.ndarray, want: np.ndarray):
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", ["F16", "BF16"])
def test_all_half_patterns(dev, dtype):
    raw = np.arange(65536, dtype="<u2").tobytes()
    _bits_equal(_decode(dev, raw, dtype, 65536), ow.to_f32(raw, dtype))


@pytest.mark.parametrize("dtype", list(NP_OF))
@pytest.mark.parametrize("n", [1, 3, 17, 1000, 100_003])
def test_to_f32_every_dtype(dev, dtype, n):
    raw = _raw(dtype, n, seed=n)
    _bits_equal(_decode(dev, raw, dtype, n), ow.to_f32(raw, dtype))


@pytest.mark.parametrize("dtype", ["F32", "F16", "BF16", "F64", "I64", "I8"])
def test_to_f32_offsets(dev, dtype):
    """Every source byte offset 0..15 (unaligned ones take the byte path) and destination offsets
    that do and do not leave the float4 stores aligned."""
    n = 777
    raw = _raw(dtype, n, seed=7)
    want = ow.to_f32(raw, dtype)
    for src_off in range(16):
        for dst_off in (0, 1, 3):
            _bits_equal(_decode(dev, raw, dtype, n, src_off, dst_off), want)


def test_to_f32_large_bf16(dev):
    n = (64 << 20) + 5
    raw = _raw("BF16", n, seed=9)
    _bits_equal(_decode(dev, raw, "BF16", n, src_off=2), ow.to_f32(raw, "BF16"))


@pytest.mark.parametrize("dtype", ["F32", "BF16", "F16"])
def test_rows(dev, dtype):
    rows, dim = 32128, 768  # the T5 shared embedding
    raw = _raw(dtype, rows * dim, seed=3) if dtype != "F32" else \
        np.random.default_rng(3).standard_normal(rows * dim).astype("<f4").tobytes()
    ids = np.array([0, 31, 5, 5, rows - 1, -1, rows, 1234, 2 ** 31 - 1, -(2 ** 31)] + list(range(100, 218)), np.int32)
    table = dev.from_array(np.frombuffer(raw, np.uint8))
    ids_d = dev.from_array(ids)
    out = dev.empty([ids.size, dim], np.float32)
    _lib.check(_lib.load().sa_rows_f32(table.ptr, _lib.SA_DT[dtype], rows, dim, ids_d.ptr, ids.size, out.ptr,
                                       dev.stream))
    _bits_equal(out.read(), ow.rows(raw, dtype, rows, dim, ids))
    for b in (table, ids_d, out):
        b.release()


@pytest.mark.parametrize("cout,cin,cp,dtype", [(128, 4, 8, "F32"), (512, 512, 0, "F32"), (64, 300, 304, "F16"),
                                               (3, 128, 0, "BF16"), (5, 1, 8, "F64")])
def test_conv3_pack(dev, cout, cin, cp, dtype):
    raw = _raw(dtype, cout * cin * 9, seed=cout + cin)
    w = dev.from_array(np.frombuffer(raw, np.uint8))
    out = dev.empty([cout * 9 * (cp or cin)], np.float32)
    _lib.check(_lib.load().sa_conv3_pack_f32(w.ptr, _lib.SA_DT[dtype], cout, cin, cp, out.ptr, dev.stream))
    _bits_equal(out.read(), ow.conv3_pack(ow.to_f32(raw, dtype), cout, cin, cp))
    w.release()
    out.release()


def _model_file(tmp_path):
    """A DiT-block-shaped file as tools/build_models.py writes it (float32), plus tensors of the other
    dtypes and a VAE conv, ~11 MB of data."""
    rng = np.random.default_rng(21)
    t = {
        "blocks.0.self_attn.qkv.weight": (rng.standard_normal((1728, 576)) / 24).astype(np.float32),
        "blocks.0.self_attn.qkv.bias": (rng.standard_normal(1728) * 0.1).astype(np.float32),
        "blocks.0.mlp.0.weight": (rng.standard_normal((1152, 576)) / 24).astype(np.float16),
        "blocks.0.mlp.0.bias": (rng.standard_normal(1152) * 0.1).astype(np.float16),
        "decoder.conv_in.weight": rng.standard_normal((512, 4, 3, 3)).astype(np.float32),
        "decoder.conv_in.bias": rng.standard_normal(512).astype(np.float32),
        "shared.weight": rng.standard_normal((1000, 768)).astype(np.float32),
        "pos": np.arange(11, dtype=np.int64),
        "odd": rng.standard_normal(3).astype(np.float64),
        "flag": np.array([True, False, True]),
    }
    buf = st_save(t, metadata={"format": "pt"})
    path = tmp_path / "model.safetensors"
    path.write_bytes(buf)
    return str(path), buf


@pytest.mark.parametrize("staging", [None, 2 << 20])
def test_file_upload_and_decode(dev, tmp_path, staging):
    path, buf = _model_file(tmp_path)
    header, _, start = ow.parse(buf)
    with SafeTensors.open(path) as st:
        pinned = PinnedBuffer(staging) if staging else None
        if pinned is None:
            res = dev.empty([st.data_bytes], np.uint8)
            _lib.check(_lib.load().sa_st_upload(st._h, 0, st.data_bytes, res.ptr, None, 0, dev.stream))
            st._resident[id(dev)] = res
        resident = st.resident(dev, staging=pinned)
        assert np.array_equal(resident.read(), np.frombuffer(buf[start:], np.uint8))
        for name, e in header.items():
            got = st.f32(dev, name).read().reshape(-1)
            _bits_equal(got, ow.to_f32(ow.tensor_bytes(buf, header, start, name), e["dtype"]))
        # a sub-range upload lands exactly there
        a, b = header["shared.weight"]["data_offsets"]
        part = dev.empty([b - a + 3], np.uint8).fill_bytes(7)
        _lib.check(_lib.load().sa_st_upload(st._h, a, b, part.ptr + 3, pinned.ptr if pinned else None,
                                            pinned.nbytes if pinned else 0, dev.stream))
        host = part.read()
        assert np.all(host[:3] == 7) and host[3:].tobytes() == buf[start + a:start + b]
        # rows, conv and vectors through the reference-shaped helpers
        ids = [3, 999, 0, 3]
        _bits_equal(st.rows(dev, "shared.weight", ids).read(),
                    ow.rows(ow.tensor_bytes(buf, header, start, "shared.weight"), "F32", 1000, 768, ids))
        conv = upload_conv3(dev, st, "decoder.conv_in.", 8)
        assert (conv["N"], conv["K"]) == (512, 72)
        _bits_equal(conv["buf"].read().reshape(-1),
                    ow.conv3_pack(ow.to_f32(ow.tensor_bytes(buf, header, start, "decoder.conv_in.weight"), "F32"),
                                  512, 4, 8))
        _bits_equal(upload_vector(dev, st, "decoder.conv_in.bias").read(),
                    ow.to_f32(ow.tensor_bytes(buf, header, start, "decoder.conv_in.bias"), "F32"))
        if pinned:
            pinned.release()


def test_loaded_weights_drive_the_linear_layer(dev, tmp_path):
    """uploadLinear from a file (float32 and float16 weights) feeding sa_linear_f32: the same result
    as the oracle's linear on the decoded weights, to the linear layer's 1e-5 bar."""
    path, buf = _model_file(tmp_path)
    header, _, start = ow.parse(buf)
    with SafeTensors.open(path) as st:
        for base, act in (("blocks.0.self_attn.qkv.", _lib.SA_ACT_NONE), ("blocks.0.mlp.0.", _lib.SA_ACT_GELU_TANH)):
            layer = upload_linear(dev, st, base)
            N, K = layer["N"], layer["K"]
            w = ow.to_f32(ow.tensor_bytes(buf, header, start, base + "weight"), header[base + "weight"]["dtype"])
            b = ow.to_f32(ow.tensor_bytes(buf, header, start, base + "bias"), header[base + "bias"]["dtype"])
            call = make_linear(base, 512, N, K, seed=4, act=act)
            x = dev.from_array(call.x)
            y = dev.empty([512, N], np.float32)
            args = _lib.LinearArgs(M=512, N=N, K=K, x=x.ptr, w=layer["buf"].ptr, bias=layer["bias"].ptr, act=act,
                                   y=y.ptr)
            dev.linear(args)
            got = y.read()
            want = ol.linear_torch_fp32(call.x, w.reshape(N, K), np.zeros(512 * N, np.float32), M=512, N=N, K=K,
                                        bias=b, act=act).reshape(512, N)
            err = ol.errors(got, want)
            assert err["finite"] and err["rel_l2"] <= 1e-5 and err["max_rel"] <= 1e-5, (base, err)
            for buf_ in (x, y, layer["buf"], layer["bias"]):
                buf_.release()


def test_pinned_staging_too_small_is_rejected(dev, tmp_path):
    path, _ = _model_file(tmp_path)
    with SafeTensors.open(path) as st:
        small = PinnedBuffer(1 << 20)
        dst = dev.empty([st.data_bytes], np.uint8)
        rc = _lib.load().sa_st_upload(st._h, 0, st.data_bytes, dst.ptr, small.ptr, small.nbytes, dev.stream)
        assert rc == _lib.SA_ERR_INVALID and b"staging" in _lib.load().sa_last_error()
        small.release()
        dst.release()
