"""Pins of the weight-loader oracle (oracle/weights.py) against independent implementations:

- the file format against the `safetensors` library (0.8.0): files it writes parse to the names,
  dtypes, shapes, offsets and metadata it reports, and every tensor decodes to the values it loads;
- bf16ToF32 against torch's bfloat16 -> float32 conversion, bit for bit, over all 65536 patterns;
- f16ToF32 (the reference's formula) against NumPy's float16 -> float32 over all 65536 patterns
  (bit for bit except NaN payloads, which the reference replaces by JS's NaN);
- F64 / I32 / I16 / I8 / U8 / BOOL against NumPy's conversions, with round-to-nearest-even ties,
  overflow to infinity and subnormals;
- I64 through the nearest double, shown by a value where that differs from rounding the integer
  to float32 directly (a plausible mistake);
- the conv re-layout against torch's permute + pad; the row gather against NumPy indexing.
"""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.numpy import save as st_save

from oracle import weights as ow


def _all_u16() -> bytes:
    return np.arange(65536, dtype="<u2").tobytes()


def test_bf16_all_patterns_match_torch():
    raw = _all_u16()
    got = ow.to_f32(raw, "BF16")
    want = torch.from_numpy(np.frombuffer(raw, dtype=np.int16).copy()).view(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_f16_all_patterns_match_numpy():
    raw = _all_u16()
    got = ow.to_f32(raw, "F16")
    want = np.frombuffer(raw, dtype="<f2").astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])
    assert np.all(got.view(np.uint32)[nan] == ow.CANONICAL_NAN)
    # signed zero, the smallest subnormal, the largest finite half, infinities
    special = np.array([0x8000, 0x0001, 0x8001, 0x7BFF, 0x7C00, 0xFC00], dtype="<u2").tobytes()
    vals = ow.to_f32(special, "F16")
    assert vals[0] == 0 and np.signbit(vals[0])
    assert vals[1] == 2.0 ** -24 and vals[2] == -(2.0 ** -24)
    assert vals[3] == 65504.0 and vals[4] == np.inf and vals[5] == -np.inf


def test_f64_rounding_overflow_and_nan():
    x = np.array([1.0, 1 + 2.0 ** -24, 1 + 3 * 2.0 ** -24, 1 + 2.0 ** -23 + 2.0 ** -24, 3.5e38, -3.5e38, 1e-46,
                  -0.0, np.nan, 2.0 ** -149, 0.1], dtype="<f8")
    got = ow.to_f32(x.tobytes(), "F64")
    with np.errstate(over="ignore"):
        want = x.astype(np.float32)
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got.view(np.uint32)[ok], want.view(np.uint32)[ok])
    assert got[1] == 1.0                         # tie to even (down)
    assert got[2] == np.float32(1 + 2.0 ** -22)  # tie to even (up)
    assert got[4] == np.inf and got[5] == -np.inf
    assert got.view(np.uint32)[8] == ow.CANONICAL_NAN


def test_i64_goes_through_the_nearest_double():
    x = 2 ** 62 + 2 ** 38 + 1  # just above a float32 midpoint; the double loses the +1 -> tie -> even
    got = ow.to_f32(np.array([x, -x, 2 ** 24 + 1, -(2 ** 63), 2 ** 63 - 1], dtype="<i8").tobytes(), "I64")
    assert got[0] == np.float32(2.0 ** 62)
    direct = 2 ** 62 + 2 ** 39  # the float32 nearest to x itself: rounding the integer directly gives this
    assert abs(x - direct) < abs(x - 2 ** 62) and got[0] != np.float32(direct)
    assert got[1] == -got[0]
    assert got[2] == np.float32(2 ** 24)  # tie to even
    assert got[3] == np.float32(-(2.0 ** 63)) and got[4] == np.float32(2.0 ** 63)
    for v, g in zip([x, -x, 2 ** 24 + 1], got):
        assert struct.unpack("<f", struct.pack("<f", float(v)))[0] == g


@pytest.mark.parametrize("dtype,npdt", [("I32", "<i4"), ("I16", "<i2"), ("I8", "i1"), ("U8", "u1"), ("BOOL", "u1")])
def test_integer_types_match_numpy(dtype, npdt):
    info = np.iinfo(np.dtype(npdt))
    rng = np.random.default_rng(3)
    x = np.concatenate([np.array([info.min, info.max, 0, 1, -1 if info.min < 0 else 2], dtype=npdt),
                        rng.integers(info.min, info.max, 1000, dtype=npdt, endpoint=True)])
    got = ow.to_f32(x.tobytes(), dtype)
    np.testing.assert_array_equal(got, x.astype(np.float64).astype(np.float32))
    if dtype == "I32":
        assert ow.to_f32(np.array([2 ** 24 + 1, 2 ** 31 - 1], dtype="<i4").tobytes(), "I32").tolist() == [2.0 ** 24, 2.0 ** 31]


def test_unsupported_dtypes_raise():
    for dt in ("U16", "U32", "U64", "F8_E4M3", "F8_E5M2", "C64"):
        with pytest.raises(ValueError, match="unsupported dtype"):
            ow.to_f32(b"\0" * 8, dt)


def _library_file():
    rng = np.random.default_rng(11)
    tensors = {
        "w.f32": rng.standard_normal((7, 5)).astype(np.float32),
        "w.f16": rng.standard_normal((3, 4, 2)).astype(np.float16),
        "w.f64": rng.standard_normal(9),
        "w.i64": rng.integers(-(2 ** 40), 2 ** 40, (4, 3)),
        "w.i32": rng.integers(-(2 ** 31), 2 ** 31 - 1, 6, dtype=np.int32),
        "w.i16": rng.integers(-300, 300, 5).astype(np.int16),
        "w.i8": rng.integers(-128, 127, 11).astype(np.int8),
        "w.u8": rng.integers(0, 255, 13).astype(np.uint8),
        "w.bool": rng.integers(0, 2, 3).astype(bool),
        "scalar": np.array(2.5, dtype=np.float32),
        "empty": np.zeros((0, 4), dtype=np.float32),
    }
    meta = {"format": "pt", "config": json.dumps({"dim": 576})}
    return tensors, meta, st_save(tensors, metadata=meta)


def test_parse_matches_safetensors_library(tmp_path):
    tensors, meta, buf = _library_file()
    header, metadata, start = ow.parse(buf)
    assert metadata == meta
    assert set(header) == set(tensors)
    path = tmp_path / "lib.safetensors"
    path.write_bytes(buf)
    with safe_open(str(path), framework="np") as f:
        assert set(f.keys()) == set(header)
        assert f.metadata() == meta
        for name in f.keys():
            want = f.get_tensor(name)
            assert list(want.shape) == header[name]["shape"]
            got = ow.to_f32(ow.tensor_bytes(buf, header, start, name), header[name]["dtype"])
            np.testing.assert_array_equal(got, want.astype(np.float64).astype(np.float32).reshape(-1))
    with pytest.raises(KeyError, match="missing tensor"):
        ow.tensor_bytes(buf, header, start, "nope")


def test_parse_bf16_tensor_matches_torch_library():
    from safetensors.torch import save as st_save_torch

    t = torch.randn(6, 10).to(torch.bfloat16)
    buf = st_save_torch({"x": t})
    header, _, start = ow.parse(buf)
    assert header["x"]["dtype"] == "BF16"
    got = ow.to_f32(ow.tensor_bytes(buf, header, start, "x"), "BF16")
    np.testing.assert_array_equal(got, t.float().numpy().reshape(-1))


def test_parse_json_semantics_of_repeated_keys():
    hdr = b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}, "b": {"dtype": "F32", "shape": [], ' \
          b'"data_offsets": [4, 8]}, "a": {"dtype": "I32", "shape": [1], "data_offsets": [4, 8]}}'
    buf = struct.pack("<Q", len(hdr)) + hdr + struct.pack("<fi", 1.5, 7)
    header, metadata, start = ow.parse(buf)
    assert list(header) == ["a", "b"] and header["a"]["dtype"] == "I32" and metadata == {}
    assert ow.to_f32(ow.tensor_bytes(buf, header, start, "a"), "I32").tolist() == [7.0]


def test_rows_matches_indexing():
    rng = np.random.default_rng(5)
    table = rng.standard_normal((50, 12)).astype(np.float32)
    ids = np.array([3, 0, 49, 3, 17])
    np.testing.assert_array_equal(ow.rows(table.tobytes(), "F32", 50, 12, ids), table[ids])
    out = ow.rows(table.tobytes(), "F32", 50, 12, [-1, 50, 2])
    assert not out[0].any() and not out[1].any()
    np.testing.assert_array_equal(out[2], table[2])


@pytest.mark.parametrize("cout,cin,cp", [(3, 4, 8), (5, 7, 0), (2, 16, 16)])
def test_conv3_pack_matches_torch_permute(cout, cin, cp):
    w = torch.randn(cout, cin, 3, 3)
    got = ow.conv3_pack(w.numpy().reshape(-1), cout, cin, cp)
    want = torch.nn.functional.pad(w.permute(0, 2, 3, 1), (0, (cp or cin) - cin)).contiguous().numpy().reshape(-1)
    np.testing.assert_array_equal(got, want)


def test_linear_shape():
    assert ow.linear_shape([1728, 576]) == (1728, 576)
    assert ow.linear_shape([512, 256, 1, 1]) == (512, 256)  # 1x1 conv shortcut (vae.js:24)
