"""CPU oracle for the safetensors weight loader (supra_weights.h).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker. The product path never calls it.

Restates app/weights.js in NumPy:

- `parse`       SafeTensors.open (weights.js:40-47): 8-byte little-endian header length, a JSON
                header (JSON.parse semantics: a repeated key keeps its first position and takes
                its last value), "__metadata__" split off, data section after the header.
- `to_f32`      toF32 (weights.js:28-37) with bf16ToF32 (:6-12) and f16ToF32 (:14-25): F32 as is,
                BF16 bits << 16, F16 by the reference's formula evaluated in float64, every other
                dtype through a float64 (JS Number) and then Float32Array's round-to-nearest-even.
                NaN results of F16/F64 decoding take the bit pattern 0x7fc00000 (JS's NaN stored
                into a Float32Array).
- `rows`        rows (weights.js:73-83): gather rows of a 2-D table by id; ids outside the table
                give zero rows here (the reference reads the bytes that follow the table).
- `conv3_pack`  uploadConv3 (weights.js:105-118): [cout, cin, 3, 3] -> [cout, 3, 3, cin_pad]
                with zero padding.
- `linear_shape` uploadLinear (weights.js:87-93): N = shape[0], K = product of the rest.

Pinned in tests/test_oracle_weights.py against the `safetensors` library (0.8.0) for the file
format, torch's bfloat16 and NumPy's float16/float64/int conversions for the decoders (all 65536
half and bfloat16 bit patterns), a double-rounding case for I64, and torch's permute for the conv
layout.
"""

from __future__ import annotations

import json
import struct

import numpy as np

# weights.js:4
BYTES = {"F64": 8, "F32": 4, "BF16": 2, "F16": 2, "I64": 8, "I32": 4, "I16": 2, "I8": 1, "U8": 1, "BOOL": 1}
_NP = {"F64": "<f8", "I64": "<i8", "I32": "<i4", "I16": "<i2", "I8": "i1", "U8": "u1", "BOOL": "u1"}
CANONICAL_NAN = np.uint32(0x7FC00000)


def parse(buf: bytes) -> tuple[dict, dict, int]:
    """(header without __metadata__, metadata, data_start) of a whole safetensors file."""
    (n,) = struct.unpack_from("<Q", buf, 0)
    header = json.loads(bytes(buf[8:8 + n]).decode("utf-8"))
    metadata = header.pop("__metadata__", None) or {}
    return header, metadata, 8 + n


def tensor_bytes(buf: bytes, header: dict, data_start: int, name: str) -> bytes:
    """f32()'s slice (weights.js:66-70): the raw bytes of one tensor."""
    if name not in header:
        raise KeyError(f"missing tensor {name}")
    a, b = header[name]["data_offsets"]
    return bytes(buf[data_start + a:data_start + b])


def bf16_to_f32(raw: bytes) -> np.ndarray:
    u16 = np.frombuffer(raw, dtype="<u2")
    return (u16.astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(raw: bytes) -> np.ndarray:
    h = np.frombuffer(raw, dtype="<u2").astype(np.int64)
    s = np.where(h & 0x8000, -1.0, 1.0)
    e = (h >> 10) & 31
    m = (h & 1023).astype(np.float64)
    with np.errstate(invalid="ignore"):
        val = np.where(e == 0, s * m * 2.0 ** -24,
                       np.where(e == 31, np.where(m != 0, np.nan, s * np.inf),
                                s * (1.0 + m / 1024.0) * np.exp2((e - 15).astype(np.float64))))
    out = val.astype(np.float32)
    out.view(np.uint32)[np.isnan(out)] = CANONICAL_NAN
    return out


def to_f32(raw: bytes, dtype: str) -> np.ndarray:
    if dtype == "F32":
        return np.frombuffer(raw, dtype="<f4").copy()
    if dtype == "BF16":
        return bf16_to_f32(raw)
    if dtype == "F16":
        return f16_to_f32(raw)
    if dtype not in _NP:
        raise ValueError(f"unsupported dtype {dtype}")
    # Number(x) then a Float32Array store: int64 -> nearest double (ties to even), then to float32
    num = np.frombuffer(raw, dtype=_NP[dtype]).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        out = num.astype(np.float32)
    out.view(np.uint32)[np.isnan(out)] = CANONICAL_NAN
    return out


def rows(table_raw: bytes, dtype: str, n_rows: int, dim: int, ids) -> np.ndarray:
    t = to_f32(table_raw, dtype).reshape(n_rows, dim) if n_rows * dim else np.zeros((n_rows, dim), np.float32)
    ids = np.asarray(ids, dtype=np.int64)
    out = np.zeros((ids.size, dim), dtype=np.float32)
    ok = (ids >= 0) & (ids < n_rows)
    out[ok] = t[ids[ok]]
    return out


def conv3_pack(w: np.ndarray, cout: int, cin: int, cin_pad: int = 0) -> np.ndarray:
    """w: float32 [cout * cin * 9] in [cout, cin, 3, 3] order -> [cout * 9 * cin_pad]."""
    cp = cin_pad or cin
    w = np.asarray(w, dtype=np.float32).reshape(cout, cin, 9)
    out = np.zeros((cout, 9, cp), dtype=np.float32)
    for t in range(9):  # out[(o*9 + t)*cp + i] = w[(o*cin + i)*9 + t]
        out[:, t, :cin] = w[:, :, t]
    return out.reshape(-1)


def linear_shape(shape) -> tuple[int, int]:
    N = int(shape[0])
    K = int(np.prod(shape[1:], dtype=np.int64)) if len(shape) > 1 else 1
    return N, K
