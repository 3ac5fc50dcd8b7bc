"""The safetensors header parser of the C library (sa_st_open / sa_st_info / metadata), host only:
no device call is made, so these run without a GPU.

Checked against the oracle's parse (json.loads, pinned to the `safetensors` library in
test_oracle_weights.py) on files the library writes and on hand-made headers covering JSON escapes,
repeated keys, padding and metadata forms, and against the error behaviour app/weights.js has by
way of JSON.parse and info() ("missing tensor <name>"), plus the stricter checks this loader adds
(offsets inside the data section, byte counts matching shape x dtype).
"""

from __future__ import annotations

import ctypes
import json
import struct

import numpy as np
import pytest
from safetensors.numpy import save as st_save

from oracle import weights as ow
from supra_attn import _lib
from supra_attn.weights import SafeTensors


def _file(header: dict | bytes, data: bytes = b"", pad: bytes = b"") -> bytes:
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    h += pad
    return struct.pack("<Q", len(h)) + h + data


def _check_against_oracle(buf: bytes):
    header, meta, start = ow.parse(buf)
    with SafeTensors.from_bytes(buf) as st:
        assert st.names() == list(header)
        got_meta = st.metadata
        assert list(got_meta) == list(meta)
        for k, v in meta.items():  # strings as stored, other values as their JSON text
            assert got_meta[k] == v if isinstance(v, str) else json.loads(got_meta[k]) == v
        assert st.data_bytes == len(buf) - start
        for name, e in header.items():
            assert st.info(name) == {"dtype": e["dtype"], "shape": e["shape"], "data_offsets": e["data_offsets"]}
            t = st.raw_info(name)
            assert t.numel == int(np.prod(e["shape"], dtype=np.int64))
            assert t.elem_bytes == ow.BYTES.get(e["dtype"], t.elem_bytes)
        data = ctypes.string_at(_lib.load().sa_st_data(st._h), st.data_bytes)
        assert data == bytes(buf[start:])
    return header


def test_library_written_file(tmp_path):
    rng = np.random.default_rng(1)
    tensors = {f"blocks.{i}.mlp.0.weight": rng.standard_normal((4, 3)).astype(np.float32) for i in range(3)}
    tensors.update({"h": rng.standard_normal(5).astype(np.float16), "i": np.arange(7, dtype=np.int64),
                    "b": np.array([True, False]), "s": np.array(1.0, dtype=np.float64)})
    buf = st_save(tensors, metadata={"format": "pt", "dim": "576"})
    _check_against_oracle(buf)
    path = tmp_path / "w.safetensors"
    path.write_bytes(buf)
    with SafeTensors.open(str(path)) as st:
        assert st.has("h") and not st.has("nope")
        assert st.metadata == {"format": "pt", "dim": "576"}
        assert st.info("i") == {"dtype": "I64", "shape": [7], "data_offsets": st.info("i")["data_offsets"]}


def test_json_forms():
    hdr = (b'  {"__metadata__": {"k": "v\\u00e9\\ud83d\\ude00", "n": 3, "o": {"x": [1, 2]}},\n'
           b'"a\\"b": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8], "extra": {"deep": [[{}]]}},'
           b'"s": {"shape": [], "data_offsets": [8, 12], "dtype": "I32"},'
           b'"z": {"dtype": "F16", "shape": [0, 5], "data_offsets": [12, 12]},'
           b'"a\\"b": {"dtype": "I32", "shape": [1, 2], "data_offsets": [0, 8]}}')
    buf = _file(hdr, b"\0" * 12, pad=b"    \t\n")
    header = _check_against_oracle(buf)
    assert list(header) == ['a"b', "s", "z"]
    with SafeTensors.from_bytes(buf) as st:
        assert st.metadata["k"] == "vé\U0001F600"
        assert st.info('a"b')["dtype"] == "I32"  # repeated key: first position, last value
        assert st.raw_info("s").ndim == 0 and st.raw_info("s").numel == 1
        assert st.raw_info("z").numel == 0


def test_empty_header_and_unknown_dtype():
    with SafeTensors.from_bytes(_file({})) as st:
        assert st.names() == [] and st.metadata == {} and st.data_bytes == 0
    buf = _file({"q": {"dtype": "F4_E2M1X", "shape": [3], "data_offsets": [0, 2]}}, b"\0\0")
    with SafeTensors.from_bytes(buf) as st:
        t = st.raw_info("q")
        assert t.dtype == _lib.SA_DT["OTHER"] and t.elem_bytes == 0 and t.dtype_name == b"F4_E2M1X"
    buf = _file({"u": {"dtype": "U16", "shape": [3], "data_offsets": [0, 6]}}, b"\0" * 6)
    with SafeTensors.from_bytes(buf) as st:
        assert st.raw_info("u").dtype == _lib.SA_DT["U16"] and st.raw_info("u").elem_bytes == 2


def _open_code(buf: bytes) -> tuple[int, str]:
    lib = _lib.load()
    arr = np.frombuffer(buf, dtype=np.uint8) if buf else np.zeros(0, np.uint8)
    h = ctypes.c_void_p()
    rc = lib.sa_st_open_memory(arr.ctypes.data if arr.size else 1, len(buf), ctypes.byref(h))
    if rc == _lib.SA_OK:
        lib.sa_st_close(h)
    return rc, lib.sa_last_error().decode()


ENTRY = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}


@pytest.mark.parametrize("buf,why", [
    (b"", "no header length"),
    (b"\x05\0\0", "no header length"),
    (struct.pack("<Q", 100) + b"{}", "exceeds the file"),
    (_file(b"[]"), "not a JSON object"),
    (_file(b'{"a": '), "tensor a: a tensor entry is not an object"),
    (_file(b'{"a": {"dtype": "F32", "shape": [2]}}', b"\0" * 8), "lacks"),
    (_file({"a": ENTRY}, b"\0" * 4), "outside"),
    (_file({"a": {**ENTRY, "data_offsets": [8, 0]}}, b"\0" * 8), "outside"),
    (_file({"a": {**ENTRY, "shape": [3]}}, b"\0" * 8), "bytes for 3 elements"),
    (_file(b'{"a": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}', b"\0" * 8), "non-negative"),
    (_file(b'{"a": {"dtype": "F32", "shape": [2.0], "data_offsets": [0, 8]}}', b"\0" * 8), "fraction"),
    (_file(b'{"a": {"dtype": "F32", "shape": [02], "data_offsets": [0, 8]}}', b"\0" * 8), "leading zero"),
    (_file(b'{"a": {"dtype": "F32", "shape": [1,1,1,1,1,1,1,1,2], "data_offsets": [0, 8]}}', b"\0" * 8), "8 dim"),
    (_file(b'{"a": {"dtype": "F32", "shape": [99999999999999999999], "data_offsets": [0, 8]}}'), "too large"),
    (_file(b'{"a": {"dtype": "F32", "shape": [4294967296, 4294967296], "data_offsets": [0, 8]}}'), "overflows"),
    (_file(b'{"a": 1}'), "not an object"),
    (_file(b'{"__metadata__": []}'), "__metadata__"),
    (_file(b'{} x'), "after its JSON"),
    (_file(b'{"a\x01": {}}'), "control character"),
    (_file(b'{"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8], "x": ' + b"[" * 80 + b"]" * 80 + b"}}",
           b"\0" * 8), "nested"),
])
def test_malformed_files_are_format_errors(buf, why):
    rc, msg = _open_code(buf)
    assert rc == _lib.SA_ERR_FORMAT, msg
    assert why in msg


def test_io_and_lookup_errors(tmp_path):
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.sa_st_open(str(tmp_path / "missing.safetensors").encode(), ctypes.byref(h)) == _lib.SA_ERR_IO
    assert h.value is None
    with SafeTensors.from_bytes(_file({"a": ENTRY}, b"\0" * 8)) as st:
        with pytest.raises(_lib.SaError, match="missing tensor b") as e:
            st.info("b")
        assert e.value.code == _lib.SA_ERR_NOT_FOUND
        t = _lib.StTensor()
        t.struct_size = 8
        assert lib.sa_st_info(st._h, b"a", ctypes.byref(t)) == _lib.SA_ERR_INVALID
        assert lib.sa_st_name(st._h, 1) is None and lib.sa_st_metadata_value(st._h, b"x") is None
        # upload range checks happen before any device call
        assert lib.sa_st_upload(st._h, 4, 12, None, None, 0, None) == _lib.SA_ERR_INVALID
        assert lib.sa_st_upload(st._h, 0, 8, None, None, 0, None) == _lib.SA_ERR_INVALID
        assert lib.sa_st_upload(st._h, 8, 8, None, None, 0, None) == _lib.SA_OK


def test_decode_argument_checks_without_a_device():
    lib = _lib.load()
    assert lib.sa_to_f32(None, _lib.SA_DT["U16"], 4, None, None) == _lib.SA_ERR_UNSUPPORTED
    assert lib.sa_to_f32(None, 99, 4, None, None) == _lib.SA_ERR_INVALID
    assert lib.sa_to_f32(None, _lib.SA_DT["F32"], 0, None, None) == _lib.SA_OK
    assert lib.sa_to_f32(None, _lib.SA_DT["F32"], -1, None, None) == _lib.SA_ERR_INVALID
    assert lib.sa_to_f32(16, _lib.SA_DT["F32"], 4, 18, None) == _lib.SA_ERR_INVALID      # dst misaligned
    assert lib.sa_to_f32(4096, _lib.SA_DT["BF16"], 64, 4096 + 64, None) == _lib.SA_ERR_ALIAS
    assert lib.sa_conv3_pack_f32(4096, _lib.SA_DT["F32"], 2, 8, 4, 65536, None) == _lib.SA_ERR_INVALID  # cin_pad < cin
    assert lib.sa_conv3_pack_f32(4096, _lib.SA_DT["F32"], 2, 8, 8, 4096, None) == _lib.SA_ERR_ALIAS
    assert lib.sa_rows_f32(4096, _lib.SA_DT["F32"], 10, 4, 1 << 20, 70000, 1 << 24, None) == _lib.SA_ERR_UNSUPPORTED
    assert lib.sa_rows_f32(4096, _lib.SA_DT["F32"], 10, 4, 1 << 20, 3, 4096 + 16, None) == _lib.SA_ERR_ALIAS
