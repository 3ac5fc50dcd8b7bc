"""ctypes binding of libsupra_attn.so (include/supra_attn.h, supra_linear.h, supra_vae.h).

Loading fails loudly when the library has not been built: there is no other implementation of the
operator behind this module.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG, "lib", "libsupra_attn.so")

SA_OK = 0
SA_ERR_INVALID = -1
SA_ERR_UNSUPPORTED = -2
SA_ERR_HIP = -3
SA_ERR_ALIAS = -4
SA_ERR_NOT_FOUND = -5
SA_ERR_IO = -6
SA_ERR_FORMAT = -7

SA_BIAS_NONE = 0
SA_BIAS_DENSE = 1
SA_BIAS_RELPOS = 2

SA_MASK_NONE = 0
SA_MASK_KEY_LEN = 1
SA_MASK_KEY_MASK = 2

SA_ACT_NONE = 0
SA_ACT_GELU = 1
SA_ACT_GELU_TANH = 2
SA_ACT_SILU = 3

SA_EPI_STORE = 0
SA_EPI_RESID = 1
SA_EPI_RESID_GATE = 2

# safetensors dtypes (include/supra_weights.h)
SA_DT = {"OTHER": 0, "F32": 1, "F16": 2, "BF16": 3, "F64": 4, "I64": 5, "I32": 6, "I16": 7, "I8": 8, "U8": 9,
         "BOOL": 10, "U16": 11, "U32": 12, "U64": 13, "F8_E4M3": 14, "F8_E5M2": 15}
SA_ST_MAX_DIMS = 8

# Every symbol include/*.h declares, with (restype, argtypes).
SIGNATURES = {
    "sa_attention_f32": (c_int, [c_void_p, c_void_p]),
    "sa_attention_f32_noalloc": (c_int, [c_void_p, c_void_p]),
    "sa_attention_kernel_name": (c_char_p, [c_void_p]),
    "sa_attention_workspace_bytes": (c_int64, [c_void_p]),
    "sa_attention_plan": (c_int, [c_void_p, c_void_p]),
    "sa_attention_variant_count": (c_int32, []),
    "sa_attention_variant": (c_int, [c_int32, c_void_p]),
    "sa_linear_f32": (c_int, [c_void_p, c_void_p]),
    "sa_linear_kernel_name": (c_char_p, [c_void_p]),
    "sa_vae_attention_f32": (c_int, [c_void_p, c_void_p]),
    "sa_vae_attention_workspace_bytes": (c_int64, [c_void_p]),
    "sa_t5_bucket_lut": (c_int, [c_int32, c_int32, c_int32, c_int32, c_int32, POINTER(c_int32)]),
    "sa_t5_position_bias": (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "sa_device_count": (c_int, [POINTER(c_int32)]),
    "sa_set_device": (c_int, [c_int32]),
    "sa_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "sa_free": (c_int, [c_void_p]),
    "sa_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "sa_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "sa_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "sa_memset": (c_int, [c_void_p, c_int, c_size_t, c_void_p]),
    "sa_stream_create": (c_int, [POINTER(c_void_p)]),
    "sa_stream_destroy": (c_int, [c_void_p]),
    "sa_stream_sync": (c_int, [c_void_p]),
    "sa_device_sync": (c_int, []),
    "sa_event_create": (c_int, [POINTER(c_void_p)]),
    "sa_event_destroy": (c_int, [c_void_p]),
    "sa_event_record": (c_int, [c_void_p, c_void_p]),
    "sa_event_elapsed_ms": (c_int, [POINTER(c_float), c_void_p, c_void_p]),
    "sa_malloc_host": (c_int, [POINTER(c_void_p), c_size_t]),
    "sa_free_host": (c_int, [c_void_p]),
    "sa_st_open": (c_int, [c_char_p, POINTER(c_void_p)]),
    "sa_st_open_memory": (c_int, [c_void_p, c_int64, POINTER(c_void_p)]),
    "sa_st_close": (c_int, [c_void_p]),
    "sa_st_count": (c_int64, [c_void_p]),
    "sa_st_name": (c_char_p, [c_void_p, c_int64]),
    "sa_st_info": (c_int, [c_void_p, c_char_p, c_void_p]),
    "sa_st_metadata_count": (c_int64, [c_void_p]),
    "sa_st_metadata_key": (c_char_p, [c_void_p, c_int64]),
    "sa_st_metadata_value": (c_char_p, [c_void_p, c_char_p]),
    "sa_st_data_bytes": (c_int64, [c_void_p]),
    "sa_st_data": (c_void_p, [c_void_p]),
    "sa_st_upload": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_void_p]),
    "sa_to_f32": (c_int, [c_void_p, c_int32, c_int64, c_void_p, c_void_p]),
    "sa_rows_f32": (c_int, [c_void_p, c_int32, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "sa_conv3_pack_f32": (c_int, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "sa_version": (c_int, []),
    "sa_last_error": (c_char_p, []),
    "sa_last_status": (c_int, []),
}

SA_NOALLOC_SCRATCH_BYTES = 32 << 20

SA_KERNEL_FLASH = 1
SA_KERNEL_WIDE = 2
SA_KERNEL_GENERIC = 3
SA_KERNEL_FLASH_SMALL = 4
SA_KERNEL_FLASH_SMALL16 = 5
SA_MASK_VARIANT_KEY_LEN_SCHEDULED = 3


class SaError(RuntimeError):
    """A non-zero status from the C ABI, with its code and sa_last_error() message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"supra_attn error {code}: {message}")
        self.code = code
        self.message = message


class AttnArgs(ctypes.Structure):
    """Mirror of sa_attn_args (include/supra_attn.h)."""

    _fields_ = [
        ("struct_size", c_uint32),
        ("B", c_int32),
        ("H", c_int32),
        ("D", c_int32),
        ("Lq", c_int32),
        ("Lk", c_int32),
        ("q", c_void_p),
        ("k", c_void_p),
        ("v", c_void_p),
        ("o", c_void_p),
        ("q_off", c_int64),
        ("k_off", c_int64),
        ("v_off", c_int64),
        ("o_off", c_int64),
        ("ldq", c_int64),
        ("ldk", c_int64),
        ("ldv", c_int64),
        ("ldo", c_int64),
        ("sq", c_int64),
        ("sk", c_int64),
        ("sv", c_int64),
        ("so", c_int64),
        ("scale", c_float),
        ("bias_mode", c_int32),
        ("bias", c_void_p),
        ("sbias", c_int64),
        ("bucket_lut", c_void_p),
        ("num_buckets", c_int32),
        ("mask_mode", c_int32),
        ("key_len", c_void_p),
        ("key_mask", c_void_p),
        ("smask", c_int64),
        ("workspace", c_void_p),
        ("workspace_bytes", c_int64),
        ("key_len_host", c_void_p),  # revision 3: host copy of key_len, for the sequence schedule
    ]

    def __init__(self, **kw):
        super().__init__()
        self.struct_size = ctypes.sizeof(AttnArgs)
        for name, val in kw.items():
            setattr(self, name, val)


class AttnPlan(ctypes.Structure):
    """Mirror of sa_attn_plan (include/supra_attn.h)."""

    _fields_ = [
        ("struct_size", c_uint32),
        ("kernel", c_int32),
        ("head_dim", c_int32),
        ("key_split", c_int32),
        ("key_chunks", c_int32),
        ("bias_mode", c_int32),
        ("mask_variant", c_int32),
        ("keys_per_step", c_int32),
        ("workgroups", c_int64),
        ("workspace_bytes", c_int64),
        ("name", c_char_p),
        ("tail_kernel", c_int32),
        ("tail_key_split", c_int32),
        ("tail_workgroups", c_int64),
        ("order_n", c_int32),  # revision 2: the host sequence schedule of a scheduled flash call
        ("sequence_order", ctypes.c_uint8 * 256),
        ("tail_folded", c_int32),  # revision 3: the units past the first round run inside it
    ]

    def __init__(self):
        super().__init__()
        self.struct_size = ctypes.sizeof(AttnPlan)

    def variant(self) -> tuple:
        """(kernel, head_dim, key_split, bias_mode, mask_variant): the compiled variant."""
        return (self.kernel, self.head_dim, self.key_split, self.bias_mode, self.mask_variant)


class LinearArgs(ctypes.Structure):
    """Mirror of sa_linear_args (include/supra_linear.h); alpha defaults to 1."""

    _fields_ = [
        ("struct_size", c_uint32),
        ("M", c_int32),
        ("N", c_int32),
        ("K", c_int32),
        ("x", c_void_p),
        ("x_off", c_int64),
        ("ldx", c_int64),
        ("w", c_void_p),
        ("ldw", c_int64),
        ("bias", c_void_p),
        ("alpha", c_float),
        ("act", c_int32),
        ("epilogue", c_int32),
        ("gate", c_void_p),
        ("gate_off", c_int64),
        ("y", c_void_p),
        ("y_off", c_int64),
        ("ldy", c_int64),
    ]

    def __init__(self, **kw):
        super().__init__()
        self.struct_size = ctypes.sizeof(LinearArgs)
        self.alpha = 1.0
        for name, val in kw.items():
            setattr(self, name, val)


class VaeAttnArgs(ctypes.Structure):
    """Mirror of sa_vae_attn_args (include/supra_vae.h); groups default 32, eps 1e-6."""

    _fields_ = [
        ("struct_size", c_uint32),
        ("HW", c_int32),
        ("C", c_int32),
        ("groups", c_int32),
        ("eps", c_float),
        ("x", c_void_p),
        ("gamma", c_void_p),
        ("beta", c_void_p),
        ("wqkv", c_void_p),
        ("bqkv", c_void_p),
        ("wo", c_void_p),
        ("bo", c_void_p),
        ("out", c_void_p),
        ("workspace", c_void_p),
        ("workspace_bytes", c_int64),
    ]

    def __init__(self, **kw):
        super().__init__()
        self.struct_size = ctypes.sizeof(VaeAttnArgs)
        self.groups = 32
        self.eps = 1e-6
        for name, val in kw.items():
            setattr(self, name, val)


class StTensor(ctypes.Structure):
    """sa_st_tensor: one safetensors header entry."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("dtype", c_int32),
        ("elem_bytes", c_int32),
        ("ndim", c_int32),
        ("shape", c_int64 * SA_ST_MAX_DIMS),
        ("numel", c_int64),
        ("begin", c_int64),
        ("end", c_int64),
        ("dtype_name", ctypes.c_char * 16),
    ]

    def __init__(self):
        super().__init__()
        self.struct_size = ctypes.sizeof(StTensor)


_LIB = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once (raises if it has not been built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `python supra2-img-web_amd/build.py`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(rc: int) -> None:
    if rc != SA_OK:
        msg = load().sa_last_error()
        raise SaError(rc, msg.decode() if msg else "")


def attention(args: AttnArgs, stream: int | None = None) -> None:
    check(load().sa_attention_f32(ctypes.byref(args), stream))


def kernel_name(args: AttnArgs) -> str:
    lib = load()
    name = lib.sa_attention_kernel_name(ctypes.byref(args))
    if name is None:
        raise SaError(-1, lib.sa_last_error().decode())
    return name.decode()


def plan(args: AttnArgs) -> AttnPlan:
    """The kernel variant, grid and workspace sa_attention_f32 would use for `args` (host only)."""
    out = AttnPlan()
    check(load().sa_attention_plan(ctypes.byref(args), ctypes.byref(out)))
    return out


def variants() -> list[AttnPlan]:
    """Every compiled kernel variant (sa_attention_variant)."""
    lib = load()
    res = []
    for i in range(lib.sa_attention_variant_count()):
        v = AttnPlan()
        check(lib.sa_attention_variant(i, ctypes.byref(v)))
        res.append(v)
    return res


def linear(args: LinearArgs, stream: int | None = None) -> None:
    check(load().sa_linear_f32(ctypes.byref(args), stream))


def linear_kernel_name(args: LinearArgs) -> str:
    lib = load()
    name = lib.sa_linear_kernel_name(ctypes.byref(args))
    if name is None:
        raise SaError(-1, lib.sa_last_error().decode())
    return name.decode()


def vae_attention(args: VaeAttnArgs, stream: int | None = None) -> None:
    check(load().sa_vae_attention_f32(ctypes.byref(args), stream))


def vae_workspace_bytes(args: VaeAttnArgs) -> int:
    lib = load()
    n = lib.sa_vae_attention_workspace_bytes(ctypes.byref(args))
    if n < 0:
        raise SaError(int(n), lib.sa_last_error().decode())
    return int(n)


def workspace_bytes(args: AttnArgs) -> int:
    """Device scratch bytes sa_attention_f32 needs for `args` (0 for most calls)."""
    lib = load()
    n = lib.sa_attention_workspace_bytes(ctypes.byref(args))
    if n < 0:
        raise SaError(int(n), lib.sa_last_error().decode())
    return int(n)


def bucket_lut(Lq: int, Lk: int, num_buckets: int = 32, max_distance: int = 128, bidirectional: bool = True):
    import numpy as np

    out = np.zeros(Lq + Lk - 1, dtype=np.int32)
    check(load().sa_t5_bucket_lut(Lq, Lk, num_buckets, max_distance, int(bidirectional),
                                  out.ctypes.data_as(POINTER(c_int32))))
    return out


def device_count() -> int:
    n = c_int32(0)
    rc = load().sa_device_count(ctypes.byref(n))
    return n.value if rc == SA_OK else 0
