"""The operator and the linear layer under HIP graph capture (GPU).

One DiT block's attention half at batch 2 - q|k|v projection (app/models/dit.js:167), batched
self-attention (dit.js:169-173) and the gated output projection (dit.js:175) - is recorded into a
HIP graph by stream capture through the C ABI, then replayed several times with eager work (copies,
fills, synchronisations) between the replays; every replay must reproduce the eager result bit for
bit. Nothing in these calls allocates, synchronises or records a memset, so they capture as they are.
The graph API is the HIP runtime's own (the library links the same runtime).
"""

from __future__ import annotations

import ctypes
from ctypes import byref, c_int, c_void_p

import numpy as np
import pytest

from supra_attn import _lib
from supra_attn.linear_workloads import DIT_DIM, DIT_TOKENS

pytestmark = pytest.mark.gpu

HIP_STREAM_CAPTURE_MODE_GLOBAL = 0


def _hip():
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime libsupra_attn.so links
    for name, args in (("hipStreamBeginCapture", [c_void_p, c_int]), ("hipStreamEndCapture", [c_void_p, c_void_p]),
                       ("hipGraphInstantiate", [c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_size_t]),
                       ("hipGraphLaunch", [c_void_p, c_void_p]), ("hipGraphExecDestroy", [c_void_p]),
                       ("hipGraphDestroy", [c_void_p])):
        fn = getattr(hip, name)
        fn.restype = c_int
        fn.argtypes = args
    return hip


def test_dit_block_attention_half_in_a_graph(dev):
    B, D, H, HD = 2, DIT_DIM, 9, 64
    R = B * DIT_TOKENS
    rng = np.random.default_rng(5)
    f = lambda *shape, s=1.0: (rng.standard_normal(shape, dtype=np.float32) * np.float32(s)).astype(np.float32)
    h = dev.from_array(f(R, D))
    w_qkv, b_qkv = dev.from_array(f(3 * D, D, s=D ** -0.5)), dev.from_array(f(3 * D, s=0.1))
    w_o, b_o = dev.from_array(f(D, D, s=D ** -0.5)), dev.from_array(f(D, s=0.1))
    mod = dev.from_array(f(6 * D))
    x0 = dev.from_array(f(R, D))
    qkv, a, x = dev.empty((R, 3 * D)), dev.empty((R, D)), dev.empty((R, D))

    lin_qkv = _lib.LinearArgs(M=R, N=3 * D, K=D, x=h.ptr, w=w_qkv.ptr, bias=b_qkv.ptr, y=qkv.ptr)
    attn = _lib.AttnArgs(B=B, H=H, D=HD, Lq=DIT_TOKENS, Lk=DIT_TOKENS, q=qkv.ptr, k=qkv.ptr, v=qkv.ptr, o=a.ptr,
                         k_off=D, v_off=2 * D, ldq=3 * D, ldk=3 * D, ldv=3 * D, ldo=D, sq=DIT_TOKENS * 3 * D,
                         sk=DIT_TOKENS * 3 * D, sv=DIT_TOKENS * 3 * D, so=DIT_TOKENS * D, scale=HD ** -0.5)
    assert _lib.workspace_bytes(attn) == 0  # no workspace: nothing to allocate around the capture
    lin_o = _lib.LinearArgs(M=R, N=D, K=D, x=a.ptr, w=w_o.ptr, bias=b_o.ptr, epilogue=_lib.SA_EPI_RESID_GATE,
                            gate=mod.ptr, gate_off=2 * D, y=x.ptr)
    lib = _lib.load()
    s = c_void_p(dev.stream)

    def reset():
        _lib.check(lib.sa_memcpy_d2d(x.ptr, x0.ptr, x.nbytes, s))

    def block():
        _lib.check(lib.sa_linear_f32(byref(lin_qkv), s))
        _lib.check(lib.sa_attention_f32(byref(attn), s))
        _lib.check(lib.sa_linear_f32(byref(lin_o), s))

    reset()
    block()
    eager = x.read()
    assert np.isfinite(eager).all() and not np.array_equal(eager, x0.read())

    hip = _hip()
    graph, exe = c_void_p(), c_void_p()
    dev.sync()
    assert hip.hipStreamBeginCapture(s, HIP_STREAM_CAPTURE_MODE_GLOBAL) == 0
    try:
        block()
    finally:
        rc_end = hip.hipStreamEndCapture(s, byref(graph))
    assert rc_end == 0 and graph.value
    assert hip.hipGraphInstantiate(byref(exe), graph, None, None, 0) == 0
    try:
        for rep in range(5):
            # eager work between replays: reset the residual stream, scribble over the intermediates
            reset()
            qkv.fill_bytes(0xFF)  # NaN patterns
            a.fill_bytes(0xFF)
            dev.sync()
            assert hip.hipGraphLaunch(exe, s) == 0
            got = x.read()  # synchronises the stream
            np.testing.assert_array_equal(got.view(np.uint32), eager.view(np.uint32), err_msg=f"replay {rep}")
    finally:
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
    for buf in (h, w_qkv, b_qkv, w_o, b_o, mod, x0, qkv, a, x):
        buf.release()
