"""sa_attention_f32_noalloc, the allocation-free entry point, against sa_attention_f32 with a
caller workspace: the same kernels, so bit for bit the same outputs, and both within the parity bar
of the PyTorch fp32 CPU path. Two calls in a row on the library's per-GPU scratch, the second one
smaller, then a flash call (no scratch), the two calls whose merge records come closest to filling
the scratch, and a captured call in a fresh process."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import attention as orc
from supra_attn import _lib, workloads
from supra_attn.runner import Staged
from cases import make_call

pytestmark = pytest.mark.gpu

TOL = 1e-5


def run_both(dev, call):
    """Outputs of sa_attention_f32 (workspace from the caller) and sa_attention_f32_noalloc (no
    workspace fields set) on the same device-resident inputs."""
    print(f"[case] noalloc {call.name} B={call.B} H={call.H} D={call.D} Lq={call.Lq} Lk={call.Lk}", flush=True)
    lib = _lib.load()
    st = Staged(dev, call, out_fill=np.float32(-7.0))
    try:
        need = _lib.workspace_bytes(st.args)
        st.launch()
        dev.sync()
        ref = st.out.read()
        st.out.upload(np.full(call.out_shape, np.float32(-7.0), dtype=np.float32))
        args = _lib.AttnArgs()
        ctypes.memmove(ctypes.byref(args), ctypes.byref(st.args), ctypes.sizeof(args))
        args.workspace = None
        args.workspace_bytes = 0
        _lib.check(lib.sa_attention_f32_noalloc(ctypes.byref(args), ctypes.c_void_p(dev.stream)))
        dev.sync()
        got = st.out.read()
    finally:
        st.release()
    return ref, got, need


def check_case(dev, call):
    ref, got, need = run_both(dev, call)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), f"{call.name}: noalloc differs from the workspace call"
    e = orc.errors(orc.output_view(got, call), orc.reference_torch(call))
    assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, f"{call.name}: {e}"
    return need


def test_noalloc_matches_the_workspace_call_twice_then_smaller(dev):
    # the VAE mid-block shape: the wide-head kernel merges 8 key chunks through the scratch
    need1 = check_case(dev, workloads.vae_mid(seed=3))
    assert 0 < need1 <= _lib.SA_NOALLOC_SCRATCH_BYTES
    # a smaller call right after, on the same scratch (ragged, fewer query groups and key chunks)
    need2 = check_case(dev, make_call(B=1, H=1, D=512, Lq=700, Lk=650, seed=41))
    assert 0 < need2 < need1
    # a head-dim-256 call with key lengths
    check_case(dev, make_call(B=2, H=1, D=256, Lq=300, Lk=520, mask_mode=_lib.SA_MASK_KEY_LEN, key_len=[520, 77],
                              seed=42))


def test_noalloc_whole_rounds_then_split_groups(dev):
    # 9 heads of the VAE size: 256 query groups unsplit, then 32 in 8 key chunks through the scratch
    need = check_case(dev, make_call(B=1, H=9, D=512, Lq=1024, Lk=1024, seed=9))
    assert need == 32 * 8 * (32 * 512 + 64) * 4


def test_noalloc_flash_call_needs_no_scratch(dev):
    need = check_case(dev, workloads.dit_self(B=2, seed=0))
    assert need == 0


@pytest.mark.parametrize("D,L", [(512, 3200), (256, 6400)])
def test_noalloc_calls_whose_records_nearly_fill_the_scratch(dev, D, L):
    """The wide-head plans keep their merge records within the 32 MiB scratch; these two come
    closest (5 key chunks: 32.9 MB at D = 512, 33.0 MB at D = 256, two rounds of workgroups) and
    run bit for bit like the workspace call."""
    need = check_case(dev, make_call(B=1, H=1, D=D, Lq=L, Lk=L, seed=D + L))
    assert 32_000_000 < need <= _lib.SA_NOALLOC_SCRATCH_BYTES


_GRAPH_CHILD = r"""
import ctypes, sys
from ctypes import byref, c_int, c_void_p
import numpy as np
from supra_attn import _lib, workloads
from supra_attn.device import Device
from supra_attn.runner import Staged
from cases import make_call

hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime libsupra_attn.so links
for name, args in (("hipStreamBeginCapture", [c_void_p, c_int]), ("hipStreamEndCapture", [c_void_p, c_void_p]),
                   ("hipGraphInstantiate", [c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_size_t]),
                   ("hipGraphLaunch", [c_void_p, c_void_p]), ("hipGraphExecDestroy", [c_void_p]),
                   ("hipGraphDestroy", [c_void_p])):
    getattr(hip, name).restype = c_int
    getattr(hip, name).argtypes = args
lib = _lib.load()
dev = Device(0)  # sa_set_device, sa_stream_create: the library's first use on the GPU, before any capture
s = c_void_p(dev.stream)

def noalloc_args(st):
    a = _lib.AttnArgs()
    ctypes.memmove(byref(a), byref(st.args), ctypes.sizeof(a))
    a.workspace = None
    a.workspace_bytes = 0
    return a

big = Staged(dev, workloads.vae_mid(seed=3))           # 8 key chunks merged through the scratch
small = Staged(dev, make_call(B=1, H=1, D=512, Lq=700, Lk=650, seed=41))
big.launch(); dev.sync(); ref = big.out.read()         # the workspace call
small.launch(); dev.sync(); ref_small = small.out.read()
a_big, a_small = noalloc_args(big), noalloc_args(small)
print("[graph] capture: the process's first allocation-free call", flush=True)
graph, exe = c_void_p(), c_void_p()
assert hip.hipStreamBeginCapture(s, 0) == 0  # global mode: any allocation or sync inside fails
rc = lib.sa_attention_f32_noalloc(byref(a_big), s)
assert hip.hipStreamEndCapture(s, byref(graph)) == 0 and graph.value
assert rc == _lib.SA_OK, lib.sa_last_error()
assert hip.hipGraphInstantiate(byref(exe), graph, None, None, 0) == 0
for rep in range(3):
    big.out.fill_bytes(0xFF)
    # eager work on the same scratch between replays: a smaller allocation-free call
    small.out.fill_bytes(0xFF)
    _lib.check(lib.sa_attention_f32_noalloc(byref(a_small), s))
    dev.sync()
    assert np.array_equal(small.out.read().view(np.uint32), ref_small.view(np.uint32)), rep
    assert hip.hipGraphLaunch(exe, s) == 0
    dev.sync()
    got = big.out.read()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"replay {rep}"
    print(f"[graph] replay {rep} bit-identical", flush=True)
hip.hipGraphExecDestroy(exe)
hip.hipGraphDestroy(graph)
big.release(); small.release()
print("GRAPH_OK", flush=True)
"""


def test_noalloc_wide_call_in_a_graph_in_a_fresh_process():
    """In a fresh process, whose first allocation-free call is made under stream capture (after
    the library's first use on the GPU, which looks up the scratch): the captured wide-head call
    (VAE shape, 8 key chunks merged through the scratch) replays bit for bit like the workspace
    call, three times, with an eager allocation-free call on the same scratch between replays."""
    import os
    import subprocess
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([root, os.path.join(root, "supra2-img-web_amd"), here,
                                         env.get("PYTHONPATH", "")])
    print("[case] noalloc graph capture in a child process", flush=True)
    res = subprocess.run([sys.executable, "-u", "-c", _GRAPH_CHILD], env=env, capture_output=True, text=True,
                         timeout=110)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "GRAPH_OK" in res.stdout
