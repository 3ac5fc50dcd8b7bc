"""GPU parity of the Node.js binding: the JS shim runs the reference call forms on the device
(tests/node/ops_gpu.js) and its outputs are checked against the CPU oracle (rel-L2 and normwise max
relative error <= 1e-5)."""

from __future__ import annotations

import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import attention as orc
from supra_attn import workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(NODE is None, reason="node is not installed")]


def _save(d, name, arr):
    np.ascontiguousarray(arr).tofile(os.path.join(d, name))
    return name


def test_reference_call_forms_through_node(tmp_path):
    d = str(tmp_path)
    cases, refs = [], {}

    s = workloads.dit_self(B=2, seed=10)
    ref_s = orc.reference_torch(s).reshape(2 * 256, 576)
    for form in ("dit_self_loop", "dit_self_batched"):
        cases.append({"name": form, "form": form, "B": 2, "qkv": _save(d, "qkv.bin", s.q)})
        refs[form] = ref_s

    c = workloads.dit_cross(B=2, key_len=(77, 1), seed=11)
    kv = c.k.reshape(2, 128, 1152)
    cases.append({"name": "dit_cross_loop", "form": "dit_cross_loop", "B": 2, "L": [77, 1],
                  "q": _save(d, "cq.bin", c.q),
                  "kv": [_save(d, "kv0.bin", kv[0, :77]), _save(d, "kv1.bin", kv[1, :1])]})
    refs["dit_cross_loop"] = orc.reference_torch(c).reshape(2 * 256, 576)
    # the guided batch of two through the batched call site: its one-key sequence is packed into fewer
    # workgroups of the 16-query small-launch kernel (the host lengths travel with the call)
    cases.append({"name": "dit_cross_callsite_b2", "form": "dit_cross_callsite", "B": 2, "L": [77, 1],
                  "q": cases[-1]["q"], "kv": cases[-1]["kv"]})
    refs["dit_cross_callsite_b2"] = refs["dit_cross_loop"]

    s4 = workloads.dit_self(B=4, seed=14)
    cases.append({"name": "dit_self_callsite", "form": "dit_self_callsite", "B": 4, "qkv": _save(d, "qkv4.bin", s4.q)})
    refs["dit_self_callsite"] = orc.reference_torch(s4).reshape(4 * 256, 576)

    lens = [77, 1, 50, 3]
    c4 = workloads.dit_cross(B=4, key_len=lens, seed=15)
    kv4 = c4.k.reshape(4, 128, 1152)
    cases.append({"name": "dit_cross_callsite", "form": "dit_cross_callsite", "B": 4, "L": lens,
                  "q": _save(d, "cq4.bin", c4.q),
                  "kv": [_save(d, f"kv4_{b}.bin", kv4[b, :lens[b]]) for b in range(4)]})
    refs["dit_cross_callsite"] = orc.reference_torch(c4).reshape(4 * 256, 576)

    t5 = workloads.t5_self(seed=12, masked_tail=0)
    t5_files = {"q": _save(d, "t5q.bin", t5.q), "k": _save(d, "t5k.bin", t5.k), "v": _save(d, "t5v.bin", t5.v),
                "table": _save(d, "t5t.bin", t5.bias)}
    cases.append(dict(name="t5_dense", form="t5_dense", L=128, **t5_files))
    refs["t5_dense"] = orc.reference_torch(t5).reshape(128, 768)

    t5m = workloads.t5_self(seed=12, masked_tail=40)
    cases.append(dict(name="t5_relpos_mask", form="t5_relpos_mask", L=128, mask=_save(d, "t5m.bin", t5m.key_mask),
                      **t5_files))
    refs["t5_relpos_mask"] = orc.reference_torch(t5m).reshape(128, 768)

    vae = workloads.vae_mid(seed=13)
    cases.append({"name": "vae", "form": "vae", "L": 1024, "q": _save(d, "vq.bin", vae.q),
                  "k": _save(d, "vk.bin", vae.k), "v": _save(d, "vv.bin", vae.v)})
    refs["vae"] = orc.reference_torch(vae).reshape(1024, 512)

    from oracle import linear as ol
    from supra_attn.linear_workloads import dit_block_linears

    lin_refs = {}
    acts = {0: "none", 1: "gelu", 2: "gelu_tanh", 3: "silu"}
    for call in [c for c in dit_block_linears(B=1) if c.name in ("qkv", "proj", "fc1", "cproj")]:
        name = "linear_" + call.name
        case = {"name": name, "form": "linear", "M": call.M, "N": call.N, "K": call.K, "act": acts[call.act],
                "x": _save(d, name + "_x.bin", call.x), "w": _save(d, name + "_w.bin", call.w),
                "bias": _save(d, name + "_b.bin", call.bias), "resid": call.epi != 0}
        if call.epi != 0:
            case["y0"] = _save(d, name + "_y0.bin", call.y0)
        if call.gate is not None:
            case.update(gate=_save(d, name + "_g.bin", call.gate), gateLen=int(call.gate.size), gOff=call.gate_off)
        cases.append(case)
        lin_refs[name] = ol.linear_torch_fp32(call.x, call.w, call.y0, **call.oracle_kwargs()).reshape(call.M, call.N)
    refs.update(lin_refs)

    from oracle import vae_block as ov
    from supra_attn.linear_workloads import vae_block

    vb = vae_block(seed=31)
    C = vb.C
    vcase = {"name": "vae_block", "form": "vae_block", "HW": vb.HW, "C": C, "x": _save(d, "vbx.bin", vb.x),
             "gamma": _save(d, "vbg.bin", vb.gamma), "beta": _save(d, "vbb.bin", vb.beta),
             "wo": _save(d, "vbwo.bin", vb.wo), "bo": _save(d, "vbbo.bin", vb.bo)}
    for i, nm in enumerate("qkv"):
        vcase["w" + nm] = _save(d, f"vbw{nm}.bin", vb.wqkv[i * C:(i + 1) * C])
        vcase["b" + nm] = _save(d, f"vbb{nm}.bin", vb.bqkv[i * C:(i + 1) * C])
    cases.append(vcase)
    refs["vae_block"] = ov.block_torch_fp32(*vb.oracle_args())

    # the safetensors loader (app/weights.js) as the model loaders call it
    from oracle import weights as ow
    from safetensors.numpy import save_file

    rng = np.random.default_rng(40)
    st_path = os.path.join(d, "model.safetensors")
    save_file({"blocks.0.self_attn.qkv.weight": (rng.standard_normal((1728, 576)) / 24).astype(np.float32),
               "blocks.0.self_attn.qkv.bias": (rng.standard_normal(1728) * 0.1).astype(np.float32),
               "blocks.0.mlp.0.weight": (rng.standard_normal((2304, 576)) / 24).astype(np.float16),
               "shared.weight": rng.standard_normal((3000, 768)).astype(np.float32),
               "decoder.conv_in.weight": rng.standard_normal((512, 4, 3, 3)).astype(np.float32),
               "decoder.conv_in.bias": rng.standard_normal(512).astype(np.float32)}, st_path)
    st_buf = open(st_path, "rb").read()
    hdr, _, start = ow.parse(st_buf)
    raw = lambda n: ow.to_f32(ow.tensor_bytes(st_buf, hdr, start, n), hdr[n]["dtype"])
    x = rng.standard_normal((256, 576)).astype(np.float32)
    cases.append({"name": "st_linear", "form": "st_linear", "file": st_path, "base": "blocks.0.self_attn.qkv.",
                  "M": 256, "x": _save(d, "stx.bin", x)})
    refs["st_linear"] = ol.linear_torch_fp32(x, raw("blocks.0.self_attn.qkv.weight").reshape(1728, 576),
                                             np.zeros(256 * 1728, np.float32), M=256, N=1728, K=576,
                                             bias=raw("blocks.0.self_attn.qkv.bias")).reshape(256, 1728)
    ids = [0, 2999, 17, 17, 1234]
    cases.append({"name": "st_rows", "form": "st_rows", "file": st_path, "table": "shared.weight", "ids": ids,
                  "exact": True})
    refs["st_rows"] = ow.rows(ow.tensor_bytes(st_buf, hdr, start, "shared.weight"), "F32", 3000, 768, ids)
    cases.append({"name": "st_conv3", "form": "st_conv3", "file": st_path, "base": "decoder.conv_in.", "cinPad": 8,
                  "exact": True})
    refs["st_conv3"] = ow.conv3_pack(raw("decoder.conv_in.weight"), 512, 4, 8)
    cases.append({"name": "st_f32", "form": "st_f32", "file": st_path, "tensor": "blocks.0.mlp.0.weight",
                  "exact": True})
    refs["st_f32"] = raw("blocks.0.mlp.0.weight")
    bf = np.arange(65536, dtype="<u2").tobytes()
    cases.append({"name": "st_to_f32", "form": "st_to_f32", "raw": _save(d, "bf16.bin", np.frombuffer(bf, np.uint8)),
                  "dtype": "BF16", "exact": True})
    refs["st_to_f32"] = ow.to_f32(bf, "BF16")

    with open(os.path.join(d, "manifest.json"), "w") as f:
        json.dump({"cases": cases}, f)
    print("[node gpu] running", [c["name"] for c in cases], flush=True)
    res = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "ops_gpu.js"), d], capture_output=True,
                         text=True, timeout=300)
    print(res.stdout, res.stderr, flush=True)
    assert res.returncode == 0, res.stderr
    assert "node: boundary checks passed" in res.stdout
    for case in cases:
        got = np.fromfile(os.path.join(d, case["name"] + ".out.bin"), dtype=np.float32)
        ref = refs[case["name"]]
        if case.get("exact"):  # decoded weights: bit for bit
            np.testing.assert_array_equal(got.view(np.uint32), np.ascontiguousarray(ref, np.float32).reshape(-1).view(np.uint32),
                                          err_msg=case["name"])
            continue
        e = orc.errors(got.reshape(ref.shape), ref)
        assert e["finite"] and e["rel_l2"] <= 1e-5 and e["max_rel"] <= 1e-5, f"{case['name']}: {e}"
