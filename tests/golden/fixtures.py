"""Loader of tests/golden/attention_cases.npz into workload calls (numpy only, no pickles)."""

from __future__ import annotations

import json
import os

import numpy as np

from supra_attn.workloads import Call

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attention_cases.npz")


def load_cases():
    """[(name, call, expected_torch_fp32, expected_fp64)]"""
    z = np.load(PATH, allow_pickle=False)
    out = []
    for name in json.loads(str(z["index"])):
        meta = json.loads(str(z[f"{name}.meta"]))
        q = z[f"{name}.q"]
        same = meta["same_qkv"]
        call = Call(name=name, B=meta["B"], H=meta["H"], D=meta["D"], Lq=meta["Lq"], Lk=meta["Lk"], q=q,
                    k=q if same else z[f"{name}.k"], v=q if same else z[f"{name}.v"],
                    out_shape=tuple(meta["out_shape"]), args=meta["args"], scale=meta["scale"],
                    bias_mode=meta["bias_mode"], mask_mode=meta["mask_mode"], same_qkv=same)
        for field in ("bias", "lut", "key_len", "key_mask"):
            key = f"{name}.{field}"
            if key in z.files:
                setattr(call, field, z[key])
        out.append((name, call, z[f"{name}.out_torch"], z[f"{name}.out_fp64"]))
    return out
