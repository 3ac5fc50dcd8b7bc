"""Writes tests/golden/attention_cases.npz: small seeded attention calls covering every layout,
bias and mask mode, with their expected outputs from the CPU oracle (PyTorch fp32 formulation, and the
fp64 brute force rounded once to float32). The reference repository commits no operator-level vectors, so these are the
build's own fixtures; the oracle they come from is pinned in tests/test_oracle.py.

    python tests/golden/gen_fixtures.py
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "supra2-img-web_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

from cases import make_call  # noqa: E402
from oracle import attention as orc  # noqa: E402
from supra_attn import _lib  # noqa: E402

OUT = os.path.join(HERE, "attention_cases.npz")


def cases():
    yield "dit_self_packed", make_call(B=2, H=1, D=64, Lq=40, Lk=40, packed=True, seed=100)
    yield "dit_cross_keylen", make_call(B=2, H=1, D=64, Lq=24, Lk=32, mask_mode=_lib.SA_MASK_KEY_LEN,
                                        key_len=[20, 1], seed=101)
    yield "t5_relpos_keymask", make_call(B=1, H=2, D=64, Lq=24, Lk=24, scale=1.0, bias_mode=_lib.SA_BIAS_RELPOS,
                                         mask_mode=_lib.SA_MASK_KEY_MASK, key_mask_p=0.8, bias_std=2.0, seed=102)
    yield "t5_dense_bias", make_call(B=1, H=2, D=64, Lq=24, Lk=24, scale=1.0, bias_mode=_lib.SA_BIAS_DENSE,
                                     bias_std=2.0, seed=103)
    yield "vae_d512", make_call(B=1, H=1, D=512, Lq=20, Lk=24, seed=104)
    empty = make_call(B=2, H=1, D=64, Lq=33, Lk=45, mask_mode=_lib.SA_MASK_KEY_MASK, seed=105)
    empty.key_mask[1, :] = 0
    yield "odd_keymask_empty_row", empty
    yield "d128_offsets", make_call(B=2, H=1, D=128, Lq=20, Lk=37, q_off=8, o_off=4, ldo_pad=12, pad_cols=4, seed=106)


def meta_of(call):
    return {"B": call.B, "H": call.H, "D": call.D, "Lq": call.Lq, "Lk": call.Lk, "scale": call.scale,
            "args": call.args, "bias_mode": call.bias_mode, "mask_mode": call.mask_mode, "same_qkv": call.same_qkv,
            "out_shape": list(call.out_shape)}


def main():
    arrays = {}
    index = []
    for name, call in cases():
        index.append(name)
        arrays[f"{name}.meta"] = np.array(json.dumps(meta_of(call)))
        arrays[f"{name}.q"] = call.q
        if not call.same_qkv:
            arrays[f"{name}.k"] = call.k
            arrays[f"{name}.v"] = call.v
        for field in ("bias", "lut", "key_len", "key_mask"):
            val = getattr(call, field)
            if val is not None:
                arrays[f"{name}.{field}"] = np.asarray(val)
        arrays[f"{name}.out_torch"] = orc.reference_torch(call).astype(np.float32)
        arrays[f"{name}.out_fp64"] = orc.reference_fp64(call).astype(np.float32)  # exact result, rounded once
    arrays["index"] = np.array(json.dumps(index))
    np.savez_compressed(OUT, **arrays)
    print(OUT, os.path.getsize(OUT), "bytes,", len(index), "cases")


if __name__ == "__main__":
    main()
