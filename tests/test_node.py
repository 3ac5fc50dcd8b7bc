"""The Node.js binding (N-API addon + JS shim): CPU checks here, GPU parity in test_node_gpu.py."""

from __future__ import annotations

import json
import os
import shutil
import subprocess

import pytest

from oracle import t5_bucket as tb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
ADDON = os.path.join(ROOT, "supra2-img-web_amd", "lib", "supra_attn.node")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def test_shim_and_addon_on_cpu(tmp_path):
    assert os.path.exists(ADDON), "build the addon first (python supra2-img-web_amd/build.py)"
    exp = {
        "Lq": 40, "Lk": 70, "lut": tb.bucket_lut(40, 70).tolist(),
        "singles": [[r, tb.relative_bucket(r)] for r in (-200, -91, -90, -20, -1, 0, 1, 15, 16, 64, 127, 500)],
    }
    f = tmp_path / "buckets.json"
    f.write_text(json.dumps(exp))
    st = _weights_fixture(tmp_path)
    res = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "shim_cpu.js"), str(f), str(st)],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all 17 checks passed" in res.stdout


def _weights_fixture(tmp_path):
    """A safetensors file written by the `safetensors` library and its header as the oracle parses it."""
    import numpy as np
    from safetensors.numpy import save_file

    from oracle import weights as ow

    rng = np.random.default_rng(2)
    path = tmp_path / "w.safetensors"
    save_file({"blocks.0.mlp.0.weight": rng.standard_normal((8, 4)).astype(np.float32),
               "blocks.0.mlp.0.bias": rng.standard_normal(8).astype(np.float16),
               "u16": np.arange(3, dtype=np.uint16), "ids": np.arange(5, dtype=np.int64)},
              str(path), metadata={"format": "pt", "dim": "576"})
    header, meta, _ = ow.parse(path.read_bytes())
    out = tmp_path / "weights.json"
    out.write_text(json.dumps({"file": str(path), "header": header, "metadata": meta}))
    return out
