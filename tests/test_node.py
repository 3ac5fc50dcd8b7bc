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
    res = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "shim_cpu.js"), str(f)],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all 11 checks passed" in res.stdout
