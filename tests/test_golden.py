"""Committed golden vectors (tests/golden/attention_cases.npz): the oracle must keep reproducing
them on the CPU, and the HIP operator must match them on the GPU (rel-L2 and normwise max relative
error <= 1e-5 against the PyTorch fp32 outputs)."""

from __future__ import annotations

import numpy as np
import pytest

from golden.fixtures import load_cases
from oracle import attention as orc

CASES = load_cases()
IDS = [c[0] for c in CASES]


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_oracle_reproduces_fixtures(case):
    name, call, exp32, exp64 = case
    np.testing.assert_allclose(orc.reference_fp64(call), exp64, rtol=2e-7, atol=1e-30)
    e = orc.errors(orc.reference_torch(call), exp32)
    assert e["max_rel"] <= 1e-6, f"{name}: {e}"
    e = orc.errors(exp32, exp64)
    assert e["rel_l2"] <= 1e-5 and e["max_rel"] <= 1e-5, f"{name}: torch vs fp64 {e}"


def test_fixture_coverage():
    kinds = {(c.bias_mode, c.mask_mode, c.D) for _, c, _, _ in CASES}
    assert {b for b, _, _ in kinds} == {0, 1, 2}
    assert {m for _, m, _ in kinds} == {0, 1, 2}
    assert {d for _, _, d in kinds} >= {64, 128, 512}


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_operator_matches_fixtures(dev, case):
    from supra_attn.runner import Staged

    name, call, exp32, exp64 = case
    print(f"[golden] {name}", flush=True)
    st = Staged(dev, call)
    out = st.run()
    st.release()
    got = orc.output_view(out, call)
    e = orc.errors(got, exp32)
    assert e["finite"] and e["rel_l2"] <= 1e-5 and e["max_rel"] <= 1e-5, f"{name}: {e}"
    e = orc.errors(got, exp64)
    assert e["rel_l2"] <= 1e-5 and e["max_rel"] <= 1e-5, f"{name} vs fp64: {e}"
