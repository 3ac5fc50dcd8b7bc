"""Pins of the VAE mid-block oracle (oracle/vae_block.py): GroupNorm against the library routine
and its defining moments, the residual path, and a closed form of the attention part, so that the
block restatement is checked piece by piece rather than against itself."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import vae_block as ov
from supra_attn.linear_workloads import vae_block


def test_groupnorm_moments_and_library():
    import torch

    rng = np.random.default_rng(0)
    HW, C, G = 64, 32, 8
    x = (3 + 2 * rng.standard_normal((HW, C))).astype(np.float32)
    n = ov.groupnorm_fp64(x, np.ones(C), np.zeros(C), G, 1e-6).reshape(HW, G, C // G)
    np.testing.assert_allclose(n.mean(axis=(0, 2)), 0, atol=1e-12)
    np.testing.assert_allclose((n ** 2).mean(axis=(0, 2)), 1, atol=1e-6)  # var / (var + eps)
    gamma, beta = rng.standard_normal(C), rng.standard_normal(C)
    t = torch.nn.functional.group_norm(torch.from_numpy(x.astype(np.float64)).t().reshape(1, C, HW), G,
                                       torch.from_numpy(gamma), torch.from_numpy(beta), 1e-6).reshape(C, HW).t()
    np.testing.assert_allclose(ov.groupnorm_fp64(x, gamma, beta, G, 1e-6), t.numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("fn", [ov.block_fp64, ov.block_torch_fp32])
def test_zero_output_projection_leaves_the_residual(fn):
    c = vae_block(HW=64, C=64, groups=8, seed=1)
    out = fn(c.x, c.gamma, c.beta, c.wqkv, c.bqkv, np.zeros_like(c.wo), c.bo, groups=8)
    np.testing.assert_allclose(out, c.x + c.bo[None, :], rtol=0, atol=1e-6)


@pytest.mark.parametrize("fn", [ov.block_fp64, ov.block_torch_fp32])
def test_zero_queries_average_the_values(fn):
    """q = 0 makes every softmax row uniform: out = x + mean_p(v) Wo^T + bo for every pixel."""
    c = vae_block(HW=48, C=32, groups=4, seed=2)
    C = c.C
    wqkv = c.wqkv.copy()
    wqkv[:C] = 0
    bqkv = c.bqkv.copy()
    bqkv[:C] = 0
    n = ov.groupnorm_fp64(c.x, c.gamma, c.beta, 4, 1e-6)
    v = n @ wqkv[2 * C:].astype(np.float64).T + bqkv[2 * C:]
    want = c.x + (v.mean(axis=0) @ c.wo.astype(np.float64).T + c.bo)[None, :]
    np.testing.assert_allclose(fn(c.x, c.gamma, c.beta, wqkv, bqkv, c.wo, c.bo, groups=4), want, rtol=1e-5, atol=1e-5)


def test_torch_fp32_agrees_with_fp64():
    c = vae_block(HW=256, C=128, groups=32, seed=3)
    a = ov.block_torch_fp32(*c.oracle_args(), groups=32)
    b = ov.block_fp64(*c.oracle_args(), groups=32)
    d = np.abs(a.astype(np.float64) - b)
    assert np.linalg.norm(d) / np.linalg.norm(b) < 1e-6 and d.max() / np.abs(b).max() < 1e-6
