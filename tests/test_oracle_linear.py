"""Pins of the linear-layer oracle (oracle/linear.py) against what the mathematics fixes, so that a
dropped term, a wrong sign or a transposed operand fails here rather than in a GPU comparison:

- the activations against library routines (normal CDF, logistic function, torch's tanh GELU in
  float64) and the identity f(x) - f(-x) = x that all three satisfy (odd part x/2);
- the product, bias, alpha and the three epilogues on small integer matrices whose results are
  worked out by hand (exact in float32);
- the strided addressing (x_off, ldx, ldw, y_off, ldy): embedding the operands in larger buffers
  gives the compact result and leaves every other output element untouched;
- the float32 PyTorch formulation against the float64 one on DiT-shaped random inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
from scipy import special, stats

from oracle import linear as ol


@pytest.mark.parametrize("act", [ol.ACT_GELU, ol.ACT_GELU_TANH, ol.ACT_SILU])
def test_activation_odd_part_is_half_identity(act):
    x = np.linspace(-9, 9, 181)
    f = ol.act_fp64(x, act)
    np.testing.assert_allclose(f - ol.act_fp64(-x, act), x, rtol=0, atol=1e-12)
    assert ol.act_fp64(np.array([0.0]), act)[0] == 0.0


def test_activations_against_library_routines():
    import torch

    x = np.linspace(-7, 7, 141)
    np.testing.assert_allclose(ol.act_fp64(x, ol.ACT_GELU), x * stats.norm.cdf(x), rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(ol.act_fp64(x, ol.ACT_SILU), x * special.expit(x), rtol=1e-13, atol=1e-15)
    t = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    np.testing.assert_allclose(ol.act_fp64(x, ol.ACT_GELU_TANH), t, rtol=1e-13, atol=1e-15)
    # the tanh form stays within 1e-3 of the exact GELU (a wrong constant would not)
    assert np.max(np.abs(ol.act_fp64(x, ol.ACT_GELU_TANH) - ol.act_fp64(x, ol.ACT_GELU))) < 1e-3


X2 = np.array([[1, 2, 0, -1], [3, 4, 1, 0]], dtype=np.float32)          # [M=2, K=4]
W3 = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [1, 1, 2, 1]], dtype=np.float32)  # [N=3, K=4]
XW = np.array([[1, 2, 2], [3, 4, 9]], dtype=np.float32)                  # X W^T by hand


@pytest.mark.parametrize("fn", [ol.linear_fp64, ol.linear_torch_fp32])
def test_integer_product_bias_alpha_and_epilogues(fn):
    y0 = np.array([[10, 20, 30], [40, 50, 60]], dtype=np.float32)
    bias = np.array([1, -1, 0.5], dtype=np.float32)
    gate = np.array([7, 7, 2, 3, -1], dtype=np.float32)  # used from gate_off = 2: [2, 3, -1]
    kw = dict(M=2, N=3, K=4)
    np.testing.assert_array_equal(fn(X2, W3, y0, **kw), XW)
    np.testing.assert_array_equal(fn(X2, W3, y0, bias=bias, **kw), XW + bias)
    np.testing.assert_array_equal(fn(X2, W3, y0, bias=bias, alpha=2.0, **kw), 2 * XW + bias)
    np.testing.assert_array_equal(fn(X2, W3, y0, bias=bias, epi=ol.EPI_RESID, **kw), y0 + XW + bias)
    got = fn(X2, W3, y0, bias=bias, gate=gate, gate_off=2, epi=ol.EPI_RESID_GATE, **kw)
    np.testing.assert_array_equal(got, y0 + np.array([2, 3, -1], dtype=np.float32) * (XW + bias))
    # activation applied after the bias, before the gate
    r = fn(X2, W3, y0, bias=bias, act=ol.ACT_SILU, gate=gate, gate_off=2, epi=ol.EPI_RESID_GATE, **kw)
    want = y0 + np.array([2, 3, -1]) * ((XW + bias) * special.expit(XW + bias))
    np.testing.assert_allclose(r, want, rtol=1e-6)


@pytest.mark.parametrize("fn", [ol.linear_fp64, ol.linear_torch_fp32])
def test_strided_addressing_matches_compact(fn):
    rng = np.random.default_rng(3)
    M, N, K = 5, 7, 6
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = rng.standard_normal((N, K)).astype(np.float32)
    compact = fn(X, W, np.zeros((M, N), np.float32), M=M, N=N, K=K)
    x_off, ldx, ldw, y_off, ldy = 3, 9, 8, 5, 11
    xb = np.full(x_off + (M - 1) * ldx + K + 4, 1e30, np.float32)
    for m in range(M):
        xb[x_off + m * ldx: x_off + m * ldx + K] = X[m]
    wb = np.full((N, ldw), 1e30, np.float32)
    wb[:, :K] = W
    yb = rng.standard_normal(y_off + (M - 1) * ldy + N + 3).astype(np.float32)
    got = fn(xb, wb, yb, M=M, N=N, K=K, x_off=x_off, ldx=ldx, ldw=ldw, y_off=y_off, ldy=ldy)
    idx = y_off + np.arange(M)[:, None] * ldy + np.arange(N)[None, :]
    np.testing.assert_allclose(got[idx], compact, rtol=1e-6, atol=1e-6)
    untouched = np.ones(yb.size, bool)
    untouched[idx.reshape(-1)] = False
    np.testing.assert_array_equal(got[untouched], yb[untouched])


@pytest.mark.parametrize("act", [ol.ACT_NONE, ol.ACT_GELU, ol.ACT_GELU_TANH, ol.ACT_SILU])
def test_torch_fp32_agrees_with_fp64(act):
    rng = np.random.default_rng(act)
    M, N, K = 64, 96, 576
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    b = (0.1 * rng.standard_normal(N)).astype(np.float32)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    g = rng.standard_normal(N).astype(np.float32)
    kw = dict(M=M, N=N, K=K, bias=b, act=act, gate=g, epi=ol.EPI_RESID_GATE)
    e = ol.errors(ol.linear_torch_fp32(X, W, y0, **kw), ol.linear_fp64(X, W, y0, **kw))
    assert e["rel_l2"] < 1e-6 and e["max_rel"] < 1e-6, e
