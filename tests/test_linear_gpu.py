"""GPU parity of the linear layer (sa_linear_f32) against the CPU oracle: relative L2 and normwise max
relative error <= 1e-5 versus the PyTorch fp32 CPU path (oracle.linear.linear_torch_fp32) and the
float64 restatement, over the whole output buffer (so elements outside the written rows/columns
must keep their previous contents)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import linear as ol
from supra_attn import _lib
from supra_attn.linear_workloads import context_kv, dit_block_linears, make_linear
from supra_attn.runner import StagedLinear

pytestmark = pytest.mark.gpu

TOL = 1e-5


def run_checked(dev, call, expect_kernel=None, check_fp64=True):
    print(f"[linear case] {call.name} M={call.M} N={call.N} K={call.K} act={call.act} epi={call.epi}", flush=True)
    st = StagedLinear(dev, call)
    try:
        if expect_kernel is not None:
            assert st.kernel == expect_kernel
        got = st.run()
    finally:
        st.release()
    kw = call.oracle_kwargs()
    ref = ol.linear_torch_fp32(call.x, call.w, call.y0, **kw)
    e = ol.errors(got, ref)
    assert e["finite"] and e["rel_l2"] <= TOL and e["max_rel"] <= TOL, f"{call.name} vs torch fp32: {e}"
    if check_fp64:
        e64 = ol.errors(got, ol.linear_fp64(call.x, call.w, call.y0, **kw))
        assert e64["rel_l2"] <= TOL and e64["max_rel"] <= TOL, f"{call.name} vs fp64: {e64}"
    return e


@pytest.mark.parametrize("idx", range(6))
def test_dit_block_linears_batch2(dev, idx):
    """qkv, proj (gated residual), q, cproj (residual), fc1 (GELU tanh), fc2 (gated residual)."""
    call = dit_block_linears(B=2)[idx]
    run_checked(dev, call)


def test_context_projection(dev):
    run_checked(dev, context_kv(L=77))


@pytest.mark.parametrize("act", [_lib.SA_ACT_GELU, _lib.SA_ACT_SILU, _lib.SA_ACT_GELU_TANH])
def test_activations(dev, act):
    run_checked(dev, make_linear(f"act{act}", 200, 320, 256, seed=act, act=act))


@pytest.mark.parametrize("M,N,K", [(1, 1, 8), (1, 577, 576), (100, 70, 40), (33, 200, 72), (257, 193, 24),
                                   (129, 65, 8), (300, 1, 1032)])
def test_ragged_shapes_mfma(dev, M, N, K):
    """Tile edges in M and N, k-tiles cut at K % 32 != 0 (K % 8 == 0 keeps the MFMA kernel)."""
    call = make_linear(f"ragged_{M}x{N}x{K}", M, N, K, seed=M + N + K, epi=_lib.SA_EPI_RESID)
    assert StagedLinear(dev, call).kernel.startswith("linear_mfma")
    run_checked(dev, call)


def test_strides_offsets_and_untouched_elements(dev):
    call = make_linear("strided", 150, 90, 64, seed=5, x_off=12, ldx=80, ldw=68, y_off=7, ldy=101,
                       epi=_lib.SA_EPI_RESID_GATE, gate_off=9, alpha=0.5)
    run_checked(dev, call)


@pytest.mark.parametrize("kw", [dict(K=36), dict(K=64, x_off=1), dict(K=40, ldw=41)])
def test_generic_kernel(dev, kw):
    K = kw.pop("K")
    call = make_linear("generic", 70, 50, K, seed=K, act=_lib.SA_ACT_SILU, epi=_lib.SA_EPI_RESID, **kw)
    assert StagedLinear(dev, call).kernel == "linear_generic"
    run_checked(dev, call)


def test_dit_qkv_full_batch(dev):
    """The batch-64 qkv projection (16384 x 1728 x 576) against the PyTorch fp32 CPU path."""
    call = dit_block_linears(B=64)[0]
    run_checked(dev, call, check_fp64=False)


@pytest.mark.parametrize("M,N,K,tile", [(16001, 1100, 584, "64x192"), (16371, 576, 2312, "64x192"),
                                        (12345, 2113, 520, "128x192"), (16384, 576, 16, "64x192"),
                                        (16384, 576, 560, "64x192"), (16330, 576, 552, "64x192")])
def test_large_tiles_ragged(dev, M, N, K, tile):
    """Each large-grid tile at full scale with ragged M and N, and K % 16 == 8 where K is ragged. The k-loop
    runs its stages in groups of NS tiles: these K leave 0, 1 or 2 tiles after the last group (the 64 x 192 tile
    has NS = 3, k-depth 16: K = 576 / 584 / 560 give 36 / 37 / 35 tiles), with and without a partial last tile."""
    call = make_linear(f"large_{M}x{N}x{K}", M, N, K, seed=M % 97 + N + K, act=_lib.SA_ACT_GELU_TANH,
                       epi=_lib.SA_EPI_RESID_GATE, gate_off=3)
    run_checked(dev, call, expect_kernel=f"linear_mfma_{tile}", check_fp64=False)


@pytest.mark.parametrize("M,N,K,epi,act,tile", [
    # k-split 32 x 32 tiles: ragged M and N; K = 64 k-tiles plus a partial tile of 1 or 7 groups of 8
    (300, 333, 520, _lib.SA_EPI_RESID_GATE, _lib.SA_ACT_GELU_TANH, "32x32_ksplit"),
    (250, 97, 568, _lib.SA_EPI_RESID, _lib.SA_ACT_SILU, "32x32_ksplit"),
    (1000, 512, 2304, _lib.SA_EPI_STORE, _lib.SA_ACT_GELU, "32x32_ksplit"),  # long K (288 MFMAs per wave)
    (33, 1152, 64, _lib.SA_EPI_STORE, _lib.SA_ACT_NONE, "32x32_ksplit"),     # one whole k-tile
    # k-split 32 x 64 tiles (1.25 to 2 64 x 64 tiles per CU): ragged; N = 970 leaves the last tile's second
    # 32-column block wholly past N; K = 136 is two k-tiles and one group of 8
    (2000, 700, 200, _lib.SA_EPI_RESID_GATE, _lib.SA_ACT_NONE, "32x64_ksplit"),
    (1500, 970, 136, _lib.SA_EPI_RESID, _lib.SA_ACT_SILU, "32x64_ksplit"),
    (1024, 1536, 512, _lib.SA_EPI_STORE, _lib.SA_ACT_NONE, "32x64_ksplit"),  # VAE q|k|v
    # 64 x 64 tiles (two tiles per CU and more, too few for the larger tiles), ragged
    (3000, 700, 200, _lib.SA_EPI_RESID_GATE, _lib.SA_ACT_NONE, "64x64"),
])
def test_small_grid_tiles(dev, M, N, K, epi, act, tile):
    """The small-grid tiles: the k-split kernel (the waves of a workgroup on different k of one 32 x 32 or
    32 x 64 tile, partial sums added in LDS, each wave storing its share of the rows) and the 64 x 64 tile."""
    call = make_linear(f"small_{M}x{N}x{K}", M, N, K, seed=M + 3 * N + K, act=act, epi=epi,
                       gate_off=5 if epi == _lib.SA_EPI_RESID_GATE else 0)
    run_checked(dev, call, expect_kernel=f"linear_mfma_{tile}")


def test_repeat_is_bitwise_identical(dev):
    call = dit_block_linears(B=2)[4]
    st = StagedLinear(dev, call)
    try:
        a = st.run()
        b = st.run()
    finally:
        st.release()
    np.testing.assert_array_equal(a, b)
