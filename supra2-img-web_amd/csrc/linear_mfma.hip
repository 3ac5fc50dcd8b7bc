// Linear layer y = epilogue(alpha * x W^T) on fp32 MFMA for gfx950: the projections either side of
// the attention operator (app/gpu/ops.js:35-43 `linear`, app/gpu/gemm.js:116-223 `matmulShader`
// with A mode "rows" and B format "f32"): the DiT qkv / proj / q / kv / cproj / fc1 / fc2 layers.
//
//   x [M, K] rows at x + x_off + m*ldx;  W [N, K] (PyTorch layout) rows at w + n*ldw
//   r = alpha * sum_k x[m][k] W[n][k] (+ bias[n]), then act (GELU erf / GELU tanh / SiLU), then
//   y[m][n] = r, y[m][n] += r, or y[m][n] += gate[gate_off + n] * r (gemm.js:127-137).
//
// Work decomposition
//   A workgroup is 4 wave64s in a 2 x 2 grid computing a BM x BN tile (BM = 64*WM, BN = 64*WN);
//   each wave owns (32*WM) x (32*WN) outputs as WM x WN 32x32 accumulators of
//   v_mfma_f32_32x32x2f32. The x rows are the MFMA A operand and the W rows the B operand, so
//   lane l of an accumulator holds column n = l%32 and rows 8*(r/4) + 4*(l/32) + r%4 of register r:
//   every store instruction writes 128 contiguous bytes of two rows.
//   K advances in tiles of BK. Within a group of 8 consecutive k, half-wave h supplies
//   k = 8g + 4h + s at MFMA step s (s = 0..3): one b128 LDS read per operand row and group feeds
//   four MFMAs, and every (x, W) pair of k meets exactly once.
//
// Tiles move HBM/L2 -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging; scalar descriptor and
// k offset, loop-invariant lane offsets), NS stages, one barrier per k-tile. The k-loop advances NS
// tiles at a time so every stage index is a compile-time constant: the steady-state loop issues
// no VALU instruction, which on gfx950 would serialize with the MFMAs of the SIMD. LDS rows are
// BK floats (BK/4 chunks of 16 bytes); chunk c of row r sits at c ^ ((r / RP) % (BK/4)) with
// RP = 64/BK rows per 256 bytes, which makes the b128 operand reads of 16 consecutive rows
// conflict-free (measured SQ_LDS_BANK_CONFLICT = 0). The operands of the next
// group of 8 k are read from LDS while the MFMAs of the current group run, and the barrier of the
// next k-tile sits before the last group's MFMAs.
//
// The epilogue shares the SIMD datapath with the fp32 MFMAs, so it is kept short: activation and
// store mode are template parameters (no per-element branches), stores are raw buffer stores with
// scalar descriptors and row offsets, whole tiles skip the bounds checks.
// Rows past M (x) or N (W) re-read the last row (finite data, never stored); the k-tile holding K
// clamps its column to K - 8 and only its valid groups of 8 are multiplied (K % 8 == 0).
//
// Tile order (TileOrder): consecutive tiles run on one XCD (xcd_remap), and the tiles are cut into
// row super-blocks of about one XCD's share of the x row blocks. Inside a super-block the N tiles go
// in groups of W panels small enough to stay in the XCD's 4 MB L2 (the host sizes the groups), and
// inside a group the row blocks go in turn, each with the group's panels. A row block's x rows are
// then read once per group, while they are hot, and a panel once per super-block, instead of all
// of W cycling through the L2 once per row block.

#include <algorithm>
#include <type_traits>

#include <cstring>

#include "common.h"
#include "kernels.h"


namespace sa {

namespace {

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Activations of app/gpu/gemm.js:21-36. The epilogue runs on the same SIMD datapath as the fp32
// MFMAs, so the two logistic forms use one hardware exp2 and one reciprocal:
//   GELU (tanh) 0.5 x (1 + tanh(u)) = x / (1 + e^(-2u)),  u = sqrt(2/pi) (x + 0.044715 x^3);
//   SiLU        x / (1 + e^(-x)).
// Both saturate correctly: e^(...) -> inf gives x * 0, e^(...) -> 0 gives x. GELU (erf) calls erff.
__device__ __forceinline__ float logistic_times(float x, float z) {  // x / (1 + e^z)
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(z * kLog2e));
}

template <int ACT>
__device__ __forceinline__ float apply_act(float v) {
  if constexpr (ACT == LIN_ACT_GELU) return 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
  if constexpr (ACT == LIN_ACT_GELU_TANH) {
    const float u = v * fmaf(0.035677408136300125f, v * v, 0.79788456080286536f);  // sqrt(2/pi) * (1, 0.044715)
    return logistic_times(v, -2.f * u);
  }
  if constexpr (ACT == LIN_ACT_SILU) return logistic_times(v, -v);
  return v;
}

// Row block and N tile of logical tile t: super-blocks of sb_rows row blocks (the last may be
// shorter), inside one the N tiles in groups of group_n (the last may be narrower), inside a group
// the row blocks, each with the group's N tiles. Bijective on [0, tiles_m * tiles_n).
struct TileOrder {
  int tiles_m, tiles_n, group_n, sb_rows;
};

// Arguments of the MFMA kernels: 80 bytes, 96 with the tile order (launches with at most 112 bytes
// of explicit arguments start sooner). Pointers carry the callers' element offsets, resid is the
// residual rows (y itself when the caller gave none), and the row strides fit 32 bits under
// linear_mfma_supported.
struct LinArgs {
  const float* x;
  const float* w;
  const float* bias;
  const float* gate;
  float* y;
  const float* resid;
  int32_t ldx, ldw, ldy;
  int32_t M, N, K;
  float alpha;
};
static_assert(sizeof(LinArgs) + sizeof(TileOrder) <= 112, "linear kernel arguments must stay within 112 bytes");

__device__ __forceinline__ void tile_coords(int t, const TileOrder& o, int& mi, int& ni) {
  const int sb_tiles = o.sb_rows * o.tiles_n;
  const int sb = t / sb_tiles;
  const int rem = t - sb * sb_tiles;
  const int rows = min(o.sb_rows, o.tiles_m - sb * o.sb_rows);
  const int g = rem / (rows * o.group_n);
  const int off = rem - g * rows * o.group_n;
  const int w = min(o.group_n, o.tiles_n - g * o.group_n);
  mi = sb * o.sb_rows + off / w;
  ni = g * o.group_n + off % w;
}

// WM x WN accumulators per wave, BK k per tile (16 or 32), NS tiles in flight (LDS stages); the
// activation and the epilogue are compile-time, so the store loop has no per-element branches.
template <int WM, int WN, int BK, int NS, int ACT, int EPI>
__global__ __launch_bounds__(256, 2) void linear_mfma_kernel(LinArgs p, TileOrder order) {
  constexpr int BM = 64 * WM;
  constexpr int BN = 64 * WN;
  constexpr int CPR = BK / 4;            // 16-byte chunks per tile row
  constexpr int RP = 64 / BK;            // tile rows per 256 bytes (one pass over the 64 banks)
  constexpr int NG = BK / 8;             // groups of 8 k per tile
  constexpr int A_TILE = BM * BK;        // floats per stage
  constexpr int B_TILE = BN * BK;
  constexpr int STAGE = A_TILE + B_TILE;
  constexpr int NIA = BM * CPR / 256;    // DMA instructions per wave and stage (64 chunks each)
  constexpr int NIB = BN * CPR / 256;
  constexpr int NI = NIA + NIB;
  static_assert(NIA * 256 == BM * CPR && NIB * 256 == BN * CPR, "tiles must split into whole wave copies");
  static_assert(NS == 2 || NS == 3, "two or three stages");
  static_assert(NG % 2 == 0, "an even number of groups per tile");

  __shared__ __attribute__((aligned(16))) float lds[NS * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int col = lane & 31;
  const int half = lane >> 5;

  int mi, ni;
  tile_coords(xcd_remap(blockIdx.x, order.tiles_m * order.tiles_n), order, mi, ni);
  const int m0 = mi * BM;
  const int n0 = ni * BN;

  const float* xbase = p.x + (int64_t)m0 * p.ldx;
  const float* wbase = p.w + (int64_t)n0 * p.ldw;
  const int mlast = min(BM, p.M - m0) - 1;  // last valid tile row
  const int nlast = min(BN, p.N - n0) - 1;

  // Per-lane byte offsets (from the tile's first row at k = 0) of this lane's 16-byte chunk in
  // each DMA instruction: instruction n of wave w fills physical chunks (n*4 + w)*64 + lane; the
  // chunk c of row r sits at physical chunk c ^ ((r / RP) % CPR).
  unsigned aoff[NIA], boff[NIB];
  int acol[NIA], bcol[NIB];  // logical column (floats) of the chunk, for the clamped k-tile
#pragma unroll
  for (int n = 0; n < NIA; ++n) {
    const int pc_all = (n * 4 + wave) * 64 + lane;
    const int row = pc_all / CPR;
    const int c = (pc_all % CPR) ^ ((row / RP) % CPR);
    acol[n] = 4 * c;
    aoff[n] = 4u * (unsigned)(min(row, mlast) * (int)p.ldx + 4 * c);
  }
#pragma unroll
  for (int n = 0; n < NIB; ++n) {
    const int pc_all = (n * 4 + wave) * 64 + lane;
    const int row = pc_all / CPR;
    const int c = (pc_all % CPR) ^ ((row / RP) % CPR);
    bcol[n] = 4 * c;
    boff[n] = 4u * (unsigned)(min(row, nlast) * (int)p.ldw + 4 * c);
  }

  // Copies through buffer descriptors: the tile's first row is the descriptor base (scalar), the
  // k-tile's column offset the scalar soffset, and the lane's row/chunk offset a loop-invariant
  // 32-bit voffset, so the copies need no per-lane address arithmetic (VALU work serializes with
  // the MFMAs on a SIMD).
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(xbase);
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(wbase);
  const int nkt = (p.K + BK - 1) / BK;
  const int nfull = p.K / BK;  // whole k-tiles; with K % BK != 0 the last tile (nfull) holds K
  // Copies of k-tile kt into LDS stage S. The stage is a compile-time constant (the main loop
  // advances NS tiles at a time), so every LDS address below is a constant offset.
  auto issue = [&](int kt, auto stage) {
    constexpr int S = decltype(stage)::value;
    float* at = lds + S * STAGE;
    float* bt = at + A_TILE;
    if (kt < nfull) {
      const unsigned soff = 4u * (unsigned)(kt * BK);
#pragma unroll
      for (int n = 0; n < NIA; ++n) buffer_to_lds16(xr, aoff[n], at + (n * 4 + wave) * 256, soff);
#pragma unroll
      for (int n = 0; n < NIB; ++n) buffer_to_lds16(wr, boff[n], bt + (n * 4 + wave) * 256, soff);
    } else {
      // the tile holding K (always tile nfull, so its offsets are loop-invariant): columns at or
      // past K re-read the last group (never multiplied)
      const int k0 = nfull * BK;
      const unsigned soff = 4u * (unsigned)k0;
      const int kmax = p.K - 8 - k0;
#pragma unroll
      for (int n = 0; n < NIA; ++n) {
        const int shift = acol[n] > kmax + 4 ? (acol[n] & ~7) - kmax : 0;  // whole groups back
        buffer_to_lds16(xr, aoff[n] - 4u * (unsigned)shift, at + (n * 4 + wave) * 256, soff);
      }
#pragma unroll
      for (int n = 0; n < NIB; ++n) {
        const int shift = bcol[n] > kmax + 4 ? (bcol[n] & ~7) - kmax : 0;
        buffer_to_lds16(wr, boff[n] - 4u * (unsigned)shift, bt + (n * 4 + wave) * 256, soff);
      }
    }
  };

  f32x16 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = zero16();

  // LDS read offsets (floats) of this lane's operand chunk in group g: row (32*i + col) of the
  // wave's block, logical chunk 2g + half; the swizzle depends on the row only through col
  const int swz = (col / RP) % CPR;
  int goff[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) goff[g] = col * BK + 4 * ((2 * g + half) ^ swz);
  const int arow0 = wm * 32 * WM * BK;  // wave's first A row, in floats
  const int brow0 = wn * 32 * WN * BK;

  // Operands of one group in registers, double-buffered: group g + 1 (or group 0 of the next
  // tile) is read from LDS while the MFMAs of group g run.
  f32x4 ra[2][WM], rb[2][WN];
  auto read_group = [&](auto stage, int g, int slot) {
    constexpr int S = decltype(stage)::value;
    const float* at = lds + S * STAGE + arow0 + goff[g];
    const float* bt = lds + S * STAGE + A_TILE + brow0 + goff[g];
#pragma unroll
    for (int i = 0; i < WM; ++i) ra[slot][i] = *reinterpret_cast<const f32x4*>(at + i * 32 * BK);
#pragma unroll
    for (int j = 0; j < WN; ++j) rb[slot][j] = *reinterpret_cast<const f32x4*>(bt + j * 32 * BK);
  };
  // tile kt (in stage S) has landed for this thread (the younger tiles may still be in flight);
  // the barrier makes it whole and guarantees every wave has read the stage the next copies
  // overwrite: tile kt + NS - 1 goes to stage (S + NS - 1) % NS, the one tile kt - 1 used
  auto sync_tile = [&](int kt, auto stage) {
    constexpr int S = decltype(stage)::value;
    if (NS == 3 && kt + 1 < nkt) {
      wait_vmcnt<(NS == 3 ? NI : 0)>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();
    if (kt + NS - 1 < nkt) issue(kt + NS - 1, std::integral_constant<int, (S + NS - 1) % NS>{});
  };
  // the MFMAs of tile kt (stage S); the operands of group g + 1, or of the next tile's group 0,
  // are read while those of group g are multiplied
  auto step = [&](int kt, auto stage) {
    constexpr int S = decltype(stage)::value;
    constexpr int S1 = (S + 1) % NS;
    const int ng = kt < nfull ? NG : (p.K - nfull * BK) >> 3;  // valid groups of 8 k in this tile
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int cur = g & 1;  // NG is even, so group 0 of every tile sits in slot 0
      if (g + 1 < NG) {
        read_group(stage, g + 1, cur ^ 1);
      } else if (kt + 1 < nkt) {
        sync_tile(kt + 1, std::integral_constant<int, S1>{});
        read_group(std::integral_constant<int, S1>{}, 0, cur ^ 1);
      }
      if (g < ng) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ra[cur][i][s], rb[cur][j][s], acc[i][j], 0, 0, 0);
      }
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1c = std::integral_constant<int, 1>;
  using S2c = std::integral_constant<int, 2 % NS>;

  issue(0, S0{});  // tile 0 (a tile always exists: K >= 8)
  if (NS == 3 && nkt > 1) issue(1, S1c{});
  sync_tile(0, S0{});
  read_group(S0{}, 0, 0);
  int kt = 0;
  for (; kt + NS <= nkt; kt += NS) {  // tile kt + u sits in stage u
    step(kt, S0{});
    step(kt + 1, S1c{});
    if constexpr (NS == 3) step(kt + 2, S2c{});
  }
  if (kt < nkt) step(kt, S0{});
  if (NS == 3 && kt + 1 < nkt) step(kt + 1, S1c{});

  // ---- epilogue: lane holds column n = nw + 32j + col, rows mw + 32i + 8(r/4) + 4*half + r%4.
  // Buffer loads/stores over the wave's output block: a scalar descriptor, a 32-bit per-lane
  // offset and a scalar per-row offset (no 64-bit address arithmetic per element); whole tiles
  // skip the bounds checks.
  const int mw = m0 + wm * 32 * WM;
  const int nw = n0 + wn * 32 * WN;
  const bool full = m0 + BM <= p.M && n0 + BN <= p.N;
  const __amdgpu_buffer_rsrc_t yr =
      __builtin_amdgcn_make_buffer_rsrc(p.y + (int64_t)mw * p.ldy + nw, 0, 0x7fffffff, 0x00020000);
  const float* rsrc_base = p.resid + (int64_t)mw * p.ldy + nw;  // residual rows
  const __amdgpu_buffer_rsrc_t rr_ = buffer_rsrc(rsrc_base);
  const int ldy4 = 4 * (int)p.ldy;
  // Plain stores are non-temporal (cache policy NT): y is not read back here, and keeping it out of
  // the L2 leaves the W panels and x rows there (measured on the 16384-row qkv layer: 1.55x fewer L2
  // fetches). The residual epilogues keep the default policy: there NT cost 3.5% (proj, cproj).
  constexpr int kStoreCpol = EPI == LIN_EPI_STORE ? 2 : 0;
  auto store = [&](auto check) {
    constexpr bool kCheck = decltype(check)::value;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int nl = 32 * j + col;
      const bool n_ok = !kCheck || nw + nl < p.N;
      const float bias_n = (p.bias && n_ok) ? p.bias[nw + nl] : 0.f;
      float gate_n = 1.f;
      if constexpr (EPI == LIN_EPI_RESID_GATE) gate_n = n_ok ? p.gate[nw + nl] : 0.f;
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        const int voff = (32 * i + 4 * half) * ldy4 + 4 * nl;
        // residual epilogues: the 16 old values of the block are loaded together, then combined
        float old[16];
        if constexpr (EPI != LIN_EPI_STORE) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int rr = 8 * (r >> 2) + (r & 3);
            old[r] = 0.f;
            if (!kCheck || (n_ok && mw + 32 * i + 4 * half + rr < p.M))
              old[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rr_, voff, rr * ldy4, 0));
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rr = 8 * (r >> 2) + (r & 3);
          if (!kCheck || (n_ok && mw + 32 * i + 4 * half + rr < p.M)) {
            float v = apply_act<ACT>(fmaf(acc[i][j][r], p.alpha, bias_n));
            if constexpr (EPI != LIN_EPI_STORE) v = fmaf(gate_n, v, old[r]);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yr, voff, rr * ldy4, kStoreCpol);
          }
        }
      }
    }
  };
  if (full) {
    store(std::false_type{});
  } else {
    store(std::true_type{});
  }
}

// Small products (under two 64 x 64 tiles per CU: the VAE projections, batch-2 DiT calls): one
// workgroup per (32*TM) x (32*TN) output tile with KS waves on each of its 32 x 32 blocks, each of
// them on different k (32 x 32 tiles with four splits, 32 x 64 tiles with two). K advances in 64-deep tiles of 8 groups of 8; the KS waves of a block
// multiply 8/KS groups each, so a wave's MFMA chain is K/KS long and short grids spread over KS
// times the waves. The partial sums meet in LDS, and the KS waves of a block add them up (in wave
// order) for 16/KS of its accumulator registers each and run the epilogue for those rows. Copies,
// swizzle and the clamped last k-tile as in linear_mfma_kernel.
template <int TM, int TN, int KS, int ACT, int EPI>
__global__ __launch_bounds__(64 * TM * TN * KS) void linear_ksplit_kernel(LinArgs p, TileOrder order) {
  constexpr int BM = 32 * TM, BN = 32 * TN, BK = 64, NS = 2;
  constexpr int NWAVE = TM * TN * KS;
  constexpr int NT = 64 * NWAVE;     // threads
  constexpr int CPR = BK / 4;        // 16-byte chunks per tile row
  constexpr int NG = BK / 8;         // groups of 8 k per tile
  constexpr int GPW = NG / KS;       // groups per wave
  constexpr int RPW = 16 / KS;       // accumulator registers each wave finishes
  constexpr int A_TILE = BM * BK;
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int NIA = BM * CPR / NT;  // DMA instructions per thread and stage
  constexpr int NIB = BN * CPR / NT;
  static_assert(NIA * NT == BM * CPR && NIB * NT == BN * CPR, "tiles must split into whole copies");
  static_assert(GPW * KS == NG && RPW * KS == 16 && RPW % 4 == 0, "k split must divide the groups and rows");
  static_assert(NWAVE * 16 * 64 <= NS * STAGE, "partial sums must fit in the tiles");

  __shared__ __attribute__((aligned(16))) float lds[NS * STAGE];  // the partial sums reuse it

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int blk = wave % (TM * TN);  // the wave's 32 x 32 block: rows 32*(blk / TN), columns 32*(blk % TN)
  const int ks = wave / (TM * TN);   // its share of k
  const int col = lane & 31;
  const int half = lane >> 5;

  int mi, ni;
  tile_coords(xcd_remap(blockIdx.x, order.tiles_m * order.tiles_n), order, mi, ni);
  const int m0 = mi * BM;
  const int n0 = ni * BN;
  const int mlast = min(BM, p.M - m0) - 1;
  const int nlast = min(BN, p.N - n0) - 1;

  // chunk of DMA instruction n: physical chunk n*NT + tid, row pc / CPR, logical chunk c at
  // physical c ^ (row % CPR)
  unsigned aoff[NIA], boff[NIB];
  int acol[NIA], bcol[NIB];
#pragma unroll
  for (int n = 0; n < NIA; ++n) {
    const int pc_all = n * NT + tid;
    const int row = pc_all / CPR;
    const int c = (pc_all % CPR) ^ (row % CPR);
    acol[n] = 4 * c;
    aoff[n] = 4u * (unsigned)(min(row, mlast) * (int)p.ldx + 4 * c);
  }
#pragma unroll
  for (int n = 0; n < NIB; ++n) {
    const int pc_all = n * NT + tid;
    const int row = pc_all / CPR;
    const int c = (pc_all % CPR) ^ (row % CPR);
    bcol[n] = 4 * c;
    boff[n] = 4u * (unsigned)(min(row, nlast) * (int)p.ldw + 4 * c);
  }
  const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(p.x + (int64_t)m0 * p.ldx);
  const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(p.w + (int64_t)n0 * p.ldw);
  const int nkt = (p.K + BK - 1) / BK;
  const int nfull = p.K / BK;
  auto issue = [&](int kt, auto stage) {
    constexpr int S = decltype(stage)::value;
    float* at = lds + S * STAGE;
    float* bt = at + A_TILE;
    // whole tiles copy at the k-tile's column; the tile holding K (always tile nfull) re-reads the
    // last group for columns at or past K (never multiplied)
    const bool last = kt >= nfull;
    const int k0 = kt * BK;
    const unsigned soff = 4u * (unsigned)k0;
    const int kmax = p.K - 8 - k0;
#pragma unroll
    for (int n = 0; n < NIA; ++n) {
      const unsigned shift = last && acol[n] > kmax + 4 ? 4u * (unsigned)((acol[n] & ~7) - kmax) : 0u;
      buffer_to_lds16(xr, aoff[n] - shift, at + (n * NWAVE + wave) * 256, soff);
    }
#pragma unroll
    for (int n = 0; n < NIB; ++n) {
      const unsigned shift = last && bcol[n] > kmax + 4 ? 4u * (unsigned)((bcol[n] & ~7) - kmax) : 0u;
      buffer_to_lds16(wr, boff[n] - shift, bt + (n * NWAVE + wave) * 256, soff);
    }
  };

  f32x16 acc = zero16();
  const int swz = col % CPR;
  const int arow = 32 * (blk / TN) + col;  // the lane's A row and B row in the tile
  const int brow = 32 * (blk % TN) + col;
  auto step = [&](int kt, auto stage) {
    constexpr int S = decltype(stage)::value;
    wait_vmcnt<0>();
    __syncthreads();  // tile kt is whole, and every wave is done with the stage the next copy fills
    if (kt + 1 < nkt) issue(kt + 1, std::integral_constant<int, S ^ 1>{});
    const int ng = kt < nfull ? NG : (p.K - nfull * BK) >> 3;  // valid groups of 8 k in this tile
    const float* at = lds + S * STAGE + arow * BK;
    const float* bt = lds + S * STAGE + A_TILE + brow * BK;
#pragma unroll
    for (int u = 0; u < GPW; ++u) {
      const int g = GPW * ks + u;
      if (g < ng) {
        const int c = 4 * ((2 * g + half) ^ swz);
        const f32x4 ra = *reinterpret_cast<const f32x4*>(at + c);
        const f32x4 rb = *reinterpret_cast<const f32x4*>(bt + c);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ra[s], rb[s], acc, 0, 0, 0);
      }
    }
  };
  issue(0, std::integral_constant<int, 0>{});
  int kt = 0;
  for (; kt + 2 <= nkt; kt += 2) {
    step(kt, std::integral_constant<int, 0>{});
    step(kt + 1, std::integral_constant<int, 1>{});
  }
  if (kt < nkt) step(kt, std::integral_constant<int, 0>{});

  // ---- partial sums through LDS: wave w's register r of lane l at red[(w*16 + r)*64 + l]
  __syncthreads();  // every wave is done with the tiles
  float* red = lds;
#pragma unroll
  for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
  __syncthreads();
  // ---- epilogue: the wave finishes registers RPW*ks .. of its block: register r holds row
  // 8(r/4) + 4*half + r%4 of column col
  const int n = n0 + 32 * (blk % TN) + col;
  if (n >= p.N) return;
  const float bias_n = p.bias ? p.bias[n] : 0.f;
  float gate_n = 1.f;
  if constexpr (EPI == LIN_EPI_RESID_GATE) gate_n = p.gate[n];
  const float* rsrc = p.resid;
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int r = RPW * ks + k;
    const int m = m0 + 32 * (blk / TN) + 8 * (r >> 2) + 4 * half + (r & 3);
    if (m < p.M) {
      float sum = red[(blk * 16 + r) * 64 + lane];
#pragma unroll
      for (int w = 1; w < KS; ++w) sum += red[((w * TM * TN + blk) * 16 + r) * 64 + lane];
      float v = apply_act<ACT>(fmaf(sum, p.alpha, bias_n));
      const int64_t e = (int64_t)m * p.ldy + n;
      if constexpr (EPI != LIN_EPI_STORE) v = fmaf(gate_n, v, rsrc[e]);
      if constexpr (EPI == LIN_EPI_STORE) {
        __builtin_nontemporal_store(v, p.y + e);  // not read back here, as in linear_mfma_kernel
      } else {
        p.y[e] = v;
      }
    }
  }
}

// Any shape and alignment: one thread per output, 16 x 16 outputs per workgroup, K in steps of
// 16 through LDS. Used when rows are not 16-byte aligned or K % 8 != 0.
__global__ __launch_bounds__(256) void linear_generic_kernel(LinearParams p) {
  __shared__ float xs[16][17];
  __shared__ float ws[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m = blockIdx.y * 16 + ty;
  const int n = blockIdx.x * 16 + tx;
  const int mload = blockIdx.y * 16 + ty;  // row loaded by this thread (x tile)
  const int nload = blockIdx.x * 16 + ty;  // row loaded by this thread (W tile)
  float acc = 0.f;
  for (int k0 = 0; k0 < p.K; k0 += 16) {
    const int k = k0 + tx;
    xs[ty][tx] = (mload < p.M && k < p.K) ? p.x[p.x_off + (int64_t)mload * p.ldx + k] : 0.f;
    ws[ty][tx] = (nload < p.N && k < p.K) ? p.w[(int64_t)nload * p.ldw + k] : 0.f;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) acc = fmaf(xs[ty][kk], ws[tx][kk], acc);
    __syncthreads();
  }
  if (m < p.M && n < p.N) {
    float v = fmaf(acc, p.alpha, p.bias ? p.bias[n] : 0.f);
    switch (p.act) {
      case LIN_ACT_GELU: v = apply_act<LIN_ACT_GELU>(v); break;
      case LIN_ACT_GELU_TANH: v = apply_act<LIN_ACT_GELU_TANH>(v); break;
      case LIN_ACT_SILU: v = apply_act<LIN_ACT_SILU>(v); break;
      default: break;
    }
    const int64_t e = p.y_off + (int64_t)m * p.ldy + n;
    if (p.epi == LIN_EPI_STORE) p.y[e] = v;
    else p.y[e] = fmaf(p.epi == LIN_EPI_RESID_GATE ? p.gate[p.gate_off + n] : 1.f, v, (p.resid ? p.resid : p.y)[e]);
  }
}

// Groups of W panels of at most 2 MB (half an XCD's L2: the other half holds the x rows in flight),
// as few and as even as possible, over super-blocks of one XCD's share of the row blocks. Grouping
// reads each x row block once per group; it is used when those extra reads come to at most twice
// W, which the plain order fetches several times per XCD once W outgrows the L2. Measured FETCH_SIZE
// at 16384 rows: qkv (W 4 MB, x 4.7 MB per XCD, 2 groups) 150 -> 54 MiB with the NT stores, fc1
// (W 5.3 MB, 3 groups) 144 -> 83 MiB; fc2 (W 5.3 MB but x 19 MB per XCD) went up 156 -> 199-256 MiB
// when grouped and keeps the plain order. Timings were unchanged (the layers are MFMA-bound).
TileOrder tile_order(const LinearParams& p, int bm, int bn) {
  constexpr int64_t kGroupBytes = 2 << 20;
  TileOrder o;
  o.tiles_m = (int)((p.M + bm - 1) / bm);
  o.tiles_n = (int)((p.N + bn - 1) / bn);
  o.sb_rows = (o.tiles_m + 7) / 8;
  o.group_n = o.tiles_n;
  const int64_t panel = (int64_t)bn * p.K * 4;
  const int64_t w_bytes = o.tiles_n * panel;
  const int64_t groups = std::min<int64_t>((w_bytes + kGroupBytes - 1) / kGroupBytes, o.tiles_n);
  if (groups > 1) {
    const int group_n = (int)((o.tiles_n + groups - 1) / groups);
    const int64_t x_share = (int64_t)o.sb_rows * bm * p.K * 4;
    const int64_t n_groups = (o.tiles_n + group_n - 1) / group_n;
    if (group_n >= 2 && (n_groups - 1) * x_share <= 2 * w_bytes) o.group_n = group_n;
  }
  return o;
}

LinArgs lin_args(const LinearParams& p) {
  LinArgs a;
  memset(&a, 0, sizeof a);
  a.x = p.x + p.x_off;
  a.w = p.w;
  a.bias = p.bias;
  a.gate = p.gate ? p.gate + p.gate_off : nullptr;
  a.y = p.y + p.y_off;
  a.resid = (p.resid ? p.resid : p.y) + p.y_off;
  a.ldx = (int32_t)p.ldx;
  a.ldw = (int32_t)p.ldw;
  a.ldy = (int32_t)p.ldy;
  a.M = p.M;
  a.N = p.N;
  a.K = p.K;
  a.alpha = p.alpha;
  return a;
}

template <int WM, int WN, int BK, int NS, int ACT, int EPI>
hipError_t launch_tiles(const LinearParams& p, hipStream_t stream) {
  const int64_t tm = (p.M + 64 * WM - 1) / (64 * WM);
  const int64_t tn = (p.N + 64 * WN - 1) / (64 * WN);
  if (tm * tn > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((linear_mfma_kernel<WM, WN, BK, NS, ACT, EPI>), dim3((unsigned)(tm * tn)), dim3(256), 0, stream,
                     lin_args(p), tile_order(p, 64 * WM, 64 * WN));
  return hipGetLastError();
}

template <int WM, int WN, int BK, int NS, int ACT>
hipError_t launch_epi(const LinearParams& p, hipStream_t stream) {
  switch (p.epi) {
    case LIN_EPI_STORE: return launch_tiles<WM, WN, BK, NS, ACT, LIN_EPI_STORE>(p, stream);
    case LIN_EPI_RESID: return launch_tiles<WM, WN, BK, NS, ACT, LIN_EPI_RESID>(p, stream);
    case LIN_EPI_RESID_GATE: return launch_tiles<WM, WN, BK, NS, ACT, LIN_EPI_RESID_GATE>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int TM, int TN, int KS, int ACT, int EPI>
hipError_t launch_ksplit_tiles(const LinearParams& p, hipStream_t stream) {
  TileOrder o;
  o.tiles_m = (p.M + 32 * TM - 1) / (32 * TM);
  o.tiles_n = (p.N + 32 * TN - 1) / (32 * TN);
  o.group_n = o.tiles_n;  // the operands of these small products stay in the L2
  o.sb_rows = (o.tiles_m + 7) / 8;
  const int64_t n = (int64_t)o.tiles_m * o.tiles_n;
  if (n > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((linear_ksplit_kernel<TM, TN, KS, ACT, EPI>), dim3((unsigned)n), dim3(64 * TM * TN * KS), 0, stream,
                     lin_args(p), o);
  return hipGetLastError();
}

template <int TM, int TN, int KS, int ACT>
hipError_t launch_ksplit_epi(const LinearParams& p, hipStream_t stream) {
  switch (p.epi) {
    case LIN_EPI_STORE: return launch_ksplit_tiles<TM, TN, KS, ACT, LIN_EPI_STORE>(p, stream);
    case LIN_EPI_RESID: return launch_ksplit_tiles<TM, TN, KS, ACT, LIN_EPI_RESID>(p, stream);
    case LIN_EPI_RESID_GATE: return launch_ksplit_tiles<TM, TN, KS, ACT, LIN_EPI_RESID_GATE>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int TM, int TN, int KS>
hipError_t launch_ksplit(const LinearParams& p, hipStream_t stream) {
  switch (p.act) {
    case LIN_ACT_NONE: return launch_ksplit_epi<TM, TN, KS, LIN_ACT_NONE>(p, stream);
    case LIN_ACT_GELU: return launch_ksplit_epi<TM, TN, KS, LIN_ACT_GELU>(p, stream);
    case LIN_ACT_GELU_TANH: return launch_ksplit_epi<TM, TN, KS, LIN_ACT_GELU_TANH>(p, stream);
    case LIN_ACT_SILU: return launch_ksplit_epi<TM, TN, KS, LIN_ACT_SILU>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int WM, int WN, int BK, int NS>
hipError_t launch_act(const LinearParams& p, hipStream_t stream) {
  switch (p.act) {
    case LIN_ACT_NONE: return launch_epi<WM, WN, BK, NS, LIN_ACT_NONE>(p, stream);
    case LIN_ACT_GELU: return launch_epi<WM, WN, BK, NS, LIN_ACT_GELU>(p, stream);
    case LIN_ACT_GELU_TANH: return launch_epi<WM, WN, BK, NS, LIN_ACT_GELU_TANH>(p, stream);
    case LIN_ACT_SILU: return launch_epi<WM, WN, BK, NS, LIN_ACT_SILU>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool linear_mfma_supported(const LinearParams& p) {
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  // copies address a tile's rows as 32-bit byte offsets from its first row (up to 128 x rows and
  // 192 W rows, plus the k offset <= the row stride); stores address up to 128 output rows likewise
  // (the same bounds keep the row strides within the 32 bits of the kernels' arguments)
  return p.K % 8 == 0 && a16(p.x) && a16(p.w) && p.x_off % 4 == 0 && p.ldx % 4 == 0 && p.ldw % 4 == 0 &&
         (int64_t)(64 * 2 + 1) * p.ldx * 4 < 0x7fffffffLL && (int64_t)(64 * 3 + 1) * p.ldw * 4 < 0x7fffffffLL &&
         (int64_t)64 * 2 * p.ldy * 4 < 0x7fffffffLL;
}

LinearTile linear_mfma_tile(const LinearParams& p, int num_cus) {
  // Measured per layer on the DiT linears at 16384 rows (after a warm-up; seven tile / k-depth /
  // stage variants): 128 x 192 tiles (2 x 3 accumulators per wave, k-depth 32, two stages) for the
  // 2304-wide fc1 (324 us; 64 x 192: 336 us); 64 x 192 tiles (one 32 x 96 strip per wave, each x
  // operand read feeding three MFMAs) with k-depth 16 and three stages at three workgroups per CU
  // for qkv (245 us; k-depth 32 / two stages 254, 128 x 192 271) and the 576-wide layers (proj/q/
  // cproj 85-88 us, fc2 320 us; 64 x 64: 90-95 and 337). Grids of fewer 64 x 64 tiles than 1.25
  // per CU take linear_ksplit_kernel, whose quarter-K waves spread them over the SIMDs (us, 64 x 64
  // -> k-split: VAE output projection 1024 x 512 x 512 11.75 -> 8.1, context k|v 77 x 1152 x 576 13.2
  // -> 6.3, batch-2 proj/q/cproj 512 x 576 x 576 12.6-13.0 -> 8.4-8.7, fc1 512 x 2304 x 576 21.4 ->
  // 19.2, fc2 512 x 576 x 2304 43.4 -> 23.0). Grids of 1.25 to 2 such tiles per CU take 32 x 64
  // tiles with k split in two, whose count is twice that and so shares out more evenly over the CUs
  // (VAE q|k|v 1024 x 1536 x 512, 384 tiles: 64 x 64 18.7-19.2, 32 x 64 / two splits 17.4, 64 x 32
  // 17.5, 64 x 32 / four splits 17.9, 64 x 64 / two splits 20.7, 32 x 32 / four splits 18.9-19.4);
  // wider grids keep 64 x 64 tiles.
  const int64_t tiles_wide = ((p.M + 127) / 128) * ((p.N + 191) / 192);
  const int64_t tiles_tall = ((p.M + 63) / 64) * ((p.N + 191) / 192);
  const int64_t tiles_64 = ((p.M + 63) / 64) * ((p.N + 63) / 64);
  if (p.N >= 2048 && tiles_wide >= num_cus) return {2, 3, 32, 2, 0};
  if ((p.N % 192 == 0 || p.N >= 1024) && tiles_tall >= 3 * (int64_t)num_cus) return {1, 3, 16, 3, 0};
  if (4 * tiles_64 < 5 * (int64_t)num_cus) return {1, 1, 64, 2, 4};
  if (tiles_64 < 2 * (int64_t)num_cus) return {1, 2, 64, 2, 2};
  return {1, 1, 32, 2, 0};
}

const char* linear_kernel_name(const LinearParams& p, int num_cus) {
  if (!linear_mfma_supported(p)) return "linear_generic";
  const LinearTile t = linear_mfma_tile(p, num_cus);
  if (t.ksplit == 4) return "linear_mfma_32x32_ksplit";
  if (t.ksplit == 2) return "linear_mfma_32x64_ksplit";
  if (t.wm == 2) return "linear_mfma_128x192";
  if (t.wn == 3) return "linear_mfma_64x192";
  return "linear_mfma_64x64";
}

hipError_t launch_linear(const LinearParams& p, int num_cus, hipStream_t stream) {
  if (!linear_mfma_supported(p)) {
    const dim3 grid((unsigned)((p.N + 15) / 16), (unsigned)((p.M + 15) / 16));
    if ((p.N + 15) / 16 > 0x7fffffff || (p.M + 15) / 16 > 65535) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(linear_generic_kernel, grid, dim3(256), 0, stream, p);
    return hipGetLastError();
  }
  const LinearTile t = linear_mfma_tile(p, num_cus);
  if (t.ksplit == 4) return launch_ksplit<1, 1, 4>(p, stream);
  if (t.ksplit == 2) return launch_ksplit<1, 2, 2>(p, stream);
  if (t.wm == 2) return launch_act<2, 3, 32, 2>(p, stream);
  if (t.wn == 3) return launch_act<1, 3, 16, 3>(p, stream);
  return launch_act<1, 1, 32, 2>(p, stream);
}

}  // namespace sa
