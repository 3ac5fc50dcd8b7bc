// Flash attention on fp32 MFMA for gfx950 (CDNA4), head dim 64 or 128.
//
// Replaces the fused WGSL kernel of app/gpu/kernels.js:164-316 (online softmax over key blocks,
// keys >= Lk masked) and, for the biased/masked calls that app/gpu/ops.js:119-147 sends down the
// unfused GEMM -> softmax(+bias) -> GEMM path, fuses the bias and the key mask into the same pass.
//
// Work decomposition
//   A workgroup is 4 wave64s. Each wave owns 32 queries of one (sequence b, head h). With
//   NSPLIT = 1 the 4 waves cover 128 consecutive queries and share every 32-key K/V tile staged
//   in LDS. With NSPLIT = 2 the waves split the key blocks instead (two query groups of 32, each
//   seeing every other key block) and their partial softmax states are merged in LDS at the end:
//   launches of under ~2 waves per SIMD then still spread over many SIMDs. (Head-dim-64 launches of
//   at most 256 query groups, such as the batch-2 DiT calls, take flash_small instead.)
//   A launch of one round of four workgroups per CU plus at most half a round (the batch-64 DiT
//   self-attention: 1152 units on 256 CUs) runs as one round whose first workgroups, one per CU, each
//   take a 64-query NSPLIT = 2 piece of the units left over after their own unit
//   (flash_mfma_fold_kernel): every CU carries the same work, and no second launch waits for the
//   round to drain.
//
// Per 32-key block a wave computes the transposed score tile S^T = K Q^T with 32x32x2 fp32 MFMAs:
//   A operand  K[key = lane%32][d], B operand Q^T[d][query = lane%32], the head dim split between
//   the two half-waves by 16-byte chunks: half-wave `half` takes chunks 2i + half (i = 0..D/8-1),
//   so each Q load instruction reads 32 contiguous bytes per row. Q stays in VGPRs for the whole
//   kernel.
//   Accumulator layout: lane l holds query l%32 and keys 8*(r/4) + 4*(l/32) + r%4 in register r,
//   so the row max and row sum of a query are in-lane over 16 registers plus one exchange with
//   lane l^32 (v_permlane32_swap).
// The probabilities P then feed O^T += V^T P^T directly from the accumulator registers: MFMA r of
//   the PV step uses P register r as its B operand (keys {8*(r/4)+r%4, 8*(r/4)+4+r%4} across the
//   half-waves) and reads V for exactly that key pair from LDS as its A operand.
//   O^T accumulates in D/32 tiles of 16 registers: lane l holds query l%32, dims
//   32*t + 8*(r/4) + 4*(l/32) + r%4.
//
// Softmax arithmetic (base 2): Q is pre-multiplied by scale*log2(e) when it is loaded, so the MFMA
//   produces u = s*scale*log2(e) directly; u += bias*log2(e); masked keys get u = -inf.
//   m = running reference (seeded with -FLT_MAX), p = exp2(u - m), l = sum p, O = sum p V;
//   output O / l, or 0 when every key is masked. The reference is moved (O and l rescaled by
//   alpha = exp2(m_old - m_new)) only when some row's block maximum exceeds it by more than
//   kRescaleSlack: otherwise p <= 2^kRescaleSlack and numerator and denominator share the same
//   stale reference, so the quotient is unchanged while most blocks skip the rescale. Every VALU
//   instruction is issue time the SIMD's MFMA pipe loses (measured: ~4 cycles per VALU op,
//   ~16 per exp), so the per-block VALU path is kept short.
//
// K/V tiles move HBM -> LDS with global_load_lds_dwordx4 (no VGPR staging), double-buffered: the
// next tile streams in while the current one is consumed, one barrier per key block. Rows past the
// last valid key re-read the last valid row (finite data, masked out of the softmax).
//
// Start-up and output (single-split kernels):
//   - At launch every resident workgroup asks for its Q rows and first K/V tile at once (48 KiB
//     each, ~48 MB over a full chip at 4 workgroups per CU); served interleaved, the median
//     workgroup waited ~11 us for its first tile while the MFMA pipes idled. The g-th workgroup of
//     each CU of the first residency (dispatch order: blockIdx / num_cus) therefore starts its loads
//     g * kStaggerTicks later, so the memory system serves one workgroup per CU first and compute
//     starts within a few microseconds while the rest streams in.
//   - O is staged through LDS (the K/V tiles are free by then) and written as whole 256-byte rows
//     instead of 32-byte pieces of 32 rows per instruction, which the memory system absorbs faster.
// LDS tiles are [KT keys][D] in 16-byte chunks, XOR-swizzled per row:
//   K: chunk c of row r at c ^ (r & 15), so the b128 reads of 16 consecutive rows hit all banks;
//   V: chunk c of row r at c ^ (8 * ((r >> 2) & 1)), so the two half-waves (rows 4 apart) read
//      disjoint bank halves.

#include <string.h>

#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace sa {

namespace {

constexpr float kRescaleSlack = 8.f;  // log2 units: p stays <= 256 between rescales

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Four workgroups (16 waves) per CU for the unbiased head-dim-64 single-split kernels, which fit
// 128 VGPRs per wave without spilling (the bias and key-mask variants would spill).
template <int D, int NSPLIT, int BIAS, int MASK>
constexpr int kMinBlocksPerCU = (D == 64 && NSPLIT == 1 && BIAS == BIAS_NONE && MASK != MASK_KEY_MASK) ? 4 : 1;

// Start-up stagger step, in ticks of the 100 MHz real-time counter (3.5 us): about the time the
// memory system takes to deliver the first tiles of one workgroup per CU over the whole chip.
constexpr unsigned kStaggerTicks = 350;

// The host sequence schedule (order[rank] = sequence): a second kernel argument of the scheduled
// variant only.
struct FlashOrder {
  uint8_t order[kMaxOrder];
};
struct NoOrder {};

// The K/V staging area of one flash_body: [stage][K tile, V tile] of 32 * NSPLIT keys, two stages
// (one for a folded piece, which shares the LDS of the kernel's first unit).
template <int D, int NSPLIT, bool FOLD = false>
constexpr int kLdsFloats = (FOLD ? 1 : 2) * 2 * 32 * NSPLIT * D;
// Names the folded kernel's instantiations of flash_body, so that they have their own LDS array.
template <int D>
struct FoldTag {};

// FOLD: the 64-query piece a workgroup of the folded launch runs after its own unit (2-way key
// split, one LDS stage, no operand prefetch: it runs within the first unit's 128 VGPRs and 32 KiB,
// staging its tiles in `lds_in`, the first unit's area, which that body passes out through
// `lds_out`; tid_in is the thread id, opaque, so that the piece recomputes its lane addressing
// instead of keeping the first unit's live; piece, in [0, p.tiles), is the piece's index in place of
// the block index). Tag names the folded kernel's instantiations, so that
// they have LDS arrays of their own; the plain kernels' instantiations (Tag void) compile to the
// code they had before the folded kernel existed.
template <int D, int NSPLIT, int BIAS, int MASK, typename Order, bool FOLD = false, typename Tag = void>
__device__ __forceinline__ void flash_body(const FlashArgs& p, const Order& ord, const int tid_in = 0,
                                           float* lds_in = nullptr, float** lds_out = nullptr, const int piece = 0) {
  constexpr int QG = 4 / NSPLIT;         // query groups (of 32) per workgroup
  constexpr int QT = 32 * QG;            // queries per workgroup
  constexpr int KT = 32 * NSPLIT;        // keys staged per step
  constexpr int QREG = D / 2;            // Q values per lane
  constexpr int NDB = D / 32;            // 32-dim output tiles
  constexpr int CPR = D / 4;             // 16-byte chunks per row
  constexpr int TILE = KT * D;           // floats per tensor per stage
  constexpr int NI = KT * CPR / 256;     // LDS-DMA instructions per thread per tensor per step
  static_assert(NI * 256 == KT * CPR, "tile must split evenly over 256 threads");
  constexpr int RB = QT + KT - 1;        // relative-bias entries needed per step
  constexpr int MSTRIDE = 16 * NDB + 2;  // merge record per lane: O tiles, m, l
  constexpr int STAGES = FOLD ? 1 : 2;
  static_assert(!FOLD || (NSPLIT == 2 && BIAS == BIAS_NONE && MASK == MASK_NONE), "only the plain split kernel folds");
  static_assert((NSPLIT - 1) * QG * 64 * MSTRIDE <= STAGES * 2 * TILE, "merge records must fit in the tiles");
  static_assert(kLdsFloats<D, NSPLIT, FOLD> == STAGES * 2 * TILE, "LDS staging size");

  __shared__ __attribute__((aligned(16))) float lds[FOLD ? 1 : kLdsFloats<D, NSPLIT>];  // [stage][K tile, V tile]
  if constexpr (!std::is_void<Tag>::value && !FOLD) *lds_out = lds;
  auto lds_at = [&](int off) -> float* {
    if constexpr (FOLD) {
      return lds_in + off;
    } else {
      return lds + off;
    }
  };

  __shared__ float lds_rb[BIAS == BIAS_RELPOS ? 2 * RB : 1];         // [stage][relative bias]
  __shared__ float lds_km[MASK == MASK_KEY_MASK ? 2 * KT : 1];       // [stage][0 or -inf per key]

  // Scheduled key-length launches (workgroups of 1-4 key blocks, a new workgroup starting whenever one
  // ends) raise the wave priority until their first loads are issued: the schedule lookup, key
  // length and address arithmetic otherwise wait behind the resident waves' MFMAs (sweep
  // cross-attention 39.6 -> 38.7 us; raised only after the unit decode it measured 40.6 us, and the
  // same boost on the self-attention launches cost them about 1 us)
  if constexpr (MASK == MASK_KEY_LEN_ORDERED) __builtin_amdgcn_s_setprio(3);
  const int tid = FOLD ? tid_in : (int)threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform in a scalar register, so per-block conditions compile to scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = wave % QG;
  const int ks = wave / QG;
  const int col = lane & 31;
  const int half = lane >> 5;

  const int q_tiles = (p.Lq + QT - 1) / QT;
  // the key-split kernels also run the leftover units of a larger launch: aux is then the first unit
  int tile = xcd_remap(FOLD ? piece : (int)blockIdx.x, p.tiles);
  if constexpr (NSPLIT > 1 && MASK != MASK_KEY_MASK) tile += p.aux;
  const int qtile = tile % q_tiles;
  tile /= q_tiles;
  const int h = tile % p.H;
  int b = tile / p.H;
  if constexpr (MASK == MASK_KEY_LEN_ORDERED) b = ord.order[b];  // the host schedule
  const int q0 = qtile * QT;
  const int qi = q0 + qg * 32 + col;
  const bool q_valid = qi < p.Lq;

  int kv_len = p.Lk;
  if constexpr (MASK == MASK_KEY_LEN || MASK == MASK_KEY_LEN_ORDERED) kv_len = min(max(static_cast<const int32_t*>(p.mask)[b], 0), p.Lk);
  const int nblk = (kv_len + 31) >> 5;
  const int nstep = (nblk + NSPLIT - 1) / NSPLIT;
  constexpr bool use_kmask = MASK == MASK_KEY_MASK;
  const uint8_t* kmask = use_kmask ? static_cast<const uint8_t*>(p.mask) + (int64_t)b * p.aux : nullptr;

  const float* kbase = p.k + (int64_t)b * p.sk + h * D;
  const float* vbase = p.v + (int64_t)b * p.sv + h * D;

  // ---- HBM -> LDS copy of one step. Lane `lane` of instruction n fills physical chunk
  // (n*4 + wave)*64 + lane of the tile: row `drow[n]`, logical chunk dck[n] (K) / dcv[n] (V).
  // Full steps address rows from a wave-uniform base plus per-lane 32-bit offsets; the step
  // holding the last valid key clamps rows past it to that key.
  auto chunk_of = [&](int n, int& row, int& ck, int& cv) {
    int pc_all = (n * 4 + wave) * 64 + lane;
    if constexpr (FOLD) {
      // a folded piece recomputes its offsets at every copy (an opaque thread id: nothing to hoist)
      int t = tid;
      asm volatile("" : "+v"(t));
      pc_all = n * 256 + t;
    }
    row = pc_all / CPR;
    const int pc = pc_all % CPR;
    ck = 4 * (pc ^ (row & 15));
    cv = 4 * (pc ^ (((row >> 2) & 1) << 3));
  };
  unsigned koff[NI], voff[NI];  // byte offsets from the step's first row
  if constexpr (!FOLD) {
#pragma unroll
    for (int n = 0; n < NI; ++n) {
      int row, ck, cv;
      chunk_of(n, row, ck, cv);
      koff[n] = 4u * (unsigned)(row * (int)p.ldk + ck);
      voff[n] = 4u * (unsigned)(row * (int)p.ldv + cv);
    }
  }
  // rows past `lim` (the key length, or Lk for a speculative issue) re-read row lim - 1
  auto issue = [&](int step, int buf, int lim) {
    float* kt = lds_at(buf * 2 * TILE);
    float* vt = kt + TILE;
    const int key0 = step * KT;
    if (key0 + KT <= lim) {
      const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(kbase + (int64_t)key0 * p.ldk);
      const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(vbase + (int64_t)key0 * p.ldv);
#pragma unroll
      for (int n = 0; n < NI; ++n) {
        const int blk64 = n * 4 + wave;  // 64-chunk (1 KiB) block of the tile
        if constexpr (FOLD) {
          // a folded piece recomputes its offsets at every copy rather than holding them
          int row, ck, cv;
          chunk_of(n, row, ck, cv);
          koff[n] = 4u * (unsigned)(row * (int)p.ldk + ck);
          voff[n] = 4u * (unsigned)(row * (int)p.ldv + cv);
        }
        buffer_to_lds16(kr, koff[n], kt + blk64 * 256);
        buffer_to_lds16(vr, voff[n], vt + blk64 * 256);
      }
    } else {
#pragma unroll
      for (int n = 0; n < NI; ++n) {
        const int blk64 = n * 4 + wave;
        int row, ck, cv;
        chunk_of(n, row, ck, cv);
        const int key = min(key0 + row, lim - 1);
        load_to_lds16(kbase + (int64_t)key * p.ldk + ck, kt + blk64 * 256);
        load_to_lds16(vbase + (int64_t)key * p.ldv + cv, vt + blk64 * 256);
      }
    }
    if constexpr (BIAS == BIAS_RELPOS) {
      // entry e covers LUT index key0 - (q0 + QT - 1) + (Lq - 1) + e
      if (tid < RB) {
        const int li = key0 - (q0 + QT - 1) + (p.Lq - 1) + tid;
        float val = 0.f;
        if (li >= 0 && li <= p.Lq + p.Lk - 2) {
          int bucket = p.lut[li];
          bucket = min(max(bucket, 0), p.num_buckets - 1);
          val = p.bias[bucket * p.H + h] * kLog2e;
        }
        lds_rb[buf * RB + tid] = val;
      }
    }
    if constexpr (use_kmask) {
      // additive key mask of the step, read unconditionally at a clamped index (branch-free)
      if (tid < KT) {
        const int key = key0 + tid;
        const uint8_t byte = kmask[min(key, p.Lk - 1)];
        lds_km[buf * KT + tid] = (key < kv_len && byte != 0) ? 0.f : -INFINITY;
      }
    }
  };

  f32x16 oacc[NDB];
#pragma unroll
  for (int t = 0; t < NDB; ++t) oacc[t] = zero16();
  float m = kMaxSeed;
  float l = 0.f;

  // ---- start-up stagger (p.aux > 0 only for the 4-workgroups-per-CU kernels): the g-th
  // workgroup of each CU in the first residency waits g steps before its first loads
  if constexpr (kMinBlocksPerCU<D, NSPLIT, BIAS, MASK> == 4) {
    if (p.aux > 0) {
      const unsigned gen = blockIdx.x / (unsigned)p.aux;
      if (gen > 0 && gen < 4) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (__builtin_amdgcn_s_memrealtime() - t0 < gen * kStaggerTicks) __builtin_amdgcn_s_sleep(2);
      }
    }
  }
  // Key-length launches of the single-split kernels issue their first two tiles before the key
  // length is known (rows past Lk clamped): one dependent load less before the first data. Keys past
  // the length are masked out of the scores, and the V rows past it, which may hold anything, are
  // zeroed in LDS before the products that read them (spec_fix below).
  constexpr bool kSpec = (MASK == MASK_KEY_LEN || MASK == MASK_KEY_LEN_ORDERED) && NSPLIT == 1;
  if constexpr (kSpec) {
    if (p.Lk > 0) issue(0, 0, p.Lk);
  } else if (nstep > 0) {
    issue(0, 0, kv_len);  // the first tile streams in while Q loads
  }

  // ---- Q into registers, pre-scaled: lane holds scale*log2(e)*Q[qi][8i + 4*half + j] in qr[4i + j]
  float qr[QREG];
  {
    // unconditional loads from a clamped row (no branch per load); rows past Lq are zeroed after
    const float* src = p.q + (int64_t)b * p.sq + (int64_t)min(qi, p.Lq - 1) * p.ldq + h * D;
    f32x4 xq[QREG / 4];
#pragma unroll
    for (int i = 0; i < QREG / 4; ++i) xq[i] = *reinterpret_cast<const f32x4*>(src + 4 * (2 * i + half));
    // Stage 1 is unused until the loop: the second step's tile streams in from the start too,
    // rather than after the first barrier (which left the two-step loops of the key-split
    // kernels waiting for their second tile).
    if constexpr (kSpec) {
      if (p.Lk > KT) issue(1, 1, p.Lk);
    } else if (STAGES == 2 && nstep > 1) {
      issue(1, 1, kv_len);
    }
    if constexpr (MASK == MASK_KEY_LEN_ORDERED) __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int i = 0; i < QREG / 4; ++i) {
      const float sc = q_valid ? p.scale_log2 : 0.f;
      qr[4 * i + 0] = xq[i][0] * sc;
      qr[4 * i + 1] = xq[i][1] * sc;
      qr[4 * i + 2] = xq[i][2] * sc;
      qr[4 * i + 3] = xq[i][3] * sc;
    }
  }


  // One loop step on LDS stage `stage`: a compile-time constant in the single-split kernels (two
  // steps per iteration, so every LDS address of a step is a base register plus an immediate
  // offset), a run-time value in the key-split kernels, whose loops run one to a few steps.
  auto step_body = [&](int step, auto stage) {
    const int buf = stage;
    // stage `buf` has landed for this thread; the barrier makes it whole, and every wave has
    // finished reading stage buf^1 (the previous step), which the next issue (from step 1 on:
    // step 1 itself was issued before the loop) overwrites
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (STAGES == 2 && step >= 1 && step + 1 < nstep) issue(step + 1, buf ^ 1, kv_len);
    const int blk = step * NSPLIT + ks;
    if (blk < nblk) {
      const int k0 = blk * 32;
      const float* kt = lds_at(buf * 2 * TILE);
      const float* vt = kt + TILE;
      // a speculatively issued tile holding the last valid key: its V rows past the key length are
      // zeroed (every thread its own chunks, rows pc / CPR) before the PV products read them
      const bool spec_fix = kSpec && step <= 1 && k0 + 32 > kv_len;
      if (spec_fix) {
        float* vw = lds_at(buf * 2 * TILE + TILE);
#pragma unroll
        for (int i = 0; i < KT * CPR / 256; ++i) {
          const int pc = tid + 256 * i;
          if (k0 + pc / CPR >= kv_len) *reinterpret_cast<f32x4*>(vw + 4 * pc) = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
      // ---- u^T = K (scaled Q)^T for 32 keys x 32 queries
      f32x16 s = zero16();
      const float* krow = kt + (ks * 32 + col) * D;
      const int ksw = col & 15;
      // Key-split variants (head dim 64) run one or two waves per SIMD with registers to spare: all
      // K operands of the block are read before the MFMA chain, so it never waits on LDS (with 4
      // waves per SIMD the other waves hide those waits and the registers are not there).
      constexpr bool kPrefetch = NSPLIT > 1 && D == 64 && !FOLD;
      f32x4 kpre[kPrefetch ? QREG / 4 : 1];
      if constexpr (kPrefetch) {
#pragma unroll
        for (int i = 0; i < QREG / 4; ++i)
          kpre[i] = *reinterpret_cast<const f32x4*>(krow + 4 * ((2 * i + half) ^ ksw));
      }
      // Key-length masks, a block with at most 16 valid keys (the last block of a sequence): its scores
      // for keys 0..15 only, as four 16x16 blocks of v_mfma_f32_16x16x1f32 at half the cycles of the
      // 32x32x2 chain. Block b takes its operands from lanes 16b..16b+15: query half b & 1 and head-dim
      // half b >> 1, i.e. each lane's own query (col) and its own Q registers, with K row col & 15.
      // The two head-dim halves are summed in-lane (block b's result sits in registers 4b..4b+3, row
      // 4(l/16) + r, column l % 16), and one v_permlane16_swap and one v_permlane32_swap per register
      // pair move keys 4h + r and 8 + 4h + r of query col to registers r and 4 + r of the 32x32 layout
      // (h = half); registers 8..15 (keys 16..31) are masked below.
      constexpr bool kShortScores = MASK == MASK_KEY_LEN || MASK == MASK_KEY_LEN_ORDERED;
      if (kShortScores && kv_len - k0 <= 16) {
        const float* krow16 = kt + (ks * 32 + (col & 15)) * D;
#pragma unroll
        for (int i = 0; i < QREG / 4; ++i) {
          const f32x4 kv = *reinterpret_cast<const f32x4*>(krow16 + 4 * ((2 * i + half) ^ ksw));
          s = __builtin_amdgcn_mfma_f32_16x16x1f32(kv[0], qr[4 * i + 0], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_16x16x1f32(kv[1], qr[4 * i + 1], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_16x16x1f32(kv[2], qr[4 * i + 2], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_16x16x1f32(kv[3], qr[4 * i + 3], s, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = s[r] + s[8 + r];       // query half 0
          const float y = s[4 + r] + s[12 + r];  // query half 1
          const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
          const auto z = __builtin_amdgcn_permlane32_swap(a[0], a[1], false, false);
          s[r] = __uint_as_float(z[0]);
          s[4 + r] = __uint_as_float(z[1]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < QREG / 4; ++i) {
          const int c = (2 * i + half) ^ ksw;
          const f32x4 kv = kPrefetch ? kpre[i] : *reinterpret_cast<const f32x4*>(krow + 4 * c);
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[0], qr[4 * i + 0], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[1], qr[4 * i + 1], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[2], qr[4 * i + 2], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[3], qr[4 * i + 3], s, 0, 0, 0);
        }
      }
      // likewise the V operands of the PV step (head dim 64), read while the softmax runs
      constexpr bool vPrefetch = NSPLIT > 1 && D == 64 && !FOLD;
      const float* vrow = vt + (ks * 32 + 4 * half) * D + col;
      float vpre[vPrefetch ? 16 * NDB : 1];
      if constexpr (vPrefetch) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int t = 0; t < NDB; ++t) vpre[r * NDB + t] = vrow[32 * (t ^ half) + (8 * (r >> 2) + (r & 3)) * D];
      }

      // ---- bias and masks
      float u[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) u[r] = s[r];
      if constexpr (BIAS == BIAS_RELPOS) {
        // rb entry for (key, qi): key - qi + (q0 + QT - 1) - step*KT
        const float* rb = lds_rb + buf * RB + (k0 - step * KT + 4 * half - qi + q0 + QT - 1);
#pragma unroll
        for (int r = 0; r < 16; ++r) u[r] += rb[8 * (r >> 2) + (r & 3)];
      } else if constexpr (BIAS == BIAS_DENSE) {
        // unconditional loads at clamped indices; out-of-range keys are masked below
        const float* brow = p.bias + (int64_t)b * p.sbias + ((int64_t)h * p.Lq + min(qi, p.Lq - 1)) * p.Lk;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
          u[r] = fmaf(brow[min(key, p.Lk - 1)], kLog2e, u[r]);
        }
      }
      if constexpr (use_kmask) {
        // the staged additive mask also covers keys past Lk
        const float* km = lds_km + buf * KT + (k0 - step * KT) + 4 * half;
#pragma unroll
        for (int r = 0; r < 16; ++r) u[r] += km[8 * (r >> 2) + (r & 3)];
      } else if (k0 + 32 > kv_len) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
          u[r] = key < kv_len ? u[r] : -INFINITY;
        }
      }

      // ---- online softmax with a lazily moved reference
      float mb = u[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mb = max_nan(mb, u[r]);
      mb = max_with_partner(mb);
      if (step == 0) {
        // the wave's first block: its maximum becomes the reference (O and l are still zero, so there is
        // nothing to rescale; -FLT_MAX stays for rows with every key masked)
        m = max_nan(m, mb);
      } else if (__builtin_amdgcn_ballot_w64(mb > m + kRescaleSlack) != 0) {
        const float m_new = max_nan(m, mb);
        const float alpha = fast_exp2(m - m_new);
        m = m_new;
        l *= alpha;
#pragma unroll
        for (int t = 0; t < NDB; ++t) oacc[t] *= alpha;
      }
      float pr[16];
      pr[0] = fast_exp2(u[0] - m);
      float ps = pr[0];  // (not 0 + pr[0]: the compiler keeps an add of zero, for -0)
#pragma unroll
      for (int r = 1; r < 16; ++r) {
        pr[r] = fast_exp2(u[r] - m);
        ps += pr[r];
      }
      l += ps;

      // ---- O^T += V^T P^T; V element (row, 32t + col) sits in chunk (8t + col/4) ^ 8*half.
      // The D/32 output tiles are independent accumulation chains: interleaving them (each P
      // register feeding one MFMA per tile in turn) keeps the MFMA pipe fed while an exp2 or an
      // LDS read is still in flight.
      auto pv_group = [&](auto g) {
#pragma unroll
        for (int r = 4 * g; r < 4 * g + 4; ++r) {
#pragma unroll
          for (int t = 0; t < NDB; ++t) {
            const float vv = vPrefetch ? vpre[r * NDB + t] : vrow[32 * (t ^ half) + (8 * (r >> 2) + (r & 3)) * D];
            oacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, pr[r], oacc[t], 0, 0, 0);
          }
        }
      };
      // Key-length masks: in the block holding the last valid key, P registers 8..15 (keys 16..31)
      // are all zero when at most 16 keys are valid, and V rows there are finite copies of the last
      // valid key, so their products are skipped with every sum bitwise the same (sweep
      // cross-attention 35.0 -> 34.0 us; skipping by groups of 8 keys, three branches, 34.6 us)
      constexpr bool kSkip = MASK == MASK_KEY_LEN || MASK == MASK_KEY_LEN_ORDERED;
      if (spec_fix) __syncthreads();  // the zeroed V rows are in place
      pv_group(std::integral_constant<int, 0>{});
      pv_group(std::integral_constant<int, 1>{});
      if (!kSkip || kv_len - k0 > 16) {
        pv_group(std::integral_constant<int, 2>{});
        pv_group(std::integral_constant<int, 3>{});
      }
    }
  };
  if constexpr (NSPLIT == 1) {
    int step = 0;
    for (; step + 1 < nstep; step += 2) {
      step_body(step, std::integral_constant<int, 0>{});
      step_body(step + 1, std::integral_constant<int, 1>{});
    }
    if (step < nstep) step_body(step, std::integral_constant<int, 0>{});
  } else {
    // the key-split kernels run one to a few steps: one copy of the body, stage chosen at run time
    for (int step = 0; step < nstep; ++step) {
      if constexpr (STAGES == 2) {
        step_body(step, step & 1);
      } else {
        // one stage: the next tile goes in once every wave is done with this one
        step_body(step, 0);
        __syncthreads();
        if (step + 1 < nstep) issue(step + 1, 0, kv_len);
      }
    }
  }

  // ---- merge the key splits: waves ks > 0 publish (O, m, l), wave ks == 0 combines
  if constexpr (NSPLIT > 1) {
    __syncthreads();  // every wave is done with the tiles the records overwrite
    float* rec = lds_at(((ks - 1) * QG + qg) * 64 * MSTRIDE + lane);
    if (ks > 0) {
#pragma unroll
      for (int t = 0; t < NDB; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) rec[(16 * t + r) * 64] = oacc[t][r];
      rec[(16 * NDB) * 64] = m;
      rec[(16 * NDB + 1) * 64] = l;
    }
    __syncthreads();
    if (ks > 0) return;
    float mt = m;
#pragma unroll
    for (int sp = 1; sp < NSPLIT; ++sp) {
      const float* o2 = lds_at(((sp - 1) * QG + qg) * 64 * MSTRIDE + lane);
      mt = fmaxf(mt, o2[(16 * NDB) * 64]);
    }
    const float a0 = fast_exp2(m - mt);
    l *= a0;
#pragma unroll
    for (int t = 0; t < NDB; ++t) oacc[t] *= a0;
#pragma unroll
    for (int sp = 1; sp < NSPLIT; ++sp) {
      const float* o2 = lds_at(((sp - 1) * QG + qg) * 64 * MSTRIDE + lane);
      const float a = fast_exp2(o2[(16 * NDB) * 64] - mt);
      l = fmaf(o2[(16 * NDB + 1) * 64], a, l);
#pragma unroll
      for (int t = 0; t < NDB; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[t][r] = fmaf(o2[(16 * t + r) * 64], a, oacc[t][r]);
    }
  }

  // ---- normalise and store: lane holds O[qi][32t + 8g + 4*half + 0..3] in registers 4g..4g+3
  const float lt = sum_with_partner(l);
  const float inv = lt > 0.f ? __builtin_amdgcn_rcpf(lt) : 0.f;  // v_rcp_f32 (1 ulp)
  if constexpr (NSPLIT == 1) {
    // through LDS: each wave writes its 32 x D tile (16-byte chunks swizzled by row, conflict-free
    // both ways) and reads it back as whole rows, CPR lanes per row
    // speculative tiles the loop never waited for (zero or one step) have landed before LDS is reused
    if constexpr (kSpec) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // every wave is done with the K/V tiles
    float* ot = lds_at(wave * 32 * D);
#pragma unroll
    for (int t = 0; t < NDB; ++t) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 x;
        x[0] = oacc[t][4 * g + 0] * inv;
        x[1] = oacc[t][4 * g + 1] * inv;
        x[2] = oacc[t][4 * g + 2] * inv;
        x[3] = oacc[t][4 * g + 3] * inv;
        const int c = (8 * t + 2 * g + half) ^ (col & 15);
        *reinterpret_cast<f32x4*>(ot + col * D + 4 * c) = x;
      }
    }
    constexpr int RPI = 64 / CPR;  // rows per store instruction
    const int rsub = lane / CPR, cidx = lane % CPR;
    float* obase = p.o + (int64_t)b * p.so + h * D;
    // The stores are non-temporal (cache policy NT): O is not read again here, and keeping it out of
    // the L2 leaves the K/V tiles the neighbouring workgroups still read there (sweep cross-attention
    // 38.8 -> 34.9 us, self-attention 86.4 -> 85.3 us; non-temporal Q loads measured slower)
    if ((int64_t)p.Lq * p.ldo < (int64_t)1 << 29) {
      // byte offsets of every row fit in 31 bits: buffer stores from a scalar base
      const __amdgpu_buffer_rsrc_t orsrc = buffer_rsrc(obase);
#pragma unroll
      for (int j = 0; j < 32 / RPI; ++j) {
        const int row = RPI * j + rsub;
        const f32x4 x = *reinterpret_cast<const f32x4*>(ot + row * D + 4 * (cidx ^ (row & 15)));
        const int qrow = q0 + qg * 32 + row;
        if (qrow < p.Lq)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), orsrc,
                                                     (unsigned)(qrow * (int)p.ldo + 4 * cidx) * 4u, 0, 2);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 32 / RPI; ++j) {
        const int row = RPI * j + rsub;
        const f32x4 x = *reinterpret_cast<const f32x4*>(ot + row * D + 4 * (cidx ^ (row & 15)));
        const int qrow = q0 + qg * 32 + row;
        if (qrow < p.Lq) __builtin_nontemporal_store(x, reinterpret_cast<f32x4*>(obase + (int64_t)qrow * p.ldo + 4 * cidx));
      }
    }
  } else if (q_valid) {
    float* dst = p.o + (int64_t)b * p.so + (int64_t)qi * p.ldo + h * D + 4 * half;
#pragma unroll
    for (int t = 0; t < NDB; ++t) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 x;
        x[0] = oacc[t][4 * g + 0] * inv;
        x[1] = oacc[t][4 * g + 1] * inv;
        x[2] = oacc[t][4 * g + 2] * inv;
        x[3] = oacc[t][4 * g + 3] * inv;
        *reinterpret_cast<f32x4*>(dst + 32 * t + 8 * g) = x;
      }
    }
  }
}

template <int D, int NSPLIT, int BIAS, int MASK>
__global__ __launch_bounds__(256, (kMinBlocksPerCU<D, NSPLIT, BIAS, MASK>)) void flash_mfma_kernel(FlashArgs p) {
  flash_body<D, NSPLIT, BIAS, MASK>(p, NoOrder{});
}

// Folded launch of an unbiased, unmasked head-dim-64 call whose 128-query units exceed one round of
// four workgroups per CU by at most half a round: one workgroup per unit of the round, and the
// workgroups dispatched first (one per CU) each run one 64-query piece of the units left over (2-way
// key split) after their own unit, so that every CU gets the same share of the leftover work and no
// second launch waits for the first one to drain.
template <int D>
__global__ __launch_bounds__(256, 4) void flash_mfma_fold_kernel(FlashArgs p) {
  static_assert(kLdsFloats<D, 2, true> <= kLdsFloats<D, 1>, "the folded piece reuses the unit's LDS");
  float* lds = nullptr;
  flash_body<D, 1, BIAS_NONE, MASK_NONE, NoOrder, false, FoldTag<D>>(p, NoOrder{}, threadIdx.x, nullptr, &lds);
  const int piece = blockIdx.x;  // the first workgroup of each CU: pieces [0, count)
  if (piece < p.fold.count) {
    FlashArgs f = p;
    f.aux = p.fold.first;
    f.tiles = p.fold.count;
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));  // opaque: the piece's lane addressing is recomputed, not kept live
    __syncthreads();               // every wave has read its output rows back out of the LDS
    flash_body<D, 2, BIAS_NONE, MASK_NONE, NoOrder, true, FoldTag<D>>(f, NoOrder{}, tid, lds, nullptr, piece);
  }
}

template <int D, int NSPLIT, int BIAS>
__global__ __launch_bounds__(256, (kMinBlocksPerCU<D, NSPLIT, BIAS, MASK_KEY_LEN_ORDERED>)) void flash_mfma_ordered_kernel(
    FlashArgs p, FlashOrder ord) {
  flash_body<D, NSPLIT, BIAS, MASK_KEY_LEN_ORDERED>(p, ord);
}

template <int D, int NSPLIT, int BIAS, int MASK>
hipError_t launch_one(FlashArgs a, const AttnParams& p, dim3 grid, int num_cus, hipStream_t stream) {
  // stagger only launches with more than one workgroup per CU
  if constexpr (kMinBlocksPerCU<D, NSPLIT, BIAS, MASK> == 4) a.aux = (int64_t)grid.x > num_cus ? num_cus : 0;
  if constexpr (MASK == MASK_KEY_LEN_ORDERED) {
    FlashOrder ord;
    memcpy(ord.order, p.order, sizeof ord.order);
    hipLaunchKernelGGL((flash_mfma_ordered_kernel<D, NSPLIT, BIAS>), grid, dim3(256), 0, stream, a, ord);
  } else {
    hipLaunchKernelGGL((flash_mfma_kernel<D, NSPLIT, BIAS, MASK>), grid, dim3(256), 0, stream, a);
  }
  return hipGetLastError();
}

template <int D, int NSPLIT, int BIAS>
hipError_t launch_mask(const FlashArgs& a, const AttnParams& p, dim3 grid, int num_cus, hipStream_t stream) {
  switch (p.mask_mode) {
    case MASK_NONE: return launch_one<D, NSPLIT, BIAS, MASK_NONE>(a, p, grid, num_cus, stream);
    case MASK_KEY_LEN:
      if (p.order_n > 0) return launch_one<D, NSPLIT, BIAS, MASK_KEY_LEN_ORDERED>(a, p, grid, num_cus, stream);
      return launch_one<D, NSPLIT, BIAS, MASK_KEY_LEN>(a, p, grid, num_cus, stream);
    case MASK_KEY_MASK: return launch_one<D, NSPLIT, BIAS, MASK_KEY_MASK>(a, p, grid, num_cus, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int D, int NSPLIT>
hipError_t launch_split(const AttnParams& p, int num_cus, hipStream_t stream) {
  constexpr int QT = 32 * (4 / NSPLIT);
  const int q_tiles = (p.Lq + QT - 1) / QT;
  const int64_t n = (int64_t)p.B * p.H * q_tiles;
  if (n > 0x7fffffff || !flash_mfma_args_fit(p)) return hipErrorInvalidConfiguration;
  // the last units may go to the small-launch kernel: this launch covers units [0, n - tail)
  const int64_t tail = flash_mfma_tail_units(p, NSPLIT, num_cus);
  const dim3 grid((unsigned)(n - tail));
  FlashArgs a = flash_args(p, n - tail);
  if constexpr (D == 64 && NSPLIT == 1) {
    if (tail > 0 && flash_mfma_tail_kernel(p, NSPLIT, num_cus) == TAIL_FOLD) {
      int64_t first = 0;
      const int64_t count = flash_mfma_tail_groups(p, NSPLIT, num_cus, &first);
      a.aux = num_cus;  // start-up stagger period
      a.fold.first = (int32_t)first;
      a.fold.count = (int32_t)count;
      hipLaunchKernelGGL((flash_mfma_fold_kernel<64>), grid, dim3(256), 0, stream, a);
      return hipGetLastError();
    }
  }
  hipError_t e;
  switch (p.bias_mode) {
    case BIAS_NONE: e = launch_mask<D, NSPLIT, BIAS_NONE>(a, p, grid, num_cus, stream); break;
    case BIAS_DENSE: e = launch_mask<D, NSPLIT, BIAS_DENSE>(a, p, grid, num_cus, stream); break;
    case BIAS_RELPOS: e = launch_mask<D, NSPLIT, BIAS_RELPOS>(a, p, grid, num_cus, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || tail == 0) return e;
  int64_t first = 0;
  const int64_t count = flash_mfma_tail_groups(p, NSPLIT, num_cus, &first);
  if (flash_mfma_tail_kernel(p, NSPLIT, num_cus) == TAIL_SMALL) return launch_flash_small_groups(p, first, count, stream);
  // 64-query units of the 2-way key-split kernel, from unit `first` on
  FlashArgs b = flash_args(p, count);
  b.aux = (int32_t)first;
  const dim3 tgrid((unsigned)count);
  if constexpr (D == 64) {
    return launch_one<64, 2, BIAS_NONE, MASK_NONE>(b, p, tgrid, num_cus, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

FlashArgs flash_args(const AttnParams& p, int64_t tiles) {
  FlashArgs a;
  memset(&a, 0, sizeof a);
  a.q = p.q + p.q_off;
  a.k = p.k + p.k_off;
  a.v = p.v + p.v_off;
  a.o = p.o + p.o_off;
  a.sq = (int32_t)p.sq;
  a.sk = (int32_t)p.sk;
  a.sv = (int32_t)p.sv;
  a.so = (int32_t)p.so;
  a.ldq = (int32_t)p.ldq;
  a.ldk = (int32_t)p.ldk;
  a.ldv = (int32_t)p.ldv;
  a.ldo = (int32_t)p.ldo;
  a.Lq = p.Lq;
  a.Lk = p.Lk;
  a.tiles = (int32_t)tiles;
  a.H = (int16_t)p.H;
  a.scale_log2 = p.scale_log2;
  if (p.mask_mode == MASK_KEY_LEN) a.mask = p.key_len;
  if (p.mask_mode == MASK_KEY_MASK) {
    a.mask = p.key_mask;
    a.aux = (int32_t)p.smask;
  }
  a.bias = p.bias;
  if (p.bias_mode == BIAS_RELPOS) {
    a.lut = p.lut;
    a.num_buckets = (int16_t)p.num_buckets;
  } else {
    a.sbias = p.sbias;
  }
  return a;
}

bool flash_mfma_args_fit(const AttnParams& p) {
  const int64_t lim = 0x7fffffff;
  return p.ldq <= lim && p.ldk <= lim && p.ldv <= lim && p.ldo <= lim && p.sq <= lim && p.sk <= lim &&
         p.sv <= lim && p.so <= lim && p.H <= 0x7fff && (p.mask_mode != MASK_KEY_MASK || p.smask <= lim) &&
         (p.bias_mode != BIAS_RELPOS || p.num_buckets <= 0x7fff);
}

const char* flash_mfma_name(int D, int nsplit) {
  if (D == 64) return nsplit == 2 ? "flash_mfma_d64_split2" : "flash_mfma_d64";
  if (D == 128) return nsplit == 2 ? "flash_mfma_d128_split2" : "flash_mfma_d128";
  return nullptr;
}

// The key splits compiled per head dim: launch_flash_mfma instantiates every (bias, mask) pair for
// each of them.
constexpr int kSplits64[] = {1, 2};  // small D = 64 launches take flash_small_kernel instead of a 4-way split
constexpr int kSplits128[] = {1, 2};

static int compiled_split(int D, int nsplit) {
  (void)D;
  return nsplit >= 2 ? 2 : 1;
}

FlashVariant flash_mfma_variant(const AttnParams& p, int nsplit) {
  int mask = p.mask_mode;
  if (mask == MASK_KEY_LEN && p.order_n > 0) mask = MASK_KEY_LEN_ORDERED;
  return {p.D, compiled_split(p.D, nsplit), p.bias_mode, mask};
}

// The 4-per-CU kernels run a launch of more units than that in rounds. Units past the last whole
// round start only as the first workgroups finish and then run at one wave per SIMD: the batch-56
// DiT self-attention call (1008 units of 128 queries) took 69.5 us, the batch-57 one (1026 units)
// 83.9 us. The units left over go to a second launch right after this one when it runs them at one
// workgroup per CU: through flash_small (4 waves per 32 queries) when their 32-query groups fit,
// else through the 2-way key-split flash kernel (64-query units). Measured on one box: batch 57
// 83.9 -> 77.7-79.6 us, batch 60 (56 units left) 85.0 -> 77.9-79.6 us (flash_small; the split
// kernel gave 81.6-82.0), batch 64 (128 left) 83.7 -> 82.3 us (split kernel; flash_small at two
// workgroups per CU gave 86.2).
int64_t flash_mfma_tail_units(const AttnParams& p, int nsplit, int num_cus) {
  // Unmasked calls only: with key lengths, the second launch would run a call's last units through
  // other arithmetic depending on whether a host copy of the lengths (the schedule) came with it,
  // and the schedule must leave the result bit for bit unchanged.
  const bool eligible = p.D == 64 && compiled_split(p.D, nsplit) == 1 && p.bias_mode == BIAS_NONE &&
                        p.mask_mode == MASK_NONE && p.Lk > 32;
  if (!eligible) return 0;
  const int64_t tiles = (int64_t)p.B * p.H * ((p.Lq + 127) / 128);
  const int64_t slots = 4 * (int64_t)num_cus;
  if (tiles <= slots) return 0;
  const int64_t rest = tiles % slots;
  return 2 * rest <= num_cus ? rest : 0;
}

int flash_mfma_tail_kernel(const AttnParams& p, int nsplit, int num_cus) {
  const int64_t tail = flash_mfma_tail_units(p, nsplit, num_cus);
  if (tail == 0) return TAIL_NONE;
  if (4 * tail <= num_cus) return TAIL_SMALL;
  // one round plus the leftover: folded into the round's first workgroups
  const int64_t tiles = (int64_t)p.B * p.H * ((p.Lq + 127) / 128);
  return tiles < 8 * (int64_t)num_cus ? TAIL_FOLD : TAIL_SPLIT2;
}

int64_t flash_mfma_tail_groups(const AttnParams& p, int nsplit, int num_cus, int64_t* first) {
  const int64_t tail = flash_mfma_tail_units(p, nsplit, num_cus);
  *first = 0;
  if (tail == 0) return 0;
  // unit t = (b*H + h)*q_tiles + qtile holds the 32-query groups from (b*H + h)*q_groups + 4*qtile
  // on (the 64-query units from (b*H + h)*q_units + 2*qtile), and the units after it the ones after
  const int64_t q_tiles = (p.Lq + 127) / 128;
  const int64_t per = flash_mfma_tail_kernel(p, nsplit, num_cus) == TAIL_SMALL ? 4 : 2;  // sub-units per unit
  const int64_t q_sub = (p.Lq + 128 / per - 1) / (128 / per);
  const int64_t t = (int64_t)p.B * p.H * q_tiles - tail;
  *first = (t / q_tiles) * q_sub + per * (t % q_tiles);
  return (int64_t)p.B * p.H * q_sub - *first;
}

int flash_mfma_unit_queries(int nsplit) { return 32 * (4 / compiled_split(64, nsplit)); }

int flash_mfma_per_cu(const AttnParams& p, int nsplit) {
  const FlashVariant v = flash_mfma_variant(p, nsplit);
  const bool four = v.D == 64 && v.nsplit == 1 && v.bias == BIAS_NONE && v.mask != MASK_KEY_MASK;
  static_assert(kMinBlocksPerCU<64, 1, BIAS_NONE, MASK_KEY_LEN_ORDERED> == 4 &&
                    kMinBlocksPerCU<64, 2, BIAS_NONE, MASK_KEY_LEN_ORDERED> == 1 &&
                    kMinBlocksPerCU<128, 1, BIAS_NONE, MASK_KEY_LEN_ORDERED> == 1 &&
                    kMinBlocksPerCU<64, 1, BIAS_DENSE, MASK_KEY_LEN_ORDERED> == 1,
                "flash_mfma_per_cu must follow kMinBlocksPerCU");
  return four ? 4 : 1;
}

int64_t flash_mfma_workgroups(const AttnParams& p, int nsplit, int num_cus) {
  const int qt = 32 * (4 / compiled_split(p.D, nsplit));
  return (int64_t)p.B * p.H * ((p.Lq + qt - 1) / qt) - flash_mfma_tail_units(p, nsplit, num_cus);
}

int flash_mfma_variants(FlashVariant* out, int cap) {
  int n = 0;
  auto add = [&](int D, int s) {
    for (int bias = BIAS_NONE; bias <= BIAS_RELPOS; ++bias)
      for (int mask = MASK_NONE; mask <= MASK_KEY_LEN_ORDERED; ++mask) {
        if (n < cap) out[n] = {D, s, bias, mask};
        ++n;
      }
  };
  for (int s : kSplits64) add(64, s);
  for (int s : kSplits128) add(128, s);
  return n;
}

hipError_t launch_flash_mfma(const AttnParams& p, int nsplit, int num_cus, hipStream_t stream) {
  if (p.D == 64) {
    if (nsplit >= 2) return launch_split<64, 2>(p, num_cus, stream);
    return launch_split<64, 1>(p, num_cus, stream);
  }
  if (p.D == 128) {
    if (nsplit >= 2) return launch_split<128, 2>(p, num_cus, stream);
    return launch_split<128, 1>(p, num_cus, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace sa
