// Attention on fp32 MFMA for wide heads (D = 256 or 512): the SD-VAE mid-block call
// (app/models/vae.js:86: one head, D = C = 512, 1024 tokens), which the reference sends down its
// unfused GEMM -> softmax -> GEMM path (app/gpu/ops.js:119-147).
//
// Work decomposition (wide_mfma_kernel, D = 256; D = 512 runs wide_rows_kernel, described there)
//   One workgroup = NW = 4 wave64s = 32 queries x one chunk of keys. Wave w owns the head-dim
//   slice [w*D/NW, (w+1)*D/NW) of Q, K, V and O:
//   per 32-key block it computes the partial score tile S_w^T = K_w Q_w^T over its slice
//   (v_mfma_f32_32x32x2f32, the same transposed layout as the flash kernel), the NW partial tiles
//   are summed through LDS in two stages in a fixed order (so every wave derives bit-identical
//   probabilities), and each wave accumulates O_w^T += V_w^T P^T for its slice. K and V slices are
//   private to their wave: each wave streams its own slice into LDS with global_load_lds_dwordx4,
//   and only the score exchange needs workgroup barriers.
//   One head of 1024 queries gives just 32 query groups, so the keys are also split across
//   workgroups (nks chunks). Each workgroup writes its partial (O, m, l) to a workspace and a
//   second, fully parallel kernel merges the chunks of every query group with the online-softmax
//   rescale (the kernel boundary orders the two; no atomics or cross-XCD fences).
//
// LDS per workgroup: K and V slices [32 keys][D/NW] per wave (XOR-swizzled as in the flash kernel)
// plus the score exchange: 80 KiB for D = 256 (two workgroups per CU).

#include <algorithm>
#include <cstring>
#include <type_traits>
#include <utility>

#include "common.h"
#include "kernels.h"

namespace sa {

namespace {

constexpr float kRescaleSlack = 8.f;

// f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N - 1>{}), in order
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Arguments of the attention kernels, packed into 112 bytes (launches start about 0.8 us sooner
// with at most 112 bytes of explicit arguments, as measured for the flash kernels): pointers carry
// the callers' element offsets, strides are 32-bit (calls with larger strides take the generic
// kernel), and `o` is the output with one key chunk, the workspace of partial records otherwise.
struct WideArgs {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  const void* mask;   // key lengths (int32) | key mask (uint8)
  const float* bias;  // dense bias
  int32_t sq, sk, sv;  // batch strides
  union {
    int32_t so;     // one key chunk: output batch stride
    int32_t first;  // key chunks: the launch's first query group (its records start at the workspace)
  };
  int32_t ldq, ldk, ldv, ldo;  // row strides
  int32_t Lq, Lk;
  int32_t sbias, smask;  // dense-bias and key-mask batch strides
  int32_t tiles;         // workgroups of the launch (the grid size, for the XCD remap)
  int32_t chunk;         // keys per chunk
  float scale_log2;
  int16_t H, nks;        // heads, key chunks per query group
};
static_assert(sizeof(WideArgs) == 112, "wide kernel arguments must stay within 112 bytes");

// Arguments of the merge kernel: query groups [first, first + groups), whose records (nks each)
// start at ws.
struct MergeArgs {
  float* o;  // output + its element offset
  const float* ws;
  int32_t H, Lq, so, ldo, q_groups, nks, nwg, first, groups;
};

// Dense bias and key mask of one 32-key block in the 32x32 score layout, where lane (col, half)
// holds query col's keys k0 + 8(r/4) + 4 half + r%4 in score register r: four runs of 4 keys per
// lane. Loaded before the block's score products (load), folded into the base-2 scores after them
// (apply). Runs are 16-byte (bias) or 4-byte (mask) loads where the rows allow it and the run lies
// inside the keys, element loads clamped to the last key otherwise; keys at or past Lk read the
// last key's entry and are masked by the caller's key bound.
template <int BIAS, int MASK>
struct BlockTerms {
  static constexpr bool kBias = BIAS == BIAS_DENSE;
  static constexpr bool kMask = MASK == MASK_KEY_MASK;
  f32x4 bv[kBias ? 4 : 1];
  uint32_t km[kMask ? 4 : 1];

  struct Rows {
    const float* brow;     // dense bias row of the lane's query (rows past Lq re-read the last row)
    const uint8_t* kmask;  // key-mask row of the sequence
    bool bias_vec, mask_vec;
    int Lk;
  };
  __device__ static Rows rows(const WideArgs& p, int b, int h, int qi) {
    Rows r;
    r.Lk = p.Lk;
    r.brow = nullptr;
    r.kmask = nullptr;
    r.bias_vec = r.mask_vec = false;
    if constexpr (kBias) {
      r.brow = p.bias + (int64_t)b * p.sbias + ((int64_t)h * p.Lq + min(qi, p.Lq - 1)) * p.Lk;
      // 16-byte runs: the table 16-byte aligned and every row start a multiple of 4 floats (keys of a
      // run start at multiples of 4)
      r.bias_vec = (reinterpret_cast<uintptr_t>(p.bias) & 15) == 0 && (p.Lk & 3) == 0 && (p.sbias & 3) == 0;
    }
    if constexpr (kMask) {
      r.kmask = static_cast<const uint8_t*>(p.mask) + (int64_t)b * p.smask;
      r.mask_vec = (reinterpret_cast<uintptr_t>(r.kmask) & 3) == 0;
    }
    return r;
  }
  __device__ void load(const Rows& r, int k0, int half) {
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const int kk = k0 + 8 * k4 + 4 * half;  // keys kk .. kk + 3
      if constexpr (kBias) {
        if (r.bias_vec && kk + 4 <= r.Lk) {
          bv[k4] = *reinterpret_cast<const f32x4*>(r.brow + kk);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[k4][e] = r.brow[min(kk + e, r.Lk - 1)];
        }
      }
      if constexpr (kMask) {
        if (r.mask_vec && kk + 4 <= r.Lk) {
          km[k4] = *reinterpret_cast<const uint32_t*>(r.kmask + kk);
        } else {
          uint32_t w = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) w |= (uint32_t)r.kmask[min(kk + e, r.Lk - 1)] << (8 * e);
          km[k4] = w;
        }
      }
    }
  }
  // u: base-2 scores; bias in natural units, so it enters times log2(e)
  __device__ void apply(float* u) const {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if constexpr (kBias) u[r] = fmaf(bv[r >> 2][r & 3], kLog2e, u[r]);
      if constexpr (kMask) u[r] = ((km[r >> 2] >> (8 * (r & 3))) & 0xffu) != 0 ? u[r] : -INFINITY;
    }
  }
};

template <int D, int NW, int BIAS, int MASK>
__global__ __launch_bounds__(64 * NW, 1) void wide_mfma_kernel(WideArgs p) {
  constexpr int DS = D / NW;      // head dims per wave
  constexpr int QREG = DS / 2;    // Q values per lane
  constexpr int NDB = DS / 32;    // 32-dim output tiles per wave
  constexpr int CPR = DS / 4;     // 16-byte chunks per slice row
  constexpr int SLICE = 32 * DS;  // floats per K or V slice tile
  constexpr int NI = 32 * CPR / 64;  // LDS-DMA instructions per slice per wave
  constexpr int REC = 32 * D + 64;   // workspace floats per partial: O [32][D], m [32], l [32]
  static_assert(NI * 64 == 32 * CPR, "slice must split into whole wave loads");

  // K and V slices in separate arrays: the compiler then only waits for the DMA into the array a
  // read touches, so V of the next block can stay in flight while K is read
  __shared__ __attribute__((aligned(16))) float lds_k[NW * SLICE];  // [wave][SLICE]
  __shared__ __attribute__((aligned(16))) float lds_v[NW * SLICE];
  __shared__ __attribute__((aligned(16))) f32x4 lds_s[NW * 4 * 64];      // [wave][r/4][lane]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31;
  const int half = lane >> 5;

  const int q_groups = (p.Lq + 31) >> 5, nks = p.nks, chunk = p.chunk;
  int tile = xcd_remap(blockIdx.x, p.tiles);
  const int kc = tile % nks;
  tile /= nks;                       // the launch's query group
  const int slot_base = tile * nks;  // its chunks' records
  if (nks > 1) tile += p.first;
  const int g = tile % q_groups;
  tile /= q_groups;
  const int h = tile % p.H;
  const int b = tile / p.H;
  const int q0 = g * 32;
  const int qi = q0 + col;
  const bool q_valid = qi < p.Lq;

  int kv_len = p.Lk;
  if constexpr (MASK == MASK_KEY_LEN) kv_len = min(max(static_cast<const int32_t*>(p.mask)[b], 0), p.Lk);
  const int kbeg = kc * chunk;
  const int kend = min(kbeg + chunk, kv_len);
  const int nblk = kend > kbeg ? (kend - kbeg + 31) >> 5 : 0;
  using Terms = BlockTerms<BIAS, MASK>;
  constexpr bool kTerms = Terms::kBias || Terms::kMask;
  const typename Terms::Rows trows = Terms::rows(p, b, h, qi);

  float* const kt = lds_k + wave * SLICE;
  float* const vt = lds_v + wave * SLICE;
  const float* kbase = p.k + (int64_t)b * p.sk + h * D + wave * DS;
  const float* vbase = p.v + (int64_t)b * p.sv + h * D + wave * DS;

  // own K / V slice of block j; rows past the chunk's last key re-read that key
  auto issue_k = [&](int j) {
    const int key0 = kbeg + 32 * j;
#pragma unroll
    for (int n = 0; n < NI; ++n) {
      const int pc_all = n * 64 + lane;
      const int row = pc_all / CPR;
      const int pc = pc_all % CPR;
      const int key = min(key0 + row, kend - 1);
      load_to_lds16(kbase + (int64_t)key * p.ldk + 4 * (pc ^ (row & 15)), kt + n * 256);
    }
  };
  auto issue_v = [&](int j) {
    const int key0 = kbeg + 32 * j;
#pragma unroll
    for (int n = 0; n < NI; ++n) {
      const int pc_all = n * 64 + lane;
      const int row = pc_all / CPR;
      const int pc = pc_all % CPR;
      const int key = min(key0 + row, kend - 1);
      load_to_lds16(vbase + (int64_t)key * p.ldv + 4 * (pc ^ (((row >> 2) & 1) << 3)), vt + n * 256);
    }
  };

  if (nblk > 0) {
    issue_k(0);
    issue_v(0);
  }

  // Q slice in registers, pre-scaled: lane holds scale*log2(e)*Q[qi][wave*DS + half*DS/2 + s]
  float qr[QREG];
  {
    const float* src = p.q + (int64_t)b * p.sq + (int64_t)qi * p.ldq + h * D + wave * DS + half * (DS / 2);
#pragma unroll
    for (int i = 0; i < QREG / 4; ++i) {
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (q_valid) x = *reinterpret_cast<const f32x4*>(src + 4 * i);
      qr[4 * i + 0] = x[0] * p.scale_log2;
      qr[4 * i + 1] = x[1] * p.scale_log2;
      qr[4 * i + 2] = x[2] * p.scale_log2;
      qr[4 * i + 3] = x[3] * p.scale_log2;
    }
  }

  f32x16 oacc[NDB];
#pragma unroll
  for (int t = 0; t < NDB; ++t) oacc[t] = zero16();
  float m = kMaxSeed;
  float l = 0.f;
  wait_vmcnt<0>();  // Q and the first block's slices

  for (int j = 0; j < nblk; ++j) {
    const int k0 = kbeg + 32 * j;
    // own K slice of block j has landed (the last NI loads in flight are V of block j, or the Q
    // loads on the first block); wave-private, so no barrier
    wait_vmcnt<NI>();
    // the block's bias / mask terms, used after the score exchange (register loads: the compiler
    // waits for them where they are used)
    Terms terms;
    if constexpr (kTerms) terms.load(trows, k0, half);
    // ---- partial scores over this wave's head-dim slice
    f32x16 s = zero16();
    const float* krow = kt + col * DS;
    const int ksw = col & 15;
#pragma unroll
    for (int i = 0; i < QREG / 4; ++i) {
      const int c = (half * (CPR / 2) + i) ^ ksw;
      const f32x4 kv = *reinterpret_cast<const f32x4*>(krow + 4 * c);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[0], qr[4 * i + 0], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[1], qr[4 * i + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[2], qr[4 * i + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[3], qr[4 * i + 3], s, 0, 0, 0);
    }
    // ---- sum the four partial tiles (fixed order: identical probabilities in every wave)
    __syncthreads();  // everyone has read the previous exchange
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      f32x4 x;
      x[0] = s[4 * k4 + 0];
      x[1] = s[4 * k4 + 1];
      x[2] = s[4 * k4 + 2];
      x[3] = s[4 * k4 + 3];
      lds_s[(wave * 4 + k4) * 64 + lane] = x;
    }
    __syncthreads();
    // Two-stage sum: wave w adds up its 1/NW of the tile over all NW partials (in wave order) and
    // writes the sum back into partial 0 at the same places, which no other wave reads; after the
    // barrier every wave reads the summed tile from partial 0.
    {
      float* ldsf = reinterpret_cast<float*>(lds_s);
      constexpr int PER_LANE = 1024 / NW / 64;  // floats of the tile each lane sums
      const int e0 = wave * (1024 / NW) + lane * PER_LANE;
      if constexpr (PER_LANE == 4) {
        f32x4 a = *reinterpret_cast<const f32x4*>(ldsf + e0);
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) a += *reinterpret_cast<const f32x4*>(ldsf + ww * 1024 + e0);
        *reinterpret_cast<f32x4*>(ldsf + e0) = a;
      } else {
        static_assert(PER_LANE == 2, "4 or 8 waves");
        float2 a = *reinterpret_cast<const float2*>(ldsf + e0);
#pragma unroll
        for (int ww = 1; ww < NW; ++ww) {
          const float2 b = *reinterpret_cast<const float2*>(ldsf + ww * 1024 + e0);
          a.x += b.x;
          a.y += b.y;
        }
        *reinterpret_cast<float2*>(ldsf + e0) = a;
      }
    }
    __syncthreads();
    float u[16];
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const f32x4 a = lds_s[k4 * 64 + lane];
      u[4 * k4 + 0] = a[0];
      u[4 * k4 + 1] = a[1];
      u[4 * k4 + 2] = a[2];
      u[4 * k4 + 3] = a[3];
    }
    if (j + 1 < nblk) issue_k(j + 1);  // own K slice consumed: the next one streams in meanwhile
    if constexpr (kTerms) terms.apply(u);
    if (k0 + 32 > kend) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
        u[r] = key < kend ? u[r] : -INFINITY;
      }
    }
    // ---- online softmax with a lazily moved reference
    float mb = u[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mb = max_nan(mb, u[r]);
    mb = max_with_partner(mb);
    if (j == 0) {
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
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      u[r] = fast_exp2(u[r] - m);
      ps += u[r];
    }
    l += ps;
    // ---- O_w^T += V_w^T P^T (V of block j: only the next K may still be in flight)
    if (j + 1 < nblk) {
      wait_vmcnt<NI>();
    } else {
      wait_vmcnt<0>();
    }
    const float* vrow = vt + (4 * half) * DS + col;
#pragma unroll
    for (int t = 0; t < NDB; ++t) {
      const float* vcol = vrow + 32 * (t ^ half);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float vv = vcol[(8 * (r >> 2) + (r & 3)) * DS];
        oacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, u[r], oacc[t], 0, 0, 0);
      }
    }
    if (j + 1 < nblk) issue_v(j + 1);  // after this wave's last read of its V slice
  }

  const float lt = sum_with_partner(l);
  if (nks == 1) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    if (q_valid) {
      float* dst = p.o + (int64_t)b * p.so + (int64_t)qi * p.ldo + h * D + wave * DS + 4 * half;
#pragma unroll
      for (int t = 0; t < NDB; ++t)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          f32x4 x;
          x[0] = oacc[t][4 * g4 + 0] * inv;
          x[1] = oacc[t][4 * g4 + 1] * inv;
          x[2] = oacc[t][4 * g4 + 2] * inv;
          x[3] = oacc[t][4 * g4 + 3] * inv;
          *reinterpret_cast<f32x4*>(dst + 32 * t + 8 * g4) = x;
        }
    }
    return;
  }

  // ---- publish this chunk's partial: O (unnormalised, relative to m), m, l; the merge kernel
  // combines the chunks of each query group
  float* rec = p.o + (int64_t)(slot_base + kc) * REC;
  float* orow = rec + col * D + wave * DS + 4 * half;
#pragma unroll
  for (int t = 0; t < NDB; ++t)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      f32x4 x;
      x[0] = oacc[t][4 * g4 + 0];
      x[1] = oacc[t][4 * g4 + 1];
      x[2] = oacc[t][4 * g4 + 2];
      x[3] = oacc[t][4 * g4 + 3];
      *reinterpret_cast<f32x4*>(orow + 32 * t + 8 * g4) = x;
    }
  if (wave == 0 && half == 0) {
    rec[32 * D + col] = m;
    rec[32 * D + 32 + col] = lt;
  }
}

// D = 512: one workgroup = 4 waves = 32 queries x one chunk of keys, taken in rounds of four
// 32-key blocks. In a round wave w computes the whole score tile of block w over all 512 head
// dims (256 MFMAs in two independent chains: K rows straight from memory into registers, Q^T from
// a copy of the query tile in LDS), the four block maxima and row sums meet in LDS (one reference
// m per query for the round, so the probabilities need no lazy rescale inside it), each wave
// publishes its probabilities, and wave w then accumulates O^T for its quarter of the head dims
// over all four blocks (V rows straight into registers, prefetched a block ahead, with head dim
// 4i + t of the quarter on row i of output tile t, so one 16-byte load feeds the four tiles).
// Each probability is computed once per round, where the head-dim-split kernel above summed
// partial score tiles through LDS and took the softmax in every wave for every block; one wave
// per SIMD, its loads software-pipelined. Writes the same partial records as wide_mfma_kernel
// (merged by wide_merge_kernel), staged through LDS into whole-row stores.
template <int BIAS, int MASK>
__global__ __launch_bounds__(256, 1) void wide_rows_kernel(WideArgs p) {
  constexpr int D = 512;
  constexpr int NG = D / 8;          // groups of 8 head dims (4 MFMAs) per score tile
  constexpr int DS = D / 4;          // output head dims per wave
  constexpr int REC = 32 * D + 64;   // workspace floats per partial: O [32][D], m [32], l [32]
  constexpr int KR = 8;              // K groups in flight ahead of the MFMAs (16 measured no faster)
  constexpr int NQ = 32 * D / 4 / 256;  // 16-byte Q chunks per thread

  __shared__ __attribute__((aligned(16))) float lds_q[32 * D];      // [quarter][query][128], then the output
  __shared__ __attribute__((aligned(16))) f32x4 lds_p[4 * 4 * 64];  // [block][r/4][lane]
  __shared__ float lds_m[4 * 32];                                   // [block][query]
  __shared__ float lds_l[4 * 32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31;
  const int half = lane >> 5;

  const int q_groups = (p.Lq + 31) >> 5, nks = p.nks, chunk = p.chunk;
  int tile = xcd_remap(blockIdx.x, p.tiles);
  const int kc = tile % nks;
  tile /= nks;                       // the launch's query group
  const int slot_base = tile * nks;  // its chunks' records
  if (nks > 1) tile += p.first;
  const int g = tile % q_groups;
  tile /= q_groups;
  const int h = tile % p.H;
  const int b = tile / p.H;
  const int q0 = g * 32;

  int kv_len = p.Lk;
  if constexpr (MASK == MASK_KEY_LEN) kv_len = min(max(static_cast<const int32_t*>(p.mask)[b], 0), p.Lk);
  const int kbeg = kc * chunk;
  const int kend = min(kbeg + chunk, kv_len);
  const int rounds = kend > kbeg ? (kend - kbeg + 127) >> 7 : 0;
  using Terms = BlockTerms<BIAS, MASK>;
  constexpr bool kTerms = Terms::kBias || Terms::kMask;
  const typename Terms::Rows trows = Terms::rows(p, b, h, q0 + col);

  const float* kbase = p.k + (int64_t)b * p.sk + h * D;
  const float* vbase = p.v + (int64_t)b * p.sv + h * D + wave * DS;

  // ---- Q tile (rows past Lq re-read the last row) into registers, then into LDS a quarter of 128
  // head dims at a time as the score products reach it: [quarter][query][32 chunks of 16 bytes],
  // chunk c of row r at c ^ (r & 15). Thread t holds physical chunks n*256 + t (n = 0..15), so
  // quarter k is its registers 4k..4k+3. (Copies straight into LDS would make the compiler wait
  // for all of them, and the K loads behind them, before the first LDS read.)
  f32x4 qst[NQ];
  {
    const float* qbase = p.q + (int64_t)b * p.sq + h * D;
#pragma unroll
    for (int n = 0; n < NQ; ++n) {
      const int pc = (n & 3) * 256 + tid;  // physical chunk within quarter n / 4
      const int row = pc >> 5;
      const int c = 32 * (n >> 2) + ((pc & 31) ^ (row & 15));
      qst[n] = *reinterpret_cast<const f32x4*>(qbase + (int64_t)min(q0 + row, p.Lq - 1) * p.ldq + 4 * c);
    }
  }

  // V rows of one block for this wave's head dims: register r holds V[key][4*col .. 4*col + 3] of
  // key 8(r/4) + 4*half + r%4 of the block. The buffer ends after the chunk's last valid key, so
  // rows past it read as zeros (their probabilities are zero) and no load needs a branch: a
  // conditional load is sunk by the compiler to its first use, which would undo the prefetch.
  unsigned vrow_off[16];  // byte offset of register r's row and columns from the block's first row
#pragma unroll
  for (int r = 0; r < 16; ++r) vrow_off[r] = 4u * (unsigned)((4 * half + 8 * (r >> 2) + (r & 3)) * (int)p.ldv + 4 * col);
  auto load_v = [&](int kb0, f32x4* dst) {
    // (in a scalar register: a clamp the compiler computes on the vector unit would make the
    // descriptor look divergent and every load a waterfall loop)
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(32, kend - kb0)));
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(vbase + (int64_t)kb0 * p.ldv), 0, rows * (int)p.ldv * 4, 0x00020000);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      dst[r] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, vrow_off[r], 0, 0));
  };

  f32x16 oacc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) oacc[t] = zero16();
  float m = kMaxSeed;
  float l = 0.f;
  // the swizzled Q chunk 2i + half of this lane's query (quarter i / 16)
  const float* qrow = lds_q + col * 128;

  for (int rd = 0; rd < rounds; ++rd) {
    const int rb0 = kbeg + 128 * rd;  // first key of the round
    if (rd > 0) __syncthreads();      // every wave is done with the previous round's exchange
    const int kb0 = rb0 + 32 * wave;  // this wave's score block
    const bool has_keys = kb0 < kend;  // false for the missing blocks of a short last round
    // K rows of the block (clamped past the chunk's last key), 16 bytes per group of 8 dims
    const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(kbase + (int64_t)kb0 * p.ldk);
    const unsigned koff = 4u * (unsigned)((min(kb0 + col, kend - 1) - kb0) * (int)p.ldk + 4 * half);
    auto load_k = [&](int i) {
      return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff + 32u * i, 0, 0));
    };
    f32x4 kring[KR];
    Terms terms;  // the block's bias / mask terms, used after its score products
    if (has_keys) {
      if constexpr (kTerms) terms.load(trows, kb0, half);
#pragma unroll
      for (int i = 0; i < KR; ++i) kring[i] = load_k(i);
    }
    // round 0 publishes the Q quarters as the products reach them
    auto q_quarter = [&](auto k) {
      constexpr int kq = decltype(k)::value;
      if (rd == 0) {
#pragma unroll
        for (int n = 4 * kq; n < 4 * kq + 4; ++n) *reinterpret_cast<f32x4*>(lds_q + n * 1024 + 4 * tid) = qst[n];
        __syncthreads();
      }
    };
    q_quarter(std::integral_constant<int, 0>{});
    f32x4 vbuf[2][16];  // V of the round's blocks, double-buffered
    float u[16];
    if (has_keys) {
      f32x16 sa = zero16(), sb = zero16();
      auto read_q = [&](int i) {
        return *reinterpret_cast<const f32x4*>(qrow + (i >> 4) * 4096 + 4 * ((2 * (i & 15) + half) ^ (col & 15)));
      };
      // Groups in pairs, group i into sa and i + 1 into sb (the compiler orders the products; pinning
      // them to alternate between the chains measured the same). The Q operands of the next pair
      // are read during this one.
      f32x4 qn0 = read_q(0), qn1 = read_q(1);
      static_for<NG / 2>([&](auto I) {
        constexpr int i = 2 * decltype(I)::value;
        const f32x4 k0v = kring[i % KR], k1v = kring[(i + 1) % KR];
        const f32x4 q0v = qn0, q1v = qn1;
        if constexpr (i + KR < NG) {
          kring[i % KR] = load_k(i + KR);
          kring[(i + 1) % KR] = load_k(i + 1 + KR);
        }
        if constexpr (i == NG - 16) load_v(rb0, vbuf[0]);  // the round's first V block streams in under the last products
        if constexpr (i + 2 < NG) {
          if constexpr ((i + 2) % 16 == 0) q_quarter(std::integral_constant<int, (i + 2) / 16>{});
          qn0 = read_q(i + 2);
          qn1 = read_q(i + 3);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sa = __builtin_amdgcn_mfma_f32_32x32x2f32(k0v[j], q0v[j], sa, 0, 0, 0);
          sb = __builtin_amdgcn_mfma_f32_32x32x2f32(k1v[j], q1v[j], sb, 0, 0, 0);
        }
        // keeps each load where it is issued: left free, the scheduler sinks the ring's loads to
        // just before their use, one group ahead of the products
        __builtin_amdgcn_sched_barrier(0);
      });
#pragma unroll
      for (int r = 0; r < 16; ++r) u[r] = (sa[r] + sb[r]) * p.scale_log2;
      if constexpr (kTerms) terms.apply(u);
      if (kb0 + 32 > kend) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb0 + 8 * (r >> 2) + 4 * half + (r & 3);
          u[r] = key < kend ? u[r] : -INFINITY;
        }
      }
    } else {
      // the score-less wave still takes part in round 0's quarter barriers
      q_quarter(std::integral_constant<int, 1>{});
      q_quarter(std::integral_constant<int, 2>{});
      q_quarter(std::integral_constant<int, 3>{});
      load_v(rb0, vbuf[0]);
#pragma unroll
      for (int r = 0; r < 16; ++r) u[r] = -INFINITY;
    }
    // ---- one reference per query for the round: the maximum over the four blocks
    float mb = u[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mb = max_nan(mb, u[r]);
    mb = max_with_partner(mb);
    if (half == 0) lds_m[wave * 32 + col] = mb;
    __syncthreads();
    float m_new = max_nan(m, lds_m[col]);
    m_new = max_nan(m_new, lds_m[32 + col]);
    m_new = max_nan(m_new, lds_m[64 + col]);
    m_new = max_nan(m_new, lds_m[96 + col]);
    if (rd > 0) {
      const float alpha = fast_exp2(m - m_new);
      l *= alpha;
#pragma unroll
      for (int t = 0; t < 4; ++t) oacc[t] *= alpha;
    }
    m = m_new;
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      u[r] = fast_exp2(u[r] - m);
      ps += u[r];
    }
    ps = sum_with_partner(ps);
    if (half == 0) lds_l[wave * 32 + col] = ps;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      f32x4 x;
      x[0] = u[4 * k4 + 0];
      x[1] = u[4 * k4 + 1];
      x[2] = u[4 * k4 + 2];
      x[3] = u[4 * k4 + 3];
      lds_p[(wave * 4 + k4) * 64 + lane] = x;
    }
    __syncthreads();
    l += lds_l[col] + lds_l[32 + col] + lds_l[64 + col] + lds_l[96 + col];
    // ---- O^T += V^T P^T over the round's blocks, this wave's 128 head dims; the next block's V
    // is requested before this block's products (a zero-row buffer past the keys: no access)
    float pr[4][16];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) {
        const f32x4 x = lds_p[(j * 4 + k4) * 64 + lane];
        pr[j][4 * k4 + 0] = x[0];
        pr[j][4 * k4 + 1] = x[1];
        pr[j][4 * k4 + 2] = x[2];
        pr[j][4 * k4 + 3] = x[3];
      }
    static_for<4>([&](auto J) {
      constexpr int j = decltype(J)::value;
      if constexpr (j + 1 < 4) load_v(rb0 + 32 * (j + 1), vbuf[(j + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      if (rb0 + 32 * j < kend) {  // wave-uniform: blocks past the chunk's keys hold no probabilities
#pragma unroll
        for (int r = 0; r < 16; ++r) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            oacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vbuf[j & 1][r][t], pr[j][r], oacc[t], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // ---- output: O^T tile t, register r holds head dim wave*128 + 4i + t of query col, with
  // i = 8(r/4) + 4*half + r%4, so the four tiles' register r are four consecutive head dims.
  // The wave stages its 32 x 128 slice in LDS (the Q tile is dead: every wave has passed the
  // last exchange, after its score products), 16-byte chunk i of query q at i ^ q, and stores
  // it back as 512-byte row pieces, two rows per instruction, instead of 16 bytes of 32 rows.
  const float inv = nks == 1 ? (l > 0.f ? 1.f / l : 0.f) : 1.f;
  float* stage = lds_q + wave * 32 * DS;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = 8 * (r >> 2) + 4 * half + (r & 3);
    f32x4 x;
    x[0] = oacc[0][r] * inv;
    x[1] = oacc[1][r] * inv;
    x[2] = oacc[2][r] * inv;
    x[3] = oacc[3][r] * inv;
    *reinterpret_cast<f32x4*>(stage + col * DS + 4 * (i ^ col)) = x;
  }
  float* dst;
  int64_t ld;
  if (nks == 1) {
    dst = p.o + (int64_t)b * p.so + (int64_t)q0 * p.ldo + h * D + wave * DS;
    ld = p.ldo;
  } else {
    float* rec = p.o + (int64_t)(slot_base + kc) * REC;
    dst = rec + wave * DS;
    ld = D;
    if (wave == 0 && half == 0) {
      rec[32 * D + col] = m;
      rec[32 * D + 32 + col] = l;
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int row = 2 * j + half;  // query q0 + row; lane col holds chunk col of it
    const f32x4 x = *reinterpret_cast<const f32x4*>(stage + row * DS + 4 * (col ^ row));
    if (nks > 1 || q0 + row < p.Lq) *reinterpret_cast<f32x4*>(dst + (int64_t)row * ld + 4 * col) = x;
  }
}

// Combines the nks partial records of every query group: one thread per (query, 4 dims),
// O = sum_c O_c exp2(m_c - m) / sum_c l_c exp2(m_c - m) with m = max_c m_c (0 if every l_c is 0).
template <int D>
__global__ __launch_bounds__(256) void wide_merge_kernel(MergeArgs p) {
  const int q_groups = p.q_groups, nks = p.nks;
  constexpr int REC = 32 * D + 64;
  constexpr int C4 = D / 4;
  // the same XCD remap as the attention kernel, whose workgroups wrote a query group's records from
  // one XCD: consecutive merge workgroups (one query group's queries) run there and find the records
  // in that XCD's L2
  const int64_t idx = (int64_t)xcd_remap(blockIdx.x, p.nwg) * 256 + threadIdx.x;
  const int64_t total = (int64_t)p.groups * 32 * C4;
  if (idx >= total) return;
  const int d4 = (int)(idx % C4);
  int64_t r = idx / C4;
  const int qq = (int)(r % 32);
  r /= 32;  // the launch's query group
  const float* recs = p.ws + r * nks * REC;
  r += p.first;  // (b*H + h)*q_groups + g
  const int g = (int)(r % q_groups);
  const int bh = (int)(r / q_groups);
  const int h = bh % p.H;
  const int b = bh / p.H;
  const int qi = g * 32 + qq;
  if (qi >= p.Lq) return;
  // One pass over the chunks in groups of 8 whose loads are all issued before any is used
  // (indexes clamped to the last chunk, surplus entries of a group skipped), with a running
  // maximum: the sums so far are rescaled when a group raises it. A query costs ceil(nks/8) load
  // round trips (one for the VAE call's 8 chunks); with a single group the rescale only touches
  // the zero-initialized sums, so the result equals the two-pass (maximum first) merge bit for bit.
  float mt = kMaxSeed;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
  for (int c0 = 0; c0 < nks; c0 += 8) {
    float mv[8], lv[8];
    f32x4 xv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float* rc = recs + (int64_t)min(c0 + u, nks - 1) * REC;
      mv[u] = rc[32 * D + qq];
      lv[u] = rc[32 * D + 32 + qq];
      xv[u] = *reinterpret_cast<const f32x4*>(rc + qq * D + 4 * d4);
    }
    float mg = mt;
#pragma unroll
    for (int u = 0; u < 8; ++u) mg = fmaxf(mg, mv[u]);  // a repeated last chunk changes nothing
    const float sc = fast_exp2(mt - mg);
    lsum *= sc;
    acc[0] *= sc;
    acc[1] *= sc;
    acc[2] *= sc;
    acc[3] *= sc;
    mt = mg;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (c0 + u >= nks) break;
      const float a = fast_exp2(mv[u] - mt);
      lsum = fmaf(lv[u], a, lsum);
      acc[0] = fmaf(xv[u][0], a, acc[0]);
      acc[1] = fmaf(xv[u][1], a, acc[1]);
      acc[2] = fmaf(xv[u][2], a, acc[2]);
      acc[3] = fmaf(xv[u][3], a, acc[3]);
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  f32x4 y;
  y[0] = acc[0] * inv;
  y[1] = acc[1] * inv;
  y[2] = acc[2] * inv;
  y[3] = acc[3] * inv;
  *reinterpret_cast<f32x4*>(p.o + (int64_t)b * p.so + (int64_t)qi * p.ldo + h * D + 4 * d4) = y;
}

// Waves per workgroup of the head-dim-split kernel (D = 256): each owns D / 4 head dims, 80 KiB of
// LDS, two workgroups per CU. (At D = 512 it ran 8 waves, two per SIMD, in 160 KiB: VAE call
// 34.9 us against 29.9 for wide_rows_kernel.)
template <int D>
constexpr int kWideWaves = 4;

template <int D, int BIAS, int MASK>
void launch_main(const WideArgs& a, dim3 grid, hipStream_t stream) {
  if constexpr (D == 512)
    hipLaunchKernelGGL((wide_rows_kernel<BIAS, MASK>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((wide_mfma_kernel<D, kWideWaves<D>, BIAS, MASK>), grid, dim3(64 * kWideWaves<D>), 0, stream, a);
}

template <int D, int BIAS>
hipError_t launch_mask(const WideArgs& a, int mask_mode, dim3 grid, hipStream_t stream) {
  switch (mask_mode) {
    case MASK_NONE: launch_main<D, BIAS, MASK_NONE>(a, grid, stream); break;
    case MASK_KEY_LEN: launch_main<D, BIAS, MASK_KEY_LEN>(a, grid, stream); break;
    case MASK_KEY_MASK: launch_main<D, BIAS, MASK_KEY_MASK>(a, grid, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

bool fits32(int64_t x) { return x >= 0 && x <= 0x7fffffff; }

template <int D>
hipError_t launch_d(const AttnParams& p, const WidePlan& plan, float* ws, hipStream_t stream) {
  const int64_t groups = (int64_t)p.B * p.H * plan.q_groups;
  const int64_t whole = plan.nks > 1 ? plan.whole : groups;  // leading groups, unsplit
  const int64_t split = groups - whole;                      // the rest, in nks chunks each
  if (whole > 0x7fffffff || split * plan.nks > 0x7fffffff) return hipErrorInvalidConfiguration;
  WideArgs a;
  memset(&a, 0, sizeof a);
  a.q = p.q + p.q_off;
  a.k = p.k + p.k_off;
  a.v = p.v + p.v_off;
  a.mask = p.mask_mode == MASK_KEY_LEN ? static_cast<const void*>(p.key_len) : static_cast<const void*>(p.key_mask);
  a.bias = p.bias;
  a.sq = (int32_t)p.sq;
  a.sk = (int32_t)p.sk;
  a.sv = (int32_t)p.sv;
  a.ldq = (int32_t)p.ldq;
  a.ldk = (int32_t)p.ldk;
  a.ldv = (int32_t)p.ldv;
  a.ldo = (int32_t)p.ldo;
  a.Lq = p.Lq;
  a.Lk = p.Lk;
  a.sbias = (int32_t)p.sbias;
  a.smask = (int32_t)p.smask;
  a.scale_log2 = p.scale_log2;
  a.H = (int16_t)p.H;
  auto attend = [&](int64_t n) -> hipError_t {
    a.tiles = (int32_t)n;
    const dim3 grid((unsigned)n);
    if (p.bias_mode == BIAS_NONE) return launch_mask<D, BIAS_NONE>(a, p.mask_mode, grid, stream);
    if (p.bias_mode == BIAS_DENSE) return launch_mask<D, BIAS_DENSE>(a, p.mask_mode, grid, stream);
    return hipErrorInvalidValue;
  };
  if (whole > 0) {
    a.o = p.o + p.o_off;
    a.so = (int32_t)p.so;
    a.nks = 1;
    a.chunk = plan.whole_chunk;
    const hipError_t e = attend(whole);
    if (e != hipSuccess || split == 0) return e;
  }
  a.o = ws;
  a.first = (int32_t)whole;
  a.nks = (int16_t)plan.nks;
  a.chunk = plan.chunk;
  const hipError_t e = attend(split * plan.nks);
  if (e != hipSuccess) return e;
  const int64_t threads = split * 32 * (D / 4);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  MergeArgs m;
  m.o = p.o + p.o_off;
  m.ws = ws;
  m.H = p.H;
  m.Lq = p.Lq;
  m.so = (int32_t)p.so;
  m.ldo = (int32_t)p.ldo;
  m.q_groups = plan.q_groups;
  m.nks = plan.nks;
  m.nwg = (int32_t)blocks;
  m.first = (int32_t)whole;
  m.groups = (int32_t)split;
  hipLaunchKernelGGL((wide_merge_kernel<D>), dim3((unsigned)blocks), dim3(256), 0, stream, m);
  return hipGetLastError();
}

}  // namespace

bool wide_mfma_supported(const AttnParams& p) {
  // 32-bit strides and at most 32767 heads (the packed arguments); other calls take the generic kernel
  const bool fit = fits32(p.sq) && fits32(p.sk) && fits32(p.sv) && fits32(p.so) && fits32(p.ldq) && fits32(p.ldk) &&
                   fits32(p.ldv) && fits32(p.ldo) && fits32(p.sbias) && fits32(p.smask) && p.H <= 32767;
  return fit && (p.D == 256 || p.D == 512) && (p.bias_mode == BIAS_NONE || p.bias_mode == BIAS_DENSE) &&
         (p.mask_mode == MASK_NONE || p.mask_mode == MASK_KEY_LEN || p.mask_mode == MASK_KEY_MASK);
}

int wide_mfma_variants(FlashVariant* out, int cap) {
  int n = 0;
  for (int D = 256; D <= 512; D *= 2)
    for (int bias = BIAS_NONE; bias <= BIAS_DENSE; ++bias)
      for (int mask = MASK_NONE; mask <= MASK_KEY_MASK; ++mask) {
        if (n < cap) out[n] = {D, 1, bias, mask};
        ++n;
      }
  return n;
}

// Key chunks per query group: of the plans whose merge records fit kWideMaxRecordBytes, the one
// with the shortest modelled makespan (ties: the first found, fewer chunks). A workgroup costs the
// key blocks of its chunk plus about two blocks of start-up and stores; workgroups run in rounds of
// one per CU (D = 512: one wave per SIMD at 400 registers) or two (D = 256: 80 KiB of LDS); a split
// adds the merge, about half a block plus one block per 22 MB of records. One block is 32 queries x
// 32 keys over all head dims (about 4.4 us of a CU at D = 512). The plans: every group in the same
// number of chunks (up to kWideMaxChunks), or, when the groups fill whole rounds and a few more,
// the whole rounds unsplit and only the groups past them in chunks, in a second launch. For one
// head of 1024 tokens this is 8 chunks of 4 blocks (256 workgroups, one round); for 2304 tokens 3
// chunks of 24 blocks (216 workgroups) rather than 4 of 20 blocks, whose 288 workgroups would take
// two rounds; for 9216 tokens (288 groups) 256 groups unsplit, then 32 groups in 8 chunks.
WidePlan wide_mfma_plan(const AttnParams& p, int num_cus) {
  WidePlan plan;
  plan.q_groups = (p.Lq + 31) / 32;
  const int64_t base = (int64_t)p.B * p.H * plan.q_groups;
  const int64_t slots = (int64_t)num_cus * (p.D == 512 ? 1 : 2);
  const int nblk = (p.Lk + 31) / 32;
  // D = 512 takes keys in rounds of four blocks (wide_rows_kernel): chunks of whole rounds
  const int unit = p.D == 512 ? 4 : 1;
  const int64_t rec_bytes = (int64_t)(32 * p.D + 64) * (int64_t)sizeof(float);
  auto rounds = [&](int64_t wgs) { return (double)((wgs + slots - 1) / slots); };
  auto merge = [&](int64_t wgs) { return 0.5 + (double)(wgs * rec_bytes) / 22e6; };
  auto fits = [&](int64_t wgs) { return wgs * rec_bytes <= kWideMaxRecordBytes; };
  const int full = (nblk + unit - 1) / unit * unit;  // blocks of an unsplit group
  double best = rounds(base) * (full + 2);
  plan.nks = 1;
  plan.chunk = plan.whole_chunk = 32 * full;
  plan.whole = 0;
  // split groups: `split` of them (the last ones) in n chunks of bpc blocks, after `whole` unsplit
  auto consider = [&](int64_t whole, int64_t split) {
    for (int want = 2; want <= kWideMaxChunks; ++want) {
      const int bpc = (nblk + want * unit - 1) / (want * unit) * unit;
      const int n = (nblk + bpc - 1) / bpc;  // chunks that hold at least one key
      if (n == 1 || !fits(split * n)) continue;
      const double cost = (whole > 0 ? rounds(whole) * (full + 2) : 0.0) + rounds(split * n) * (bpc + 2) +
                          merge(split * n);
      if (cost < best) {
        best = cost;
        plan.nks = n;
        plan.chunk = 32 * bpc;
        plan.whole = whole;
      }
    }
  };
  consider(0, base);
  if (base > slots && base % slots != 0 && base <= 0x7fffffff) consider(base / slots * slots, base % slots);
  plan.ws_floats = plan.nks > 1 ? (base - plan.whole) * plan.nks * (int64_t)(32 * p.D + 64) : 0;
  return plan;
}

const char* wide_mfma_name(int D) { return D == 512 ? "wide_mfma_d512" : "wide_mfma_d256"; }

hipError_t launch_wide_mfma(const AttnParams& p, const WidePlan& plan, float* ws, hipStream_t stream) {
  if (p.D == 512) return launch_d<512>(p, plan, ws, stream);
  if (p.D == 256) return launch_d<256>(p, plan, ws, stream);
  return hipErrorInvalidValue;
}

}  // namespace sa
