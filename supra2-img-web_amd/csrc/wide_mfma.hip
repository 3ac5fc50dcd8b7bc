// Attention on fp32 MFMA for wide heads (D = 256 or 512): the SD-VAE mid-block call
// (app/models/vae.js:86: one head, D = C = 512, 1024 tokens), which the reference sends down its
// unfused GEMM -> softmax -> GEMM path (app/gpu/ops.js:119-147).
//
// Work decomposition
//   One workgroup = NW wave64s = 32 queries x one chunk of keys (NW = 8 for D = 512: two waves per
//   SIMD; 4 for D = 256). Wave w owns the head-dim slice [w*D/NW, (w+1)*D/NW) of Q, K, V and O:
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
// plus the score exchange: 160 KiB for D = 512 (one workgroup per CU), 80 KiB for D = 256.

#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace sa {

namespace {

constexpr float kRescaleSlack = 8.f;


__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

template <int D, int NW, int MASK>
__global__ __launch_bounds__(64 * NW, 1) void wide_mfma_kernel(AttnParams p, int q_groups, int nks, int chunk, float* ws) {
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

  int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int kc = tile % nks;
  tile /= nks;
  const int g = tile % q_groups;
  tile /= q_groups;
  const int h = tile % p.H;
  const int b = tile / p.H;
  const int q0 = g * 32;
  const int qi = q0 + col;
  const bool q_valid = qi < p.Lq;
  const int slot_base = ((b * p.H + h) * q_groups + g) * nks;

  int kv_len = p.Lk;
  if constexpr (MASK == MASK_KEY_LEN) kv_len = min(max(p.key_len[b], 0), p.Lk);
  const int kbeg = kc * chunk;
  const int kend = min(kbeg + chunk, kv_len);
  const int nblk = kend > kbeg ? (kend - kbeg + 31) >> 5 : 0;

  float* const kt = lds_k + wave * SLICE;
  float* const vt = lds_v + wave * SLICE;
  const float* kbase = p.k + p.k_off + (int64_t)b * p.sk + h * D + wave * DS;
  const float* vbase = p.v + p.v_off + (int64_t)b * p.sv + h * D + wave * DS;

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
    const float* src = p.q + p.q_off + (int64_t)b * p.sq + (int64_t)qi * p.ldq + h * D + wave * DS + half * (DS / 2);
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
      float* dst = p.o + p.o_off + (int64_t)b * p.so + (int64_t)qi * p.ldo + h * D + wave * DS + 4 * half;
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
  float* rec = ws + (int64_t)(slot_base + kc) * REC;
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

// Combines the nks partial records of every query group: one thread per (query, 4 dims),
// O = sum_c O_c exp2(m_c - m) / sum_c l_c exp2(m_c - m) with m = max_c m_c (0 if every l_c is 0).
template <int D>
__global__ __launch_bounds__(256) void wide_merge_kernel(AttnParams p, int q_groups, int nks, const float* ws) {
  constexpr int REC = 32 * D + 64;
  constexpr int C4 = D / 4;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.H * q_groups * 32 * C4;
  if (idx >= total) return;
  const int d4 = (int)(idx % C4);
  int64_t r = idx / C4;
  const int qq = (int)(r % 32);
  r /= 32;  // (b*H + h)*q_groups + g
  const int g = (int)(r % q_groups);
  const int bh = (int)(r / q_groups);
  const int h = bh % p.H;
  const int b = bh / p.H;
  const int qi = g * 32 + qq;
  if (qi >= p.Lq) return;
  const float* recs = ws + r * nks * REC;
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
  *reinterpret_cast<f32x4*>(p.o + p.o_off + (int64_t)b * p.so + (int64_t)qi * p.ldo + h * D + 4 * d4) = y;
}

// Waves per workgroup: each owns D / NW head dims. D = 512 runs 8 waves (two per SIMD, 160 KiB of
// LDS), D = 256 runs 4 (80 KiB, two workgroups per CU).
template <int D>
constexpr int kWideWaves = D == 512 ? 8 : 4;

template <int D>
hipError_t launch_d(const AttnParams& p, const WidePlan& plan, float* ws, hipStream_t stream) {
  constexpr int NW = kWideWaves<D>;
  const int64_t n = (int64_t)p.B * p.H * plan.q_groups * plan.nks;
  if (n > 0x7fffffff) return hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)n), block(64 * NW);
  if (p.mask_mode == MASK_KEY_LEN)
    hipLaunchKernelGGL((wide_mfma_kernel<D, NW, MASK_KEY_LEN>), grid, block, 0, stream, p, plan.q_groups, plan.nks,
                       plan.chunk, ws);
  else
    hipLaunchKernelGGL((wide_mfma_kernel<D, NW, MASK_NONE>), grid, block, 0, stream, p, plan.q_groups, plan.nks,
                       plan.chunk, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || plan.nks == 1) return e;
  const int64_t threads = (int64_t)p.B * p.H * plan.q_groups * 32 * (D / 4);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((wide_merge_kernel<D>), dim3((unsigned)blocks), dim3(256), 0, stream, p, plan.q_groups, plan.nks, ws);
  return hipGetLastError();
}

}  // namespace

bool wide_mfma_supported(const AttnParams& p) {
  return (p.D == 256 || p.D == 512) && p.bias_mode == BIAS_NONE &&
         (p.mask_mode == MASK_NONE || p.mask_mode == MASK_KEY_LEN);
}

WidePlan wide_mfma_plan(const AttnParams& p, int num_cus) {
  WidePlan plan;
  plan.q_groups = (p.Lq + 31) / 32;
  const int64_t base = (int64_t)p.B * p.H * plan.q_groups;
  const int per_cu = p.D == 512 ? 1 : 2;  // LDS: 144 KiB (D=512) or 80 KiB (D=256) per workgroup
  const int64_t target = (int64_t)num_cus * per_cu;
  const int nblk = (p.Lk + 31) / 32;
  int nks = 1;
  if (base < target) nks = (int)((target + base - 1) / base);
  nks = std::max(1, std::min({nks, nblk, kWideMaxChunks}));
  const int blocks_per_chunk = (nblk + nks - 1) / nks;
  plan.chunk = 32 * blocks_per_chunk;
  plan.nks = (p.Lk + plan.chunk - 1) / plan.chunk;  // chunks that hold at least one key
  plan.ws_floats = plan.nks > 1 ? base * plan.nks * (int64_t)(32 * p.D + 64) : 0;
  return plan;
}

const char* wide_mfma_name(int D) { return D == 512 ? "wide_mfma_d512" : "wide_mfma_d256"; }

hipError_t launch_wide_mfma(const AttnParams& p, const WidePlan& plan, float* ws, hipStream_t stream) {
  if (p.D == 512) return launch_d<512>(p, plan, ws, stream);
  if (p.D == 256) return launch_d<256>(p, plan, ws, stream);
  return hipErrorInvalidValue;
}

}  // namespace sa
