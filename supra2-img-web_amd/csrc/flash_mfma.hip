// Flash attention on fp32 MFMA for gfx950 (CDNA4), head dim 64 or 128.
//
// Replaces the fused WGSL kernel of app/gpu/kernels.js:164-316 (online softmax over key blocks,
// keys >= Lk masked) and, for the biased/masked calls that app/gpu/ops.js:119-147 sends down the
// unfused GEMM -> softmax(+bias) -> GEMM path, fuses the bias and the key mask into the same pass.
//
// Work decomposition
//   A workgroup is 4 wave64s. Each wave owns 32 queries of one (sequence b, head h). With
//   NSPLIT = 1 the 4 waves cover 128 consecutive queries and share every 32-key K/V tile staged
//   in LDS. With NSPLIT = 2 or 4 the waves split the key blocks instead (4/NSPLIT query groups of
//   32, each seeing every NSPLIT-th key block) and their partial softmax states are merged in LDS
//   at the end: small launches (the B=2 DiT call has only 144 groups of 32 queries) then still
//   spread over many SIMDs.
//
// Per 32-key block a wave computes the transposed score tile S^T = K Q^T with 32x32x2 fp32 MFMAs:
//   A operand  K[key = lane%32][d], B operand Q^T[d][query = lane%32], the head dim split between
//   the two half-waves (d = half*D/2 + s, s = 0..D/2-1). Q stays in VGPRs for the whole kernel.
//   Accumulator layout: lane l holds query l%32 and keys 8*(r/4) + 4*(l/32) + r%4 in register r,
//   so the row max and row sum of a query are in-lane over 16 registers plus one exchange with
//   lane l^32 (v_permlane32_swap).
// The probabilities P then feed O^T += V^T P^T directly from the accumulator registers: MFMA r of
//   the PV step uses P register r as its B operand (keys {8*(r/4)+r%4, 8*(r/4)+4+r%4} across the
//   half-waves) and reads V for exactly that key pair from LDS as its A operand.
//   O^T accumulates in D/32 tiles of 16 registers: lane l holds query l%32, dims
//   32*t + 8*(r/4) + 4*(l/32) + r%4.
//
// Softmax arithmetic (base 2): u = s*scale*log2(e) + bias*log2(e); masked keys get u = -inf;
//   m = running max (seeded with -FLT_MAX), p = exp2(u - m), alpha = exp2(m_old - m_new),
//   l = l*alpha + sum p, O = O*alpha + P V; output O / l, or 0 when every key is masked.
//
// LDS: K tile [KT keys][D+4] (b128 reads of 16 consecutive rows hit distinct banks),
//      V tile [KT keys][D+8] (rows 4 apart land 32 banks apart for the two half-waves).

#include "common.h"
#include "kernels.h"

namespace sa {

namespace {

template <int D, int NSPLIT, int BIAS>
__global__ __launch_bounds__(256) void flash_mfma_kernel(AttnParams p, int q_tiles) {
  constexpr int QG = 4 / NSPLIT;       // query groups (of 32) per workgroup
  constexpr int QT = 32 * QG;          // queries per workgroup
  constexpr int KT = 32 * NSPLIT;      // keys staged per step
  constexpr int KSTR = D + 4;
  constexpr int VSTR = D + 8;
  constexpr int QREG = D / 2;          // Q values per lane
  constexpr int NDB = D / 32;          // 32-dim output tiles
  constexpr int F4_ROW = D / 4;        // float4 per row
  constexpr int NL = KT * F4_ROW / 256;  // float4 loads per thread per tensor per step
  static_assert(NL * 256 == KT * F4_ROW, "tile must split evenly over 256 threads");
  constexpr int RB = QT + KT - 1;      // relative-bias entries needed per step
  constexpr int MSTRIDE = 16 * NDB + 2;  // merge record per lane: O tiles, m, l
  constexpr int LDS_KV = KT * (KSTR + VSTR);
  constexpr int LDS_MERGE = (NSPLIT - 1) * QG * 64 * MSTRIDE;
  constexpr int LDS_FLOATS = LDS_KV > LDS_MERGE ? LDS_KV : LDS_MERGE;

  __shared__ __attribute__((aligned(16))) float lds[LDS_FLOATS];
  __shared__ float lds_rb[BIAS == BIAS_RELPOS ? RB : 1];
  float* const lds_k = lds;
  float* const lds_v = lds + KT * KSTR;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int qg = wave % QG;
  const int ks = wave / QG;
  const int col = lane & 31;
  const int half = lane >> 5;

  int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int qtile = tile % q_tiles;
  tile /= q_tiles;
  const int h = tile % p.H;
  const int b = tile / p.H;
  const int q0 = qtile * QT;
  const int qi = q0 + qg * 32 + col;
  const bool q_valid = qi < p.Lq;

  int kv_len = p.Lk;
  if (p.mask_mode == MASK_KEY_LEN) kv_len = min(max(p.key_len[b], 0), p.Lk);
  const int nblk = (kv_len + 31) >> 5;
  const int nstep = (nblk + NSPLIT - 1) / NSPLIT;
  const bool use_kmask = p.mask_mode == MASK_KEY_MASK;
  const uint8_t* kmask = use_kmask ? p.key_mask + (int64_t)b * p.smask : nullptr;

  // ---- Q into registers: lane holds Q[qi][half*D/2 + s], s = 0..D/2-1
  float qr[QREG];
  {
    const float* src = p.q + p.q_off + (int64_t)b * p.sq + (int64_t)qi * p.ldq + h * D + half * (D / 2);
#pragma unroll
    for (int i = 0; i < QREG / 4; ++i) {
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (q_valid) x = *reinterpret_cast<const f32x4*>(src + 4 * i);
      qr[4 * i + 0] = x[0];
      qr[4 * i + 1] = x[1];
      qr[4 * i + 2] = x[2];
      qr[4 * i + 3] = x[3];
    }
  }

  const float* kbase = p.k + p.k_off + (int64_t)b * p.sk + h * D;
  const float* vbase = p.v + p.v_off + (int64_t)b * p.sv + h * D;

  // ---- K/V staging: thread t moves float4 #(n*256 + t) of the KT x D tile (row-major)
  f32x4 pk[NL], pv[NL];
  float prb = 0.f;
  auto load_step = [&](int step) {
    const int key0 = step * KT;
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      const int idx = n * 256 + tid;
      const int row = idx / F4_ROW;
      const int c4 = idx % F4_ROW;
      const int key = key0 + row;
      f32x4 zk = {0.f, 0.f, 0.f, 0.f};
      f32x4 zv = zk;
      if (key < kv_len) {
        zk = *reinterpret_cast<const f32x4*>(kbase + (int64_t)key * p.ldk + 4 * c4);
        zv = *reinterpret_cast<const f32x4*>(vbase + (int64_t)key * p.ldv + 4 * c4);
      }
      pk[n] = zk;
      pv[n] = zv;
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
        prb = val;
      }
    }
  };
  auto store_step = [&]() {
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      const int idx = n * 256 + tid;
      const int row = idx / F4_ROW;
      const int c4 = idx % F4_ROW;
      *reinterpret_cast<f32x4*>(lds_k + row * KSTR + 4 * c4) = pk[n];
      *reinterpret_cast<f32x4*>(lds_v + row * VSTR + 4 * c4) = pv[n];
    }
    if constexpr (BIAS == BIAS_RELPOS) {
      if (tid < RB) lds_rb[tid] = prb;
    }
  };

  f32x16 oacc[NDB];
#pragma unroll
  for (int t = 0; t < NDB; ++t) oacc[t] = f32x16{0.f};
  float m = kMaxSeed;
  float l = 0.f;

  if (nstep > 0) {
    load_step(0);
    store_step();
  }

  for (int step = 0; step < nstep; ++step) {
    __syncthreads();
    if (step + 1 < nstep) load_step(step + 1);
    const int blk = step * NSPLIT + ks;
    if (blk < nblk) {
      const int k0 = blk * 32;
      // ---- S^T = K Q^T for 32 keys x 32 queries
      f32x16 s = f32x16{0.f};
      const float* krow = lds_k + (ks * 32 + col) * KSTR + half * (D / 2);
#pragma unroll
      for (int i = 0; i < QREG / 4; ++i) {
        const f32x4 kv = *reinterpret_cast<const f32x4*>(krow + 4 * i);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[0], qr[4 * i + 0], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[1], qr[4 * i + 1], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[2], qr[4 * i + 2], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[3], qr[4 * i + 3], s, 0, 0, 0);
      }

      // ---- scores in the base-2 domain, bias and masks
      float u[16];
      if constexpr (BIAS == BIAS_NONE) {
#pragma unroll
        for (int r = 0; r < 16; ++r) u[r] = s[r] * p.scale_log2;
      } else if constexpr (BIAS == BIAS_RELPOS) {
        // rb entry for (key, qi): key - qi + (q0 + QT - 1) - step*KT
        const int rb0 = k0 - step * KT + 4 * half - qi + q0 + QT - 1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int e = rb0 + 8 * (r >> 2) + (r & 3);
          u[r] = fmaf(s[r], p.scale_log2, lds_rb[e]);
        }
      } else {  // BIAS_DENSE
        const float* brow = p.bias + (int64_t)b * p.sbias + ((int64_t)h * p.Lq + (q_valid ? qi : 0)) * p.Lk;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
          const float bv = (q_valid && key < kv_len) ? brow[key] * kLog2e : 0.f;
          u[r] = fmaf(s[r], p.scale_log2, bv);
        }
      }
      if (k0 + 32 > kv_len || use_kmask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
          bool keep = key < kv_len;
          if (use_kmask && keep) keep = kmask[key] != 0;
          if (!keep) u[r] = -INFINITY;
        }
      }

      // ---- online softmax
      float mb = u[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mb = fmaxf(mb, u[r]);
      mb = max_with_partner(mb);
      const float m_new = fmaxf(m, mb);
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        u[r] = fast_exp2(u[r] - m_new);
        ps += u[r];
      }
      l = fmaf(l, alpha, ps);
#pragma unroll
      for (int t = 0; t < NDB; ++t) oacc[t] *= alpha;

      // ---- O^T += V^T P^T
      const float* vcol = lds_v + (ks * 32 + 4 * half) * VSTR + col;
#pragma unroll
      for (int t = 0; t < NDB; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float vv = vcol[(8 * (r >> 2) + (r & 3)) * VSTR + 32 * t];
          oacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, u[r], oacc[t], 0, 0, 0);
        }
      }
    }
    __syncthreads();
    if (step + 1 < nstep) store_step();
  }

  // ---- merge the key splits: waves ks > 0 publish (O, m, l), wave ks == 0 combines
  if constexpr (NSPLIT > 1) {
    float* rec = lds + ((ks - 1) * QG + qg) * 64 * MSTRIDE + lane;
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
      const float* o2 = lds + ((sp - 1) * QG + qg) * 64 * MSTRIDE + lane;
      mt = fmaxf(mt, o2[(16 * NDB) * 64]);
    }
    const float a0 = fast_exp2(m - mt);
    l *= a0;
#pragma unroll
    for (int t = 0; t < NDB; ++t) oacc[t] *= a0;
#pragma unroll
    for (int sp = 1; sp < NSPLIT; ++sp) {
      const float* o2 = lds + ((sp - 1) * QG + qg) * 64 * MSTRIDE + lane;
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
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (q_valid) {
    float* dst = p.o + p.o_off + (int64_t)b * p.so + (int64_t)qi * p.ldo + h * D + 4 * half;
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

template <int D, int NSPLIT>
hipError_t launch_split(const AttnParams& p, hipStream_t stream) {
  constexpr int QT = 32 * (4 / NSPLIT);
  const int q_tiles = (p.Lq + QT - 1) / QT;
  const int64_t n = (int64_t)p.B * p.H * q_tiles;
  if (n > 0x7fffffff) return hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)n), block(256);
  switch (p.bias_mode) {
    case BIAS_NONE:
      hipLaunchKernelGGL((flash_mfma_kernel<D, NSPLIT, BIAS_NONE>), grid, block, 0, stream, p, q_tiles);
      break;
    case BIAS_DENSE:
      hipLaunchKernelGGL((flash_mfma_kernel<D, NSPLIT, BIAS_DENSE>), grid, block, 0, stream, p, q_tiles);
      break;
    case BIAS_RELPOS:
      hipLaunchKernelGGL((flash_mfma_kernel<D, NSPLIT, BIAS_RELPOS>), grid, block, 0, stream, p, q_tiles);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

const char* flash_mfma_name(int D, int nsplit) {
  if (D == 64) return nsplit == 4 ? "flash_mfma_d64_split4" : nsplit == 2 ? "flash_mfma_d64_split2" : "flash_mfma_d64";
  if (D == 128) return nsplit == 2 ? "flash_mfma_d128_split2" : "flash_mfma_d128";
  return nullptr;
}

hipError_t launch_flash_mfma(const AttnParams& p, int nsplit, hipStream_t stream) {
  if (p.D == 64) {
    if (nsplit == 4) return launch_split<64, 4>(p, stream);
    if (nsplit == 2) return launch_split<64, 2>(p, stream);
    return launch_split<64, 1>(p, stream);
  }
  if (p.D == 128) {
    if (nsplit >= 2) return launch_split<128, 2>(p, stream);
    return launch_split<128, 1>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace sa
