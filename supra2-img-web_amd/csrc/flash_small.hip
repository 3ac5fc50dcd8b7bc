// Attention on fp32 MFMA for small launches with head dim 64: the batch-2 DiT self- and
// cross-attention calls (app/models/dit.js:172, 184) and a T5 prompt (app/models/t5.js:80), whose
// few groups of 32 queries leave most of the chip idle under the flash kernel's 128-query
// workgroups. Same contract as the flash kernel (app/gpu/kernels.js:164-316, and the biased and
// masked chain of app/gpu/ops.js:119-147 fused in).
//
// Work decomposition
//   One workgroup per group of 32 queries of one (sequence, head); its key blocks (32 keys each)
//   are dealt to the NW = 4 waves (block j to wave j % NW), and every wave keeps its own online-softmax
//   state (m, l, O). K, V and Q go from memory into registers, so a wave waits only for its own
//   loads and no barrier comes before the end, where the NW partial states are merged through LDS
//   by every thread of the workgroup and stored as whole 256-byte rows. V is loaded in the layout
//   the MFMAs consume (two whole rows per instruction); K and Q are loaded as whole rows and
//   transposed through a wave-private LDS tile. The next block of a wave streams into a second
//   register set while the current one is consumed.
//   Scores: S^T = K Q^T with v_mfma_f32_32x32x2f32 as in the flash kernel: lane l holds query l%32
//   and keys 8(r/4) + 4(l/32) + r%4 in register r; the head dim is split between the half-waves by
//   16-byte chunks 2i + half, and Q stays pre-scaled by scale * log2(e) in registers.
//   Output: O^T += V^T P^T, P straight from the score registers. Row m of output tile t holds head
//   dim 2m + t, so a lane's V operands for one key are a single 8-byte load (dims 2m, 2m + 1).
//   Relative-position bias: the 63 table values a block needs (key - query spans -31..31 around
//   the block's diagonal offset) are gathered once per wave, one per lane, then moved to the lanes
//   that add them with ds_bpermute (a register permute, no LDS storage).
//   Masks: per-sequence key lengths bound the blocks; K rows are loaded up to Lk - 1 before the
//   length is known (their scores are replaced by -inf), V rows only up to the last valid key.

#include <string.h>

#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace sa {

namespace {

constexpr float kRescaleSlack = 8.f;  // log2 units: p stays <= 256 between rescales
constexpr int kD = 64;
constexpr int kWaves = 4;

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// K rows of one block as loaded: kr[i] = chunk lane % 16 of key row 4i + lane / 16 (whole rows per
// instruction); transposed through LDS into the MFMA layout when the block is consumed.
struct KBlock {
  f32x4 kr[8];
};
// V operands of one block: vr[r] = V[key(r)][2*col .. 2*col + 1], key(r) = 8(r/4) + r%4 + 4*half.
struct VBlock {
  float2 vr[16];
};
// Bias and mask operands of one block, loaded with its K and V: the relative-position bucket of
// entry `lane` (rel = k0 - q0 - 31 + lane; the table value is fetched at use), or the dense-bias
// values / key-mask bytes of the lane's 16 keys.
template <int BIAS, int MASK>
struct BBlock {
  int bucket;
  f32x4 bv[BIAS == BIAS_DENSE ? 4 : 1];       // keys 8g + 4*half + 0..3 in bv[g]
  uint32_t km[MASK == MASK_KEY_MASK ? 4 : 1];  // their mask bytes, little-endian in km[g]
};

template <int NW, int BIAS, int MASK>
__global__ __launch_bounds__(64 * NW, 1) void flash_small_kernel(FlashArgs p) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31;
  const int half = lane >> 5;

  const int q_groups = (p.Lq + 31) >> 5;
  // aux: the key-mask row stride with a key mask, else the first 32-query group of the launch
  int tile = xcd_remap(blockIdx.x, p.tiles) + (MASK == MASK_KEY_MASK ? 0 : p.aux);
  const int g = tile % q_groups;
  tile /= q_groups;
  const int h = tile % p.H;
  const int b = tile / p.H;
  const int q0 = g * 32;
  const int qi = q0 + col;
  const bool q_valid = qi < p.Lq;

  const float* kbase = p.k + (int64_t)b * p.sk + h * kD;
  const float* vbase = p.v + (int64_t)b * p.sv + h * kD;

  // K rows up to Lk - 1 (the key length may still be in flight); V rows up to the last valid key.
  // K and Q are read as whole 256-byte rows, four per instruction, and turned into the MFMA layout
  // (a lane's own row) through a wave-private LDS tile: read straight in that layout, every load
  // instruction touched 32 rows, and the first block of a batch-2 call waited on the L1 for it
  // (DiT self-attention batch 2 9.30 -> 8.54 us, cross 6.47 -> 5.94, T5 7.47 -> 6.64; whole-row
  // loads with no transpose at all, results discarded, measured 7.97 / 5.45 / 6.35).
  auto load_k = [&](KBlock& kb, int j) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      kb.kr[i] = *reinterpret_cast<const f32x4*>(kbase + (int64_t)min(j * 32 + 4 * i + (lane >> 4), p.Lk - 1) * p.ldk +
                                                 4 * (lane & 15));
  };
  // wave-private 32 x 64 tile: 16-byte chunk c of row r at c ^ (r & 15) (conflict-free both ways).
  // (Transposing the next block's K behind the current block's products, with a second tile for
  // Q, measured 0.1 us slower at batch 2.)
  __shared__ __attribute__((aligned(16))) float lds_t[NW * 32 * kD];
  float* const tt = lds_t + wave * 32 * kD;
  auto transpose = [&](const f32x4 (&rows)[8], f32x4 (&out)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 4 * i + (lane >> 4);
      *reinterpret_cast<f32x4*>(tt + r * kD + 4 * ((lane & 15) ^ (r & 15))) = rows[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = *reinterpret_cast<const f32x4*>(tt + col * kD + 4 * ((2 * i + half) ^ (col & 15)));
  };
  auto load_v = [&](VBlock& vb, int j, int kv_len) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = min(j * 32 + 8 * (r >> 2) + (r & 3) + 4 * half, kv_len - 1);
      vb.vr[r] = *reinterpret_cast<const float2*>(vbase + (int64_t)key * p.ldv + 2 * col);
    }
  };

  const uint8_t* kmask = MASK == MASK_KEY_MASK ? static_cast<const uint8_t*>(p.mask) + (int64_t)b * p.aux : nullptr;
  const float* brow = nullptr;
  if constexpr (BIAS == BIAS_DENSE) brow = p.bias + (int64_t)b * p.sbias + ((int64_t)h * p.Lq + min(qi, p.Lq - 1)) * p.Lk;
  // The lane's 16 keys are four runs of 4 (keys k0 + 8g + 4*half + 0..3): one 16-byte dense-bias load
  // and one 4-byte mask load per run when the rows allow it (whole block inside Lk, aligned rows),
  // element loads at clamped indices otherwise.
  const bool bias_vec = BIAS == BIAS_DENSE && ((reinterpret_cast<uintptr_t>(p.bias) | (uintptr_t)p.Lk |
                                                (uintptr_t)(p.sbias * 4)) & 15) == 0;
  const bool mask_vec = MASK == MASK_KEY_MASK && (reinterpret_cast<uintptr_t>(kmask) & 3) == 0;
  using BB = BBlock<BIAS, MASK>;
  auto load_b = [&](BB& bb, int j) {
    const int k0 = j * 32;
    if constexpr (BIAS == BIAS_RELPOS) {
      const int li = k0 - q0 - 31 + lane + (p.Lq - 1);
      // -1 marks a lane past the LUT (no bias there); bucket ids below 0 clamp to 0, and above the
      // table to its last row (where used), as in every kernel
      bb.bucket = (lane < 63 && li >= 0 && li <= p.Lq + p.Lk - 2) ? max(p.lut[li], 0) : -1;
    }
    if constexpr (BIAS == BIAS_DENSE) {
      if (bias_vec && k0 + 32 <= p.Lk) {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) bb.bv[gq] = *reinterpret_cast<const f32x4*>(brow + k0 + 8 * gq + 4 * half);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) bb.bv[r >> 2][r & 3] = brow[min(k0 + 8 * (r >> 2) + 4 * half + (r & 3), p.Lk - 1)];
      }
    }
    if constexpr (MASK == MASK_KEY_MASK) {
      if (mask_vec && k0 + 32 <= p.Lk) {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) bb.km[gq] = *reinterpret_cast<const uint32_t*>(kmask + k0 + 8 * gq + 4 * half);
      } else {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          uint32_t w = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) w |= (uint32_t)kmask[min(k0 + 8 * gq + 4 * half + e, p.Lk - 1)] << (8 * e);
          bb.km[gq] = w;
        }
      }
    }
  };

  // ---- loads of the first block, issued before anything waits (bias / mask operands first: the
  // relative-position table value depends on the bucket)
  const int blk0 = wave;
  KBlock kb0, kb1;
  VBlock vb0, vb1;
  BB bb0, bb1;
  if (blk0 * 32 < p.Lk) {
    load_b(bb0, blk0);
    load_k(kb0, blk0);
  }

  int kv_len = p.Lk;
  if constexpr (MASK == MASK_KEY_LEN) kv_len = min(max(static_cast<const int32_t*>(p.mask)[b], 0), p.Lk);
  const int nblk = (kv_len + 31) >> 5;
  if (blk0 < nblk) load_v(vb0, blk0, kv_len);

  // ---- Q in registers, pre-scaled: qr[4i + j] = scale*log2(e)*Q[qi][8i + 4*half + j]
  float qr[32];
  {
    f32x4 rows[8], xq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      rows[i] = *reinterpret_cast<const f32x4*>(p.q + (int64_t)b * p.sq +
                                                (int64_t)min(q0 + 4 * i + (lane >> 4), p.Lq - 1) * p.ldq + h * kD + 4 * (lane & 15));
    transpose(rows, xq);
    const float sc = q_valid ? p.scale_log2 : 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qr[4 * i + 0] = xq[i][0] * sc;
      qr[4 * i + 1] = xq[i][1] * sc;
      qr[4 * i + 2] = xq[i][2] * sc;
      qr[4 * i + 3] = xq[i][3] * sc;
    }
  }

  f32x16 oacc0 = zero16(), oacc1 = zero16();
  float m = kMaxSeed;
  float l = 0.f;

  auto compute = [&](int j, const KBlock& kb, const VBlock& vb, const BB& bb) {
    const int k0 = j * 32;
    // relative-position bias: lane e (< 63) holds the table value of entry e (rel = k0 - q0 - 31 + e),
    // fetched before the score MFMAs so that they cover its latency
    float rb = 0.f;
    if constexpr (BIAS == BIAS_RELPOS) {
      if (bb.bucket >= 0) rb = p.bias[min(bb.bucket, p.num_buckets - 1) * p.H + h];
    }
    f32x4 kk[8];  // kk[i] = K[key k0 + col][chunk 2i + half]
    transpose(kb.kr, kk);
    f32x16 s = zero16();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[i][0], qr[4 * i + 0], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[i][1], qr[4 * i + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[i][2], qr[4 * i + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[i][3], qr[4 * i + 3], s, 0, 0, 0);
    }
    // keep the permutes of the table value after the MFMAs, which then cover the table load
    if constexpr (BIAS == BIAS_RELPOS) __builtin_amdgcn_sched_barrier(0);
    float u[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) u[r] = s[r];
    if constexpr (BIAS == BIAS_RELPOS) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int e = 31 + 8 * (r >> 2) + 4 * half + (r & 3) - col;  // 0..62
        u[r] = fmaf(__int_as_float(__builtin_amdgcn_ds_bpermute(e << 2, __float_as_int(rb))), kLog2e, u[r]);
      }
    } else if constexpr (BIAS == BIAS_DENSE) {
#pragma unroll
      for (int r = 0; r < 16; ++r) u[r] = fmaf(bb.bv[r >> 2][r & 3], kLog2e, u[r]);
    }
    if constexpr (MASK == MASK_KEY_MASK) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
        const uint32_t byte = (bb.km[r >> 2] >> (8 * (r & 3))) & 0xffu;
        u[r] = (key < p.Lk && byte != 0) ? u[r] : -INFINITY;
      }
    } else if (k0 + 32 > kv_len) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
        u[r] = key < kv_len ? u[r] : -INFINITY;
      }
    }
    // ---- online softmax with a lazily moved reference (as in the flash kernel)
    float mb = u[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mb = max_nan(mb, u[r]);
    mb = max_with_partner(mb);
    if (j == blk0) {
      // the wave's first block: its maximum becomes the reference (O and l are still zero, so there is
      // nothing to rescale; -FLT_MAX stays for rows with every key masked)
      m = max_nan(m, mb);
    } else if (__builtin_amdgcn_ballot_w64(mb > m + kRescaleSlack) != 0) {
      const float m_new = max_nan(m, mb);
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      l *= alpha;
      oacc0 *= alpha;
      oacc1 *= alpha;
    }
    float pr[16];
    pr[0] = fast_exp2(u[0] - m);
    float ps = pr[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) {
      pr[r] = fast_exp2(u[r] - m);
      ps += pr[r];
    }
    l += ps;
    // ---- O^T += V^T P^T: row m of tile t is dim 2m + t
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      oacc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(vb.vr[r].x, pr[r], oacc0, 0, 0, 0);
      oacc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(vb.vr[r].y, pr[r], oacc1, 0, 0, 0);
    }
  };

  // ---- this wave's blocks j = wave, wave + NW, ...; the next block streams into the other
  // register set while the current one is consumed (two blocks per iteration: fixed names)
  for (int j = blk0; j < nblk; j += 2 * NW) {
    if (j + NW < nblk) {
      load_b(bb1, j + NW);
      load_k(kb1, j + NW);
      load_v(vb1, j + NW, kv_len);
    }
    compute(j, kb0, vb0, bb0);
    if (j + NW >= nblk) break;
    if (j + 2 * NW < nblk) {
      load_b(bb0, j + 2 * NW);
      load_k(kb0, j + 2 * NW);
      load_v(vb0, j + 2 * NW, kv_len);
    }
    compute(j + NW, kb1, vb1, bb1);
  }

  // ---- merge the NW partial states: records in LDS, then every thread combines 4 dims of one query
  // Record rows of kD floats, 16-byte chunk c of row r at c ^ (r & 15): the writes (16 query rows
  // per 16 lanes, the same chunk each) and the combine reads (whole rows) are both conflict-free.
  // (Rows padded to 68 floats instead kept the writes conflict-free, but the reads of four padded
  // rows per wave then stalled 128 cycles per workgroup on bank conflicts, SQ_LDS_BANK_CONFLICT.)
  __shared__ __attribute__((aligned(16))) float lds_o[NW * 32 * kD];
  __shared__ float lds_m[NW * 32];
  __shared__ float lds_l[NW * 32];
  const float lt = sum_with_partner(l);
  {
    // lane (col, half) holds dims 16g + 8*half + 0..7 of query col in registers 4g..4g+3 of both tiles
    float* row = lds_o + (wave * 32 + col) * kD;
    const int sw = col & 15;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      f32x4 lo, hi;
      lo[0] = oacc0[4 * gq + 0];
      lo[1] = oacc1[4 * gq + 0];
      lo[2] = oacc0[4 * gq + 1];
      lo[3] = oacc1[4 * gq + 1];
      hi[0] = oacc0[4 * gq + 2];
      hi[1] = oacc1[4 * gq + 2];
      hi[2] = oacc0[4 * gq + 3];
      hi[3] = oacc1[4 * gq + 3];
      *reinterpret_cast<f32x4*>(row + 4 * ((4 * gq + 2 * half) ^ sw)) = lo;
      *reinterpret_cast<f32x4*>(row + 4 * ((4 * gq + 2 * half + 1) ^ sw)) = hi;
    }
    if (half == 0) {
      lds_m[wave * 32 + col] = m;
      lds_l[wave * 32 + col] = lt;
    }
  }
  __syncthreads();
  float* obase = p.o + (int64_t)b * p.so + h * kD;
  for (int item = tid; item < 32 * 16; item += 64 * NW) {
    const int q = item >> 4, c = item & 15;
    float mt = lds_m[q];
#pragma unroll
    for (int w = 1; w < NW; ++w) mt = max_nan(mt, lds_m[w * 32 + q]);
    float lsum = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float a = fast_exp2(lds_m[w * 32 + q] - mt);
      lsum = fmaf(lds_l[w * 32 + q], a, lsum);
      const f32x4 x = *reinterpret_cast<const f32x4*>(lds_o + (w * 32 + q) * kD + 4 * (c ^ (q & 15)));
      acc[0] = fmaf(x[0], a, acc[0]);
      acc[1] = fmaf(x[1], a, acc[1]);
      acc[2] = fmaf(x[2], a, acc[2]);
      acc[3] = fmaf(x[3], a, acc[3]);
    }
    const float inv = lsum > 0.f ? __builtin_amdgcn_rcpf(lsum) : 0.f;  // v_rcp_f32 (1 ulp)
    acc *= inv;
    // non-temporal, as in the flash kernel: O is not read again here
    if (q0 + q < p.Lq) __builtin_nontemporal_store(acc, reinterpret_cast<f32x4*>(obase + (int64_t)(q0 + q) * p.ldo + 4 * c));
  }
}

template <int NW, int BIAS>
hipError_t launch_mask(const FlashArgs& a, int mask_mode, dim3 grid, hipStream_t stream) {
  switch (mask_mode) {
    case MASK_NONE:
      hipLaunchKernelGGL((flash_small_kernel<NW, BIAS, MASK_NONE>), grid, dim3(64 * NW), 0, stream, a);
      break;
    case MASK_KEY_LEN:
      hipLaunchKernelGGL((flash_small_kernel<NW, BIAS, MASK_KEY_LEN>), grid, dim3(64 * NW), 0, stream, a);
      break;
    case MASK_KEY_MASK:
      hipLaunchKernelGGL((flash_small_kernel<NW, BIAS, MASK_KEY_MASK>), grid, dim3(64 * NW), 0, stream, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int NW>
hipError_t launch_nw(const AttnParams& p, int64_t first, int64_t n, hipStream_t stream) {
  if (first + n > 0x7fffffff || !flash_mfma_args_fit(p)) return hipErrorInvalidConfiguration;
  if (first > 0 && p.mask_mode == MASK_KEY_MASK) return hipErrorInvalidValue;  // aux holds the mask stride
  FlashArgs a = flash_args(p, n);
  if (p.mask_mode != MASK_KEY_MASK) a.aux = (int32_t)first;
  const dim3 grid((unsigned)n);
  switch (p.bias_mode) {
    case BIAS_NONE: return launch_mask<NW, BIAS_NONE>(a, p.mask_mode, grid, stream);
    case BIAS_DENSE: return launch_mask<NW, BIAS_DENSE>(a, p.mask_mode, grid, stream);
    case BIAS_RELPOS: return launch_mask<NW, BIAS_RELPOS>(a, p.mask_mode, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// Four waves, one per SIMD. Measured on the batch-2 DiT self-attention call (eight key blocks):
// 9.25 us with four waves of two blocks each against 9.99 us with eight waves of one block (two
// per SIMD), whose merge doubles and whose register budget halves.
int flash_small_waves(const AttnParams&) { return kWaves; }

int64_t flash_small_workgroups(const AttnParams& p) { return (int64_t)p.B * p.H * ((p.Lq + 31) / 32); }

const char* flash_small_name(int) { return "flash_small_d64"; }

int flash_small_variants(FlashVariant* out, int cap) {
  int n = 0;
  for (int bias = BIAS_NONE; bias <= BIAS_RELPOS; ++bias)
    for (int mask = MASK_NONE; mask <= MASK_KEY_MASK; ++mask) {
      if (n < cap) out[n] = {kD, kWaves, bias, mask};
      ++n;
    }
  return n;
}

hipError_t launch_flash_small(const AttnParams& p, hipStream_t stream) {
  if (p.D != kD) return hipErrorInvalidValue;
  return launch_nw<kWaves>(p, 0, flash_small_workgroups(p), stream);
}

hipError_t launch_flash_small_groups(const AttnParams& p, int64_t first, int64_t count, hipStream_t stream) {
  if (p.D != kD || first < 0 || count <= 0 || first + count > flash_small_workgroups(p)) return hipErrorInvalidValue;
  return launch_nw<kWaves>(p, first, count, stream);
}

}  // namespace sa
