// Attention on fp32 MFMA for small head-dim-64 launches, in groups of 16 queries: launches whose
// 16-query groups still number at most one per CU (a T5 prompt, app/models/t5.js:80: 12 heads x 128
// queries = 96 groups; the per-sample DiT calls, app/models/dit.js:172 and 184: 9 heads x 256
// queries = 144). Same contract as the flash kernel (app/gpu/kernels.js:164-316, with the biased and
// masked chain of app/gpu/ops.js:119-147 fused in).
//
// Why 16 queries. The 32-query small-launch kernel (flash_small.hip) deals a group's 32-key blocks to
// its 4 waves, one per SIMD, so a SIMD's work is its blocks' products: 64 32x32x2 MFMAs = 4096
// cycles per block. Such launches leave CUs idle; with groups of 16 queries on v_mfma_f32_16x16x4f32
// the same call spreads over twice the CUs and a block costs a SIMD half the cycles (32 + 32 MFMAs
// of 32 cycles), so the wave chains halve.
//
// Layouts (v_mfma_f32_16x16x4f32: A[i][k] from lane i + 16k, B[k][j] from lane j + 16k, register r
// of lane l = D[4(l/16) + r][l % 16]; qc = l % 16 the lane's query, g = l / 16 its row group):
//   Scores: S^T = K Q^T as two 16-key tiles. Step (t, c) contracts head dim 16t + 4g + c in lane
//   group g, so the lane's Q operands are Q[qc][16t + 4g .. + 3] (four 16-byte loads, kept
//   pre-scaled by scale * log2(e)) and one 16-byte K load per tile and t feeds four steps. Lane l
//   then holds query qc and keys 4g + r (tile 0) and 16 + 4g + r (tile 1) of the block.
//   PV: O^T += V^T P^T, step s pairing lane group g with key 4g + s (s < 4) or 16 + 4g + s - 4, so
//   the B operand is the lane's own score register s. Output tile t row i is head dim 4i + t, so
//   one 16-byte load V[key][4 qc .. 4 qc + 3] feeds the four tiles (four 256-byte rows per
//   instruction), and lane l ends holding dims 16g + 4r + t of query qc in tile t register r.
//   Row maxima and sums of a query span the four lane groups: v_permlane16_swap then
//   v_permlane32_swap.
// Masks and bias as in flash_small: K rows are read up to Lk - 1 (the key length may still be in
// flight; scores past it become -inf by a select), V rows up to the last valid key, except for the
// wave's first block, whose V rows are read up to Lk - 1 as well and zeroed past the key length
// before the PV products (so no load waits for the key length); the relative
// bias of a block (key - query spans -15..31 around its diagonal offset) is gathered one entry per
// lane and moved to the score registers with ds_bpermute.
//
// Packed sequences (the key-length variant whose host copy of the lengths came along): a sequence
// of at most one key block keeps three of the four waves of its workgroups idle, of two blocks two.
// Where a launch has more groups than CUs, the host gives such sequences 2 (or 1) waves per 16-query
// group, so their workgroups hold 2 (4) groups, until the launch fits one workgroup per CU: a
// batch-2 guided DiT cross call (77 keys, and 1 key for the unconditioned half,
// app/models/dit.js:184) then takes 144 + 72 workgroups instead of 2 x 144. The waves per group are
// 2-bit codes per sequence in the kernel arguments.

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace sa {

namespace {

constexpr float kRescaleSlack = 8.f;  // log2 units: p stays <= 256 between rescales
constexpr int kD = 64;
constexpr int kQG = 16;  // queries per workgroup
constexpr int kNW = 4;   // waves per workgroup, one per SIMD
constexpr int kMaxPacked = 16;  // sequences of a packed launch (2 bits each in FlashArgs::aux)

// One block's operands as loaded: K of the two 16-key tiles, V in the PV operand layout, and the
// bias / mask operands of the lane's 8 keys.
template <int BIAS, int MASK>
struct Block16 {
  f32x4 k[2][4];  // k[tile][t] = K[k0 + 16 tile + qc][16t + 4g .. + 3]
  f32x4 v[8];     // v[s] = V[k0 + key(s)][4 qc .. 4 qc + 3]
  int bucket;     // relative bias: bucket of entry `lane` (-1: none)
  f32x4 bv[BIAS == BIAS_DENSE ? 2 : 1];        // dense bias of keys 16 tile + 4g + 0..3 in bv[tile]
  uint32_t km[MASK == MASK_KEY_MASK ? 2 : 1];  // their mask bytes, little-endian
};

template <int BIAS, int MASK>
__global__ __launch_bounds__(64 * kNW, 1) void flash_small16_kernel(FlashArgs p) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qc = lane & 15;
  const int rg = lane >> 4;

  constexpr bool kPacked = MASK == MASK_KEY_LEN_ORDERED;
  constexpr bool kKeyLen = MASK == MASK_KEY_LEN || kPacked;
  const int q_groups = (p.Lq + kQG - 1) / kQG;
  int tile = xcd_remap(blockIdx.x, p.tiles);
  // lw: log2 of the waves per 16-query group. The workgroup holds the 4 >> lw groups g0, g0 + 1, ...
  // of one (sequence, head); wave w works on group g0 + (w >> lw), key blocks w % 2^lw + i 2^lw.
  int lw = 2, b, h, g0;
  if constexpr (kPacked) {
    // sequences in batch order, each with H heads x ceil(q_groups / (4 >> lw)) workgroups, lw of
    // sequence s in bits 2s, 2s + 1 of aux (the host counts the grid from the same codes)
    const uint32_t code = static_cast<uint32_t>(p.aux);
    b = 0;
    int per_head;
    for (;;) {
      lw = min((int)(code >> (2 * b)) & 3, 2);
      per_head = (q_groups + (4 >> lw) - 1) >> (2 - lw);
      if (tile < p.H * per_head || b == kMaxPacked - 1) break;
      tile -= p.H * per_head;
      ++b;
    }
    h = tile / per_head;
    g0 = (tile - h * per_head) << (2 - lw);
  } else {
    g0 = tile % q_groups;
    tile /= q_groups;
    h = tile % p.H;
    b = tile / p.H;
  }
  const int nwg = 1 << lw;                   // waves per group
  const int gq = g0 + (wave >> lw);          // this wave's group
  const bool g_valid = gq < q_groups;        // (the last workgroup of a head may hold fewer groups)
  const int q0 = gq * kQG;
  const int qi = q0 + qc;
  const bool q_valid = qi < p.Lq;

  const float* kbase = p.k + (int64_t)b * p.sk + h * kD;
  const float* vbase = p.v + (int64_t)b * p.sv + h * kD;
  const uint8_t* kmask = MASK == MASK_KEY_MASK ? static_cast<const uint8_t*>(p.mask) + (int64_t)b * p.aux : nullptr;
  const float* brow = nullptr;
  if constexpr (BIAS == BIAS_DENSE) brow = p.bias + (int64_t)b * p.sbias + ((int64_t)h * p.Lq + min(qi, p.Lq - 1)) * p.Lk;
  // vector loads of the dense-bias / key-mask runs when the rows allow it and the block is whole
  const bool bias_vec = BIAS == BIAS_DENSE && ((reinterpret_cast<uintptr_t>(p.bias) | (uintptr_t)p.Lk |
                                                (uintptr_t)(p.sbias * 4)) & 15) == 0;
  const bool mask_vec = MASK == MASK_KEY_MASK && (reinterpret_cast<uintptr_t>(kmask) & 3) == 0;

  using BB = Block16<BIAS, MASK>;
  auto load_b = [&](BB& bb, int j) {
    const int k0 = j * 32;
    if constexpr (BIAS == BIAS_RELPOS) {
      // entry e = lane covers key - query = k0 - q0 - 15 + e (e < 47); ids below 0 clamp to 0, above
      // the table to its last row (where used), as in every kernel
      const int li = k0 - q0 - 15 + lane + (p.Lq - 1);
      bb.bucket = (lane < 47 && li >= 0 && li <= p.Lq + p.Lk - 2) ? max(p.lut[li], 0) : -1;
    }
    if constexpr (BIAS == BIAS_DENSE) {
      if (bias_vec && k0 + 32 <= p.Lk) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) bb.bv[tt] = *reinterpret_cast<const f32x4*>(brow + k0 + 16 * tt + 4 * rg);
      } else {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int e = 0; e < 4; ++e) bb.bv[tt][e] = brow[min(k0 + 16 * tt + 4 * rg + e, p.Lk - 1)];
      }
    }
    if constexpr (MASK == MASK_KEY_MASK) {
      if (mask_vec && k0 + 32 <= p.Lk) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) bb.km[tt] = *reinterpret_cast<const uint32_t*>(kmask + k0 + 16 * tt + 4 * rg);
      } else {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          uint32_t w = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) w |= (uint32_t)kmask[min(k0 + 16 * tt + 4 * rg + e, p.Lk - 1)] << (8 * e);
          bb.km[tt] = w;
        }
      }
    }
  };
  auto load_k = [&](BB& bb, int j) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const float* row = kbase + (int64_t)min(j * 32 + 16 * tt + qc, p.Lk - 1) * p.ldk + 4 * rg;
#pragma unroll
      for (int t = 0; t < 4; ++t) bb.k[tt][t] = *reinterpret_cast<const f32x4*>(row + 16 * t);
    }
  };
  // V rows of block j up to row `last` (the last valid key, or Lk - 1 for the first block: see below)
  auto load_v = [&](BB& bb, int j, int last) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int key = min(j * 32 + (s < 4 ? 4 * rg + s : 16 + 4 * rg + s - 4), last);
      bb.v[s] = *reinterpret_cast<const f32x4*>(vbase + (int64_t)key * p.ldv + 4 * qc);
    }
  };

  // ---- the key length, then the first block's operands and Q (in the order they are needed). The
  // first block's V rows are read up to Lk - 1, like K, so that they need not wait for the key
  // length; rows at or past it become zeros before the PV products.
  int kv_len = p.Lk;
  if constexpr (kKeyLen) kv_len = min(max(static_cast<const int32_t*>(p.mask)[b], 0), p.Lk);
  const int blk0 = wave & (nwg - 1);
  BB bb0, bb1;
  if (g_valid && blk0 * 32 < p.Lk) {
    load_b(bb0, blk0);
    load_k(bb0, blk0);
    load_v(bb0, blk0, p.Lk - 1);
  }
  const int nblk = g_valid ? (kv_len + 31) >> 5 : 0;
  f32x4 qv[4];  // qv[t] = scale*log2(e) * Q[qi][16t + 4g .. + 3]
  {
    const float* qrow = p.q + (int64_t)b * p.sq + (int64_t)min(qi, p.Lq - 1) * p.ldq + h * kD + 4 * rg;
#pragma unroll
    for (int t = 0; t < 4; ++t) qv[t] = *reinterpret_cast<const f32x4*>(qrow + 16 * t);
    const float sc = q_valid ? p.scale_log2 : 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) qv[t] *= sc;
  }

  f32x4 oacc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) oacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = kMaxSeed;
  float l = 0.f;

  auto compute = [&](int j, BB& bb) {
    const int k0 = j * 32;
    float rb = 0.f;
    if constexpr (BIAS == BIAS_RELPOS) {
      if (bb.bucket >= 0) rb = p.bias[min(bb.bucket, p.num_buckets - 1) * p.H + h];
    }
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(bb.k[0][t][c], qv[t][c], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(bb.k[1][t][c], qv[t][c], s1, 0, 0, 0);
      }
    if constexpr (BIAS == BIAS_RELPOS) __builtin_amdgcn_sched_barrier(0);  // the permutes after the MFMAs
    float u[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u[r] = s0[r];
      u[4 + r] = s1[r];
    }
    if constexpr (BIAS == BIAS_RELPOS) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int e = 16 * (r >> 2) + 4 * rg + (r & 3) - qc + 15;  // 0..46
        u[r] = fmaf(__int_as_float(__builtin_amdgcn_ds_bpermute(e << 2, __float_as_int(rb))), kLog2e, u[r]);
      }
    } else if constexpr (BIAS == BIAS_DENSE) {
#pragma unroll
      for (int r = 0; r < 8; ++r) u[r] = fmaf(bb.bv[r >> 2][r & 3], kLog2e, u[r]);
    }
    if constexpr (MASK == MASK_KEY_MASK) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int key = k0 + 16 * (r >> 2) + 4 * rg + (r & 3);
        const uint32_t byte = (bb.km[r >> 2] >> (8 * (r & 3))) & 0xffu;
        u[r] = (key < p.Lk && byte != 0) ? u[r] : -INFINITY;
      }
    } else if (k0 + 32 > kv_len) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int key = k0 + 16 * (r >> 2) + 4 * rg + (r & 3);
        u[r] = key < kv_len ? u[r] : -INFINITY;
      }
    }
    // ---- online softmax with a lazily moved reference (as in the flash kernel)
    float mb = u[0];
#pragma unroll
    for (int r = 1; r < 8; ++r) mb = max_nan(mb, u[r]);
    mb = max_over_rows4(mb);
    if (j == blk0) {
      m = max_nan(m, mb);  // the wave's first block sets the reference (nothing to rescale yet)
    } else if (__builtin_amdgcn_ballot_w64(mb > m + kRescaleSlack) != 0) {
      const float m_new = max_nan(m, mb);
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int t = 0; t < 4; ++t) oacc[t] *= alpha;
    }
    float pr[8];
    pr[0] = fast_exp2(u[0] - m);
    float ps = pr[0];
#pragma unroll
    for (int r = 1; r < 8; ++r) {
      pr[r] = fast_exp2(u[r] - m);
      ps += pr[r];
    }
    l += ps;  // this lane's 8 keys; the four row groups are summed at the end
    if (j == blk0 && k0 + 32 > kv_len) {
      // the first block's V rows past the key length (read before it was known) may hold anything,
      // and p = 0 does not cancel a NaN or an infinity there
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int key = k0 + (s < 4 ? 4 * rg + s : 16 + 4 * rg + s - 4);
        if (key >= kv_len) bb.v[s] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    // ---- O^T += V^T P^T: step s on key 4g + s (s < 4) or 16 + 4g + s - 4 of the block
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) oacc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(bb.v[s][t], pr[s], oacc[t], 0, 0, 0);
  };

  // ---- this wave's blocks j = blk0, blk0 + nwg, ...; the next block streams into the other operand
  // set while the current one is consumed (two blocks per iteration: fixed names)
  for (int j = blk0; j < nblk; j += 2 * nwg) {
    if (j + nwg < nblk) {
      load_b(bb1, j + nwg);
      load_k(bb1, j + nwg);
      load_v(bb1, j + nwg, kv_len - 1);
    }
    compute(j, bb0);
    if (j + nwg >= nblk) break;
    if (j + 2 * nwg < nblk) {
      load_b(bb0, j + 2 * nwg);
      load_k(bb0, j + 2 * nwg);
      load_v(bb0, j + 2 * nwg, kv_len - 1);
    }
    compute(j + nwg, bb1);
  }

  const float lt = sum_over_rows4(l);
  if (kPacked && lw == 0) {
    // one wave per group: nothing to merge. Lane (qc, g) holds dims 16g + 4r + t of query qc in
    // oacc[t][r], so it stores 4 x 16 bytes of its query's row.
    const float inv = lt > 0.f ? __builtin_amdgcn_rcpf(lt) : 0.f;  // v_rcp_f32 (1 ulp)
    if (qi < p.Lq) {
      float* orow = p.o + (int64_t)b * p.so + (int64_t)qi * p.ldo + h * kD + 16 * rg;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        f32x4 x = {oacc[0][r], oacc[1][r], oacc[2][r], oacc[3][r]};
        x *= inv;
        __builtin_nontemporal_store(x, reinterpret_cast<f32x4*>(orow + 4 * r));
      }
    }
    return;  // (lw is the same for the whole workgroup: no wave waits at the barrier below)
  }

  // ---- merge the partial states of each group's waves: records in LDS (row of a query: 16 chunks
  // of 16 bytes, chunk c at c ^ (query & 15): conflict-free writes of one chunk by 16 queries and
  // reads of whole rows), then every thread combines and stores 16 bytes of one query per group
  __shared__ __attribute__((aligned(16))) float lds_o[kNW * kQG * kD];
  __shared__ float lds_m[kNW * kQG];
  __shared__ float lds_l[kNW * kQG];
  {
    float* row = lds_o + (wave * kQG + qc) * kD;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f32x4 x;
      x[0] = oacc[0][r];
      x[1] = oacc[1][r];
      x[2] = oacc[2][r];
      x[3] = oacc[3][r];
      *reinterpret_cast<f32x4*>(row + 4 * ((4 * rg + r) ^ qc)) = x;  // dims 16g + 4r .. + 3
    }
    if (rg == 0) {
      lds_m[wave * kQG + qc] = m;
      lds_l[wave * kQG + qc] = lt;
    }
  }
  __syncthreads();
  // NW waves per group, 4 / NW groups, as constants, so that the groups' LDS reads are issued together
  auto merge = [&](auto nw_const) {
    constexpr int NW = decltype(nw_const)::value;
#pragma unroll
    for (int sub = 0; sub < kNW / NW; ++sub) {  // 256 threads: 16 queries x 16 chunks of each group
      const int q = tid >> 4, c = tid & 15;
      const int w0 = sub * NW;  // the group's first wave
      float mt = lds_m[w0 * kQG + q];
#pragma unroll
      for (int w = 1; w < NW; ++w) mt = max_nan(mt, lds_m[(w0 + w) * kQG + q]);
      float lsum = 0.f;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float a = fast_exp2(lds_m[(w0 + w) * kQG + q] - mt);
        lsum = fmaf(lds_l[(w0 + w) * kQG + q], a, lsum);
        const f32x4 x = *reinterpret_cast<const f32x4*>(lds_o + ((w0 + w) * kQG + q) * kD + 4 * (c ^ q));
        acc[0] = fmaf(x[0], a, acc[0]);
        acc[1] = fmaf(x[1], a, acc[1]);
        acc[2] = fmaf(x[2], a, acc[2]);
        acc[3] = fmaf(x[3], a, acc[3]);
      }
      const float inv = lsum > 0.f ? __builtin_amdgcn_rcpf(lsum) : 0.f;  // v_rcp_f32 (1 ulp)
      acc *= inv;
      // non-temporal, as in the flash kernel: O is not read again here
      const int qo = (g0 + sub) * kQG + q;
      if (qo < p.Lq)
        __builtin_nontemporal_store(acc, reinterpret_cast<f32x4*>(p.o + (int64_t)b * p.so + (int64_t)qo * p.ldo + h * kD + 4 * c));
    }
  };
  if (kPacked && lw == 1)
    merge(std::integral_constant<int, 2>{});
  else
    merge(std::integral_constant<int, kNW>{});
}

template <int BIAS>
hipError_t launch_mask16(const FlashArgs& a, int mask_mode, dim3 grid, hipStream_t stream) {
  switch (mask_mode) {
    case MASK_NONE:
      hipLaunchKernelGGL((flash_small16_kernel<BIAS, MASK_NONE>), grid, dim3(64 * kNW), 0, stream, a);
      break;
    case MASK_KEY_LEN:
      hipLaunchKernelGGL((flash_small16_kernel<BIAS, MASK_KEY_LEN>), grid, dim3(64 * kNW), 0, stream, a);
      break;
    case MASK_KEY_MASK:
      hipLaunchKernelGGL((flash_small16_kernel<BIAS, MASK_KEY_MASK>), grid, dim3(64 * kNW), 0, stream, a);
      break;
    case MASK_KEY_LEN_ORDERED:
      hipLaunchKernelGGL((flash_small16_kernel<BIAS, MASK_KEY_LEN_ORDERED>), grid, dim3(64 * kNW), 0, stream, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Workgroups of a launch whose sequence s has log2 waves per 16-query group lw[s].
int64_t packed_workgroups(const AttnParams& p, const int* lw) {
  const int64_t q_groups = (p.Lq + kQG - 1) / kQG;
  int64_t n = 0;
  for (int s = 0; s < p.B; ++s) n += (int64_t)p.H * ((q_groups + (4 >> lw[s]) - 1) >> (2 - lw[s]));
  return n;
}

// The packed variant's codes: log2 of the waves per 16-query group of each sequence, 2 bits per
// sequence. A workgroup holding several groups costs more than one group per CU with idle waves
// (each CU then fetches several Q tiles and runs several softmax chains), so packing is the least
// that makes the launch fit one workgroup per CU: sequences of at most two key blocks go to 2 waves
// per group, shortest first, until the launch fits; if it does not, those of at most one block go
// on to 1 wave per group, shortest first. False when the call does not take the packed variant:
// it needs key lengths with their host copy, at most kMaxPacked sequences, and an unpacked launch
// of more than kSmallLaunchCUs workgroups.
bool small16_packing(const AttnParams& p, uint32_t* code) {
  if (p.mask_mode != MASK_KEY_LEN || p.key_len_host == nullptr || p.B > kMaxPacked) return false;
  if ((int64_t)p.B * p.H * ((p.Lq + kQG - 1) / kQG) <= kSmallLaunchCUs) return false;
  int nblk[kMaxPacked], lw[kMaxPacked], by_len[kMaxPacked];
  for (int s = 0; s < p.B; ++s) {
    nblk[s] = (std::min(std::max(p.key_len_host[s], 0), p.Lk) + 31) / 32;
    lw[s] = 2;
    by_len[s] = s;
  }
  std::stable_sort(by_len, by_len + p.B, [&](int x, int y) { return nblk[x] < nblk[y]; });
  bool packs = false, fits = false;
  for (int pass = 1; pass >= 0 && !fits; --pass)  // 2 waves per group, then 1
    for (int i = 0; i < p.B && !fits; ++i) {
      const int s = by_len[i];
      if (nblk[s] > (pass == 1 ? 2 : 1)) break;
      lw[s] = pass;
      packs = true;
      fits = packed_workgroups(p, lw) <= kSmallLaunchCUs;
    }
  uint32_t c = 0;
  for (int s = 0; s < p.B; ++s) c |= (uint32_t)lw[s] << (2 * s);
  *code = c;
  return packs;
}

// The grid of a launch and whether (with which codes) it packs, from one read of the host lengths:
// the kernel's workgroup decode relies on the grid being exactly the codes' workgroups.
int64_t small16_grid(const AttnParams& p, uint32_t* code, bool* packed) {
  *code = 0;
  *packed = small16_packing(p, code);
  if (!*packed) return (int64_t)p.B * p.H * ((p.Lq + kQG - 1) / kQG);
  int lw[kMaxPacked];
  for (int s = 0; s < p.B; ++s) lw[s] = (*code >> (2 * s)) & 3;
  return packed_workgroups(p, lw);
}

}  // namespace

int64_t flash_small16_workgroups(const AttnParams& p) {
  uint32_t code;
  bool packed;
  return small16_grid(p, &code, &packed);
}

FlashVariant flash_small16_variant(const AttnParams& p) {
  uint32_t code = 0;
  return {kD, kNW, p.bias_mode, small16_packing(p, &code) ? MASK_KEY_LEN_ORDERED : p.mask_mode};
}

const char* flash_small16_name() { return "flash_small16_d64"; }

int flash_small16_variants(FlashVariant* out, int cap) {
  int n = 0;
  for (int bias = BIAS_NONE; bias <= BIAS_RELPOS; ++bias)
    for (int mask = MASK_NONE; mask <= MASK_KEY_LEN_ORDERED; ++mask) {
      if (n < cap) out[n] = {kD, kNW, bias, mask};
      ++n;
    }
  return n;
}

hipError_t launch_flash_small16(const AttnParams& p, hipStream_t stream) {
  uint32_t code;
  bool packed;
  const int64_t n = small16_grid(p, &code, &packed);
  if (p.D != kD || n > 0x7fffffff || !flash_mfma_args_fit(p)) return hipErrorInvalidValue;
  FlashArgs a = flash_args(p, n);  // aux: the key-mask row stride (key-mask calls), the packing codes
  int mask = p.mask_mode;
  if (packed) {
    mask = MASK_KEY_LEN_ORDERED;
    a.aux = (int32_t)code;
  }
  const dim3 grid((unsigned)n);
  switch (p.bias_mode) {
    case BIAS_NONE: return launch_mask16<BIAS_NONE>(a, mask, grid, stream);
    case BIAS_DENSE: return launch_mask16<BIAS_DENSE>(a, mask, grid, stream);
    case BIAS_RELPOS: return launch_mask16<BIAS_RELPOS>(a, mask, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sa
