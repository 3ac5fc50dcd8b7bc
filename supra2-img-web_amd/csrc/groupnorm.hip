// GroupNorm over an NHWC image for the SD-VAE mid-block attention (app/models/vae.js:81, the
// reference's groupnormStatsShader + groupnormApplyShader, app/gpu/kernels.js:117-162):
//
//   y[p][c] = (x[p][c] - mean_g) * rstd_g * gamma[c] + beta[c],  g = c / (C / G),
//   mean_g and the biased variance over all pixels p and the C/G channels of group g,
//   rstd_g = 1 / sqrt(var_g + eps).
//
// Two kernels, both spread over the whole chip (one workgroup per group, as the reference runs it,
// would use 32 of 256 CUs):
//   1. statistics: workgroup (g, s) takes a chunk of pixels of group g and writes its count, mean
//      and centred sum of squares;
//   2. apply: each of about two workgroups per CU combines the chunk statistics of every group,
//      then normalizes its slice of the image.
// Both read and write float4 items when the group width, C and the pointers allow it.

#include <algorithm>
#include <type_traits>
#include <stdint.h>

#include "common.h"
#include "kernels.h"

namespace sa {

namespace {

// Sum over the 256 threads of the workgroup: cross-lane shuffles within each wave, then the four
// wave sums through LDS.
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int t = threadIdx.x;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((t & 63) == 0) red[t >> 6] = v;
  __syncthreads();
  const float s = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return s;
}

// One pixel's slice of its group holds cg channels: with VEC (cg, C and the pointers multiples
// of 4 floats / 16 bytes) it is read as cg/4 float4 items, otherwise as cg floats.
template <bool VEC>
__device__ __forceinline__ float item_sum(const float* p) {
  if constexpr (VEC) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
    return (v[0] + v[1]) + (v[2] + v[3]);
  }
  return *p;
}

template <bool VEC>
__device__ __forceinline__ float item_sq(const float* p, float mean) {
  if constexpr (VEC) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) q = fmaf(v[k] - mean, v[k] - mean, q);
    return q;
  }
  const float d = *p - mean;
  return d * d;
}

// part[(g * S + s) * 3 + {0, 1, 2}] = count, mean, centred sum of squares of pixels
// [s * chunk, min((s + 1) * chunk, HW)) of group g (a mean pass, then a centred pass over the
// chunk: the reference's two-pass form, for accuracy).
template <bool VEC>
__global__ __launch_bounds__(256) void groupnorm_stats_kernel(const float* __restrict__ x, float* __restrict__ part,
                                                              int HW, int C, int cg, int S, int chunk) {
  __shared__ float red[4];
  const int g = blockIdx.x / S;
  const int s = blockIdx.x % S;
  const int p0 = s * chunk;
  const int np = max(0, min(chunk, HW - p0));
  const int w = VEC ? cg / 4 : cg;  // items per pixel slice
  const int64_t items = (int64_t)np * w;
  const int64_t n = (int64_t)np * cg;
  const float* base = x + (int64_t)p0 * C + g * cg;
  auto item = [&](int64_t i) {
    const int64_t pix = i / w;
    return base + pix * C + (VEC ? 4 : 1) * (i - pix * w);
  };
  // The thread's first KEEP items stay in registers for the centred pass (a chunk of the VAE
  // image is one item per thread); later ones are read again.
  constexpr int KEEP = 4;
  using Item = typename std::conditional<VEC, f32x4, float>::type;
  Item kept[KEEP];
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < KEEP; ++k) {
    const int64_t i = threadIdx.x + 256 * k;
    if (i < items) {
      kept[k] = *reinterpret_cast<const Item*>(item(i));
      acc += item_sum<VEC>(reinterpret_cast<const float*>(&kept[k]));
    }
  }
  for (int64_t i = threadIdx.x + 256 * KEEP; i < items; i += 256) acc += item_sum<VEC>(item(i));
  const float mean = n > 0 ? block_sum(acc, red) / (float)n : 0.f;
  float m2 = 0.f;
#pragma unroll
  for (int k = 0; k < KEEP; ++k) {
    if (threadIdx.x + 256 * k < items) m2 += item_sq<VEC>(reinterpret_cast<const float*>(&kept[k]), mean);
  }
  for (int64_t i = threadIdx.x + 256 * KEEP; i < items; i += 256) m2 += item_sq<VEC>(item(i), mean);
  m2 = n > 0 ? block_sum(m2, red) : 0.f;
  if (threadIdx.x == 0) {
    part[3 * blockIdx.x + 0] = (float)n;
    part[3 * blockIdx.x + 1] = mean;
    part[3 * blockIdx.x + 2] = m2;
  }
}

// Each workgroup combines the chunk statistics of every group (Chan et al.'s pairwise update:
// exact in exact arithmetic, no E[x^2] - E[x]^2 cancellation) - with STAGED the 3*G*S values are
// first copied to LDS in one coalesced pass, so the per-group loops read LDS instead of making a
// chain of dependent global loads - then normalizes items [i0, i0 + per_block) of the image
// (float4 items when VEC).
template <bool VEC, bool STAGED>
__global__ __launch_bounds__(256) void groupnorm_apply_kernel(const float* __restrict__ x, const float* __restrict__ part,
                                                              const float* __restrict__ gamma,
                                                              const float* __restrict__ beta, float* __restrict__ y,
                                                              int HW, int C, int cg, int G, int S, float eps,
                                                              int64_t per_block) {
  extern __shared__ float sm[];  // [G][2]: mean, rstd; then (STAGED) the [G*S][3] chunk statistics
  float* stats = sm;
  const float* src = part;
  const int w = VEC ? C / 4 : C;  // items per pixel row
  const int64_t total = (int64_t)HW * w;
  const int64_t i0 = (int64_t)blockIdx.x * per_block;
  const int64_t i1 = min(total, i0 + per_block);
  // The thread's first item (and its gamma, beta) is loaded before the statistics are combined, so
  // the two memory round trips overlap instead of running one after the other.
  using Item = typename std::conditional<VEC, f32x4, float>::type;
  const int64_t ifirst = i0 + threadIdx.x;
  Item v0{}, ga0{}, be0{};
  int64_t e0 = 0;
  int c0 = 0;
  if (ifirst < i1) {
    const int64_t row = ifirst / w;
    c0 = (VEC ? 4 : 1) * (int)(ifirst - row * w);
    e0 = row * C + c0;
    v0 = *reinterpret_cast<const Item*>(x + e0);
    ga0 = *reinterpret_cast<const Item*>(gamma + c0);
    be0 = *reinterpret_cast<const Item*>(beta + c0);
  }
  if constexpr (STAGED) {
    float* staged = sm + 2 * G;
    for (int i = threadIdx.x; i < 3 * G * S; i += 256) staged[i] = part[i];
    __syncthreads();
    src = staged;
  }
  for (int g = threadIdx.x; g < G; g += 256) {
    float n = 0.f, mean = 0.f, m2 = 0.f;
    for (int s = 0; s < S; ++s) {
      const float* e = src + 3 * (g * S + s);
      const float nb = e[0];
      if (nb == 0.f) continue;
      const float n_new = n + nb;
      const float d = e[1] - mean;
      mean += d * (nb / n_new);
      m2 += e[2] + d * d * (n * nb / n_new);
      n = n_new;
    }
    stats[2 * g] = mean;
    stats[2 * g + 1] = rsqrtf(m2 / n + eps);
  }
  __syncthreads();
  if (ifirst < i1) {
    const int g = c0 / cg;  // with VEC the four channels share a group (cg % 4 == 0)
    const float mean = stats[2 * g], rstd = stats[2 * g + 1];
    if constexpr (VEC) {
      f32x4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = fmaf((v0[k] - mean) * rstd, ga0[k], be0[k]);
      *reinterpret_cast<f32x4*>(y + e0) = o;
    } else {
      y[e0] = fmaf((v0 - mean) * rstd, ga0, be0);
    }
  }
  for (int64_t i = ifirst + 256; i < i1; i += 256) {
    const int64_t row = i / w;
    const int c = (VEC ? 4 : 1) * (int)(i - row * w);
    const int g = c / cg;  // with VEC the four channels share a group (cg % 4 == 0)
    const float mean = stats[2 * g], rstd = stats[2 * g + 1];
    const int64_t e = row * C + c;
    if constexpr (VEC) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(x + e);
      const f32x4 ga = *reinterpret_cast<const f32x4*>(gamma + c);
      const f32x4 be = *reinterpret_cast<const f32x4*>(beta + c);
      f32x4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = fmaf((v[k] - mean) * rstd, ga[k], be[k]);
      *reinterpret_cast<f32x4*>(y + e) = o;
    } else {
      y[e] = fmaf((x[e] - mean) * rstd, gamma[c], beta[c]);
    }
  }
}

template <bool VEC>
hipError_t launch_vec(const float* x, const float* gamma, const float* beta, float* y, float* part, int HW, int C,
                      int groups, float eps, hipStream_t stream) {
  const int S = groupnorm_chunks(HW, groups);
  const int chunk = (HW + S - 1) / S;
  hipLaunchKernelGGL(groupnorm_stats_kernel<VEC>, dim3(groups * S), dim3(256), 0, stream, x, part, HW, C, C / groups,
                     S, chunk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // about two workgroups per CU of 256-item slices
  const int64_t total = (int64_t)HW * (VEC ? C / 4 : C);
  const int64_t per_block = std::max<int64_t>(256, ((total + 511) / 512 + 255) / 256 * 256);
  const int64_t blocks = (total + per_block - 1) / per_block;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  const size_t staged_bytes = (size_t)(2 * groups + 3 * groups * S) * sizeof(float);
  if (staged_bytes <= 48 * 1024) {
    hipLaunchKernelGGL((groupnorm_apply_kernel<VEC, true>), dim3((unsigned)blocks), dim3(256), staged_bytes, stream, x,
                       part, gamma, beta, y, HW, C, C / groups, groups, S, eps, per_block);
  } else {
    hipLaunchKernelGGL((groupnorm_apply_kernel<VEC, false>), dim3((unsigned)blocks), dim3(256),
                       (size_t)groups * 2 * sizeof(float), stream, x, part, gamma, beta, y, HW, C, C / groups, groups,
                       S, eps, per_block);
  }
  return hipGetLastError();
}

}  // namespace

int groupnorm_chunks(int HW, int groups) {
  // about 512 statistics workgroups, at least 64 pixels each
  const int s = max(1, min((512 + groups - 1) / groups, (HW + 63) / 64));
  return s;
}

hipError_t launch_groupnorm(const float* x, const float* gamma, const float* beta, float* y, float* part, int HW, int C,
                            int groups, float eps, hipStream_t stream) {
  if (groups <= 0 || C % groups != 0 || (int64_t)groups * 2 * 4 > 64 * 1024) return hipErrorInvalidValue;
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool vec = (C / groups) % 4 == 0 && C % 4 == 0 && a16(x) && a16(y) && a16(gamma) && a16(beta);
  return vec ? launch_vec<true>(x, gamma, beta, y, part, HW, C, groups, eps, stream)
             : launch_vec<false>(x, gamma, beta, y, part, HW, C, groups, eps, stream);
}

}  // namespace sa
