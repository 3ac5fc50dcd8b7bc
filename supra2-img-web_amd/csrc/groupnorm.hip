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
//      and centred sum of squares (a mean pass, then a centred pass over the chunk: the reference's
//      two-pass form, for accuracy);
//   2. apply: each workgroup combines the chunk statistics of every group (Chan et al.'s pairwise
//      update: exact in exact arithmetic, no E[x^2] - E[x]^2 cancellation) into LDS, then normalizes
//      whole pixel rows.

#include "common.h"
#include "kernels.h"

namespace sa {

namespace {

constexpr int kGnRows = 8;  // pixel rows per apply workgroup

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

// part[(g * S + s) * 3 + {0, 1, 2}] = count, mean, centred sum of squares of pixels
// [s * chunk, min((s + 1) * chunk, HW)) of group g.
__global__ __launch_bounds__(256) void groupnorm_stats_kernel(const float* __restrict__ x, float* __restrict__ part,
                                                              int HW, int C, int cg, int S, int chunk) {
  __shared__ float red[4];
  const int g = blockIdx.x / S;
  const int s = blockIdx.x % S;
  const int p0 = s * chunk;
  const int np = max(0, min(chunk, HW - p0));
  const int64_t n = (int64_t)np * cg;
  const float* base = x + (int64_t)p0 * C + g * cg;
  float acc = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 256) acc += base[(i / cg) * C + i % cg];
  const float mean = n > 0 ? block_sum(acc, red) / (float)n : 0.f;
  float m2 = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 256) {
    const float d = base[(i / cg) * C + i % cg] - mean;
    m2 = fmaf(d, d, m2);
  }
  m2 = n > 0 ? block_sum(m2, red) : 0.f;
  if (threadIdx.x == 0) {
    part[3 * blockIdx.x + 0] = (float)n;
    part[3 * blockIdx.x + 1] = mean;
    part[3 * blockIdx.x + 2] = m2;
  }
}

__global__ __launch_bounds__(256) void groupnorm_apply_kernel(const float* __restrict__ x, const float* __restrict__ part,
                                                              const float* __restrict__ gamma,
                                                              const float* __restrict__ beta, float* __restrict__ y,
                                                              int HW, int C, int cg, int G, int S, float eps) {
  extern __shared__ float stats[];  // [G][2]: mean, rstd
  for (int g = threadIdx.x; g < G; g += 256) {
    float n = 0.f, mean = 0.f, m2 = 0.f;
    for (int s = 0; s < S; ++s) {
      const float nb = part[3 * (g * S + s)];
      if (nb == 0.f) continue;
      const float mb = part[3 * (g * S + s) + 1];
      const float n_new = n + nb;
      const float d = mb - mean;
      mean += d * (nb / n_new);
      m2 += part[3 * (g * S + s) + 2] + d * d * (n * nb / n_new);
      n = n_new;
    }
    stats[2 * g] = mean;
    stats[2 * g + 1] = rsqrtf(m2 / n + eps);
  }
  __syncthreads();
  const int p0 = blockIdx.x * kGnRows;
  const int rows = min(kGnRows, HW - p0);
  for (int i = threadIdx.x; i < rows * C; i += 256) {
    const int c = i % C;
    const int g = c / cg;
    const int64_t e = (int64_t)p0 * C + i;
    y[e] = fmaf((x[e] - stats[2 * g]) * stats[2 * g + 1], gamma[c], beta[c]);
  }
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
  const int S = groupnorm_chunks(HW, groups);
  const int chunk = (HW + S - 1) / S;
  hipLaunchKernelGGL(groupnorm_stats_kernel, dim3(groups * S), dim3(256), 0, stream, x, part, HW, C, C / groups, S,
                     chunk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(groupnorm_apply_kernel, dim3((HW + kGnRows - 1) / kGnRows), dim3(256), groups * 2 * sizeof(float),
                     stream, x, part, gamma, beta, y, HW, C, C / groups, groups, S, eps);
  return hipGetLastError();
}

}  // namespace sa
