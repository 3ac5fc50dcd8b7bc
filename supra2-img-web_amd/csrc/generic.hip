// Generic attention kernel: any head dim up to 1024, any alignment, every bias and mask mode.
//
// Covers what the MFMA kernels do not: head dims other than 64/128 and rows that are not
// 16-byte aligned, the cases app/gpu/ops.js:111-112 sends to its unfused path. One workgroup of
// 256 threads handles one query row: keys are processed 256 at a time (one score per thread,
// workgroup max/sum reductions), the running output row is held as ceil(D/256) values per thread.
// Softmax arithmetic is the same as in the MFMA kernels (base 2, running max, zero output when
// every key is masked).
//
// Also holds the dense relative-position bias builder (app/models/t5.js:55-65).

#include "common.h"
#include "kernels.h"

namespace sa {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxPerThread = GENERIC_MAX_D / kThreads;

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Workgroup-wide reductions over 4 waves; `red` holds 4 floats.
__device__ __forceinline__ float block_max(float x, float* red) {
  x = wave_max(x);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = x;
  __syncthreads();
  const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_sum(float x, float* red) {
  x = wave_sum(x);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = x;
  __syncthreads();
  const float r = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kThreads) void generic_kernel(AttnParams p) {
  extern __shared__ float sh[];
  float* q_row = sh;                  // [D]
  float* probs = sh + p.D;            // [256]
  float* red = probs + kThreads;      // [4]

  const int t = threadIdx.x;
  int row = blockIdx.x;
  const int i = row % p.Lq;
  row /= p.Lq;
  const int h = row % p.H;
  const int b = row / p.H;
  const int D = p.D;

  const float* qsrc = p.q + p.q_off + (int64_t)b * p.sq + (int64_t)i * p.ldq + (int64_t)h * D;
  for (int d = t; d < D; d += kThreads) q_row[d] = qsrc[d];

  int kv_len = p.Lk;
  if (p.mask_mode == MASK_KEY_LEN) kv_len = min(max(p.key_len[b], 0), p.Lk);
  const float* kb = p.k + p.k_off + (int64_t)b * p.sk + (int64_t)h * D;
  const float* vb = p.v + p.v_off + (int64_t)b * p.sv + (int64_t)h * D;
  const uint8_t* kmask = p.mask_mode == MASK_KEY_MASK ? p.key_mask + (int64_t)b * p.smask : nullptr;

  float acc[kMaxPerThread];
#pragma unroll
  for (int c = 0; c < kMaxPerThread; ++c) acc[c] = 0.f;
  float m = kMaxSeed, l = 0.f;
  __syncthreads();

  for (int c0 = 0; c0 < kv_len; c0 += kThreads) {
    const int j = c0 + t;
    float u = -INFINITY;
    if (j < kv_len && (kmask == nullptr || kmask[j] != 0)) {
      const float* krow = kb + (int64_t)j * p.ldk;
      float s = 0.f;
      for (int d = 0; d < D; ++d) s = fmaf(q_row[d], krow[d], s);
      float bv = 0.f;
      if (p.bias_mode == BIAS_DENSE) {
        bv = p.bias[(int64_t)b * p.sbias + ((int64_t)h * p.Lq + i) * p.Lk + j] * kLog2e;
      } else if (p.bias_mode == BIAS_RELPOS) {
        int bucket = p.lut[j - i + p.Lq - 1];
        bucket = min(max(bucket, 0), p.num_buckets - 1);
        bv = p.bias[bucket * p.H + h] * kLog2e;
      }
      u = fmaf(s, p.scale_log2, bv);
    }
    const float mb = block_max(u, red);
    const float m_new = fmaxf(m, mb);
    const float alpha = fast_exp2(m - m_new);
    m = m_new;
    const float pj = fast_exp2(u - m_new);
    l = fmaf(l, alpha, block_sum(pj, red));
    probs[t] = pj;
    __syncthreads();
    const int nk = min(kThreads, kv_len - c0);
#pragma unroll
    for (int c = 0; c < kMaxPerThread; ++c) {
      const int d = t + c * kThreads;
      if (d < D) {
        float a = acc[c] * alpha;
        const float* vcol = vb + (int64_t)c0 * p.ldv + d;
        for (int jj = 0; jj < nk; ++jj) a = fmaf(probs[jj], vcol[(int64_t)jj * p.ldv], a);
        acc[c] = a;
      }
    }
    __syncthreads();
  }

  const float inv = l > 0.f ? 1.f / l : 0.f;
  float* dst = p.o + p.o_off + (int64_t)b * p.so + (int64_t)i * p.ldo + (int64_t)h * D;
#pragma unroll
  for (int c = 0; c < kMaxPerThread; ++c) {
    const int d = t + c * kThreads;
    if (d < D) dst[d] = acc[c] * inv;
  }
}

__global__ __launch_bounds__(256) void position_bias_kernel(const float* table, const int32_t* lut, int num_buckets, int H, int Lq,
                                     int Lk, float* out, int64_t n) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // launched with 256 threads (no blockDim read)
  if (idx >= n) return;
  const int j = (int)(idx % Lk);
  const int64_t r = idx / Lk;
  const int i = (int)(r % Lq);
  const int h = (int)(r / Lq);
  int bucket = lut[j - i + Lq - 1];
  bucket = min(max(bucket, 0), num_buckets - 1);
  out[idx] = table[bucket * H + h];
}

}  // namespace

hipError_t launch_generic(const AttnParams& p, hipStream_t stream) {
  const int64_t rows = (int64_t)p.B * p.H * p.Lq;
  if (rows > 0x7fffffff || p.D > GENERIC_MAX_D) return hipErrorInvalidConfiguration;
  const size_t shmem = (size_t)(p.D + kThreads + 4) * sizeof(float);
  hipLaunchKernelGGL(generic_kernel, dim3((unsigned)rows), dim3(kThreads), shmem, stream, p);
  return hipGetLastError();
}

hipError_t launch_position_bias(const float* table, const int32_t* lut, int num_buckets, int H, int Lq, int Lk,
                                float* out, hipStream_t stream) {
  const int64_t n = (int64_t)H * Lq * Lk;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(position_bias_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, table, lut, num_buckets, H,
                     Lq, Lk, out, n);
  return hipGetLastError();
}

}  // namespace sa
