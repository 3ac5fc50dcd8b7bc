// Device helpers shared by the attention kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <float.h>
#include <stdint.h>

namespace sa {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
// Running-max seed: finite, so that (m_old - m_new) is never (-inf) - (-inf) on rows whose keys
// are all masked so far; exp2(-FLT_MAX - x) is 0 for any real x.
constexpr float kMaxSeed = -FLT_MAX;

// Workgroups are handed to the 8 XCDs round-robin (workgroup i runs on XCD i % 8). Remap the
// hardware index so that consecutive logical tiles (the query tiles of one head) run on one XCD
// and share its L2. Bijective on [0, n).
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  constexpr int kXcds = 8;
  const int q = n / kXcds, r = n % kXcds;
  const int xcd = bid % kXcds, local = bid / kXcds;
  return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// Exchange with the lane 32 away (v_permlane32_swap): returns {own, partner} in some order, so
// symmetric reductions (max, +) can combine the two results directly.
__device__ __forceinline__ float max_with_partner(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_with_partner(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace sa
