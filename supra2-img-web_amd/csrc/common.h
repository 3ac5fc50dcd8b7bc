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

// IEEE 754-2019 maximum (a NaN operand gives NaN): one v_maximum3_f32 per two new operands on gfx950,
// where fmaxf also canonicalizes its operands. A NaN score ends in a NaN output either way.
__device__ __forceinline__ float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Exchange with the lane 32 away (v_permlane32_swap): returns {own, partner} in some order, so
// symmetric reductions (max, +) can combine the two results directly.
__device__ __forceinline__ float max_with_partner(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_nan(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_with_partner(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The same over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (v_permlane16_swap pairs lanes l and l ^ 16):
// in the 16x16 MFMA accumulator layout they hold one column in its four row groups. Every one of
// the four lanes gets the same bits (the additions are commutative).
__device__ __forceinline__ float max_over_rows4(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_with_partner(max_nan(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ __forceinline__ float sum_over_rows4(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return sum_with_partner(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Waits until at most N of this wave's vector-memory loads (LDS copies included) are outstanding:
// the older ones have completed, in issue order.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void global_void_t;

// Moves 16 bytes per lane from global memory to LDS: lane i writes lds_wave_base + 16*i.
__device__ __forceinline__ void load_to_lds16(const void* src, float* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)lds_wave_base, 16, 0, 0);
}

// Buffer resource over [base, base + 2 GiB): a scalar descriptor, so a copy's per-lane address is
// a 32-bit offset and a per-block base moves on the scalar unit (no 64-bit VALU address math).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}

// As load_to_lds16, from byte offset `voff` (per lane) + `soff` (uniform) of the buffer `r`.
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t r, unsigned voff, float* lds_wave_base,
                                                unsigned soff = 0) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds_wave_base, 16, voff, soff, 0, 0);
}

}  // namespace sa
