// Device-side weight decoding from a resident copy of a safetensors data section: toF32 (every dtype
// app/weights.js:28-37 decodes), rows (the embedding gather, :73-83) and the 3x3 conv re-layout of
// uploadConv3 (:105-118). The reference runs these on the CPU per tensor; here they are HBM-bound
// kernels over the bytes already in device memory.
//
// Decoding (bit-exact with the reference's results):
//   F32   bit copy (a Float32Array view, :29)
//   BF16  bits << 16 (bf16ToF32, :6-12)
//   F16   the exact float32 of the half value (f16ToF32, :14-25): normal (1 + m/1024) 2^(e-15),
//         subnormal m 2^-24 with its sign (so -0 stays -0), e = 31 -> +-Inf or NaN; every NaN is the
//         quiet NaN 0x7fc00000 (the bit pattern JS's NaN takes in a Float32Array)
//   F64   rounded to the nearest float32, ties to even (Float32Array.from, :36); NaN -> 0x7fc00000
//   I64   to the nearest double (Number() of the BigInt), then to the nearest float32
//   I32   to the nearest float32; I16, I8, U8, BOOL exactly (BOOL bytes as their value)

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "supra_weights.h"
#include "status.h"

namespace sa {

namespace {

constexpr uint32_t kCanonicalNaN = 0x7fc00000u;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

int dtype_bytes(int32_t dt) {
  switch (dt) {
    case SA_DT_F32: case SA_DT_I32: return 4;
    case SA_DT_F16: case SA_DT_BF16: case SA_DT_I16: return 2;
    case SA_DT_F64: case SA_DT_I64: return 8;
    case SA_DT_I8: case SA_DT_U8: case SA_DT_BOOL: return 1;
    default: return 0;  // not decoded
  }
}

// Raw element type of each decoded dtype.
template <int DT> struct Raw;
template <> struct Raw<SA_DT_F32> { using T = uint32_t; };
template <> struct Raw<SA_DT_F16> { using T = uint16_t; };
template <> struct Raw<SA_DT_BF16> { using T = uint16_t; };
template <> struct Raw<SA_DT_F64> { using T = uint64_t; };
template <> struct Raw<SA_DT_I64> { using T = uint64_t; };
template <> struct Raw<SA_DT_I32> { using T = uint32_t; };
template <> struct Raw<SA_DT_I16> { using T = uint16_t; };
template <> struct Raw<SA_DT_I8> { using T = uint8_t; };
template <> struct Raw<SA_DT_U8> { using T = uint8_t; };
template <> struct Raw<SA_DT_BOOL> { using T = uint8_t; };

__device__ __forceinline__ float half_to_f32(uint32_t h) {
  const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
  if (e == 31u) return __uint_as_float(m ? kCanonicalNaN : ((s << 31) | 0x7f800000u));
  if (e == 0u) {
    const float v = (float)m * 0x1p-24f;  // exact: m < 2^10
    return s ? -v : v;
  }
  return __uint_as_float((s << 31) | ((e + 112u) << 23) | (m << 13));
}

template <int DT>
__device__ __forceinline__ float decode(typename Raw<DT>::T r) {
  if constexpr (DT == SA_DT_F32) return __uint_as_float(r);
  if constexpr (DT == SA_DT_BF16) return __uint_as_float((uint32_t)r << 16);
  if constexpr (DT == SA_DT_F16) return half_to_f32(r);
  if constexpr (DT == SA_DT_F64) {
    const double d = __longlong_as_double((long long)r);
    return d != d ? __uint_as_float(kCanonicalNaN) : (float)d;
  }
  if constexpr (DT == SA_DT_I64) return (float)(double)(int64_t)r;
  if constexpr (DT == SA_DT_I32) return (float)(int32_t)r;
  if constexpr (DT == SA_DT_I16) return (float)(int16_t)r;
  if constexpr (DT == SA_DT_I8) return (float)(int8_t)r;
  if constexpr (DT == SA_DT_U8 || DT == SA_DT_BOOL) return (float)r;
}

// Little-endian element assembled from single bytes (any source alignment).
template <int DT>
__device__ __forceinline__ typename Raw<DT>::T load_bytes(const uint8_t* p) {
  using T = typename Raw<DT>::T;
  T v = 0;
#pragma unroll
  for (int b = 0; b < (int)sizeof(T); ++b) v |= (T)p[b] << (8 * b);
  return v;
}

constexpr int kThreads = 256;

// Quads (4 consecutive elements, one float4 of output) per thread and pass: 64 source bytes in
// flight per lane whatever the element size.
template <int DT>
constexpr int kQuadsPerThread = 16 / (int)sizeof(typename Raw<DT>::T);

// Four consecutive elements from p (element-aligned); VEC: p is aligned to min(4 * sizeof(T), 16)
// bytes, so the four come in one (two, for 8-byte types) vector loads.
template <int DT, bool VEC>
__device__ __forceinline__ void load_quad(const typename Raw<DT>::T* p, typename Raw<DT>::T (&e)[4]) {
  using T = typename Raw<DT>::T;
  if constexpr (VEC && sizeof(T) == 1) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
    __builtin_memcpy(e, &v, 4);
  } else if constexpr (VEC && sizeof(T) == 2) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    __builtin_memcpy(e, &v, 8);
  } else if constexpr (VEC && sizeof(T) == 4) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    __builtin_memcpy(e, &v, 16);
  } else if constexpr (VEC && sizeof(T) == 8) {
    const u32x4 a = reinterpret_cast<const u32x4*>(p)[0];
    const u32x4 b = reinterpret_cast<const u32x4*>(p)[1];
    __builtin_memcpy(e, &a, 16);
    __builtin_memcpy(e + 2, &b, 16);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = p[i];
  }
}

// dst[i] = decode(src[i]) for i < n. Elements [0, head) and [head + 4*quads, n) one per thread;
// the middle as quads: lane j of a pass writes output float4 j, so every store instruction of a
// wave covers 1 KiB of whole lines (dst + head is 16-byte aligned), and every load instruction
// reads the matching contiguous source bytes. nthreads: the grid's threads, an argument rather than
// gridDim (reading the grid size makes the runtime pass its hidden arguments, and launches start later).
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) void to_f32_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                          int64_t n, int64_t head, int64_t quads, int64_t nthreads) {
  using T = typename Raw<DT>::T;
  constexpr int U = kQuadsPerThread<DT>;
  const int64_t tid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const T* s = reinterpret_cast<const T*>(src);
  const int64_t tail0 = head + quads * 4;
  for (int64_t i = tid; i < head; i += nthreads) dst[i] = decode<DT>(s[i]);
  for (int64_t i = tail0 + tid; i < n; i += nthreads) dst[i] = decode<DT>(s[i]);

  const T* sq = s + head;
  f32x4* dq = reinterpret_cast<f32x4*>(dst + head);
  for (int64_t base = tid; base < quads; base += nthreads * U) {
    T e[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = base + (int64_t)u * nthreads;
      if (k < quads) load_quad<DT, VEC>(sq + 4 * k, e[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = base + (int64_t)u * nthreads;
      if (k < quads) dq[k] = f32x4{decode<DT>(e[u][0]), decode<DT>(e[u][1]), decode<DT>(e[u][2]), decode<DT>(e[u][3])};
    }
  }
}

// Any source alignment: every element assembled from bytes.
template <int DT>
__global__ __launch_bounds__(kThreads) void to_f32_bytes_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                                int64_t n, int64_t nthreads) {
  using T = typename Raw<DT>::T;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += nthreads)
    dst[i] = decode<DT>(load_bytes<DT>(src + i * (int64_t)sizeof(T)));
}

// Embedding rows: workgroup (r, c) decodes columns [c*kThreads*4, ...) of output row r.
template <int DT>
__global__ __launch_bounds__(kThreads) void rows_kernel(const uint8_t* __restrict__ table, int64_t rows, int64_t dim,
                                                        const int32_t* __restrict__ ids, float* __restrict__ dst) {
  using T = typename Raw<DT>::T;
  const int64_t r = blockIdx.y;
  const int32_t id = ids[r];
  const bool valid = id >= 0 && (int64_t)id < rows;
  const uint8_t* row = table + (valid ? (int64_t)id : 0) * dim * (int64_t)sizeof(T);
  float* out = dst + r * dim;
  const int64_t c0 = (int64_t)blockIdx.x * kThreads * 4 + threadIdx.x;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t c = c0 + (int64_t)u * kThreads;
    if (c < dim) out[c] = valid ? decode<DT>(load_bytes<DT>(row + c * (int64_t)sizeof(T))) : 0.f;
  }
}

// uploadConv3 re-layout: workgroup (c, o) moves input channels [c*kConvCh, (c+1)*kConvCh) of
// output channel o. The 9*kConvCh source elements are contiguous: they are decoded into LDS in
// order, then written as 9 rows of the [3, 3, cin_pad] destination (stride-9 LDS reads: 9 is odd,
// so the 64 lanes hit distinct banks).
constexpr int kConvCh = 256;

template <int DT>
__global__ __launch_bounds__(kThreads) void conv3_pack_kernel(const uint8_t* __restrict__ w, int cin, int cin_pad,
                                                              float* __restrict__ dst) {
  using T = typename Raw<DT>::T;
  __shared__ float tile[kConvCh * 9];
  const int o = blockIdx.y;
  const int i0 = blockIdx.x * kConvCh;
  const int nch = min(kConvCh, cin - i0);  // source channels in this chunk (may be <= 0: padding only)
  const uint8_t* src = w + ((int64_t)o * cin + i0) * 9 * (int64_t)sizeof(T);
  for (int k = threadIdx.x; k < nch * 9; k += kThreads) tile[k] = decode<DT>(load_bytes<DT>(src + (int64_t)k * sizeof(T)));
  __syncthreads();
  const int span = min(kConvCh, cin_pad - i0);
  for (int k = threadIdx.x; k < 9 * span; k += kThreads) {
    const int t = k / span, i = k % span;
    dst[((int64_t)o * 9 + t) * cin_pad + i0 + i] = i < nch ? tile[i * 9 + t] : 0.f;
  }
}

int grid_for(int64_t work_items) {
  const int64_t g = (work_items + kThreads - 1) / kThreads;
  return (int)(g < 1 ? 1 : (g > 8192 ? 8192 : g));
}

template <int DT>
hipError_t launch_to_f32(const uint8_t* src, float* dst, int64_t n, hipStream_t stream) {
  using T = typename Raw<DT>::T;
  if ((uintptr_t)src % sizeof(T) != 0) {
    const unsigned g = grid_for(n);
    hipLaunchKernelGGL(to_f32_bytes_kernel<DT>, dim3(g), dim3(kThreads), 0, stream, src, dst, n, (int64_t)g * kThreads);
    return hipGetLastError();
  }
  int64_t head = (int64_t)((16 - (uintptr_t)dst % 16) % 16) / 4;  // dst + head is 16-byte aligned
  if (head > n) head = n;
  const int64_t quads = (n - head) / 4;
  const uintptr_t vec_align = sizeof(T) * 4 < 16 ? sizeof(T) * 4 : 16;
  const bool vec = ((uintptr_t)(src + head * (int64_t)sizeof(T)) % vec_align) == 0;
  constexpr int64_t U = kQuadsPerThread<DT>;
  const int64_t singles = n - quads * 4;  // head and tail elements
  const int64_t threads = (quads + U - 1) / U > singles ? (quads + U - 1) / U : singles;
  int64_t blocks = (threads + kThreads - 1) / kThreads;
  if (blocks < 1) blocks = 1;
  if (blocks > (1 << 30)) blocks = 1 << 30;  // the loops stride over the rest
  const int64_t nthreads = (int64_t)blocks * kThreads;
  if (vec)
    hipLaunchKernelGGL((to_f32_kernel<DT, true>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, src, dst, n, head, quads,
                       nthreads);
  else
    hipLaunchKernelGGL((to_f32_kernel<DT, false>), dim3((unsigned)blocks), dim3(kThreads), 0, stream, src, dst, n, head,
                       quads, nthreads);
  return hipGetLastError();
}

// Runs F<DT>::run(args...) for the decoded dtype `dt`.
template <template <int> class F, class... A>
hipError_t dispatch(int32_t dt, A... args) {
  switch (dt) {
    case SA_DT_F32: return F<SA_DT_F32>::run(args...);
    case SA_DT_F16: return F<SA_DT_F16>::run(args...);
    case SA_DT_BF16: return F<SA_DT_BF16>::run(args...);
    case SA_DT_F64: return F<SA_DT_F64>::run(args...);
    case SA_DT_I64: return F<SA_DT_I64>::run(args...);
    case SA_DT_I32: return F<SA_DT_I32>::run(args...);
    case SA_DT_I16: return F<SA_DT_I16>::run(args...);
    case SA_DT_I8: return F<SA_DT_I8>::run(args...);
    case SA_DT_U8: return F<SA_DT_U8>::run(args...);
    case SA_DT_BOOL: return F<SA_DT_BOOL>::run(args...);
    default: return hipErrorInvalidValue;
  }
}

template <int DT> struct ToF32 {
  static hipError_t run(const uint8_t* src, float* dst, int64_t n, hipStream_t s) { return launch_to_f32<DT>(src, dst, n, s); }
};

template <int DT> struct Rows {
  static hipError_t run(const uint8_t* table, int64_t rows, int64_t dim, const int32_t* ids, int64_t n_ids, float* dst,
                        hipStream_t s) {
    const dim3 grid((unsigned)((dim + kThreads * 4 - 1) / (kThreads * 4)), (unsigned)n_ids);
    hipLaunchKernelGGL(rows_kernel<DT>, grid, dim3(kThreads), 0, s, table, rows, dim, ids, dst);
    return hipGetLastError();
  }
};

template <int DT> struct Conv3 {
  static hipError_t run(const uint8_t* w, int cout, int cin, int cin_pad, float* dst, hipStream_t s) {
    const dim3 grid((unsigned)((cin_pad + kConvCh - 1) / kConvCh), (unsigned)cout);
    hipLaunchKernelGGL(conv3_pack_kernel<DT>, grid, dim3(kThreads), 0, s, w, cin, cin_pad, dst);
    return hipGetLastError();
  }
};

int check_dtype(int32_t dtype) {
  if (dtype_bytes(dtype) == 0) {
    if (dtype >= SA_DT_U16 && dtype <= SA_DT_F8_E5M2) return fail(SA_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
    return fail(SA_ERR_INVALID, "unknown dtype %d", dtype);
  }
  return SA_OK;
}

bool overlap(const void* a, int64_t abytes, const void* b, int64_t bbytes) {
  const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
  return a0 < b0 + (uintptr_t)bbytes && b0 < a0 + (uintptr_t)abytes;
}

}  // namespace

}  // namespace sa

using sa::fail;
using sa::ok;

extern "C" {

int sa_to_f32(const void* src, int32_t dtype, int64_t n, float* dst, void* stream) {
  int rc = sa::check_dtype(dtype);
  if (rc != SA_OK) return rc;
  if (n < 0) return fail(SA_ERR_INVALID, "n = %lld", (long long)n);
  if (n == 0) return ok();
  if (!src || !dst) return fail(SA_ERR_INVALID, "NULL pointer");
  if ((uintptr_t)dst % 4 != 0) return fail(SA_ERR_INVALID, "dst is not 4-byte aligned");
  if (sa::overlap(src, n * sa::dtype_bytes(dtype), dst, n * 4)) return fail(SA_ERR_ALIAS, "dst overlaps src");
  const hipError_t e = sa::dispatch<sa::ToF32>(dtype, static_cast<const uint8_t*>(src), dst, n, (hipStream_t)stream);
  return e == hipSuccess ? ok() : sa::hip_fail(e, "to_f32");
}

int sa_rows_f32(const void* table, int32_t dtype, int64_t rows, int64_t dim, const int32_t* ids, int64_t n_ids, float* dst,
                void* stream) {
  int rc = sa::check_dtype(dtype);
  if (rc != SA_OK) return rc;
  if (rows < 0 || dim < 0 || n_ids < 0) return fail(SA_ERR_INVALID, "negative size");
  if (n_ids == 0 || dim == 0) return ok();
  if (!table && rows > 0) return fail(SA_ERR_INVALID, "table is NULL");
  if (!ids || !dst) return fail(SA_ERR_INVALID, "NULL pointer");
  if ((uintptr_t)dst % 4 != 0) return fail(SA_ERR_INVALID, "dst is not 4-byte aligned");
  if (n_ids > 65535) return fail(SA_ERR_UNSUPPORTED, "%lld ids (at most 65535 per call)", (long long)n_ids);
  if ((dim + 1023) / 1024 > 0x7fffffff) return fail(SA_ERR_UNSUPPORTED, "dim %lld", (long long)dim);
  if (sa::overlap(dst, n_ids * dim * 4, ids, n_ids * 4) ||
      (rows > 0 && sa::overlap(dst, n_ids * dim * 4, table, rows * dim * sa::dtype_bytes(dtype))))
    return fail(SA_ERR_ALIAS, "dst overlaps the table or the ids");
  const hipError_t e = sa::dispatch<sa::Rows>(dtype, static_cast<const uint8_t*>(table), rows, dim, ids, n_ids, dst,
                                              (hipStream_t)stream);
  return e == hipSuccess ? ok() : sa::hip_fail(e, "rows_f32");
}

int sa_conv3_pack_f32(const void* w, int32_t dtype, int32_t cout, int32_t cin, int32_t cin_pad, float* dst, void* stream) {
  int rc = sa::check_dtype(dtype);
  if (rc != SA_OK) return rc;
  if (cout < 0 || cin < 0 || cin_pad < 0) return fail(SA_ERR_INVALID, "negative size");
  const int cp = cin_pad ? cin_pad : cin;
  if (cp < cin) return fail(SA_ERR_INVALID, "cin_pad %d < cin %d", cin_pad, cin);
  if (cout == 0 || cp == 0) return ok();
  if (!dst || (!w && cin > 0)) return fail(SA_ERR_INVALID, "NULL pointer");
  if ((uintptr_t)dst % 4 != 0) return fail(SA_ERR_INVALID, "dst is not 4-byte aligned");
  if (cout > 65535) return fail(SA_ERR_UNSUPPORTED, "cout %d (at most 65535)", cout);
  if (cin > 0 && sa::overlap(dst, (int64_t)cout * 9 * cp * 4, w, (int64_t)cout * cin * 9 * sa::dtype_bytes(dtype)))
    return fail(SA_ERR_ALIAS, "dst overlaps w");
  const hipError_t e = sa::dispatch<sa::Conv3>(dtype, static_cast<const uint8_t*>(w), (int)cout, (int)cin, cp, dst,
                                               (hipStream_t)stream);
  return e == hipSuccess ? ok() : sa::hip_fail(e, "conv3_pack_f32");
}

}  // extern "C"
