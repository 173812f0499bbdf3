// Shared device/host helpers for the gfx950 kernel library.
//
// Every exported entry point is `extern "C"`, returns an int status (0 = ok)
// and records a message retrievable with mi355x_last_error().  Nothing here
// allocates device memory or synchronises a stream.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/mi355x_kernels.h"

namespace mi {

// ----------------------------------------------------------------------------
// Error handling
// ----------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define MI_REQUIRE(cond, ...)                                   \
  do {                                                          \
    if (!(cond)) return ::mi::fail(MI355X_EINVAL, __VA_ARGS__); \
  } while (0)

// Check the launch that was just issued.
int check_launch(const char* what);

// ----------------------------------------------------------------------------
// Scalar types
// ----------------------------------------------------------------------------
typedef __bf16 bf16;
typedef _Float16 f16;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }  // RNE
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }

inline size_t dtype_size(int dt) {
  switch (dt) {
    case MI355X_F32: return 4;
    case MI355X_BF16: return 2;
    case MI355X_F16: return 2;
    case MI355X_I64: return 8;
    case MI355X_I32: return 4;
    case MI355X_BOOL: return 1;
    case MI355X_U8: return 1;
    case MI355X_F64: return 8;
    case MI355X_I8: return 1;
    case MI355X_I16: return 2;
  }
  return 0;
}
inline bool is_float_dtype(int dt) {
  return dt == MI355X_F32 || dt == MI355X_BF16 || dt == MI355X_F16 || dt == MI355X_F64;
}

// ----------------------------------------------------------------------------
// Wavefront (64-lane) reductions with cross-lane ops
// ----------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
// max that propagates NaN (torch.max / torch.maximum semantics; fmaxf
// returns the other operand when one is NaN)
__device__ __forceinline__ float nan_max(float a, float b) { return (b > a || b != b) ? b : a; }
// Maximum of V values, NaN if any is NaN: pairs of NaN-propagating maxima,
// which gfx950 issues as one three-input v_maximum3_f32 per two values.
template <int V>
__device__ __forceinline__ float max_nan(const float (&v)[V]) {
  float m = v[0];
  int e = 1;
#pragma unroll
  for (; e + 1 < V; e += 2) m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, v[e]), v[e + 1]);
  if (e < V) m = __builtin_elementwise_maximum(m, v[e]);
  return m;
}
__device__ __forceinline__ float wave_max_nan(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = nan_max(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Block reduction for blockDim.x a multiple of 64 and <= 1024.  `scratch`
// needs blockDim.x/64 floats.  Every thread receives the result.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float r = 0.f;
  for (int i = 0; i < nw; ++i) r += scratch[i];
  return r;
}
__device__ __forceinline__ float block_max(float v, float* scratch) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float r = -INFINITY;
  for (int i = 0; i < nw; ++i) r = fmaxf(r, scratch[i]);
  return r;
}

// ----------------------------------------------------------------------------
// Streaming global accesses
// ----------------------------------------------------------------------------
// Loads/stores with the non-temporal hint, for data a kernel touches once.
// A plain 1 GiB copy moves about 6.2 TB/s with the hint and 5.5 TB/s without
// it; of the library's streaming kernels only AdamW (whose moments and
// parameters are touched once per step) measured faster with it.
// MI_STREAM=0 turns the hint off (for A/B measurements).
#ifndef MI_STREAM
#define MI_STREAM 1
#endif
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// V is 8 bytes or a multiple of 16 bytes (moved as 16-byte words).
template <typename V>
__device__ __forceinline__ V ld_stream(const V* p) {
#if MI_STREAM
  if constexpr (sizeof(V) == 8) {
    return __builtin_bit_cast(V, __builtin_nontemporal_load((const u32x2*)p));
  } else {
    static_assert(sizeof(V) % 16 == 0, "8-byte or 16-byte-multiple accesses");
    struct W {
      u32x4 w[sizeof(V) / 16];
    } r;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(V) / 16); ++i) r.w[i] = __builtin_nontemporal_load((const u32x4*)p + i);
    return __builtin_bit_cast(V, r);
  }
#else
  return *p;
#endif
}
template <typename V>
__device__ __forceinline__ void st_stream(V* p, const V& v) {
#if MI_STREAM
  if constexpr (sizeof(V) == 8) {
    __builtin_nontemporal_store(__builtin_bit_cast(u32x2, v), (u32x2*)p);
  } else {
    static_assert(sizeof(V) % 16 == 0, "8-byte or 16-byte-multiple accesses");
    struct W {
      u32x4 w[sizeof(V) / 16];
    };
    const W r = __builtin_bit_cast(W, v);
#pragma unroll
    for (int i = 0; i < (int)(sizeof(V) / 16); ++i) __builtin_nontemporal_store(r.w[i], (u32x4*)p + i);
  }
#else
  *p = v;
#endif
}

inline unsigned ceil_div(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace mi
