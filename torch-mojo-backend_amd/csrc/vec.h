// 4-wide vector loads/stores of f32/bf16/f16 rows as float[4].
#pragma once
#include "common.h"

namespace mi {

template <typename T>
struct Vec4;

template <>
struct Vec4<float> {
  static __device__ __forceinline__ void load(const float* p, float* v) {
    float4 t = *(const float4*)p;
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  }
  static __device__ __forceinline__ void store(float* p, const float* v) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  }
};

template <>
struct Vec4<bf16> {
  static __device__ __forceinline__ void load(const bf16* p, float* v) {
    bf16x4 t = *(const bf16x4*)p;
    v[0] = (float)t[0]; v[1] = (float)t[1]; v[2] = (float)t[2]; v[3] = (float)t[3];
  }
  static __device__ __forceinline__ void store(bf16* p, const float* v) {
    bf16x4 t;
    t[0] = (bf16)v[0]; t[1] = (bf16)v[1]; t[2] = (bf16)v[2]; t[3] = (bf16)v[3];
    *(bf16x4*)p = t;
  }
};

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
template <>
struct Vec4<f16> {
  static __device__ __forceinline__ void load(const f16* p, float* v) {
    f16x4 t = *(const f16x4*)p;
    v[0] = (float)t[0]; v[1] = (float)t[1]; v[2] = (float)t[2]; v[3] = (float)t[3];
  }
  static __device__ __forceinline__ void store(f16* p, const float* v) {
    f16x4 t;
    t[0] = (f16)v[0]; t[1] = (f16)v[1]; t[2] = (f16)v[2]; t[3] = (f16)v[3];
    *(f16x4*)p = t;
  }
};

// Scalar element access
template <typename T>
__device__ __forceinline__ float ldf(const T* p, int64_t i) { return to_f32(p[i]); }
template <typename T>
__device__ __forceinline__ void stf(T* p, int64_t i, float v) { p[i] = from_f32<T>(v); }

}  // namespace mi
