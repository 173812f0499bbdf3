// GELU forward/backward, exact (erf) and tanh forms.
//
// Read-once/write-once elementwise passes: 8 elements per thread per step
// (one 16-byte bf16 access or two 16-byte f32 accesses), computed in f32 and
// rounded once to the storage type, as ATen does for reduced precision.
//   exact: y = 0.5 x (1 + erf(x/sqrt2)),  dy/dx = Phi(x) + x phi(x)
//   tanh:  y = 0.5 x (1 + tanh(k (x + 0.044715 x^3))),  k = sqrt(2/pi)
#include <math.h>

#include "common.h"

namespace mi {
namespace {

constexpr int kThreads = 256;
constexpr float kInvSqrt2 = 0.70710678118654752440f;
constexpr float kInvSqrt2Pi = 0.39894228040143267794f;
constexpr float kSqrt2OverPi = 0.79788456080286535588f;
constexpr float kTanhC = 0.044715f;
constexpr float kNegHalfLog2e = -0.72134752044448170368f;  // -log2(e) / 2

__device__ __forceinline__ float gelu_f(float x, int approx) {
  if (approx) {
    const float inner = kSqrt2OverPi * (x + kTanhC * x * x * x);
    return 0.5f * x * (1.f + tanhf(inner));
  }
  return 0.5f * x * (1.f + erff(x * kInvSqrt2));
}

__device__ __forceinline__ float gelu_grad_f(float dy, float x, int approx) {
  if (approx) {
    const float x2 = x * x;
    const float inner = kSqrt2OverPi * (x + kTanhC * x2 * x);
    const float t = tanhf(inner);
    const float left = 0.5f * x;
    const float right = 1.f + t;
    const float left_d = 0.5f * right;
    const float tanh_d = 1.f - t * t;
    const float inner_d = kSqrt2OverPi * (1.f + 3.f * kTanhC * x2);
    const float right_d = left * tanh_d * inner_d;
    return dy * (left_d + right_d);
  }
  const float cdf = 0.5f * (1.f + erff(x * kInvSqrt2));
  // exp(-x^2/2) as one hardware exp2 (relative error ~1e-6 against expf,
  // far below the bf16/f16 rounding of the result; 0 below 2^-126)
  const float pdf = kInvSqrt2Pi * __builtin_amdgcn_exp2f(kNegHalfLog2e * x * x);
  return dy * (cdf + x * pdf);
}

__device__ __forceinline__ bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <typename T>
struct alignas(16) Pack8 {
  T v[8];
};

template <typename T>
__global__ void __launch_bounds__(kThreads) gelu_fwd_kernel(T* __restrict__ y, const T* __restrict__ x,
                                                            int64_t n, int approx) {
  const int64_t n8 = (aligned16(y) && aligned16(x)) ? n / 8 : 0;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n8; i += stride) {
    Pack8<T> a = ((const Pack8<T>*)x)[i];
    Pack8<T> r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = from_f32<T>(gelu_f(to_f32(a.v[e]), approx));
    ((Pack8<T>*)y)[i] = r;
  }
  for (int64_t i = n8 * 8 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
    y[i] = from_f32<T>(gelu_f(to_f32(x[i]), approx));
}

template <typename T>
__global__ void __launch_bounds__(kThreads) gelu_bwd_kernel(T* __restrict__ dx, const T* __restrict__ dy,
                                                            const T* __restrict__ x, int64_t n,
                                                            int approx) {
  const int64_t n8 = (aligned16(dx) && aligned16(dy) && aligned16(x)) ? n / 8 : 0;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  // two 16-byte accesses of each operand in flight per thread
  for (; i + stride < n8; i += 2 * stride) {
    const Pack8<T> a0 = ((const Pack8<T>*)x)[i], a1 = ((const Pack8<T>*)x)[i + stride];
    const Pack8<T> g0 = ((const Pack8<T>*)dy)[i], g1 = ((const Pack8<T>*)dy)[i + stride];
    Pack8<T> r0, r1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      r0.v[e] = from_f32<T>(gelu_grad_f(to_f32(g0.v[e]), to_f32(a0.v[e]), approx));
      r1.v[e] = from_f32<T>(gelu_grad_f(to_f32(g1.v[e]), to_f32(a1.v[e]), approx));
    }
    ((Pack8<T>*)dx)[i] = r0;
    ((Pack8<T>*)dx)[i + stride] = r1;
  }
  for (; i < n8; i += stride) {
    Pack8<T> a = ((const Pack8<T>*)x)[i];
    Pack8<T> g = ((const Pack8<T>*)dy)[i];
    Pack8<T> r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = from_f32<T>(gelu_grad_f(to_f32(g.v[e]), to_f32(a.v[e]), approx));
    ((Pack8<T>*)dx)[i] = r;
  }
  for (int64_t i = n8 * 8 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
    dx[i] = from_f32<T>(gelu_grad_f(to_f32(dy[i]), to_f32(x[i]), approx));
}

// GeGLU: y = gelu(gate) * up (the Gemma-3-shaped MLP), with gelu(gate)
// rounded to the storage type before the product, as the two ATen ops do.
template <typename T>
__global__ void __launch_bounds__(kThreads) geglu_fwd_kernel(T* __restrict__ y, const T* __restrict__ gate,
                                                             const T* __restrict__ up, int64_t n, int approx) {
  const int64_t n8 = (aligned16(y) && aligned16(gate) && aligned16(up)) ? n / 8 : 0;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n8; i += stride) {
    Pack8<T> g = ((const Pack8<T>*)gate)[i];
    Pack8<T> u = ((const Pack8<T>*)up)[i];
    Pack8<T> r;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      r.v[e] = from_f32<T>(to_f32(from_f32<T>(gelu_f(to_f32(g.v[e]), approx))) * to_f32(u.v[e]));
    ((Pack8<T>*)y)[i] = r;
  }
  for (int64_t i = n8 * 8 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
    y[i] = from_f32<T>(to_f32(from_f32<T>(gelu_f(to_f32(gate[i]), approx))) * to_f32(up[i]));
}

// GeGLU backward, bit-exact with its ATen chain: d_up = grad * a with
// a = gelu(gate) rounded to T, d_gate = gelu_backward(grad * up rounded to
// T, gate); one pass reads grad, gate and up and writes both gradients.
template <typename T>
__global__ void __launch_bounds__(kThreads) geglu_bwd_kernel(T* __restrict__ dgate, T* __restrict__ dup,
                                                             const T* __restrict__ grad, const T* __restrict__ gate,
                                                             const T* __restrict__ up, int64_t n, int approx) {
  auto one = [approx](float gr, float g, float u, float& dg, float& du) {
    const float a = to_f32(from_f32<T>(gelu_f(g, approx)));
    du = gr * a;
    dg = gelu_grad_f(to_f32(from_f32<T>(gr * u)), g, approx);
  };
  const int64_t n8 = (aligned16(dgate) && aligned16(dup) && aligned16(grad) && aligned16(gate) && aligned16(up))
                         ? n / 8 : 0;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n8; i += stride) {
    const Pack8<T> gr = ((const Pack8<T>*)grad)[i], g = ((const Pack8<T>*)gate)[i], u = ((const Pack8<T>*)up)[i];
    Pack8<T> rg, ru;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float dg, du;
      one(to_f32(gr.v[e]), to_f32(g.v[e]), to_f32(u.v[e]), dg, du);
      rg.v[e] = from_f32<T>(dg);
      ru.v[e] = from_f32<T>(du);
    }
    ((Pack8<T>*)dgate)[i] = rg;
    ((Pack8<T>*)dup)[i] = ru;
  }
  for (int64_t i = n8 * 8 + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
    float dg, du;
    one(to_f32(grad[i]), to_f32(gate[i]), to_f32(up[i]), dg, du);
    dgate[i] = from_f32<T>(dg);
    dup[i] = from_f32<T>(du);
  }
}

unsigned grid_for(int64_t n) {
  int64_t b = (n / 8 + kThreads - 1) / kThreads;
  if (b < 1) b = 1;
  if (b > 8192) b = 8192;
  return (unsigned)b;
}


}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi355x_gelu_fwd(void* y, const void* x, int64_t n, int approximate, int dtype,
                               mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0, "mi355x_gelu_fwd: negative size");
  if (n == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MI355X_F32: gelu_fwd_kernel<float><<<grid_for(n), kThreads, 0, s>>>((float*)y, (const float*)x, n, approximate); break;
    case MI355X_BF16: gelu_fwd_kernel<bf16><<<grid_for(n), kThreads, 0, s>>>((bf16*)y, (const bf16*)x, n, approximate); break;
    case MI355X_F16: gelu_fwd_kernel<f16><<<grid_for(n), kThreads, 0, s>>>((f16*)y, (const f16*)x, n, approximate); break;
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_gelu_fwd: unsupported dtype %d", dtype);
  }
  return check_launch("mi355x_gelu_fwd");
}

extern "C" int mi355x_gelu_bwd(void* dx, const void* dy, const void* x, int64_t n, int approximate,
                               int dtype, mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0, "mi355x_gelu_bwd: negative size");
  if (n == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MI355X_F32: gelu_bwd_kernel<float><<<grid_for(n), kThreads, 0, s>>>((float*)dx, (const float*)dy, (const float*)x, n, approximate); break;
    case MI355X_BF16: gelu_bwd_kernel<bf16><<<grid_for(n), kThreads, 0, s>>>((bf16*)dx, (const bf16*)dy, (const bf16*)x, n, approximate); break;
    case MI355X_F16: gelu_bwd_kernel<f16><<<grid_for(n), kThreads, 0, s>>>((f16*)dx, (const f16*)dy, (const f16*)x, n, approximate); break;
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_gelu_bwd: unsupported dtype %d", dtype);
  }
  return check_launch("mi355x_gelu_bwd");
}

extern "C" int mi355x_geglu_fwd(void* y, const void* gate, const void* up, int64_t n, int approximate, int dtype,
                                mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0, "mi355x_geglu_fwd: bad size");
  if (n == 0) return MI355X_OK;
  MI_REQUIRE(y && gate && up, "mi355x_geglu_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MI355X_F32: geglu_fwd_kernel<float><<<grid_for(n), kThreads, 0, s>>>((float*)y, (const float*)gate, (const float*)up, n, approximate); break;
    case MI355X_BF16: geglu_fwd_kernel<bf16><<<grid_for(n), kThreads, 0, s>>>((bf16*)y, (const bf16*)gate, (const bf16*)up, n, approximate); break;
    case MI355X_F16: geglu_fwd_kernel<f16><<<grid_for(n), kThreads, 0, s>>>((f16*)y, (const f16*)gate, (const f16*)up, n, approximate); break;
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_geglu_fwd: unsupported dtype %d", dtype);
  }
  return check_launch("mi355x_geglu_fwd");
}

extern "C" int mi355x_geglu_bwd(void* dgate, void* dup, const void* grad, const void* gate, const void* up, int64_t n,
                                int approximate, int dtype, mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0, "mi355x_geglu_bwd: bad size");
  if (n == 0) return MI355X_OK;
  MI_REQUIRE(dgate && dup && grad && gate && up, "mi355x_geglu_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MI355X_F32:
      geglu_bwd_kernel<float><<<grid_for(n), kThreads, 0, s>>>((float*)dgate, (float*)dup, (const float*)grad,
                                                               (const float*)gate, (const float*)up, n, approximate);
      break;
    case MI355X_BF16:
      geglu_bwd_kernel<bf16><<<grid_for(n), kThreads, 0, s>>>((bf16*)dgate, (bf16*)dup, (const bf16*)grad,
                                                              (const bf16*)gate, (const bf16*)up, n, approximate);
      break;
    case MI355X_F16:
      geglu_bwd_kernel<f16><<<grid_for(n), kThreads, 0, s>>>((f16*)dgate, (f16*)dup, (const f16*)grad,
                                                             (const f16*)gate, (const f16*)up, n, approximate);
      break;
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_geglu_bwd: unsupported dtype %d", dtype);
  }
  return check_launch("mi355x_geglu_bwd");
}
