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
constexpr float kLog2eF = 1.44269504088896340736f;
// 8-element packs per thread per trip, their loads issued together: two for
// the forward (one input stream, more math per byte moved), one where two
// input streams are read (measured at [16384, 3072] bf16)
constexpr int kUFwd = 2, kUBwd = 1;

// erfc(a) for a >= 0, branch-free, after the Chebyshev-fitted form of
// Numerical Recipes (Press et al., 2nd ed., section 6.2, "erfcc"):
//   erfc(a) = t exp(-a^2 + P(t)),  t = 1 / (1 + a/2),
// P of degree 9, relative error below 1.2e-7 for every a >= 0, so the
// far tail keeps its relative accuracy.  One reciprocal and one exp2.
__device__ __forceinline__ float erfc_nr(float a) {
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, a, 1.f));
  float q = fmaf(0.17087277f, t, -0.82215223f);
  q = fmaf(q, t, 1.48851587f);
  q = fmaf(q, t, -1.13520398f);
  q = fmaf(q, t, 0.27886807f);
  q = fmaf(q, t, -0.18628806f);
  q = fmaf(q, t, 0.09678418f);
  q = fmaf(q, t, 0.37409196f);
  q = fmaf(q, t, 1.00002368f);
  q = fmaf(q, t, -1.26551223f);
  return t * __builtin_amdgcn_exp2f(kLog2eF * fmaf(-a, a, q));  // 0 once a^2 passes ~88
}

// Phi(x) = erfc(-x / sqrt2) / 2, taken from the erfc of |x| / sqrt2 on
// either side, so that Phi of a negative x is never 1 + erf(x / sqrt2)
// with its cancellation.
__device__ __forceinline__ float phi_fast(float x) {
  const float h = 0.5f * erfc_nr(fabsf(x) * kInvSqrt2);
  return x < 0.f ? h : 1.f - h;
}

// sigmoid(2u) = (1 + tanh(u)) / 2 with e = exp(-2u) (held below 1e30, so
// that 1 - s = e s stays finite), branch-free: exp2 saturating to 0 or the
// bound gives s = 1 or ~0.
__device__ __forceinline__ float sigmoid2(float u, float& e) {
  e = fminf(__builtin_amdgcn_exp2f(-2.f * kLog2eF * u), 1e30f);
  return __builtin_amdgcn_rcpf(1.f + e);
}

// F (fast): the branch-free forms above, for 16-bit storage types, whose
// rounding hides their error; f32 storage keeps the libm erf/tanh in the
// textbook forms 0.5 x (1 + erf), 0.5 x (1 + tanh), as ATen evaluates them,
// so an f32 run tracks an f32 reference step for step.
template <bool A, bool F>
__device__ __forceinline__ float gelu_f(float x) {
  if constexpr (A) {
    const float inner = kSqrt2OverPi * (x + kTanhC * x * x * x);
    if constexpr (F) {
      float e;
      return x * sigmoid2(inner, e);  // 0.5 x (1 + tanh(inner))
    } else {
      return 0.5f * x * (1.f + tanhf(inner));
    }
  } else if constexpr (F) {
    return x * phi_fast(x);
  } else {
    return 0.5f * x * (1.f + erff(x * kInvSqrt2));
  }
}

template <bool A, bool F>
__device__ __forceinline__ float gelu_grad_f(float dy, float x) {
  if constexpr (A) {
    const float x2 = x * x;
    const float inner = kSqrt2OverPi * (x + kTanhC * x2 * x);
    const float inner_d = kSqrt2OverPi * (1.f + 3.f * kTanhC * x2);
    if constexpr (F) {
      // with s = (1 + t) / 2:  d/dx = s + 2 x s (1 - s) inner'
      float e;
      const float s = sigmoid2(inner, e);
      return dy * fmaf(2.f * x * s * (e * s), inner_d, s);
    } else {
      const float t = tanhf(inner);
      const float left = 0.5f * x;
      const float right = 1.f + t;
      const float left_d = 0.5f * right;
      const float tanh_d = 1.f - t * t;
      const float right_d = left * tanh_d * inner_d;
      return dy * (left_d + right_d);
    }
  } else {
    // Phi(x) + x phi(x), phi(x) = exp(-x^2 / 2) / sqrt(2 pi), the exp as one
    // hardware exp2 (relative error ~1e-6 against expf; 0 below 2^-126)
    const float cdf = F ? phi_fast(x) : 0.5f * (1.f + erff(x * kInvSqrt2));
    const float e = __builtin_amdgcn_exp2f(-0.5f * kLog2eF * x * x);
    return dy * fmaf(x * kInvSqrt2Pi, e, cdf);
  }
}

template <typename T>
constexpr bool kFast = sizeof(T) < 4;

__device__ __forceinline__ bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <typename T>
struct alignas(16) Pack8 {
  T v[8];
};

template <typename T>
__device__ __forceinline__ Pack8<T> ld8(const T* p, int64_t i) { return ((const Pack8<T>*)p)[i]; }
template <typename T>
__device__ __forceinline__ void st8(T* p, int64_t i, const Pack8<T>& v) { ((Pack8<T>*)p)[i] = v; }

// Every kernel below walks its 8-element packs in trips of kUFwd or kUBwd packs per
// thread (the trip's loads all issued before its math), then single packs,
// then the elements past the last whole pack (or every element when an
// operand is not 16-byte aligned).
template <typename T, bool A>
__global__ void __launch_bounds__(kThreads) gelu_fwd_kernel(T* __restrict__ y, const T* __restrict__ x, int64_t n) {
  const int64_t n8 = (aligned16(y) && aligned16(x)) ? n / 8 : 0;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  for (; i + (kUFwd - 1) * stride < n8; i += kUFwd * stride) {
    Pack8<T> a[kUFwd];
#pragma unroll
    for (int u = 0; u < kUFwd; ++u) a[u] = ld8(x, i + u * stride);
#pragma unroll
    for (int u = 0; u < kUFwd; ++u) {
      Pack8<T> r;
#pragma unroll
      for (int e = 0; e < 8; ++e) r.v[e] = from_f32<T>(gelu_f<A, kFast<T>>(to_f32(a[u].v[e])));
      st8(y, i + u * stride, r);
    }
  }
  for (; i < n8; i += stride) {
    const Pack8<T> a = ld8(x, i);
    Pack8<T> r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = from_f32<T>(gelu_f<A, kFast<T>>(to_f32(a.v[e])));
    st8(y, i, r);
  }
  for (int64_t j = n8 * 8 + (int64_t)blockIdx.x * kThreads + threadIdx.x; j < n; j += stride)
    y[j] = from_f32<T>(gelu_f<A, kFast<T>>(to_f32(x[j])));
}

template <typename T, bool A>
__global__ void __launch_bounds__(kThreads) gelu_bwd_kernel(T* __restrict__ dx, const T* __restrict__ dy,
                                                            const T* __restrict__ x, int64_t n) {
  const int64_t n8 = (aligned16(dx) && aligned16(dy) && aligned16(x)) ? n / 8 : 0;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  for (; i + (kUBwd - 1) * stride < n8; i += kUBwd * stride) {
    Pack8<T> a[kUBwd], g[kUBwd];
#pragma unroll
    for (int u = 0; u < kUBwd; ++u) {
      a[u] = ld8(x, i + u * stride);
      g[u] = ld8(dy, i + u * stride);
    }
#pragma unroll
    for (int u = 0; u < kUBwd; ++u) {
      Pack8<T> r;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        r.v[e] = from_f32<T>(gelu_grad_f<A, kFast<T>>(to_f32(g[u].v[e]), to_f32(a[u].v[e])));
      st8(dx, i + u * stride, r);
    }
  }
  for (; i < n8; i += stride) {
    const Pack8<T> a = ld8(x, i), g = ld8(dy, i);
    Pack8<T> r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = from_f32<T>(gelu_grad_f<A, kFast<T>>(to_f32(g.v[e]), to_f32(a.v[e])));
    st8(dx, i, r);
  }
  for (int64_t j = n8 * 8 + (int64_t)blockIdx.x * kThreads + threadIdx.x; j < n; j += stride)
    dx[j] = from_f32<T>(gelu_grad_f<A, kFast<T>>(to_f32(dy[j]), to_f32(x[j])));
}

// GeGLU: y = gelu(gate) * up (the Gemma-3-shaped MLP), with gelu(gate)
// rounded to the storage type before the product, as the two ATen ops do.
template <typename T, bool A>
__device__ __forceinline__ float geglu_f(float g, float u) {
  return to_f32(from_f32<T>(gelu_f<A, kFast<T>>(g))) * u;
}

template <typename T, bool A>
__global__ void __launch_bounds__(kThreads) geglu_fwd_kernel(T* __restrict__ y, const T* __restrict__ gate,
                                                             const T* __restrict__ up, int64_t n) {
  const int64_t n8 = (aligned16(y) && aligned16(gate) && aligned16(up)) ? n / 8 : 0;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  for (; i + (kUBwd - 1) * stride < n8; i += kUBwd * stride) {
    Pack8<T> g[kUBwd], u8[kUBwd];
#pragma unroll
    for (int u = 0; u < kUBwd; ++u) {
      g[u] = ld8(gate, i + u * stride);
      u8[u] = ld8(up, i + u * stride);
    }
#pragma unroll
    for (int u = 0; u < kUBwd; ++u) {
      Pack8<T> r;
#pragma unroll
      for (int e = 0; e < 8; ++e) r.v[e] = from_f32<T>(geglu_f<T, A>(to_f32(g[u].v[e]), to_f32(u8[u].v[e])));
      st8(y, i + u * stride, r);
    }
  }
  for (; i < n8; i += stride) {
    const Pack8<T> g = ld8(gate, i), u8 = ld8(up, i);
    Pack8<T> r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = from_f32<T>(geglu_f<T, A>(to_f32(g.v[e]), to_f32(u8.v[e])));
    st8(y, i, r);
  }
  for (int64_t j = n8 * 8 + (int64_t)blockIdx.x * kThreads + threadIdx.x; j < n; j += stride)
    y[j] = from_f32<T>(geglu_f<T, A>(to_f32(gate[j]), to_f32(up[j])));
}

// GeGLU backward, bit-exact with its ATen chain: d_up = grad * a with
// a = gelu(gate) rounded to T, d_gate = gelu_backward(grad * up rounded to
// T, gate); one pass reads grad, gate and up and writes both gradients.
template <typename T, bool A>
__device__ __forceinline__ void geglu_grad(float gr, float g, float u, T& dg, T& du) {
  du = from_f32<T>(gr * to_f32(from_f32<T>(gelu_f<A, kFast<T>>(g))));
  dg = from_f32<T>(gelu_grad_f<A, kFast<T>>(to_f32(from_f32<T>(gr * u)), g));
}

template <typename T, bool A>
__global__ void __launch_bounds__(kThreads) geglu_bwd_kernel(T* __restrict__ dgate, T* __restrict__ dup,
                                                             const T* __restrict__ grad, const T* __restrict__ gate,
                                                             const T* __restrict__ up, int64_t n) {
  const int64_t n8 = (aligned16(dgate) && aligned16(dup) && aligned16(grad) && aligned16(gate) && aligned16(up))
                         ? n / 8 : 0;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n8; i += stride) {
    const Pack8<T> gr = ld8(grad, i), g = ld8(gate, i), u = ld8(up, i);
    Pack8<T> rg, ru;
#pragma unroll
    for (int e = 0; e < 8; ++e) geglu_grad<T, A>(to_f32(gr.v[e]), to_f32(g.v[e]), to_f32(u.v[e]), rg.v[e], ru.v[e]);
    st8(dgate, i, rg);
    st8(dup, i, ru);
  }
  for (int64_t j = n8 * 8 + (int64_t)blockIdx.x * kThreads + threadIdx.x; j < n; j += stride)
    geglu_grad<T, A>(to_f32(grad[j]), to_f32(gate[j]), to_f32(up[j]), dgate[j], dup[j]);
}

// One trip of u packs per thread where the grid allows (at most 65535
// blocks; larger inputs loop).
unsigned grid_for(int64_t n, int u) {
  int64_t b = (n / 8 + kThreads * u - 1) / (kThreads * u);
  if (b < 1) b = 1;
  if (b > 65535) b = 65535;
  return (unsigned)b;
}

}  // namespace
}  // namespace mi

using namespace mi;

namespace {
// Calls go(T{}) with T the storage type of the dtype code, then checks the launch.
template <typename F>
int act_dispatch(const char* name, int dtype, F&& go) {
  switch (dtype) {
    case MI355X_F32: go(float{}); break;
    case MI355X_BF16: go(bf16{}); break;
    case MI355X_F16: go(f16{}); break;
    default: return fail(MI355X_EUNSUPPORTED, "%s: unsupported dtype %d", name, dtype);
  }
  return check_launch(name);
}
}  // namespace

extern "C" int mi355x_gelu_fwd(void* y, const void* x, int64_t n, int approximate, int dtype,
                               mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0, "mi355x_gelu_fwd: negative size");
  if (n == 0) return MI355X_OK;
  return act_dispatch("mi355x_gelu_fwd", dtype, [&](auto tag) {
    using T = decltype(tag);
    const unsigned g = grid_for(n, kUFwd);
    hipStream_t s = (hipStream_t)stream;
    if (approximate) gelu_fwd_kernel<T, true><<<g, kThreads, 0, s>>>((T*)y, (const T*)x, n);
    else gelu_fwd_kernel<T, false><<<g, kThreads, 0, s>>>((T*)y, (const T*)x, n);
  });
}

extern "C" int mi355x_gelu_bwd(void* dx, const void* dy, const void* x, int64_t n, int approximate,
                               int dtype, mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0, "mi355x_gelu_bwd: negative size");
  if (n == 0) return MI355X_OK;
  return act_dispatch("mi355x_gelu_bwd", dtype, [&](auto tag) {
    using T = decltype(tag);
    const unsigned g = grid_for(n, kUBwd);
    hipStream_t s = (hipStream_t)stream;
    if (approximate) gelu_bwd_kernel<T, true><<<g, kThreads, 0, s>>>((T*)dx, (const T*)dy, (const T*)x, n);
    else gelu_bwd_kernel<T, false><<<g, kThreads, 0, s>>>((T*)dx, (const T*)dy, (const T*)x, n);
  });
}

extern "C" int mi355x_geglu_fwd(void* y, const void* gate, const void* up, int64_t n, int approximate, int dtype,
                                mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0, "mi355x_geglu_fwd: bad size");
  if (n == 0) return MI355X_OK;
  MI_REQUIRE(y && gate && up, "mi355x_geglu_fwd: null pointer");
  return act_dispatch("mi355x_geglu_fwd", dtype, [&](auto tag) {
    using T = decltype(tag);
    const unsigned g = grid_for(n, kUBwd);
    hipStream_t s = (hipStream_t)stream;
    if (approximate) geglu_fwd_kernel<T, true><<<g, kThreads, 0, s>>>((T*)y, (const T*)gate, (const T*)up, n);
    else geglu_fwd_kernel<T, false><<<g, kThreads, 0, s>>>((T*)y, (const T*)gate, (const T*)up, n);
  });
}

extern "C" int mi355x_geglu_bwd(void* dgate, void* dup, const void* grad, const void* gate, const void* up, int64_t n,
                                int approximate, int dtype, mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0, "mi355x_geglu_bwd: bad size");
  if (n == 0) return MI355X_OK;
  MI_REQUIRE(dgate && dup && grad && gate && up, "mi355x_geglu_bwd: null pointer");
  return act_dispatch("mi355x_geglu_bwd", dtype, [&](auto tag) {
    using T = decltype(tag);
    const unsigned g = grid_for(n, kUBwd);
    hipStream_t s = (hipStream_t)stream;
    if (approximate) geglu_bwd_kernel<T, true><<<g, kThreads, 0, s>>>((T*)dgate, (T*)dup, (const T*)grad, (const T*)gate, (const T*)up, n);
    else geglu_bwd_kernel<T, false><<<g, kThreads, 0, s>>>((T*)dgate, (T*)dup, (const T*)grad, (const T*)gate, (const T*)up, n);
  });
}
