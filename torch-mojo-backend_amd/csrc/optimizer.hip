// Multi-tensor optimizer kernels: fused AdamW, per-tensor norms and in-place
// foreach updates.
//
// All three use the same launch shape: up to kBatch tensors per launch,
// described in the kernel arguments, each split into fixed-size chunks; the
// grid is the total chunk count and a block locates its (tensor, chunk) by a
// binary search over the chunk prefix sums.  Contiguous f32 data moves as float4.
//
// AdamW (torch.optim.AdamW, decoupled weight decay), per element:
//   g *= grad_mul (if given);  g = maximize ? -g : g;  g /= grad_scale (if given)
//   p -= lr*wd*p                         (skipped when wd == 0)
//   m = b1*m + (1-b1)*g;  v = b2*v + (1-b2)*g*g
//   vmax = max(vmax, v)                  (amsgrad)
//   p -= (lr/(1-b1^t)) * m / (sqrt(v or vmax)/sqrt(1-b2^t) + eps)
// with t read from the device step tensor (already incremented by the
// caller's _foreach_add_), lr from a device scalar if given, and the whole
// update skipped when *found_inf != 0.  HBM traffic per element: 16 B read
// (p, g, m, v) + 12 B written (p, m, v) = 28 B, + 2 B when the kernel also
// writes the parameter's bf16/f16 copy for the next autocast forward.
#include <math.h>

#include "common.h"

namespace mi {
namespace {

constexpr int kThreads = 256;
// Tensors per launch.  The batch descriptors travel as kernel arguments
// (up to ~12 KB here; gfx950 kernels take at least 16 KB), so a GPT-2 sized
// parameter list updates in one launch per parameter group.
constexpr int kAdamBatch = 160;
// 4096 elements per block, four float4 of each array per thread, all loads
// issued before the first update: 0.591 ms for 124.4M parameters against
// 0.655 ms with 16384-element chunks (gfx950).
constexpr int64_t kAdamChunk = 4096;

struct AdamBatch {
  mi355x_adamw_tensor t[kAdamBatch];
  void* low[kAdamBatch];  // optional 16-bit copy of each updated param (element type TL)
  int64_t chunk_start[kAdamBatch + 1];
  int n;
};

// The tensor whose chunk range [starts[k], starts[k+1]) holds `chunk`
// (binary search; empty tensors have empty ranges and are never returned).
__device__ __forceinline__ int find_tensor(const int64_t* starts, int n, int64_t chunk) {
  int lo = 0, hi = n - 1;  // starts[lo] <= chunk < starts[hi + 1]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (starts[mid] <= chunk) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

struct AdamScalars {
  float lr, b1, b2, wd, eps;
  int flags;
  const float* lr_ptr;
  const float* grad_scale;
  const float* found_inf;
  const float* grad_mul;
};

template <typename TL>
__device__ __forceinline__ void store_low4(TL* dst, const float4& p) {
  typedef TL tl4 __attribute__((ext_vector_type(4)));
  tl4 v;
  v[0] = (TL)p.x, v[1] = (TL)p.y, v[2] = (TL)p.z, v[3] = (TL)p.w;
  *(tl4*)dst = v;
}

__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v, float* vmax,
                                          float lr, float b1, float b2, float wd, float eps,
                                          float step_size, float bc2_sqrt, bool decay) {
  if (decay) p -= lr * wd * p;
  m = b1 * m + (1.f - b1) * g;
  v = b2 * v + (1.f - b2) * g * g;
  float vv = v;
  if (vmax) {
    *vmax = nan_max(*vmax, v);
    vv = *vmax;
  }
  const float denom = sqrtf(vv) / bc2_sqrt + eps;
  p -= step_size * m / denom;
}

template <typename TL>
__global__ void __launch_bounds__(kThreads) adamw_kernel(AdamBatch b, AdamScalars s) {
  if (s.found_inf && *s.found_inf != 0.f) return;
  const int64_t chunk = blockIdx.x;
  const int k = find_tensor(b.chunk_start, b.n, chunk);
  const mi355x_adamw_tensor& t = b.t[k];
  TL* const low = (TL*)b.low[k];
  const int64_t begin = (chunk - b.chunk_start[k]) * kAdamChunk;
  const int64_t end = min(t.numel, begin + kAdamChunk);
  const float lr = s.lr_ptr ? *s.lr_ptr : s.lr;
  const float step = *t.step;
  const float bc1 = 1.f - powf(s.b1, step);
  const float bc2 = 1.f - powf(s.b2, step);
  const float step_size = lr / bc1;
  const float bc2_sqrt = sqrtf(bc2);
  const bool decay = s.wd != 0.f;
  const bool maximize = s.flags & MI355X_ADAMW_MAXIMIZE;
  const float inv_scale = s.grad_scale ? 1.f / *s.grad_scale : 1.f;
  const bool has_mul = s.grad_mul != nullptr;
  const float gmul = has_mul ? *s.grad_mul : 1.f;
  const bool vec = ((((uintptr_t)t.param | (uintptr_t)t.grad | (uintptr_t)t.exp_avg |
                      (uintptr_t)t.exp_avg_sq) & 15) == 0) && (((uintptr_t)low & 7) == 0) &&
                   t.max_exp_avg_sq == nullptr && (begin % 4 == 0);
  int64_t i = begin;
  if (vec) {
    const int64_t nv = (end - begin) / 4;
    // Two float4 of each array per thread per iteration: all eight loads are
    // in flight before the first update.
    auto update = [&](float4& p, const float4& g, float4& m, float4& v) {
      float gg[4] = {g.x, g.y, g.z, g.w};
      float pp[4] = {p.x, p.y, p.z, p.w}, mm[4] = {m.x, m.y, m.z, m.w}, vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float g0 = has_mul ? gg[j] * gmul : gg[j];
        float gj = (maximize ? -g0 : g0) * inv_scale;
        adam_elem(pp[j], gj, mm[j], vv[j], nullptr, lr, s.b1, s.b2, s.wd, s.eps, step_size, bc2_sqrt, decay);
      }
      p = make_float4(pp[0], pp[1], pp[2], pp[3]);
      m = make_float4(mm[0], mm[1], mm[2], mm[3]);
      v = make_float4(vv[0], vv[1], vv[2], vv[3]);
    };
    float4* P = (float4*)(t.param + begin);
    const float4* G = (const float4*)(t.grad + begin);
    float4* M = (float4*)(t.exp_avg + begin);
    float4* V = (float4*)(t.exp_avg_sq + begin);
    int64_t q = threadIdx.x;
    constexpr int U = 4;
    for (; q + (U - 1) * kThreads < nv; q += U * kThreads) {
      float4 pp[U], gg[U], mm[U], vv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        pp[u] = ld_stream(P + q + u * kThreads);
        gg[u] = ld_stream(G + q + u * kThreads);
        mm[u] = ld_stream(M + q + u * kThreads);
        vv[u] = ld_stream(V + q + u * kThreads);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) update(pp[u], gg[u], mm[u], vv[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        st_stream(P + q + u * kThreads, pp[u]);
        st_stream(M + q + u * kThreads, mm[u]);
        st_stream(V + q + u * kThreads, vv[u]);
        if (low) store_low4(low + begin + (q + u * kThreads) * 4, pp[u]);
      }
    }
    for (; q < nv; q += kThreads) {
      float4 p0 = P[q], m0 = M[q], v0 = V[q];
      const float4 g0 = G[q];
      update(p0, g0, m0, v0);
      P[q] = p0, M[q] = m0, V[q] = v0;
      if (low) store_low4(low + begin + q * 4, p0);
    }
    i = begin + nv * 4;
  }
  for (int64_t e = i + threadIdx.x; e < end; e += kThreads) {
    float p = t.param[e], m = t.exp_avg[e], v = t.exp_avg_sq[e];
    float g = t.grad[e];
    if (has_mul) g *= gmul;
    g = (maximize ? -g : g) * inv_scale;
    adam_elem(p, g, m, v, t.max_exp_avg_sq ? t.max_exp_avg_sq + e : nullptr, lr, s.b1, s.b2, s.wd,
              s.eps, step_size, bc2_sqrt, decay);
    t.param[e] = p;
    t.exp_avg[e] = m;
    t.exp_avg_sq[e] = v;
    if (low) low[e] = (TL)p;
  }
}

// ---------------------------------------------------------------------------
// foreach norm
// ---------------------------------------------------------------------------
constexpr int kNormBatch = 160;
constexpr int64_t kNormChunk = 32768;

struct NormBatch {
  const void* in[kNormBatch];
  void* out[kNormBatch];
  int64_t numel[kNormBatch];
  int64_t chunk_start[kNormBatch + 1];
  int n;
};

// kind: 0 = sum x^2, 1 = sum |x|, 2 = max |x|
template <typename T>
__global__ void __launch_bounds__(kThreads) norm_partial(NormBatch b, int kind, float* part) {
  __shared__ float red[kThreads / 64];
  const int64_t chunk = blockIdx.x;
  const int k = find_tensor(b.chunk_start, b.n, chunk);
  const T* x = (const T*)b.in[k];
  const int64_t begin = (chunk - b.chunk_start[k]) * kNormChunk;
  const int64_t end = min(b.numel[k], begin + kNormChunk);
  float acc = 0.f;
  auto take = [&](float v) {
    if (kind == 0) acc += v * v;
    else if (kind == 1) acc += fabsf(v);
    else acc = nan_max(acc, fabsf(v));
  };
  int64_t e0 = begin;
  if ((((uintptr_t)x) & 15) == 0) {
    // 16-byte loads, two per thread per iteration (8 or 16 elements)
    constexpr int V = 16 / sizeof(T);
    typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
    const int64_t nv = (end - begin) / V;
    const u32x4* X = (const u32x4*)(x + begin);
    int64_t q = threadIdx.x;
    for (; q + kThreads < nv; q += 2 * kThreads) {
      const u32x4 a = X[q], b2 = X[q + kThreads];
      const T* ta = (const T*)&a;
      const T* tb = (const T*)&b2;
#pragma unroll
      for (int j = 0; j < V; ++j) take(to_f32(ta[j])), take(to_f32(tb[j]));
    }
    if (q < nv) {
      const u32x4 a = X[q];
      const T* ta = (const T*)&a;
#pragma unroll
      for (int j = 0; j < V; ++j) take(to_f32(ta[j]));
    }
    e0 = begin + nv * V;
  }
  for (int64_t e = e0 + threadIdx.x; e < end; e += kThreads) take(to_f32(x[e]));
  if (kind == 2) {
    acc = wave_max_nan(acc);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    acc = red[0];
    for (int w = 1; w < kThreads / 64; ++w) acc = nan_max(acc, red[w]);
  } else {
    acc = block_sum(acc, red);
  }
  if (threadIdx.x == 0) part[chunk] = acc;
}

template <typename TO>
__global__ void __launch_bounds__(kThreads) norm_final(NormBatch b, int kind, const float* part) {
  __shared__ float red[kThreads / 64];
  const int k = blockIdx.x;
  const int64_t c0 = b.chunk_start[k], c1 = b.chunk_start[k + 1];
  float acc = 0.f;
  for (int64_t c = c0 + threadIdx.x; c < c1; c += kThreads)
    acc = kind == 2 ? nan_max(acc, part[c]) : acc + part[c];
  if (kind == 2) {
    acc = wave_max_nan(acc);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    acc = red[0];
    for (int w = 1; w < kThreads / 64; ++w) acc = nan_max(acc, red[w]);
  } else {
    acc = block_sum(acc, red);
  }
  if (threadIdx.x == 0) {
    const float r = kind == 0 ? sqrtf(acc) : acc;
    *(TO*)b.out[k] = from_f32<TO>(r);
  }
}

// ---------------------------------------------------------------------------
// foreach apply
// ---------------------------------------------------------------------------
constexpr int kApplyBatch = 160;
constexpr int64_t kApplyChunk = 16384;

struct ApplyBatch {
  void* a[kApplyBatch];
  const void* b[kApplyBatch];
  const void* c[kApplyBatch];
  double scal[kApplyBatch];
  int64_t numel[kApplyBatch];
  int64_t chunk_start[kApplyBatch + 1];
  int n;
  int has_scal;
};

__device__ __forceinline__ float apply_val(int op, float x, float y, float z, bool has_b, float s0, float sc,
                                           bool has_ts, float tsv, bool has_scal) {
  switch (op) {
    case MI355X_OP_ADD: return x + s0 * (has_b ? y : 1.f);
    case MI355X_OP_MUL: return x * (has_ts ? tsv : (has_scal ? sc : (has_b ? y : s0)));
    case MI355X_OP_DIV: return x / (has_ts ? tsv : (has_scal ? sc : (has_b ? y : s0)));
    case MI355X_OP_LERP: return (fabsf(s0) < 0.5f) ? x + s0 * (y - x) : y - (y - x) * (1.f - s0);
    case MI355X_OP_ADDCMUL: return x + sc * y * z;
    case MI355X_OP_ADDCDIV: return x + sc * (y / z);
    case MI355X_OP_SQRT: return sqrtf(x);
  }
  return x;
}

template <typename T>
__global__ void __launch_bounds__(kThreads) apply_kernel(ApplyBatch b, int op, float s0, const float* ts) {
  const int64_t chunk = blockIdx.x;
  const int k = find_tensor(b.chunk_start, b.n, chunk);
  T* a = (T*)b.a[k];
  const T* bb = (const T*)b.b[k];
  const T* cc = (const T*)b.c[k];
  const float sc = b.has_scal ? (float)b.scal[k] : s0;
  const float tsv = ts ? *ts : 0.f;
  const bool has_b = bb != nullptr, has_ts = ts != nullptr, has_scal = b.has_scal != 0;
  const int64_t begin = (chunk - b.chunk_start[k]) * kApplyChunk;
  const int64_t end = min(b.numel[k], begin + kApplyChunk);
  int64_t e0 = begin;
  if constexpr (sizeof(T) == 4) {
    if (((((uintptr_t)a) | ((uintptr_t)bb) | ((uintptr_t)cc)) & 15) == 0) {
      const int64_t nv = (end - begin) / 4;
      float4* A4 = (float4*)(a + begin);
      const float4* B4 = (const float4*)(bb + begin);
      const float4* C4 = (const float4*)(cc + begin);
      for (int64_t q = threadIdx.x; q < nv; q += kThreads) {
        const float4 x = A4[q];
        const float4 y = bb ? B4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 z = cc ? C4[q] : make_float4(1.f, 1.f, 1.f, 1.f);
        A4[q] = make_float4(apply_val(op, x.x, y.x, z.x, has_b, s0, sc, has_ts, tsv, has_scal),
                            apply_val(op, x.y, y.y, z.y, has_b, s0, sc, has_ts, tsv, has_scal),
                            apply_val(op, x.z, y.z, z.z, has_b, s0, sc, has_ts, tsv, has_scal),
                            apply_val(op, x.w, y.w, z.w, has_b, s0, sc, has_ts, tsv, has_scal));
      }
      e0 = begin + nv * 4;
    }
  }
  for (int64_t e = e0 + threadIdx.x; e < end; e += kThreads) {
    const float y = bb ? to_f32(bb[e]) : 0.f, z = cc ? to_f32(cc[e]) : 1.f;
    a[e] = from_f32<T>(apply_val(op, to_f32(a[e]), y, z, has_b, s0, sc, has_ts, tsv, has_scal));
  }
}

int64_t chunks_of(int64_t numel, int64_t chunk) { return (numel + chunk - 1) / chunk; }

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi355x_fused_adamw_ex(const mi355x_adamw_tensor* tensors, void* const* param_low, int low_dtype,
                                     int n, double lr, const float* lr_ptr, double beta1, double beta2,
                                     double weight_decay, double eps, int flags, const float* grad_scale,
                                     const float* found_inf, const float* grad_mul, mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0 && (n == 0 || tensors), "mi355x_fused_adamw: bad tensor list");
  MI_REQUIRE(!param_low || low_dtype == MI355X_BF16 || low_dtype == MI355X_F16,
             "mi355x_fused_adamw: the parameter copies must be bf16 or f16");
  hipStream_t s = (hipStream_t)stream;
  AdamScalars sc{(float)lr, (float)beta1, (float)beta2, (float)weight_decay, (float)eps, flags,
                 lr_ptr, grad_scale, found_inf, grad_mul};
  for (int base = 0; base < n; base += kAdamBatch) {
    AdamBatch b{};
    b.n = 0;
    int64_t chunks = 0;
    for (int j = base; j < n && b.n < kAdamBatch; ++j) {
      const mi355x_adamw_tensor& t = tensors[j];
      MI_REQUIRE(t.numel >= 0, "mi355x_fused_adamw: negative numel");
      MI_REQUIRE(t.numel == 0 || (t.param && t.grad && t.exp_avg && t.exp_avg_sq && t.step),
                 "mi355x_fused_adamw: null pointer in tensor %d", j);
      MI_REQUIRE(!(flags & MI355X_ADAMW_AMSGRAD) || t.numel == 0 || t.max_exp_avg_sq,
                 "mi355x_fused_adamw: amsgrad needs max_exp_avg_sq (tensor %d)", j);
      b.t[b.n] = t;
      b.low[b.n] = param_low ? param_low[j] : nullptr;
      if (!(flags & MI355X_ADAMW_AMSGRAD)) b.t[b.n].max_exp_avg_sq = nullptr;
      b.chunk_start[b.n] = chunks;
      chunks += chunks_of(t.numel, kAdamChunk);
      ++b.n;
    }
    b.chunk_start[b.n] = chunks;
    if (chunks == 0) continue;
    if (low_dtype == MI355X_F16) adamw_kernel<f16><<<(unsigned)chunks, kThreads, 0, s>>>(b, sc);
    else adamw_kernel<bf16><<<(unsigned)chunks, kThreads, 0, s>>>(b, sc);
    int rc = check_launch("mi355x_fused_adamw");
    if (rc) return rc;
  }
  return MI355X_OK;
}

extern "C" int mi355x_fused_adamw(const mi355x_adamw_tensor* tensors, int n, double lr,
                                  const float* lr_ptr, double beta1, double beta2,
                                  double weight_decay, double eps, int flags,
                                  const float* grad_scale, const float* found_inf,
                                  mi355x_stream_t stream) {
  return mi355x_fused_adamw_ex(tensors, nullptr, 0, n, lr, lr_ptr, beta1, beta2, weight_decay, eps, flags,
                               grad_scale, found_inf, nullptr, stream);
}

extern "C" int64_t mi355x_foreach_norm_workspace_bytes(const int64_t* numels, int n) {
  int64_t total = 0;
  for (int j = 0; j < n; ++j) total += chunks_of(numels[j], kNormChunk);
  return total * (int64_t)sizeof(float) + 256;
}

extern "C" int mi355x_foreach_norm(void* const* outs, int out_dtype, const void* const* ins,
                                   int in_dtype, const int64_t* numels, int n, double ord,
                                   void* workspace, int64_t ws_bytes, mi355x_stream_t stream) {
  int kind;
  if (ord == 2.0) kind = 0;
  else if (ord == 1.0) kind = 1;
  else if (isinf(ord) && ord > 0) kind = 2;
  else return fail(MI355X_EUNSUPPORTED, "mi355x_foreach_norm: ord %g not supported", ord);
  MI_REQUIRE(in_dtype == MI355X_F32 || in_dtype == MI355X_BF16 || in_dtype == MI355X_F16,
             "mi355x_foreach_norm: unsupported input dtype");
  MI_REQUIRE(out_dtype == MI355X_F32 || out_dtype == MI355X_BF16 || out_dtype == MI355X_F16,
             "mi355x_foreach_norm: unsupported output dtype");
  const int64_t need = mi355x_foreach_norm_workspace_bytes(numels, n);
  if (n > 0 && (!workspace || ws_bytes < need))
    return fail(MI355X_EWORKSPACE, "mi355x_foreach_norm: workspace %lld < %lld", (long long)ws_bytes, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  for (int base = 0; base < n; base += kNormBatch) {
    NormBatch b{};
    int64_t chunks = 0;
    b.n = 0;
    for (int j = base; j < n && b.n < kNormBatch; ++j) {
      b.in[b.n] = ins[j];
      b.out[b.n] = outs[j];
      b.numel[b.n] = numels[j];
      b.chunk_start[b.n] = chunks;
      chunks += chunks_of(numels[j], kNormChunk);
      ++b.n;
    }
    b.chunk_start[b.n] = chunks;
    if (chunks > 0) {
      switch (in_dtype) {
        case MI355X_F32: norm_partial<float><<<(unsigned)chunks, kThreads, 0, s>>>(b, kind, part); break;
        case MI355X_BF16: norm_partial<bf16><<<(unsigned)chunks, kThreads, 0, s>>>(b, kind, part); break;
        default: norm_partial<f16><<<(unsigned)chunks, kThreads, 0, s>>>(b, kind, part); break;
      }
    }
    switch (out_dtype) {
      case MI355X_F32: norm_final<float><<<b.n, kThreads, 0, s>>>(b, kind, part); break;
      case MI355X_BF16: norm_final<bf16><<<b.n, kThreads, 0, s>>>(b, kind, part); break;
      default: norm_final<f16><<<b.n, kThreads, 0, s>>>(b, kind, part); break;
    }
    int rc = check_launch("mi355x_foreach_norm");
    if (rc) return rc;
    part += chunks;
  }
  return MI355X_OK;
}

extern "C" int mi355x_foreach_apply(int op, void* const* a, const void* const* b,
                                    const void* const* c, const double* scalars,
                                    const int64_t* numels, int n, int dtype, double s0,
                                    const float* tensor_scalar, mi355x_stream_t stream) {
  switch (op) {
    case MI355X_OP_ADD: case MI355X_OP_MUL: case MI355X_OP_DIV: case MI355X_OP_SQRT: break;
    case MI355X_OP_LERP: MI_REQUIRE(b, "mi355x_foreach_apply: lerp needs b"); break;
    case MI355X_OP_ADDCMUL: case MI355X_OP_ADDCDIV: MI_REQUIRE(b && c, "mi355x_foreach_apply: needs b and c"); break;
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_foreach_apply: op %d not supported", op);
  }
  MI_REQUIRE(dtype == MI355X_F32 || dtype == MI355X_BF16 || dtype == MI355X_F16,
             "mi355x_foreach_apply: unsupported dtype");
  hipStream_t s = (hipStream_t)stream;
  for (int base = 0; base < n; base += kApplyBatch) {
    ApplyBatch bt{};
    int64_t chunks = 0;
    bt.n = 0;
    bt.has_scal = scalars != nullptr;
    for (int j = base; j < n && bt.n < kApplyBatch; ++j) {
      bt.a[bt.n] = a[j];
      bt.b[bt.n] = b ? b[j] : nullptr;
      bt.c[bt.n] = c ? c[j] : nullptr;
      bt.scal[bt.n] = scalars ? scalars[j] : 0.0;
      bt.numel[bt.n] = numels[j];
      bt.chunk_start[bt.n] = chunks;
      chunks += chunks_of(numels[j], kApplyChunk);
      ++bt.n;
    }
    bt.chunk_start[bt.n] = chunks;
    if (chunks == 0) continue;
    switch (dtype) {
      case MI355X_F32: apply_kernel<float><<<(unsigned)chunks, kThreads, 0, s>>>(bt, op, (float)s0, tensor_scalar); break;
      case MI355X_BF16: apply_kernel<bf16><<<(unsigned)chunks, kThreads, 0, s>>>(bt, op, (float)s0, tensor_scalar); break;
      default: apply_kernel<f16><<<(unsigned)chunks, kThreads, 0, s>>>(bt, op, (float)s0, tensor_scalar); break;
    }
    int rc = check_launch("mi355x_foreach_apply");
    if (rc) return rc;
  }
  return MI355X_OK;
}
