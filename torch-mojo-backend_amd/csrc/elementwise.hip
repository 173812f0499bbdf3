// Strided copy/cast, fill, arange and the generic elementwise map.
//
// These are the plumbing kernels of the eager device: dtype casts under
// autocast, residual/bias adds, comparisons, factories.  All operand layouts
// are described by (shape, strides) in elements; the host wrapper first
// merges dimensions that are contiguous for every operand, so the common
// dense case reaches the vectorised path with ndim == 1.
#include <math.h>

#include "common.h"
#include "vec.h"

namespace mi {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxOperands = 4;  // out + 3 inputs

struct Geo {
  int ndim;
  int nops;
  int64_t shape[MI355X_MAX_RANK];
  int64_t st[kMaxOperands][MI355X_MAX_RANK];
};

// ---------------------------------------------------------------------------
// Host: coalesce dims (drop size-1 dims, merge dims contiguous for all ops)
// ---------------------------------------------------------------------------
int build_geo(Geo& g, int nops, const int64_t* const* strides,
              const int64_t* shape, int ndim, int64_t* numel) {
  if (ndim < 0 || ndim > MI355X_MAX_RANK)
    return fail(MI355X_EINVAL, "rank %d exceeds %d", ndim, MI355X_MAX_RANK);
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] < 0) return fail(MI355X_EINVAL, "negative extent %lld", (long long)shape[d]);
    n *= shape[d];
  }
  *numel = n;
  g.nops = nops;
  int nd = 0;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] == 1) continue;
    if (nd > 0) {
      bool mergeable = true;
      for (int j = 0; j < nops; ++j)
        if (g.st[j][nd - 1] != strides[j][d] * shape[d]) mergeable = false;
      if (mergeable) {
        g.shape[nd - 1] *= shape[d];
        for (int j = 0; j < nops; ++j) g.st[j][nd - 1] = strides[j][d];
        continue;
      }
    }
    g.shape[nd] = shape[d];
    for (int j = 0; j < nops; ++j) g.st[j][nd] = strides[j][d];
    ++nd;
  }
  g.ndim = nd;
  return MI355X_OK;
}

bool geo_dense(const Geo& g) {
  if (g.ndim == 0) return true;
  if (g.ndim != 1) return false;
  for (int j = 0; j < g.nops; ++j)
    if (g.st[j][0] != 1) return false;
  return true;
}

unsigned grid_for(int64_t n, int per_thread = 1) {
  int64_t b = (n + (int64_t)kThreads * per_thread - 1) / ((int64_t)kThreads * per_thread);
  if (b < 1) b = 1;
  if (b > 65536) b = 65536;
  return (unsigned)b;
}

// ---------------------------------------------------------------------------
// Typed loads/stores with a runtime dtype (the branch is wave-uniform)
// ---------------------------------------------------------------------------
template <typename C>
__device__ __forceinline__ C cvt_from_f(double x) { return (C)x; }

template <typename C>
__device__ __forceinline__ C ld(const void* p, int dt, int64_t i) {
  switch (dt) {
    case MI355X_F32: return (C)((const float*)p)[i];
    case MI355X_BF16: return (C)(float)((const bf16*)p)[i];
    case MI355X_F16: return (C)(float)((const f16*)p)[i];
    case MI355X_F64: return (C)((const double*)p)[i];
    case MI355X_I64: return (C)((const int64_t*)p)[i];
    case MI355X_I32: return (C)((const int32_t*)p)[i];
    case MI355X_I16: return (C)((const int16_t*)p)[i];
    case MI355X_I8: return (C)((const int8_t*)p)[i];
    case MI355X_U8: return (C)((const uint8_t*)p)[i];
    default: return (C)(((const uint8_t*)p)[i] != 0);
  }
}

template <typename C>
__device__ __forceinline__ void st(void* p, int dt, int64_t i, C v) {
  switch (dt) {
    case MI355X_F32: ((float*)p)[i] = (float)v; break;
    case MI355X_BF16: ((bf16*)p)[i] = (bf16)(float)v; break;
    case MI355X_F16: ((f16*)p)[i] = (f16)(float)v; break;
    case MI355X_F64: ((double*)p)[i] = (double)v; break;
    case MI355X_I64: ((int64_t*)p)[i] = (int64_t)v; break;
    case MI355X_I32: ((int32_t*)p)[i] = (int32_t)v; break;
    case MI355X_I16: ((int16_t*)p)[i] = (int16_t)v; break;
    case MI355X_I8: ((int8_t*)p)[i] = (int8_t)v; break;
    case MI355X_U8: ((uint8_t*)p)[i] = (uint8_t)v; break;
    default: ((uint8_t*)p)[i] = (v != (C)0) ? 1 : 0; break;
  }
}

// float -> integer conversions must not be UB for NaN/out of range.
template <>
__device__ __forceinline__ void st<float>(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case MI355X_F32: ((float*)p)[i] = v; break;
    case MI355X_BF16: ((bf16*)p)[i] = (bf16)v; break;
    case MI355X_F16: ((f16*)p)[i] = (f16)v; break;
    case MI355X_F64: ((double*)p)[i] = (double)v; break;
    case MI355X_BOOL: ((uint8_t*)p)[i] = (v != 0.f) ? 1 : 0; break;
    default: {
      int64_t iv = isfinite(v) ? (int64_t)v : 0;
      switch (dt) {
        case MI355X_I64: ((int64_t*)p)[i] = iv; break;
        case MI355X_I32: ((int32_t*)p)[i] = (int32_t)iv; break;
        case MI355X_I16: ((int16_t*)p)[i] = (int16_t)iv; break;
        case MI355X_I8: ((int8_t*)p)[i] = (int8_t)iv; break;
        default: ((uint8_t*)p)[i] = (uint8_t)iv; break;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Operators
// ---------------------------------------------------------------------------
template <typename C>
struct Ops;

template <typename F>
struct FloatOps {
  static __device__ __forceinline__ F apply(int op, F a, F b, F c, F s0, F s1) {
    switch (op) {
      case MI355X_OP_ADD: return a + s0 * b;
      case MI355X_OP_SUB: return a - s0 * b;
      case MI355X_OP_MUL: return a * b;
      case MI355X_OP_DIV: return a / b;
      case MI355X_OP_MAXIMUM: return (a != a || b != b) ? (a + b) : (a > b ? a : b);
      case MI355X_OP_MINIMUM: return (a != a || b != b) ? (a + b) : (a < b ? a : b);
      case MI355X_OP_POW: return pow(a, b);
      case MI355X_OP_EQ: return a == b;
      case MI355X_OP_NE: return a != b;
      case MI355X_OP_LT: return a < b;
      case MI355X_OP_LE: return a <= b;
      case MI355X_OP_GT: return a > b;
      case MI355X_OP_GE: return a >= b;
      case MI355X_OP_LOGICAL_AND: return (a != 0) && (b != 0);
      case MI355X_OP_LOGICAL_OR: return (a != 0) || (b != 0);
      case MI355X_OP_LOGICAL_XOR: return (a != 0) != (b != 0);
      case MI355X_OP_REMAINDER: {
        F r = fmod(a, b);
        if (r != 0 && ((r < 0) != (b < 0))) r += b;
        return r;
      }
      case MI355X_OP_FLOOR_DIVIDE:
      case MI355X_OP_DIV_FLOOR: {
        if (b == 0) return a / b;
        F m = fmod(a, b);
        F q = (a - m) / b;
        if (m != 0 && ((b < 0) != (m < 0))) q -= 1;
        F fq = floor(q);
        if (q - fq > (F)0.5) fq += 1;
        return (q == 0) ? copysign((F)0, a / b) : fq;
      }
      case MI355X_OP_DIV_TRUNC: return trunc(a / b);
      case MI355X_OP_WHERE: return (a != 0) ? b : c;
      case MI355X_OP_ADDCMUL: return a + s0 * b * c;
      case MI355X_OP_ADDCDIV: return a + s0 * (b / c);
      case MI355X_OP_LERP: return (fabs(s0) < (F)0.5) ? a + s0 * (b - a) : b - (b - a) * ((F)1 - s0);
      case MI355X_OP_IDENTITY: return a;
      case MI355X_OP_NEG: return -a;
      case MI355X_OP_ABS: return fabs(a);
      case MI355X_OP_EXP: return exp(a);
      case MI355X_OP_LOG: return log(a);
      case MI355X_OP_SQRT: return sqrt(a);
      case MI355X_OP_RSQRT: return (F)1 / sqrt(a);
      case MI355X_OP_RECIPROCAL: return (F)1 / a;
      case MI355X_OP_SIN: return sin(a);
      case MI355X_OP_COS: return cos(a);
      case MI355X_OP_TAN: return tan(a);
      case MI355X_OP_ATAN: return atan(a);
      case MI355X_OP_ASIN: return asin(a);
      case MI355X_OP_ACOS: return acos(a);
      case MI355X_OP_SINH: return sinh(a);
      case MI355X_OP_COSH: return cosh(a);
      case MI355X_OP_ASINH: return asinh(a);
      case MI355X_OP_ACOSH: return acosh(a);
      case MI355X_OP_ATANH: return atanh(a);
      case MI355X_OP_TANH: return tanh(a);
      case MI355X_OP_SIGMOID: return (F)1 / ((F)1 + exp(-a));
      case MI355X_OP_ERF: return erf(a);
      case MI355X_OP_RELU: return (a != a) ? a : (a > 0 ? a : (F)0);
      case MI355X_OP_SILU: return a / ((F)1 + exp(-a));
      case MI355X_OP_LOG1P: return log1p(a);
      case MI355X_OP_EXPM1: return expm1(a);
      case MI355X_OP_LOG2: return log2(a);
      case MI355X_OP_EXP2: return exp2(a);
      case MI355X_OP_LOG10: return log10(a);
      case MI355X_OP_FLOOR: return floor(a);
      case MI355X_OP_CEIL: return ceil(a);
      case MI355X_OP_ROUND: return rint(a);
      case MI355X_OP_TRUNC: return trunc(a);
      case MI355X_OP_SIGN: return (a != a) ? a : (F)((a > 0) - (a < 0));
      case MI355X_OP_POW_SCALAR:
        if (s0 == (F)2) return a * a;
        if (s0 == (F)0.5) return sqrt(a);
        if (s0 == (F)1) return a;
        return pow(a, s0);
      case MI355X_OP_SQUARE: return a * a;
      case MI355X_OP_CLAMP: return (a != a) ? a : fmin(fmax(a, s0), s1);
      case MI355X_OP_CLAMP_MIN: return (a != a) ? a : fmax(a, s0);
      case MI355X_OP_CLAMP_MAX: return (a != a) ? a : fmin(a, s0);
      case MI355X_OP_LOGICAL_NOT: return a == 0;
      case MI355X_OP_ISNAN: return a != a;
      case MI355X_OP_ISINF: return isinf(a);
      case MI355X_OP_ISFINITE: return isfinite(a);
      case MI355X_OP_RSUB: return s0 - a * s1;
    }
    return a;
  }
};

template <>
struct Ops<float> : FloatOps<float> {};
template <>
struct Ops<double> : FloatOps<double> {};

template <>
struct Ops<int64_t> {
  static __device__ __forceinline__ int64_t apply(int op, int64_t a, int64_t b, int64_t c,
                                                  int64_t s0, int64_t s1) {
    switch (op) {
      case MI355X_OP_ADD: return a + s0 * b;
      case MI355X_OP_SUB: return a - s0 * b;
      case MI355X_OP_MUL: return a * b;
      case MI355X_OP_MAXIMUM: return a > b ? a : b;
      case MI355X_OP_MINIMUM: return a < b ? a : b;
      case MI355X_OP_EQ: return a == b;
      case MI355X_OP_NE: return a != b;
      case MI355X_OP_LT: return a < b;
      case MI355X_OP_LE: return a <= b;
      case MI355X_OP_GT: return a > b;
      case MI355X_OP_GE: return a >= b;
      case MI355X_OP_LOGICAL_AND: return (a != 0) && (b != 0);
      case MI355X_OP_LOGICAL_OR: return (a != 0) || (b != 0);
      case MI355X_OP_LOGICAL_XOR: return (a != 0) != (b != 0);
      case MI355X_OP_BITWISE_AND: return a & b;
      case MI355X_OP_BITWISE_OR: return a | b;
      case MI355X_OP_BITWISE_XOR: return a ^ b;
      case MI355X_OP_REMAINDER: {
        if (b == 0) return 0;
        int64_t r = a % b;
        if (r != 0 && ((r < 0) != (b < 0))) r += b;
        return r;
      }
      case MI355X_OP_FLOOR_DIVIDE:
      case MI355X_OP_DIV_FLOOR: {
        if (b == 0) return 0;
        int64_t q = a / b;
        if ((a % b != 0) && ((a < 0) != (b < 0))) q -= 1;
        return q;
      }
      case MI355X_OP_DIV_TRUNC: return b == 0 ? 0 : a / b;
      case MI355X_OP_WHERE: return (a != 0) ? b : c;
      case MI355X_OP_ADDCMUL: return a + s0 * b * c;
      case MI355X_OP_IDENTITY: return a;
      case MI355X_OP_NEG: return -a;
      case MI355X_OP_ABS: return a < 0 ? -a : a;
      case MI355X_OP_RELU: return a > 0 ? a : 0;
      case MI355X_OP_SIGN: return (a > 0) - (a < 0);
      case MI355X_OP_SQUARE: return a * a;
      case MI355X_OP_CLAMP: return a < s0 ? s0 : (a > s1 ? s1 : a);
      case MI355X_OP_CLAMP_MIN: return a < s0 ? s0 : a;
      case MI355X_OP_CLAMP_MAX: return a > s0 ? s0 : a;
      case MI355X_OP_LOGICAL_NOT: return a == 0;
      case MI355X_OP_BITWISE_NOT: return ~a;
      case MI355X_OP_ISNAN: return 0;
      case MI355X_OP_ISINF: return 0;
      case MI355X_OP_ISFINITE: return 1;
      case MI355X_OP_FLOOR:
      case MI355X_OP_CEIL:
      case MI355X_OP_ROUND:
      case MI355X_OP_TRUNC: return a;
      case MI355X_OP_RSUB: return s0 - a * s1;
    }
    return a;
  }
};

// ---------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------
template <typename I>
__device__ __forceinline__ void offsets(const Geo& g, I idx, int64_t* off) {
  for (int j = 0; j < g.nops; ++j) off[j] = 0;
  for (int d = g.ndim - 1; d >= 0; --d) {
    I ext = (I)g.shape[d];
    I cidx = idx % ext;
    idx /= ext;
    for (int j = 0; j < g.nops; ++j) off[j] += (int64_t)cidx * g.st[j][d];
  }
}

struct MapArgs {
  int op;
  int nin;
  void* out;
  const void* in[3];
  int out_dt;
  int in_dt[3];
  double s0, s1;
};

template <typename C, typename I>
__global__ void __launch_bounds__(kThreads) map_strided(MapArgs a, Geo g, I n) {
  const C s0 = (C)a.s0, s1 = (C)a.s1;
  for (I i = (I)blockIdx.x * kThreads + threadIdx.x; i < n; i += (I)gridDim.x * kThreads) {
    int64_t off[kMaxOperands];
    offsets<I>(g, i, off);
    C x = a.nin > 0 ? (a.in[0] ? ld<C>(a.in[0], a.in_dt[0], off[1]) : s1) : (C)0;
    C y = a.nin > 1 ? (a.in[1] ? ld<C>(a.in[1], a.in_dt[1], off[2]) : s1) : (C)0;
    C z = a.nin > 2 ? (a.in[2] ? ld<C>(a.in[2], a.in_dt[2], off[3]) : s1) : (C)0;
    st<C>(a.out, a.out_dt, off[0], Ops<C>::apply(a.op, x, y, z, s0, s1));
  }
}

template <typename C>
__global__ void __launch_bounds__(kThreads) map_dense(MapArgs a, int64_t n) {
  const C s0 = (C)a.s0, s1 = (C)a.s1;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    C x = a.nin > 0 ? (a.in[0] ? ld<C>(a.in[0], a.in_dt[0], i) : s1) : (C)0;
    C y = a.nin > 1 ? (a.in[1] ? ld<C>(a.in[1], a.in_dt[1], i) : s1) : (C)0;
    C z = a.nin > 2 ? (a.in[2] ? ld<C>(a.in[2], a.in_dt[2], i) : s1) : (C)0;
    st<C>(a.out, a.out_dt, i, Ops<C>::apply(a.op, x, y, z, s0, s1));
  }
}

// Vectorised dense binary add/sub/mul/div with an f32 output and f32 or
// bf16 inputs (residual adds of a bf16 branch into the f32 stream, grad
// accumulation): 4 elements per access, the bf16 side widened exactly.
template <typename TX, typename TY>
__device__ __forceinline__ float4 ld4(const TX* p, int64_t i);
template <>
__device__ __forceinline__ float4 ld4<float, float>(const float* p, int64_t i) { return ((const float4*)p)[i]; }
template <>
__device__ __forceinline__ float4 ld4<bf16, float>(const bf16* p, int64_t i) {
  bf16x4 v = ((const bf16x4*)p)[i];
  return float4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

template <typename TX, typename TY>
__global__ void __launch_bounds__(kThreads) binary_x4(int op, float* __restrict__ out, const TX* __restrict__ x,
                                                      const TY* __restrict__ y, float alpha, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * kThreads) {
    const float4 a = ld4<TX, float>(x, i);
    const float4 b = ld4<TY, float>(y, i);
    float4 r;
    if (op == MI355X_OP_ADD) {
      r.x = a.x + alpha * b.x; r.y = a.y + alpha * b.y; r.z = a.z + alpha * b.z; r.w = a.w + alpha * b.w;
    } else if (op == MI355X_OP_SUB) {
      r.x = a.x - alpha * b.x; r.y = a.y - alpha * b.y; r.z = a.z - alpha * b.z; r.w = a.w - alpha * b.w;
    } else if (op == MI355X_OP_MUL) {
      r.x = a.x * b.x; r.y = a.y * b.y; r.z = a.z * b.z; r.w = a.w * b.w;
    } else {
      r.x = a.x / b.x; r.y = a.y / b.y; r.z = a.z / b.z; r.w = a.w / b.w;
    }
    ((float4*)out)[i] = r;
  }
}

// Dense binary add/sub/mul/div of two bf16 tensors into bf16 (a residual
// stream kept in bf16): 8 elements per 16-byte access, computed in f32 as
// map_dense does and rounded once.
__global__ void __launch_bounds__(kThreads) binary_x8_bf16(int op, bf16* __restrict__ out, const bf16* __restrict__ x,
                                                           const bf16* __restrict__ y, float alpha, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * kThreads) {
    const bf16x8 a = ((const bf16x8*)x)[i], b = ((const bf16x8*)y)[i];
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float u = (float)a[e], v = (float)b[e];
      float w;
      if (op == MI355X_OP_ADD) w = u + alpha * v;
      else if (op == MI355X_OP_SUB) w = u - alpha * v;
      else if (op == MI355X_OP_MUL) w = u * v;
      else w = u / v;
      r[e] = (bf16)w;
    }
    ((bf16x8*)out)[i] = r;
  }
}

// out = x (op) y with y one dense row of inner4 float4s broadcast over the
// `outer` rows of x and out (a position embedding added to every sequence).
template <typename TX, typename TY>
__global__ void __launch_bounds__(kThreads) binary_x4_rows(int op, float* __restrict__ out, const TX* __restrict__ x,
                                                           const TY* __restrict__ y, float alpha, int64_t inner4,
                                                           int64_t outer) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < inner4; i += (int64_t)gridDim.x * kThreads) {
    const float4 b = ld4<TY, float>(y, i);
    for (int64_t o = blockIdx.y; o < outer; o += gridDim.y) {
      const int64_t k = o * inner4 + i;
      const float4 a = ld4<TX, float>(x, k);
      float4 r;
      if (op == MI355X_OP_ADD) {
        r.x = a.x + alpha * b.x; r.y = a.y + alpha * b.y; r.z = a.z + alpha * b.z; r.w = a.w + alpha * b.w;
      } else if (op == MI355X_OP_SUB) {
        r.x = a.x - alpha * b.x; r.y = a.y - alpha * b.y; r.z = a.z - alpha * b.z; r.w = a.w - alpha * b.w;
      } else if (op == MI355X_OP_MUL) {
        r.x = a.x * b.x; r.y = a.y * b.y; r.z = a.z * b.z; r.w = a.w * b.w;
      } else {
        r.x = a.x / b.x; r.y = a.y / b.y; r.z = a.z / b.z; r.w = a.w / b.w;
      }
      ((float4*)out)[k] = r;
    }
  }
}

// Dense casts f32 <-> bf16, 8 elements per thread-iteration.
__global__ void __launch_bounds__(kThreads) cast_f32_bf16(bf16* __restrict__ out,
                                                          const float* __restrict__ in,
                                                          int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * kThreads) {
    float4 a = ((const float4*)in)[2 * i];
    float4 b = ((const float4*)in)[2 * i + 1];
    bf16x8 r;
    r[0] = (bf16)a.x; r[1] = (bf16)a.y; r[2] = (bf16)a.z; r[3] = (bf16)a.w;
    r[4] = (bf16)b.x; r[5] = (bf16)b.y; r[6] = (bf16)b.z; r[7] = (bf16)b.w;
    ((bf16x8*)out)[i] = r;
  }
}
// out = a + r (f32, as binary_x4's add) and low = out rounded to TL, in one
// pass: the gradient sum the autograd engine forms for a residual stream,
// and the copy the next autocast linear's backward casts it to.
template <typename TR, typename TL>
__global__ void __launch_bounds__(kThreads) add_cast_x4(float* __restrict__ out, TL* __restrict__ low,
                                                        const float* __restrict__ a, const TR* __restrict__ r,
                                                        int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += (int64_t)gridDim.x * kThreads) {
    const float4 x = ((const float4*)a)[i];
    const float4 y = ld4<TR, float>(r, i);
    float4 v;
    v.x = x.x + y.x; v.y = x.y + y.y; v.z = x.z + y.z; v.w = x.w + y.w;
    ((float4*)out)[i] = v;
    float o[4] = {v.x, v.y, v.z, v.w};
    Vec4<TL>::store(low + 4 * i, o);
  }
}

__global__ void __launch_bounds__(kThreads) cast_bf16_f32(float* __restrict__ out,
                                                          const bf16* __restrict__ in,
                                                          int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * kThreads) {
    bf16x8 v = ((const bf16x8*)in)[i];
    float4 a, b;
    a.x = (float)v[0]; a.y = (float)v[1]; a.z = (float)v[2]; a.w = (float)v[3];
    b.x = (float)v[4]; b.y = (float)v[5]; b.z = (float)v[6]; b.w = (float)v[7];
    ((float4*)out)[2 * i] = a;
    ((float4*)out)[2 * i + 1] = b;
  }
}
// Same-dtype copy of `rows` rows of `row_bytes` (16-byte multiples) between
// row strides (slices, concatenation): one 64-lane wave per row.
__global__ void __launch_bounds__(kThreads) copy_rows_b128(uint8_t* __restrict__ dst, int64_t dst_rs,
                                                           const uint8_t* __restrict__ src, int64_t src_rs,
                                                           int64_t rows, int64_t row_bytes) {
  const int lane = threadIdx.x & 63;
  const int64_t nv = row_bytes / 16;
  for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += (int64_t)gridDim.x * 4) {
    const uint4* s = (const uint4*)(src + r * src_rs);
    uint4* d = (uint4*)(dst + r * dst_rs);
    for (int64_t k = lane; k < nv; k += 64) d[k] = s[k];
  }
}

// Dense same-dtype copy, 16 bytes per thread-iteration.
__global__ void __launch_bounds__(kThreads) copy_b128(uint4* __restrict__ out,
                                                      const uint4* __restrict__ in, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * kThreads)
    out[i] = in[i];
}
__global__ void __launch_bounds__(kThreads) copy_bytes(uint8_t* __restrict__ out,
                                                       const uint8_t* __restrict__ in, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    out[i] = in[i];
}

template <typename C>
__global__ void __launch_bounds__(kThreads) arange_kernel(void* out, int dt, int64_t n, double start,
                                                          double step) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    st<C>(out, dt, i, (C)(start + step * (double)i));
}

int compute_kind(int out_dt, int nin, const int* in_dts) {
  bool any_f64 = out_dt == MI355X_F64;
  bool all_int = true;
  for (int j = 0; j < nin; ++j) {
    if (in_dts[j] == MI355X_F64) any_f64 = true;
    if (is_float_dtype(in_dts[j])) all_int = false;
  }
  if (is_float_dtype(out_dt)) all_int = false;
  if (any_f64) return 1;
  if (all_int) return 2;
  return 0;
}

int launch_map(const MapArgs& a, const Geo& g, int64_t n, int kind, hipStream_t s) {
  if (n == 0) return MI355X_OK;
  const unsigned grid = grid_for(n, 4);
  if (geo_dense(g)) {
    if (kind == 0) map_dense<float><<<grid, kThreads, 0, s>>>(a, n);
    else if (kind == 1) map_dense<double><<<grid, kThreads, 0, s>>>(a, n);
    else map_dense<int64_t><<<grid, kThreads, 0, s>>>(a, n);
  } else if (n < (int64_t)1 << 31) {
    if (kind == 0) map_strided<float, uint32_t><<<grid, kThreads, 0, s>>>(a, g, (uint32_t)n);
    else if (kind == 1) map_strided<double, uint32_t><<<grid, kThreads, 0, s>>>(a, g, (uint32_t)n);
    else map_strided<int64_t, uint32_t><<<grid, kThreads, 0, s>>>(a, g, (uint32_t)n);
  } else {
    if (kind == 0) map_strided<float, int64_t><<<grid, kThreads, 0, s>>>(a, g, n);
    else if (kind == 1) map_strided<double, int64_t><<<grid, kThreads, 0, s>>>(a, g, n);
    else map_strided<int64_t, int64_t><<<grid, kThreads, 0, s>>>(a, g, n);
  }
  return check_launch("mi355x_map");
}

bool valid_dtype(int dt) { return dt >= MI355X_F32 && dt <= MI355X_BOOL; }

inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi355x_copy(void* dst, int dst_dtype, const int64_t* dst_strides, const void* src,
                           int src_dtype, const int64_t* src_strides, const int64_t* shape,
                           int ndim, mi355x_stream_t stream) {
  MI_REQUIRE(valid_dtype(dst_dtype) && valid_dtype(src_dtype), "mi355x_copy: bad dtype");
  const int64_t* strides[2] = {dst_strides, src_strides};
  Geo g;
  int64_t n;
  int rc = build_geo(g, 2, strides, shape, ndim, &n);
  if (rc) return rc;
  if (n == 0) return MI355X_OK;
  MI_REQUIRE(dst && src, "mi355x_copy: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (geo_dense(g)) {
    if (dst_dtype == src_dtype) {
      const int64_t bytes = n * (int64_t)dtype_size(dst_dtype);
      if (bytes % 16 == 0 && aligned(dst, 16) && aligned(src, 16)) {
        copy_b128<<<grid_for(bytes / 16, 4), kThreads, 0, s>>>((uint4*)dst, (const uint4*)src,
                                                                 bytes / 16);
      } else {
        copy_bytes<<<grid_for(bytes, 8), kThreads, 0, s>>>((uint8_t*)dst, (const uint8_t*)src,
                                                             bytes);
      }
      return check_launch("mi355x_copy");
    }
    if (n % 8 == 0 && aligned(dst, 32) && aligned(src, 32)) {
      if (dst_dtype == MI355X_BF16 && src_dtype == MI355X_F32) {
        cast_f32_bf16<<<grid_for(n / 8, 2), kThreads, 0, s>>>((bf16*)dst, (const float*)src, n / 8);
        return check_launch("mi355x_copy");
      }
      if (dst_dtype == MI355X_F32 && src_dtype == MI355X_BF16) {
        cast_bf16_f32<<<grid_for(n / 8, 2), kThreads, 0, s>>>((float*)dst, (const bf16*)src, n / 8);
        return check_launch("mi355x_copy");
      }
    }
  }
  if (g.ndim == 2 && dst_dtype == src_dtype && g.st[0][1] == 1 && g.st[1][1] == 1) {
    const int64_t es = (int64_t)dtype_size(dst_dtype);
    const int64_t rb = g.shape[1] * es, drs = g.st[0][0] * es, srs = g.st[1][0] * es;
    if (rb % 16 == 0 && drs % 16 == 0 && srs % 16 == 0 && aligned(dst, 16) && aligned(src, 16)) {
      int64_t blocks = (g.shape[0] + 3) / 4;
      if (blocks > 65536) blocks = 65536;
      copy_rows_b128<<<(unsigned)blocks, kThreads, 0, s>>>((uint8_t*)dst, drs, (const uint8_t*)src, srs,
                                                            g.shape[0], rb);
      return check_launch("mi355x_copy");
    }
  }
  MapArgs a{};
  a.op = MI355X_OP_IDENTITY;
  a.nin = 1;
  a.out = dst;
  a.out_dt = dst_dtype;
  a.in[0] = src;
  a.in_dt[0] = src_dtype;
  // Casting integer <- integer and float <- float keeps the widest exact type.
  int kind = compute_kind(dst_dtype, 1, &src_dtype);
  if (kind == 0 && (dst_dtype == MI355X_I64 || src_dtype == MI355X_I64)) kind = 1;
  return launch_map(a, g, n, kind, s);
}

extern "C" int mi355x_fill(void* dst, int dtype, const int64_t* strides, const int64_t* shape,
                           int ndim, double value, mi355x_stream_t stream) {
  MI_REQUIRE(valid_dtype(dtype), "mi355x_fill: bad dtype");
  const int64_t* st1[1] = {strides};
  Geo g;
  int64_t n;
  int rc = build_geo(g, 1, st1, shape, ndim, &n);
  if (rc) return rc;
  if (n == 0) return MI355X_OK;
  MI_REQUIRE(dst, "mi355x_fill: null pointer");
  MapArgs a{};
  a.op = MI355X_OP_IDENTITY;
  a.nin = 0;
  a.out = dst;
  a.out_dt = dtype;
  // With nin == 0 the map evaluates IDENTITY on 0; use ADD: 0 + s0*1 needs b.
  // Instead express fill as RSUB: s0 - a*s1 with a = 0.
  a.op = MI355X_OP_RSUB;
  a.s0 = value;
  a.s1 = 0.0;
  int kind = (dtype == MI355X_F64) ? 1 : (is_float_dtype(dtype) ? 0 : 2);
  return launch_map(a, g, n, kind, (hipStream_t)stream);
}

extern "C" int mi355x_arange(void* dst, int dtype, int64_t n, double start, double step,
                             mi355x_stream_t stream) {
  MI_REQUIRE(valid_dtype(dtype), "mi355x_arange: bad dtype");
  MI_REQUIRE(n >= 0, "mi355x_arange: negative length");
  if (n == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  if (is_float_dtype(dtype))
    arange_kernel<double><<<grid_for(n), kThreads, 0, s>>>(dst, dtype, n, start, step);
  else
    arange_kernel<int64_t><<<grid_for(n), kThreads, 0, s>>>(dst, dtype, n, start, step);
  return check_launch("mi355x_arange");
}

extern "C" int mi355x_add_cast(float* out, void* low, int low_dtype, const float* a, const void* r, int r_dtype,
                               int64_t n, mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0, "mi355x_add_cast: negative size");
  if (n == 0) return MI355X_OK;
  MI_REQUIRE(out && low && a && r, "mi355x_add_cast: null pointer");
  MI_REQUIRE(low_dtype == MI355X_BF16 || low_dtype == MI355X_F16, "mi355x_add_cast: the copy must be bf16 or f16");
  MI_REQUIRE(r_dtype == MI355X_F32 || r_dtype == MI355X_BF16, "mi355x_add_cast: r must be f32 or bf16");
  MI_REQUIRE(n % 4 == 0 && aligned(out, 16) && aligned(a, 16) && aligned(low, 8) &&
                 aligned(r, r_dtype == MI355X_F32 ? 16 : 8),
             "mi355x_add_cast: needs a multiple of 4 elements and aligned vectors");
  hipStream_t s = (hipStream_t)stream;
  const unsigned grid = grid_for(n / 4, 2);
  if (r_dtype == MI355X_F32) {
    if (low_dtype == MI355X_BF16) add_cast_x4<float, bf16><<<grid, kThreads, 0, s>>>(out, (bf16*)low, a, (const float*)r, n / 4);
    else add_cast_x4<float, f16><<<grid, kThreads, 0, s>>>(out, (f16*)low, a, (const float*)r, n / 4);
  } else {
    if (low_dtype == MI355X_BF16) add_cast_x4<bf16, bf16><<<grid, kThreads, 0, s>>>(out, (bf16*)low, a, (const bf16*)r, n / 4);
    else add_cast_x4<bf16, f16><<<grid, kThreads, 0, s>>>(out, (f16*)low, a, (const bf16*)r, n / 4);
  }
  return check_launch("mi355x_add_cast");
}

extern "C" int mi355x_map(int op, void* out, int out_dtype, int nin, const void* const* ins,
                          const int* in_dtypes, const int64_t* strides, const int64_t* shape,
                          int ndim, double s0, double s1, mi355x_stream_t stream) {
  MI_REQUIRE(nin >= 0 && nin <= 3, "mi355x_map: nin must be 0..3");
  MI_REQUIRE(valid_dtype(out_dtype), "mi355x_map: bad out dtype");
  for (int j = 0; j < nin; ++j) MI_REQUIRE(valid_dtype(in_dtypes[j]), "mi355x_map: bad in dtype");
  MI_REQUIRE(ndim >= 0 && ndim <= MI355X_MAX_RANK, "mi355x_map: bad rank %d", ndim);
  const int64_t* st[kMaxOperands];
  for (int j = 0; j <= nin; ++j) st[j] = strides + (int64_t)j * ndim;
  Geo g;
  int64_t n;
  int rc = build_geo(g, nin + 1, st, shape, ndim, &n);
  if (rc) return rc;
  if (n == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  const int kind = compute_kind(out_dtype, nin, in_dtypes);
  // Integer arithmetic cannot express true division and transcendental ops.
  if (kind == 2) {
    switch (op) {
      case MI355X_OP_DIV: case MI355X_OP_POW: case MI355X_OP_ADDCDIV: case MI355X_OP_LERP:
      case MI355X_OP_EXP: case MI355X_OP_LOG: case MI355X_OP_SQRT: case MI355X_OP_RSQRT:
      case MI355X_OP_RECIPROCAL: case MI355X_OP_SIN: case MI355X_OP_COS: case MI355X_OP_TANH:
      case MI355X_OP_SIGMOID: case MI355X_OP_ERF: case MI355X_OP_SILU: case MI355X_OP_POW_SCALAR:
        return fail(MI355X_EUNSUPPORTED, "mi355x_map: op %d needs a floating output", op);
    }
  }
  const auto f32_or_bf16 = [](int d) { return d == MI355X_F32 || d == MI355X_BF16; };
  if (g.ndim == 1 && geo_dense(g) && nin == 2 && ins[0] && ins[1] && out_dtype == MI355X_F32 &&
      f32_or_bf16(in_dtypes[0]) && f32_or_bf16(in_dtypes[1]) && n % 4 == 0 && aligned(out, 16) &&
      aligned(ins[0], 8) && aligned(ins[1], 8) &&
      (in_dtypes[0] == MI355X_BF16 || aligned(ins[0], 16)) && (in_dtypes[1] == MI355X_BF16 || aligned(ins[1], 16)) &&
      (op == MI355X_OP_ADD || op == MI355X_OP_SUB || op == MI355X_OP_MUL || op == MI355X_OP_DIV)) {
    const unsigned grid = grid_for(n / 4, 2);
    const float al = (float)s0;
    float* o = (float*)out;
    const bool xb = in_dtypes[0] == MI355X_BF16, yb = in_dtypes[1] == MI355X_BF16;
    if (!xb && !yb) binary_x4<float, float><<<grid, kThreads, 0, s>>>(op, o, (const float*)ins[0], (const float*)ins[1], al, n / 4);
    else if (!xb) binary_x4<float, bf16><<<grid, kThreads, 0, s>>>(op, o, (const float*)ins[0], (const bf16*)ins[1], al, n / 4);
    else if (!yb) binary_x4<bf16, float><<<grid, kThreads, 0, s>>>(op, o, (const bf16*)ins[0], (const float*)ins[1], al, n / 4);
    else binary_x4<bf16, bf16><<<grid, kThreads, 0, s>>>(op, o, (const bf16*)ins[0], (const bf16*)ins[1], al, n / 4);
    return check_launch("mi355x_map");
  }
  if (g.ndim == 1 && geo_dense(g) && nin == 2 && ins[0] && ins[1] && out_dtype == MI355X_BF16 &&
      in_dtypes[0] == MI355X_BF16 && in_dtypes[1] == MI355X_BF16 && n % 8 == 0 && aligned(out, 16) &&
      aligned(ins[0], 16) && aligned(ins[1], 16) &&
      (op == MI355X_OP_ADD || op == MI355X_OP_SUB || op == MI355X_OP_MUL || op == MI355X_OP_DIV)) {
    binary_x8_bf16<<<grid_for(n / 8, 2), kThreads, 0, s>>>(op, (bf16*)out, (const bf16*)ins[0], (const bf16*)ins[1],
                                                          (float)s0, n / 8);
    return check_launch("mi355x_map");
  }
  // y one dense row broadcast over the rows of a dense x and out
  if (g.ndim == 2 && nin == 2 && ins[0] && ins[1] && out_dtype == MI355X_F32 && f32_or_bf16(in_dtypes[0]) &&
      f32_or_bf16(in_dtypes[1]) && g.st[0][1] == 1 && g.st[1][1] == 1 && g.st[2][1] == 1 &&
      g.st[0][0] == g.shape[1] && g.st[1][0] == g.shape[1] && g.st[2][0] == 0 && g.shape[1] % 4 == 0 &&
      aligned(out, 16) && aligned(ins[0], 16) && aligned(ins[1], 16) &&
      (op == MI355X_OP_ADD || op == MI355X_OP_SUB || op == MI355X_OP_MUL || op == MI355X_OP_DIV)) {
    const int64_t inner4 = g.shape[1] / 4, outer = g.shape[0];
    const unsigned gx = grid_for(inner4);
    int64_t gy = 4096 / gx;
    gy = gy < 1 ? 1 : (gy > outer ? outer : (gy > 65535 ? 65535 : gy));
    const dim3 grid(gx, (unsigned)gy);
    const float al = (float)s0;
    float* o = (float*)out;
    const bool xb = in_dtypes[0] == MI355X_BF16, yb = in_dtypes[1] == MI355X_BF16;
    if (!xb && !yb) binary_x4_rows<float, float><<<grid, kThreads, 0, s>>>(op, o, (const float*)ins[0], (const float*)ins[1], al, inner4, outer);
    else if (!xb) binary_x4_rows<float, bf16><<<grid, kThreads, 0, s>>>(op, o, (const float*)ins[0], (const bf16*)ins[1], al, inner4, outer);
    else if (!yb) binary_x4_rows<bf16, float><<<grid, kThreads, 0, s>>>(op, o, (const bf16*)ins[0], (const float*)ins[1], al, inner4, outer);
    else binary_x4_rows<bf16, bf16><<<grid, kThreads, 0, s>>>(op, o, (const bf16*)ins[0], (const bf16*)ins[1], al, inner4, outer);
    return check_launch("mi355x_map");
  }
  MapArgs a{};
  a.op = op;
  a.nin = nin;
  a.out = out;
  a.out_dt = out_dtype;
  for (int j = 0; j < nin; ++j) {
    a.in[j] = ins[j];
    a.in_dt[j] = in_dtypes[j];
  }
  a.s0 = s0;
  a.s1 = s1;
  return launch_map(a, g, n, kind, s);
}
