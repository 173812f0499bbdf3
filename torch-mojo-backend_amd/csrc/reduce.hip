// Reductions over the middle axis of an [outer, r, inner] strided view, and
// arg-reductions.
//
// inner == 1 (row reduction): one 256-thread block per (o, r-split).
// inner  > 1 (column reduction, e.g. the bias gradient sum over tokens): a
//   block covers 64 consecutive columns x 4 row-lanes, so each load
//   instruction reads 64 consecutive elements.
// When outer*inner alone cannot fill the chip, r is split into chunks whose
// partials land in a workspace [splits, outer, inner] and a second kernel
// combines them in split order (deterministic, no atomics).
#include <math.h>

#include "common.h"

namespace mi {
namespace {

constexpr int kThreads = 256;
constexpr int kTargetBlocks = 2048;

template <typename A>
struct RedOp {
  int op;
  __device__ __forceinline__ A init() const {
    switch (op) {
      case MI355X_RED_MAX: return lowest();
      case MI355X_RED_MIN: return highest();
      case MI355X_RED_PROD: case MI355X_RED_ALL: return (A)1;
      default: return (A)0;
    }
  }
  static __device__ __forceinline__ A lowest();
  static __device__ __forceinline__ A highest();
  // Fold one input value.
  __device__ __forceinline__ A fold(A acc, A v) const {
    switch (op) {
      case MI355X_RED_SUM: case MI355X_RED_MEAN: return acc + v;
      case MI355X_RED_MAX: return is_nan(acc) ? acc : (is_nan(v) || v > acc ? v : acc);
      case MI355X_RED_MIN: return is_nan(acc) ? acc : (is_nan(v) || v < acc ? v : acc);
      case MI355X_RED_NORM2: case MI355X_RED_SUMSQ: return acc + v * v;
      case MI355X_RED_AMAX: { A a = v < (A)0 ? -v : v; return is_nan(acc) ? acc : (is_nan(a) || a > acc ? a : acc); }
      case MI355X_RED_PROD: return acc * v;
      case MI355X_RED_ANY: return (acc != (A)0 || v != (A)0) ? (A)1 : (A)0;
      case MI355X_RED_ALL: return (acc != (A)0 && v != (A)0) ? (A)1 : (A)0;
      case MI355X_RED_NORM1: return acc + (v < (A)0 ? -v : v);
    }
    return acc;
  }
  // Combine two partial accumulators.
  __device__ __forceinline__ A combine(A a, A b) const {
    switch (op) {
      case MI355X_RED_MAX: case MI355X_RED_AMAX:
        return is_nan(a) ? a : (is_nan(b) || b > a ? b : a);
      case MI355X_RED_MIN: return is_nan(a) ? a : (is_nan(b) || b < a ? b : a);
      case MI355X_RED_PROD: return a * b;
      case MI355X_RED_ANY: return (a != (A)0 || b != (A)0) ? (A)1 : (A)0;
      case MI355X_RED_ALL: return (a != (A)0 && b != (A)0) ? (A)1 : (A)0;
      default: return a + b;
    }
  }
  __device__ __forceinline__ A finish(A acc, int64_t r) const {
    if (op == MI355X_RED_MEAN) return acc / (A)r;
    if (op == MI355X_RED_NORM2) return (A)sqrt((double)acc);
    return acc;
  }
  static __device__ __forceinline__ bool is_nan(A x) { return x != x; }
};
template <> __device__ __forceinline__ float RedOp<float>::lowest() { return -INFINITY; }
template <> __device__ __forceinline__ float RedOp<float>::highest() { return INFINITY; }
template <> __device__ __forceinline__ double RedOp<double>::lowest() { return -INFINITY; }
template <> __device__ __forceinline__ double RedOp<double>::highest() { return INFINITY; }
template <> __device__ __forceinline__ int64_t RedOp<int64_t>::lowest() { return INT64_MIN; }
template <> __device__ __forceinline__ int64_t RedOp<int64_t>::highest() { return INT64_MAX; }
template <> __device__ __forceinline__ float RedOp<float>::finish(float acc, int64_t r) const {
  if (op == MI355X_RED_MEAN) return acc / (float)r;
  if (op == MI355X_RED_NORM2) return sqrtf(acc);
  return acc;
}

template <typename A>
__device__ __forceinline__ A load_as(const void* p, int dt, int64_t i) {
  switch (dt) {
    case MI355X_F32: return (A)((const float*)p)[i];
    case MI355X_BF16: return (A)(float)((const bf16*)p)[i];
    case MI355X_F16: return (A)(float)((const f16*)p)[i];
    case MI355X_F64: return (A)((const double*)p)[i];
    case MI355X_I64: return (A)((const int64_t*)p)[i];
    case MI355X_I32: return (A)((const int32_t*)p)[i];
    case MI355X_I16: return (A)((const int16_t*)p)[i];
    case MI355X_I8: return (A)((const int8_t*)p)[i];
    case MI355X_U8: return (A)((const uint8_t*)p)[i];
    default: return (A)(((const uint8_t*)p)[i] != 0);
  }
}
template <typename A>
__device__ __forceinline__ void store_as(void* p, int dt, int64_t i, A v) {
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
    default: ((uint8_t*)p)[i] = (v != (A)0) ? 1 : 0; break;
  }
}

struct RedArgs {
  int op;
  const void* in;
  int in_dt;
  void* out;   // final output (splits == 1) ...
  int out_dt;
  void* part;  // ... or partials [splits, outer, inner] of type A
  int64_t outer, r, inner, s_o, s_r, s_i;
  int64_t chunk;  // r per split
};

// inner == 1: block per (o, split)
template <typename A>
__global__ void __launch_bounds__(kThreads) reduce_rows(RedArgs a) {
  __shared__ A red[kThreads / 64];
  const RedOp<A> R{a.op};
  const int64_t o = blockIdx.x;
  const int split = blockIdx.y;
  const int64_t r0 = (int64_t)split * a.chunk;
  const int64_t r1 = min(a.r, r0 + a.chunk);
  A acc = R.init();
  const int64_t base = o * a.s_o;
  for (int64_t r = r0 + threadIdx.x; r < r1; r += kThreads)
    acc = R.fold(acc, load_as<A>(a.in, a.in_dt, base + r * a.s_r));
  // wave combine
  for (int off = 32; off > 0; off >>= 1) acc = R.combine(acc, __shfl_xor(acc, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    A t = red[0];
    for (int w = 1; w < kThreads / 64; ++w) t = R.combine(t, red[w]);
    if (a.part) ((A*)a.part)[(int64_t)split * a.outer + o] = t;
    else store_as<A>(a.out, a.out_dt, o, R.finish(t, a.r));
  }
}

// inner > 1: block covers 64 columns x 4 row lanes
template <typename A>
__global__ void __launch_bounds__(kThreads) reduce_cols(RedArgs a) {
  __shared__ A red[4][64];
  const RedOp<A> R{a.op};
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t i = (int64_t)blockIdx.x * 64 + tx;
  const int64_t o = blockIdx.y;
  const int split = blockIdx.z;
  const int64_t r0 = (int64_t)split * a.chunk;
  const int64_t r1 = min(a.r, r0 + a.chunk);
  A acc = R.init();
  if (i < a.inner) {
    const int64_t base = o * a.s_o + i * a.s_i;
    for (int64_t r = r0 + ty; r < r1; r += 4) acc = R.fold(acc, load_as<A>(a.in, a.in_dt, base + r * a.s_r));
  }
  red[ty][tx] = acc;
  __syncthreads();
  if (ty == 0 && i < a.inner) {
    A t = red[0][tx];
    for (int w = 1; w < 4; ++w) t = R.combine(t, red[w][tx]);
    const int64_t oi = o * a.inner + i;
    if (a.part) ((A*)a.part)[(int64_t)split * a.outer * a.inner + oi] = t;
    else store_as<A>(a.out, a.out_dt, oi, R.finish(t, a.r));
  }
}

// Sum over rows of a dense [r, inner] f32/bf16/f16 matrix (the bias gradient
// sum(dY, 0)): a thread owns 8 consecutive columns (one 16-byte load per row
// for 16-bit types, two for f32); 32 column groups x 8 row lanes per block,
// row lanes combined through LDS in a fixed order.
template <typename T>
__global__ void __launch_bounds__(kThreads) colsum8(RedArgs a) {
  __shared__ float red[8][32][9];
  const int cg = threadIdx.x & 31, rl = threadIdx.x >> 5;
  const int64_t c0 = ((int64_t)blockIdx.x * 32 + cg) * 8;
  const int split = blockIdx.y;
  const int64_t r0 = (int64_t)split * a.chunk;
  const int64_t r1 = min(a.r, r0 + a.chunk);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c0 < a.inner) {
    const T* base = (const T*)a.in + c0;
    for (int64_t r = r0 + rl; r < r1; r += 8) {
      struct alignas(16) P { T v[8]; } p = *(const P*)(base + r * a.inner);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += to_f32(p.v[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[rl][cg][e] = acc[e];
  __syncthreads();
  if (rl == 0 && c0 < a.inner) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = red[0][cg][e];
      for (int w = 1; w < 8; ++w) t += red[w][cg][e];
      if (a.part) ((float*)a.part)[(int64_t)split * a.inner + c0 + e] = t;
      else store_as<float>(a.out, a.out_dt, c0 + e, t);
    }
  }
}

// Sum colsum8's per-split partials [splits][inner]: 32 columns x 8 split
// lanes per block; lane l adds splits l, l+8, ... and the lanes are combined
// in a fixed order, so the result does not depend on scheduling.
__global__ void __launch_bounds__(kThreads) colsum_combine(RedArgs a, int splits) {
  __shared__ float red[8][33];
  const int cx = threadIdx.x & 31, sl = threadIdx.x >> 5;
  const int64_t c = (int64_t)blockIdx.x * 32 + cx;
  float t = 0.f;
  if (c < a.inner)
    for (int sp = sl; sp < splits; sp += 8) t += ((const float*)a.part)[(int64_t)sp * a.inner + c];
  red[sl][cx] = t;
  __syncthreads();
  if (sl == 0 && c < a.inner) {
    for (int w = 1; w < 8; ++w) t += red[w][cx];
    store_as<float>(a.out, a.out_dt, c, t);
  }
}

template <typename A>
__global__ void __launch_bounds__(kThreads) reduce_combine(RedArgs a, int splits) {
  const RedOp<A> R{a.op};
  const int64_t n = a.outer * a.inner;
  for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < n; k += (int64_t)gridDim.x * kThreads) {
    A t = ((const A*)a.part)[k];
    for (int s = 1; s < splits; ++s) t = R.combine(t, ((const A*)a.part)[(int64_t)s * n + k]);
    store_as<A>(a.out, a.out_dt, k, R.finish(t, a.r));
  }
}

int acc_kind(int op, int in_dt) {
  if (in_dt == MI355X_F64) return 1;
  if (!is_float_dtype(in_dt)) {
    if (op == MI355X_RED_MEAN || op == MI355X_RED_NORM2) return 0;
    return 2;
  }
  return 0;
}

void plan(int64_t outer, int64_t r, int64_t inner, int* splits, int64_t* chunk) {
  const int64_t base = inner == 1 ? outer : ((inner + 63) / 64) * outer;
  const int64_t min_chunk = inner == 1 ? 2048 : 256;
  int64_t s = 1;
  if (base < kTargetBlocks && r > min_chunk) {
    s = (kTargetBlocks + base - 1) / base;
    const int64_t max_s = (r + min_chunk - 1) / min_chunk;
    if (s > max_s) s = max_s;
    if (s > 1024) s = 1024;
  }
  if (s < 1) s = 1;
  int64_t c = (r + s - 1) / s;
  if (c < 1) c = 1;
  *splits = (int)((r + c - 1) / c);
  if (*splits < 1) *splits = 1;
  *chunk = c;
}

// Dense column sums: about 1024 blocks of 256 columns x (chunk) rows, at
// least 32 rows per block.
void colsum_plan(int64_t r, int64_t inner, int* splits, int64_t* chunk) {
  const int64_t gx = (inner + 255) / 256;
  int64_t s = (1024 + gx - 1) / gx;
  const int64_t max_s = (r + 31) / 32;
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  int64_t c = (r + s - 1) / s;
  if (c < 1) c = 1;
  *splits = (int)((r + c - 1) / c);
  if (*splits < 1) *splits = 1;
  *chunk = c;
}

template <typename A>
int run(RedArgs a, int splits, hipStream_t s) {
  if (splits > 1) {
    if (a.inner == 1) reduce_rows<A><<<dim3((unsigned)a.outer, splits), kThreads, 0, s>>>(a);
    else reduce_cols<A><<<dim3(ceil_div(a.inner, 64), (unsigned)a.outer, splits), kThreads, 0, s>>>(a);
    const int64_t n = a.outer * a.inner;
    int64_t g = (n + kThreads - 1) / kThreads;
    if (g > 4096) g = 4096;
    reduce_combine<A><<<(unsigned)g, kThreads, 0, s>>>(a, splits);
  } else {
    a.part = nullptr;
    if (a.inner == 1) reduce_rows<A><<<dim3((unsigned)a.outer, 1), kThreads, 0, s>>>(a);
    else reduce_cols<A><<<dim3(ceil_div(a.inner, 64), (unsigned)a.outer, 1), kThreads, 0, s>>>(a);
  }
  return check_launch("mi355x_reduce");
}

// ---------------------------------------------------------------------------
// arg-reductions
// ---------------------------------------------------------------------------
template <typename A>
__device__ __forceinline__ bool better(bool is_min, A v, int64_t vi, A b, int64_t bi) {
  const bool vn = v != v, bn = b != b;
  if (bn) return vn && vi < bi;  // first NaN wins
  if (vn) return true;
  if (is_min ? (v < b) : (v > b)) return true;
  return v == b && vi < bi;
}

template <typename A>
__global__ void __launch_bounds__(kThreads) argreduce_rows(int is_min, int64_t* out_idx, void* out_val,
                                                          const void* in, int dt, int64_t r,
                                                          int64_t s_o, int64_t s_r) {
  __shared__ A sv[kThreads];
  __shared__ int64_t si[kThreads];
  const int64_t o = blockIdx.x;
  A best = load_as<A>(in, dt, o * s_o);
  int64_t bi = 0;
  for (int64_t k = threadIdx.x; k < r; k += kThreads) {
    A v = load_as<A>(in, dt, o * s_o + k * s_r);
    if (better<A>(is_min, v, k, best, bi)) best = v, bi = k;
  }
  sv[threadIdx.x] = best;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      A v = sv[threadIdx.x + w];
      int64_t vi = si[threadIdx.x + w];
      if (better<A>(is_min, v, vi, sv[threadIdx.x], si[threadIdx.x])) sv[threadIdx.x] = v, si[threadIdx.x] = vi;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out_idx[o] = si[0];
    if (out_val) store_as<A>(out_val, dt, o, sv[0]);
  }
}

template <typename A>
__global__ void __launch_bounds__(kThreads) argreduce_cols(int is_min, int64_t* out_idx, void* out_val,
                                                          const void* in, int dt, int64_t outer,
                                                          int64_t r, int64_t inner, int64_t s_o,
                                                          int64_t s_r, int64_t s_i) {
  const int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (k >= outer * inner) return;
  const int64_t o = k / inner, i = k % inner;
  const int64_t base = o * s_o + i * s_i;
  A best = load_as<A>(in, dt, base);
  int64_t bi = 0;
  for (int64_t j = 1; j < r; ++j) {
    A v = load_as<A>(in, dt, base + j * s_r);
    if (better<A>(is_min, v, j, best, bi)) best = v, bi = j;
  }
  out_idx[k] = bi;
  if (out_val) store_as<A>(out_val, dt, k, best);
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int64_t mi355x_reduce_workspace_bytes(int64_t outer, int64_t r, int64_t inner) {
  int splits;
  int64_t chunk;
  plan(outer, r, inner, &splits, &chunk);
  int64_t need = splits <= 1 ? 0 : (int64_t)splits * outer * inner * 8;
  if (outer == 1 && inner > 1) {  // the dense column-sum path may split further
    colsum_plan(r, inner, &splits, &chunk);
    if (splits > 1 && (int64_t)splits * inner * 4 > need) need = (int64_t)splits * inner * 4;
  }
  return need;
}

extern "C" int mi355x_reduce(int op, void* out, int out_dtype, const void* in, int in_dtype,
                             int64_t outer, int64_t r, int64_t inner, int64_t s_o, int64_t s_r,
                             int64_t s_i, void* workspace, int64_t ws_bytes,
                             mi355x_stream_t stream) {
  MI_REQUIRE(op >= MI355X_RED_SUM && op <= MI355X_RED_NORM1, "mi355x_reduce: bad op %d", op);
  MI_REQUIRE(outer >= 0 && r >= 0 && inner >= 0, "mi355x_reduce: negative extent");
  if (outer * inner == 0) return MI355X_OK;
  MI_REQUIRE(outer < (1ll << 31), "mi355x_reduce: outer too large");
  int splits;
  int64_t chunk;
  plan(outer, r, inner, &splits, &chunk);
  if (splits > 1) {
    const int64_t need = mi355x_reduce_workspace_bytes(outer, r, inner);
    if (!workspace || ws_bytes < need)
      return fail(MI355X_EWORKSPACE, "mi355x_reduce: workspace %lld < %lld", (long long)ws_bytes,
                  (long long)need);
  }
  RedArgs a{op, in, in_dtype, out, out_dtype, workspace, outer, r, inner, s_o, s_r, s_i, chunk};
  hipStream_t s = (hipStream_t)stream;
  // Dense column sums (bias gradients): vectorised kernel, own split plan.
  if (op == MI355X_RED_SUM && outer == 1 && inner > 1 && inner % 8 == 0 && s_i == 1 &&
      s_r == inner && ((uintptr_t)in % 16) == 0 &&
      (in_dtype == MI355X_F32 || in_dtype == MI355X_BF16 || in_dtype == MI355X_F16)) {
    colsum_plan(r, inner, &splits, &chunk);
    a.chunk = chunk;
    if (splits > 1) {
      const int64_t need = mi355x_reduce_workspace_bytes(outer, r, inner);
      if (!workspace || ws_bytes < need)
        return fail(MI355X_EWORKSPACE, "mi355x_reduce: workspace %lld < %lld", (long long)ws_bytes,
                    (long long)need);
    } else {
      a.part = nullptr;
    }
    dim3 grid(ceil_div(inner, 256), splits);
    if (in_dtype == MI355X_F32) colsum8<float><<<grid, kThreads, 0, s>>>(a);
    else if (in_dtype == MI355X_BF16) colsum8<bf16><<<grid, kThreads, 0, s>>>(a);
    else colsum8<f16><<<grid, kThreads, 0, s>>>(a);
    if (splits > 1) colsum_combine<<<ceil_div(inner, 32), kThreads, 0, s>>>(a, splits);
    return check_launch("mi355x_reduce");
  }
  switch (acc_kind(op, in_dtype)) {
    case 1: return run<double>(a, splits, s);
    case 2: return run<int64_t>(a, splits, s);
    default: return run<float>(a, splits, s);
  }
}

extern "C" int mi355x_argreduce(int is_min, int64_t* out_idx, void* out_val, const void* in,
                                int dtype, int64_t outer, int64_t r, int64_t inner, int64_t s_o,
                                int64_t s_r, int64_t s_i, mi355x_stream_t stream) {
  MI_REQUIRE(r > 0, "mi355x_argreduce: empty reduction");
  if (outer * inner == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool f64 = dtype == MI355X_F64;
  const bool integral = !is_float_dtype(dtype);
  if (inner == 1) {
    MI_REQUIRE(outer < (1ll << 31), "mi355x_argreduce: outer too large");
    if (f64) argreduce_rows<double><<<(unsigned)outer, kThreads, 0, s>>>(is_min, out_idx, out_val, in, dtype, r, s_o, s_r);
    else if (integral) argreduce_rows<int64_t><<<(unsigned)outer, kThreads, 0, s>>>(is_min, out_idx, out_val, in, dtype, r, s_o, s_r);
    else argreduce_rows<float><<<(unsigned)outer, kThreads, 0, s>>>(is_min, out_idx, out_val, in, dtype, r, s_o, s_r);
  } else {
    const unsigned g = ceil_div(outer * inner, kThreads);
    if (f64) argreduce_cols<double><<<g, kThreads, 0, s>>>(is_min, out_idx, out_val, in, dtype, outer, r, inner, s_o, s_r, s_i);
    else if (integral) argreduce_cols<int64_t><<<g, kThreads, 0, s>>>(is_min, out_idx, out_val, in, dtype, outer, r, inner, s_o, s_r, s_i);
    else argreduce_cols<float><<<g, kThreads, 0, s>>>(is_min, out_idx, out_val, in, dtype, outer, r, inner, s_o, s_r, s_i);
  }
  return check_launch("mi355x_argreduce");
}
