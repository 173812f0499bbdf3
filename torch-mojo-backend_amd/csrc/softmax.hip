// Row softmax / log_softmax forward and backward over the contiguous last dim.
//
// Forward is two passes over the row: an online (max, sum-of-exp) pass whose
// per-lane partials are merged with the usual rescaling, then the output pass
//   log:     y = x - max - log(sum)
//   softmax: y = exp(x - max) / sum
// Backward: one pass for the row sum, one for the output
//   log:     dx = dy - exp(y) * sum(dy)
//   softmax: dx = y * (dy - sum(dy * y))
// Everything is f32 internally.  Short rows use one wave per row, long rows
// (the vocabulary-sized log_softmax) one 512-thread block per row.
#include <math.h>

#include "common.h"

namespace mi {
namespace {

struct MS {
  float m, s;
};

__device__ __forceinline__ MS ms_fold(MS a, float x) {
  if (x == -INFINITY) return a;  // contributes exp(-inf) = 0
  if (x != x) return MS{x, a.s};  // NaN poisons the row
  if (x > a.m) {
    const float s = (a.m == -INFINITY) ? 0.f : a.s * expf(a.m - x);
    return MS{x, s + 1.f};
  }
  return MS{a.m, a.s + expf(x - a.m)};
}

__device__ __forceinline__ MS ms_merge(MS a, MS b) {
  if (a.m != a.m || b.m != b.m) return MS{a.m != a.m ? a.m : b.m, 0.f};
  if (a.m == -INFINITY) return b;
  if (b.m == -INFINITY) return a;
  const float m = fmaxf(a.m, b.m);
  return MS{m, a.s * expf(a.m - m) + b.s * expf(b.m - m)};
}

__device__ __forceinline__ MS wave_ms(MS v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    MS o{__shfl_xor(v.m, off, 64), __shfl_xor(v.s, off, 64)};
    v = ms_merge(v, o);
  }
  return v;
}

template <typename TI, typename TO, int THREADS, bool WAVE_ROW>
__global__ void __launch_bounds__(THREADS)
    softmax_fwd_kernel(TO* __restrict__ y, const TI* __restrict__ x, int64_t rows, int64_t cols,
                       int log) {
  __shared__ MS red[THREADS / 64];
  const int lane = threadIdx.x & 63;
  int64_t row;
  int tid, nth;
  if (WAVE_ROW) {
    row = (int64_t)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6);
    tid = lane;
    nth = 64;
    if (row >= rows) return;
  } else {
    row = blockIdx.x;
    tid = threadIdx.x;
    nth = THREADS;
  }
  const TI* xr = x + row * cols;
  MS acc{-INFINITY, 0.f};
  for (int64_t c = tid; c < cols; c += nth) acc = ms_fold(acc, to_f32(xr[c]));
  acc = wave_ms(acc);
  if (!WAVE_ROW) {
    if (lane == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    acc = red[0];
    for (int w = 1; w < THREADS / 64; ++w) acc = ms_merge(acc, red[w]);
  }
  const float m = acc.m;
  const float lse = m + logf(acc.s);
  const float inv = 1.f / acc.s;
  TO* yr = y + row * cols;
  for (int64_t c = tid; c < cols; c += nth) {
    const float v = to_f32(xr[c]);
    yr[c] = from_f32<TO>(log ? v - lse : expf(v - m) * inv);
  }
}

template <typename TG, typename TY, typename TO, int THREADS, bool WAVE_ROW>
__global__ void __launch_bounds__(THREADS)
    softmax_bwd_kernel(TO* __restrict__ dx, const TG* __restrict__ dy, const TY* __restrict__ y,
                       int64_t rows, int64_t cols, int log) {
  __shared__ float red[THREADS / 64];
  const int lane = threadIdx.x & 63;
  int64_t row;
  int tid, nth;
  if (WAVE_ROW) {
    row = (int64_t)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6);
    tid = lane;
    nth = 64;
    if (row >= rows) return;
  } else {
    row = blockIdx.x;
    tid = threadIdx.x;
    nth = THREADS;
  }
  const TG* g = dy + row * cols;
  const TY* yr = y + row * cols;
  float s = 0.f;
  if (log) {
    for (int64_t c = tid; c < cols; c += nth) s += to_f32(g[c]);
  } else {
    for (int64_t c = tid; c < cols; c += nth) s += to_f32(g[c]) * to_f32(yr[c]);
  }
  s = wave_sum(s);
  if (!WAVE_ROW) {
    if (lane == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = 0.f;
    for (int w = 0; w < THREADS / 64; ++w) s += red[w];
  }
  TO* o = dx + row * cols;
  for (int64_t c = tid; c < cols; c += nth) {
    const float gv = to_f32(g[c]), yv = to_f32(yr[c]);
    o[c] = from_f32<TO>(log ? gv - expf(yv) * s : yv * (gv - s));
  }
}

template <typename TI, typename TO>
int fwd(void* y, const void* x, int64_t rows, int64_t cols, int log, hipStream_t s) {
  if (cols <= 1024) {
    softmax_fwd_kernel<TI, TO, 256, true><<<ceil_div(rows, 4), 256, 0, s>>>((TO*)y, (const TI*)x, rows, cols, log);
  } else {
    softmax_fwd_kernel<TI, TO, 512, false><<<(unsigned)rows, 512, 0, s>>>((TO*)y, (const TI*)x, rows, cols, log);
  }
  return check_launch("mi355x_softmax_fwd");
}

template <typename TG, typename TY, typename TO>
int bwd(void* dx, const void* dy, const void* y, int64_t rows, int64_t cols, int log, hipStream_t s) {
  if (cols <= 1024) {
    softmax_bwd_kernel<TG, TY, TO, 256, true><<<ceil_div(rows, 4), 256, 0, s>>>((TO*)dx, (const TG*)dy, (const TY*)y, rows, cols, log);
  } else {
    softmax_bwd_kernel<TG, TY, TO, 512, false><<<(unsigned)rows, 512, 0, s>>>((TO*)dx, (const TG*)dy, (const TY*)y, rows, cols, log);
  }
  return check_launch("mi355x_softmax_bwd");
}

bool fdt(int d) { return d == MI355X_F32 || d == MI355X_BF16 || d == MI355X_F16; }

}  // namespace
}  // namespace mi

using namespace mi;

#define MI_DISPATCH_F(dt, T, ...)                \
  switch (dt) {                                  \
    case MI355X_F32: { typedef float T; __VA_ARGS__; break; } \
    case MI355X_BF16: { typedef bf16 T; __VA_ARGS__; break; } \
    default: { typedef f16 T; __VA_ARGS__; break; }          \
  }

extern "C" int mi355x_softmax_fwd(void* y, int y_dtype, const void* x, int x_dtype, int64_t rows,
                                  int64_t cols, int log, mi355x_stream_t stream) {
  MI_REQUIRE(fdt(y_dtype) && fdt(x_dtype), "mi355x_softmax_fwd: unsupported dtype");
  MI_REQUIRE(rows >= 0 && cols >= 0 && rows < (1ll << 31), "mi355x_softmax_fwd: bad shape");
  if (rows == 0 || cols == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  int rc = 0;
  MI_DISPATCH_F(x_dtype, TI, MI_DISPATCH_F(y_dtype, TO, rc = (fwd<TI, TO>(y, x, rows, cols, log, s))));
  return rc;
}

extern "C" int mi355x_softmax_bwd(void* dx, int dx_dtype, const void* dy, int dy_dtype,
                                  const void* y, int y_dtype, int64_t rows, int64_t cols, int log,
                                  mi355x_stream_t stream) {
  MI_REQUIRE(fdt(dx_dtype) && fdt(dy_dtype) && fdt(y_dtype), "mi355x_softmax_bwd: unsupported dtype");
  MI_REQUIRE(rows >= 0 && cols >= 0 && rows < (1ll << 31), "mi355x_softmax_bwd: bad shape");
  if (rows == 0 || cols == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  int rc = 0;
  MI_DISPATCH_F(dy_dtype, TG,
                MI_DISPATCH_F(y_dtype, TY,
                              MI_DISPATCH_F(dx_dtype, TO, rc = (bwd<TG, TY, TO>(dx, dy, y, rows, cols, log, s)))));
  return rc;
}
