// Rotary position embedding over rows of D (head_dim) elements, half-split
// ("rotate_half") form, for [B, H, T, D] views with unit head_dim stride:
//   y[i]      = x[i] cos[t][i]           - x[i+D/2] sin[t][i]
//   y[i+D/2]  = x[i+D/2] cos[t][i+D/2]   + x[i] sin[t][i+D/2]
// and, with `inverse` (the transposed map, i.e. the backward):
//   y[i]      = x[i] cos[t][i]           + x[i+D/2] sin[t][i+D/2]
//   y[i+D/2]  = x[i+D/2] cos[t][i+D/2]   - x[i] sin[t][i]
// cos/sin are dense [T][D] tables in the input dtype; computed in f32 and
// rounded once.  One thread handles 4 (i, i+D/2) pairs: read once, write once.
#include "common.h"
#include "vec.h"

namespace mi {
namespace {

constexpr int kThreads = 256;

template <typename T>
__global__ void __launch_bounds__(kThreads)
    rope_kernel(T* __restrict__ y, int64_t ys_b, int64_t ys_h, int64_t ys_t, const T* __restrict__ x, int64_t xs_b,
                int64_t xs_h, int64_t xs_t, const T* __restrict__ cos_t, const T* __restrict__ sin_t, int64_t H,
                int64_t T_, int D, int64_t total, int inverse) {
  const int half = D / 2, per_row = half / 4;
  for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * kThreads) {
    const int64_t row = idx / per_row;
    const int i = (int)(idx - row * per_row) * 4;
    const int64_t t = row % T_, bh = row / T_;
    const int64_t h = bh % H, b = bh / H;
    const T* xr = x + b * xs_b + h * xs_h + t * xs_t;
    T* yr = y + b * ys_b + h * ys_h + t * ys_t;
    const T* cr = cos_t + t * D;
    const T* sr = sin_t + t * D;
    float x1[4], x2[4], c1[4], c2[4], s1[4], s2[4], o1[4], o2[4];
    Vec4<T>::load(xr + i, x1);
    Vec4<T>::load(xr + i + half, x2);
    Vec4<T>::load(cr + i, c1);
    Vec4<T>::load(cr + i + half, c2);
    Vec4<T>::load(sr + i, s1);
    Vec4<T>::load(sr + i + half, s2);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (inverse) {
        o1[e] = x1[e] * c1[e] + x2[e] * s2[e];
        o2[e] = x2[e] * c2[e] - x1[e] * s1[e];
      } else {
        o1[e] = x1[e] * c1[e] - x2[e] * s1[e];
        o2[e] = x2[e] * c2[e] + x1[e] * s2[e];
      }
    }
    Vec4<T>::store(yr + i, o1);
    Vec4<T>::store(yr + i + half, o2);
  }
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi355x_rope(void* y, const int64_t* y_bht, const void* x, const int64_t* x_bht, const void* cos_table,
                           const void* sin_table, int64_t batch, int64_t heads, int64_t seq, int64_t d, int inverse,
                           int dtype, mi355x_stream_t stream) {
  MI_REQUIRE(batch >= 0 && heads >= 0 && seq >= 0 && d > 0, "mi355x_rope: bad shape");
  MI_REQUIRE(d % 8 == 0 && d <= 4096, "mi355x_rope: head_dim %lld must be a multiple of 8", (long long)d);
  const int64_t rows = batch * heads * seq;
  if (rows == 0) return MI355X_OK;
  MI_REQUIRE(y && x && cos_table && sin_table, "mi355x_rope: null pointer");
  const size_t es = dtype == MI355X_F32 ? 4 : 2;
  for (const int64_t* st : {y_bht, x_bht})
    MI_REQUIRE(st[0] % 4 == 0 && st[1] % 4 == 0 && st[2] % 4 == 0, "mi355x_rope: strides must be multiples of 4");
  MI_REQUIRE(((uintptr_t)y % (4 * es)) == 0 && ((uintptr_t)x % (4 * es)) == 0 &&
                 ((uintptr_t)cos_table % (4 * es)) == 0 && ((uintptr_t)sin_table % (4 * es)) == 0,
             "mi355x_rope: operands must be aligned to 4 elements");
  const int64_t total = rows * (d / 8);
  int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 16384) blocks = 16384;
  hipStream_t s = (hipStream_t)stream;
#define ROPE(T)                                                                                               \
  rope_kernel<T><<<(unsigned)blocks, kThreads, 0, s>>>((T*)y, y_bht[0], y_bht[1], y_bht[2], (const T*)x,      \
                                                       x_bht[0], x_bht[1], x_bht[2], (const T*)cos_table,     \
                                                       (const T*)sin_table, heads, seq, (int)d, total, inverse)
  switch (dtype) {
    case MI355X_F32: ROPE(float); break;
    case MI355X_BF16: ROPE(bf16); break;
    case MI355X_F16: ROPE(f16); break;
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_rope: unsupported dtype %d", dtype);
  }
#undef ROPE
  return check_launch("mi355x_rope");
}
