// Row softmax / log_softmax forward and backward over the contiguous last dim.
//
// Forward is two passes over the row: an online (max, sum-of-exp) pass whose
// per-lane partials are merged with the usual rescaling, then the output pass
//   log:     y = x - max - log(sum)
//   softmax: y = exp(x - max) / sum
// Backward: one pass for the row sum, one for the output
//   log:     dx = dy - exp(y) * sum(dy)
//   softmax: dx = y * (dy - sum(dy * y))
// Everything is f32 internally.  Short rows use one wave per row; long rows
// of one element type (the vocabulary-sized log_softmax) a 512/1024-thread
// block per row holding the row in registers; other long rows a 512-thread
// block per row.
#include <math.h>

#include <type_traits>

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

// ---------------------------------------------------------------------------
// Long rows with one element type throughout (the vocabulary-sized
// log_softmax of the reference's bf16 path).  A 512- or 1024-thread block
// owns a row and holds it in registers as aligned 16-byte chunks, so x (and dy, y
// in the backward) are read from HBM once.  A row starts at row * cols
// elements, which is generally not 16-byte aligned: chunk j covers row
// elements j*V - p .. j*V - p + V-1 (p = the row's phase), the first and
// last chunks are shared with the neighbouring rows and masked, and every
// operand has the same phase because all bases are 16-byte aligned and
// share the element type.  Interior output chunks are 16-byte stores, the
// two edge chunks element stores.
// ---------------------------------------------------------------------------

template <typename T>
struct Chunk16 {
  static constexpr int V = 16 / sizeof(T);
  uint4 w;
  __device__ __forceinline__ float get(int e) const {
    if constexpr (sizeof(T) == 4) {
      return __uint_as_float((&w.x)[e]);
    } else {
      const uint32_t u = (&w.x)[e >> 1];
      const unsigned short h = (e & 1) ? (unsigned short)(u >> 16) : (unsigned short)(u & 0xffff);
      return to_f32(__builtin_bit_cast(T, h));
    }
  }
};

// Row geometry shared by every operand of the row.
struct RowChunks {
  int p;    // elements of the first aligned chunk that precede the row
  int nch;  // aligned chunks holding elements of the row
  int64_t off;  // element offset of the first aligned chunk from the base
};
template <typename T>
__device__ __forceinline__ RowChunks row_chunks(const T* base, int64_t row, int64_t cols) {
  constexpr int V = 16 / sizeof(T);
  const int64_t first = row * cols;
  RowChunks g;
  g.p = (int)(first % V);
  g.off = first - g.p;
  g.nch = (int)((cols + g.p + V - 1) / V);
  return g;
}

// Block-wide merge of per-thread (max, sum of exp2((x - max) log2e), NaN).
template <int THREADS>
__device__ __forceinline__ void block_ms(float& m, float& s, bool& nan, float* rm, float* rs, int* rn) {
  constexpr float kL2e = 1.4426950408889634f;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float om = __shfl_xor(m, off, 64), os = __shfl_xor(s, off, 64);
    nan |= __shfl_xor((int)nan, off, 64) != 0;
    const float nm = fmaxf(m, om);
    if (nm != -INFINITY) {
      s = (m == -INFINITY ? 0.f : s * exp2f((m - nm) * kL2e)) + (om == -INFINITY ? 0.f : os * exp2f((om - nm) * kL2e));
      m = nm;
    }
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) rm[wid] = m, rs[wid] = s, rn[wid] = nan;
  __syncthreads();
  m = -INFINITY, s = 0.f, nan = false;
  for (int w = 0; w < THREADS / 64; ++w) {
    nan |= rn[w] != 0;
    const float om = rm[w], os = rs[w], nm = fmaxf(m, om);
    if (nm != -INFINITY) {
      s = (m == -INFINITY ? 0.f : s * exp2f((m - nm) * kL2e)) + (om == -INFINITY ? 0.f : os * exp2f((om - nm) * kL2e));
      m = nm;
    }
  }
}

// The long-row kernels read and write every row once, with the
// non-temporal hint (log_softmax bf16 [16384, 50257]: forward 0.70 -> 0.65
// ms, backward 0.98 -> 0.88 ms).
template <typename T>
__device__ __forceinline__ void store_chunk(T* base, int64_t off, int j, int p, int64_t cols, const float* o) {
  constexpr int V = 16 / sizeof(T);
  const int k0 = j * V - p;
  T* dst = base + off + (int64_t)j * V;
  if (k0 >= 0 && k0 + V <= cols) {
    struct alignas(16) Out { T v[V]; } out;
#pragma unroll
    for (int e = 0; e < V; ++e) out.v[e] = from_f32<T>(o[e]);
    st_stream((Out*)dst, out);
  } else {
#pragma unroll
    for (int e = 0; e < V; ++e)
      if (k0 + e >= 0 && k0 + e < cols) dst[e] = from_f32<T>(o[e]);
  }
}

template <typename T, int NCH, int THREADS>
__global__ void __launch_bounds__(THREADS)
    softmax_fwd_rowreg(T* __restrict__ y, const T* __restrict__ x, int64_t cols, int log) {
  constexpr int V = 16 / sizeof(T);
  constexpr float kL2e = 1.4426950408889634f;
  __shared__ float rm[THREADS / 64], rs[THREADS / 64];
  __shared__ int rn[THREADS / 64];
  const RowChunks g = row_chunks(x, blockIdx.x, cols);
  const uint4* src = (const uint4*)(x + g.off);
  Chunk16<T> c[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int j = threadIdx.x + i * THREADS;
    c[i].w = j < g.nch ? ld_stream(src + j) : make_uint4(0, 0, 0, 0);
  }
  float m = -INFINITY, s = 0.f;
  bool nan = false;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int j = threadIdx.x + i * THREADS;
    if (j >= g.nch) break;
    const int k0 = j * V - g.p;
    float v[V];
    const bool interior = k0 >= 0 && k0 + V <= cols;
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = (interior || (k0 + e >= 0 && k0 + e < cols)) ? c[i].get(e) : -INFINITY;
    // one NaN test per chunk: the chunk maximum propagates NaN
    const float cm = max_nan(v);
    if (cm != cm) {
      nan = true;
      continue;
    }
    if (cm == -INFINITY) continue;
    if (cm > m) {
      s = (m == -INFINITY) ? 0.f : s * exp2f((m - cm) * kL2e);
      m = cm;
    }
    // terms of the sum (>= 1, from the maximum) need no subnormal results;
    // v - m, not an FMA against m log2(e), whose rounding (relative to m)
    // would cost f32 rows about 1e-6 of accuracy
#pragma unroll
    for (int e = 0; e < V; ++e) s += __builtin_amdgcn_exp2f((v[e] - m) * kL2e);
  }
  block_ms<THREADS>(m, s, nan, rm, rs, rn);
  if (nan) m = NAN;
  const float lse = m + logf(s);
  const float inv = 1.f / s;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int j = threadIdx.x + i * THREADS;
    if (j >= g.nch) break;
    float o[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float v = c[i].get(e);
      o[e] = log ? v - lse : exp2f((v - m) * kL2e) * inv;
    }
    store_chunk(y, g.off, j, g.p, cols, o);
  }
}

// log:     dx = dy - exp(y) * sum(dy)   (dy in registers, then y streamed)
// softmax: dx = y * (dy - sum(dy * y))  (dy and y in registers)
template <typename T, int NCH, int THREADS, bool LOG>
__global__ void __launch_bounds__(THREADS)
    softmax_bwd_rowreg(T* __restrict__ dx, const T* __restrict__ dy, const T* __restrict__ y, int64_t cols) {
  constexpr int V = 16 / sizeof(T);
  __shared__ float red[THREADS / 64];
  const RowChunks g = row_chunks(dy, blockIdx.x, cols);
  const uint4* gsrc = (const uint4*)(dy + g.off);
  const uint4* ysrc = (const uint4*)(y + g.off);
  Chunk16<T> cg[NCH], cy[LOG ? 1 : NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int j = threadIdx.x + i * THREADS;
    cg[i].w = j < g.nch ? ld_stream(gsrc + j) : make_uint4(0, 0, 0, 0);
    if constexpr (!LOG) cy[i].w = j < g.nch ? ysrc[j] : make_uint4(0, 0, 0, 0);
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int j = threadIdx.x + i * THREADS;
    if (j >= g.nch) break;
    const int k0 = j * V - g.p;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      if (k0 + e >= 0 && k0 + e < cols) {
        if constexpr (LOG) sum += cg[i].get(e);
        else sum += cg[i].get(e) * cy[i].get(e);
      }
    }
  }
  sum = block_sum(sum, red);
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int j = threadIdx.x + i * THREADS;
    if (j >= g.nch) break;
    Chunk16<T> yc;
    if constexpr (LOG) yc.w = ld_stream(ysrc + j);
    else yc = cy[i];
    float o[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float gv = cg[i].get(e), yv = yc.get(e);
      // exp(y) as one hardware exp2 of y log2(e)
      o[e] = LOG ? gv - __builtin_amdgcn_exp2f(yv * 1.4426950408889634f) * sum : yv * (gv - sum);
    }
    store_chunk(dx, g.off, j, g.p, cols, o);
  }
}

// Launch shape of the register-resident kernels for a long row: threads per
// row and 16-byte chunks per thread (0 threads: the row does not fit).  512
// threads keep two rows in flight per CU.
struct RowShape {
  int threads, nch;
};
template <typename T>
RowShape row_shape(int64_t cols) {
  constexpr int V = 16 / sizeof(T);
  const int64_t nch = (cols + V - 1) / V + 1;
  if (nch <= 8 * 512) return {512, 8};
  if (nch <= 16 * 512) return {512, 16};
  if (nch <= 16 * 1024) return {1024, 16};
  return {0, 0};
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <typename TI, typename TO>
int fwd(void* y, const void* x, int64_t rows, int64_t cols, int log, hipStream_t s) {
  if constexpr (std::is_same<TI, TO>::value) {
    const RowShape rs = cols > 1024 && aligned16(x) && aligned16(y) ? row_shape<TI>(cols) : RowShape{0, 0};
    if (rs.threads) {
      // 512 x 16 chunks per row at 50257 bf16 columns: 1024 x 8 ran at 47%
      // of HBM bandwidth, 256 x 32 at 53%, 512 x 16 at 66%
      auto k = rs.threads == 1024 ? softmax_fwd_rowreg<TI, 16, 1024>
                                  : (rs.nch == 8 ? softmax_fwd_rowreg<TI, 8, 512> : softmax_fwd_rowreg<TI, 16, 512>);
      k<<<(unsigned)rows, rs.threads, 0, s>>>((TO*)y, (const TI*)x, cols, log);
      return check_launch("mi355x_softmax_fwd");
    }
  }
  if (cols <= 1024) {
    softmax_fwd_kernel<TI, TO, 256, true><<<ceil_div(rows, 4), 256, 0, s>>>((TO*)y, (const TI*)x, rows, cols, log);
  } else {
    softmax_fwd_kernel<TI, TO, 512, false><<<(unsigned)rows, 512, 0, s>>>((TO*)y, (const TI*)x, rows, cols, log);
  }
  return check_launch("mi355x_softmax_fwd");
}

template <typename TG, typename TY, typename TO>
int bwd(void* dx, const void* dy, const void* y, int64_t rows, int64_t cols, int log, hipStream_t s) {
  if constexpr (std::is_same<TG, TY>::value && std::is_same<TG, TO>::value) {
    // the softmax form keeps two row copies in registers: 8 chunks at most;
    // the log form keeps dy only and reads y in the output pass
    const RowShape rs = cols > 1024 && aligned16(dx) && aligned16(dy) && aligned16(y) ? row_shape<TG>(cols)
                                                                                      : RowShape{0, 0};
    if (rs.threads && (log || rs.nch == 8)) {
      auto k = rs.threads == 1024 ? softmax_bwd_rowreg<TG, 16, 1024, true>
               : rs.nch == 16     ? softmax_bwd_rowreg<TG, 16, 512, true>
               : log              ? softmax_bwd_rowreg<TG, 8, 512, true>
                                  : softmax_bwd_rowreg<TG, 8, 512, false>;
      k<<<(unsigned)rows, rs.threads, 0, s>>>((TO*)dx, (const TG*)dy, (const TY*)y, cols);
      return check_launch("mi355x_softmax_bwd");
    }
  }
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
