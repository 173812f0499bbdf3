// Fused softmax cross-entropy over logits [n, c] (row stride ld) and int64
// targets: the log_softmax -> nll_loss chain of the training step without
// materialising log-probabilities or a dense one-hot gradient.
//
// Rows are visited as aligned 16-byte chunks.  A row of the [16384, 50257]
// logits starts at any 2-byte boundary (phase p = its start's offset inside
// a 16-byte granule, uniform per row): aligned chunk j covers elements
// [V*j - p, V*j - p + V) (V = 16 / sizeof(T)); elements outside [0, c) are
// masked.  A chunk never leaves the 16-byte granules the row touches, so no
// load crosses into memory the row does not own a byte of.
//
// Forward, one 256-thread block per row: an online (max, sum) in the exp2
// domain with one rescale per chunk (max of the chunk first), four chunks in
// flight per thread; lse_i = ln(sum) + max.  Row loss = lse_i - x_i[t_i] (0
// for ignore_index).  A one-block kernel reduces the row losses in a fixed
// order into the mean or sum and writes total_weight.
// Backward, one block per row: dx_i = g_i * (exp(x_i - lse_i) - onehot(t_i)),
// g_i = grad (per row for reduction none, else the scalar, / total_weight
// for mean), zero for ignored rows and for the padding columns [c, ld_dx).
// dx rows are 16-byte aligned (ld_dx a multiple of V), so each thread writes
// whole 16-byte dx chunks, two per iteration; the V logits one needs come
// from two aligned chunks shifted by the row's phase (v_alignbyte).  Only
// the first and last chunks of a row (and, backward, the target's chunk)
// take the per-element masks; the rest go straight to exp2.
// HBM traffic: forward reads the logits once; backward reads them once and
// writes dx once.
#include <math.h>

#include <algorithm>

#include "common.h"

namespace mi {
namespace {

constexpr int kRowThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <typename T>
struct Chunk {
  static constexpr int V = 16 / sizeof(T);
  uint4 w;
  __device__ __forceinline__ float get(int e) const {
    if constexpr (sizeof(T) == 4) return __uint_as_float((&w.x)[e]);
    else {
      const uint32_t u = (&w.x)[e >> 1];
      const unsigned short h = (e & 1) ? (unsigned short)(u >> 16) : (unsigned short)(u & 0xffff);
      return to_f32(__builtin_bit_cast(T, h));
    }
  }
};

// Row geometry: aligned base, phase and the number of aligned chunks that
// hold elements of [0, c).
template <typename T>
struct RowGeo {
  static constexpr int V = 16 / sizeof(T);
  const uint4* base;
  int p;
  int64_t nch;
  __device__ __forceinline__ RowGeo(const T* r, int64_t c) {
    const uintptr_t a = (uintptr_t)r & ~(uintptr_t)15;
    base = (const uint4*)a;
    p = (int)(((uintptr_t)r - a) / sizeof(T));
    nch = (c + p + V - 1) / V;
  }
};

// exp2 on the hardware instruction: arguments here are <= 0 (or -inf), and
// results below the f32 normal range only feed sums and bf16/f16 gradients.
__device__ __forceinline__ float hw_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// One aligned chunk (number j of the row) into a thread's running (max,
// sum of exp2((x - max) * log2e)); NaN sets `nan` and skips the chunk.
template <typename T>
__device__ __forceinline__ void ce_take_chunk(const Chunk<T>& ch, int j, const RowGeo<T>& geo, int ci, float& m,
                                              float& sum, bool& nan) {
  constexpr int V = Chunk<T>::V;
  const int k0 = j * V - geo.p;
  float v[V];
  if (k0 >= 0 && k0 + V <= ci) {
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = ch.get(e);
  } else {  // the row's first or last chunk
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = (k0 + e >= 0 && k0 + e < ci) ? ch.get(e) : -INFINITY;
  }
  // one NaN test per chunk: the chunk maximum propagates NaN
  const float cm = max_nan(v);
  if (cm != cm) {
    nan = true;
    return;
  }
  if (cm == -INFINITY) return;
  if (cm > m) {
    sum = (m == -INFINITY) ? 0.f : sum * hw_exp2((m - cm) * kLog2e);
    m = cm;
  }
#pragma unroll
  for (int e = 0; e < V; ++e) sum += hw_exp2((v[e] - m) * kLog2e);
}

// The block's (max, sum) merged (wave, then block, in a fixed order) into
// the row's log-sum-exp, its loss lse - x[t] (0 for ignore_index) and
// validity; thread 0 writes them and returns the lse (NaN when a NaN was
// seen); the other threads return garbage.
template <typename T>
__device__ __forceinline__ float ce_finish_row(float m, float sum, bool nan, float* red_m, float* red_s, int* red_nan,
                                               const T* r, int64_t row, float* lse, float* row_loss,
                                               float* row_valid, const int64_t* target, int64_t c,
                                               int64_t ignore_index, int32_t* err) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float om = __shfl_xor(m, off, 64), os = __shfl_xor(sum, off, 64);
    nan |= __shfl_xor((int)nan, off, 64) != 0;
    const float nm = fmaxf(m, om);
    if (nm != -INFINITY) {
      sum = (m == -INFINITY ? 0.f : sum * exp2f((m - nm) * kLog2e)) +
            (om == -INFINITY ? 0.f : os * exp2f((om - nm) * kLog2e));
      m = nm;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    red_m[threadIdx.x >> 6] = m;
    red_s[threadIdx.x >> 6] = sum;
    red_nan[threadIdx.x >> 6] = nan;
  }
  __syncthreads();
  float l = 0.f;
  if (threadIdx.x == 0) {
    float tm = -INFINITY, ts = 0.f;
    bool tn = false;
    for (int w = 0; w < kRowThreads / 64; ++w) {
      tn |= red_nan[w] != 0;
      const float om = red_m[w], os = red_s[w];
      const float nm = fmaxf(tm, om);
      if (nm == -INFINITY) continue;
      ts = (tm == -INFINITY ? 0.f : ts * exp2f((tm - nm) * kLog2e)) +
           (om == -INFINITY ? 0.f : os * exp2f((om - nm) * kLog2e));
      tm = nm;
    }
    l = tn ? __int_as_float(0x7fc00000) : tm + log2f(ts) * kLn2;
    lse[row] = l;
    const int64_t tg = target[row];
    float loss = 0.f, valid = 0.f;
    if (tg != ignore_index) {
      if (tg < 0 || tg >= c) {
        if (err) *err = 1;
      } else {
        loss = l - to_f32(r[tg]);
        valid = 1.f;
      }
    }
    row_loss[row] = loss;
    row_valid[row] = valid;
  }
  return l;
}

template <typename T>
__global__ void __launch_bounds__(kRowThreads)
    ce_fwd_rows(float* __restrict__ row_loss, float* __restrict__ row_valid, float* __restrict__ lse,
                const T* __restrict__ x, int64_t ld, const int64_t* __restrict__ target, int64_t n,
                int64_t c, int64_t ignore_index, int32_t* err) {
  constexpr int U = 4;
  __shared__ float red_m[kRowThreads / 64], red_s[kRowThreads / 64];
  __shared__ int red_nan[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const T* r = x + row * ld;
  const RowGeo<T> geo(r, c);
  const int nch = (int)geo.nch, ci = (int)c;
  float m = -INFINITY, sum = 0.f;  // max and sum of exp2((x - m) * log2e)
  bool nan = false;
  for (int j0 = threadIdx.x; j0 < nch; j0 += kRowThreads * U) {
    Chunk<T> ch[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + u * kRowThreads;
      if (j < nch) ch[u].w = geo.base[j];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + u * kRowThreads;
      if (j >= nch) break;
      ce_take_chunk<T>(ch[u], j, geo, ci, m, sum, nan);
    }
  }
  ce_finish_row<T>(m, sum, nan, red_m, red_s, red_nan, r, row, lse, row_loss, row_valid, target, c, ignore_index,
                   err);
}

__global__ void __launch_bounds__(1024) ce_fwd_reduce(float* __restrict__ out, float* __restrict__ total,
                                                      const float* __restrict__ row_loss,
                                                      const float* __restrict__ row_valid, int64_t n,
                                                      int reduction) {
  __shared__ float red[16];
  float s = 0.f, w = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += row_loss[i], w += row_valid[i];
  s = block_sum(s, red);
  w = block_sum(w, red);
  if (threadIdx.x == 0) {
    out[0] = reduction == 1 ? s / w : s;
    total[0] = w;
  }
}

// The V elements of x starting at element V*t of the row: aligned chunks t
// and t+1 shifted right by the row phase (bytes b = p * sizeof(T)).
__device__ __forceinline__ uint4 shift_pair(uint4 lo, uint4 hi, int bytes) {
  const uint32_t W[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  const int r = bytes & 3;
  uint4 o;
  uint32_t* ow = &o.x;
  switch (bytes >> 2) {  // uniform per row
#define CE_SHIFT(Q)                                                                            \
  case Q:                                                                                      \
    for (int i = 0; i < 4; ++i) ow[i] = __builtin_amdgcn_alignbyte(W[i + Q + 1], W[i + Q], r); \
    break;
    CE_SHIFT(0)
    CE_SHIFT(1)
    CE_SHIFT(2)
    CE_SHIFT(3)
#undef CE_SHIFT
  }
  return o;
}

// dx of the V elements from k0 on: g * (exp(x - lse) - onehot), 0 past c.
template <typename T, typename TD>
__device__ __forceinline__ uint4 ce_dx_chunk(const Chunk<T>& ch, int k0, int ci, int tgi, float g, float l) {
  constexpr int V = Chunk<T>::V;
  struct alignas(16) Out { TD v[V]; } out;
  if (k0 + V <= ci && (tgi < k0 || tgi >= k0 + V)) {
#pragma unroll
    for (int e = 0; e < V; ++e) out.v[e] = from_f32<TD>(g * hw_exp2((ch.get(e) - l) * kLog2e));
  } else {  // the last chunk, padding past c, or the target's chunk
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int k = k0 + e;
      float d = 0.f;
      if (k < ci) d = g * (hw_exp2((ch.get(e) - l) * kLog2e) - (k == tgi ? 1.f : 0.f));
      out.v[e] = from_f32<TD>(d);
    }
  }
  return *(const uint4*)&out;
}

// The backward writes every element of the row.  It has no reduction, so
// rows are split over blocks: block b covers 16-byte output chunks
// (b % nb) * 256 .. +255 of row b / nb, one chunk per thread (gfx950,
// [16384, 50257] bf16: 0.565 ms, against 0.604 ms for one 1024-thread
// block per row looping over it and 0.59-0.66 ms for 2-8 chunks per thread).
constexpr int kBwdThreads = 256;

template <typename T, typename TD>
__global__ void __launch_bounds__(kBwdThreads)
    ce_bwd_chunks(TD* __restrict__ dx, int64_t ld_dx, const T* __restrict__ x, int64_t ld,
                  const float* __restrict__ lse, const int64_t* __restrict__ target,
                  const float* __restrict__ grad, int grad_per_row, const float* __restrict__ total,
                  int64_t n, int64_t c, int64_t ignore_index, int nb) {
  constexpr int V = Chunk<T>::V;
  static_assert(sizeof(TD) == sizeof(T), "dx chunks follow the logits chunks");
  const int64_t row = blockIdx.x / nb;
  const int t = (int)(blockIdx.x - row * nb) * kBwdThreads + threadIdx.x;
  const int nout = (int)(ld_dx / V);
  if (t >= nout) return;
  const int64_t tg = target[row];
  float g = grad[grad_per_row ? row : 0];
  if (!grad_per_row && total) g /= total[0];
  const bool valid = tg != ignore_index && tg >= 0 && tg < c;
  if (!valid) g = 0.f;
  const float l = lse[row];
  const RowGeo<T> geo(x + row * ld, c);
  const int bytes = geo.p * (int)sizeof(T);
  const int nch = (int)geo.nch, ci = (int)c, tgi = valid ? (int)tg : -1;
  const int k0 = t * V;
  uint4 lo = make_uint4(0, 0, 0, 0), hi = lo;
  if (k0 < ci) {
    lo = geo.base[t];
    if (bytes && t + 1 < nch) hi = geo.base[t + 1];
  }
  Chunk<T> ch;
  ch.w = bytes ? shift_pair(lo, hi, bytes) : lo;
  ((uint4*)(dx + row * ld_dx))[t] = ce_dx_chunk<T, TD>(ch, k0, ci, tgi, g, l);
}

// Forward and backward in one pass, for a row whose loss is read only
// after its backward (a training step): the row's aligned chunks stay in
// registers (NC per thread), the (max, sum) runs over them in ce_fwd_rows'
// order and merge (so lse and the loss have its bits), and the dx chunks are
// ce_bwd_chunks' from the same registers: the logits are read once instead
// of twice (a row whose start is not 16-byte aligned takes each dx chunk's
// second source chunk from the next lane's registers).  Rows have at
// most NC * kRowThreads chunks.  `total` (the valid-target count, for
// reduction mean) is written by ce_count_valid before this kernel.
template <typename T, typename TD, int NC>
__global__ void __launch_bounds__(kRowThreads)
    ce_fused_rows(TD* __restrict__ dx, int64_t ld_dx, float* __restrict__ row_loss, float* __restrict__ row_valid,
                  float* __restrict__ lse, const T* __restrict__ x, int64_t ld, const int64_t* __restrict__ target,
                  const float* __restrict__ grad, const float* __restrict__ total, int64_t c, int64_t ignore_index,
                  int32_t* err) {
  constexpr int V = Chunk<T>::V;
  static_assert(sizeof(TD) == sizeof(T), "dx chunks follow the logits chunks");
  __shared__ float red_m[kRowThreads / 64], red_s[kRowThreads / 64], l_s;
  __shared__ int red_nan[kRowThreads / 64];
  __shared__ uint4 first[kRowThreads / 64][NC + 1];  // each wave's lane-0 chunks (the next chunk of lane 63)
  const int64_t row = blockIdx.x;
  const T* r = x + row * ld;
  const RowGeo<T> geo(r, c);
  const int nch = (int)geo.nch, ci = (int)c;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  Chunk<T> ch[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int j = threadIdx.x + k * kRowThreads;
    ch[k].w = j < nch ? geo.base[j] : make_uint4(0, 0, 0, 0);
  }
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < NC; ++k) first[wave][k] = ch[k].w;
    first[wave][NC] = make_uint4(0, 0, 0, 0);
  }
  float m = -INFINITY, sum = 0.f;
  bool nan = false;
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int j = threadIdx.x + k * kRowThreads;
    if (j >= nch) break;
    ce_take_chunk<T>(ch[k], j, geo, ci, m, sum, nan);
  }
  const float l0 = ce_finish_row<T>(m, sum, nan, red_m, red_s, red_nan, r, row, lse, row_loss, row_valid, target,
                                    c, ignore_index, err);
  if (threadIdx.x == 0) l_s = l0;
  __syncthreads();
  const float l = l_s;
  const int64_t tg = target[row];
  float g = grad[0];
  if (total) g /= total[0];
  const bool valid = tg != ignore_index && tg >= 0 && tg < c;
  if (!valid) g = 0.f;
  const int tgi = valid ? (int)tg : -1;
  const int nout = (int)(ld_dx / V);
  const int bytes = geo.p * (int)sizeof(T);
  uint4* out = (uint4*)(dx + row * ld_dx);
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int t = threadIdx.x + k * kRowThreads;
    if (k * kRowThreads >= nout) break;  // uniform: every lane takes part in the shuffles below
    const int k0 = t * V;
    Chunk<T> cs;
    if (bytes) {  // uniform per row
      // chunk t + 1: the next lane's (lane 63: the next wave's lane 0, or
      // wave 0's lane 0 one group on), zero past the row
      uint4 hi;
      hi.x = __shfl_down(ch[k].w.x, 1, 64);
      hi.y = __shfl_down(ch[k].w.y, 1, 64);
      hi.z = __shfl_down(ch[k].w.z, 1, 64);
      hi.w = __shfl_down(ch[k].w.w, 1, 64);
      if (lane == 63) hi = wave < kRowThreads / 64 - 1 ? first[wave + 1][k] : first[0][k + 1];
      if (t + 1 >= nch) hi = make_uint4(0, 0, 0, 0);
      cs.w = k0 < ci ? shift_pair(ch[k].w, hi, bytes) : make_uint4(0, 0, 0, 0);
    } else {
      cs.w = k0 < ci ? ch[k].w : make_uint4(0, 0, 0, 0);
    }
    if (t < nout) out[t] = ce_dx_chunk<T, TD>(cs, k0, ci, tgi, g, l);
  }
}

// total[0] = the number of rows whose target is neither ignore_index nor
// outside [0, c) (the sum of ce_fwd_rows' row_valid, exact in f32).
__global__ void __launch_bounds__(1024) ce_count_valid(float* __restrict__ total, const int64_t* __restrict__ target,
                                                       int64_t n, int64_t c, int64_t ignore_index) {
  __shared__ float red[16];
  float w = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) {
    const int64_t t = target[i];
    w += (t != ignore_index && t >= 0 && t < c) ? 1.f : 0.f;
  }
  w = block_sum(w, red);
  if (threadIdx.x == 0) total[0] = w;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int64_t mi355x_cross_entropy_workspace_bytes(int64_t n) { return 2 * n * (int64_t)sizeof(float) + 256; }

extern "C" int mi355x_cross_entropy_fwd(void* out, float* total_weight, float* lse, const void* logits,
                                        int dtype, int64_t ld, const int64_t* target, int64_t n,
                                        int64_t c, int reduction, int64_t ignore_index,
                                        int32_t* err_flag, void* workspace, int64_t ws_bytes,
                                        mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0 && c > 0 && ld >= c, "mi355x_cross_entropy_fwd: bad shape");
  MI_REQUIRE(c < (1ll << 30), "mi355x_cross_entropy_fwd: too many classes");
  MI_REQUIRE(reduction >= 0 && reduction <= 2, "mi355x_cross_entropy_fwd: bad reduction");
  MI_REQUIRE(dtype_size(dtype) == 0 || ((uintptr_t)logits % dtype_size(dtype)) == 0,
             "mi355x_cross_entropy_fwd: misaligned logits");
  if (n == 0) return MI355X_OK;
  MI_REQUIRE(n < (1ll << 31), "mi355x_cross_entropy_fwd: too many rows");
  const int64_t need = mi355x_cross_entropy_workspace_bytes(n);
  if (!workspace || ws_bytes < need)
    return fail(MI355X_EWORKSPACE, "mi355x_cross_entropy_fwd: workspace %lld < %lld", (long long)ws_bytes, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  float* row_loss = reduction == 0 ? (float*)out : (float*)workspace;
  float* row_valid = (float*)workspace + n;
  switch (dtype) {
    case MI355X_F32: ce_fwd_rows<float><<<(unsigned)n, kRowThreads, 0, s>>>(row_loss, row_valid, lse, (const float*)logits, ld, target, n, c, ignore_index, err_flag); break;
    case MI355X_BF16: ce_fwd_rows<bf16><<<(unsigned)n, kRowThreads, 0, s>>>(row_loss, row_valid, lse, (const bf16*)logits, ld, target, n, c, ignore_index, err_flag); break;
    case MI355X_F16: ce_fwd_rows<f16><<<(unsigned)n, kRowThreads, 0, s>>>(row_loss, row_valid, lse, (const f16*)logits, ld, target, n, c, ignore_index, err_flag); break;
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_cross_entropy_fwd: unsupported dtype %d", dtype);
  }
  float* dummy = (float*)workspace;  // reduction none still reports total_weight
  ce_fwd_reduce<<<1, 1024, 0, s>>>(reduction == 0 ? dummy : (float*)out, total_weight, row_loss, row_valid, n,
                                   reduction == 0 ? 2 : reduction);
  return check_launch("mi355x_cross_entropy_fwd");
}

extern "C" int mi355x_cross_entropy_bwd(void* dx, int dx_dtype, int64_t ld_dx, const void* logits,
                                        int dtype, int64_t ld, const float* lse,
                                        const int64_t* target, const float* grad_out,
                                        int reduction, const float* total_weight, int64_t n,
                                        int64_t c, int64_t ignore_index, mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0 && c > 0 && ld >= c && ld_dx >= c, "mi355x_cross_entropy_bwd: bad shape");
  MI_REQUIRE(c < (1ll << 30) && ld_dx < (1ll << 30), "mi355x_cross_entropy_bwd: too many classes");
  const int64_t v = 16 / (int64_t)dtype_size(dx_dtype);
  MI_REQUIRE(ld_dx % v == 0 && ((uintptr_t)dx % 16) == 0,
             "mi355x_cross_entropy_bwd: dx rows must be 16-byte aligned (ld_dx a multiple of %lld)", (long long)v);
  MI_REQUIRE(((uintptr_t)logits % dtype_size(dtype)) == 0, "mi355x_cross_entropy_bwd: misaligned logits");
  if (n == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  const int per_row = reduction == 0;
  const float* tw = reduction == 1 ? total_weight : nullptr;
  const int nb = (int)ceil_div(ld_dx / v, kBwdThreads);
  // one block per (row, chunk of kBwdThreads 16-byte pieces): the grid's
  // work-items must stay below 2^32
  MI_REQUIRE(n * nb * kBwdThreads < (1ll << 32), "mi355x_cross_entropy_bwd: too many rows (%lld x %d blocks of %d)",
             (long long)n, nb, kBwdThreads);
#define CE_BWD(TX, TD)                                                                                     \
  ce_bwd_chunks<TX, TD><<<(unsigned)(n * nb), kBwdThreads, 0, s>>>((TD*)dx, ld_dx, (const TX*)logits, ld, \
                                                                  lse, target, grad_out, per_row, tw, n,  \
                                                                  c, ignore_index, nb)
  if (dtype == MI355X_BF16 && dx_dtype == MI355X_BF16) CE_BWD(bf16, bf16);
  else if (dtype == MI355X_F32 && dx_dtype == MI355X_F32) CE_BWD(float, float);
  else if (dtype == MI355X_F16 && dx_dtype == MI355X_F16) CE_BWD(f16, f16);
  else return fail(MI355X_EUNSUPPORTED, "mi355x_cross_entropy_bwd: unsupported dtypes %d/%d", dtype, dx_dtype);
#undef CE_BWD
  return check_launch("mi355x_cross_entropy_bwd");
}

extern "C" int mi355x_cross_entropy_fwd_bwd(void* out, float* total_weight, float* lse, void* dx, int64_t ld_dx,
                                            const void* logits, int dtype, int64_t ld, const int64_t* target,
                                            const float* grad_out, int64_t n, int64_t c, int reduction,
                                            int64_t ignore_index, int32_t* err_flag, void* workspace,
                                            int64_t ws_bytes, mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0 && c > 0 && ld >= c && ld_dx >= c, "mi355x_cross_entropy_fwd_bwd: bad shape");
  MI_REQUIRE(reduction == 1 || reduction == 2, "mi355x_cross_entropy_fwd_bwd: reduction must be mean or sum");
  MI_REQUIRE(out && total_weight && lse && dx && logits && target && grad_out,
             "mi355x_cross_entropy_fwd_bwd: null pointer");
  const int64_t es = (int64_t)dtype_size(dtype);
  MI_REQUIRE(es > 0, "mi355x_cross_entropy_fwd_bwd: bad dtype");
  const int64_t v = 16 / es;
  constexpr int kMaxNC = 32;
  // chunks per row: the logits' (any phase) and dx's
  const int64_t chunks = std::max((c + 2 * v - 2) / v, ld_dx / v);
  MI_REQUIRE((uintptr_t)logits % es == 0 && (uintptr_t)dx % 16 == 0 && ld_dx % v == 0,
             "mi355x_cross_entropy_fwd_bwd: misaligned logits or dx");
  if (chunks > (int64_t)kMaxNC * kRowThreads || c >= (1ll << 30))
    return fail(MI355X_EUNSUPPORTED, "mi355x_cross_entropy_fwd_bwd: rows of at most %d 16-byte chunks",
                kMaxNC * kRowThreads);
  if (n == 0) return MI355X_OK;
  MI_REQUIRE(n < (1ll << 31), "mi355x_cross_entropy_fwd_bwd: too many rows");
  const int64_t need = mi355x_cross_entropy_workspace_bytes(n);
  if (!workspace || ws_bytes < need)
    return fail(MI355X_EWORKSPACE, "mi355x_cross_entropy_fwd_bwd: workspace %lld < %lld", (long long)ws_bytes,
                (long long)need);
  hipStream_t s = (hipStream_t)stream;
  float* row_loss = (float*)workspace;
  float* row_valid = (float*)workspace + n;
  ce_count_valid<<<1, 1024, 0, s>>>(total_weight, target, n, c, ignore_index);
  const float* tw = reduction == 1 ? total_weight : nullptr;
  auto go = [&](auto tag) {
    using T = decltype(tag);
#define CE_FUSED(NC_)                                                                                            ce_fused_rows<T, T, NC_><<<(unsigned)n, kRowThreads, 0, s>>>((T*)dx, ld_dx, row_loss, row_valid, lse,                                                                        (const T*)logits, ld, target, grad_out, tw, c,                                                                ignore_index, err_flag)
    if (chunks <= 8 * kRowThreads) CE_FUSED(8);
    else if (chunks <= 16 * kRowThreads) CE_FUSED(16);
    else if (chunks <= 25 * kRowThreads) CE_FUSED(25);
    else CE_FUSED(32);
#undef CE_FUSED
  };
  switch (dtype) {
    case MI355X_F32: go(float{}); break;
    case MI355X_BF16: go(bf16{}); break;
    case MI355X_F16: go(f16{}); break;
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_cross_entropy_fwd_bwd: unsupported dtype %d", dtype);
  }
  ce_fwd_reduce<<<1, 1024, 0, s>>>((float*)out, total_weight, row_loss, row_valid, n, reduction);
  return check_launch("mi355x_cross_entropy_fwd_bwd");
}
