// Fused softmax cross-entropy over logits [n, c] (row stride ld) and int64
// targets: the log_softmax -> nll_loss chain of the training step without
// materialising log-probabilities or a dense one-hot gradient.
//
// Forward, one 512-thread block per row: an online (max, sum-of-exp) pass
// gives lse_i; row loss = lse_i - x_i[t_i] (0 for ignore_index).  A second
// one-block kernel reduces the row losses in a fixed order into the mean or
// sum and writes total_weight (the count of non-ignored rows).
// Backward, one block per row: dx_i = g_i * (exp(x_i - lse_i) - onehot(t_i)),
// g_i = grad (per row for reduction none, else the scalar, / total_weight
// for mean), zero for ignored rows; columns [c, ld_dx) of dx are zero-filled.
// HBM traffic: forward reads the logits once; backward reads them once and
// writes dx once.
#include <math.h>

#include "common.h"

namespace mi {
namespace {

constexpr int kRowThreads = 512;

struct MS {
  float m, s;
};
__device__ __forceinline__ MS ms_fold(MS a, float x) {
  if (x == -INFINITY) return a;
  if (x != x) return MS{x, a.s};
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

// Visit x[0..c) of one row with 16-byte loads where aligned.
template <typename T, typename F>
__device__ __forceinline__ void for_row(const T* r, int64_t c, F&& f) {
  constexpr int V = 16 / sizeof(T);
  int64_t head = (int64_t)(((16 - ((uintptr_t)r & 15)) & 15) / sizeof(T));
  if (((uintptr_t)r % sizeof(T)) != 0) head = c;
  if (head > c) head = c;
  for (int64_t k = threadIdx.x; k < head; k += kRowThreads) f(k, to_f32(r[k]));
  const int64_t nv = (c - head) / V;
  const T* body = r + head;
  for (int64_t q = threadIdx.x; q < nv; q += kRowThreads) {
    struct alignas(16) P { T v[V]; } p = ((const P*)body)[q];
#pragma unroll
    for (int e = 0; e < V; ++e) f(head + q * V + e, to_f32(p.v[e]));
  }
  for (int64_t k = head + nv * V + threadIdx.x; k < c; k += kRowThreads) f(k, to_f32(r[k]));
}

template <typename T>
__global__ void __launch_bounds__(kRowThreads)
    ce_fwd_rows(float* __restrict__ row_loss, float* __restrict__ row_valid, float* __restrict__ lse,
                const T* __restrict__ x, int64_t ld, const int64_t* __restrict__ target, int64_t n,
                int64_t c, int64_t ignore_index, int32_t* err) {
  __shared__ MS red[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const T* r = x + row * ld;
  MS acc{-INFINITY, 0.f};
  for_row(r, c, [&](int64_t, float v) { acc = ms_fold(acc, v); });
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    MS o{__shfl_xor(acc.m, off, 64), __shfl_xor(acc.s, off, 64)};
    acc = ms_merge(acc, o);
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    MS t = red[0];
    for (int w = 1; w < kRowThreads / 64; ++w) t = ms_merge(t, red[w]);
    const float l = t.m + logf(t.s);
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

template <typename TX, typename TD>
__global__ void __launch_bounds__(kRowThreads)
    ce_bwd_rows(TD* __restrict__ dx, int64_t ld_dx, const TX* __restrict__ x, int64_t ld,
                const float* __restrict__ lse, const int64_t* __restrict__ target,
                const float* __restrict__ grad, int grad_per_row, const float* __restrict__ total,
                int64_t n, int64_t c, int64_t ignore_index) {
  const int64_t row = blockIdx.x;
  const int64_t tg = target[row];
  float g = grad[grad_per_row ? row : 0];
  if (!grad_per_row && total) g /= total[0];
  const bool valid = tg != ignore_index && tg >= 0 && tg < c;
  const float l = lse[row];
  TD* o = dx + row * ld_dx;
  const TX* r = x + row * ld;
  constexpr int V = 16 / sizeof(TD);
  // x is read element-wise through for_row; dx rows are written in the same
  // index order (each thread owns the indices it reads).
  if (!valid) g = 0.f;
  for_row(r, c, [&](int64_t k, float v) {
    float p = expf(v - l);
    o[k] = from_f32<TD>(g * (p - (k == tg ? 1.f : 0.f)));
  });
  (void)V;
  for (int64_t k = c + threadIdx.x; k < ld_dx; k += kRowThreads) o[k] = from_f32<TD>(0.f);
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
  MI_REQUIRE(reduction >= 0 && reduction <= 2, "mi355x_cross_entropy_fwd: bad reduction");
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
  if (n == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  const int per_row = reduction == 0;
  const float* tw = reduction == 1 ? total_weight : nullptr;
#define CE_BWD(TX, TD)                                                                                   \
  ce_bwd_rows<TX, TD><<<(unsigned)n, kRowThreads, 0, s>>>((TD*)dx, ld_dx, (const TX*)logits, ld, lse, \
                                                          target, grad_out, per_row, tw, n, c,       \
                                                          ignore_index)
  if (dtype == MI355X_BF16 && dx_dtype == MI355X_BF16) CE_BWD(bf16, bf16);
  else if (dtype == MI355X_F32 && dx_dtype == MI355X_F32) CE_BWD(float, float);
  else if (dtype == MI355X_F16 && dx_dtype == MI355X_F16) CE_BWD(f16, f16);
  else if (dtype == MI355X_BF16 && dx_dtype == MI355X_F32) CE_BWD(bf16, float);
  else return fail(MI355X_EUNSUPPORTED, "mi355x_cross_entropy_bwd: unsupported dtypes %d/%d", dtype, dx_dtype);
#undef CE_BWD
  return check_launch("mi355x_cross_entropy_bwd");
}
