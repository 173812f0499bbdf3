// NLL loss forward/backward over log-probabilities [N, C] and int64 targets.
//
// Forward: loss_n = -w[t_n] * logp[n, t_n] (0 for ignore_index), reduced by
// one block in a fixed order (deterministic); total_weight = sum of w[t_n].
// Backward writes every element of grad_input once: one block per row, the
// row zero-filled with 16-byte stores (scalar head/tail for unaligned rows)
// and the target element set to -w[t]*g (/ total_weight for mean).
#include "common.h"

namespace mi {
namespace {

constexpr int kRedThreads = 1024;

template <typename T>
__global__ void __launch_bounds__(kRedThreads)
    nll_fwd_kernel(T* __restrict__ out, T* __restrict__ total, const T* __restrict__ logp,
                   const int64_t* __restrict__ target, const T* __restrict__ weight, int64_t n,
                   int64_t c, int reduction, int64_t ignore_index, int32_t* err) {
  __shared__ float red[kRedThreads / 64];
  float ls = 0.f, ws = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += kRedThreads) {
    const int64_t t = target[i];
    float loss = 0.f, w = 0.f;
    if (t != ignore_index) {
      if (t < 0 || t >= c) {
        if (err) *err = 1;
      } else {
        w = weight ? to_f32(weight[t]) : 1.f;
        loss = -to_f32(logp[i * c + t]) * w;
      }
    }
    if (reduction == 0) out[i] = from_f32<T>(loss);
    ls += loss;
    ws += w;
  }
  ls = block_sum(ls, red);
  ws = block_sum(ws, red);
  if (threadIdx.x == 0) {
    if (reduction == 1) out[0] = from_f32<T>(ls / ws);
    else if (reduction == 2) out[0] = from_f32<T>(ls);
    total[0] = from_f32<T>(ws);
  }
}

template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
};

template <typename T>
__global__ void __launch_bounds__(256)
    nll_bwd_kernel(T* __restrict__ gi, const T* __restrict__ grad_out,
                   const int64_t* __restrict__ target, const T* __restrict__ weight,
                   const T* __restrict__ total_weight, int64_t n, int64_t c, int reduction,
                   int64_t ignore_index) {
  constexpr int V = Vec16<T>::N;
  for (int64_t row = blockIdx.x; row < n; row += gridDim.x) {
    const int64_t t = target[row];
    float val = 0.f;
    if (t != ignore_index && t >= 0 && t < c) {
      const float w = weight ? to_f32(weight[t]) : 1.f;
      const float g = to_f32(grad_out[reduction == 0 ? row : 0]);
      val = -w * g;
      if (reduction == 1) val /= to_f32(total_weight[0]);
    }
    const T tv = from_f32<T>(val);
    const T zero = from_f32<T>(0.f);
    T* r = gi + row * c;
    // scalar head up to 16-byte alignment
    int64_t head = (int64_t)(((16 - ((uintptr_t)r & 15)) & 15) / sizeof(T));
    if (((uintptr_t)r % sizeof(T)) != 0) head = c;  // cannot vectorise
    if (head > c) head = c;
    for (int64_t k = threadIdx.x; k < head; k += 256) r[k] = (k == t) ? tv : zero;
    const int64_t nv = (c - head) / V;
    T* body = r + head;
    for (int64_t k = threadIdx.x; k < nv; k += 256) {
      struct alignas(16) P { T v[V]; } p;
#pragma unroll
      for (int e = 0; e < V; ++e) p.v[e] = (head + k * V + e == t) ? tv : zero;
      ((P*)body)[k] = p;
    }
    for (int64_t k = head + nv * V + threadIdx.x; k < c; k += 256) r[k] = (k == t) ? tv : zero;
  }
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int64_t mi355x_nll_workspace_bytes(int64_t n) {
  (void)n;
  return 0;
}

extern "C" int mi355x_nll_fwd(void* out, void* total_weight, const void* logp, int dtype,
                              const int64_t* target, const void* weight, int64_t n, int64_t c,
                              int reduction, int64_t ignore_index, int32_t* err_flag,
                              void* workspace, int64_t ws_bytes, mi355x_stream_t stream) {
  (void)workspace;
  (void)ws_bytes;
  MI_REQUIRE(n >= 0 && c >= 0, "mi355x_nll_fwd: bad shape");
  MI_REQUIRE(reduction >= 0 && reduction <= 2, "mi355x_nll_fwd: bad reduction %d", reduction);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MI355X_F32:
      nll_fwd_kernel<float><<<1, kRedThreads, 0, s>>>((float*)out, (float*)total_weight, (const float*)logp, target, (const float*)weight, n, c, reduction, ignore_index, err_flag);
      break;
    case MI355X_BF16:
      nll_fwd_kernel<bf16><<<1, kRedThreads, 0, s>>>((bf16*)out, (bf16*)total_weight, (const bf16*)logp, target, (const bf16*)weight, n, c, reduction, ignore_index, err_flag);
      break;
    case MI355X_F16:
      nll_fwd_kernel<f16><<<1, kRedThreads, 0, s>>>((f16*)out, (f16*)total_weight, (const f16*)logp, target, (const f16*)weight, n, c, reduction, ignore_index, err_flag);
      break;
    default:
      return fail(MI355X_EUNSUPPORTED, "mi355x_nll_fwd: unsupported dtype %d", dtype);
  }
  return check_launch("mi355x_nll_fwd");
}

extern "C" int mi355x_nll_bwd(void* grad_input, const void* grad_out, const int64_t* target,
                              const void* weight, const void* total_weight, int64_t n, int64_t c,
                              int reduction, int64_t ignore_index, int dtype,
                              mi355x_stream_t stream) {
  MI_REQUIRE(n >= 0 && c >= 0, "mi355x_nll_bwd: bad shape");
  if (n == 0 || c == 0) return MI355X_OK;
  hipStream_t s = (hipStream_t)stream;
  const unsigned grid = (unsigned)(n < 65536 ? n : 65536);
  switch (dtype) {
    case MI355X_F32:
      nll_bwd_kernel<float><<<grid, 256, 0, s>>>((float*)grad_input, (const float*)grad_out, target, (const float*)weight, (const float*)total_weight, n, c, reduction, ignore_index);
      break;
    case MI355X_BF16:
      nll_bwd_kernel<bf16><<<grid, 256, 0, s>>>((bf16*)grad_input, (const bf16*)grad_out, target, (const bf16*)weight, (const bf16*)total_weight, n, c, reduction, ignore_index);
      break;
    case MI355X_F16:
      nll_bwd_kernel<f16><<<grid, 256, 0, s>>>((f16*)grad_input, (const f16*)grad_out, target, (const f16*)weight, (const f16*)total_weight, n, c, reduction, ignore_index);
      break;
    default:
      return fail(MI355X_EUNSUPPORTED, "mi355x_nll_bwd: unsupported dtype %d", dtype);
  }
  return check_launch("mi355x_nll_bwd");
}
