// Fused attention for the inputs the MFMA kernels do not take: f32 inputs,
// any head_dim up to 256, and the backward of grouped-K/V-head and
// sliding-window attention.  Everything is computed in f32.
//
// Semantics are those of attention.hip: S = scale Q K^T over the visible keys
// (top-left causal: key j visible to query i iff j <= i; with a window w > 0
// also i - j < w), O = softmax(S) V, LSE = natural-log row log-sum-exp;
// backward D_i = sum(dO_i O_i), P = exp(S - LSE), dP = dO V^T,
// dS = P (dP - D), dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO.  With
// grouped K/V heads (H = g * H_kv), query head h reads K/V head h / g, and
// the dK/dV of a K/V head sum over its g query heads (the reference's
// fused gate, eager_kernels/aten_fast.py:7462-7530, accepts f32 and head_dim
// up to 256; flash_attention_bwd_kernels.mojo:13-26 gives the backward).
//
// Layout: a block of 256 threads owns 32 rows (queries, or keys in the dK/dV
// pass); 8 consecutive lanes share a row, lane part p holding head-dim
// elements p, p + 8, p + 16, ...  Row dot products are reduced across the 8
// lanes with xor shuffles.  Tiles of 32 rows of the other operand are staged
// through LDS as f32 (the 8 lanes of a row read 8 consecutive floats; every
// row group of a wave reads the same address, a broadcast).
#include <math.h>

#include "common.h"

namespace mi {
namespace {

constexpr int kGT = 256;             // threads per block
constexpr int kTPR = 8;              // lanes per row
constexpr int kRows = kGT / kTPR;    // rows per block
// rows per staged tile: 32, or 16 at head_dim > 128 (two f32 tiles stay
// within 64 KB of LDS)
template <int E>
constexpr int kTileOf = E == 32 ? 16 : 32;
constexpr int kMaxD = 256;
constexpr float kLog2eG = 1.4426950408889634f;
constexpr float kLn2G = 0.6931471805599453f;

struct GenArgs {
  void* o; int64_t o_b, o_h, o_s;
  float* lse;
  const void* q; int64_t q_b, q_h, q_s;
  const void* k; int64_t k_b, k_h, k_s;
  const void* v; int64_t v_b, v_h, v_s;
  const void* dout; int64_t do_b, do_h, do_s;
  void* dq; int64_t dq_b, dq_h, dq_s;
  void* dk; int64_t dk_b, dk_h, dk_s;
  void* dv; int64_t dv_b, dv_h, dv_s;
  float* delta;
  int64_t B, H, HK, Sq, Skv, D;
  float scale_log2, scale;
  int causal;
  int64_t window;
};

__device__ __forceinline__ bool visible(const GenArgs& p, int64_t i, int64_t j) {
  if (j >= p.Skv) return false;
  if (p.causal && j > i) return false;
  if (p.window > 0 && i - j >= p.window) return false;
  return true;
}

// Sum over the 8 lanes of a row group.
__device__ __forceinline__ float row_sum8(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  x += __shfl_xor(x, 4, 64);
  return x;
}

// This lane's E elements of row `r` (head-dim element part + 8t), as f32.
template <typename T, int E>
__device__ __forceinline__ void load_row(float (&x)[E], const T* row, int part, int64_t D, bool ok) {
#pragma unroll
  for (int t = 0; t < E; ++t) {
    const int64_t d = part + kTPR * t;
    x[t] = (ok && d < D) ? to_f32(row[d]) : 0.f;
  }
}

// Stage rows [r0, r0 + TR) of a [rows, D] operand (row stride rs) into
// LDS as f32 [TR][DP]; rows past `nrows` read as zero.
template <typename T, int DP, int TR>
__device__ __forceinline__ void stage_rows(float* dst, const T* src, int64_t rs, int64_t r0, int64_t nrows,
                                           int64_t D) {
  for (int idx = threadIdx.x; idx < TR * DP; idx += kGT) {
    const int r = idx / DP, d = idx - r * DP;
    const int64_t gr = r0 + r;
    dst[idx] = (gr < nrows && d < D) ? to_f32(src[gr * rs + d]) : 0.f;
  }
}

template <typename T>
__device__ __forceinline__ void store_row(T* row, const float* x, int part, int64_t D, int E) {
  for (int t = 0; t < E; ++t) {
    const int64_t d = part + kTPR * t;
    if (d < D) row[d] = from_f32<T>(x[t]);
  }
}

// ---------------------------------------------------------------------------
// forward: a block owns 32 queries of one (batch, head)
// ---------------------------------------------------------------------------
template <typename T, int E>
__global__ void __launch_bounds__(kGT) gen_fwd(GenArgs p) {
  constexpr int DP = E * kTPR, kTile = kTileOf<E>;
  __shared__ float Ks[kTile * DP];
  __shared__ float Vs[kTile * DP];
  const int part = threadIdx.x & (kTPR - 1), row = threadIdx.x / kTPR;
  const int64_t b = blockIdx.z, h = blockIdx.y, hk = h / (p.H / p.HK);
  const int64_t q0 = (int64_t)blockIdx.x * kRows, qi = q0 + row;
  const bool qok = qi < p.Sq;
  const T* Q = (const T*)p.q + b * p.q_b + h * p.q_h;
  const T* K = (const T*)p.k + b * p.k_b + hk * p.k_h;
  const T* V = (const T*)p.v + b * p.v_b + hk * p.v_h;

  float qv[E], o[E];
  load_row<T, E>(qv, Q + qi * p.q_s, part, p.D, qok);
#pragma unroll
  for (int t = 0; t < E; ++t) qv[t] *= p.scale_log2, o[t] = 0.f;
  float m = -INFINITY, l = 0.f;

  // keys any query of the block can see
  const int64_t qlast = min(p.Sq, q0 + kRows) - 1;
  int64_t kbeg = 0, kend = p.Skv;
  if (p.causal) kend = min(kend, qlast + 1);
  if (p.window > 0) kbeg = max((int64_t)0, q0 - p.window + 1);
  kbeg = kbeg / kTile * kTile;
  for (int64_t kb0 = kbeg; kb0 < kend; kb0 += kTile) {
    __syncthreads();
    stage_rows<T, DP, kTile>(Ks, K, p.k_s, kb0, p.Skv, p.D);
    stage_rows<T, DP, kTile>(Vs, V, p.v_s, kb0, p.Skv, p.D);
    __syncthreads();
    float s[kTile];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int t = 0; t < E; ++t) acc = fmaf(qv[t], Ks[j * DP + part + kTPR * t], acc);
      acc = row_sum8(acc);
      s[j] = visible(p, qi, kb0 + j) ? acc : -INFINITY;
      mx = fmaxf(mx, s[j]);
    }
    if (mx == -INFINITY) continue;  // nothing visible to this row in the tile
    const float m_new = fmaxf(m, mx);
    const float alpha = exp2f(m - m_new);  // m = -inf on the first visible tile: alpha = 0
    l *= alpha;
#pragma unroll
    for (int t = 0; t < E; ++t) o[t] *= alpha;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      const float pj = exp2f(s[j] - m_new);
      l += pj;
#pragma unroll
      for (int t = 0; t < E; ++t) o[t] = fmaf(pj, Vs[j * DP + part + kTPR * t], o[t]);
    }
    m = m_new;
  }
  if (!qok) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int t = 0; t < E; ++t) o[t] *= inv;
  store_row<T>((T*)p.o + b * p.o_b + h * p.o_h + qi * p.o_s, o, part, p.D, E);
  if (part == 0) p.lse[(b * p.H + h) * p.Sq + qi] = l > 0.f ? (m + log2f(l)) * kLn2G : -INFINITY;
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
// D_i = sum_d dO[i, d] O[i, d]
template <typename T, int E>
__global__ void __launch_bounds__(kGT) gen_bwd_delta(GenArgs p) {
  const int part = threadIdx.x & (kTPR - 1);
  const int64_t row = (int64_t)blockIdx.x * kRows + threadIdx.x / kTPR;  // over B*H*Sq
  const bool ok = row < p.B * p.H * p.Sq;
  const int64_t i = ok ? row % p.Sq : 0, bh = ok ? row / p.Sq : 0;
  const int64_t h = bh % p.H, b = bh / p.H;
  float ov[E], dv[E];
  load_row<T, E>(ov, (const T*)p.o + b * p.o_b + h * p.o_h + i * p.o_s, part, p.D, ok);
  load_row<T, E>(dv, (const T*)p.dout + b * p.do_b + h * p.do_h + i * p.do_s, part, p.D, ok);
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < E; ++t) acc = fmaf(ov[t], dv[t], acc);
  acc = row_sum8(acc);
  if (ok && part == 0) p.delta[row] = acc;
}

// dQ: a block owns 32 queries of one (batch, head) and walks the visible keys
template <typename T, int E>
__global__ void __launch_bounds__(kGT) gen_bwd_dq(GenArgs p) {
  constexpr int DP = E * kTPR, kTile = kTileOf<E>;
  __shared__ float Ks[kTile * DP];
  __shared__ float Vs[kTile * DP];
  const int part = threadIdx.x & (kTPR - 1), row = threadIdx.x / kTPR;
  const int64_t b = blockIdx.z, h = blockIdx.y, hk = h / (p.H / p.HK);
  const int64_t q0 = (int64_t)blockIdx.x * kRows, qi = q0 + row;
  const bool qok = qi < p.Sq;
  const T* K = (const T*)p.k + b * p.k_b + hk * p.k_h;
  const T* V = (const T*)p.v + b * p.v_b + hk * p.v_h;
  float qv[E], dov[E], dq[E];
  load_row<T, E>(qv, (const T*)p.q + b * p.q_b + h * p.q_h + qi * p.q_s, part, p.D, qok);
  load_row<T, E>(dov, (const T*)p.dout + b * p.do_b + h * p.do_h + qi * p.do_s, part, p.D, qok);
#pragma unroll
  for (int t = 0; t < E; ++t) qv[t] *= p.scale_log2, dq[t] = 0.f;
  const int64_t ri = (b * p.H + h) * p.Sq + qi;
  const float lse2 = qok ? p.lse[ri] * kLog2eG : 0.f;
  const float di = qok ? p.delta[ri] : 0.f;

  const int64_t qlast = min(p.Sq, q0 + kRows) - 1;
  int64_t kbeg = 0, kend = p.Skv;
  if (p.causal) kend = min(kend, qlast + 1);
  if (p.window > 0) kbeg = max((int64_t)0, q0 - p.window + 1);
  kbeg = kbeg / kTile * kTile;
  for (int64_t kb0 = kbeg; kb0 < kend; kb0 += kTile) {
    __syncthreads();
    stage_rows<T, DP, kTile>(Ks, K, p.k_s, kb0, p.Skv, p.D);
    stage_rows<T, DP, kTile>(Vs, V, p.v_s, kb0, p.Skv, p.D);
    __syncthreads();
#pragma unroll 4
    for (int j = 0; j < kTile; ++j) {
      float sa = 0.f, pa = 0.f;
#pragma unroll
      for (int t = 0; t < E; ++t) {
        sa = fmaf(qv[t], Ks[j * DP + part + kTPR * t], sa);
        pa = fmaf(dov[t], Vs[j * DP + part + kTPR * t], pa);
      }
      sa = row_sum8(sa);
      pa = row_sum8(pa);
      const float pj = (qok && visible(p, qi, kb0 + j)) ? exp2f(sa - lse2) : 0.f;
      const float ds = pj * (pa - di);
#pragma unroll
      for (int t = 0; t < E; ++t) dq[t] = fmaf(ds, Ks[j * DP + part + kTPR * t], dq[t]);
    }
  }
  if (!qok) return;
#pragma unroll
  for (int t = 0; t < E; ++t) dq[t] *= p.scale;
  store_row<T>((T*)p.dq + b * p.dq_b + h * p.dq_h + qi * p.dq_s, dq, part, p.D, E);
}

// dK/dV: a block owns 32 keys of one (batch, K/V head) and walks, for each
// query head of its group, the queries that can see them
template <typename T, int E>
__global__ void __launch_bounds__(kGT) gen_bwd_dkv(GenArgs p) {
  constexpr int DP = E * kTPR, kTile = kTileOf<E>;
  __shared__ float Qs[kTile * DP];
  __shared__ float Ds[kTile * DP];
  __shared__ float lse_s[kTile], del_s[kTile];
  const int part = threadIdx.x & (kTPR - 1), row = threadIdx.x / kTPR;
  const int64_t b = blockIdx.z, hk = blockIdx.y, g = p.H / p.HK;
  const int64_t k0 = (int64_t)blockIdx.x * kRows, kj = k0 + row;
  const bool kok = kj < p.Skv;
  float kv[E], vv[E], dk[E], dv[E];
  load_row<T, E>(kv, (const T*)p.k + b * p.k_b + hk * p.k_h + kj * p.k_s, part, p.D, kok);
  load_row<T, E>(vv, (const T*)p.v + b * p.v_b + hk * p.v_h + kj * p.v_s, part, p.D, kok);
#pragma unroll
  for (int t = 0; t < E; ++t) kv[t] *= p.scale_log2, dk[t] = dv[t] = 0.f;

  // queries that can see some key of the block
  const int64_t klast = min(p.Skv, k0 + kRows) - 1;
  int64_t qbeg = 0, qend = p.Sq;
  if (p.causal) qbeg = k0;
  if (p.window > 0) qend = min(qend, klast + p.window);
  qbeg = qbeg / kTile * kTile;
  for (int64_t r = 0; r < g; ++r) {
    const int64_t h = hk * g + r;
    const T* Q = (const T*)p.q + b * p.q_b + h * p.q_h;
    const T* dO = (const T*)p.dout + b * p.do_b + h * p.do_h;
    const float* LSE = p.lse + (b * p.H + h) * p.Sq;
    const float* DEL = p.delta + (b * p.H + h) * p.Sq;
    for (int64_t qb0 = qbeg; qb0 < qend; qb0 += kTile) {
      __syncthreads();
      stage_rows<T, DP, kTile>(Qs, Q, p.q_s, qb0, p.Sq, p.D);
      stage_rows<T, DP, kTile>(Ds, dO, p.do_s, qb0, p.Sq, p.D);
      if (threadIdx.x < kTile) {
        const int64_t qi = qb0 + threadIdx.x;
        lse_s[threadIdx.x] = qi < p.Sq ? LSE[qi] * kLog2eG : 0.f;
        del_s[threadIdx.x] = qi < p.Sq ? DEL[qi] : 0.f;
      }
      __syncthreads();
#pragma unroll 4
      for (int i = 0; i < kTile; ++i) {
        float sa = 0.f, pa = 0.f;
#pragma unroll
        for (int t = 0; t < E; ++t) {
          sa = fmaf(kv[t], Qs[i * DP + part + kTPR * t], sa);
          pa = fmaf(vv[t], Ds[i * DP + part + kTPR * t], pa);
        }
        sa = row_sum8(sa);
        pa = row_sum8(pa);
        const int64_t qi = qb0 + i;
        const float pi = (kok && qi < p.Sq && visible(p, qi, kj)) ? exp2f(sa - lse_s[i]) : 0.f;
        const float ds = pi * (pa - del_s[i]);
#pragma unroll
        for (int t = 0; t < E; ++t) {
          dv[t] = fmaf(pi, Ds[i * DP + part + kTPR * t], dv[t]);
          dk[t] = fmaf(ds, Qs[i * DP + part + kTPR * t], dk[t]);
        }
      }
    }
  }
  if (!kok) return;
#pragma unroll
  for (int t = 0; t < E; ++t) dk[t] *= p.scale;
  store_row<T>((T*)p.dk + b * p.dk_b + hk * p.dk_h + kj * p.dk_s, dk, part, p.D, E);
  store_row<T>((T*)p.dv + b * p.dv_b + hk * p.dv_h + kj * p.dv_s, dv, part, p.D, E);
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
int gen_check(int64_t B, int64_t H, int64_t HK, int64_t Sq, int64_t Skv, int64_t D, int dtype, int causal,
              int64_t window, const char* what) {
  if (dtype != MI355X_F32 && dtype != MI355X_BF16 && dtype != MI355X_F16)
    return fail(MI355X_EUNSUPPORTED, "%s: dtype %d not supported (f32/bf16/f16)", what, dtype);
  if (D <= 0 || D > kMaxD) return fail(MI355X_EUNSUPPORTED, "%s: head_dim %lld not in 1..256", what, (long long)D);
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0 || B >= 65536 || H >= 65536)
    return fail(MI355X_EINVAL, "%s: bad shape", what);
  if (HK < 1 || H % HK != 0)
    return fail(MI355X_EINVAL, "%s: heads (%lld) must be a multiple of kv_heads (%lld)", what, (long long)H,
                (long long)HK);
  if (window < 0 || (window > 0 && !causal)) return fail(MI355X_EINVAL, "%s: a sliding window needs causal attention", what);
  return MI355X_OK;
}

template <typename T, int E>
int gen_fwd_launch(const GenArgs& a, hipStream_t s) {
  gen_fwd<T, E><<<dim3(ceil_div(a.Sq, kRows), (unsigned)a.H, (unsigned)a.B), kGT, 0, s>>>(a);
  return check_launch("mi355x_attn_fwd_gen");
}

template <typename T, int E>
int gen_bwd_launch(const GenArgs& a, hipStream_t s) {
  gen_bwd_delta<T, E><<<ceil_div(a.B * a.H * a.Sq, kRows), kGT, 0, s>>>(a);
  gen_bwd_dq<T, E><<<dim3(ceil_div(a.Sq, kRows), (unsigned)a.H, (unsigned)a.B), kGT, 0, s>>>(a);
  gen_bwd_dkv<T, E><<<dim3(ceil_div(a.Skv, kRows), (unsigned)a.HK, (unsigned)a.B), kGT, 0, s>>>(a);
  return check_launch("mi355x_attn_bwd_gen");
}

// dispatch on dtype and the per-lane element count (8, 16 or 32)
#define MI_GEN_DISPATCH(dtype, D, FN, ...)                                      \
  do {                                                                          \
    const int e_ = D <= 64 ? 8 : (D <= 128 ? 16 : 32);                          \
    if (dtype == MI355X_F32) {                                                  \
      if (e_ == 8) return FN<float, 8>(__VA_ARGS__);                            \
      if (e_ == 16) return FN<float, 16>(__VA_ARGS__);                          \
      return FN<float, 32>(__VA_ARGS__);                                        \
    }                                                                           \
    if (dtype == MI355X_BF16) {                                                 \
      if (e_ == 8) return FN<bf16, 8>(__VA_ARGS__);                             \
      if (e_ == 16) return FN<bf16, 16>(__VA_ARGS__);                           \
      return FN<bf16, 32>(__VA_ARGS__);                                         \
    }                                                                           \
    if (e_ == 8) return FN<f16, 8>(__VA_ARGS__);                                \
    if (e_ == 16) return FN<f16, 16>(__VA_ARGS__);                              \
    return FN<f16, 32>(__VA_ARGS__);                                            \
  } while (0)

GenArgs gen_args(const void* q, const int64_t* q_bhs, const void* k, const int64_t* k_bhs, const void* v,
                 const int64_t* v_bhs, int64_t batch, int64_t heads, int64_t kv_heads, int64_t sq, int64_t skv,
                 int64_t d, double scale, int causal, int64_t window) {
  GenArgs a{};
  a.q = q; a.q_b = q_bhs[0]; a.q_h = q_bhs[1]; a.q_s = q_bhs[2];
  a.k = k; a.k_b = k_bhs[0]; a.k_h = k_bhs[1]; a.k_s = k_bhs[2];
  a.v = v; a.v_b = v_bhs[0]; a.v_h = v_bhs[1]; a.v_s = v_bhs[2];
  a.B = batch; a.H = heads; a.HK = kv_heads; a.Sq = sq; a.Skv = skv; a.D = d;
  a.scale = (float)scale;
  a.scale_log2 = (float)(scale * 1.4426950408889634);
  a.causal = causal;
  a.window = window;
  return a;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi355x_attn_fwd_gen(void* o, const int64_t* o_bhs, float* lse, const void* q, const int64_t* q_bhs,
                                   const void* k, const int64_t* k_bhs, const void* v, const int64_t* v_bhs,
                                   int64_t batch, int64_t heads, int64_t kv_heads, int64_t sq, int64_t skv,
                                   int64_t d, double scale, int causal, int64_t window, int dtype,
                                   mi355x_stream_t stream) {
  int rc = gen_check(batch, heads, kv_heads, sq, skv, d, dtype, causal, window, "mi355x_attn_fwd_gen");
  if (rc) return rc;
  MI_REQUIRE(o && lse && q && k && v, "mi355x_attn_fwd_gen: null pointer");
  GenArgs a = gen_args(q, q_bhs, k, k_bhs, v, v_bhs, batch, heads, kv_heads, sq, skv, d, scale, causal, window);
  a.o = o; a.o_b = o_bhs[0]; a.o_h = o_bhs[1]; a.o_s = o_bhs[2];
  a.lse = lse;
  MI_GEN_DISPATCH(dtype, d, gen_fwd_launch, a, (hipStream_t)stream);
}

namespace mi {
// attention.hip: the MFMA backward for grouped/windowed bf16/f16 attention
// (-1 when it does not take the inputs)
int attn_bwd_grouped_mfma(void* dq, const int64_t* dq_bhs, void* dk, const int64_t* dk_bhs, void* dv,
                          const int64_t* dv_bhs, const void* dout, const int64_t* do_bhs, const void* q,
                          const int64_t* q_bhs, const void* k, const int64_t* k_bhs, const void* v,
                          const int64_t* v_bhs, const void* o, const int64_t* o_bhs, const float* lse,
                          int64_t batch, int64_t heads, int64_t kv_heads, int64_t sq, int64_t skv, int64_t d,
                          double scale, int causal, int64_t window, int dtype, void* workspace,
                          hipStream_t stream);
}  // namespace mi

// Two floats per query row (the MFMA path keeps -D and -LSE log2(e), the f32
// path D) and, with grouped heads, the MFMA path's per-query-head dK and dV
// partials in f32.
extern "C" int64_t mi355x_attn_bwd_gen_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads, int64_t sq,
                                                       int64_t skv, int64_t d) {
  int64_t bytes = 2 * batch * heads * sq * (int64_t)sizeof(float) + 256;
  if (kv_heads >= 1 && heads > kv_heads) bytes += 2 * batch * heads * skv * d * (int64_t)sizeof(float) + 256;
  return bytes;
}

extern "C" int mi355x_attn_bwd_gen(void* dq, const int64_t* dq_bhs, void* dk, const int64_t* dk_bhs, void* dv,
                                   const int64_t* dv_bhs, const void* dout, const int64_t* do_bhs, const void* q,
                                   const int64_t* q_bhs, const void* k, const int64_t* k_bhs, const void* v,
                                   const int64_t* v_bhs, const void* o, const int64_t* o_bhs, const float* lse,
                                   int64_t batch, int64_t heads, int64_t kv_heads, int64_t sq, int64_t skv,
                                   int64_t d, double scale, int causal, int64_t window, int dtype,
                                   void* workspace, int64_t ws_bytes, mi355x_stream_t stream) {
  int rc = gen_check(batch, heads, kv_heads, sq, skv, d, dtype, causal, window, "mi355x_attn_bwd_gen");
  if (rc) return rc;
  MI_REQUIRE(dq && dk && dv && dout && q && k && v && o && lse, "mi355x_attn_bwd_gen: null pointer");
  const int64_t need = mi355x_attn_bwd_gen_workspace_bytes(batch, heads, kv_heads, sq, skv, d);
  if (!workspace || ws_bytes < need)
    return fail(MI355X_EWORKSPACE, "mi355x_attn_bwd_gen: workspace %lld < %lld", (long long)ws_bytes,
                (long long)need);
  const int mrc = attn_bwd_grouped_mfma(dq, dq_bhs, dk, dk_bhs, dv, dv_bhs, dout, do_bhs, q, q_bhs, k, k_bhs, v,
                                        v_bhs, o, o_bhs, lse, batch, heads, kv_heads, sq, skv, d, scale, causal,
                                        window, dtype, workspace, (hipStream_t)stream);
  if (mrc >= 0) return mrc;  // bf16/f16 at head_dim 64/128/256: MFMA kernels
  GenArgs a = gen_args(q, q_bhs, k, k_bhs, v, v_bhs, batch, heads, kv_heads, sq, skv, d, scale, causal, window);
  a.o = (void*)o; a.o_b = o_bhs[0]; a.o_h = o_bhs[1]; a.o_s = o_bhs[2];
  a.lse = (float*)lse;
  a.dout = dout; a.do_b = do_bhs[0]; a.do_h = do_bhs[1]; a.do_s = do_bhs[2];
  a.dq = dq; a.dq_b = dq_bhs[0]; a.dq_h = dq_bhs[1]; a.dq_s = dq_bhs[2];
  a.dk = dk; a.dk_b = dk_bhs[0]; a.dk_h = dk_bhs[1]; a.dk_s = dk_bhs[2];
  a.dv = dv; a.dv_b = dv_bhs[0]; a.dv_h = dv_bhs[1]; a.dv_s = dv_bhs[2];
  a.delta = (float*)workspace;
  MI_GEN_DISPATCH(dtype, d, gen_bwd_launch, a, (hipStream_t)stream);
}
