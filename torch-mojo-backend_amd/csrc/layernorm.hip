// LayerNorm forward/backward over rows of `cols` contiguous elements.
//
// Forward: one 64-lane wave per row; the row stays in registers (4 elements
// per lane per vector, NV vectors) so x is read once and y written once: the
// HBM traffic is rows*cols*(2*sizeof(T)) + 8*rows bytes.  Mean and variance
// use two passes over the registers (no cancellation), variance biased, as
// ATen's layer_norm does (mean/rstd in f32).
//
// Backward: the same wave-per-row layout computes
//   xhat = (x-mean)*rstd, g = dy*gamma,
//   dx   = rstd * (g - mean(g) - xhat*mean(g*xhat)),
// while each lane accumulates dgamma += dy*xhat and dbeta += dy for its
// columns over the rows its block owns.  Each wave loads its next row before
// it computes the current one.  Block partials go to a workspace
// [blocks, cols] and a second kernel sums them in a fixed order, so the
// result is deterministic.
#include "common.h"
#include "vec.h"

namespace mi {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxBwdBlocks = 1024;

// y = (x - mean) * rstd * gamma + beta (gamma 1 and beta 0 when absent):
// every forward kernel and ln_apply evaluate it through this one function,
// so y recomputed later from x and the saved statistics has the same bits.
__device__ __forceinline__ float ln_out(float x, float mu, float r, float g, float b) {
  return (x - mu) * r * g + b;
}

// y (optional when y_low is given) and y_low (optional, element type TL): a
// second copy of y rounded to a 16-bit type, the operand an autocast matmul
// consumes next.  A caller that needs only the 16-bit copy passes y = null
// and can produce y later with mi355x_layer_norm_apply.
template <typename T, typename TL, int NV>
__global__ void __launch_bounds__(kThreads)
    ln_fwd_wave(T* __restrict__ y, TL* __restrict__ y_low, float* __restrict__ mean_out,
                float* __restrict__ rstd_out, const T* __restrict__ x, const T* __restrict__ gamma,
                const T* __restrict__ beta, int64_t rows, int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  float v[NV][4];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (c < cols) {
      Vec4<T>::load(xr + c, v[j]);
    } else {
      v[j][0] = v[j][1] = v[j][2] = v[j][3] = 0.f;
    }
    s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
  }
  const float inv_n = 1.f / (float)cols;
  const float mu = wave_sum(s) * inv_n;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (c < cols) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[j][e] - mu;
        q += d * d;
      }
    }
  }
  const float var = wave_sum(q) * inv_n;
  const float r = 1.f / sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (c < cols) {
      float g[4] = {1.f, 1.f, 1.f, 1.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
      if (gamma) Vec4<T>::load(gamma + c, g);
      if (beta) Vec4<T>::load(beta + c, b);
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = ln_out(v[j][e], mu, r, g[e], b[e]);
      if (y) Vec4<T>::store(y + row * cols + c, o);
      if (y_low) Vec4<TL>::store(y_low + row * cols + c, o);
    }
  }
  if (lane == 0) {
    if (mean_out) mean_out[row] = mu;
    if (rstd_out) rstd_out[row] = r;
  }
}

// The residual add fused in front of the norm: x = a + r (r of type TR,
// added in f32 and rounded to T exactly as the separate add would), x stored
// to x_out, then y = LayerNorm(x) as ln_fwd_wave.  One pass over a and r
// instead of an add (read a, r; write x) followed by a norm (read x again).
template <typename T, typename TR, typename TL, int NV>
__global__ void __launch_bounds__(kThreads)
    ln_fwd_add_wave(T* __restrict__ y, TL* __restrict__ y_low, float* __restrict__ mean_out,
                    float* __restrict__ rstd_out, T* __restrict__ x_out, const T* __restrict__ a,
                    const TR* __restrict__ r, const T* __restrict__ gamma, const T* __restrict__ beta,
                    int64_t rows, int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float v[NV][4];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (c < cols) {
      float av[4], rv[4];
      Vec4<T>::load(a + base + c, av);
      Vec4<TR>::load(r + base + c, rv);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[j][e] = to_f32(from_f32<T>(av[e] + rv[e]));
      Vec4<T>::store(x_out + base + c, v[j]);
    } else {
      v[j][0] = v[j][1] = v[j][2] = v[j][3] = 0.f;
    }
    s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
  }
  const float inv_n = 1.f / (float)cols;
  const float mu = wave_sum(s) * inv_n;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (c < cols) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[j][e] - mu;
        q += d * d;
      }
    }
  }
  const float var = wave_sum(q) * inv_n;
  const float rs = 1.f / sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (c < cols) {
      float g[4] = {1.f, 1.f, 1.f, 1.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
      if (gamma) Vec4<T>::load(gamma + c, g);
      if (beta) Vec4<T>::load(beta + c, b);
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = ln_out(v[j][e], mu, rs, g[e], b[e]);
      if (y) Vec4<T>::store(y + base + c, o);
      if (y_low) Vec4<TL>::store(y_low + base + c, o);
    }
  }
  if (lane == 0) {
    if (mean_out) mean_out[row] = mu;
    if (rstd_out) rstd_out[row] = rs;
  }
}

// Any `cols`: one block per row, three passes over the row.
template <typename T, typename TL>
__global__ void __launch_bounds__(kThreads)
    ln_fwd_block(T* __restrict__ y, TL* __restrict__ y_low, float* __restrict__ mean_out,
                 float* __restrict__ rstd_out, const T* __restrict__ x, const T* __restrict__ gamma,
                 const T* __restrict__ beta, int64_t rows, int64_t cols, float eps) {
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) s += to_f32(xr[c]);
  const float mu = block_sum(s, red) / (float)cols;
  float q = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const float d = to_f32(xr[c]) - mu;
    q += d * d;
  }
  const float var = block_sum(q, red) / (float)cols;
  const float r = 1.f / sqrtf(var + eps);
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const float o = ln_out(to_f32(xr[c]), mu, r, gamma ? to_f32(gamma[c]) : 1.f, beta ? to_f32(beta[c]) : 0.f);
    if (y) y[row * cols + c] = from_f32<T>(o);
    if (y_low) y_low[row * cols + c] = from_f32<TL>(o);
  }
  if (threadIdx.x == 0) {
    if (mean_out) mean_out[row] = mu;
    if (rstd_out) rstd_out[row] = r;
  }
}

// y from x and the statistics a forward saved (mean, rstd per row): the
// output of a forward that wrote only its 16-bit copy, produced when it is
// first read.  Four elements per thread when the rows allow 16-byte access.
template <typename T, bool V4>
__global__ void __launch_bounds__(kThreads)
    ln_apply(T* __restrict__ y, const T* __restrict__ x, const float* __restrict__ mean,
             const float* __restrict__ rstd, const T* __restrict__ gamma, const T* __restrict__ beta,
             int64_t rows, int64_t cols) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  if constexpr (V4) {
    const int64_t n4 = rows * cols / 4;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
      const int64_t row = i * 4 / cols, c = i * 4 - row * cols;
      float v[4], g[4] = {1.f, 1.f, 1.f, 1.f}, b[4] = {0.f, 0.f, 0.f, 0.f}, o[4];
      Vec4<T>::load(x + i * 4, v);
      if (gamma) Vec4<T>::load(gamma + c, g);
      if (beta) Vec4<T>::load(beta + c, b);
      const float mu = mean[row], r = rstd[row];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = ln_out(v[e], mu, r, g[e], b[e]);
      Vec4<T>::store(y + i * 4, o);
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < rows * cols; i += stride) {
      const int64_t row = i / cols, c = i - row * cols;
      y[i] = from_f32<T>(ln_out(to_f32(x[i]), mean[row], rstd[row], gamma ? to_f32(gamma[c]) : 1.f,
                                beta ? to_f32(beta[c]) : 0.f));
    }
  }
}

// RMSNorm forward (the Gemma-3-shaped workload's norm; torch's rms_norm):
// y = x * rstd * w, rstd = 1/sqrt(mean(x^2) + eps), statistics in f32; the
// weight may be f32 on a 16-bit x (Gemma scales by 1 + w computed in f32).
template <typename T, typename W, int NV>
__global__ void __launch_bounds__(kThreads)
    rms_fwd_wave(T* __restrict__ y, float* __restrict__ rstd_out, const T* __restrict__ x,
                 const W* __restrict__ w, int64_t rows, int cols, float eps, float w_off) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  float v[NV][4];
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (c < cols) {
      Vec4<T>::load(xr + c, v[j]);
    } else {
      v[j][0] = v[j][1] = v[j][2] = v[j][3] = 0.f;
    }
    q += (v[j][0] * v[j][0] + v[j][1] * v[j][1]) + (v[j][2] * v[j][2] + v[j][3] * v[j][3]);
  }
  const float r = 1.f / sqrtf(wave_sum(q) / (float)cols + eps);
  T* yr = y + row * cols;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    if (c < cols) {
      float g[4] = {1.f, 1.f, 1.f, 1.f};
      if (w) Vec4<W>::load(w + c, g);
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = v[j][e] * r * (w ? g[e] + w_off : 1.f);
      Vec4<T>::store(yr + c, o);
    }
  }
  if (lane == 0 && rstd_out) rstd_out[row] = r;
}

template <typename T, typename W>
__global__ void __launch_bounds__(kThreads)
    rms_fwd_block(T* __restrict__ y, float* __restrict__ rstd_out, const T* __restrict__ x,
                  const W* __restrict__ w, int64_t rows, int64_t cols, float eps, float w_off) {
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  float q = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const float d = to_f32(xr[c]);
    q += d * d;
  }
  const float r = 1.f / sqrtf(block_sum(q, red) / (float)cols + eps);
  T* yr = y + row * cols;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    float o = to_f32(xr[c]) * r;
    if (w) o *= to_f32(w[c]) + w_off;
    yr[c] = from_f32<T>(o);
  }
  if (threadIdx.x == 0 && rstd_out) rstd_out[row] = r;
}

// One row of x and dy for this lane's columns.  Columns past `cols` read
// column 0 (always in bounds) and are zeroed, so the loads need no branch and
// the row stays in registers.
template <typename T, int NV>
__device__ __forceinline__ void ln_load_row(const T* __restrict__ x, const T* __restrict__ dy, int64_t base,
                                            const int (&coff)[NV], const bool (&cv)[NV], float (&xv)[NV][4],
                                            float (&dv)[NV][4]) {
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    Vec4<T>::load(x + base + coff[j], xv[j]);
    Vec4<T>::load(dy + base + coff[j], dv[j]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xv[j][e] = cv[j] ? xv[j][e] : 0.f;
      dv[j][e] = cv[j] ? dv[j][e] : 0.f;
    }
  }
}

// RMS: the rms_norm backward (no mean: mean may be null; the scale is
// gamma + goff): dx = r (g w - x r m2), m2 = mean over the row of g w x r,
// dw partials = sum of g x r over the block's rows.
template <typename T, int NV, int W, bool RMS = false>
__global__ void __launch_bounds__(64 * W)
    ln_bwd_wave(T* __restrict__ dx, float* __restrict__ part_g, float* __restrict__ part_b,
                const T* __restrict__ dy, const T* __restrict__ x, const float* __restrict__ mean,
                const float* __restrict__ rstd, const T* __restrict__ gamma, int64_t rows, int cols,
                int64_t rows_per_block, float goff = 0.f) {
  __shared__ float lds[2][W][NV * 256];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const bool want_params = part_g != nullptr;
  int coff[NV];
  bool cv[NV];
  float pg[NV][4], pb[NV][4], gm[NV][4];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    cv[j] = c < cols;
    coff[j] = cv[j] ? c : 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) pg[j][e] = pb[j][e] = 0.f, gm[j][e] = 1.f;
    if (gamma) {
      Vec4<T>::load(gamma + coff[j], gm[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) gm[j][e] = cv[j] ? gm[j][e] + goff : 0.f;
    }
  }
  const float inv_n = 1.f / (float)cols;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = min(rows, r0 + rows_per_block);
  // The host sizes the grid so every block owns at least one row.  Each wave
  // takes rows r0+wid, r0+wid+W, ... and loads the next one before it
  // computes the current one (the last prefetch re-reads row r1-1).
  const int64_t last = r1 - 1;
  int64_t row = r0 + wid;
  float xa[NV][4], da[NV][4];
  float mu = 0.f, rs = 0.f;
  {
    const int64_t first = min(row, last);
    ln_load_row<T, NV>(x, dy, first * cols, coff, cv, xa, da);
    mu = RMS ? 0.f : mean[first];
    rs = rstd[first];
  }
  for (; row < r1; row += W) {
    const int64_t nxt = min(row + W, last);
    float xn[NV][4], dn[NV][4];
    ln_load_row<T, NV>(x, dy, nxt * cols, coff, cv, xn, dn);
    const float mu_n = RMS ? 0.f : mean[nxt], rs_n = rstd[nxt];
    float xh[NV][4], gy[NV][4];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xh[j][e] = (xa[j][e] - mu) * rs;
        gy[j][e] = da[j][e] * gm[j][e];
        s1 += gy[j][e];
        s2 += gy[j][e] * xh[j][e];
        pg[j][e] += da[j][e] * xh[j][e];
        pb[j][e] += da[j][e];
      }
    if (dx) {
      const float m1 = RMS ? 0.f : wave_sum(s1) * inv_n;
      const float m2 = wave_sum(s2) * inv_n;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        if (cv[j]) {
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = rs * (gy[j][e] - m1 - xh[j][e] * m2);
          Vec4<T>::store(dx + row * cols + coff[j], o);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) xa[j][e] = xn[j][e], da[j][e] = dn[j][e];
    mu = mu_n;
    rs = rs_n;
  }
  if (!want_params) return;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lds[0][wid][(j * 64 + lane) * 4 + e] = pg[j][e];
      lds[1][wid][(j * 64 + lane) * 4 + e] = pb[j][e];
    }
  __syncthreads();
  for (int c = threadIdx.x; c < cols; c += 64 * W) {
    float g = 0.f, b = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) g += lds[0][w][c], b += lds[1][w][c];
    part_g[(int64_t)blockIdx.x * cols + c] = g;
    part_b[(int64_t)blockIdx.x * cols + c] = b;
  }
}

// Any `cols`: dx with one block per row.
template <typename T>
__global__ void __launch_bounds__(kThreads)
    ln_bwd_dx_block(T* __restrict__ dx, const T* __restrict__ dy, const T* __restrict__ x,
                    const float* __restrict__ mean, const float* __restrict__ rstd,
                    const T* __restrict__ gamma, int64_t cols) {
  __shared__ float red[kWaves];
  const int64_t row = blockIdx.x;
  const float mu = mean[row], rs = rstd[row];
  float s1 = 0.f, s2 = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const float g = to_f32(dy[row * cols + c]) * (gamma ? to_f32(gamma[c]) : 1.f);
    const float xh = (to_f32(x[row * cols + c]) - mu) * rs;
    s1 += g;
    s2 += g * xh;
  }
  const float m1 = block_sum(s1, red) / (float)cols;
  const float m2 = block_sum(s2, red) / (float)cols;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const float g = to_f32(dy[row * cols + c]) * (gamma ? to_f32(gamma[c]) : 1.f);
    const float xh = (to_f32(x[row * cols + c]) - mu) * rs;
    dx[row * cols + c] = from_f32<T>(rs * (g - m1 - xh * m2));
  }
}

// Any `cols`: dgamma/dbeta partials, one thread per column per row chunk.
template <typename T>
__global__ void __launch_bounds__(kThreads)
    ln_bwd_params_cols(float* __restrict__ part_g, float* __restrict__ part_b,
                       const T* __restrict__ dy, const T* __restrict__ x,
                       const float* __restrict__ mean, const float* __restrict__ rstd,
                       int64_t rows, int64_t cols, int64_t rows_per_block) {
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_block;
  const int64_t r1 = min(rows, r0 + rows_per_block);
  float g = 0.f, b = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const float d = to_f32(dy[r * cols + c]);
    g += d * (to_f32(x[r * cols + c]) - mean[r]) * rstd[r];
    b += d;
  }
  part_g[(int64_t)blockIdx.y * cols + c] = g;
  part_b[(int64_t)blockIdx.y * cols + c] = b;
}

// dgamma/dbeta = sum of the block partials [nparts, cols] in a fixed order,
// so the result is deterministic.  A block owns 16 columns; its 16 row groups
// (ty) each sum partials ty, ty+16, ... with 16 loads issued before their
// adds, then group sums are combined in LDS in group order.  With at most a
// few hundred partials this is one latency-bound pass over an L2-resident
// workspace.
constexpr int kSumCols = 16, kSumGroups = 16;

template <typename T>
__global__ void __launch_bounds__(kSumCols * kSumGroups)
    ln_bwd_params_sum(T* __restrict__ dgamma, T* __restrict__ dbeta, const float* __restrict__ part_g,
                      const float* __restrict__ part_b, int nparts, int64_t cols) {
  __shared__ float lg[kSumGroups][kSumCols + 1], lb[kSumGroups][kSumCols + 1];
  const int tx = threadIdx.x % kSumCols, ty = threadIdx.x / kSumCols;
  const int64_t c = (int64_t)blockIdx.x * kSumCols + tx;
  float g = 0.f, b = 0.f;
  if (c < cols) {
    // 16 partials of each kind in flight per thread (one round trip for the
    // usual 256 partials), added in partial order
    constexpr int U = 16;
    int q = ty;
    for (; q + (U - 1) * kSumGroups < nparts; q += U * kSumGroups) {
      float vg[U], vb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        vg[u] = part_g[(int64_t)(q + u * kSumGroups) * cols + c];
        vb[u] = part_b[(int64_t)(q + u * kSumGroups) * cols + c];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) g += vg[u], b += vb[u];
    }
    for (; q < nparts; q += kSumGroups) g += part_g[(int64_t)q * cols + c], b += part_b[(int64_t)q * cols + c];
  }
  lg[ty][tx] = g;
  lb[ty][tx] = b;
  __syncthreads();
  if (ty == 0 && c < cols) {
    float sg = 0.f, sb = 0.f;
#pragma unroll
    for (int y = 0; y < kSumGroups; ++y) sg += lg[y][tx], sb += lb[y][tx];
    if (dgamma) dgamma[c] = from_f32<T>(sg);
    if (dbeta) dbeta[c] = from_f32<T>(sb);
  }
}

inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int wave_nv(int64_t cols) {
  if (cols % 4 != 0 || cols > 2048) return 0;
  const int64_t v = (cols + 255) / 256;
  if (v <= 1) return 1;
  if (v <= 2) return 2;
  if (v <= 3) return 3;
  if (v <= 4) return 4;
  return 8;
}

// Backward rows per block: about 16 (four per wave), with at most
// kMaxBwdBlocks partials; the block count is then trimmed so that every block
// owns at least one row.
int64_t bwd_rows_per_block(int64_t rows) {
  static const char* forced = getenv("MI355X_LN_BWD_BLOCKS");  // tuning override: maximum block count
  const int64_t max_blocks = forced ? atoll(forced) : 256;
  int64_t b = (rows + 31) / 32;
  if (b > max_blocks) b = max_blocks;
  if (b > kMaxBwdBlocks) b = kMaxBwdBlocks;
  if (b < 1) b = 1;
  return rows > 0 ? (rows + b - 1) / b : 1;
}

int bwd_waves() {
  static const char* forced = getenv("MI355X_LN_BWD_WAVES");  // tuning override: 4 or 8
  return forced && atoi(forced) == 8 ? 8 : 4;
}

int bwd_blocks(int64_t rows) {
  const int64_t rpb = bwd_rows_per_block(rows);
  return rows > 0 ? (int)((rows + rpb - 1) / rpb) : 1;
}

template <typename T, typename TL>
int fwd_impl(T* y, TL* y_low, float* mean, float* rstd, const T* x, const T* g, const T* b, int64_t rows,
             int64_t cols, float eps, hipStream_t s) {
  const size_t al = 4 * sizeof(T);
  const int nv = (aligned(x, al) && aligned(y, al) && aligned(g, al) && aligned(b, al) &&
                  aligned(y_low, 4 * sizeof(TL))) ? wave_nv(cols) : 0;
  const unsigned grid = ceil_div(rows, kWaves);
  switch (nv) {
#define LN_FWD_CASE(V) \
    case V: ln_fwd_wave<T, TL, V><<<grid, kThreads, 0, s>>>(y, y_low, mean, rstd, x, g, b, rows, (int)cols, eps); break;
    LN_FWD_CASE(1)
    LN_FWD_CASE(2)
    LN_FWD_CASE(3)
    LN_FWD_CASE(4)
    LN_FWD_CASE(8)
#undef LN_FWD_CASE
    default: ln_fwd_block<T, TL><<<(unsigned)rows, kThreads, 0, s>>>(y, y_low, mean, rstd, x, g, b, rows, cols, eps);
  }
  return check_launch("mi355x_layer_norm_fwd");
}

template <typename T, typename TR, typename TL>
int fwd_add_impl(T* y, TL* y_low, float* mean, float* rstd, T* x_out, const T* a, const TR* r, const T* g,
                 const T* b, int64_t rows, int64_t cols, float eps, hipStream_t s) {
  const size_t al = 4 * sizeof(T);
  const int nv = (aligned(a, al) && aligned(x_out, al) && aligned(r, 4 * sizeof(TR)) && aligned(y, al) &&
                  aligned(g, al) && aligned(b, al) && aligned(y_low, 4 * sizeof(TL))) ? wave_nv(cols) : 0;
  const unsigned grid = ceil_div(rows, kWaves);
  switch (nv) {
#define LN_FWD_ADD_CASE(V)                                                                                \
    case V:                                                                                               \
      ln_fwd_add_wave<T, TR, TL, V><<<grid, kThreads, 0, s>>>(y, y_low, mean, rstd, x_out, a, r, g, b, rows, \
                                                               (int)cols, eps);                          \
      break;
    LN_FWD_ADD_CASE(1)
    LN_FWD_ADD_CASE(2)
    LN_FWD_ADD_CASE(3)
    LN_FWD_ADD_CASE(4)
    LN_FWD_ADD_CASE(8)
#undef LN_FWD_ADD_CASE
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_layer_norm_fwd_add: rows of %lld elements or unaligned operands",
                         (long long)cols);
  }
  return check_launch("mi355x_layer_norm_fwd_add");
}

template <typename T, typename W>
int rms_impl(T* y, float* rstd, const T* x, const W* w, int64_t rows, int64_t cols, float eps, float w_off,
             hipStream_t s) {
  const int nv = (aligned(x, 4 * sizeof(T)) && aligned(y, 4 * sizeof(T)) && aligned(w, 4 * sizeof(W))) ? wave_nv(cols) : 0;
  const unsigned grid = ceil_div(rows, kWaves);
  switch (nv) {
    case 1: rms_fwd_wave<T, W, 1><<<grid, kThreads, 0, s>>>(y, rstd, x, w, rows, (int)cols, eps, w_off); break;
    case 2: rms_fwd_wave<T, W, 2><<<grid, kThreads, 0, s>>>(y, rstd, x, w, rows, (int)cols, eps, w_off); break;
    case 3: rms_fwd_wave<T, W, 3><<<grid, kThreads, 0, s>>>(y, rstd, x, w, rows, (int)cols, eps, w_off); break;
    case 4: rms_fwd_wave<T, W, 4><<<grid, kThreads, 0, s>>>(y, rstd, x, w, rows, (int)cols, eps, w_off); break;
    case 8: rms_fwd_wave<T, W, 8><<<grid, kThreads, 0, s>>>(y, rstd, x, w, rows, (int)cols, eps, w_off); break;
    default: rms_fwd_block<T, W><<<(unsigned)rows, kThreads, 0, s>>>(y, rstd, x, w, rows, cols, eps, w_off);
  }
  return check_launch("mi355x_rms_norm_fwd");
}

template <typename T>
int rms_dispatch_w(void* y, float* rstd, const void* x, const void* w, int w_dtype, int64_t rows, int64_t cols,
                   float eps, float w_off, hipStream_t s) {
  if (!w || w_dtype == MI355X_F32)
    return rms_impl<T, float>((T*)y, rstd, (const T*)x, (const float*)w, rows, cols, eps, w_off, s);
  return rms_impl<T, T>((T*)y, rstd, (const T*)x, (const T*)w, rows, cols, eps, w_off, s);
}

template <typename T>
int bwd_impl(T* dx, T* dgamma, T* dbeta, const T* dy, const T* x, const float* mean,
             const float* rstd, const T* gamma, int64_t rows, int64_t cols, float* ws,
             hipStream_t s) {
  const bool params = dgamma || dbeta;
  const int nb = bwd_blocks(rows);
  const int64_t rpb = bwd_rows_per_block(rows);
  float* pg = params ? ws : nullptr;
  float* pb = params ? ws + (int64_t)nb * cols : nullptr;
  const size_t al = 4 * sizeof(T);
  const int nv = (aligned(dx, al) && aligned(dy, al) && aligned(x, al) && aligned(gamma, al)) ? wave_nv(cols) : 0;
  if (nv) {
    if (!dx && !params) return MI355X_OK;
    switch (nv) {
#define LN_BWD_CASE(V)                                                                          \
  case V:                                                                                       \
    if (bwd_waves() == 8)                                                                       \
      ln_bwd_wave<T, V, 8><<<nb, 512, 0, s>>>(dx, pg, pb, dy, x, mean, rstd, gamma, rows,       \
                                              (int)cols, rpb);                                  \
    else                                                                                        \
      ln_bwd_wave<T, V, 4><<<nb, 256, 0, s>>>(dx, pg, pb, dy, x, mean, rstd, gamma, rows,       \
                                              (int)cols, rpb);                                  \
    break;
      LN_BWD_CASE(1)
      LN_BWD_CASE(2)
      LN_BWD_CASE(3)
      LN_BWD_CASE(4)
      LN_BWD_CASE(8)
#undef LN_BWD_CASE
    }
  } else {
    if (dx) ln_bwd_dx_block<T><<<(unsigned)rows, kThreads, 0, s>>>(dx, dy, x, mean, rstd, gamma, cols);
    if (params) {
      dim3 grid(ceil_div(cols, kThreads), nb);
      ln_bwd_params_cols<T><<<grid, kThreads, 0, s>>>(pg, pb, dy, x, mean, rstd, rows, cols, rpb);
    }
  }
  if (params) {
    ln_bwd_params_sum<T><<<ceil_div(cols, kSumCols), kSumCols * kSumGroups, 0, s>>>(dgamma, dbeta, pg, pb,
                                                                                   nb, cols);
  }
  return check_launch("mi355x_layer_norm_bwd");
}

// rms_norm backward: the LayerNorm wave kernel without the mean terms, the
// weight gradient summed from the same block partials.
template <typename T>
int rms_bwd_impl(T* dx, T* dw, const T* dy, const T* x, const float* rstd, const T* w, float w_off, int64_t rows,
                 int64_t cols, float* ws, hipStream_t s) {
  const size_t al = 4 * sizeof(T);
  const int nv = (aligned(dx, al) && aligned(dy, al) && aligned(x, al) && aligned(w, al)) ? wave_nv(cols) : 0;
  if (!nv)
    return fail(MI355X_EUNSUPPORTED, "mi355x_rms_norm_bwd: needs 4-element aligned rows of at most 2048 (got %lld)",
                (long long)cols);
  const int nb = bwd_blocks(rows);
  const int64_t rpb = bwd_rows_per_block(rows);
  float* pg = dw ? ws : nullptr;
  float* pb = dw ? ws + (int64_t)nb * cols : nullptr;
  switch (nv) {
#define RMS_BWD_CASE(V)                                                                                      \
  case V:                                                                                                    \
    ln_bwd_wave<T, V, 4, true><<<nb, 256, 0, s>>>(dx, pg, pb, dy, x, nullptr, rstd, w, rows, (int)cols, rpb,  \
                                                  w_off);                                                    \
    break;
    RMS_BWD_CASE(1)
    RMS_BWD_CASE(2)
    RMS_BWD_CASE(3)
    RMS_BWD_CASE(4)
    RMS_BWD_CASE(8)
#undef RMS_BWD_CASE
  }
  if (dw) ln_bwd_params_sum<T><<<ceil_div(cols, kSumCols), kSumCols * kSumGroups, 0, s>>>(dw, nullptr, pg, pb, nb, cols);
  return check_launch("mi355x_rms_norm_bwd");
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi355x_rms_norm_bwd(void* dx, void* dweight, const void* dy, const void* x, const float* rstd,
                                   const void* weight, double weight_offset, int64_t rows, int64_t cols, int dtype,
                                   void* workspace, int64_t ws_bytes, mi355x_stream_t stream) {
  MI_REQUIRE(rows >= 0 && cols > 0, "mi355x_rms_norm_bwd: bad shape [%lld, %lld]", (long long)rows, (long long)cols);
  MI_REQUIRE(dx && dy && x && rstd, "mi355x_rms_norm_bwd: null pointer");
  MI_REQUIRE(weight || !dweight, "mi355x_rms_norm_bwd: a weight gradient needs the weight");
  hipStream_t s = (hipStream_t)stream;
  if (rows == 0) {
    if (!dweight) return MI355X_OK;
    const int64_t shape[1] = {cols}, strides[1] = {1};
    return mi355x_fill(dweight, dtype, strides, shape, 1, 0.0, stream);
  }
  if (dweight) {
    const int64_t need = mi355x_layer_norm_bwd_workspace_bytes(rows, cols);
    if (!workspace || ws_bytes < need)
      return fail(MI355X_EWORKSPACE, "mi355x_rms_norm_bwd: workspace %lld < %lld bytes", (long long)ws_bytes,
                  (long long)need);
  }
  switch (dtype) {
    case MI355X_F32:
      return rms_bwd_impl<float>((float*)dx, (float*)dweight, (const float*)dy, (const float*)x, rstd,
                                 (const float*)weight, (float)weight_offset, rows, cols, (float*)workspace, s);
    case MI355X_BF16:
      return rms_bwd_impl<bf16>((bf16*)dx, (bf16*)dweight, (const bf16*)dy, (const bf16*)x, rstd,
                                (const bf16*)weight, (float)weight_offset, rows, cols, (float*)workspace, s);
    case MI355X_F16:
      return rms_bwd_impl<f16>((f16*)dx, (f16*)dweight, (const f16*)dy, (const f16*)x, rstd, (const f16*)weight,
                               (float)weight_offset, rows, cols, (float*)workspace, s);
  }
  return fail(MI355X_EUNSUPPORTED, "mi355x_rms_norm_bwd: unsupported dtype %d", dtype);
}

extern "C" int mi355x_layer_norm_fwd_ex(void* y, void* y_low, int low_dtype, float* mean, float* rstd,
                                        const void* x, const void* gamma, const void* beta, int64_t rows,
                                        int64_t cols, double eps, int dtype, mi355x_stream_t stream) {
  MI_REQUIRE(rows >= 0 && cols > 0, "mi355x_layer_norm_fwd: bad shape [%lld, %lld]",
             (long long)rows, (long long)cols);
  if (rows == 0) return MI355X_OK;
  MI_REQUIRE(x && (y || y_low), "mi355x_layer_norm_fwd: null pointer");
  MI_REQUIRE(!y_low || (dtype == MI355X_F32 && (low_dtype == MI355X_BF16 || low_dtype == MI355X_F16)),
             "mi355x_layer_norm_fwd: the low-precision copy needs f32 input and a bf16/f16 copy");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MI355X_F32:
      if (y_low && low_dtype == MI355X_F16)
        return fwd_impl<float, f16>((float*)y, (f16*)y_low, mean, rstd, (const float*)x, (const float*)gamma,
                                    (const float*)beta, rows, cols, (float)eps, s);
      return fwd_impl<float, bf16>((float*)y, (bf16*)y_low, mean, rstd, (const float*)x, (const float*)gamma,
                                   (const float*)beta, rows, cols, (float)eps, s);
    case MI355X_BF16:
      return fwd_impl<bf16, bf16>((bf16*)y, nullptr, mean, rstd, (const bf16*)x, (const bf16*)gamma,
                                  (const bf16*)beta, rows, cols, (float)eps, s);
    case MI355X_F16:
      return fwd_impl<f16, f16>((f16*)y, nullptr, mean, rstd, (const f16*)x, (const f16*)gamma,
                                (const f16*)beta, rows, cols, (float)eps, s);
  }
  return fail(MI355X_EUNSUPPORTED, "mi355x_layer_norm_fwd: unsupported dtype %d", dtype);
}

extern "C" int mi355x_layer_norm_fwd_add(void* y, void* y_low, int low_dtype, float* mean, float* rstd,
                                         void* x_out, const void* a, const void* r, int r_dtype,
                                         const void* gamma, const void* beta, int64_t rows, int64_t cols,
                                         double eps, int dtype, mi355x_stream_t stream) {
  MI_REQUIRE(rows >= 0 && cols > 0, "mi355x_layer_norm_fwd_add: bad shape [%lld, %lld]", (long long)rows,
             (long long)cols);
  if (rows == 0) return MI355X_OK;
  MI_REQUIRE((y || y_low) && x_out && a && r, "mi355x_layer_norm_fwd_add: null pointer");
  MI_REQUIRE(dtype == MI355X_F32, "mi355x_layer_norm_fwd_add: f32 rows only (got dtype %d)", dtype);
  MI_REQUIRE(r_dtype == MI355X_F32 || r_dtype == MI355X_BF16 || r_dtype == MI355X_F16,
             "mi355x_layer_norm_fwd_add: unsupported residual dtype %d", r_dtype);
  MI_REQUIRE(!y_low || low_dtype == MI355X_BF16 || low_dtype == MI355X_F16,
             "mi355x_layer_norm_fwd_add: the low-precision copy must be bf16 or f16");
  hipStream_t s = (hipStream_t)stream;
  const float e = (float)eps;
  float* Y = (float*)y;
  float* X = (float*)x_out;
  const float* A = (const float*)a;
  const float* G = (const float*)gamma;
  const float* B = (const float*)beta;
#define LN_ADD(TR)                                                                                           \
  do {                                                                                                      \
    if (y_low && low_dtype == MI355X_F16)                                                                   \
      return fwd_add_impl<float, TR, f16>(Y, (f16*)y_low, mean, rstd, X, A, (const TR*)r, G, B, rows, cols, e, s); \
    return fwd_add_impl<float, TR, bf16>(Y, (bf16*)y_low, mean, rstd, X, A, (const TR*)r, G, B, rows, cols, e, s); \
  } while (0)
  if (r_dtype == MI355X_BF16) LN_ADD(bf16);
  if (r_dtype == MI355X_F16) LN_ADD(f16);
  LN_ADD(float);
#undef LN_ADD
}

extern "C" int mi355x_layer_norm_fwd(void* y, float* mean, float* rstd, const void* x,
                                     const void* gamma, const void* beta, int64_t rows,
                                     int64_t cols, double eps, int dtype, mi355x_stream_t stream) {
  return mi355x_layer_norm_fwd_ex(y, nullptr, 0, mean, rstd, x, gamma, beta, rows, cols, eps, dtype, stream);
}

extern "C" int mi355x_layer_norm_apply(void* y, const void* x, const float* mean, const float* rstd,
                                       const void* gamma, const void* beta, int64_t rows, int64_t cols,
                                       int dtype, mi355x_stream_t stream) {
  MI_REQUIRE(rows >= 0 && cols > 0, "mi355x_layer_norm_apply: bad shape [%lld, %lld]", (long long)rows,
             (long long)cols);
  if (rows == 0) return MI355X_OK;
  MI_REQUIRE(y && x && mean && rstd, "mi355x_layer_norm_apply: null pointer");
  hipStream_t s = (hipStream_t)stream;
  auto go = [&](auto tag) {
    using T = decltype(tag);
    const size_t al = 4 * sizeof(T);
    const bool v4 = cols % 4 == 0 && aligned(x, al) && aligned(y, al) && aligned(gamma, al) && aligned(beta, al);
    const int64_t n = v4 ? rows * cols / 4 : rows * cols;
    const unsigned grid = (unsigned)(n / kThreads + 1 < 65536 ? n / kThreads + 1 : 65536);
    if (v4)
      ln_apply<T, true><<<grid, kThreads, 0, s>>>((T*)y, (const T*)x, mean, rstd, (const T*)gamma,
                                                   (const T*)beta, rows, cols);
    else
      ln_apply<T, false><<<grid, kThreads, 0, s>>>((T*)y, (const T*)x, mean, rstd, (const T*)gamma,
                                                    (const T*)beta, rows, cols);
  };
  switch (dtype) {
    case MI355X_F32: go(float{}); break;
    case MI355X_BF16: go(bf16{}); break;
    case MI355X_F16: go(f16{}); break;
    default: return fail(MI355X_EUNSUPPORTED, "mi355x_layer_norm_apply: unsupported dtype %d", dtype);
  }
  return check_launch("mi355x_layer_norm_apply");
}

extern "C" int64_t mi355x_layer_norm_bwd_workspace_bytes(int64_t rows, int64_t cols) {
  return 2 * (int64_t)bwd_blocks(rows) * cols * (int64_t)sizeof(float);
}

extern "C" int mi355x_layer_norm_bwd(void* dx, void* dgamma, void* dbeta, const void* dy,
                                     const void* x, const float* mean, const float* rstd,
                                     const void* gamma, int64_t rows, int64_t cols, int dtype,
                                     void* workspace, int64_t ws_bytes, mi355x_stream_t stream) {
  MI_REQUIRE(rows >= 0 && cols > 0, "mi355x_layer_norm_bwd: bad shape");
  hipStream_t s = (hipStream_t)stream;
  if (rows == 0) {
    // Empty batch: parameter gradients are zero.
    const int64_t shape[1] = {cols}, strides[1] = {1};
    if (dgamma) { int rc = mi355x_fill(dgamma, dtype, strides, shape, 1, 0.0, stream); if (rc) return rc; }
    if (dbeta) { int rc = mi355x_fill(dbeta, dtype, strides, shape, 1, 0.0, stream); if (rc) return rc; }
    return MI355X_OK;
  }
  if (dgamma || dbeta) {
    const int64_t need = mi355x_layer_norm_bwd_workspace_bytes(rows, cols);
    if (!workspace || ws_bytes < need)
      return fail(MI355X_EWORKSPACE, "mi355x_layer_norm_bwd: workspace %lld < %lld bytes",
                  (long long)ws_bytes, (long long)need);
  }
  switch (dtype) {
    case MI355X_F32:
      return bwd_impl<float>((float*)dx, (float*)dgamma, (float*)dbeta, (const float*)dy,
                             (const float*)x, mean, rstd, (const float*)gamma, rows, cols,
                             (float*)workspace, s);
    case MI355X_BF16:
      return bwd_impl<bf16>((bf16*)dx, (bf16*)dgamma, (bf16*)dbeta, (const bf16*)dy,
                            (const bf16*)x, mean, rstd, (const bf16*)gamma, rows, cols,
                            (float*)workspace, s);
    case MI355X_F16:
      return bwd_impl<f16>((f16*)dx, (f16*)dgamma, (f16*)dbeta, (const f16*)dy, (const f16*)x,
                           mean, rstd, (const f16*)gamma, rows, cols, (float*)workspace, s);
  }
  return fail(MI355X_EUNSUPPORTED, "mi355x_layer_norm_bwd: unsupported dtype %d", dtype);
}

extern "C" int mi355x_rms_norm_fwd(void* y, float* rstd, const void* x, const void* weight, int weight_dtype,
                                   double weight_offset, int64_t rows, int64_t cols, double eps, int dtype,
                                   mi355x_stream_t stream) {
  MI_REQUIRE(rows >= 0 && cols > 0, "mi355x_rms_norm_fwd: bad shape [%lld, %lld]", (long long)rows, (long long)cols);
  if (rows == 0) return MI355X_OK;
  MI_REQUIRE(y && x, "mi355x_rms_norm_fwd: null pointer");
  MI_REQUIRE(!weight || weight_dtype == MI355X_F32 || weight_dtype == dtype,
             "mi355x_rms_norm_fwd: weight dtype must be f32 or the input dtype");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MI355X_F32: return rms_dispatch_w<float>(y, rstd, x, weight, weight_dtype, rows, cols, (float)eps, (float)weight_offset, s);
    case MI355X_BF16: return rms_dispatch_w<bf16>(y, rstd, x, weight, weight_dtype, rows, cols, (float)eps, (float)weight_offset, s);
    case MI355X_F16: return rms_dispatch_w<f16>(y, rstd, x, weight, weight_dtype, rows, cols, (float)eps, (float)weight_offset, s);
  }
  return fail(MI355X_EUNSUPPORTED, "mi355x_rms_norm_fwd: unsupported dtype %d", dtype);
}
