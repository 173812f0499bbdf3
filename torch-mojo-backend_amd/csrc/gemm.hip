// GEMM: C[b] = A[b] * B[b] (+ bias row) (+ C if beta), f32 accumulation.
//
// bf16/f16 inputs run on MFMA (v_mfma_f32_16x16x32_*).  A 256-thread block
// (4 waves, 2x2) owns a 128x128 C tile; each wave a 64x64 sub-tile made of
// 4x4 MFMA tiles (64 f32 accumulators per lane).  K advances 32 at a time
// through LDS tiles stored K-contiguous ([row][k], rows padded to 80 bytes
// so the 16-byte fragment reads of 8 consecutive rows hit distinct banks).
//
// Both operand layouts of the three training GEMMs are read in place:
//   fwd  x*W^T : A k-contiguous, B k-contiguous (W rows)
//   dX   dY*W  : A k-contiguous, B n-contiguous
//   dW   dY^T*X: A m-contiguous, B n-contiguous
// A k-contiguous operand is copied to LDS with 16-byte global loads and
// 16-byte LDS stores; an m/n-contiguous one is loaded 16 bytes (8 rows of
// one k) at a time and scattered into the k-contiguous LDS layout.  The next
// K tile's global loads are issued before the current tile's MFMAs, so
// memory latency overlaps the matrix work.
//
// f32 inputs use a plain 64x64 register-tiled FMA kernel (the f32 model path
// without autocast).
#include "common.h"
#include "mfma.h"

namespace mi {
namespace {

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDS_STRIDE = BK + 8;  // elements per LDS row (80 bytes)
constexpr int kThreads = 256;

struct GemmArgs {
  void* c;
  int c_dt;
  int64_t c_rs, c_bs;
  const void* a;
  int64_t a_rs, a_cs, a_bs;
  const void* b;
  int64_t b_rs, b_cs, b_bs;
  const void* bias;
  int bias_dt;
  int beta;
  int64_t m, n, k;
  int vec_a, vec_b;  // 16-byte global loads allowed
};

template <typename T>
struct alignas(16) V8 {
  T v[8];
};

__device__ __forceinline__ float ld_any(const void* p, int dt, int64_t i) {
  switch (dt) {
    case MI355X_F32: return ((const float*)p)[i];
    case MI355X_BF16: return (float)((const bf16*)p)[i];
    default: return (float)((const f16*)p)[i];
  }
}
__device__ __forceinline__ void st_any(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case MI355X_F32: ((float*)p)[i] = v; break;
    case MI355X_BF16: ((bf16*)p)[i] = (bf16)v; break;
    default: ((f16*)p)[i] = (f16)v; break;
  }
}

// Global -> registers for one operand tile of ROWS x BK.
// K_CONTIG: element (row, k) at base + row*rs + k.  Else at base + row + k*ks.
template <typename T, bool K_CONTIG>
struct TileLoader {
  // Each thread moves 2 chunks of 8 elements.
  V8<T> buf[2];

  __device__ __forceinline__ void load(const T* base, int64_t rs_or_ks, int64_t row0, int64_t rows,
                                       int64_t k0, int64_t kdim, bool vec) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int chunk = threadIdx.x + c * kThreads;
      if (K_CONTIG) {
        const int r = chunk >> 2, kc = (chunk & 3) * 8;
        const int64_t gr = row0 + r, gk = k0 + kc;
        const T* p = base + gr * rs_or_ks + gk;
        if (vec && gr < rows && gk + 8 <= kdim) {
          buf[c] = *(const V8<T>*)p;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            buf[c].v[e] = (gr < rows && gk + e < kdim) ? p[e] : (T)0.f;
        }
      } else {
        const int kk = chunk >> 4, rc = (chunk & 15) * 8;
        const int64_t gr = row0 + rc, gk = k0 + kk;
        const T* p = base + gk * rs_or_ks + gr;
        if (vec && gk < kdim && gr + 8 <= rows) {
          buf[c] = *(const V8<T>*)p;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            buf[c].v[e] = (gk < kdim && gr + e < rows) ? p[e] : (T)0.f;
        }
      }
    }
  }

  __device__ __forceinline__ void store(T* lds) const {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int chunk = threadIdx.x + c * kThreads;
      if (K_CONTIG) {
        const int r = chunk >> 2, kc = (chunk & 3) * 8;
        *(V8<T>*)(lds + r * LDS_STRIDE + kc) = buf[c];
      } else {
        const int kk = chunk >> 4, rc = (chunk & 15) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) lds[(rc + e) * LDS_STRIDE + kk] = buf[c].v[e];
      }
    }
  }
};

template <typename T, bool A_K, bool B_K>
__global__ void __launch_bounds__(kThreads) gemm_mfma(GemmArgs g) {
  typedef typename Mfma<T>::frag frag;
  __shared__ __attribute__((aligned(16))) T As[BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) T Bs[BN * LDS_STRIDE];

  const int64_t batch = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const T* A = (const T*)g.a + batch * g.a_bs;
  const T* B = (const T*)g.b + batch * g.b_bs;
  const int64_t a_ld = A_K ? g.a_rs : g.a_cs;  // stride between rows (A_K) or between k (else)
  const int64_t b_ld = B_K ? g.b_cs : g.b_rs;  // B viewed as [n][k]: row stride (B_K) or k stride

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 15, lg = lane >> 4;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  TileLoader<T, A_K> la;
  TileLoader<T, B_K> lb;
  la.load(A, a_ld, m0, g.m, 0, g.k, g.vec_a);
  lb.load(B, b_ld, n0, g.n, 0, g.k, g.vec_b);

  for (int64_t k0 = 0; k0 < g.k; k0 += BK) {
    __syncthreads();
    la.store(As);
    lb.store(Bs);
    __syncthreads();
    if (k0 + BK < g.k) {
      la.load(A, a_ld, m0, g.m, k0 + BK, g.k, g.vec_a);
      lb.load(B, b_ld, n0, g.n, k0 + BK, g.k, g.vec_b);
    }
    frag af[4], bfr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[i] = *(const frag*)(As + (wm * 64 + i * 16 + lr) * LDS_STRIDE + lg * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bfr[j] = *(const frag*)(Bs + (wn * 64 + j * 16 + lr) * LDS_STRIDE + lg * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = Mfma<T>::mma(af[i], bfr[j], acc[i][j]);
  }

  // epilogue: lane holds C[4*lg + e][lr] of each 16x16 tile
  char* C = (char*)g.c;
  const int64_t c_es = g.c_dt == MI355X_F32 ? 4 : 2;
  void* Cb = C + batch * g.c_bs * c_es;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t col = n0 + wn * 64 + j * 16 + lr;
    if (col >= g.n) continue;
    const float bias = g.bias ? ld_any(g.bias, g.bias_dt, col) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = m0 + wm * 64 + i * 16 + lg * 4 + e;
        if (row < g.m) {
          const int64_t off = row * g.c_rs + col;
          float v = acc[i][j][e] + bias;
          if (g.beta) v += ld_any(Cb, g.c_dt, off);
          st_any(Cb, g.c_dt, off, v);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// f32: 64x64 tile, 256 threads, 4x4 outputs per thread.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) gemm_f32(GemmArgs g) {
  __shared__ float As[16][64 + 4];
  __shared__ float Bs[16][64 + 4];
  const int64_t batch = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  const float* A = (const float*)g.a + batch * g.a_bs;
  const float* B = (const float*)g.b + batch * g.b_bs;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < g.k; k0 += 16) {
    for (int e = threadIdx.x; e < 16 * 64; e += 256) {
      const int kk = e / 64, r = e % 64;
      const int64_t gm = m0 + r, gk = k0 + kk, gn = n0 + r;
      As[kk][r] = (gm < g.m && gk < g.k) ? A[gm * g.a_rs + gk * g.a_cs] : 0.f;
      Bs[kk][r] = (gn < g.n && gk < g.k) ? B[gk * g.b_rs + gn * g.b_cs] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i], b[i] = Bs[kk][tx * 4 + i];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
  void* Cb = (char*)g.c + batch * g.c_bs * (g.c_dt == MI355X_F32 ? 4 : 2);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = m0 + ty * 4 + i;
    if (row >= g.m) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + tx * 4 + j;
      if (col >= g.n) continue;
      float v = acc[i][j] + (g.bias ? ld_any(g.bias, g.bias_dt, col) : 0.f);
      const int64_t off = row * g.c_rs + col;
      if (g.beta) v += ld_any(Cb, g.c_dt, off);
      st_any(Cb, g.c_dt, off, v);
    }
  }
}

template <typename T>
int launch_mfma(const GemmArgs& g, int64_t batch, hipStream_t s) {
  dim3 grid(ceil_div(g.n, BN), ceil_div(g.m, BM), (unsigned)batch);
  const bool ak = g.a_cs == 1, bk = g.b_rs == 1;
  if (ak && bk) gemm_mfma<T, true, true><<<grid, kThreads, 0, s>>>(g);
  else if (ak && !bk) gemm_mfma<T, true, false><<<grid, kThreads, 0, s>>>(g);
  else if (!ak && bk) gemm_mfma<T, false, true><<<grid, kThreads, 0, s>>>(g);
  else gemm_mfma<T, false, false><<<grid, kThreads, 0, s>>>(g);
  return check_launch("mi355x_gemm");
}

bool fdt(int d) { return d == MI355X_F32 || d == MI355X_BF16 || d == MI355X_F16; }

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int64_t mi355x_gemm_workspace_bytes(int64_t batch, int64_t m, int64_t n, int64_t k,
                                               int ab_dtype) {
  (void)batch; (void)m; (void)n; (void)k; (void)ab_dtype;
  return 0;
}

extern "C" int mi355x_gemm(void* c, int c_dtype, int64_t c_rs, int64_t c_bs, const void* a,
                           int64_t a_rs, int64_t a_cs, int64_t a_bs, const void* b, int64_t b_rs,
                           int64_t b_cs, int64_t b_bs, int ab_dtype, const void* bias,
                           int bias_dtype, int beta, int64_t batch, int64_t m, int64_t n,
                           int64_t k, void* workspace, int64_t ws_bytes, mi355x_stream_t stream) {
  (void)workspace; (void)ws_bytes;
  MI_REQUIRE(fdt(ab_dtype) && fdt(c_dtype), "mi355x_gemm: unsupported dtype");
  MI_REQUIRE(!bias || fdt(bias_dtype), "mi355x_gemm: unsupported bias dtype");
  MI_REQUIRE(batch >= 1 && m >= 0 && n >= 0 && k >= 0, "mi355x_gemm: bad shape");
  MI_REQUIRE(batch < 65536 && m < (1ll << 31) && n < (1ll << 31), "mi355x_gemm: shape too large");
  if (m == 0 || n == 0) return MI355X_OK;
  MI_REQUIRE(k > 0, "mi355x_gemm: k == 0 must be handled by the caller");
  MI_REQUIRE(a_rs == 1 || a_cs == 1, "mi355x_gemm: A needs a unit row or column stride");
  MI_REQUIRE(b_rs == 1 || b_cs == 1, "mi355x_gemm: B needs a unit row or column stride");
  MI_REQUIRE(c && a && b, "mi355x_gemm: null pointer");
  hipStream_t s = (hipStream_t)stream;
  GemmArgs g{c, c_dtype, c_rs, c_bs, a, a_rs, a_cs, a_bs, b, b_rs, b_cs, b_bs, bias, bias_dtype,
             beta, m, n, k, 0, 0};
  if (ab_dtype == MI355X_F32) {
    dim3 grid(ceil_div(n, 64), ceil_div(m, 64), (unsigned)batch);
    gemm_f32<<<grid, 256, 0, s>>>(g);
    return check_launch("mi355x_gemm");
  }
  // 16-byte global loads need 8-element aligned leading dims and bases.
  auto ok16 = [](const void* p, int64_t ld, int64_t bs) {
    return ((uintptr_t)p % 16 == 0) && (ld % 8 == 0) && (bs % 8 == 0);
  };
  g.vec_a = ok16(a, a_cs == 1 ? a_rs : a_cs, a_bs);
  g.vec_b = ok16(b, b_rs == 1 ? b_cs : b_rs, b_bs);
  if (ab_dtype == MI355X_BF16) return launch_mfma<bf16>(g, batch, s);
  return launch_mfma<f16>(g, batch, s);
}
