// GEMM: C[b] = A[b] * B[b] (+ bias row) (+ C if beta), f32 accumulation.
//
// bf16/f16 inputs run on MFMA (v_mfma_f32_16x16x32_*).  A 256-thread block
// (4 waves, 2x2) owns a BM x BN tile of C; each wave a (BM/2) x (BN/2)
// sub-tile of 16x16 MFMA tiles.  The largest configuration (256x256, 128x128
// per wave, 256 f32 accumulators per lane) reads 64 A and 64 B elements per
// 64x64x... MFMA set, i.e. 64 flop per LDS byte, enough to keep the matrix
// cores ahead of LDS bandwidth; smaller tiles are used when they fill the
// 256 CUs better.
//
// K advances 64 at a time.  LDS holds each operand tile k-contiguous
// ([row][64], rows padded to 144 bytes so the 16-byte fragment reads of 16
// consecutive rows hit distinct banks).  Tiles are double-buffered: the
// next K tile's global loads are issued into registers before the current
// tile's MFMAs and written to the other LDS buffer after them, one barrier
// per K step.
//
// Both operand layouts of the three training GEMMs are read in place:
//   fwd  x*W^T : A k-contiguous, B k-contiguous (W rows)
//   dX   dY*W  : A k-contiguous, B n-contiguous
//   dW   dY^T*X: A m-contiguous, B n-contiguous
// A k-contiguous tile is copied with 16-byte loads/stores.  An m/n-contiguous
// one is loaded as 8x8 element blocks (eight 16-byte rows of 8 m at 8 k),
// transposed in registers with byte permutes and stored as eight 16-byte
// k-contiguous rows.
//
// Weight-gradient shapes have a small C (e.g. 768x768) and a long K (the
// token count); they are split along K into partial f32 tiles in a caller
// workspace, summed (with bias/beta and the output cast) by a second pass.
//
// f32 inputs use a plain 64x64 register-tiled FMA kernel.
#include <stdio.h>
#include <stdlib.h>

#include "common.h"
#include "mfma.h"

extern __shared__ __attribute__((aligned(16))) char gemm_smem[];

namespace mi {
namespace {

constexpr int BK = 64;
constexpr int LDS_ROW = BK + 8;  // elements (144 bytes)
constexpr int kThreads = 256;
constexpr int kCUs = 256;

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
  float* part;       // split-K partials [splits][batch][m][n] (f32) or null
  int64_t kchunk;    // K per split
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

// KPT x 8 -> 8 x KPT transpose of 16-bit values: in[i] holds 8 values of
// k-row i (4 dwords); out[m] receives the KPT values of column m (KPT/2
// dwords, low dword first).
template <int KPT>
__device__ __forceinline__ void transpose_k8(const uint4* in, uint32_t (&out)[8][KPT / 2]) {
  uint32_t w[KPT][4];
#pragma unroll
  for (int i = 0; i < KPT; ++i) w[i][0] = in[i].x, w[i][1] = in[i].y, w[i][2] = in[i].z, w[i][3] = in[i].w;
#pragma unroll
  for (int m = 0; m < 8; ++m)
#pragma unroll
    for (int j = 0; j < KPT / 2; ++j)
      out[m][j] = __builtin_amdgcn_perm(w[2 * j + 1][m >> 1], w[2 * j][m >> 1],
                                        (m & 1) ? 0x07060302u : 0x05040100u);
}

// Global -> registers -> LDS for one ROWS x BK operand tile.
// K_CONTIG: element (row, k) at base + row*ld + k; else at base + row + k*ld.
template <typename T, int ROWS, bool K_CONTIG, int NT>
struct Stage {
  static constexpr int CHUNKS = ROWS * BK / 8;      // 16-byte chunks
  static constexpr int PER_THREAD = CHUNKS / NT;
  static_assert(PER_THREAD == 8 || PER_THREAD == 4 || PER_THREAD == 2, "tile/thread mismatch");
  static_assert(K_CONTIG || (ROWS / 8) * (BK / PER_THREAD) == NT, "transposed staging map");
  uint4 r[PER_THREAD];

  __device__ __forceinline__ void load(const T* base, int64_t ld, int64_t row0, int64_t rows,
                                       int64_t k0, int64_t kend, bool vec) {
    if (K_CONTIG) {
#pragma unroll
      for (int c = 0; c < PER_THREAD; ++c) {
        const int chunk = threadIdx.x + c * NT;
        const int rr = chunk >> 3, kc = (chunk & 7) * 8;
        const int64_t gr = row0 + rr, gk = k0 + kc;
        const T* p = base + gr * ld + gk;
        if (vec && gr < rows && gk + 8 <= kend) {
          r[c] = *(const uint4*)p;
        } else {
          V8<T> v;
#pragma unroll
          for (int e = 0; e < 8; ++e) v.v[e] = (gr < rows && gk + e < kend) ? p[e] : (T)0.f;
          r[c] = *(uint4*)&v;
        }
      }
    } else {
      // a (KPT k) x (8 rows) block per thread; k groups vary fastest so a
      // wave's LDS stores cover whole 128-byte row spans
      constexpr int KPT = PER_THREAD, KG = BK / KPT;
      const int kq = threadIdx.x % KG, rb = threadIdx.x / KG;
      const int64_t gr = row0 + rb * 8;
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const int64_t gk = k0 + kq * KPT + i;
        const T* p = base + gk * ld + gr;
        if (vec && gk < kend && gr + 8 <= rows) {
          r[i] = *(const uint4*)p;
        } else {
          V8<T> v;
#pragma unroll
          for (int e = 0; e < 8; ++e) v.v[e] = (gk < kend && gr + e < rows) ? p[e] : (T)0.f;
          r[i] = *(uint4*)&v;
        }
      }
    }
  }

  __device__ __forceinline__ void store(T* lds) const {
    if (K_CONTIG) {
#pragma unroll
      for (int c = 0; c < PER_THREAD; ++c) {
        const int chunk = threadIdx.x + c * NT;
        const int rr = chunk >> 3, kc = (chunk & 7) * 8;
        *(uint4*)(lds + rr * LDS_ROW + kc) = r[c];
      }
    } else {
      constexpr int KPT = PER_THREAD, KG = BK / KPT;
      const int kq = threadIdx.x % KG, rb = threadIdx.x / KG;
      uint32_t t[8][KPT / 2];
      transpose_k8<KPT>(r, t);
#pragma unroll
      for (int mrow = 0; mrow < 8; ++mrow) {
        T* dst = lds + (rb * 8 + mrow) * LDS_ROW + kq * KPT;
        if constexpr (KPT == 8) *(uint4*)dst = make_uint4(t[mrow][0], t[mrow][1], t[mrow][2], t[mrow][3]);
        else if constexpr (KPT == 4) *(uint2*)dst = make_uint2(t[mrow][0], t[mrow][1]);
        else *(uint32_t*)dst = t[mrow][0];
      }
    }
  }
};

template <typename T, int BM, int BN, bool A_K, bool B_K>
__global__ void __launch_bounds__((BM / 64) * (BN / 64) * 64)
    gemm_mfma(GemmArgs g) {
  typedef typename Mfma<T>::frag frag;
  constexpr int WAVES_N = BN / 64;
  constexpr int NT = (BM / 64) * WAVES_N * 64;
  constexpr int WM = 64, WN = 64;  // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;
  // LDS: [A buf0][A buf1][B buf0][B buf1]; pointers are formed by offsets
  // from the __shared__ array so they stay in the LDS address space.
  T* const lds = reinterpret_cast<T*>(gemm_smem);

  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  // split-K: blockIdx.z = split * batch_count + batch
  int64_t bidx = blockIdx.z, split = 0, nb = gridDim.z;
  if (g.part) {
    const int64_t splits = (g.k + g.kchunk - 1) / g.kchunk;
    nb = gridDim.z / splits;
    split = blockIdx.z / nb;
    bidx = blockIdx.z % nb;
  }
  const int64_t kbeg = split * (g.part ? g.kchunk : g.k);
  const int64_t kend = g.part ? min(g.k, kbeg + g.kchunk) : g.k;
  const T* A = (const T*)g.a + bidx * g.a_bs;
  const T* B = (const T*)g.b + bidx * g.b_bs;
  const int64_t a_ld = A_K ? g.a_rs : g.a_cs;
  const int64_t b_ld = B_K ? g.b_cs : g.b_rs;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int lr = lane & 15, lg = lane >> 4;

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  Stage<T, BM, A_K, NT> sa;
  Stage<T, BN, B_K, NT> sb;
  sa.load(A, a_ld, m0, g.m, kbeg, kend, g.vec_a);
  sb.load(B, b_ld, n0, g.n, kbeg, kend, g.vec_b);
  sa.store(lds);
  sb.store(lds + 2 * BM * LDS_ROW);
  __syncthreads();

  int cur = 0;
  for (int64_t k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) {
      sa.load(A, a_ld, m0, g.m, k0 + BK, kend, g.vec_a);
      sb.load(B, b_ld, n0, g.n, k0 + BK, kend, g.vec_b);
    }
    const T* as = lds + cur * BM * LDS_ROW + (wm * WM + lr) * LDS_ROW + lg * 8;
    const T* bs = lds + 2 * BM * LDS_ROW + cur * BN * LDS_ROW + (wn * WN + lr) * LDS_ROW + lg * 8;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      frag af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *(const frag*)(as + i * 16 * LDS_ROW + ks * 32);
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[j] = *(const frag*)(bs + j * 16 * LDS_ROW + ks * 32);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::mma(af[i], bfr[j], acc[i][j]);
    }
    if (more) {
      sa.store(lds + (cur ^ 1) * BM * LDS_ROW);
      sb.store(lds + 2 * BM * LDS_ROW + (cur ^ 1) * BN * LDS_ROW);
    }
    __syncthreads();
    cur ^= 1;
  }

  // epilogue: lane holds C[4*lg + e][lr] of each 16x16 tile
  if (g.part) {
    float* P = g.part + (split * nb + bidx) * g.m * g.n;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn * WN + j * 16 + lr;
      if (col >= g.n) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t row = m0 + wm * WM + i * 16 + lg * 4 + e;
          if (row < g.m) P[row * g.n + col] = acc[i][j][e];
        }
    }
    return;
  }
  const int64_t c_es = g.c_dt == MI355X_F32 ? 4 : 2;
  void* Cb = (char*)g.c + bidx * g.c_bs * c_es;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = n0 + wn * WN + j * 16 + lr;
    if (col >= g.n) continue;
    const float bias = g.bias ? ld_any(g.bias, g.bias_dt, col) : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = m0 + wm * WM + i * 16 + lg * 4 + e;
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

// Sum split-K partials: C = sum_s part[s] (+bias) (+C).
__global__ void __launch_bounds__(256) splitk_reduce(GemmArgs g, int splits, int64_t nb) {
  const int64_t mn = g.m * g.n;
  const int64_t total = nb * mn;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int64_t bi = idx / mn, rem = idx % mn;
    const int64_t row = rem / g.n, col = rem % g.n;
    float v = 0.f;
    for (int s = 0; s < splits; ++s) v += g.part[(s * nb + bi) * mn + rem];
    if (g.bias) v += ld_any(g.bias, g.bias_dt, col);
    const int64_t c_es = g.c_dt == MI355X_F32 ? 4 : 2;
    void* Cb = (char*)g.c + bi * g.c_bs * c_es;
    const int64_t off = row * g.c_rs + col;
    if (g.beta) v += ld_any(Cb, g.c_dt, off);
    st_any(Cb, g.c_dt, off, v);
  }
}

// ---------------------------------------------------------------------------
// Fast path: A and B both k-contiguous, 16-byte aligned rows, K % 64 == 0.
//
// Operand tiles go global -> LDS directly (global_load_lds_dwordx4: each
// wave instruction fills 1 KB of LDS, lane i writing bytes [16i, 16i+16)),
// so no registers are spent on staging and the next K tile streams in while
// the current one feeds the MFMAs.  LDS rows are 128 bytes (64 k) with the
// 16-byte chunks XOR-swizzled by row: phys = k_chunk ^ ((row >> 1) & 7),
// which makes the 16 rows read by one fragment load land on 16 distinct
// 16-byte bank groups.  A lane's global address is chosen so that its fixed
// LDS slot receives the swizzled chunk.
// Blocks are ordered so consecutive tiles of one XCD share operand panels.
// ---------------------------------------------------------------------------
typedef const void __attribute__((address_space(1)))* gptr_t;
typedef void __attribute__((address_space(3)))* lptr_t;

// Direct loads of one ROWS x 64 tile into LDS.  Thread (wave w, lane l)
// handles rows r = 8*(it*WAVES + w) + l/8 for it = 0..; with WAVES even the
// swizzled chunk of its slot is the same for every `it`, so the per-thread
// source address is one base plus it * 8*WAVES rows.
template <int ROWS, int NT>
struct TileLoad {
  static constexpr int WAVES = NT / 64;
  static constexpr int ITERS = ROWS / (8 * WAVES);
  static_assert(WAVES % 2 == 0, "swizzle invariance needs an even wave count");
  const char* src;    // thread's source for it = 0 at k = 0 (its chunk included)
  int64_t row_step;   // bytes between it and it+1
  int64_t first_row;  // row of it = 0 (for clamping)
  int64_t ld;
  int chunk;          // 16-byte chunk of the 64-element k slab this lane loads

  __device__ __forceinline__ void init(const char* base, int64_t ld_bytes, int64_t row0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = wave * 8 + (lane >> 3);
    chunk = (lane & 7) ^ ((r >> 1) & 7);
    first_row = row0 + r;
    ld = ld_bytes;
    src = base + first_row * ld_bytes + chunk * 16;
    row_step = (int64_t)8 * WAVES * ld_bytes;
  }
  // k0_bytes: byte offset along k; dst: LDS tile; rows: valid row count;
  // kend_bytes: end of the valid k range (a chunk starting past it reloads
  // chunk 0: its values are masked out of the MFMAs, the address stays valid).
  // KT = false: K is a multiple of 64 and no clamp is needed.
  template <bool KT>
  __device__ __forceinline__ void issue(int64_t k0_bytes, char* dst, int64_t rows, bool full,
                                        int64_t kend_bytes) const {
    const int wave = threadIdx.x >> 6;
    const int64_t coff = (KT && k0_bytes + chunk * 16 >= kend_bytes) ? k0_bytes - chunk * 16 : k0_bytes;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const char* p = src + it * row_step + coff;
      if (!full) {
        const int64_t row = first_row + it * 8 * WAVES;
        if (row >= rows) p -= (row - (rows - 1)) * ld;
      }
      __builtin_amdgcn_global_load_lds((gptr_t)p, (lptr_t)(dst + (it * WAVES + wave) * 1024), 16, 0, 0);
    }
  }
};

// m/n-contiguous operand tile: 64 k-rows of ROWS elements, 16-byte chunks
// XOR-swizzled by s(k) = (k & 3) | ((k >> 1) & 12), a bijection on the 16
// k-rows one transposing fragment read touches.
__device__ __forceinline__ int kswz(int k) { return (k & 3) | ((k >> 1) & 12); }

template <int ROWS, int NT>
struct TileLoadT {
  static constexpr int ROWB = ROWS * 2;
  static constexpr int CPR = ROWS / 8;     // chunks per k-row
  static constexpr int KPI = 1024 / ROWB;  // k-rows per 1 KB instruction
  static constexpr int WAVES = NT / 64;
  static constexpr int ITERS = 64 / KPI / WAVES;
  const char* base;
  int64_t ld;  // bytes between k-rows
  int64_t row0, rows;
  int krow_l, phys;

  __device__ __forceinline__ void init(const char* b, int64_t ld_bytes, int64_t r0, int64_t nrows) {
    const int lane = threadIdx.x & 63;
    base = b;
    ld = ld_bytes;
    row0 = r0;
    rows = nrows;
    krow_l = lane / CPR;
    phys = lane % CPR;
  }
  // k-rows past kend reload row kend-1 (masked out of the MFMAs); a last
  // partial chunk of rows reads into the row padding (k stride >= rows
  // rounded up to 8, checked by the caller).
  template <bool KT>
  __device__ __forceinline__ void issue(int64_t k0, char* dst, bool full, int64_t kend) const {
    const int wave = threadIdx.x >> 6;
    const int64_t last_chunk = ((rows - 1) >> 3) << 3;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int blk = it * WAVES + wave;
      const int kr = blk * KPI + krow_l;
      const int chunk = phys ^ kswz(kr);
      int64_t m = row0 + chunk * 8;
      if (!full && m > last_chunk) m = last_chunk;
      int64_t k = k0 + kr;
      if (KT && k >= kend) k = kend - 1;
      const char* src = base + k * ld + m * 2;
      __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)(dst + blk * 1024), 16, 0, 0);
    }
  }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// MFMA fragment (rows r0..r0+15, k = ks*32 + 8g + 0..7) from an m/n-
// contiguous tile with two transposing reads: within a 16-lane group, lane i
// receives element i%4 of the 4-element pieces of lanes i/4, 4+i/4, 8+i/4,
// 12+i/4, so source lane 4e+q supplies k-row (.. + e), columns r0+4q..+3.
template <typename T, int ROWS>
__device__ __forceinline__ typename Mfma<T>::frag mn_frag(const char* tile, int r0, int ks) {
  constexpr int ROWB = ROWS * 2;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, src = lane & 15;
  const int m = r0 + 4 * (src & 3);
  const int k1 = ks * 32 + 8 * g + (src >> 2), k2 = k1 + 4;
  const int o1 = k1 * ROWB + (((m >> 3) ^ kswz(k1)) << 4) + ((m & 7) << 1);
  const int o2 = k2 * ROWB + (((m >> 3) ^ kswz(k2)) << 4) + ((m & 7) << 1);
  s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + o1));
  s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + o2));
  typename Mfma<T>::frag f;
  short* fs = (short*)&f;
#pragma unroll
  for (int e = 0; e < 4; ++e) fs[e] = a[e], fs[4 + e] = b[e];
  return f;
}

template <int ROWS, int NT, bool K_CONTIG>
struct OperandLoad;
template <int ROWS, int NT>
struct OperandLoad<ROWS, NT, true> {
  TileLoad<ROWS, NT> t;
  int64_t rows;
  __device__ __forceinline__ void init(const char* b, int64_t ld, int64_t r0, int64_t n) { t.init(b, ld, r0); rows = n; }
  template <bool KT>
  __device__ __forceinline__ void issue(int64_t k0_elems, char* dst, bool full, int64_t kend) const {
    t.template issue<KT>(k0_elems * 2, dst, rows, full, kend * 2);
  }
};
template <int ROWS, int NT>
struct OperandLoad<ROWS, NT, false> {
  TileLoadT<ROWS, NT> t;
  __device__ __forceinline__ void init(const char* b, int64_t ld, int64_t r0, int64_t n) { t.init(b, ld, r0, n); }
  template <bool KT>
  __device__ __forceinline__ void issue(int64_t k0_elems, char* dst, bool full, int64_t kend) const {
    t.template issue<KT>(k0_elems, dst, full, kend);
  }
};

// Zero the fragment slots whose k index (k0 + ks*32 + 8*g + slot) is >= kend.
template <typename F>
__device__ __forceinline__ void mask_k(F& f, int64_t kbase, int64_t kend) {
  short* fs = (short*)&f;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (kbase + e >= kend) fs[e] = 0;
}

// KT: K is not a multiple of 64, so the last k step clamps its loads and
// masks the fragments past K.
template <typename T, int BM, int BN, bool A_K, bool B_K, bool KT>
__global__ void __launch_bounds__(256, 1) gemm_nt_fast(GemmArgs g, int tiles_m, int tiles_n) {
  typedef typename Mfma<T>::frag frag;
  constexpr int NT = 256;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128, STAGE = A_BYTES + B_BYTES;
  char* const lds = gemm_smem;

  // XCD-aware tile order: hardware places block b on XCD b % 8.
  int64_t splits = 1, split = 0, bidx = 0;
  const int64_t per_batch = (int64_t)tiles_m * tiles_n;
  int64_t b = blockIdx.x;
  const int64_t nblocks = gridDim.x;
  if (nblocks % 8 == 0) b = (b % 8) * (nblocks / 8) + b / 8;
  if (g.part) splits = (g.k + g.kchunk - 1) / g.kchunk;
  const int64_t tile_of_all = b;
  const int64_t tb = tile_of_all / per_batch;  // (split, batch) combined
  const int64_t t = tile_of_all % per_batch;
  const int64_t nb = (nblocks / per_batch) / splits;
  split = tb / nb;
  bidx = tb % nb;
  const int64_t tm = t / tiles_n, tn = t % tiles_n;
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t kbeg = g.part ? split * g.kchunk : 0;
  const int64_t kend = g.part ? min(g.k, kbeg + g.kchunk) : g.k;

  const char* A = (const char*)g.a + bidx * g.a_bs * (int64_t)sizeof(T);
  const char* B = (const char*)g.b + bidx * g.b_bs * (int64_t)sizeof(T);
  // A_K: bytes between rows; else bytes between k-rows.  Same for B.
  const int64_t a_ldb = (A_K ? g.a_rs : g.a_cs) * (int64_t)sizeof(T);
  const int64_t b_ldb = (B_K ? g.b_cs : g.b_rs) * (int64_t)sizeof(T);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 15, lg = lane >> 4;

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  OperandLoad<BM, NT, A_K> la;
  OperandLoad<BN, NT, B_K> lb;
  la.init(A, a_ldb, m0, g.m);
  lb.init(B, b_ldb, n0, g.n);
  const bool full_a = m0 + BM <= g.m, full_b = n0 + BN <= g.n;
  la.template issue<KT>(kbeg, lds, full_a, kend);
  lb.template issue<KT>(kbeg, lds + A_BYTES, full_b, kend);
  // k-contiguous fragment rows wm*WM + i*16 + lr share the swizzle of lr
  const int sw = (lr >> 1) & 7;

  int cur = 0;
  for (int64_t k0 = kbeg; k0 < kend; k0 += 64) {
    __builtin_amdgcn_s_waitcnt(0x3f70 & 0xc07f);  // vmcnt(0)
    __syncthreads();
    if (k0 + 64 < kend) {
      char* nxt = lds + (cur ^ 1) * STAGE;
      la.template issue<KT>(k0 + 64, nxt, full_a, kend);
      lb.template issue<KT>(k0 + 64, nxt + A_BYTES, full_b, kend);
    }
    const char* at = lds + cur * STAGE;
    const char* bt = at + A_BYTES;
    const bool tail = KT && k0 + 64 > kend;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int coff = ((ks * 4 + lg) ^ sw) * 16;
      const int64_t kfrag = k0 + ks * 32 + lg * 8;
      frag bfr[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (B_K) bfr[j] = *(const frag*)(bt + (wn * WN + lr) * 128 + j * 2048 + coff);
        else bfr[j] = mn_frag<T, BN>(bt, wn * WN + j * 16, ks);
        if (tail) mask_k(bfr[j], kfrag, kend);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        frag af;
        if constexpr (A_K) af = *(const frag*)(at + (wm * WM + lr) * 128 + i * 2048 + coff);
        else af = mn_frag<T, BM>(at, wm * WM + i * 16, ks);
        if (tail) mask_k(af, kfrag, kend);
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::mma(af, bfr[j], acc[i][j]);
      }
    }
    cur ^= 1;
  }

  if (g.part) {
    float* P = g.part + (split * nb + bidx) * g.m * g.n;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn * WN + j * 16 + lr;
      if (col >= g.n) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t row = m0 + wm * WM + i * 16 + lg * 4 + e;
          if (row < g.m) P[row * g.n + col] = acc[i][j][e];
        }
    }
    return;
  }
  const int64_t c_es = g.c_dt == MI355X_F32 ? 4 : 2;
  char* Cb = (char*)g.c + bidx * g.c_bs * c_es;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = n0 + wn * WN + j * 16 + lr;
    if (col >= g.n) continue;
    const float bias = g.bias ? ld_any(g.bias, g.bias_dt, col) : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = m0 + wm * WM + i * 16 + lg * 4 + e;
        if (row >= g.m) continue;
        const int64_t off = row * g.c_rs + col;
        float v = acc[i][j][e] + bias;
        if (g.beta) v += ld_any(Cb, g.c_dt, off);
        if (g.c_dt == MI355X_BF16) ((bf16*)Cb)[off] = (bf16)v;
        else if (g.c_dt == MI355X_F32) ((float*)Cb)[off] = v;
        else ((f16*)Cb)[off] = (f16)v;
      }
    }
  }
}

// Pack an operand into a k-contiguous [rows][ld] buffer of 16-bit elements,
// zero-filling k in [K, ld).  Source element (row, k) is at
//   transposed: src + b*sbs + k*sk + row      (row-contiguous source)
//   straight:   src + b*sbs + row*sr + k      (k-contiguous, any row stride)
// 64x64 tiles through LDS keep both the reads and the writes coalesced.
__global__ void __launch_bounds__(256) pack_k_contig(uint16_t* __restrict__ dst, int64_t ld,
                                                     int64_t dst_bs, const uint16_t* __restrict__ src,
                                                     int64_t stride, int64_t sbs, int64_t rows,
                                                     int64_t kdim, int transposed) {
  __shared__ uint16_t tile[64][65];
  const int64_t b = blockIdx.z;
  const int64_t row0 = (int64_t)blockIdx.y * 64, k0 = (int64_t)blockIdx.x * 64;
  const uint16_t* S = src + b * sbs;
  uint16_t* D = dst + b * dst_bs;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  if (transposed) {
    for (int i = ty; i < 64; i += 4) {  // i: k offset, tx: row offset (contiguous)
      const int64_t k = k0 + i, r = row0 + tx;
      tile[i][tx] = (k < kdim && r < rows) ? S[k * stride + r] : (uint16_t)0;
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {  // i: row offset, tx: k offset (contiguous)
      const int64_t r = row0 + i, k = k0 + tx;
      if (r < rows && k < ld) D[r * ld + k] = tile[tx][i];
    }
  } else {
    for (int i = ty; i < 64; i += 4) {
      const int64_t r = row0 + i, k = k0 + tx;
      if (r < rows && k < ld) D[r * ld + k] = k < kdim ? S[r * stride + k] : (uint16_t)0;
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

// ---------------------------------------------------------------------------
// planning
// ---------------------------------------------------------------------------
struct Plan {
  int bm, bn;
  int splits;
  int64_t kchunk;
};

// Pick the block tile that finishes in the fewest rounds of the 256 CUs
// (weighted by per-tile efficiency), then split K when the output alone
// cannot fill the chip.
Plan plan_gemm(int64_t batch, int64_t m, int64_t n, int64_t k, bool fast) {
  struct Cfg { int bm, bn, per_cu; double eff; };
  const Cfg fast_cfgs[] = {{256, 128, 1, 1.0}, {128, 256, 1, 1.0}, {128, 128, 2, 0.6}};
  const Cfg gen_cfgs[] = {{256, 128, 1, 1.0}, {128, 256, 1, 1.0}, {128, 128, 2, 0.9}};
  const Cfg* cfgs = fast ? fast_cfgs : gen_cfgs;
  const int ncfg = 3;
  Plan best{128, 128, 1, k};
  double best_cost = 1e300;
  for (int i = 0; i < ncfg; ++i) {
    const Cfg& c = cfgs[i];
    const int64_t tiles = ((m + c.bm - 1) / c.bm) * ((n + c.bn - 1) / c.bn) * batch;
    const int64_t slots = (int64_t)kCUs * c.per_cu;
    const int64_t rounds = (tiles + slots - 1) / slots;
    const double cost = (double)rounds * c.bm * c.bn / (c.per_cu * c.eff);
    if (cost < best_cost - 1e-9) best_cost = cost, best = Plan{c.bm, c.bn, 1, k};
  }
  // Tuning override, e.g. MI355X_GEMM_TILE=256x128 (fast path only).
  static const char* forced = getenv("MI355X_GEMM_TILE");
  if (fast && forced) {
    int fm = 0, fn = 0;
    if (sscanf(forced, "%dx%d", &fm, &fn) == 2 && (fm == 128 || fm == 256) && (fn == 128 || fn == 256) &&
        !(fm == 256 && fn == 256))
      best = Plan{fm, fn, 1, k};
  }
  const int64_t tiles = ((m + best.bm - 1) / best.bm) * ((n + best.bn - 1) / best.bn) * batch;
  if (tiles < kCUs && k >= 2048) {
    int64_t s = (2 * kCUs + tiles - 1) / tiles;
    const int64_t max_s = k / 512;
    if (s > max_s) s = max_s;
    if (s > 64) s = 64;
    if (s > 1) {
      int64_t chunk = (k + s - 1) / s;
      chunk = (chunk + 63) / 64 * 64;
      best.splits = (int)((k + chunk - 1) / chunk);
      best.kchunk = chunk;
    }
  }
  return best;
}

template <typename T, int BM, int BN>
int launch_cfg(const GemmArgs& g, int64_t batch, int splits, hipStream_t s) {
  constexpr int NT = (BM / 64) * (BN / 64) * 64;
  dim3 grid(ceil_div(g.n, BN), ceil_div(g.m, BM), (unsigned)(batch * splits));
  const size_t lds = 2 * (BM + BN) * LDS_ROW * sizeof(T);
  const bool ak = g.a_cs == 1, bk = g.b_rs == 1;
  if (ak && bk) gemm_mfma<T, BM, BN, true, true><<<grid, NT, lds, s>>>(g);
  else if (ak && !bk) gemm_mfma<T, BM, BN, true, false><<<grid, NT, lds, s>>>(g);
  else if (!ak && bk) gemm_mfma<T, BM, BN, false, true><<<grid, NT, lds, s>>>(g);
  else gemm_mfma<T, BM, BN, false, false><<<grid, NT, lds, s>>>(g);
  return check_launch("mi355x_gemm");
}

template <typename T, int BM, int BN, bool KT>
int launch_fast_kt(const GemmArgs& g, int64_t blocks, size_t lds, int tm, int tn, hipStream_t s) {
  const bool ak = g.a_cs == 1, bk = g.b_rs == 1;
  if (ak && bk) gemm_nt_fast<T, BM, BN, true, true, KT><<<(unsigned)blocks, 256, lds, s>>>(g, tm, tn);
  else if (ak) gemm_nt_fast<T, BM, BN, true, false, KT><<<(unsigned)blocks, 256, lds, s>>>(g, tm, tn);
  else if (bk) gemm_nt_fast<T, BM, BN, false, true, KT><<<(unsigned)blocks, 256, lds, s>>>(g, tm, tn);
  else gemm_nt_fast<T, BM, BN, false, false, KT><<<(unsigned)blocks, 256, lds, s>>>(g, tm, tn);
  return check_launch("mi355x_gemm");
}

template <typename T, int BM, int BN>
int launch_fast_cfg(const GemmArgs& g, int64_t batch, int splits, hipStream_t s) {
  const int tm = (int)ceil_div(g.m, BM), tn = (int)ceil_div(g.n, BN);
  const int64_t blocks = (int64_t)tm * tn * batch * splits;
  const size_t lds = 2 * (BM + BN) * 128;
  if (g.k % 64) return launch_fast_kt<T, BM, BN, true>(g, blocks, lds, tm, tn, s);
  return launch_fast_kt<T, BM, BN, false>(g, blocks, lds, tm, tn, s);
}

int splitk_finish(const GemmArgs& g, int64_t batch, int splits, hipStream_t s) {
  const int64_t total = batch * g.m * g.n;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  splitk_reduce<<<(unsigned)blocks, 256, 0, s>>>(g, splits, batch);
  return check_launch("mi355x_gemm splitk_reduce");
}

template <typename T>
int launch_mfma(GemmArgs g, int64_t batch, const Plan& p, hipStream_t s) {
  int rc;
  if (p.bm == 256) rc = launch_cfg<T, 256, 128>(g, batch, p.splits, s);
  else if (p.bn == 256) rc = launch_cfg<T, 128, 256>(g, batch, p.splits, s);
  else rc = launch_cfg<T, 128, 128>(g, batch, p.splits, s);
  if (rc || !g.part) return rc;
  return splitk_finish(g, batch, p.splits, s);
}

template <typename T>
int launch_fast(GemmArgs g, int64_t batch, const Plan& p, hipStream_t s) {
  int rc;
  if (p.bm == 256) rc = launch_fast_cfg<T, 256, 128>(g, batch, p.splits, s);
  else if (p.bn == 256) rc = launch_fast_cfg<T, 128, 256>(g, batch, p.splits, s);
  else rc = launch_fast_cfg<T, 128, 128>(g, batch, p.splits, s);
  if (rc || !g.part) return rc;
  return splitk_finish(g, batch, p.splits, s);
}

bool fdt(int d) { return d == MI355X_F32 || d == MI355X_BF16 || d == MI355X_F16; }

// Workspace layout of the MFMA path: [split-K partials][packed A][packed B].
struct WsLayout {
  bool pack_a, pack_b;
  int64_t kp;
  int64_t part_bytes, a_bytes, b_bytes, total;
  Plan plan;
};

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

WsLayout ws_layout(int64_t batch, int64_t m, int64_t n, int64_t k, const void* a, int64_t a_rs,
                   int64_t a_cs, int64_t a_bs, const void* b, int64_t b_rs, int64_t b_cs,
                   int64_t b_bs) {
  WsLayout w{};
  w.kp = (k + 63) / 64 * 64;
  // In place when K tiles are whole and every 16-byte load is aligned:
  // k-contiguous operands need an 8-element row stride, m/n-contiguous ones
  // an 8-element k stride and a row count that is a multiple of 8.
  // K tails are masked in the kernel; a last partial 8-element chunk may
  // read into row padding, so the contiguous extent must be padded to 8.
  auto up8 = [](int64_t v) { return (v + 7) / 8 * 8; };
  auto in_place = [&](const void* p, int64_t rs, int64_t cs, int64_t bs, int64_t nrows) {
    if (bs % 8 != 0 || (p != nullptr && !aligned16(p))) return false;
    if (cs == 1) return rs % 8 == 0 && rs >= up8(k);
    return cs % 8 == 0 && cs >= up8(nrows);
  };
  // An m/n-contiguous operand that is small next to the product (a weight in
  // dX = dY W) is still packed: the copy costs under ~3% of the GEMM and the
  // k-contiguous fragment reads are cheaper than transposing ones.
  const double small_rows = 2e-4 * (double)m * (double)n;
  w.pack_a = !in_place(a, a_rs, a_cs, a_bs, m) || (a_cs != 1 && (double)m < small_rows);
  // B as [n rows][k]: row stride b_cs, k stride b_rs
  w.pack_b = !in_place(b, b_cs, b_rs, b_bs, n) || (b_rs != 1 && (double)n < small_rows);
  w.plan = plan_gemm(batch, m, n, w.kp, true);
  auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
  w.part_bytes = w.plan.splits > 1 ? up((int64_t)w.plan.splits * batch * m * n * 4) : 0;
  const int64_t ab = a_bs == 0 ? 1 : batch, bb = b_bs == 0 ? 1 : batch;
  w.a_bytes = w.pack_a ? up(ab * m * w.kp * 2) : 0;
  w.b_bytes = w.pack_b ? up(bb * n * w.kp * 2) : 0;
  w.total = w.part_bytes + w.a_bytes + w.b_bytes;
  return w;
}

int pack(uint16_t* dst, const void* src, int64_t batch, int64_t rows, int64_t kdim, int64_t ld,
         int64_t row_stride, int64_t k_stride, int64_t sbs, hipStream_t s) {
  // row_stride == 1: rows contiguous (transpose); else k_stride == 1 (straight)
  const bool transposed = row_stride == 1 && k_stride != 1;
  dim3 grid(ceil_div(ld, 64), ceil_div(rows, 64), (unsigned)batch);
  pack_k_contig<<<grid, 256, 0, s>>>(dst, ld, rows * ld, (const uint16_t*)src,
                                      transposed ? k_stride : row_stride, sbs, rows, kdim,
                                      transposed ? 1 : 0);
  return check_launch("mi355x_gemm pack");
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int64_t mi355x_gemm_workspace_bytes(const void* a, int64_t a_rs, int64_t a_cs,
                                               int64_t a_bs, const void* b, int64_t b_rs,
                                               int64_t b_cs, int64_t b_bs, int ab_dtype,
                                               int64_t batch, int64_t m, int64_t n, int64_t k) {
  if (ab_dtype == MI355X_F32 || m <= 0 || n <= 0 || k <= 0) return 0;
  return ws_layout(batch, m, n, k, a, a_rs, a_cs, a_bs, b, b_rs, b_cs, b_bs).total;
}

extern "C" int mi355x_gemm(void* c, int c_dtype, int64_t c_rs, int64_t c_bs, const void* a,
                           int64_t a_rs, int64_t a_cs, int64_t a_bs, const void* b, int64_t b_rs,
                           int64_t b_cs, int64_t b_bs, int ab_dtype, const void* bias,
                           int bias_dtype, int beta, int64_t batch, int64_t m, int64_t n,
                           int64_t k, void* workspace, int64_t ws_bytes, mi355x_stream_t stream) {
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
             beta, m, n, k, 0, 0, nullptr, k};
  if (ab_dtype == MI355X_F32) {
    dim3 grid(ceil_div(n, 64), ceil_div(m, 64), (unsigned)batch);
    gemm_f32<<<grid, 256, 0, s>>>(g);
    return check_launch("mi355x_gemm");
  }
  WsLayout w = ws_layout(batch, m, n, k, a, a_rs, a_cs, a_bs, b, b_rs, b_cs, b_bs);
  if (w.total > 0 && (!workspace || ws_bytes < w.total))
    return fail(MI355X_EWORKSPACE, "mi355x_gemm: workspace %lld < %lld", (long long)ws_bytes,
                (long long)w.total);
  char* ws = (char*)workspace;
  if (w.pack_a) {
    uint16_t* pa = (uint16_t*)(ws + w.part_bytes);
    const int64_t nb = a_bs == 0 ? 1 : batch;
    int rc = pack(pa, a, nb, m, k, w.kp, a_rs, a_cs, a_bs, s);
    if (rc) return rc;
    g.a = pa; g.a_rs = w.kp; g.a_cs = 1; g.a_bs = a_bs == 0 ? 0 : m * w.kp;
  }
  if (w.pack_b) {
    uint16_t* pb = (uint16_t*)(ws + w.part_bytes + w.a_bytes);
    const int64_t nb = b_bs == 0 ? 1 : batch;
    // B viewed as [n rows][k]: row stride b_cs, k stride b_rs
    int rc = pack(pb, b, nb, n, k, w.kp, b_cs, b_rs, b_bs, s);
    if (rc) return rc;
    g.b = pb; g.b_rs = 1; g.b_cs = w.kp; g.b_bs = b_bs == 0 ? 0 : n * w.kp;
  }
  // packed operands are zero-padded to kp; the kernel masks k >= K
  if (w.plan.splits > 1) {
    g.part = (float*)ws;
    g.kchunk = w.plan.kchunk;
  }
  if (ab_dtype == MI355X_BF16) return launch_fast<bf16>(g, batch, w.plan, s);
  return launch_fast<f16>(g, batch, w.plan, s);
}
