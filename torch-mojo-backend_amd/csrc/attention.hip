// Fused flash attention on MFMA (bf16/f16 in, f32 accumulation).
//
// Semantics (the reference's fused path, flash_attention_bwd_kernels.mojo:
// 13-26, 63-66, 1403-1404):
//   S = scale * Q K^T, masked (causal: key j visible to query i iff j <= i,
//   top-left aligned, also when Sq != Skv), O = softmax(S) V,
//   LSE_i = natural-log log-sum-exp of row i (f32, [B, H, Sq]).
//   Backward: D_i = sum(dO_i * O_i), P = exp(S - LSE), dV = P^T dO,
//   dP = dO V^T, dS = P * (dP - D), dQ = scale dS K, dK = scale dS^T Q.
//
// Layout strategy.  Every product is issued in the orientation that keeps
// the per-query softmax state in the lane that owns the query:
//   forward   S^T = K Q^T   (lane = query column, 4 keys per lane-group)
//             O^T += V^T P^T (P^T fed straight from the S^T accumulators)
// The MFMA k index of the P^T operand is a permutation of the keys (lane
// group g carries keys 4g..4g+3 of two 16-key tiles); V^T is read from a
// transposed LDS tile with the same permutation, which the MFMA sum does not
// observe.  Q lives in registers for the whole key loop; K and V^T tiles of
// 64 keys are staged through LDS.  Blocks take 128 queries (4 waves x 32) and
// the heaviest causal blocks are scheduled first.
//
// Backward is two kernels plus a row-term pass (no atomics, every output
// written exactly once):
//   dK/dV: a block owns 64 keys (a wave 16); it walks the query blocks that
//          can see them, recomputing S and dP with the key tile as the MFMA
//          column, and accumulates dV^T = dO^T P and dK^T = Q^T dS.
//   dQ:    a block owns 64 queries (a wave 16); it walks the visible key
//          blocks, recomputing S^T and dP^T, and accumulates dQ^T = K^T dS^T.
#include <math.h>

#include <mutex>

#include "common.h"
#include "mfma.h"

// D = 64 forward: waves per 128-query block (4: 32 queries per wave) and
// blocks per CU it is compiled for (the second __launch_bounds__ argument is
// the minimum number of waves per SIMD, which sets the register budget).
#ifndef ATTN_FWD_WAVES
#define ATTN_FWD_WAVES 4
#endif
#ifndef ATTN_FWD_BLOCKS
#define ATTN_FWD_BLOCKS 2
#endif
// Backward (D = 64): waves per SIMD the dK/dV and dQ kernels are compiled for.
#ifndef ATTN_BWD_WAVES
#define ATTN_BWD_WAVES 2
#endif
#ifndef ATTN_ASM_DMA
#define ATTN_ASM_DMA 1
#endif

namespace mi {
namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <typename T>
struct alignas(16) V8 {
  T v[8];
};
template <typename T>
struct alignas(8) V4 {
  T v[4];
};

struct AttnArgs {
  void* o; int64_t o_b, o_h, o_s;
  float* lse;
  const void* q; int64_t q_b, q_h, q_s;
  const void* k; int64_t k_b, k_h, k_s;
  const void* v; int64_t v_b, v_h, v_s;
  int64_t B, H, Sq, Skv;
  float scale_log2;  // scale * log2(e)
  float scale;
  int causal;
  int64_t group;   // query heads per K/V head (grouped-query attention), >= 1
  int64_t window;  // > 0: query i sees keys i-window+1 .. i (causal only); 0: none
};

// Stage a 64-row x D tile (rows row0.., row stride rs) into LDS: row-major
// [64][D+8] and/or transposed [D][64+8].  Rows past nrows read as zero.
template <typename T, int D>
__device__ __forceinline__ void stage_tile(T* rm, T* tr, const T* g, int64_t rs, int64_t row0,
                                           int64_t nrows) {
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  for (int c = threadIdx.x; c < 64 * CPR; c += kThreads) {
    const int r = c / CPR, dc = (c % CPR) * 8;
    V8<T> val;
    if (row0 + r < nrows) {
      val = *(const V8<T>*)(g + (row0 + r) * rs + dc);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) val.v[e] = (T)0.f;
    }
    if (rm) *(V8<T>*)(rm + r * (D + 8) + dc) = val;
    if (tr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) tr[(dc + e) * 72 + r] = val.v[e];
    }
  }
}

template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag zero_frag() {
  typename Mfma<T>::frag f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (T)0.f;
  return f;
}

// 8 keys of the permuted k index from a transposed [D][72] tile:
// slots 0-3 = cols t0*16+4g..+3, slots 4-7 = cols t1*16+4g..+3.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag perm_frag(const T* tr, int row, int t0, int t1,
                                                            int g) {
  typename Mfma<T>::frag f;
  V4<T> a = *(const V4<T>*)(tr + row * 72 + t0 * 16 + 4 * g);
  V4<T> b = *(const V4<T>*)(tr + row * 72 + t1 * 16 + 4 * g);
#pragma unroll
  for (int e = 0; e < 4; ++e) f[e] = a.v[e], f[4 + e] = b.v[e];
  return f;
}

// XCD-aware, heaviest-first block coordinates over a (tiles, H, B) grid.
// The hardware deals workgroups to the 8 XCDs round-robin by linear id, so
// ids are renumbered to give each XCD a contiguous range of (b, h) pairs:
// all tiles of one pair share one L2, and its K/V (or Q/dO) come from HBM
// once instead of once per XCD.  Inside an XCD's range the tile index
// varies slowest, so the heaviest causal tiles (tile 0 after the kernels'
// own reversal for query tiles; key tile 0 for dK/dV) of all its pairs are
// dispatched first and spread over the CUs, and the light ones fill in
// behind them instead of several heavy tiles landing on one CU.
struct BlockCoord {
  int64_t x, h, b;
};
// A block's linear id and the (x, y, z) grid it is placed in.  Kernels that
// serve two grids from one launch pass a virtual id here.
struct GridPos {
  uint32_t nx, ny, nz, l;
};
__device__ __forceinline__ GridPos hw_grid() {
  return GridPos{gridDim.x, gridDim.y, gridDim.z, blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)};
}
constexpr uint32_t kCUsPerXCD = 32;
__device__ __forceinline__ BlockCoord block_coord(GridPos g, bool zigzag = false) {
  const uint32_t nx = g.nx, ny = g.ny, n = nx * ny * g.nz;
  const uint32_t l = g.l;
  BlockCoord c;
  if ((n & 7) == 0 && ((n >> 3) % nx) == 0) {
    const uint32_t pairs = (n >> 3) / nx;  // (b, h) pairs per XCD
    uint32_t i = l >> 3;
    // zigzag: every other round of kCUsPerXCD slots takes its tiles in
    // reverse (light to heavy), so a CU that got a heavy tile in one round
    // gets a light one in the next and the per-CU sums even out.
    if (zigzag) {
      const uint32_t r = i / kCUsPerXCD, j = r * kCUsPerXCD + (kCUsPerXCD - 1 - i % kCUsPerXCD);
      if ((r & 1) && j < (n >> 3)) i = j;
    }
    c.x = i / pairs;
    const uint32_t pair = (l & 7) * pairs + (i - (uint32_t)c.x * pairs);
    c.h = pair % ny;
    c.b = pair / ny;
  } else {
    c.x = l % nx;
    const uint32_t r = l / nx;
    c.h = r % ny;
    c.b = r / ny;
  }
  return c;
}
__device__ __forceinline__ BlockCoord block_coord(bool zigzag = false) { return block_coord(hw_grid(), zigzag); }

// Reductions over the four 16-lane groups of a wave (the key rows of an
// S^T tile): v_permlane16_swap / v_permlane32_swap with both operands = x
// leave x's partner row (lane +-16, then +-32) in the second result.
__device__ __forceinline__ float group_max(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group_sum(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// 2^x on the transcendental unit (results below 2^-126 flush to zero, which
// softmax weights never miss).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename T, int D, bool POS>
__global__ void __launch_bounds__(kThreads) attn_fwd_kernel(AttnArgs p) {
  typedef typename Mfma<T>::frag frag;
  constexpr int KS = D / 32;  // MFMA k-steps over the head dim
  constexpr int DT = D / 16;  // 16-wide head-dim tiles
  __shared__ __attribute__((aligned(16))) T Ks[64 * (D + 8)];
  __shared__ __attribute__((aligned(16))) T Vt[D * 72];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  const BlockCoord bc = block_coord();
  const int64_t qblock = p.causal ? (int64_t)gridDim.x - 1 - bc.x : bc.x;
  const int64_t q0 = qblock * 128;
  const int64_t b = bc.b, h = bc.h;
  const T* Q = (const T*)p.q + b * p.q_b + h * p.q_h;
  const T* K = (const T*)p.k + b * p.k_b + h * p.k_h;
  const T* V = (const T*)p.v + b * p.v_b + h * p.v_h;

  // Q^T operand fragments (query column = lane row index)
  frag qf[2][KS];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t qi = q0 + wave * 32 + qt * 16 + lr;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[qt][ks] = qi < p.Sq ? *(const frag*)(Q + qi * p.q_s + ks * 32 + lg * 8) : zero_frag<T>();
  }
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
  f32x4 oacc[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt][0] = oacc[dt][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  int64_t kv_end = p.Skv;
  if (p.causal) kv_end = min(p.Skv, q0 + 128);
  for (int64_t kb0 = 0; kb0 < kv_end; kb0 += 64) {
    __syncthreads();
    stage_tile<T, D>(Ks, nullptr, K, p.k_s, kb0, p.Skv);
    stage_tile<T, D>(nullptr, Vt, V, p.v_s, kb0, p.Skv);
    __syncthreads();

    f32x4 s[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      frag kf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = *(const frag*)(Ks + (kt * 16 + lr) * (D + 8) + ks * 32 + lg * 8);
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) a = Mfma<T>::mma(kf[ks], qf[qt][ks], a);
        s[kt][qt] = a;
      }
    }
    // Online softmax in the exp2 domain.  With a positive scale the row max
    // is taken on the raw scores and p = 2^(s*c - m) is one FMA + one exp;
    // each lane keeps a partial row sum (its 16 keys per tile) under the
    // shared max, summed across the four lane groups once at the end.  O is
    // rescaled only when some row's max grew.
    const bool need_mask = (kb0 + 64 > p.Skv) || (p.causal && kb0 + 64 > q0 + wave * 32);
    const float c = p.scale_log2;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      int lim = 63;  // keys kb0 + 0..lim are visible to this lane's query
      if (need_mask) {
        const int64_t qi = q0 + wave * 32 + qt * 16 + lr;
        int64_t lm = p.Skv - 1 - kb0;
        if (p.causal && qi - kb0 < lm) lm = qi - kb0;
        lim = (int)max((int64_t)-1, min((int64_t)63, lm));
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = POS ? s[kt][qt][e] : s[kt][qt][e] * c;
          if (need_mask && kt * 16 + lg * 4 + e > lim) v = -INFINITY;
          s[kt][qt][e] = v;
          mx = fmaxf(mx, v);
        }
      mx = group_max(mx);
      const float m_new = fmaxf(m[qt], POS ? mx * c : mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      float rs = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pv = fast_exp2(POS ? fmaf(s[kt][qt][e], c, -m_use) : s[kt][qt][e] - m_use);
          s[kt][qt][e] = pv;
          rs += pv;
        }
      const float alpha = fast_exp2(m[qt] - m_use);
      l[qt] = l[qt] * alpha + rs;
      m[qt] = m_new;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt][qt] *= alpha;
      }
    }
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
      frag pf[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pf[qt][e] = (T)s[2 * ks2][qt][e];
          pf[qt][4 + e] = (T)s[2 * ks2 + 1][qt][e];
        }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const frag vf = perm_frag<T>(Vt, dt * 16 + lr, 2 * ks2, 2 * ks2 + 1, lg);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) oacc[dt][qt] = Mfma<T>::mma(vf, pf[qt], oacc[dt][qt]);
      }
    }
  }

  // epilogue: lane holds O[query lr][d = dt*16 + 4*lg + e]
  T* O = (T*)p.o + b * p.o_b + h * p.o_h;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) l[qt] = group_sum(l[qt]);
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int64_t qi = q0 + wave * 32 + qt * 16 + lr;
    if (qi >= p.Sq) continue;
    const float inv = l[qt] > 0.f ? 1.f / l[qt] : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      V4<T> o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o4.v[e] = (T)(oacc[dt][qt][e] * inv);
      *(V4<T>*)(O + qi * p.o_s + dt * 16 + lg * 4) = o4;
    }
    if (lg == 0)
      p.lse[(b * p.H + h) * p.Sq + qi] = l[qt] > 0.f ? (m[qt] + log2f(l[qt])) * kLn2 : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// forward, head_dim 64/128: direct-to-LDS K/V staging + transposing reads.
//
// K and V tiles (64 keys) are copied global -> LDS with global_load_lds
// (1 KB per wave instruction), double-buffered so the next key block streams
// in during the current block's math, and stored row-major with the 16-byte
// chunks of each row XOR-swizzled (conflict-free 16-row fragment reads).
// The V^T operand of O^T += V^T P^T is read straight from the row-major V
// tile with ds_read_b64_tr_b16: within a 16-lane group, lane i receives
// element i%4 of the 4-element pieces supplied by lanes i/4, 4+i/4, 8+i/4 and
// 12+i/4, so two such reads give each lane the 8 (permuted) keys of its
// head-dim row.
// ---------------------------------------------------------------------------
typedef const void __attribute__((address_space(1)))* gptr_t;
typedef void __attribute__((address_space(3)))* lptr_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int D>
struct KvLayout {
  static constexpr int ROWB = D * 2;          // bytes per row
  static constexpr int CH = D / 8;            // 16-byte chunks per row
  static constexpr int TILE = 64 * ROWB;      // one 64-row tile
  static constexpr int RPI = 1024 / ROWB;     // rows per 1 KB load instruction
  // Chunk swizzle of row r, chosen from LDS bank-conflict counter
  // measurements of the two read patterns: 16-byte fragment reads (16
  // consecutive rows at one chunk) and ds_read_b64_tr_b16 reads (rows
  // 4g + j, adjacent chunks c, c ^ 1).  Both run without bank conflicts.
  //   D = 64 (128-byte rows):  r & 7
  //   D = 128 (256-byte rows): bit 0 = r3, bits 1-2 = r0-r1, bit 3 = r2 ^ r3
  static __device__ __forceinline__ int swz(int row) {
    if constexpr (D == 256) return row & 15;  // 512-byte rows: 16 rows at one chunk hit 16 bank groups
    return D == 64 ? (row & 7)
                   : (((row >> 3) & 1) | ((row & 3) << 1) | ((((row >> 2) ^ (row >> 3)) & 1) << 3));
  }
  // byte offset of element (row, col) in a swizzled tile
  static __device__ __forceinline__ int off(int row, int col) {
    return row * ROWB + (((col >> 3) ^ swz(row)) << 4) + ((col & 7) << 1);
  }
};

__host__ __device__ inline int64_t ceil_div64(int64_t a, int64_t b) { return a <= 0 ? 0 : (a + b - 1) / b; }


extern __shared__ __attribute__((aligned(1024))) char attn_dyn_lds[];

template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

// Fragment of 8 permuted keys for head-dim row `d`: slots 0-3 = keys
// t0*16+4g+0..3, slots 4-7 = keys t1*16+4g+0..3 (g = lane/16).
template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::frag tr_frag(const char* tile, int dt, int t0, int t1) {
  typedef KvLayout<D> L;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, src = lane & 15;
  const int col = dt * 16 + 4 * (src & 3);
  const int r0 = t0 * 16 + 4 * g + (src >> 2), r1 = t1 * 16 + 4 * g + (src >> 2);
  s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + L::off(r0, col)));
  s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + L::off(r1, col)));
  typename Mfma<T>::frag f;
  short* fs = (short*)&f;
#pragma unroll
  for (int e = 0; e < 4; ++e) fs[e] = a[e], fs[4 + e] = b[e];
  return f;
}

// This lane's byte offsets of tr_frag's reads at tile row 0, one per
// head-dim block dt.  Row t0*16 + r has the swizzle of r (it uses only the
// row's low four bits), so tr_frag(tile, dt, t0, t1) reads tile +
// t0*16*ROWB + o[dt] and tile + t1*16*ROWB + o[dt]: with the offsets kept
// in registers the per-step address arithmetic folds into immediates.
template <int D>
struct TrOffsets {
  int o[D / 16];
  __device__ __forceinline__ TrOffsets() {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, src = lane & 15;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) o[dt] = KvLayout<D>::off(4 * g + (src >> 2), dt * 16 + 4 * (src & 3));
  }
};

template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::frag tr_frag_at(const char* tile, const TrOffsets<D>& to, int dt,
                                                             int t0, int t1) {
  constexpr int RB = 16 * KvLayout<D>::ROWB;
  s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + t0 * RB + to.o[dt]));
  s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + t1 * RB + to.o[dt]));
  typename Mfma<T>::frag f;
  short* fs = (short*)&f;
#pragma unroll
  for (int e = 0; e < 4; ++e) fs[e] = a[e], fs[4 + e] = b[e];
  return f;
}

// Tile loader (K/V in the forward and dQ pass, Q/dO in the dK/dV pass):
// each thread's byte offsets within a full tile are computed once, so a tile
// costs one scalar row-offset product plus one 64-bit add per load (a 64-bit
// vector multiply per load, as recomputing them would take, runs at a
// quarter of the VALU rate).  Rows past the end (only in the last tile)
// reload the last row; their scores are masked.
template <int D, int NW>
struct KvTileLoad {
  typedef KvLayout<D> L;
  static constexpr int IT = L::TILE / 1024 / NW;  // 1 KB load instructions per thread
  const char* g;
  int64_t rs;
  int64_t off[IT];   // r * rs + chunk * 16
  static __device__ __forceinline__ int row_of(int it) {
    return (it * NW + wave_id()) * L::RPI + (int)(threadIdx.x & 63) / L::CH;
  }
  static __device__ __forceinline__ int coff_of(int row) {
    return (((int)(threadIdx.x & 63) % L::CH) ^ L::swz(row)) * 16;
  }
  __device__ __forceinline__ void init(const char* base, int64_t rs_bytes) {
    g = base;
    rs = rs_bytes;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int r = row_of(it);
      off[it] = r * rs + coff_of(r);
    }
  }
  __device__ __forceinline__ void issue(int64_t row0, int64_t nrows, char* dst) const {
    const int wave = wave_id();
    if (row0 + 64 <= nrows) {
      const char* tb = g + row0 * rs;
#pragma unroll
      for (int it = 0; it < IT; ++it) load(tb + off[it], dst + (it * NW + wave) * 1024);
    } else {
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int r = row_of(it);
        const int64_t gr = min(row0 + r, nrows - 1);
        load(g + gr * rs + coff_of(r), dst + (it * NW + wave) * 1024);
      }
    }
  }
  static __device__ __forceinline__ void load(const char* src, char* dst) {
#if ATTN_ASM_DMA
    dma_b128(src, lds_base_of(dst));
#else
    __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)dst, 16, 0, 0);
#endif
  }
};

// Forward step softmax (per 16-query tile, exp2 domain).  The running max m
// is only a reference: it moves (and O, l are rescaled) when a row's max
// exceeds it by more than kSlack, so most steps skip the rescale and p stays
// below 2^kSlack.  Row sums l come from an extra MFMA of a ones fragment
// against P (the same bf16 P that multiplies V).
constexpr float kSlack = 8.f;

template <typename T, int D, bool POS, int NW, int QPW>
__global__ void __launch_bounds__(64 * NW, D == 64 ? ATTN_FWD_BLOCKS * NW / 4 : 1) attn_fwd_v2(AttnArgs p) {
  constexpr int QT = QPW / 16, QPB = NW * QPW;  // 16-query tiles per wave, queries per block
  typedef typename Mfma<T>::frag frag;
  typedef KvLayout<D> L;
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int STAGE = 2 * L::TILE;  // K tile + V tile
  char* lds;
  if constexpr (D == 256) {
    lds = attn_dyn_lds;  // 2 x 64 KB, launched with dynamic LDS
  } else {
    __shared__ __attribute__((aligned(1024))) char lds_static[2 * STAGE];
    lds = lds_static;
  }

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  const BlockCoord bc = block_coord(/*zigzag=*/true);
  const int64_t qblock = p.causal ? (int64_t)gridDim.x - 1 - bc.x : bc.x;
  const int64_t q0 = qblock * QPB;
  const int64_t b = bc.b, h = bc.h, hk = h / p.group;  // K/V head of this query head
  const T* Q = (const T*)p.q + b * p.q_b + h * p.q_h;
  KvTileLoad<D, NW> kl, vl;
  kl.init((const char*)((const T*)p.k + b * p.k_b + hk * p.k_h), p.k_s * (int64_t)sizeof(T));
  vl.init((const char*)((const T*)p.v + b * p.v_b + hk * p.v_h), p.v_s * (int64_t)sizeof(T));

  frag qf[QT][KS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int64_t qi = q0 + wave * QPW + qt * 16 + lr;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[qt][ks] = qi < p.Sq ? *(const frag*)(Q + qi * p.q_s + ks * 32 + lg * 8) : zero_frag<T>();
  }
  frag ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (T)1.0f;
  float m[QT];
  f32x4 oacc[DT][QT], lacc[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m[qt] = -INFINITY;
    lacc[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  int64_t kv_end = p.Skv;
  if (p.causal) kv_end = min(p.Skv, q0 + QPB);
  // first 64-key tile any query of the block can see (sliding window)
  const int64_t j0 = p.window > 0 ? max((int64_t)0, q0 - p.window + 1) / 64 : 0;
  kl.issue(j0 * 64, p.Skv, lds);
  vl.issue(j0 * 64, p.Skv, lds + L::TILE);
  const int sw = L::swz(lr);  // fragment rows kt*16 + lr share the swizzle of lr
  const TrOffsets<D> tro;
  const float c = p.scale_log2;
  int buf = 0;
  // One step per 64 keys: the unmasked steps first, then the ones that
  // cross this wave's causal diagonal or the key end.  Two loops, so the
  // unmasked steps carry no mask code; every wave runs the same number of
  // steps (and barriers).
  auto step = [&](int64_t j, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int64_t kb0 = j * 64;
    __builtin_amdgcn_s_waitcnt(0xc07f & 0x3f70);  // vmcnt(0)
    __syncthreads();
    if (kb0 + 64 < kv_end) {
      char* nx = lds + (buf ^ 1) * STAGE;
      kl.issue(kb0 + 64, p.Skv, nx);
      vl.issue(kb0 + 64, p.Skv, nx + L::TILE);
    }
    const char* Kt = lds + buf * STAGE;
    const char* Vt = Kt + L::TILE;
    buf ^= 1;
    // a tile none of this wave's queries can see (past the causal diagonal
    // of its last query, or before the window of its first) adds nothing:
    // the wave keeps the block's loads and barriers and skips the math
    if constexpr (MASK) {
      const int64_t qf = q0 + wave * QPW;
      if (p.causal && kb0 > qf + QPW - 1) return;
      if (p.window > 0 && kb0 + 63 < qf - p.window + 1) return;
    }
      // Per query tile, the keys kb0 + lo..lim are visible to this lane's query.
      int lo[QT], lim[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        lo[qt] = 0;
        lim[qt] = 63;
        if constexpr (MASK) {
          const int64_t qi = q0 + wave * QPW + qt * 16 + lr;
          int64_t lm = p.Skv - 1 - kb0;
          if (p.causal && qi - kb0 < lm) lm = qi - kb0;
          lim[qt] = (int)max((int64_t)-1, min((int64_t)63, lm));
          if (p.window > 0) lo[qt] = (int)max((int64_t)0, min((int64_t)64, qi - p.window + 1 - kb0));
        }
      }
      // S^T tiles, each masked and folded into the row maxima right after
      // its MFMAs, so that work can issue beside the next tile's MFMAs.
      f32x4 s[4][QT];
      float mx[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) mx[qt] = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        frag kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          kf[ks] = *(const frag*)(Kt + (kt * 16 + lr) * L::ROWB + (((ks * 4 + lg) ^ sw) << 4));
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) a = Mfma<T>::mma(kf[ks], qf[qt][ks], a);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = POS ? a[e] : a[e] * c;
            if (MASK && (kt * 16 + lg * 4 + e > lim[qt] || kt * 16 + lg * 4 + e < lo[qt])) v = -INFINITY;
            a[e] = v;
            mx[qt] = fmaxf(mx[qt], v);
          }
          s[kt][qt] = a;
        }
      }
      // One rescale decision for the wave's query tiles (a uniform branch):
      // the exponentials and P V products after it are one branch-free
      // region, so the second key half's exponentials can issue beside the
      // first half's MFMAs.
      float mxc[QT];
      bool need = false;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const float g = group_max(mx[qt]);
        mxc[qt] = POS ? g * c : g;
        need |= mxc[qt] > m[qt] + kSlack;
      }
      if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const float m_new = fmaxf(m[qt], mxc[qt]);
          // a row with every key so far masked (m_new = -inf, nothing
          // accumulated) keeps its state: exp2(-inf - -inf) would be NaN
          const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m[qt] - m_new);
          lacc[qt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[dt][qt] *= alpha;
          m[qt] = m_new;
        }
      }
      float m_use[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) m_use[qt] = m[qt] == -INFINITY ? 0.f : m[qt];
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        frag pf[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float x = s[2 * ks2 + h][qt][e];
              pf[qt][4 * h + e] = (T)fast_exp2(POS ? fmaf(x, c, -m_use[qt]) : x - m_use[qt]);
            }
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) lacc[qt] = Mfma<T>::mma(ones, pf[qt], lacc[qt]);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const frag vf = tr_frag_at<T, D>(Vt, tro, dt, 2 * ks2, 2 * ks2 + 1);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) oacc[dt][qt] = Mfma<T>::mma(vf, pf[qt], oacc[dt][qt]);
        }
      }
  };
  const int64_t nkb = (kv_end + 63) / 64;
  // masked [j0, jl) (window's lower edge), unmasked [jl, ju), masked [ju, nkb)
  int64_t ju = min(nkb, p.Skv / 64);
  if (p.causal) ju = min(ju, (q0 + wave * QPW) / 64);
  int64_t jl = j0;
  if (p.window > 0) jl = min(nkb, max(j0, ceil_div64(q0 + wave * QPW + QPW - p.window, 64)));
  ju = max(ju, jl);
  int64_t j = j0;
  for (; j < jl; ++j) step(j, BoolTag<true>{});
  for (; j < ju; ++j) step(j, BoolTag<false>{});
  for (; j < nkb; ++j) step(j, BoolTag<true>{});

  // every element of lacc[qt] holds query lr's full row sum
  float l[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) l[qt] = lacc[qt][0];
  T* O = (T*)p.o + b * p.o_b + h * p.o_h;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int64_t qi = q0 + wave * QPW + qt * 16 + lr;
    if (qi >= p.Sq) continue;
    const float inv = l[qt] > 0.f ? 1.f / l[qt] : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      V4<T> o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o4.v[e] = (T)(oacc[dt][qt][e] * inv);
      *(V4<T>*)(O + qi * p.o_s + dt * 16 + lg * 4) = o4;
    }
    if (lg == 0)
      p.lse[(b * p.H + h) * p.Sq + qi] = l[qt] > 0.f ? (m[qt] + log2f(l[qt])) * kLn2 : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
struct AttnBwdArgs {
  AttnArgs f;  // o = forward output (read), q/k/v inputs, lse
  const void* dout; int64_t do_b, do_h, do_s;
  void* dq; int64_t dq_b, dq_h, dq_s;
  void* dk; int64_t dk_b, dk_h, dk_s;
  void* dv; int64_t dv_b, dv_h, dv_s;
  float* ndelta;  // [B, H, Sq]: -D, written by attn_bwd_delta
  float* nlse2;   // [B, H, Sq]: -LSE * log2(e), written by attn_bwd_delta
  float* kv_part; // grouped backward: per-query-head dK, dV partials (f32), or null
  // (stored negated: the dK/dV and dQ steps add them, which saves a negation
  // per score)
};

// D_i = sum_d dO[i, d] * O[i, d]: D/8 lanes per row, one 16-byte load of
// each operand per lane, reduced across the row's lanes.
template <typename T, int D>
__global__ void __launch_bounds__(kThreads) attn_bwd_delta(AttnBwdArgs p) {
  constexpr int CPR = D / 8;              // lanes per row
  constexpr int RPB = kThreads / CPR;     // rows per block
  // rows over B*H*Sq, fewer than 2^31 (checked at launch): 32-bit index
  // arithmetic (64-bit division is a long instruction sequence)
  const uint32_t row = blockIdx.x * (uint32_t)RPB + threadIdx.x / CPR;
  const int ch = threadIdx.x % CPR;
  const uint32_t total = (uint32_t)(p.f.B * p.f.H * p.f.Sq), sq = (uint32_t)p.f.Sq, nh = (uint32_t)p.f.H;
  float acc = 0.f;
  if (row < total) {
    const uint32_t bh = row / sq, i = row - bh * sq;
    const uint32_t b = bh / nh, h = bh - b * nh;
    const V8<T> o = *(const V8<T>*)((const T*)p.f.o + b * p.f.o_b + h * p.f.o_h + i * p.f.o_s + ch * 8);
    const V8<T> d = *(const V8<T>*)((const T*)p.dout + b * p.do_b + h * p.do_h + i * p.do_s + ch * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += to_f32(o.v[e]) * to_f32(d.v[e]);
  }
#pragma unroll
  for (int off = CPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < total && ch == 0) {
    p.ndelta[row] = -acc;
    p.nlse2[row] = -p.f.lse[row] * kLog2e;
  }
}


template <typename T, int D>
__global__ void __launch_bounds__(kThreads) attn_bwd_dkv(AttnBwdArgs p) {
  typedef typename Mfma<T>::frag frag;
  constexpr int KS = D / 32, DT = D / 16;
  __shared__ __attribute__((aligned(16))) T Qs[64 * (D + 8)];
  __shared__ __attribute__((aligned(16))) T Qt[D * 72];
  __shared__ __attribute__((aligned(16))) T dOs[64 * (D + 8)];
  __shared__ __attribute__((aligned(16))) T dOt[D * 72];
  __shared__ float lse_s[64], delta_s[64];

  const AttnArgs& f = p.f;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  const BlockCoord bc = block_coord();
  const int64_t k0 = bc.x * 64;
  const int64_t b = bc.b, h = bc.h;
  const T* Q = (const T*)f.q + b * f.q_b + h * f.q_h;
  const T* K = (const T*)f.k + b * f.k_b + h * f.k_h;
  const T* V = (const T*)f.v + b * f.v_b + h * f.v_h;
  const T* dO = (const T*)p.dout + b * p.do_b + h * p.do_h;
  const float* LSE = f.lse + (b * f.H + h) * f.Sq;
  const float* DEL = p.ndelta + (b * f.H + h) * f.Sq;

  const int64_t kw = k0 + wave * 16;  // this wave's 16 keys
  const int64_t kj = kw + lr;        // key of this lane's MFMA column
  frag kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kf[ks] = kj < f.Skv ? *(const frag*)(K + kj * f.k_s + ks * 32 + lg * 8) : zero_frag<T>();
    vf[ks] = kj < f.Skv ? *(const frag*)(V + kj * f.v_s + ks * 32 + lg * 8) : zero_frag<T>();
  }
  f32x4 dva[DT], dka[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dva[dt] = dka[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t qstart = f.causal ? (k0 / 64) * 64 : 0;
  for (int64_t qb0 = qstart; qb0 < f.Sq; qb0 += 64) {
    __syncthreads();
    stage_tile<T, D>(Qs, Qt, Q, f.q_s, qb0, f.Sq);
    stage_tile<T, D>(dOs, dOt, dO, p.do_s, qb0, f.Sq);
    if (threadIdx.x < 64) {
      const int64_t qi = qb0 + threadIdx.x;
      lse_s[threadIdx.x] = qi < f.Sq ? LSE[qi] * kLog2e : 0.f;
      delta_s[threadIdx.x] = qi < f.Sq ? -DEL[qi] : 0.f;
    }
    __syncthreads();
    // S and dP tiles: lane = key column, rows = queries 4*lg + e of tile qt
    f32x4 pt[4], ds[4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      f32x4 sa = {0.f, 0.f, 0.f, 0.f}, pa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const frag qa = *(const frag*)(Qs + (qt * 16 + lr) * (D + 8) + ks * 32 + lg * 8);
        const frag da = *(const frag*)(dOs + (qt * 16 + lr) * (D + 8) + ks * 32 + lg * 8);
        sa = Mfma<T>::mma(qa, kf[ks], sa);
        pa = Mfma<T>::mma(da, vf[ks], pa);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int qr = qt * 16 + lg * 4 + e;
        const int64_t qi = qb0 + qr;
        float pv = exp2f(sa[e] * f.scale_log2 - lse_s[qr]);
        if (qi >= f.Sq || kj >= f.Skv || (f.causal && kj > qi)) pv = 0.f;
        pt[qt][e] = pv;
        ds[qt][e] = pv * (pa[e] - delta_s[qr]);
      }
    }
    // dV^T += dO^T P ; dK^T += Q^T dS   (k index = queries, permuted)
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      frag pb, sb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pb[e] = (T)pt[2 * qs][e];
        pb[4 + e] = (T)pt[2 * qs + 1][e];
        sb[e] = (T)ds[2 * qs][e];
        sb[4 + e] = (T)ds[2 * qs + 1][e];
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const frag dof = perm_frag<T>(dOt, dt * 16 + lr, 2 * qs, 2 * qs + 1, lg);
        const frag qtf = perm_frag<T>(Qt, dt * 16 + lr, 2 * qs, 2 * qs + 1, lg);
        dva[dt] = Mfma<T>::mma(dof, pb, dva[dt]);
        dka[dt] = Mfma<T>::mma(qtf, sb, dka[dt]);
      }
    }
  }
  if (kj >= f.Skv) return;
  T* dK = (T*)p.dk + b * p.dk_b + h * p.dk_h + kj * p.dk_s;
  T* dV = (T*)p.dv + b * p.dv_b + h * p.dv_h + kj * p.dv_s;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    V4<T> k4, v4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      k4.v[e] = (T)(dka[dt][e] * f.scale);
      v4.v[e] = (T)dva[dt][e];
    }
    *(V4<T>*)(dK + dt * 16 + lg * 4) = k4;
    *(V4<T>*)(dV + dt * 16 + lg * 4) = v4;
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(kThreads) attn_bwd_dq(AttnBwdArgs p) {
  typedef typename Mfma<T>::frag frag;
  constexpr int KS = D / 32, DT = D / 16;
  __shared__ __attribute__((aligned(16))) T Ks[64 * (D + 8)];
  __shared__ __attribute__((aligned(16))) T Kt[D * 72];
  __shared__ __attribute__((aligned(16))) T Vs[64 * (D + 8)];

  const AttnArgs& f = p.f;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  const BlockCoord bc = block_coord();
  const int64_t qblock = f.causal ? (int64_t)gridDim.x - 1 - bc.x : bc.x;
  const int64_t q0 = qblock * 64;
  const int64_t b = bc.b, h = bc.h;
  const T* Q = (const T*)f.q + b * f.q_b + h * f.q_h;
  const T* K = (const T*)f.k + b * f.k_b + h * f.k_h;
  const T* V = (const T*)f.v + b * f.v_b + h * f.v_h;
  const T* dO = (const T*)p.dout + b * p.do_b + h * p.do_h;

  const int64_t qi = q0 + wave * 16 + lr;  // this lane's query (MFMA column)
  const bool qok = qi < f.Sq;
  frag qf[KS], df[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[ks] = qok ? *(const frag*)(Q + qi * f.q_s + ks * 32 + lg * 8) : zero_frag<T>();
    df[ks] = qok ? *(const frag*)(dO + qi * p.do_s + ks * 32 + lg * 8) : zero_frag<T>();
  }
  const float lse2 = qok ? f.lse[(b * f.H + h) * f.Sq + qi] * kLog2e : 0.f;
  const float dlt = qok ? -p.ndelta[(b * f.H + h) * f.Sq + qi] : 0.f;
  f32x4 dqa[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqa[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  int64_t kv_end = f.Skv;
  if (f.causal) kv_end = min(f.Skv, q0 + 64);
  for (int64_t kb0 = 0; kb0 < kv_end; kb0 += 64) {
    __syncthreads();
    stage_tile<T, D>(Ks, Kt, K, f.k_s, kb0, f.Skv);
    stage_tile<T, D>(Vs, nullptr, V, f.v_s, kb0, f.Skv);
    __syncthreads();
    f32x4 ds[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4 sa = {0.f, 0.f, 0.f, 0.f}, pa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const frag ka = *(const frag*)(Ks + (kt * 16 + lr) * (D + 8) + ks * 32 + lg * 8);
        const frag va = *(const frag*)(Vs + (kt * 16 + lr) * (D + 8) + ks * 32 + lg * 8);
        sa = Mfma<T>::mma(ka, qf[ks], sa);
        pa = Mfma<T>::mma(va, df[ks], pa);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t kj = kb0 + kt * 16 + lg * 4 + e;
        float pv = exp2f(sa[e] * f.scale_log2 - lse2);
        if (!qok || kj >= f.Skv || (f.causal && kj > qi)) pv = 0.f;
        ds[kt][e] = pv * (pa[e] - dlt);
      }
    }
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
      frag sb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sb[e] = (T)ds[2 * ks2][e];
        sb[4 + e] = (T)ds[2 * ks2 + 1][e];
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const frag kf = perm_frag<T>(Kt, dt * 16 + lr, 2 * ks2, 2 * ks2 + 1, lg);
        dqa[dt] = Mfma<T>::mma(kf, sb, dqa[dt]);
      }
    }
  }
  if (!qok) return;
  T* dQ = (T*)p.dq + b * p.dq_b + h * p.dq_h + qi * p.dq_s;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    V4<T> q4;
#pragma unroll
    for (int e = 0; e < 4; ++e) q4.v[e] = (T)(dqa[dt][e] * f.scale);
    *(V4<T>*)(dQ + dt * 16 + lg * 4) = q4;
  }
}

// ---------------------------------------------------------------------------
// backward, head_dim 64/128: direct-to-LDS staging + transposing reads.
//
// dK/dV: a block owns 128 keys (32 per wave, held as MFMA B operands in
// registers).  Per 64-query block it stages Q, dO, LSE and D (the row terms)
// into LDS with direct loads, double-buffered, then per pair of 16-query
// tiles computes S and dP (query tile = MFMA rows, keys = columns), P and dS
// in registers, and accumulates dV^T += dO^T P and dK^T += Q^T dS with the
// dO^T / Q^T operands read transposed from the row-major tiles.
// dQ: a block owns 128 queries (32 per wave); per 64-key block it stages K
// and V, computes S^T and dP^T (key tile = MFMA rows, queries = columns) and
// accumulates dQ^T += K^T dS^T with K^T read transposed.
// ---------------------------------------------------------------------------
template <int D>
constexpr int kDkvLds = 2 * (2 * KvLayout<D>::TILE + 512);  // 2 stages of Q, dO, LSE[64], D[64]
template <int D>
constexpr int kDqLds = 2 * (2 * KvLayout<D>::TILE);  // 2 stages of K, V

template <typename T, int D>
__device__ __forceinline__ void dkv_body(const AttnBwdArgs& p, GridPos gp, char* lds) {
  typedef typename Mfma<T>::frag frag;
  typedef KvLayout<D> L;
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int STAGE = 2 * L::TILE + 512;  // Q tile, dO tile, LSE[64], D[64]

  const AttnArgs& f = p.f;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  const BlockCoord bc = block_coord(gp);
  const int64_t k0 = bc.x * 128;
  const int64_t b = bc.b, h = bc.h;
  const char* Q = (const char*)((const T*)f.q + b * f.q_b + h * f.q_h);
  const T* K = (const T*)f.k + b * f.k_b + h * f.k_h;
  const T* V = (const T*)f.v + b * f.v_b + h * f.v_h;
  const char* dO = (const char*)((const T*)p.dout + b * p.do_b + h * p.do_h);
  const float* LSE = p.nlse2 + (b * f.H + h) * f.Sq;   // -LSE * log2(e)
  const float* DEL = p.ndelta + (b * f.H + h) * f.Sq;  // -D
  const int64_t qs_b = f.q_s * (int64_t)sizeof(T), dos_b = p.do_s * (int64_t)sizeof(T);

  const int64_t kw = k0 + wave * 32;
  frag kf[2][KS], vf[2][KS];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t kj = kw + t * 16 + lr;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kf[t][ks] = kj < f.Skv ? *(const frag*)(K + kj * f.k_s + ks * 32 + lg * 8) : zero_frag<T>();
      vf[t][ks] = kj < f.Skv ? *(const frag*)(V + kj * f.v_s + ks * 32 + lg * 8) : zero_frag<T>();
    }
  }
  f32x4 dva[DT][2], dka[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    dva[dt][0] = dva[dt][1] = dka[dt][0] = dka[dt][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  KvTileLoad<D, 4> ql, dl;
  ql.init(Q, qs_b);
  dl.init(dO, dos_b);
  auto issue = [&](int64_t qb0, char* st) {
    ql.issue(qb0, f.Sq, st);
    dl.issue(qb0, f.Sq, st + L::TILE);
    if (wave < 2) {
      int64_t qi = qb0 + lane;
      if (qi >= f.Sq) qi = f.Sq - 1;
      const float* src = (wave == 0 ? LSE : DEL) + qi;
      dma_b32(src, lds_base_of(st + 2 * L::TILE + wave * 256));
    }
  };

  const int64_t qstart = f.causal ? (k0 / 64) * 64 : 0;
  const int sw = L::swz(lr);
  const TrOffsets<D> tro;
  int buf = 0;
  if (qstart < f.Sq) issue(qstart, lds);
  // One step per 64 queries.  Masks are needed only where the tile crosses
  // this wave's causal diagonal (the first steps), the query end (the last
  // step) or the key end (every step); the steps are split into three loops
  // (masked, unmasked, masked) so the unmasked ones carry no mask code.  All
  // waves run the same number of steps, hence of barriers.
  auto step = [&](int64_t j, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int64_t qb0 = qstart + j * 64;
    __builtin_amdgcn_s_waitcnt(0xc07f & 0x3f70);  // vmcnt(0)
    __syncthreads();
    if (qb0 + 64 < f.Sq) issue(qb0 + 64, lds + (buf ^ 1) * STAGE);
    const char* Qt = lds + buf * STAGE;
    const char* dOt = Qt + L::TILE;
    const float* lse_s = (const float*)(Qt + 2 * L::TILE);
    const float* del_s = lse_s + 64;
    buf ^= 1;
    if (f.causal && kw > qb0 + 63) return;  // every key of this wave is after every query
      const int q_lim = (int)min((int64_t)64, f.Sq - qb0);   // query rows < q_lim exist
      const int k_lim = (int)min((int64_t)32, f.Skv - kw);   // key rows < k_lim exist
      const int kq = (int)max((int64_t)-128, min((int64_t)128, kw - qb0));  // key row 0 minus query row 0
      const float c = f.scale_log2;
      // Masked steps keep query row qr of key row kr iff lo[t] <= qr <
      // q_lim (lo = the causal diagonal), tested as one unsigned compare
      // (qr - lo[t]) < span[t]; a dropped score's exponent is -inf, so the
      // exp2 runs unconditionally and gives 0 (no branch per element).
      int lo[2], span[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int kr = t * 16 + lr;
        lo[t] = f.causal ? max(0, kq + kr) : 0;
        span[t] = kr < k_lim ? max(0, q_lim - lo[t]) : 0;
      }
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) {
        // on the causal diagonal, a pair of query tiles that lies wholly
        // before this wave's first key contributes nothing
        if (MASK && f.causal && qs * 32 + 31 < kq) continue;
        f32x4 pt[2][2], ds[2][2];  // [query tile in pair][key tile]
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int qt = 2 * qs + u;
          frag qa[KS], da[KS];
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const int off = (qt * 16 + lr) * L::ROWB + (((ks * 4 + lg) ^ sw) << 4);
            qa[ks] = *(const frag*)(Qt + off);
            da[ks] = *(const frag*)(dOt + off);
          }
          const float4 l4 = *(const float4*)(lse_s + qt * 16 + 4 * lg);
          const float4 d4 = *(const float4*)(del_s + qt * 16 + 4 * lg);
          const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            // dP - D: the accumulator of dO V^T starts at -D
            f32x4 sa = {0.f, 0.f, 0.f, 0.f}, pa = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
              sa = Mfma<T>::mma(qa[ks], kf[t][ks], sa);
              pa = Mfma<T>::mma(da[ks], vf[t][ks], pa);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float x = fmaf(sa[e], c, lv[e]);
              if constexpr (MASK) {
                const int qr = qt * 16 + 4 * lg + e;
                x = (unsigned)(qr - lo[t]) < (unsigned)span[t] ? x : -INFINITY;
              }
              const float pv = fast_exp2(x);
              pt[u][t][e] = pv;
              ds[u][t][e] = pv * pa[e];
            }
          }
        }
        frag pb[2], sb[2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pb[t][e] = (T)pt[0][t][e];
            pb[t][4 + e] = (T)pt[1][t][e];
            sb[t][e] = (T)ds[0][t][e];
            sb[t][4 + e] = (T)ds[1][t][e];
          }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const frag dof = tr_frag_at<T, D>(dOt, tro, dt, 2 * qs, 2 * qs + 1);
          const frag qtf = tr_frag_at<T, D>(Qt, tro, dt, 2 * qs, 2 * qs + 1);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            dva[dt][t] = Mfma<T>::mma(dof, pb[t], dva[dt][t]);
            dka[dt][t] = Mfma<T>::mma(qtf, sb[t], dka[dt][t]);
          }
        }
      }
  };
  const int64_t nqb = qstart < f.Sq ? (f.Sq - qstart + 63) / 64 : 0;
  int64_t j1 = 0, j2 = nqb;  // masked [0, j1), unmasked [j1, j2), masked [j2, nqb)
  if (kw + 32 > f.Skv) {
    j1 = nqb;
  } else {
    if (f.causal) j1 = min(nqb, max((int64_t)0, ceil_div64(kw + 31 - qstart, 64)));
    j2 = max(j1, min(nqb, (f.Sq - qstart) / 64));
  }
  int64_t j = 0;
  for (; j < j1; ++j) step(j, BoolTag<true>{});
  for (; j < j2; ++j) step(j, BoolTag<false>{});
  for (; j < nqb; ++j) step(j, BoolTag<true>{});
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t kj = kw + t * 16 + lr;
    if (kj >= f.Skv) continue;
    T* dK = (T*)p.dk + b * p.dk_b + h * p.dk_h + kj * p.dk_s;
    T* dV = (T*)p.dv + b * p.dv_b + h * p.dv_h + kj * p.dv_s;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      V4<T> k4, v4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        k4.v[e] = (T)(dka[dt][t][e] * f.scale);
        v4.v[e] = (T)dva[dt][t][e];
      }
      *(V4<T>*)(dK + dt * 16 + lg * 4) = k4;
      *(V4<T>*)(dV + dt * 16 + lg * 4) = v4;
    }
  }
}

template <typename T, int D>
__device__ __forceinline__ void dq_body(const AttnBwdArgs& p, GridPos gp, char* lds) {
  typedef typename Mfma<T>::frag frag;
  typedef KvLayout<D> L;
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int STAGE = 2 * L::TILE;  // K tile, V tile

  const AttnArgs& f = p.f;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  const BlockCoord bc = block_coord(gp);
  const int64_t qblock = f.causal ? (int64_t)gp.nx - 1 - bc.x : bc.x;
  const int64_t q0 = qblock * 128;
  const int64_t b = bc.b, h = bc.h;
  const T* Q = (const T*)f.q + b * f.q_b + h * f.q_h;
  const char* K = (const char*)((const T*)f.k + b * f.k_b + h * f.k_h);
  const char* V = (const char*)((const T*)f.v + b * f.v_b + h * f.v_h);
  const T* dO = (const T*)p.dout + b * p.do_b + h * p.do_h;
  const int64_t ks_b = f.k_s * (int64_t)sizeof(T), vs_b = f.v_s * (int64_t)sizeof(T);

  const int64_t qw = q0 + wave * 32;
  frag qf[2][KS], df[2][KS];
  float lse2[2], dlt[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t qi = qw + u * 16 + lr;
    const bool ok = qi < f.Sq;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[u][ks] = ok ? *(const frag*)(Q + qi * f.q_s + ks * 32 + lg * 8) : zero_frag<T>();
      df[u][ks] = ok ? *(const frag*)(dO + qi * p.do_s + ks * 32 + lg * 8) : zero_frag<T>();
    }
    lse2[u] = ok ? p.nlse2[(b * f.H + h) * f.Sq + qi] : 0.f;  // -LSE * log2(e)
    dlt[u] = ok ? p.ndelta[(b * f.H + h) * f.Sq + qi] : 0.f;  // -D, the start of dP - D
  }
  f32x4 dqa[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqa[dt][0] = dqa[dt][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  int64_t kv_end = f.Skv;
  if (f.causal) kv_end = min(f.Skv, q0 + 128);
  const int sw = L::swz(lr);
  const TrOffsets<D> tro;
  int buf = 0;
  KvTileLoad<D, 4> kl, vl;
  kl.init(K, ks_b);
  vl.init(V, vs_b);
  kl.issue(0, f.Skv, lds);
  vl.issue(0, f.Skv, lds + L::TILE);
  // One step per 64 keys: unmasked steps first, then the ones that cross
  // this wave's causal diagonal or the key end (or all of them when the
  // wave's queries cross the query end); same step count on every wave.
  auto step = [&](int64_t j, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int64_t kb0 = j * 64;
    __builtin_amdgcn_s_waitcnt(0xc07f & 0x3f70);  // vmcnt(0)
    __syncthreads();
    if (kb0 + 64 < kv_end) {
      char* nx = lds + (buf ^ 1) * STAGE;
      kl.issue(kb0 + 64, f.Skv, nx);
      vl.issue(kb0 + 64, f.Skv, nx + L::TILE);
    }
    const char* Kt = lds + buf * STAGE;
    const char* Vt = Kt + L::TILE;
    buf ^= 1;
    if (f.causal && kb0 > qw + 31) return;  // every key after every query of this wave
      const int q_lim = (int)min((int64_t)32, f.Sq - qw);    // query rows < q_lim exist
      const int k_lim = (int)min((int64_t)64, f.Skv - kb0);  // key rows < k_lim exist
      const int qk = (int)max((int64_t)-128, min((int64_t)128, qw - kb0));  // query row 0 minus key row 0
      const float c = f.scale_log2;
      // Masked steps keep key row kr of query row qr iff kr < lim[u]
      // (the key end, the causal diagonal, nothing past the query end); a
      // dropped score's exponent is -inf (no branch per element).
      int lim[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int qr = u * 16 + lr;
        lim[u] = qr < q_lim ? (f.causal ? min(k_lim, qk + qr + 1) : k_lim) : 0;
      }
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        // on the causal diagonal, a pair of key tiles that lies wholly after
        // this wave's last query contributes nothing
        if (MASK && f.causal && ks2 * 32 > qk + 31) continue;
        f32x4 ds[2][2];  // [key tile in pair][query tile]
#pragma unroll
        for (int v2 = 0; v2 < 2; ++v2) {
          const int kt = 2 * ks2 + v2;
          frag ka[KS], va[KS];
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const int off = (kt * 16 + lr) * L::ROWB + (((ks * 4 + lg) ^ sw) << 4);
            ka[ks] = *(const frag*)(Kt + off);
            va[ks] = *(const frag*)(Vt + off);
          }
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            f32x4 sa = {0.f, 0.f, 0.f, 0.f}, pa = {dlt[u], dlt[u], dlt[u], dlt[u]};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
              sa = Mfma<T>::mma(ka[ks], qf[u][ks], sa);
              pa = Mfma<T>::mma(va[ks], df[u][ks], pa);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float x = fmaf(sa[e], c, lse2[u]);
              if constexpr (MASK) x = kt * 16 + 4 * lg + e < lim[u] ? x : -INFINITY;
              ds[v2][u][e] = fast_exp2(x) * pa[e];
            }
          }
        }
        frag sb[2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sb[u][e] = (T)ds[0][u][e];
            sb[u][4 + e] = (T)ds[1][u][e];
          }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const frag ktf = tr_frag_at<T, D>(Kt, tro, dt, 2 * ks2, 2 * ks2 + 1);
#pragma unroll
          for (int u = 0; u < 2; ++u) dqa[dt][u] = Mfma<T>::mma(ktf, sb[u], dqa[dt][u]);
        }
      }
  };
  const int64_t nkb = (kv_end + 63) / 64;
  int64_t ju = 0;  // unmasked [0, ju), masked [ju, nkb)
  if (qw + 32 <= f.Sq) {
    ju = min(nkb, f.Skv / 64);
    if (f.causal) ju = min(ju, qw < 63 ? (int64_t)0 : (qw - 63) / 64 + 1);
  }
  int64_t j = 0;
  for (; j < ju; ++j) step(j, BoolTag<false>{});
  for (; j < nkb; ++j) step(j, BoolTag<true>{});
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t qi = qw + u * 16 + lr;
    if (qi >= f.Sq) continue;
    T* dQ = (T*)p.dq + b * p.dq_b + h * p.dq_h + qi * p.dq_s;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      V4<T> q4;
#pragma unroll
      for (int e = 0; e < 4; ++e) q4.v[e] = (T)(dqa[dt][u][e] * f.scale);
      *(V4<T>*)(dQ + dt * 16 + lg * 4) = q4;
    }
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(kThreads, D == 64 ? ATTN_BWD_WAVES : 1) attn_bwd_dkv_v2(AttnBwdArgs p) {
  __shared__ __attribute__((aligned(1024))) char lds[kDkvLds<D>];
  dkv_body<T, D>(p, hw_grid(), lds);
}

template <typename T, int D>
__global__ void __launch_bounds__(kThreads, D == 64 ? ATTN_BWD_WAVES : 1) attn_bwd_dq_v2(AttnBwdArgs p) {
  __shared__ __attribute__((aligned(1024))) char lds[kDqLds<D>];
  dq_body<T, D>(p, hw_grid(), lds);
}

// dK/dV and dQ blocks from one launch over a 1-D grid of 2 x (tiles x H x B)
// blocks.  The two kinds alternate inside each XCD's share of the grid, so
// both keep their XCD-aware, heaviest-first order and the light blocks of
// one kind fill the causal tail left by the heavy blocks of the other.
// Block l runs on XCD l % 8; its slot i = l / 8 within that XCD carries the
// kind and virtual id w * 8 + l % 8 keeps the XCD (w: the slot's rank among
// the slots of its kind).  Each XCD deals its slots to its four shader
// engines in turn, in order (i % 4 picks the engine), and waits for the
// engine whose turn it is to have room: with the kind in bit 0 of i, two
// engines got every dK/dV block and two every dQ block, and the dQ engines
// idled while the heavier dK/dV blocks held the dispatch (probe of block
// start and end times at config 1: 4-5 us stalls after each round).  The
// kind sits in bit 2 instead when the XCD's slot count allows, so every
// engine alternates between the kinds.
#ifndef ATTN_BWD_KIND_BIT
#define ATTN_BWD_KIND_BIT 2
#endif
template <typename T, int D>
__global__ void __launch_bounds__(kThreads, D == 64 ? ATTN_BWD_WAVES : 1) attn_bwd_dkv_dq(AttnBwdArgs p, uint32_t nkx, uint32_t nqx) {
  __shared__ __attribute__((aligned(1024))) char lds[kDkvLds<D> > kDqLds<D> ? kDkvLds<D> : kDqLds<D>];
  const uint32_t l = blockIdx.x, i = l >> 3;
  constexpr uint32_t KB = ATTN_BWD_KIND_BIT;
  // slots per XCD: gridDim.x / 8; bit KB needs them in whole groups of 2 << KB
  const bool hi = ((gridDim.x >> 3) & ((2u << KB) - 1)) == 0;
  const uint32_t kind = hi ? (i >> KB) & 1 : i & 1;
  const uint32_t w = hi ? ((i >> (KB + 1)) << KB) | (i & ((1u << KB) - 1)) : i >> 1;
  const uint32_t v = w * 8 + (l & 7);
  if (kind) dq_body<T, D>(p, GridPos{nqx, (uint32_t)p.f.H, (uint32_t)p.f.B, v}, lds);
  else dkv_body<T, D>(p, GridPos{nkx, (uint32_t)p.f.H, (uint32_t)p.f.B, v}, lds);
}

// ---------------------------------------------------------------------------
// backward with grouped K/V heads and sliding windows (MFMA), head_dim
// 64/128/256
//
// dK/dV: a block owns 64 keys of one K/V head (a wave 16, their K and V rows
// held in registers) and walks, for each of the group's query heads, the
// 64-query steps that can see them (causal: query >= key; window w: query <
// key + w), staging Q, dO and the row terms of the step through LDS; the
// group's contributions add up in the same accumulators, so dK and dV of a
// K/V head are the sums over its query heads without atomics.
// dQ: a block owns 64 queries of one query head (a wave 16) and walks the
// visible 64-key steps of its K/V head.
// Per step and wave the visible (query, key) pairs are one interval of query
// rows per key (dK/dV) or of key rows per query (dQ), tested with a single
// unsigned compare; steps wholly inside every wave's visible band skip the
// test, and pairs of 16-row tiles wholly outside it skip their MFMAs.
// ---------------------------------------------------------------------------
template <int D>
constexpr int kGqaDkvLds = 2 * (2 * KvLayout<D>::TILE + 512);  // 2 stages of Q, dO, -LSE log2e[64], -D[64]
template <int D>
constexpr int kGqaDqLds = 2 * (2 * KvLayout<D>::TILE);  // 2 stages of K, V

template <typename T, int D>
__global__ void __launch_bounds__(kThreads, 1) attn_bwd_gqa_dkv(AttnBwdArgs p) {
  typedef typename Mfma<T>::frag frag;
  typedef KvLayout<D> L;
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int STAGE = 2 * L::TILE + 512;
  char* const lds = attn_dyn_lds;
  const AttnArgs& f = p.f;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  const int64_t k0 = (int64_t)blockIdx.x * 64;
  // with partials, block (x, hk * group + gi) takes query head gi of the
  // group alone; without, it walks the whole group
  const int64_t hsplit = p.kv_part ? f.group : 1;
  const int64_t hk = blockIdx.y / hsplit, gfirst = blockIdx.y - hk * hsplit, b = blockIdx.z;
  const int64_t kw = k0 + wave * 16, kj = kw + lr;
  const T* K = (const T*)f.k + b * f.k_b + hk * f.k_h;
  const T* V = (const T*)f.v + b * f.v_b + hk * f.v_h;
  frag kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kf[ks] = kj < f.Skv ? *(const frag*)(K + kj * f.k_s + ks * 32 + lg * 8) : zero_frag<T>();
    vf[ks] = kj < f.Skv ? *(const frag*)(V + kj * f.v_s + ks * 32 + lg * 8) : zero_frag<T>();
  }
  f32x4 dva[DT], dka[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dva[dt] = dka[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // queries that can see keys k0 .. k0 + 63, in 64-query steps from qstart
  int64_t qhi = f.Sq;
  if (f.window > 0) qhi = min(qhi, k0 + 63 + f.window);
  const int64_t qstart = f.causal ? (k0 / 64) * 64 : 0;
  const int64_t nqb = qhi > qstart ? (qhi - qstart + 63) / 64 : 0;
  const int64_t nheads = p.kv_part ? 1 : f.group;
  const int64_t total = nqb * nheads;  // steps over (query head, query block)
  const int64_t qs_b = f.q_s * (int64_t)sizeof(T), dos_b = p.do_s * (int64_t)sizeof(T);
  KvTileLoad<D, 4> ql, dl;
  ql.init(nullptr, qs_b);
  dl.init(nullptr, dos_b);
  auto issue = [&](int64_t st, char* dst) {
    const int64_t gi = st / nqb, qb0 = qstart + (st - gi * nqb) * 64;
    const int64_t h = hk * f.group + gfirst + gi;
    ql.g = (const char*)((const T*)f.q + b * f.q_b + h * f.q_h);
    dl.g = (const char*)((const T*)p.dout + b * p.do_b + h * p.do_h);
    ql.issue(qb0, f.Sq, dst);
    dl.issue(qb0, f.Sq, dst + L::TILE);
    if (wave < 2) {
      const int64_t qi = min(qb0 + lane, f.Sq - 1);
      const float* src = (wave == 0 ? p.nlse2 : p.ndelta) + (b * f.H + h) * f.Sq + qi;
      dma_b32(src, lds_base_of(dst + 2 * L::TILE + wave * 256));
    }
  };
  const int sw = L::swz(lr);
  const TrOffsets<D> tro;
  const float c = f.scale_log2;
  auto compute = [&](const char* Qt, int64_t qb0, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const char* dOt = Qt + L::TILE;
    const float* lse_s = (const float*)(Qt + 2 * L::TILE);
    const float* del_s = lse_s + 64;
    const int64_t kq = kw - qb0;  // key row 0 minus query row 0
    // query rows lo <= qr < lo + span see this lane's key
    int lo = 0, span = 64;
    if constexpr (MASK) {
      const int64_t lo64 = f.causal ? max((int64_t)0, kq + lr) : 0;
      int64_t hi = min((int64_t)64, f.Sq - qb0);
      if (f.window > 0) hi = min(hi, kq + lr + f.window);
      lo = (int)min((int64_t)64, lo64);
      span = kj < f.Skv ? (int)max((int64_t)0, hi - lo64) : 0;
    }
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      if (MASK && f.causal && qs * 32 + 31 < kq) continue;                // every query before every key
      if (MASK && f.window > 0 && qs * 32 >= kq + 15 + f.window) continue;  // past every key's window
      f32x4 pt[2], ds[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int qt = 2 * qs + u;
        const float4 l4 = *(const float4*)(lse_s + qt * 16 + 4 * lg);
        const float4 d4 = *(const float4*)(del_s + qt * 16 + 4 * lg);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, pa = {d4.x, d4.y, d4.z, d4.w};  // dP - D
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int off = (qt * 16 + lr) * L::ROWB + (((ks * 4 + lg) ^ sw) << 4);
          sa = Mfma<T>::mma(*(const frag*)(Qt + off), kf[ks], sa);
          pa = Mfma<T>::mma(*(const frag*)(dOt + off), vf[ks], pa);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = fmaf(sa[e], c, lv[e]);
          if constexpr (MASK) x = (unsigned)(qt * 16 + 4 * lg + e - lo) < (unsigned)span ? x : -INFINITY;
          const float pv = fast_exp2(x);
          pt[u][e] = pv;
          ds[u][e] = pv * pa[e];
        }
      }
      frag pb, sb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pb[e] = (T)pt[0][e];
        pb[4 + e] = (T)pt[1][e];
        sb[e] = (T)ds[0][e];
        sb[4 + e] = (T)ds[1][e];
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        dva[dt] = Mfma<T>::mma(tr_frag_at<T, D>(dOt, tro, dt, 2 * qs, 2 * qs + 1), pb, dva[dt]);
        dka[dt] = Mfma<T>::mma(tr_frag_at<T, D>(Qt, tro, dt, 2 * qs, 2 * qs + 1), sb, dka[dt]);
      }
    }
  };
  int buf = 0;
  if (total > 0) issue(0, lds);
  for (int64_t st = 0; st < total; ++st) {
    __builtin_amdgcn_s_waitcnt(0xc07f & 0x3f70);  // vmcnt(0)
    __syncthreads();
    if (st + 1 < total) issue(st + 1, lds + (buf ^ 1) * STAGE);
    const char* Qt = lds + buf * STAGE;
    buf ^= 1;
    const int64_t qb0 = qstart + (st % nqb) * 64;
    if (f.causal && kw > qb0 + 63) continue;                     // every query before every key
    if (f.window > 0 && qb0 >= kw + 15 + f.window) continue;     // past every key's window
    const bool inside = (!f.causal || qb0 >= kw + 15) && (f.window <= 0 || qb0 + 63 < kw + f.window) &&
                        qb0 + 64 <= f.Sq && kw + 16 <= f.Skv;
    if (inside) compute(Qt, qb0, BoolTag<false>{});
    else compute(Qt, qb0, BoolTag<true>{});
  }
  if (kj < f.Skv && p.kv_part) {
    // f32 partials [gi][b][hk][key][D], dK's then dV's; summed by attn_bwd_gqa_sum
    const int64_t hkn = f.H / f.group, plane = f.group * f.B * hkn * f.Skv * D;
    float* pk = p.kv_part + (((gfirst * f.B + b) * hkn + hk) * f.Skv + kj) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      *(float4*)(pk + dt * 16 + lg * 4) = float4{dka[dt][0], dka[dt][1], dka[dt][2], dka[dt][3]};
      *(float4*)(pk + plane + dt * 16 + lg * 4) = float4{dva[dt][0], dva[dt][1], dva[dt][2], dva[dt][3]};
    }
  } else if (kj < f.Skv) {
    T* dK = (T*)p.dk + b * p.dk_b + hk * p.dk_h + kj * p.dk_s;
    T* dV = (T*)p.dv + b * p.dv_b + hk * p.dv_h + kj * p.dv_s;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      V4<T> k4, v4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        k4.v[e] = (T)(dka[dt][e] * f.scale);
        v4.v[e] = (T)dva[dt][e];
      }
      *(V4<T>*)(dK + dt * 16 + lg * 4) = k4;
      *(V4<T>*)(dV + dt * 16 + lg * 4) = v4;
    }
  }
}

// dK = scale * sum over the group's query heads of the dK partials, dV = the
// sum of the dV partials, in head order (deterministic); four head-dim
// elements per thread.
template <typename T, int D>
__global__ void __launch_bounds__(kThreads) attn_bwd_gqa_sum(AttnBwdArgs p) {
  const AttnArgs& f = p.f;
  const int64_t hkn = f.H / f.group, rows = f.B * hkn * f.Skv, plane = f.group * rows * D;
  const int64_t i4 = (int64_t)blockIdx.x * kThreads + threadIdx.x;  // over rows * D / 4
  if (i4 >= rows * (D / 4)) return;
  const int64_t row = i4 / (D / 4), d = (i4 - row * (D / 4)) * 4;
  const int64_t key = row % f.Skv, bh = row / f.Skv, hk = bh % hkn, b = bh / hkn;
  float4 sk = {0.f, 0.f, 0.f, 0.f}, sv = sk;
  for (int64_t g = 0; g < f.group; ++g) {
    const float4 a = *(const float4*)(p.kv_part + g * rows * D + row * D + d);
    const float4 c = *(const float4*)(p.kv_part + plane + g * rows * D + row * D + d);
    sk.x += a.x, sk.y += a.y, sk.z += a.z, sk.w += a.w;
    sv.x += c.x, sv.y += c.y, sv.z += c.z, sv.w += c.w;
  }
  V4<T> k4, v4;
  k4.v[0] = (T)(sk.x * f.scale), k4.v[1] = (T)(sk.y * f.scale), k4.v[2] = (T)(sk.z * f.scale), k4.v[3] = (T)(sk.w * f.scale);
  v4.v[0] = (T)sv.x, v4.v[1] = (T)sv.y, v4.v[2] = (T)sv.z, v4.v[3] = (T)sv.w;
  *(V4<T>*)((T*)p.dk + b * p.dk_b + hk * p.dk_h + key * p.dk_s + d) = k4;
  *(V4<T>*)((T*)p.dv + b * p.dv_b + hk * p.dv_h + key * p.dv_s + d) = v4;
}

template <typename T, int D>
__global__ void __launch_bounds__(kThreads, 1) attn_bwd_gqa_dq(AttnBwdArgs p) {
  typedef typename Mfma<T>::frag frag;
  typedef KvLayout<D> L;
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int STAGE = 2 * L::TILE;
  char* const lds = attn_dyn_lds;
  const AttnArgs& f = p.f;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int lr = lane & 15, lg = lane >> 4;
  // causal: the heaviest query blocks first
  const int64_t qblock = f.causal && f.window <= 0 ? (int64_t)gridDim.x - 1 - blockIdx.x : blockIdx.x;
  const int64_t q0 = qblock * 64;
  const int64_t h = blockIdx.y, b = blockIdx.z, hk = h / f.group;
  const int64_t qw = q0 + wave * 16, qi = qw + lr;
  const bool qok = qi < f.Sq;
  const T* Q = (const T*)f.q + b * f.q_b + h * f.q_h;
  const T* dO = (const T*)p.dout + b * p.do_b + h * p.do_h;
  frag qf[KS], df[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[ks] = qok ? *(const frag*)(Q + qi * f.q_s + ks * 32 + lg * 8) : zero_frag<T>();
    df[ks] = qok ? *(const frag*)(dO + qi * p.do_s + ks * 32 + lg * 8) : zero_frag<T>();
  }
  const float nl2 = qok ? p.nlse2[(b * f.H + h) * f.Sq + qi] : 0.f;   // -LSE log2e
  const float ndl = qok ? p.ndelta[(b * f.H + h) * f.Sq + qi] : 0.f;  // -D, the start of dP - D
  f32x4 dqa[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqa[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  int64_t khi = f.Skv;
  if (f.causal) khi = min(khi, q0 + 64);
  const int64_t klo = f.window > 0 ? max((int64_t)0, q0 - f.window + 1) : 0;
  const int64_t kstart = (klo / 64) * 64;
  const int64_t nkb = khi > kstart ? (khi - kstart + 63) / 64 : 0;
  KvTileLoad<D, 4> kl, vl;
  kl.init((const char*)((const T*)f.k + b * f.k_b + hk * f.k_h), f.k_s * (int64_t)sizeof(T));
  vl.init((const char*)((const T*)f.v + b * f.v_b + hk * f.v_h), f.v_s * (int64_t)sizeof(T));
  const int sw = L::swz(lr);
  const TrOffsets<D> tro;
  const float c = f.scale_log2;
  auto compute = [&](const char* Kt, int64_t kb0, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const char* Vt = Kt + L::TILE;
    const int64_t qk = qw - kb0;  // query row 0 minus key row 0
    // key rows lo <= kr < lo + span are visible to this lane's query
    int lo = 0, span = 64;
    if constexpr (MASK) {
      const int64_t lo64 = f.window > 0 ? max((int64_t)0, qk + lr - f.window + 1) : 0;
      int64_t hi = min((int64_t)64, f.Skv - kb0);
      if (f.causal) hi = min(hi, qk + lr + 1);
      lo = (int)min((int64_t)64, lo64);
      span = qok ? (int)max((int64_t)0, hi - lo64) : 0;
    }
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
      if (MASK && f.causal && ks2 * 32 > qk + 15) continue;                      // after every query
      if (MASK && f.window > 0 && ks2 * 32 + 31 < qk - f.window + 1) continue;  // before every window
      f32x4 ds[2];
#pragma unroll
      for (int v2 = 0; v2 < 2; ++v2) {
        const int kt = 2 * ks2 + v2;
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, pa = {ndl, ndl, ndl, ndl};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int off = (kt * 16 + lr) * L::ROWB + (((ks * 4 + lg) ^ sw) << 4);
          sa = Mfma<T>::mma(*(const frag*)(Kt + off), qf[ks], sa);
          pa = Mfma<T>::mma(*(const frag*)(Vt + off), df[ks], pa);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float x = fmaf(sa[e], c, nl2);
          if constexpr (MASK) x = (unsigned)(kt * 16 + 4 * lg + e - lo) < (unsigned)span ? x : -INFINITY;
          ds[v2][e] = fast_exp2(x) * pa[e];
        }
      }
      frag sb;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sb[e] = (T)ds[0][e];
        sb[4 + e] = (T)ds[1][e];
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        dqa[dt] = Mfma<T>::mma(tr_frag_at<T, D>(Kt, tro, dt, 2 * ks2, 2 * ks2 + 1), sb, dqa[dt]);
    }
  };
  int buf = 0;
  if (nkb > 0) {
    kl.issue(kstart, f.Skv, lds);
    vl.issue(kstart, f.Skv, lds + L::TILE);
  }
  for (int64_t j = 0; j < nkb; ++j) {
    const int64_t kb0 = kstart + j * 64;
    __builtin_amdgcn_s_waitcnt(0xc07f & 0x3f70);  // vmcnt(0)
    __syncthreads();
    if (j + 1 < nkb) {
      char* nx = lds + (buf ^ 1) * STAGE;
      kl.issue(kb0 + 64, f.Skv, nx);
      vl.issue(kb0 + 64, f.Skv, nx + L::TILE);
    }
    const char* Kt = lds + buf * STAGE;
    buf ^= 1;
    if (f.causal && kb0 > qw + 15) continue;                           // every key after every query
    if (f.window > 0 && kb0 + 63 < qw - f.window + 1) continue;        // before every query's window
    const bool inside = (!f.causal || kb0 + 63 <= qw) && (f.window <= 0 || kb0 > qw + 15 - f.window) &&
                        kb0 + 64 <= f.Skv && qw + 16 <= f.Sq;
    if (inside) compute(Kt, kb0, BoolTag<false>{});
    else compute(Kt, kb0, BoolTag<true>{});
  }
  if (!qok) return;
  T* dQ = (T*)p.dq + b * p.dq_b + h * p.dq_h + qi * p.dq_s;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    V4<T> q4;
#pragma unroll
    for (int e = 0; e < 4; ++e) q4.v[e] = (T)(dqa[dt][e] * f.scale);
    *(V4<T>*)(dQ + dt * 16 + lg * 4) = q4;
  }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------
bool strides_ok(const void* ptr, const int64_t* bhs) {
  return ((uintptr_t)ptr % 16 == 0) && bhs[0] % 8 == 0 && bhs[1] % 8 == 0 && bhs[2] % 8 == 0;
}

int check_common(int64_t B, int64_t H, int64_t Sq, int64_t Skv, int64_t D, int dtype, bool fwd = false) {
  if (dtype != MI355X_BF16 && dtype != MI355X_F16)
    return fail(MI355X_EUNSUPPORTED, "mi355x_attn: dtype %d not supported (bf16/f16 only)", dtype);
  if (D != 32 && D != 64 && D != 128 && !(fwd && D == 256))
    return fail(MI355X_EUNSUPPORTED, "mi355x_attn: head_dim %lld not supported (32/64/128%s)", (long long)D,
                fwd ? "/256" : "; 256 is forward-only");
  if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0 || B >= 65536 || H >= 65536)
    return fail(MI355X_EINVAL, "mi355x_attn: bad shape");
  return MI355X_OK;
}

template <typename T, int D>
int fwd_launch(const AttnArgs& a, hipStream_t s) {
  if constexpr (D == 256) {
    // 64-query blocks of 4 waves x 16 queries; K/V stages need 128 KB of LDS
    constexpr int NW = 4, QPW = 16;
    constexpr size_t kLds = 4 * KvLayout<256>::TILE;
    dim3 grid(ceil_div(a.Sq, NW * QPW), (unsigned)a.H, (unsigned)a.B);
    auto kp = attn_fwd_v2<T, D, true, NW, QPW>;
    auto kn = attn_fwd_v2<T, D, false, NW, QPW>;
    static bool attr = false;
    if (!attr) {
      if (hipFuncSetAttribute((const void*)kp, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds) != hipSuccess ||
          hipFuncSetAttribute((const void*)kn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds) != hipSuccess)
        return fail(MI355X_ELAUNCH, "mi355x_attn_fwd: cannot raise the LDS limit for head_dim 256");
      attr = true;
    }
    if (a.scale_log2 > 0.f) kp<<<grid, 64 * NW, kLds, s>>>(a);
    else kn<<<grid, 64 * NW, kLds, s>>>(a);
    return check_launch("mi355x_attn_fwd");
  }
  dim3 grid(ceil_div(a.Sq, 128), (unsigned)a.H, (unsigned)a.B);
  if constexpr (D == 64 || D == 128) {
    constexpr int NW = D == 64 ? ATTN_FWD_WAVES : 4;
    constexpr int QPW = 128 / NW;
    if (a.scale_log2 > 0.f) attn_fwd_v2<T, D, true, NW, QPW><<<grid, 64 * NW, 0, s>>>(a);
    else attn_fwd_v2<T, D, false, NW, QPW><<<grid, 64 * NW, 0, s>>>(a);
  }
  else if (a.scale_log2 > 0.f) attn_fwd_kernel<T, D, true><<<grid, kThreads, 0, s>>>(a);
  else attn_fwd_kernel<T, D, false><<<grid, kThreads, 0, s>>>(a);
  return check_launch("mi355x_attn_fwd");
}

template <typename T, int D>
int bwd_launch(const AttnBwdArgs& a, hipStream_t s) {
  const int64_t rows = a.f.B * a.f.H * a.f.Sq;
  MI_REQUIRE(rows < (1ll << 31), "mi355x_attn_bwd: batch x heads x query rows must be below 2^31");
  attn_bwd_delta<T, D><<<ceil_div(rows, kThreads / (D / 8)), kThreads, 0, s>>>(a);
  if constexpr (D == 64 || D == 128) {
    const uint32_t nkx = (uint32_t)ceil_div(a.f.Skv, 128), nqx = (uint32_t)ceil_div(a.f.Sq, 128);
    const int64_t hb = a.f.H * a.f.B;
    if (nkx == nqx && (hb * nkx) % 8 == 0) {
      attn_bwd_dkv_dq<T, D><<<(unsigned)(2 * hb * nkx), kThreads, 0, s>>>(a, nkx, nqx);
    } else {
      attn_bwd_dkv_v2<T, D><<<dim3(nkx, (unsigned)a.f.H, (unsigned)a.f.B), kThreads, 0, s>>>(a);
      attn_bwd_dq_v2<T, D><<<dim3(nqx, (unsigned)a.f.H, (unsigned)a.f.B), kThreads, 0, s>>>(a);
    }
  } else {
    dim3 gk(ceil_div(a.f.Skv, 64), (unsigned)a.f.H, (unsigned)a.f.B);
    attn_bwd_dkv<T, D><<<gk, kThreads, 0, s>>>(a);
    dim3 gq(ceil_div(a.f.Sq, 64), (unsigned)a.f.H, (unsigned)a.f.B);
    attn_bwd_dq<T, D><<<gq, kThreads, 0, s>>>(a);
  }
  return check_launch("mi355x_attn_bwd");
}

#define MI_ATTN_FWD_DISPATCH(dtype, D, FN, ...)                               \
  do {                                                                        \
    if (D == 256) {                                                           \
      if (dtype == MI355X_BF16) return FN<bf16, 256>(__VA_ARGS__);            \
      return FN<f16, 256>(__VA_ARGS__);                                       \
    }                                                                         \
    MI_ATTN_DISPATCH(dtype, D, FN, __VA_ARGS__);                              \
  } while (0)

#define MI_ATTN_DISPATCH(dtype, D, FN, ...)                                   \
  do {                                                                        \
    if (dtype == MI355X_BF16) {                                               \
      if (D == 32) return FN<bf16, 32>(__VA_ARGS__);                          \
      if (D == 64) return FN<bf16, 64>(__VA_ARGS__);                          \
      return FN<bf16, 128>(__VA_ARGS__);                                      \
    }                                                                         \
    if (D == 32) return FN<f16, 32>(__VA_ARGS__);                             \
    if (D == 64) return FN<f16, 64>(__VA_ARGS__);                             \
    return FN<f16, 128>(__VA_ARGS__);                                         \
  } while (0)

template <typename T, int D>
int gqa_bwd_launch(const AttnBwdArgs& a, hipStream_t s) {
  const int64_t rows = a.f.B * a.f.H * a.f.Sq;
  MI_REQUIRE(rows < (1ll << 31), "mi355x_attn_bwd: batch x heads x query rows must be below 2^31");
  attn_bwd_delta<T, D><<<ceil_div(rows, kThreads / (D / 8)), kThreads, 0, s>>>(a);
  auto kkv = attn_bwd_gqa_dkv<T, D>;
  auto kq = attn_bwd_gqa_dq<T, D>;
  constexpr int lkv = kGqaDkvLds<D>, lq = kGqaDqLds<D>;
  static std::once_flag once;
  static hipError_t attr_err = hipSuccess;
  std::call_once(once, [&] {
    attr_err = hipFuncSetAttribute((const void*)kkv, hipFuncAttributeMaxDynamicSharedMemorySize, lkv);
    if (attr_err == hipSuccess)
      attr_err = hipFuncSetAttribute((const void*)kq, hipFuncAttributeMaxDynamicSharedMemorySize, lq);
  });
  if (attr_err != hipSuccess)
    return fail(MI355X_ELAUNCH, "mi355x_attn_bwd_gen: cannot raise the LDS limit: %s", hipGetErrorString(attr_err));
  // grouped heads: one dK/dV block per (key block, query head), partials summed after
  const unsigned gy = (unsigned)(a.kv_part ? a.f.H : a.f.H / a.f.group);
  kkv<<<dim3(ceil_div(a.f.Skv, 64), gy, (unsigned)a.f.B), kThreads, lkv, s>>>(a);
  kq<<<dim3(ceil_div(a.f.Sq, 64), (unsigned)a.f.H, (unsigned)a.f.B), kThreads, lq, s>>>(a);
  if (a.kv_part) {
    const int64_t n4 = a.f.B * (a.f.H / a.f.group) * a.f.Skv * (D / 4);
    attn_bwd_gqa_sum<T, D><<<ceil_div(n4, kThreads), kThreads, 0, s>>>(a);
  }
  return check_launch("mi355x_attn_bwd_gen");
}

}  // namespace

// MFMA backward for grouped K/V heads and/or a sliding window, called by
// mi355x_attn_bwd_gen (attention_generic.hip) for bf16/f16 at head_dim
// 64/128/256 with 16-byte aligned operands; returns -1 (nothing launched)
// for inputs it does not take.  The workspace holds 2 floats per query row
// and, with grouped heads, the per-query-head dK/dV partials
// (mi355x_attn_bwd_gen_workspace_bytes).
int attn_bwd_grouped_mfma(void* dq, const int64_t* dq_bhs, void* dk, const int64_t* dk_bhs, void* dv,
                          const int64_t* dv_bhs, const void* dout, const int64_t* do_bhs, const void* q,
                          const int64_t* q_bhs, const void* k, const int64_t* k_bhs, const void* v,
                          const int64_t* v_bhs, const void* o, const int64_t* o_bhs, const float* lse,
                          int64_t batch, int64_t heads, int64_t kv_heads, int64_t sq, int64_t skv, int64_t d,
                          double scale, int causal, int64_t window, int dtype, void* workspace,
                          hipStream_t stream) {
  if ((dtype != MI355X_BF16 && dtype != MI355X_F16) || (d != 64 && d != 128 && d != 256)) return -1;
  if (kv_heads < 1 || heads % kv_heads != 0 || heads / kv_heads > 65535 || batch >= 65536) return -1;
  if (window > 0 && !causal) return -1;
  if (!(strides_ok(q, q_bhs) && strides_ok(k, k_bhs) && strides_ok(v, v_bhs) && strides_ok(dout, do_bhs) &&
        strides_ok(o, o_bhs)))
    return -1;
  for (const int64_t* st : {dq_bhs, dk_bhs, dv_bhs})
    if (st[0] % 4 || st[1] % 4 || st[2] % 4) return -1;
  if (((uintptr_t)dq | (uintptr_t)dk | (uintptr_t)dv) % 8) return -1;
  AttnBwdArgs a;
  a.f = AttnArgs{(void*)o, o_bhs[0], o_bhs[1], o_bhs[2], (float*)lse, q, q_bhs[0], q_bhs[1], q_bhs[2],
                 k, k_bhs[0], k_bhs[1], k_bhs[2], v, v_bhs[0], v_bhs[1], v_bhs[2],
                 batch, heads, sq, skv, (float)(scale * 1.4426950408889634), (float)scale, causal,
                 heads / kv_heads, window};
  a.dout = dout; a.do_b = do_bhs[0]; a.do_h = do_bhs[1]; a.do_s = do_bhs[2];
  a.dq = dq; a.dq_b = dq_bhs[0]; a.dq_h = dq_bhs[1]; a.dq_s = dq_bhs[2];
  a.dk = dk; a.dk_b = dk_bhs[0]; a.dk_h = dk_bhs[1]; a.dk_s = dk_bhs[2];
  a.dv = dv; a.dv_b = dv_bhs[0]; a.dv_h = dv_bhs[1]; a.dv_s = dv_bhs[2];
  a.ndelta = (float*)workspace;
  a.nlse2 = a.ndelta + batch * heads * sq;
  // partials after the row terms, 256-byte aligned (grouped heads only)
  a.kv_part = heads > kv_heads
                  ? (float*)(((uintptr_t)(a.nlse2 + batch * heads * sq) + 255) & ~(uintptr_t)255)
                  : nullptr;
  const bool bf = dtype == MI355X_BF16;
  if (d == 64) return bf ? gqa_bwd_launch<bf16, 64>(a, stream) : gqa_bwd_launch<f16, 64>(a, stream);
  if (d == 128) return bf ? gqa_bwd_launch<bf16, 128>(a, stream) : gqa_bwd_launch<f16, 128>(a, stream);
  return bf ? gqa_bwd_launch<bf16, 256>(a, stream) : gqa_bwd_launch<f16, 256>(a, stream);
}

}  // namespace mi

using namespace mi;

extern "C" int mi355x_attn_fwd_ex(void* o, const int64_t* o_bhs, float* lse, const void* q,
                                  const int64_t* q_bhs, const void* k, const int64_t* k_bhs,
                                  const void* v, const int64_t* v_bhs, int64_t batch, int64_t heads,
                                  int64_t kv_heads, int64_t sq, int64_t skv, int64_t d, double scale,
                                  int causal, int64_t window, int dtype, mi355x_stream_t stream) {
  int rc = check_common(batch, heads, sq, skv, d, dtype, true);
  if (rc) return rc;
  MI_REQUIRE(kv_heads >= 1 && heads % kv_heads == 0,
             "mi355x_attn_fwd_ex: heads (%lld) must be a multiple of kv_heads (%lld)", (long long)heads,
             (long long)kv_heads);
  MI_REQUIRE(window >= 0 && (window == 0 || causal), "mi355x_attn_fwd_ex: a sliding window needs causal attention");
  MI_REQUIRE(d != 32 || (kv_heads == heads && window == 0),
             "mi355x_attn_fwd_ex: head_dim 32 supports neither grouped K/V heads nor a window");
  MI_REQUIRE(strides_ok(q, q_bhs) && strides_ok(k, k_bhs) && strides_ok(v, v_bhs),
             "mi355x_attn_fwd: q/k/v need 16-byte aligned bases and strides that are multiples of 8");
  MI_REQUIRE(((uintptr_t)o % 8 == 0) && o_bhs[0] % 4 == 0 && o_bhs[1] % 4 == 0 && o_bhs[2] % 4 == 0,
             "mi355x_attn_fwd: o needs 8-byte aligned rows");
  AttnArgs a{o, o_bhs[0], o_bhs[1], o_bhs[2], lse, q, q_bhs[0], q_bhs[1], q_bhs[2],
             k, k_bhs[0], k_bhs[1], k_bhs[2], v, v_bhs[0], v_bhs[1], v_bhs[2],
             batch, heads, sq, skv, (float)(scale * 1.4426950408889634), (float)scale, causal,
             heads / kv_heads, window};
  MI_ATTN_FWD_DISPATCH(dtype, d, fwd_launch, a, (hipStream_t)stream);
}

extern "C" int mi355x_attn_fwd(void* o, const int64_t* o_bhs, float* lse, const void* q,
                               const int64_t* q_bhs, const void* k, const int64_t* k_bhs,
                               const void* v, const int64_t* v_bhs, int64_t batch, int64_t heads,
                               int64_t sq, int64_t skv, int64_t d, double scale, int causal,
                               int dtype, mi355x_stream_t stream) {
  if (d == 256) return fail(MI355X_EUNSUPPORTED, "mi355x_attn_fwd: head_dim 256 goes through mi355x_attn_fwd_ex");
  return mi355x_attn_fwd_ex(o, o_bhs, lse, q, q_bhs, k, k_bhs, v, v_bhs, batch, heads, heads, sq, skv, d, scale,
                            causal, 0, dtype, stream);
}

extern "C" int64_t mi355x_attn_bwd_workspace_bytes(int64_t batch, int64_t heads, int64_t sq,
                                                   int64_t skv, int64_t d) {
  (void)skv; (void)d;
  return 2 * batch * heads * sq * (int64_t)sizeof(float) + 256;
}

// Scratch of mi355x_attn_bwd_noalloc: the row terms D and LSE*log2(e)
// (2 floats per query row) in a file-scope device array, so that entry
// point needs no workspace and calls no allocator.  Each GPU the library
// runs on holds its own copy for the life of the process; host code reaches
// it only through the address hipGetSymbolAddress returns for the current
// device (the array's name is a host-side stand-in, not a device address).
constexpr int64_t kAttnScratchBytes = 32ll << 20;  // 32 MiB: up to 4M query rows (B*H*Sq)
static __device__ __align__(256) char scratch[kAttnScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// The address of `scratch` on the device that owns `stream` (looked up once
// per device, with that device current; the caller's current device is
// restored); nullptr with the error recorded on failure.
void* scratch_for_stream(hipStream_t stream) {
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur < 0) {
    set_error("mi355x_attn_bwd_noalloc: no current HIP device");
    return nullptr;
  }
  int dev = cur;
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess) {
      set_error("mi355x_attn_bwd_noalloc: cannot query the stream's device");
      return nullptr;
    }
    dev = (int)sdev;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("mi355x_attn_bwd_noalloc: device %d out of range", dev);
    return nullptr;
  }
  std::call_once(g_scratch_once[dev], [dev, cur] {
    void* ptr = nullptr;
    hipError_t e = dev == cur ? hipSuccess : hipSetDevice(dev);
    if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    g_scratch_err[dev] = e;
    g_scratch_ptr[dev] = e == hipSuccess ? ptr : nullptr;
  });
  if (!g_scratch_ptr[dev])
    set_error("mi355x_attn_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
              hipGetErrorString(g_scratch_err[dev]));
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int mi355x_attn_bwd(void* dq, const int64_t* dq_bhs, void* dk, const int64_t* dk_bhs,
                               void* dv, const int64_t* dv_bhs, const void* dout,
                               const int64_t* do_bhs, const void* q, const int64_t* q_bhs,
                               const void* k, const int64_t* k_bhs, const void* v,
                               const int64_t* v_bhs, const void* o, const int64_t* o_bhs,
                               const float* lse, int64_t batch, int64_t heads, int64_t sq,
                               int64_t skv, int64_t d, double scale, int causal, int dtype,
                               void* workspace, int64_t ws_bytes, mi355x_stream_t stream) {
  int rc = check_common(batch, heads, sq, skv, d, dtype);
  if (rc) return rc;
  MI_REQUIRE(strides_ok(q, q_bhs) && strides_ok(k, k_bhs) && strides_ok(v, v_bhs) &&
                 strides_ok(dout, do_bhs) && strides_ok(o, o_bhs),
             "mi355x_attn_bwd: q/k/v/o/dout need 16-byte aligned bases and strides that are multiples of 8");
  for (const int64_t* s : {dq_bhs, dk_bhs, dv_bhs})
    MI_REQUIRE(s[0] % 4 == 0 && s[1] % 4 == 0 && s[2] % 4 == 0, "mi355x_attn_bwd: grads need 8-byte aligned rows");
  const int64_t need = mi355x_attn_bwd_workspace_bytes(batch, heads, sq, skv, d);
  if (!workspace || ws_bytes < need)
    return fail(MI355X_EWORKSPACE, "mi355x_attn_bwd: workspace %lld < %lld", (long long)ws_bytes, (long long)need);
  AttnBwdArgs a;
  a.f = AttnArgs{(void*)o, o_bhs[0], o_bhs[1], o_bhs[2], (float*)lse, q, q_bhs[0], q_bhs[1], q_bhs[2],
                 k, k_bhs[0], k_bhs[1], k_bhs[2], v, v_bhs[0], v_bhs[1], v_bhs[2],
                 batch, heads, sq, skv, (float)(scale * 1.4426950408889634), (float)scale, causal, 1, 0};
  a.dout = dout; a.do_b = do_bhs[0]; a.do_h = do_bhs[1]; a.do_s = do_bhs[2];
  a.dq = dq; a.dq_b = dq_bhs[0]; a.dq_h = dq_bhs[1]; a.dq_s = dq_bhs[2];
  a.dk = dk; a.dk_b = dk_bhs[0]; a.dk_h = dk_bhs[1]; a.dk_s = dk_bhs[2];
  a.dv = dv; a.dv_b = dv_bhs[0]; a.dv_h = dv_bhs[1]; a.dv_s = dv_bhs[2];
  a.ndelta = (float*)workspace;
  a.nlse2 = a.ndelta + batch * heads * sq;
  a.kv_part = nullptr;
  MI_ATTN_DISPATCH(dtype, d, bwd_launch, a, (hipStream_t)stream);
}

extern "C" int mi355x_attn_bwd_noalloc(void* dq, const int64_t* dq_bhs, void* dk, const int64_t* dk_bhs,
                                       void* dv, const int64_t* dv_bhs, const void* dout,
                                       const int64_t* do_bhs, const void* q, const int64_t* q_bhs,
                                       const void* k, const int64_t* k_bhs, const void* v,
                                       const int64_t* v_bhs, const void* o, const int64_t* o_bhs,
                                       const float* lse, int64_t batch, int64_t heads, int64_t sq,
                                       int64_t skv, int64_t d, double scale, int causal, int dtype,
                                       mi355x_stream_t stream) {
  if (batch <= 0 || heads <= 0 || sq <= 0)
    return fail(MI355X_EINVAL, "mi355x_attn_bwd_noalloc: bad shape");
  const int64_t need = mi355x_attn_bwd_workspace_bytes(batch, heads, sq, skv, d);
  if (need > kAttnScratchBytes)
    return fail(MI355X_EINVAL,
                "mi355x_attn_bwd_noalloc: %lld query rows need %lld bytes of scratch, more than its %lld "
                "(at most %lld rows); use mi355x_attn_bwd with a workspace",
                (long long)(batch * heads * sq), (long long)need, (long long)kAttnScratchBytes,
                (long long)((kAttnScratchBytes - 256) / 8));
  void* ws = scratch_for_stream((hipStream_t)stream);
  if (!ws) return MI355X_ELAUNCH;
  // every scratch word the kernels read is written first by attn_bwd_delta
  // in the same call, so nothing is cleared
  return mi355x_attn_bwd(dq, dq_bhs, dk, dk_bhs, dv, dv_bhs, dout, do_bhs, q, q_bhs, k, k_bhs, v, v_bhs, o,
                         o_bhs, lse, batch, heads, sq, skv, d, scale, causal, dtype, ws, kAttnScratchBytes,
                         stream);
}
