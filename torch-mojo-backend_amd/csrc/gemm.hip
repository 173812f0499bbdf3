// GEMM: C[b] = A[b] * B[b] (+ bias row) (+ C if beta), f32 accumulation.
//
// bf16/f16 inputs run on MFMA (v_mfma_f32_16x16x32_*).  One kernel template
// covers every layout of the training GEMMs:
//   fwd  x*W^T : A k-contiguous, B k-contiguous (W rows)
//   dX   dY*W  : A k-contiguous, B n-contiguous
//   dW   dY^T*X: A m-contiguous, B n-contiguous
// Operand tiles (64 k per step) go global -> LDS directly with
// global_load_lds_dwordx4 (each wave instruction fills 1 KB, lane i writing
// bytes [16i, 16i+16)), two stages deep: the next step's loads are issued
// right after the barrier and stream in under the current step's MFMAs.
//   k-contiguous tile: [row][64 k] rows of 128 bytes, 16-byte chunks
//     XOR-swizzled by (row >> 1) & 7 so a fragment read of 16 rows hits 16
//     distinct bank groups;
//   m/n-contiguous tile: [k][rows] with chunks swizzled by kswz(k); fragments
//     are read transposed with ds_read_b64_tr_b16.
// A lane's global source address is chosen so that its fixed LDS slot
// receives the swizzled chunk, so staging costs no registers.
//
// Three block configurations (waves arranged WGM x WGN, each wave owning a
// (BM/WGM) x (BN/WGN) sub-tile of 16x16 MFMA tiles):
//   C128: 128x128, 4 waves of 64x64, 64 KB LDS, two blocks per CU;
//   C192: 128x192, 4 waves of 64x96, 80 KB LDS, two blocks per CU (B
//         k-contiguous only); N = 768, 2304, 3072 split into whole rounds;
//   C256: 256x256, 8 waves of 128x64, 128 KB LDS, one block per CU (fewer
//         LDS bytes per flop; preferred when its tiles fill the CUs evenly).
// The block -> tile map is XCD-aware (the hardware deals workgroups to the 8
// XCDs round-robin): each XCD walks a contiguous run of tiles, so the blocks
// sharing an L2 share operand panels.  Index math is 32-bit and the edge
// clamps are folded into per-thread base pointers once, so the prologue
// stays short next to a K = 768 main loop.
//
// Small outputs with a long K (weight gradients) are split along K into f32
// partial tiles in a caller workspace and summed (bias/beta/cast fused) by
// a second pass.  f32 inputs use a plain 64x64 register-tiled FMA kernel.
#include <stdio.h>
#include <stdlib.h>

#include "common.h"
#include "mfma.h"

#ifndef GEMM_XCD_FLAT
#define GEMM_XCD_FLAT 1
#endif
#include "vec.h"

extern __shared__ __attribute__((aligned(16))) char gemm_smem[];

namespace mi {
namespace {

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
  float* part;     // split-K partials [splits][batch][m][n] (f32) or null
  int64_t kchunk;  // K per split
  int tiles_n;     // tiles along n
  int batch;       // batch count (grid.y = splits * batch)
  int ab_dt;       // operand dtype (for rounding through it)
  int round_c;     // round C (and the row sums) through ab_dt before storing
  void* rowsum;    // optional sum over k of A's rows [batch][m], or null
  int rowsum_dt;
  float* rs_part;  // split-K row-sum partials [splits * rs_slots][batch][m]
};

// v rounded to the 16-bit operand dtype and widened back.
__device__ __forceinline__ float round_through(float v, int dt) {
  return dt == MI355X_BF16 ? (float)(bf16)v : (float)(f16)v;
}

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
    if (g.round_c) v = round_through(v, g.ab_dt);
    st_any(Cb, g.c_dt, off, v);
  }
}

// splitk_reduce for n % 4 == 0 with 4-aligned C strides and fewer than 2^31
// elements: each thread sums four adjacent columns with 16-byte partial
// loads and 32-bit index math.
template <typename CT>
__device__ __forceinline__ void splitk_reduce4_body(const GemmArgs& g, int splits, int nb, uint32_t blk,
                                                    uint32_t nblk) {
  const uint32_t n4 = (uint32_t)(g.n / 4), mn4 = (uint32_t)g.m * n4;
  const uint32_t total = (uint32_t)nb * mn4;
  const float4* P = (const float4*)g.part;
  for (uint32_t i = blk * 256u + threadIdx.x; i < total; i += nblk * 256u) {
    const uint32_t bi = i / mn4, rem = i - bi * mn4;
    const uint32_t row = rem / n4, col = (rem - row * n4) * 4;
    float4 a = P[i];
    for (int sp = 1; sp < splits; ++sp) {
      const float4 q = P[(uint32_t)sp * total + i];
      a.x += q.x, a.y += q.y, a.z += q.z, a.w += q.w;
    }
    float v[4] = {a.x, a.y, a.z, a.w};
    if (g.bias)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += ld_any(g.bias, g.bias_dt, col + e);
    CT* C = (CT*)g.c + (int64_t)bi * g.c_bs + (int64_t)row * g.c_rs + col;
    float old[4];
    if (g.beta) {
      Vec4<CT>::load(C, old);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += old[e];
    }
    if (g.round_c)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = round_through(v[e], g.ab_dt);
    Vec4<CT>::store(C, v);
  }
}

template <typename CT>
__global__ void __launch_bounds__(256) splitk_reduce4(GemmArgs g, int splits, int nb) {
  splitk_reduce4_body<CT>(g, splits, nb, blockIdx.x, gridDim.x);
}

// Sum the row-sum partials ([slots][nb * m]) into rowsum[batch][m].  A block
// takes 32 rows at a time with 8 threads per row, each summing every 8th
// slot, then combines the 8 in LDS.
__device__ __forceinline__ void rowsum_reduce_body(const GemmArgs& g, int slots, int64_t nb, uint32_t blk,
                                                   uint32_t nblk) {
  __shared__ float red[8][33];
  const int64_t total = nb * g.m;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int64_t base = (int64_t)blk * 32; base < total; base += (int64_t)nblk * 32) {
    const int64_t idx = base + tx;
    float v = 0.f;
    if (idx < total) {
      int s = ty;
      for (; s + 24 < slots; s += 32) {
        const float a0 = g.rs_part[s * total + idx], a1 = g.rs_part[(s + 8) * total + idx];
        const float a2 = g.rs_part[(s + 16) * total + idx], a3 = g.rs_part[(s + 24) * total + idx];
        v += (a0 + a1) + (a2 + a3);
      }
      for (; s < slots; s += 8) v += g.rs_part[s * total + idx];
    }
    red[ty][tx] = v;
    __syncthreads();
    if (ty == 0 && idx < total) {
      float r = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) r += red[j][tx];
      if (g.round_c) r = round_through(r, g.ab_dt);
      st_any(g.rowsum, g.rowsum_dt, idx, r);
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(256) rowsum_reduce(GemmArgs g, int slots, int64_t nb) {
  rowsum_reduce_body(g, slots, nb, blockIdx.x, gridDim.x);
}

// The two finishing sums of a split-K GEMM with row sums in one launch:
// blocks [0, nbc) sum the C partials, the rest the row-sum partials.
template <typename CT>
__global__ void __launch_bounds__(256) splitk_rowsum_reduce(GemmArgs g, int splits, int nb, int slots,
                                                             uint32_t nbc) {
  if (blockIdx.x < nbc) splitk_reduce4_body<CT>(g, splits, nb, blockIdx.x, nbc);
  else rowsum_reduce_body(g, slots, nb, blockIdx.x - nbc, gridDim.x - nbc);
}

// Row swizzle of a k-contiguous tile with BK-element (2*BK-byte) rows: row r
// stores its 16-byte chunk c in slot c ^ rswz(r).  A fragment read (16 rows
// at one chunk) then covers every bank once: BK = 64, 8 chunks, rows paired
// by (r >> 1); BK = 32, 4 chunks, rows grouped by (r >> 2).
template <int BK>
__device__ __forceinline__ int rswz(int r) { return BK == 64 ? ((r >> 1) & 7) : ((r >> 2) & 3); }

// k-contiguous operand tile: ROWS rows x BK k, loaded by NT threads, one
// 1 KB instruction per RPI rows.  Thread (wave w, lane l) handles rows
// r = RPI*(it*WAVES + w) + l/CPR; with WAVES even the swizzled chunk of its
// slot, (l % CPR) ^ rswz(r), is the same for every `it`.  Rows past the
// operand's end reload its last row (their results are never stored).
template <int ROWS, int NT, int BK>
struct TileLoad {
  static constexpr int CPR = BK / 8;    // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;  // rows per 1 KB instruction
  static constexpr int WAVES = NT / 64;
  static constexpr int ITERS = ROWS / (RPI * WAVES);
  static_assert(WAVES % 2 == 0 && ITERS * RPI * WAVES == ROWS, "tile/thread mismatch");
  const char* src[ITERS];  // row base + this lane's chunk, at k = 0
  int chunk;

  __device__ __forceinline__ void init(const char* base, int64_t ld_bytes, int64_t row0, int64_t rows) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int r = wave * RPI + lane / CPR;
    chunk = (lane % CPR) ^ rswz<BK>(r);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      int64_t row = row0 + r + it * RPI * WAVES;
      if (row > rows - 1) row = rows - 1;
      src[it] = base + row * ld_bytes + chunk * 16;
    }
  }
  // KT: the K range may end inside this BK slab; a chunk starting past
  // kend_bytes reloads chunk 0 (masked out of the MFMAs, address valid).
  template <bool KT>
  __device__ __forceinline__ void issue(int64_t k0_bytes, char* dst, int64_t kend_bytes) const {
    const int64_t koff = (KT && k0_bytes + chunk * 16 >= kend_bytes) ? k0_bytes - chunk * 16 : k0_bytes;
    // one scalar LDS base per call; each instruction's slot is a constant offset
    const unsigned lds0 = lds_base_of(dst) + wave_id() * 1024;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) dma_b128(src[it] + koff, lds0 + it * WAVES * 1024);
  }
  template <bool KT>
  __device__ __forceinline__ void issue_range(int64_t k0_bytes, char* dst, int64_t kend_bytes, int lo, int hi) const {
    const int64_t koff = (KT && k0_bytes + chunk * 16 >= kend_bytes) ? k0_bytes - chunk * 16 : k0_bytes;
    const unsigned lds0 = lds_base_of(dst) + wave_id() * 1024;
#pragma unroll
    for (int it = 0; it < ITERS; ++it)
      if (it >= lo && it < hi) dma_b128(src[it] + koff, lds0 + it * WAVES * 1024);
  }
};

// m/n-contiguous operand tile: BK k-rows of ROWS elements, 16-byte chunks
// XOR-swizzled by s(k) = 2 * ((k & 3) | ((k >> 1) & 4)).  A transposing
// fragment read serves each half-wave from 8 k-rows x 2 adjacent chunks
// (c, c ^ 1); s takes 8 distinct even values on those k-rows, so the 16
// (k-row, chunk) pairs land on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int kswz(int k) { return 2 * ((k & 3) | ((k >> 1) & 4)); }

template <int ROWS, int NT, int BK>
struct TileLoadT {
  static constexpr int ROWB = ROWS * 2;
  static constexpr int CPR = ROWS / 8;     // chunks per k-row
  static constexpr int KPI = 1024 / ROWB;  // k-rows per 1 KB instruction
  static constexpr int WAVES = NT / 64;
  static constexpr int ITERS = BK / KPI / WAVES;
  static_assert(CPR >= 16 && ITERS * KPI * WAVES == BK, "tile/thread mismatch");
  const char* base;
  int64_t ld;              // bytes between k-rows
  int64_t col_off[ITERS];  // byte offset of this lane's (clamped) chunk
  int kr[ITERS];           // this lane's k-row within the slab

  // A last partial chunk of rows reads into the row padding (the k stride
  // is at least the row count rounded up to 8, checked by the caller).
  __device__ __forceinline__ void init(const char* b, int64_t ld_bytes, int64_t r0, int64_t rows) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    base = b;
    ld = ld_bytes;
    const int64_t last_chunk = ((rows - 1) >> 3) << 3;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      kr[it] = (it * WAVES + wave) * KPI + lane / CPR;
      int64_t m = r0 + ((lane % CPR) ^ kswz(kr[it])) * 8;
      if (m > last_chunk) m = last_chunk;
      col_off[it] = m * 2;
    }
  }
  // KT: k-rows at or past kend reload row kend-1 (masked out of the MFMAs).
  template <bool KT>
  __device__ __forceinline__ void issue(int64_t k0, char* dst, int64_t kend) const {
    const unsigned lds0 = lds_base_of(dst) + wave_id() * 1024;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      int64_t k = k0 + kr[it];
      if (KT && k >= kend) k = kend - 1;
      dma_b128(base + k * ld + col_off[it], lds0 + it * WAVES * 1024);
    }
  }
  template <bool KT>
  __device__ __forceinline__ void issue_range(int64_t k0, char* dst, int64_t kend, int lo, int hi) const {
    const unsigned lds0 = lds_base_of(dst) + wave_id() * 1024;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      if (it < lo || it >= hi) continue;
      int64_t k = k0 + kr[it];
      if (KT && k >= kend) k = kend - 1;
      dma_b128(base + k * ld + col_off[it], lds0 + it * WAVES * 1024);
    }
  }
};

template <int ROWS, int NT, bool K_CONTIG, int BK>
struct OperandLoad;
template <int ROWS, int NT, int BK>
struct OperandLoad<ROWS, NT, true, BK> {
  TileLoad<ROWS, NT, BK> t;
  __device__ __forceinline__ void init(const char* b, int64_t ld, int64_t r0, int64_t n) { t.init(b, ld, r0, n); }
  template <bool KT>
  __device__ __forceinline__ void issue(int64_t k0, char* dst, int64_t kend) const {
    t.template issue<KT>(k0 * 2, dst, kend * 2);
  }
  template <bool KT>
  __device__ __forceinline__ void issue_range(int64_t k0, char* dst, int64_t kend, int lo, int hi) const {
    t.template issue_range<KT>(k0 * 2, dst, kend * 2, lo, hi);
  }
  static constexpr int ITERS = TileLoad<ROWS, NT, BK>::ITERS;
};
template <int ROWS, int NT, int BK>
struct OperandLoad<ROWS, NT, false, BK> {
  TileLoadT<ROWS, NT, BK> t;
  __device__ __forceinline__ void init(const char* b, int64_t ld, int64_t r0, int64_t n) { t.init(b, ld, r0, n); }
  template <bool KT>
  __device__ __forceinline__ void issue(int64_t k0, char* dst, int64_t kend) const {
    t.template issue<KT>(k0, dst, kend);
  }
  template <bool KT>
  __device__ __forceinline__ void issue_range(int64_t k0, char* dst, int64_t kend, int lo, int hi) const {
    t.template issue_range<KT>(k0, dst, kend, lo, hi);
  }
  static constexpr int ITERS = TileLoadT<ROWS, NT, BK>::ITERS;
};


// CNT MFMA fragments (rows r0 + 16i .. +15, k = ks*32 + 8g + 0..7) from an
// m/n-contiguous tile, two transposing reads each: within a 16-lane group,
// lane i receives element i%4 of the 4-element pieces of lanes i/4, 4+i/4,
// 8+i/4, 12+i/4, so source lane 4e+q supplies k-row (.. + e), columns
// r0+4q..+3.
template <typename T, int ROWS, int CNT>
__device__ __forceinline__ void mn_frags(const char* tile, int r0, int ks, typename Mfma<T>::frag (&f)[CNT]) {
  constexpr int ROWB = ROWS * 2;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, src = lane & 15;
  const int k1 = ks * 32 + 8 * g + (src >> 2), k2 = k1 + 4;
#pragma unroll
  for (int i = 0; i < CNT; ++i) {
    const int m = r0 + i * 16 + 4 * (src & 3);
    const s16x4 a = ds_read_tr(tile + k1 * ROWB + (((m >> 3) ^ kswz(k1)) << 4) + ((m & 7) << 1));
    const s16x4 b = ds_read_tr(tile + k2 * ROWB + (((m >> 3) ^ kswz(k2)) << 4) + ((m & 7) << 1));
    f[i] = join_frag<typename Mfma<T>::frag>(a, b);
  }
}

// Zero the fragment slots whose k index (kbase + slot) is >= kend.
template <typename F>
__device__ __forceinline__ void mask_k(F& f, int64_t kbase, int64_t kend) {
  short* fs = (short*)&f;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (kbase + e >= kend) fs[e] = 0;
}

// Block configurations.
#ifndef GEMM_STAGES_128
#define GEMM_STAGES_128 2
#endif
#ifndef GEMM_STAGES_192
#define GEMM_STAGES_192 2
#endif
template <int CFG>
struct TileCfg;
template <>
struct TileCfg<0> {  // C128
  static constexpr int BM = 128, BN = 128, BK = 64, WGM = 2, WGN = 2, STAGES = GEMM_STAGES_128;
  static constexpr int MIN_BLOCKS = STAGES * (BM + BN) * BK * 2 * 2 <= 160 * 1024 ? 2 : 1;
};
template <>
struct TileCfg<1> {  // C256
  static constexpr int BM = 256, BN = 256, BK = 64, WGM = 2, WGN = 4, STAGES = 2, MIN_BLOCKS = 1;
};
template <>
struct TileCfg<2> {  // C192: 128x192, waves of 64x96, 40 KB per stage (k-contiguous B only)
  static constexpr int BM = 128, BN = 192, BK = 64, WGM = 2, WGN = 2, STAGES = GEMM_STAGES_192;
  static constexpr int MIN_BLOCKS = STAGES * (BM + BN) * BK * 2 * 2 <= 160 * 1024 ? 2 : 1;
};
// C256 in 32-k stages, three deep (96 KB): for weight gradients, whose
// operands are both m/n-contiguous.  Their transposing fragment reads make
// a 64-k step long; halving it and keeping two stages in flight hides the
// loads better (gfx950, cfg 2 shapes: 7-13% over 64-k stages).
template <>
struct TileCfg<3> {
  static constexpr int BM = 256, BN = 256, BK = 32, WGM = 2, WGN = 4, STAGES = 3, MIN_BLOCKS = 1;
};

// s_waitcnt immediate for vmcnt(n), other counters not waited on.
constexpr int vmcnt_imm(int n) { return 0x0f70 | (n & 15) | ((n >> 4) << 14); }

// Write one wave's accumulators to C (pointing at the wave tile's first
// element), adding the preloaded bias and, with BETA, the old C.  Offsets
// inside the tile are 32-bit (the host checks the row stride); EDGE adds the
// bounds checks that only partial tiles need.  Each store instruction covers
// four 16-column runs, and the j loop fills whole 128-byte lines.
template <typename CT, typename T, bool BETA, bool EDGE, bool ROUND, int TM, int TN>
__device__ __forceinline__ void store_tile(CT* __restrict__ C, int c_rs, const f32x4 (&acc)[TM][TN],
                                           const float (&bias)[TN], int rows_left, int cols_left, int lr,
                                           int lg) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = i * 16 + lg * 4 + e;
      if (EDGE && r >= rows_left) continue;
      CT* row = C + r * c_rs;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int c = j * 16 + lr;
        if (EDGE && c >= cols_left) continue;
        float v = acc[i][j][e] + bias[j];
        if (BETA) v += (float)row[c];
        if (ROUND) v = (float)(T)v;
        row[c] = (CT)v;
      }
    }
}

// Full wave tiles without beta: the accumulators go through a per-wave LDS
// slab 16 rows at a time (one MFMA row of tiles, f32, rows padded by 4
// floats) and leave as row-contiguous 16-byte stores: 8 bf16/f16 or 4 f32
// per lane instead of one element per store.  The slab holds 16 x (WN + 4)
// floats; `lane` is the wave lane.  Requires 16-byte aligned rows of C.
// NT: non-temporal stores, for outputs no kernel reads soon enough to find
// them in a cache (split-K partials, summed right after, keep normal
// stores); a training step ran 0.2 ms faster with them.
template <typename CT, typename T, bool ROUND, bool NT, int TM, int TN>
__device__ __forceinline__ void store_tile_lds(CT* __restrict__ C, int c_rs, const f32x4 (&acc)[TM][TN],
                                               const float (&bias)[TN], float* slab, int lr, int lg, int lane) {
#ifndef GEMM_SLAB_PAD
#define GEMM_SLAB_PAD 4
#endif
  // slab row stride in floats: 4 * LD = 16 (mod 64) puts the four 16-lane
  // groups of a store (rows lg*4 + e) on disjoint banks
  constexpr int WN = TN * 16, LD = WN + GEMM_SLAB_PAD;
  constexpr int E = 16 / sizeof(CT);             // elements per 16-byte store
  constexpr int CHUNKS = 16 * WN / E;            // 16-byte chunks per 16-row slab
  static_assert(WN % E == 0 && CHUNKS % 64 == 0, "slab shape");
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[i][j][e] + bias[j];
        if (ROUND) v = (float)(T)v;
        slab[(lg * 4 + e) * LD + j * 16 + lr] = v;
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int it = 0; it < CHUNKS / 64; ++it) {
      const int ch = it * 64 + lane, r = ch / (WN / E), c = (ch % (WN / E)) * E;
      const float* src = slab + r * LD + c;
      struct alignas(16) Out { CT v[E]; } out;
#pragma unroll
      for (int e = 0; e < E; ++e) out.v[e] = (CT)src[e];
      if constexpr (NT)
        __builtin_nontemporal_store(__builtin_bit_cast(f32x4, out), (f32x4*)(C + (i * 16 + r) * c_rs + c));
      else
        *(Out*)(C + (i * 16 + r) * c_rs + c) = out;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

template <typename CT, typename T, int TM, int TN>
__device__ __forceinline__ void store_any(CT* C, int c_rs, const f32x4 (&acc)[TM][TN], const float (&bias)[TN],
                                          bool beta, bool round, int rows_left, int cols_left, int lr, int lg) {
  const bool edge = rows_left < TM * 16 || cols_left < TN * 16;
#define ST(B, E, R) store_tile<CT, T, B, E, R>(C, c_rs, acc, bias, rows_left, cols_left, lr, lg)
  if (round) {  // round-through stores are only used without beta
    if (edge) ST(false, true, true);
    else ST(false, false, true);
  } else if (beta) {
    if (edge) ST(true, true, false);
    else ST(true, false, false);
  } else {
    if (edge) ST(false, true, false);
    else ST(false, false, false);
  }
#undef ST
}

// RS: also sum A's rows over k, from the fragments the MFMAs consume, with
// one extra MFMA against a fragment of ones (every column of its 16x16
// result is the row sum).  With split K the 32-k substeps are dealt round
// robin over the tiles_n * WGN waves that hold the same rows (one substep in
// that many per wave), each writing its own partial slot; without split K
// the waves of the first wave column of the first column tile do it all.
template <typename T, int CFG, bool A_K, bool B_K, bool KT, bool RS>
__global__ void __launch_bounds__(64 * TileCfg<CFG>::WGM * TileCfg<CFG>::WGN, TileCfg<CFG>::MIN_BLOCKS)
    gemm_tile(GemmArgs g) {
  typedef typename Mfma<T>::frag frag;
  typedef TileCfg<CFG> C;
  constexpr int BM = C::BM, BN = C::BN;
  constexpr int NT = 64 * C::WGM * C::WGN;
  constexpr int WM = BM / C::WGM, WN = BN / C::WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int BK = C::BK, ROWB = BK * 2;  // k per stage, bytes of a k-contiguous row
  constexpr int A_BYTES = BM * ROWB, STAGE = A_BYTES + BN * ROWB, S = C::STAGES;
  char* const lds = gemm_smem;

#if GEMM_XCD_FLAT
  // XCD-aware order over the whole grid: the hardware deals workgroups to
  // the 8 XCDs round-robin in dispatch order (x fastest, then y), so XCD
  // L % 8 gets every 8th block.  Each XCD is given one contiguous run of the
  // (split, batch)-major tile list instead: its blocks share A/B panels and,
  // with split K, one or two K ranges, so each L2 fetches about 1/8 of the
  // operands (dealing a plane's tiles over all XCDs made every L2 fetch
  // every split's panels).  A bijection for any grid size.
  const uint32_t nt = gridDim.x;
  uint32_t L = blockIdx.x + nt * blockIdx.y;
  {
    const uint32_t total = nt * gridDim.y, xcd = L & 7, q = total >> 3, r = total & 7;
    L = xcd * q + min(xcd, r) + (L >> 3);
  }
  const uint32_t plane = L / nt, t = L - plane * nt;
  const uint32_t tm = t / (uint32_t)g.tiles_n, tn = t - tm * (uint32_t)g.tiles_n;
  const uint32_t split = plane / (uint32_t)g.batch, bidx = plane - split * (uint32_t)g.batch;
#else
  // XCD-aware tile order within one (split, batch) plane.
  uint32_t t = blockIdx.x;
  const uint32_t nt = gridDim.x;
  if ((nt & 7) == 0) t = (t & 7) * (nt >> 3) + (t >> 3);
  const uint32_t tm = t / (uint32_t)g.tiles_n, tn = t - tm * (uint32_t)g.tiles_n;
  const uint32_t split = blockIdx.y / (uint32_t)g.batch, bidx = blockIdx.y - split * (uint32_t)g.batch;
#endif
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  int64_t kbeg = 0, kend = g.k;
  if (g.part) {
    kbeg = (int64_t)split * g.kchunk;
    kend = min(g.k, kbeg + g.kchunk);
  }

  const char* A = (const char*)g.a + (int64_t)bidx * g.a_bs * (int64_t)sizeof(T);
  const char* B = (const char*)g.b + (int64_t)bidx * g.b_bs * (int64_t)sizeof(T);
  // A_K: bytes between rows; else bytes between k-rows.  Same for B.
  const int64_t a_ldb = (A_K ? g.a_rs : g.a_cs) * (int64_t)sizeof(T);
  const int64_t b_ldb = (B_K ? g.b_cs : g.b_rs) * (int64_t)sizeof(T);

  const int lane = threadIdx.x & 63, wave = wave_id();  // scalar: the row-sum test branches on it
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int lr = lane & 15, lg = lane >> 4;

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  OperandLoad<BM, NT, A_K, BK> la;
  OperandLoad<BN, NT, B_K, BK> lb;
  constexpr int PER_STAGE = decltype(la.t)::ITERS + decltype(lb.t)::ITERS;  // DMA instructions per stage
  static_assert(S == 2 || (S - 2) * PER_STAGE < 64, "vmcnt range");
  la.init(A, a_ldb, m0, g.m);
  lb.init(B, b_ldb, n0, g.n);
  // Prologue: stages 0 .. S-2 in flight.
#pragma unroll
  for (int st = 0; st < S - 1; ++st) {
    if (kbeg + st * BK < kend) {
      la.template issue<KT>(kbeg + st * BK, lds + st * STAGE, kend);
      lb.template issue<KT>(kbeg + st * BK, lds + st * STAGE + A_BYTES, kend);
    }
  }
  // k-contiguous fragment rows (.. + lr) share the swizzle of lr
  const int sw = rswz<BK>(lr);
  const int rs_slots = g.part ? g.tiles_n * C::WGN : 1;
  const int rs_slot = g.part ? (int)tn * C::WGN + wn : 0;
  const bool rs_on = RS && (g.part || (tn == 0 && wn == 0));
  int rs_q = 0;  // this wave's substep counter modulo rs_slots
  f32x4 rsum[TM];
  frag ones;
#pragma unroll
  for (int i = 0; i < TM; ++i) rsum[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (T)1.0f;

  int cur = 0;
  for (int64_t k0 = kbeg; k0 < kend; k0 += BK) {
    // This step's tiles have landed when at most the later stages' loads
    // (S-2 stages, if issued) are still outstanding.
    if (S > 2 && k0 + (S - 2) * BK < kend) __builtin_amdgcn_s_waitcnt(vmcnt_imm((S - 2) * PER_STAGE));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    // the next stage goes to the slot read in the previous step (every wave
    // is past it); its loads are issued after this step's first B fragment
    // reads, so the first MFMAs do not wait behind the load issue (training
    // step 22.22 -> 22.03 ms, three runs each on one box; issuing them after
    // the reads only for k-contiguous A gave nothing).  The 256x256 tiles
    // (eight MFMA rows per wave) spread the load instructions over the MFMA
    // rows of the first 32-k substep instead, so the load issue no longer
    // stalls the wave in one burst: the forward fc and lm_head launches run
    // 3.4-5.8% faster in the training step (kernel trace, two boxes); the
    // same spread lost 2-6% on the 128x128 and 128x192 tiles and the 32-k
    // 256x256 weight-gradient tiles, which keep the single burst.
    const bool more = k0 + (S - 1) * BK < kend;
    char* const nxt = lds + (cur == 0 ? S - 1 : cur - 1) * STAGE;
    const char* at = lds + cur * STAGE;
    const char* bt = at + A_BYTES;
    const bool tail = KT && k0 + BK > kend;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      const bool rs_now = rs_on && rs_q == rs_slot;
      if (RS && ++rs_q == rs_slots) rs_q = 0;
      const int coff = ((ks * 4 + lg) ^ sw) * 16;
      const int64_t kfrag = k0 + ks * 32 + lg * 8;
      frag bfr[TN], afr[A_K ? 1 : TM];
      if constexpr (!B_K) mn_frags<T, BN, TN>(bt, wn * WN, ks, bfr);
      if constexpr (!A_K) mn_frags<T, BM, TM>(at, wm * WM, ks, afr);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (B_K) bfr[j] = *(const frag*)(bt + (wn * WN + j * 16 + lr) * ROWB + coff);
        if (tail) mask_k(bfr[j], kfrag, kend);
      }
      if (CFG != 1 && ks == 0 && more) {
        la.template issue<KT>(k0 + (S - 1) * BK, nxt, kend);
        lb.template issue<KT>(k0 + (S - 1) * BK, nxt + A_BYTES, kend);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if (CFG == 1 && ks == 0 && more) {
          // load instructions q in [lo, hi) of this stage's list (A's, then B's)
          constexpr int NA = decltype(la)::ITERS, NQ = NA + decltype(lb)::ITERS;
          const int lo = i * NQ / TM, hi = (i + 1) * NQ / TM;
          la.template issue_range<KT>(k0 + (S - 1) * BK, nxt, kend, lo, hi);
          lb.template issue_range<KT>(k0 + (S - 1) * BK, nxt + A_BYTES, kend, lo - NA, hi - NA);
        }
        frag af;
        if constexpr (A_K) af = *(const frag*)(at + (wm * WM + i * 16 + lr) * ROWB + coff);
        else af = afr[i];
        if (tail) mask_k(af, kfrag, kend);
        if (RS && rs_now) rsum[i] = Mfma<T>::mma(af, ones, rsum[i]);
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::mma(af, bfr[j], acc[i][j]);
      }
    }
    cur = cur == S - 1 ? 0 : cur + 1;
  }

  // every wave is past its last LDS read: the stages become store slabs
  __syncthreads();
  float* const slab = (float*)lds + wave * (16 * (WN + GEMM_SLAB_PAD));
  const int64_t row0 = m0 + wm * WM, col0 = n0 + wn * WN;
  if (RS && rs_on && lr == 0) {
    // lane (lg, 0) holds rows 4*lg .. 4*lg+3 of each 16-row fragment
    const int64_t slot = (int64_t)split * rs_slots + rs_slot;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t r = row0 + i * 16 + lg * 4 + e;
        if (r >= g.m) continue;
        if (g.part) {
          g.rs_part[(slot * g.batch + bidx) * g.m + r] = rsum[i][e];
        } else {
          const float v = g.round_c ? round_through(rsum[i][e], g.ab_dt) : rsum[i][e];
          st_any(g.rowsum, g.rowsum_dt, (int64_t)bidx * g.m + r, v);
        }
      }
  }
  const int rows_left = (int)min(g.m - row0, (int64_t)WM), cols_left = (int)min(g.n - col0, (int64_t)WN);
  if (rows_left <= 0 || cols_left <= 0) return;
  float bias[TN];
  if (g.part) {
#pragma unroll
    for (int j = 0; j < TN; ++j) bias[j] = 0.f;
    float* P = g.part + ((int64_t)split * g.batch + bidx) * g.m * g.n + row0 * g.n + col0;
    if (rows_left == WM && cols_left == WN && (g.n & 3) == 0 && ((uintptr_t)g.part & 15) == 0)
      store_tile_lds<float, T, false, false>(P, (int)g.n, acc, bias, slab, lr, lg, lane);
    else
      store_any<float, T>(P, (int)g.n, acc, bias, false, false, rows_left, cols_left, lr, lg);
    return;
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int c = j * 16 + lr;
    bias[j] = (g.bias && c < cols_left) ? ld_any(g.bias, g.bias_dt, col0 + c) : 0.f;
  }
  const int64_t c_es = g.c_dt == MI355X_F32 ? 4 : 2;
  char* Cb = (char*)g.c + ((int64_t)bidx * g.c_bs + row0 * g.c_rs + col0) * c_es;
  const int c_rs = (int)g.c_rs;
  const bool rnd = g.round_c && g.c_dt == MI355X_F32;  // 16-bit outputs are already rounded
  const bool full = rows_left == WM && cols_left == WN && !g.beta && ((uintptr_t)g.c & 15) == 0 &&
                    (c_rs * c_es) % 16 == 0 && (g.c_bs * c_es) % 16 == 0;
  if (full) {
    if (g.c_dt == MI355X_BF16) store_tile_lds<bf16, T, false, true>((bf16*)Cb, c_rs, acc, bias, slab, lr, lg, lane);
    else if (g.c_dt == MI355X_F16) store_tile_lds<f16, T, false, true>((f16*)Cb, c_rs, acc, bias, slab, lr, lg, lane);
    else if (rnd) store_tile_lds<float, T, true, true>((float*)Cb, c_rs, acc, bias, slab, lr, lg, lane);
    else store_tile_lds<float, T, false, true>((float*)Cb, c_rs, acc, bias, slab, lr, lg, lane);
    return;
  }
  if (g.c_dt == MI355X_BF16) store_any<bf16, T>((bf16*)Cb, c_rs, acc, bias, g.beta, false, rows_left, cols_left, lr, lg);
  else if (g.c_dt == MI355X_F32) store_any<float, T>((float*)Cb, c_rs, acc, bias, g.beta, rnd, rows_left, cols_left, lr, lg);
  else store_any<f16, T>((f16*)Cb, c_rs, acc, bias, g.beta, false, rows_left, cols_left, lr, lg);
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

// pack_k_contig with 16-byte global accesses, for sources whose base, row or
// k stride and batch stride are 8-element aligned (and, transposed, whose row
// count is a multiple of 8).  A 64x64 tile moves as 512 16-byte chunks, two
// per thread each way.  The LDS tile is [k][row] with a 65-element pitch: the
// 2-byte scatter of a loaded chunk and the 2-byte gather of a stored one then
// hit distinct banks across the wave.
__global__ void __launch_bounds__(256) pack_k_contig_v8(uint16_t* __restrict__ dst, int64_t ld,
                                                        int64_t dst_bs, const uint16_t* __restrict__ src,
                                                        int64_t stride, int64_t sbs, int64_t rows,
                                                        int64_t kdim, int transposed) {
  const int64_t b = blockIdx.z;
  const int64_t row0 = (int64_t)blockIdx.y * 64, k0 = (int64_t)blockIdx.x * 64;
  const uint16_t* S = src + b * sbs;
  uint16_t* D = dst + b * dst_bs;
  const int t = threadIdx.x;
  if (!transposed) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t r = row0 + (t >> 3) + 32 * j, k = k0 + (t & 7) * 8;
      if (r >= rows || k >= ld) continue;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (k + 8 <= kdim) {
        v = *(const uint4*)(S + r * stride + k);
      } else if (k < kdim) {
        uint16_t e8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) e8[e] = k + e < kdim ? S[r * stride + k + e] : (uint16_t)0;
        v = *(const uint4*)e8;
      }
      *(uint4*)(D + r * ld + k) = v;
    }
    return;
  }
  __shared__ uint16_t tile[64][65];  // [k][row]
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int kl = (t >> 3) + 32 * j, rl = (t & 7) * 8;
    const int64_t k = k0 + kl, r = row0 + rl;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (k < kdim && r < rows) v = *(const uint4*)(S + k * stride + r);
    const uint16_t* e8 = (const uint16_t*)&v;
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[kl][rl + e] = e8[e];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int rl = (t >> 3) + 32 * j, kc = (t & 7) * 8;
    const int64_t r = row0 + rl, k = k0 + kc;
    if (r >= rows || k >= ld) continue;
    uint16_t e8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) e8[e] = tile[kc + e][rl];
    *(uint4*)(D + r * ld + k) = *(const uint4*)e8;
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
  int cfg;  // 0 = C128, 1 = C256, 2 = C192, 3 = C256 in 32-k stages
  int splits;
  int64_t kchunk;
};

int64_t tiles_of(int cfg, int64_t batch, int64_t m, int64_t n) {
  const bool c256 = cfg == 1 || cfg == 3;
  const int64_t bm = c256 ? 256 : 128, bn = c256 ? 256 : (cfg == 2 ? 192 : 128);
  return ((m + bm - 1) / bm) * ((n + bn - 1) / bn) * batch;
}

// Row-sum partial slots per split: one per wave column of every column tile.
int64_t rs_slots_of(int cfg, int64_t n) {
  const bool c256 = cfg == 1 || cfg == 3;
  const int64_t bn = c256 ? 256 : (cfg == 2 ? 192 : 128), wgn = c256 ? 4 : 2;
  return (n + bn - 1) / bn * wgn;
}

// Pick the configuration that finishes in the least time: whole rounds of
// the CUs' block slots (two C128 blocks or one C256 block per CU) times the
// per-round time measured on gfx950 at K = 768..3072 (a C256 round does
// twice a C128 round's work in 1.82x its time).  An m-contiguous A (a weight
// gradient dY^T X) reads both operands through transposing LDS reads, which
// C256 tiles halve per flop: when both sides span a 256 tile it takes them,
// in 32-k stages (the 50304 x 768 embedding gradient: 1.53 -> 1.35 ms, the
// 768 x 3072 one 105 -> 84 us with 7 K splits).  Then split K when the
// output alone cannot fill the chip.
Plan plan_gemm(int64_t batch, int64_t m, int64_t n, int64_t k, bool a_kcontig, bool b_kcontig) {
  Plan best{0, 1, k};
  const int64_t t128 = tiles_of(0, batch, m, n), t256 = tiles_of(1, batch, m, n), t192 = tiles_of(2, batch, m, n);
  const double c128 = (double)((t128 + 2 * kCUs - 1) / (2 * kCUs));
  const double c256 = 1.82 * (double)((t256 + kCUs - 1) / kCUs);
  const double c192 = 1.5 * (double)((t192 + 2 * kCUs - 1) / (2 * kCUs));
  double cbest = c128;
  if (t256 >= kCUs && c256 < cbest) best.cfg = 1, cbest = c256;
  if (b_kcontig && t192 >= kCUs && c192 < cbest) best.cfg = 2, cbest = c192;
  // Weight gradients (m-contiguous A) take the 32-k C256 stages when their
  // 256x256 tiles fill the CUs (wte: 50304 x 768); smaller ones take
  // split-K C128, whose K ranges the XCD-ordered grid keeps in one or two
  // L2s (config 2 shapes, TF/s: 768 x 768 646 against 501, 2304 x 768 912
  // against 839, 768 x 3072 933 against 915).
  if (!a_kcontig && m >= 256 && n >= 256 && t256 >= kCUs) best.cfg = 3;
  static const char* forced = getenv("MI355X_GEMM_TILE");  // tuning override: "128", "192", "256" or "256.32"
  if (forced) {
    const double f = atof(forced);
    best.cfg = f == 256 ? 1 : (f > 256 && !a_kcontig ? 3 : (f == 192 && b_kcontig ? 2 : 0));
  }
  const int64_t tiles = tiles_of(best.cfg, batch, m, n);
  if (best.cfg == 3 && tiles >= kCUs && k >= 8192) {
    // One block per CU: a last round that is mostly empty costs a whole
    // round.  K splits that fill the rounds better win when the gain is
    // large (the 50304 x 768 embedding gradient, K = 16384: 591 tiles are
    // 2.3 rounds; two splits make 4.6 of half length: 1.49 -> 1.29 ms plus
    // a 75 us partial sum, train step -0.12 ms).
    const double r1 = (double)((tiles + kCUs - 1) / kCUs);
    int64_t bs = 1;
    double bcost = r1;
    for (int64_t sp = 2; sp <= 4; ++sp) {
      const double c = (double)((tiles * sp + kCUs - 1) / kCUs) / (double)sp + 0.05 * (double)sp;
      if (c < bcost * 0.9) bs = sp, bcost = c;
    }
    if (bs > 1) {
      int64_t chunk = (k + bs - 1) / bs;
      chunk = (chunk + 63) / 64 * 64;
      best.splits = (int)((k + chunk - 1) / chunk);
      best.kchunk = chunk;
    }
  }
  if (tiles < kCUs && k >= 2048) {
    // as many K splits as keep every block in the first round of block
    // slots: a second, partly filled round would double the time
    const int64_t slots = best.cfg == 1 || best.cfg == 3 ? kCUs : 2 * kCUs;  // block slots of the chosen config
    int64_t s = slots / tiles;
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

// Launch one kernel instantiation; the first launch of each opts it into
// more than 64 KB of dynamic LDS when it needs that.
template <typename T, int CFG, bool A_K, bool B_K, bool KT, bool RS>
int launch_kernel(const GemmArgs& g, dim3 grid, hipStream_t s) {
  typedef TileCfg<CFG> C;
  constexpr int NT = 64 * C::WGM * C::WGN;
  constexpr size_t lds = C::STAGES * (size_t)(C::BM + C::BN) * C::BK * 2;
  static bool attr = false;
  if (lds > 65536 && !attr) {
    if (hipFuncSetAttribute((const void*)gemm_tile<T, CFG, A_K, B_K, KT, RS>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return fail(MI355X_ELAUNCH, "mi355x_gemm: cannot reserve %zu bytes of LDS", lds);
    attr = true;
  }
  gemm_tile<T, CFG, A_K, B_K, KT, RS><<<grid, NT, lds, s>>>(g);
  return check_launch("mi355x_gemm");
}

template <typename T, int CFG, bool KT, bool RS>
int launch_layout(const GemmArgs& g, dim3 grid, hipStream_t s) {
  const bool ak = g.a_cs == 1, bk = g.b_rs == 1;
  if constexpr (CFG == 3) {  // chosen for m-contiguous A only
    if (ak) return fail(MI355X_EINVAL, "mi355x_gemm: 32-k C256 tiles take an m-contiguous A");
    if (bk) return launch_kernel<T, CFG, false, true, KT, RS>(g, grid, s);
    return launch_kernel<T, CFG, false, false, KT, RS>(g, grid, s);
  } else if constexpr (CFG == 2) {  // 192-wide B tiles are only loaded k-contiguous
    if (!bk) return fail(MI355X_EINVAL, "mi355x_gemm: 128x192 tiles need a k-contiguous B");
    if (ak) return launch_kernel<T, CFG, true, true, KT, RS>(g, grid, s);
    return launch_kernel<T, CFG, false, true, KT, RS>(g, grid, s);
  } else {
    if (ak && bk) return launch_kernel<T, CFG, true, true, KT, RS>(g, grid, s);
    if (ak) return launch_kernel<T, CFG, true, false, KT, RS>(g, grid, s);
    if (bk) return launch_kernel<T, CFG, false, true, KT, RS>(g, grid, s);
    return launch_kernel<T, CFG, false, false, KT, RS>(g, grid, s);
  }
}

template <typename T, int CFG, bool KT>
int launch_tile(GemmArgs g, int64_t batch, int splits, hipStream_t s) {
  typedef TileCfg<CFG> C;
  const int tm = (int)ceil_div(g.m, C::BM), tn = (int)ceil_div(g.n, C::BN);
  g.tiles_n = tn;
  g.batch = (int)batch;
  dim3 grid((unsigned)(tm * tn), (unsigned)(batch * splits));
  if (g.rowsum) return launch_layout<T, CFG, KT, true>(g, grid, s);
  return launch_layout<T, CFG, KT, false>(g, grid, s);
}

// Sum the split-K partials into C and, with rs_slots > 0, the row-sum
// partials into the row sums; returns -1 when the C sum needs the scalar
// kernel (then the caller sums the row sums itself).
int splitk_finish(const GemmArgs& g, int64_t batch, int splits, int rs_slots, hipStream_t s) {
  const int64_t total = batch * g.m * g.n;
  const int64_t c_align = g.c_dt == MI355X_F32 ? 16 : 8;
  if (g.n % 4 == 0 && g.c_rs % 4 == 0 && g.c_bs % 4 == 0 && (uintptr_t)g.c % c_align == 0 &&
      (int64_t)splits * total < (1ll << 31)) {
    int64_t blocks = (total / 4 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (rs_slots > 0) {
      const int64_t rblocks = min((batch * g.m + 31) / 32, (int64_t)65536);
      const unsigned grid = (unsigned)(blocks + rblocks);
      switch (g.c_dt) {
        case MI355X_F32: splitk_rowsum_reduce<float><<<grid, 256, 0, s>>>(g, splits, (int)batch, rs_slots, (uint32_t)blocks); break;
        case MI355X_BF16: splitk_rowsum_reduce<bf16><<<grid, 256, 0, s>>>(g, splits, (int)batch, rs_slots, (uint32_t)blocks); break;
        default: splitk_rowsum_reduce<f16><<<grid, 256, 0, s>>>(g, splits, (int)batch, rs_slots, (uint32_t)blocks); break;
      }
      return check_launch("mi355x_gemm splitk_rowsum_reduce");
    }
    switch (g.c_dt) {
      case MI355X_F32: splitk_reduce4<float><<<(unsigned)blocks, 256, 0, s>>>(g, splits, (int)batch); break;
      case MI355X_BF16: splitk_reduce4<bf16><<<(unsigned)blocks, 256, 0, s>>>(g, splits, (int)batch); break;
      default: splitk_reduce4<f16><<<(unsigned)blocks, 256, 0, s>>>(g, splits, (int)batch); break;
    }
    return check_launch("mi355x_gemm splitk_reduce");
  }
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  splitk_reduce<<<(unsigned)blocks, 256, 0, s>>>(g, splits, batch);
  const int rc = check_launch("mi355x_gemm splitk_reduce");
  return rc ? rc : -1;
}

template <typename T>
int launch_mfma(GemmArgs g, int64_t batch, const Plan& p, hipStream_t s) {
  const bool kt = g.k % 64 != 0;
  int rc;
  if (p.cfg == 1) rc = kt ? launch_tile<T, 1, true>(g, batch, p.splits, s) : launch_tile<T, 1, false>(g, batch, p.splits, s);
  else if (p.cfg == 3) rc = kt ? launch_tile<T, 3, true>(g, batch, p.splits, s) : launch_tile<T, 3, false>(g, batch, p.splits, s);
  else if (p.cfg == 2) rc = kt ? launch_tile<T, 2, true>(g, batch, p.splits, s) : launch_tile<T, 2, false>(g, batch, p.splits, s);
  else rc = kt ? launch_tile<T, 0, true>(g, batch, p.splits, s) : launch_tile<T, 0, false>(g, batch, p.splits, s);
  if (rc || !g.part) return rc;
  const int rs_slots = g.rowsum ? (int)(p.splits * rs_slots_of(p.cfg, g.n)) : 0;
  rc = splitk_finish(g, batch, p.splits, rs_slots, s);
  if (rc != -1) return rc;  // done (or failed)
  if (!g.rowsum) return MI355X_OK;
  const int64_t blocks = min((batch * g.m + 31) / 32, (int64_t)65536);
  rowsum_reduce<<<(unsigned)blocks, 256, 0, s>>>(g, (int)(p.splits * rs_slots_of(p.cfg, g.n)), batch);
  return check_launch("mi355x_gemm rowsum_reduce");
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
  // In place when every 16-byte load is aligned: k-contiguous operands need
  // an 8-element row stride, m/n-contiguous ones an 8-element k stride.  K
  // tails are masked in the kernel; a last partial 8-element chunk may read
  // into row padding, so the contiguous extent must be padded to 8.
  auto up8 = [](int64_t v) { return (v + 7) / 8 * 8; };
  auto in_place = [&](const void* p, int64_t rs, int64_t cs, int64_t bs, int64_t nrows) {
    if (bs % 8 != 0 || (p != nullptr && !aligned16(p))) return false;
    if (cs == 1) return rs % 8 == 0 && rs >= up8(k);
    return cs % 8 == 0 && cs >= up8(nrows);
  };
  // An m/n-contiguous operand that is small next to the product (a weight in
  // dX = dY W) is still packed: the copy costs under ~3% of the GEMM and the
  // k-contiguous fragment reads are cheaper than transposing ones.
  static const char* no_small_pack = getenv("MI355X_GEMM_NO_SMALL_PACK");  // tuning override
  // Not at k <= 1024: there one pass over the weight is a large share of the
  // GEMM, and the transposing reads cost little over so few k-steps (dX of a
  // 768-wide projection: 908 -> 977 TF/s in place).
  const double small_rows = no_small_pack || k <= 1024 ? 0.0 : 2e-4 * (double)m * (double)n;
  w.pack_a = !in_place(a, a_rs, a_cs, a_bs, m) || (a_cs != 1 && (double)m < small_rows);
  // B as [n rows][k]: row stride b_cs, k stride b_rs
  w.pack_b = !in_place(b, b_cs, b_rs, b_bs, n) || (b_rs != 1 && (double)n < small_rows);
  w.plan = plan_gemm(batch, m, n, k, w.pack_a || a_cs == 1, w.pack_b || b_rs == 1);
  auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
  // split-K partials of C, then of the optional row sums of A
  w.part_bytes = w.plan.splits > 1 ? up((int64_t)w.plan.splits * batch * m * n * 4) +
                                         up((int64_t)w.plan.splits * rs_slots_of(w.plan.cfg, n) * batch * m * 4)
                                   : 0;
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
  const int64_t stride = transposed ? k_stride : row_stride;
  const bool v8 = aligned16(src) && stride % 8 == 0 && sbs % 8 == 0 && ld % 64 == 0 &&
                  (!transposed || rows % 8 == 0);
  if (v8) {
    pack_k_contig_v8<<<grid, 256, 0, s>>>(dst, ld, rows * ld, (const uint16_t*)src, stride, sbs, rows, kdim,
                                          transposed ? 1 : 0);
    return check_launch("mi355x_gemm pack");
  }
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

extern "C" int mi355x_gemm_ex(void* c, int c_dtype, int64_t c_rs, int64_t c_bs, const void* a,
                              int64_t a_rs, int64_t a_cs, int64_t a_bs, const void* b, int64_t b_rs,
                              int64_t b_cs, int64_t b_bs, int ab_dtype, const void* bias,
                              int bias_dtype, int flags, void* a_rowsum, int a_rowsum_dtype,
                              int64_t batch, int64_t m, int64_t n, int64_t k, void* workspace,
                              int64_t ws_bytes, mi355x_stream_t stream) {
  MI_REQUIRE(fdt(ab_dtype) && fdt(c_dtype), "mi355x_gemm: unsupported dtype");
  MI_REQUIRE(!bias || fdt(bias_dtype), "mi355x_gemm: unsupported bias dtype");
  MI_REQUIRE(!a_rowsum || fdt(a_rowsum_dtype), "mi355x_gemm: unsupported row-sum dtype");
  MI_REQUIRE((flags & ~(MI355X_GEMM_BETA | MI355X_GEMM_ROUND)) == 0, "mi355x_gemm: unknown flags %d", flags);
  const int beta = (flags & MI355X_GEMM_BETA) ? 1 : 0;
  const int round_c = (flags & MI355X_GEMM_ROUND) ? 1 : 0;
  MI_REQUIRE(!(beta && round_c), "mi355x_gemm: ROUND cannot be combined with BETA");
  MI_REQUIRE(batch >= 1 && m >= 0 && n >= 0 && k >= 0, "mi355x_gemm: bad shape");
  MI_REQUIRE(batch < 65536 && m < (1ll << 31) && n < (1ll << 31), "mi355x_gemm: shape too large");
  if (m == 0 || n == 0) return MI355X_OK;
  MI_REQUIRE(k > 0, "mi355x_gemm: k == 0 must be handled by the caller");
  MI_REQUIRE(a_rs == 1 || a_cs == 1, "mi355x_gemm: A needs a unit row or column stride");
  MI_REQUIRE(b_rs == 1 || b_cs == 1, "mi355x_gemm: B needs a unit row or column stride");
  MI_REQUIRE(c && a && b, "mi355x_gemm: null pointer");
  hipStream_t s = (hipStream_t)stream;
  GemmArgs g{c, c_dtype, c_rs, c_bs, a, a_rs, a_cs, a_bs, b, b_rs, b_cs, b_bs, bias, bias_dtype,
             beta, m, n, k, nullptr, k, 1, 1, ab_dtype, round_c, a_rowsum, a_rowsum_dtype, nullptr};
  if (ab_dtype == MI355X_F32) {
    MI_REQUIRE(!a_rowsum && !round_c, "mi355x_gemm: row sums and ROUND need 16-bit operands");
    dim3 grid(ceil_div(n, 64), ceil_div(m, 64), (unsigned)batch);
    gemm_f32<<<grid, 256, 0, s>>>(g);
    return check_launch("mi355x_gemm");
  }
  WsLayout w = ws_layout(batch, m, n, k, a, a_rs, a_cs, a_bs, b, b_rs, b_cs, b_bs);
  MI_REQUIRE(batch * w.plan.splits < 65536, "mi355x_gemm: batch x splits too large");
  MI_REQUIRE(tiles_of(w.plan.cfg, 1, m, n) < (1ll << 31), "mi355x_gemm: shape too large");
  // the epilogue addresses a tile with 32-bit offsets: 256 rows of C (or of
  // the n-wide split-K partials) must span less than 2^31 elements
  MI_REQUIRE(c_rs < (1ll << 22) && n < (1ll << 22), "mi355x_gemm: C row stride too large");
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
    g.rs_part = (float*)(ws + (((int64_t)w.plan.splits * batch * m * n * 4 + 255) / 256 * 256));
  }
  if (ab_dtype == MI355X_BF16) return launch_mfma<bf16>(g, batch, w.plan, s);
  return launch_mfma<f16>(g, batch, w.plan, s);
}

extern "C" int mi355x_gemm(void* c, int c_dtype, int64_t c_rs, int64_t c_bs, const void* a,
                           int64_t a_rs, int64_t a_cs, int64_t a_bs, const void* b, int64_t b_rs,
                           int64_t b_cs, int64_t b_bs, int ab_dtype, const void* bias,
                           int bias_dtype, int beta, int64_t batch, int64_t m, int64_t n,
                           int64_t k, void* workspace, int64_t ws_bytes, mi355x_stream_t stream) {
  return mi355x_gemm_ex(c, c_dtype, c_rs, c_bs, a, a_rs, a_cs, a_bs, b, b_rs, b_cs, b_bs, ab_dtype, bias,
                        bias_dtype, beta ? MI355X_GEMM_BETA : 0, nullptr, 0, batch, m, n, k, workspace,
                        ws_bytes, stream);
}
