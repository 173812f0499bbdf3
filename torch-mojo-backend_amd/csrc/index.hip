// Row gathers (index_select, embedding forward) and the deterministic
// embedding backward.
//
// Gathers copy whole rows: one 64-lane wave per output row, 16-byte accesses
// when the row size and pointers allow, so every row is one coalesced read
// and one coalesced write.  An index outside [0, rows) is never dereferenced:
// its row is zero-filled and the caller's error flag is raised.
//
// Embedding backward (the counterpart of embedding_dense_backward, which
// ATen's CPU kernel computes as an index_add in index order):
//   1. stable radix sort of (idx[n], n) pairs -> positions grouped by row,
//      ascending within each row;
//   2. one wave per weight row finds its segment (a wave-wide 64-ary search)
//      and sums the grad rows in that order into f32, then writes the row
//      once.
// Every weight row is written exactly once (no zero pre-pass, no atomics),
// and the per-row summation order equals the sequential CPU order, so f32
// results match ATen's CPU result bit for bit.
#include <hipcub/hipcub.hpp>

#include "common.h"
#include "vec.h"

namespace mi {
namespace {

constexpr int kThreads = 256;

// out[o, j, :] = in[o*so + idx[j]*sj, :], row of `row_bytes` bytes.
template <typename V>
__global__ void __launch_bounds__(kThreads)
    gather_rows(uint8_t* __restrict__ out, const uint8_t* __restrict__ in,
                const int64_t* __restrict__ idx, int64_t outer, int64_t n_idx, int64_t rows,
                int64_t row_bytes, int64_t so_bytes, int64_t sj_bytes, int32_t* err) {
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (job >= outer * n_idx) return;
  const int64_t o = job / n_idx, j = job % n_idx;
  const int64_t r = idx[j];
  V* dst = (V*)(out + job * row_bytes);
  const int64_t nv = row_bytes / (int64_t)sizeof(V);
  if (r < 0 || r >= rows) {
    if (lane == 0 && err) *err = 1;
    V z;
    memset(&z, 0, sizeof(V));
    for (int64_t k = lane; k < nv; k += 64) dst[k] = z;
    return;
  }
  const V* src = (const V*)(in + o * so_bytes + r * sj_bytes);
  for (int64_t k = lane; k < nv; k += 64) dst[k] = src[k];
}

int launch_gather(void* out, const void* in, const int64_t* idx, int64_t outer, int64_t n_idx,
                  int64_t rows, int64_t row_bytes, int64_t so_bytes, int64_t sj_bytes,
                  int32_t* err, hipStream_t s) {
  const int64_t jobs = outer * n_idx;
  if (jobs == 0 || row_bytes == 0) return MI355X_OK;
  const unsigned grid = ceil_div(jobs, kThreads / 64);
  auto al = [](int64_t v, int64_t a) { return v % a == 0; };
  const bool a16 = al(row_bytes, 16) && al(so_bytes, 16) && al(sj_bytes, 16) &&
                   al((int64_t)(uintptr_t)out, 16) && al((int64_t)(uintptr_t)in, 16);
  const bool a4 = al(row_bytes, 4) && al(so_bytes, 4) && al(sj_bytes, 4) &&
                  al((int64_t)(uintptr_t)out, 4) && al((int64_t)(uintptr_t)in, 4);
  if (a16)
    gather_rows<uint4><<<grid, kThreads, 0, s>>>((uint8_t*)out, (const uint8_t*)in, idx, outer, n_idx,
                                                 rows, row_bytes, so_bytes, sj_bytes, err);
  else if (a4)
    gather_rows<uint32_t><<<grid, kThreads, 0, s>>>((uint8_t*)out, (const uint8_t*)in, idx, outer,
                                                    n_idx, rows, row_bytes, so_bytes, sj_bytes, err);
  else
    gather_rows<uint8_t><<<grid, kThreads, 0, s>>>((uint8_t*)out, (const uint8_t*)in, idx, outer,
                                                   n_idx, rows, row_bytes, so_bytes, sj_bytes, err);
  return check_launch("gather_rows");
}

__global__ void iota_i32(int32_t* v, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) v[i] = (int32_t)i;
}

// First index in [0, n) whose sorted key is >= target (n if none), found by
// the whole wave: each round the 64 lanes probe 64 evenly spaced keys and a
// ballot narrows the range 64-fold, so a search of n = 16384 keys costs
// three dependent loads instead of fourteen.  Wave-uniform result.
__device__ __forceinline__ int64_t wave_lower_bound(const int64_t* __restrict__ keys, int64_t n,
                                                     int64_t target, int lane) {
  int64_t lo = 0, hi = n;  // the answer lies in [lo, hi]
  while (hi - lo > 64) {
    const int64_t step = (hi - lo + 63) / 64;
    const int64_t i = lo + (int64_t)lane * step;
    const bool ge = i >= hi || keys[i] >= target;
    const uint64_t m = __ballot(ge);
    const int f = m ? __ffsll((unsigned long long)m) - 1 : 64;  // first probe >= target
    const int64_t nlo = f == 0 ? lo : lo + (int64_t)(f - 1) * step + 1;
    const int64_t nhi = f == 64 ? hi : min(hi, lo + (int64_t)f * step);
    lo = nlo;
    hi = nhi;
  }
  const int64_t i = lo + lane;
  const bool ge = i >= hi || keys[i] >= target;
  const uint64_t m = __ballot(ge);
  return m ? lo + (__ffsll((unsigned long long)m) - 1) : hi;
}

// One wave per weight row (four rows per block, grid-stride): ordered
// segment sum.  Each lane owns a fixed set of columns and adds the row's
// grad rows in sorted (= index) order, 16 bytes at a time when the row
// allows it.
//
// ACC: gw = base + sum (the sum rounded to T first, then added, as a
// separate `base + dense_sum` would); rows no index names (and the padding
// row) are copied from base, or left untouched when base is gw itself.
template <typename T, bool ACC>
__global__ void __launch_bounds__(kThreads)
    embedding_bwd_rows(T* gw, const T* __restrict__ go, const T* base,
                       const int64_t* __restrict__ keys, const int32_t* __restrict__ pos,
                       int64_t n, int64_t num_weights, int64_t dim, int64_t padding_idx, bool vec4) {
  const int lane = threadIdx.x & 63;
  constexpr int RPB = kThreads / 64;
  for (int64_t row = (int64_t)blockIdx.x * RPB + (threadIdx.x >> 6); row < num_weights;
       row += (int64_t)gridDim.x * RPB) {
    const int64_t lo = wave_lower_bound(keys, n, row, lane);
    const int64_t end = row == padding_idx ? lo : wave_lower_bound(keys, n, row + 1, lane);
    if (ACC && lo == end) {  // wave-uniform
      if (base != gw) {
        if (vec4) {
          for (int64_t c = (int64_t)lane * 4; c < dim; c += 64 * 4) {
            float v[4];
            Vec4<T>::load(base + row * dim + c, v);
            Vec4<T>::store(gw + row * dim + c, v);
          }
        } else {
          for (int64_t c = lane; c < dim; c += 64) gw[row * dim + c] = base[row * dim + c];
        }
      }
      continue;
    }
    if (vec4) {
      for (int64_t c = (int64_t)lane * 4; c < dim; c += 64 * 4) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int64_t k = lo; k < end; ++k) {
          float v[4];
          Vec4<T>::load(go + (int64_t)pos[k] * dim + c, v);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[e] += v[e];
        }
        if constexpr (ACC) {
          float cur[4];
          Vec4<T>::load(base + row * dim + c, cur);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[e] = cur[e] + to_f32(from_f32<T>(acc[e]));
        }
        Vec4<T>::store(gw + row * dim + c, acc);
      }
    } else {
      for (int64_t c = lane; c < dim; c += 64) {
        float acc = 0.f;
        for (int64_t k = lo; k < end; ++k) acc += to_f32(go[(int64_t)pos[k] * dim + c]);
        if constexpr (ACC) acc = to_f32(base[row * dim + c]) + to_f32(from_f32<T>(acc));
        gw[row * dim + c] = from_f32<T>(acc);
      }
    }
  }
}

struct EmbWs {
  size_t keys_off, vals_in_off, vals_out_off, temp_off, temp_bytes, total;
};

EmbWs emb_ws_layout(int64_t n) {
  size_t temp = 0;
  hipcub::DeviceRadixSort::SortPairs(nullptr, temp, (const int64_t*)nullptr, (int64_t*)nullptr,
                                     (const int32_t*)nullptr, (int32_t*)nullptr, (int)n);
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  EmbWs w;
  w.keys_off = 0;
  w.vals_in_off = up(w.keys_off + (size_t)n * 8);
  w.vals_out_off = up(w.vals_in_off + (size_t)n * 4);
  w.temp_off = up(w.vals_out_off + (size_t)n * 4);
  w.temp_bytes = temp;
  w.total = up(w.temp_off + temp);
  return w;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi355x_index_select(void* out, const void* in, int dtype, const int64_t* idx,
                                   int64_t outer, int64_t n_idx, int64_t in_rows, int64_t inner,
                                   int64_t in_so, int64_t in_sj, int32_t* err_flag,
                                   mi355x_stream_t stream) {
  const int64_t es = (int64_t)dtype_size(dtype);
  MI_REQUIRE(es > 0, "mi355x_index_select: bad dtype");
  MI_REQUIRE(outer >= 0 && n_idx >= 0 && inner >= 0, "mi355x_index_select: negative extent");
  return launch_gather(out, in, idx, outer, n_idx, in_rows, inner * es, in_so * es, in_sj * es,
                       err_flag, (hipStream_t)stream);
}

extern "C" int mi355x_embedding_fwd(void* out, const void* weight, int dtype, const int64_t* idx,
                                    int64_t n_idx, int64_t num_weights, int64_t dim,
                                    int64_t w_row_stride, int32_t* err_flag,
                                    mi355x_stream_t stream) {
  const int64_t es = (int64_t)dtype_size(dtype);
  MI_REQUIRE(es > 0, "mi355x_embedding_fwd: bad dtype");
  MI_REQUIRE(n_idx >= 0 && dim >= 0 && num_weights >= 0, "mi355x_embedding_fwd: bad shape");
  return launch_gather(out, weight, idx, 1, n_idx, num_weights, dim * es, 0, w_row_stride * es,
                       err_flag, (hipStream_t)stream);
}

extern "C" int64_t mi355x_embedding_bwd_workspace_bytes(int64_t n_idx, int64_t num_weights) {
  (void)num_weights;
  return (int64_t)emb_ws_layout(n_idx).total;
}

namespace {
int embedding_bwd_impl(const char* name, bool accumulate, void* grad_weight, const void* base, const void* grad_out,
                       int dtype,
                       const int64_t* idx, int64_t n_idx, int64_t num_weights, int64_t dim, int64_t padding_idx,
                       void* workspace, int64_t ws_bytes, hipStream_t s) {
  MI_REQUIRE(n_idx >= 0 && n_idx < (1ll << 31), "%s: bad index count", name);
  MI_REQUIRE(num_weights >= 0 && dim >= 0, "%s: bad shape", name);
  if (num_weights == 0 || dim == 0) return MI355X_OK;
  const EmbWs w = emb_ws_layout(n_idx);
  if (n_idx > 0 && (!workspace || ws_bytes < (int64_t)w.total))
    return fail(MI355X_EWORKSPACE, "%s: workspace %lld < %lld", name, (long long)ws_bytes, (long long)w.total);
  uint8_t* wsb = (uint8_t*)workspace;
  int64_t* keys = (int64_t*)(wsb + w.keys_off);
  int32_t* vin = (int32_t*)(wsb + w.vals_in_off);
  int32_t* vout = (int32_t*)(wsb + w.vals_out_off);
  if (n_idx > 0) {
    iota_i32<<<ceil_div(n_idx, kThreads), kThreads, 0, s>>>(vin, n_idx);
    size_t temp = w.temp_bytes;
    hipError_t e = hipcub::DeviceRadixSort::SortPairs(wsb + w.temp_off, temp, idx, keys, vin, vout,
                                                      (int)n_idx, 0, 64, s);
    if (e != hipSuccess) return fail(MI355X_ELAUNCH, "%s: sort failed: %s", name, hipGetErrorString(e));
  }
  const int64_t blocks = (num_weights + kThreads / 64 - 1) / (kThreads / 64);
  const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
  const size_t es = (size_t)dtype_size(dtype);
  const bool vec4 = dim % 4 == 0 && ((uintptr_t)grad_weight % (4 * es)) == 0 &&
                    ((uintptr_t)grad_out % (4 * es)) == 0 && ((uintptr_t)base % (4 * es)) == 0;
  auto go = [&](auto tag) {
    using T = decltype(tag);
    if (accumulate)
      embedding_bwd_rows<T, true><<<grid, kThreads, 0, s>>>((T*)grad_weight, (const T*)grad_out, (const T*)base,
                                                            keys, vout, n_idx, num_weights, dim, padding_idx, vec4);
    else
      embedding_bwd_rows<T, false><<<grid, kThreads, 0, s>>>((T*)grad_weight, (const T*)grad_out, nullptr, keys,
                                                             vout, n_idx, num_weights, dim, padding_idx, vec4);
  };
  switch (dtype) {
    case MI355X_F32: go(float{}); break;
    case MI355X_BF16: go(bf16{}); break;
    case MI355X_F16: go(f16{}); break;
    default: return fail(MI355X_EUNSUPPORTED, "%s: unsupported dtype %d", name, dtype);
  }
  return check_launch(name);
}
}  // namespace

extern "C" int mi355x_embedding_bwd(void* grad_weight, const void* grad_out, int dtype,
                                    const int64_t* idx, int64_t n_idx, int64_t num_weights,
                                    int64_t dim, int64_t padding_idx, void* workspace,
                                    int64_t ws_bytes, mi355x_stream_t stream) {
  return embedding_bwd_impl("mi355x_embedding_bwd", false, grad_weight, nullptr, grad_out, dtype, idx, n_idx,
                            num_weights, dim, padding_idx, workspace, ws_bytes, (hipStream_t)stream);
}

extern "C" int mi355x_embedding_bwd_accumulate(void* grad_weight, const void* base, const void* grad_out,
                                               int dtype, const int64_t* idx, int64_t n_idx, int64_t num_weights,
                                               int64_t dim, int64_t padding_idx, void* workspace,
                                               int64_t ws_bytes, mi355x_stream_t stream) {
  MI_REQUIRE(grad_weight && base, "mi355x_embedding_bwd_accumulate: null pointer");
  return embedding_bwd_impl("mi355x_embedding_bwd_accumulate", true, grad_weight, base, grad_out, dtype, idx, n_idx,
                            num_weights, dim, padding_idx, workspace, ws_bytes, (hipStream_t)stream);
}
