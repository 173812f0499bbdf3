// CDNA4 (gfx950) MFMA helpers shared by the GEMM and attention kernels.
//
// v_mfma_f32_16x16x32_{bf16,f16}: one wave computes a 16x16 f32 tile
//   C[m][n] += sum_{k<32} A[m][k] * B[k][n]
// Operand layout (lane l, g = l/16):
//   A: 8 values A[l%16][8g .. 8g+7]
//   B: 8 values B[8g .. 8g+7][l%16]
//   C: 4 values C[4g .. 4g+3][l%16]
// Only the pairing of k indices between A and B matters to the product, so
// a kernel may feed any permutation of the 32 k values as long as A and B
// use the same one (the attention kernels rely on this).
#pragma once
#include "common.h"

namespace mi {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// This thread's wave within the block, in a scalar register.  Conditions
// built from it are then scalar branches.  As a per-lane value the compiler
// would treat them as divergent and guard their code with the exec mask,
// and an MFMA under an exec mask still executes, reading operands whose
// (masked-off) VALU set-up never ran.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

template <typename T>
struct Mfma;

template <>
struct Mfma<bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<f16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

}  // namespace mi
