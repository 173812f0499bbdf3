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

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Byte offset of a shared-memory pointer within the block's LDS.
__device__ __forceinline__ unsigned lds_off(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Direct global -> LDS loads (global_load_lds_dword{,x4}: each lane's 4 or 16
// bytes land at lds_base + 4/16 * lane), issued from inline assembly.  The
// builtin form is not used because the compiler then treats every later
// transposing LDS read as a possible reader of the in-flight load and puts a
// vmcnt(0) in front of it, so a pipeline that issues the next tiles before
// reading the current one would wait for its newest loads on every step.
// Callers wait for these loads themselves (explicit vmcnt waits + barriers).
// lds_base must be wave-uniform; it is written to M0 here.
__device__ __forceinline__ void dma_b128(const void* gptr, unsigned lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "s"(lds_base) : "memory", "m0");
}
__device__ __forceinline__ void dma_b32(const void* gptr, unsigned lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" : : "v"(gptr), "s"(lds_base) : "memory", "m0");
}
// Wave-uniform LDS byte offset of a shared-memory pointer.
__device__ __forceinline__ unsigned lds_base_of(const void* p) { return __builtin_amdgcn_readfirstlane(lds_off(p)); }

// Transposing 8-byte LDS read (ds_read_b64_tr_b16).
__device__ __forceinline__ s16x4 ds_read_tr(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
}

// Fragment from two transposed 4-element pieces: slots 0-3 = a, 4-7 = b.
template <typename F>
__device__ __forceinline__ F join_frag(s16x4 a, s16x4 b) {
  F f;
  short* fs = (short*)&f;
#pragma unroll
  for (int e = 0; e < 4; ++e) fs[e] = a[e], fs[4 + e] = b[e];
  return f;
}

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
