// Operand helpers of the int8 x ternary MFMA (v_mfma_i32_32x32x32_i8) shared
// by the GEMM kernels.  The row-half decode body regroups the packed words
// across lanes for v_mfma_i32_16x16x64_i8 before unpacking them here.
//
// Weights are stored as offset codes u = w + 1 in {0,1,2}, 2 bits each, in
// MFMA operand order: dword q of lane `lane` in superblock ks of column tile
// nt holds the 16 codes of column nt*32 + (lane & 31) for rows
// ks*128 + q*32 + (lane >> 5)*16 + j, code j at bit 8*(j & 3) + 2*(j >> 2).
// Unpacking one dword into the 16 B operand bytes is one shift and one AND
// per operand dword.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace btl {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v4i unpack_b(uint32_t d) {
  const int m = 0x03030303;
  v4i b;
  b.x = (int)(d & m);
  b.y = (int)((d >> 2) & m);
  b.z = (int)((d >> 4) & m);
  b.w = (int)((d >> 6) & m);
  return b;
}

__device__ __forceinline__ v4i ld128(const void* p) { return *reinterpret_cast<const v4i*>(p); }

// 16-byte load through a pointer known to address global memory.  A pointer
// read from memory (a table of weight addresses) is generic to the compiler,
// which then emits a flat load; flat loads count in the LDS/scalar counter as
// well, so every later LDS wait would also wait for them.
__device__ __forceinline__ v4i ldg128(const void* p) {
  return *(const __attribute__((address_space(1))) v4i*)p;
}

// Row of element r (0..15) of a lane's 32x32 MFMA accumulator (its column is
// lane & 31).
__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// Sum of the 16 int8 operand bytes of a lane (one v_dot4 per dword).
__device__ __forceinline__ int32_t bytes_sum(v4i a, int32_t acc) {
  acc = __builtin_amdgcn_sdot4(a.x, 0x01010101, acc, false);
  acc = __builtin_amdgcn_sdot4(a.y, 0x01010101, acc, false);
  acc = __builtin_amdgcn_sdot4(a.z, 0x01010101, acc, false);
  return __builtin_amdgcn_sdot4(a.w, 0x01010101, acc, false);
}

}  // namespace btl
