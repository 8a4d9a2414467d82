// Shared helpers of the gfx950 BitLinear library: bf16 conversion, error
// reporting, argument checks and the quantities that describe the layouts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "btl.h"

namespace btl {

// ---- bf16 (round to nearest even; NaN stays a quiet NaN) --------------
__host__ __device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
__host__ __device__ __forceinline__ uint16_t f2bf(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  // v_cvt_pk_bf16_f32: round to nearest even in one instruction.
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
#endif
}

// Two values at once, f2bf of each: lo in bits 15:0, hi in bits 31:16 (one
// v_cvt_pk_bf16_f32 on the device).
__host__ __device__ __forceinline__ uint32_t f2bf_pair(float lo, float hi) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
#else
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
#endif
}

// ---- errors -------------------------------------------------------------
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
int check_launch(const char* what);

// Co-residency of a grid whose workgroups wait on each other: BTL_OK when
// `grid` workgroups fit at once (per_cu x cus), else BTL_ERR_LAUNCH with a
// message.  check_coresident_launch queries the kernel's occupancy and the
// CUs the stream may use.
int coresident_check(const char* who, int64_t grid, int64_t per_cu, int64_t cus);
int stream_cus(hipStream_t s);
int kernel_per_cu(const void* kernel, int threads);
int check_coresident_launch(const char* who, const void* kernel, int threads, int64_t grid, hipStream_t s);

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// ---- layout quantities ----------------------------------------------------
// Weights: K rows (in_features) x N columns (out_features); the device layout
// is N/32 column tiles x ceil(K/128) superblocks x 1 KiB.
inline int64_t ksb(int64_t K) { return (K + 127) / 128; }
// Activations: ceil(M/32) blocks of 32 rows, each ksb(K) superblocks x 4 KiB.
inline int64_t mblocks(int64_t M) { return (M + 31) / 32; }
inline int64_t round_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// ---- GEMM plan (shared by sizing functions and launches) ----------------
struct GemmPlan {
  bool prefill;   // M > 32: tiled kernel over 32-row blocks
  bool fused;     // decode: activation prologue and GEMM in one launch
  int tpw;        // decode: column tiles per workgroup (2 for the relu2 pair)
  int waves;      // decode: waves per workgroup (4 or 8), splitting the slice's K
  int ngroups;    // decode: workgroups along N
  int splitk;     // decode: workgroups along K
  int mh;         // fused decode: workgroups along M (2: 16 rows each)
  bool half16;    // fused decode, M <= 16: one 16-row workgroup per column group
  int64_t ws_bytes;
};
GemmPlan plan_gemm(int64_t M, int64_t K, int64_t N, int epilogue, int splitk_req);

// Byte offsets inside the fused workspace (the first kSyncBytes hold the
// handshake words of the single-launch decode kernel, its error word among
// them).
struct FusedLayout {
  int64_t xa, a_dq, rowsum, gemm_ws, total;
};
FusedLayout fused_layout(int64_t M, int64_t K, int64_t N, int epilogue, int splitk_req);

}  // namespace btl
