// The decode GEMM formulated on the VALU with v_dot4_i32_i8 instead of MFMA:
// a measured alternative to the MFMA decode kernels (the int32 accumulators of
// y = q @ w for M <= 32 token rows, exact).  bench.py times it beside
// btl_gemm_i8t2 on the same operands; the library's decode paths use MFMA.
//
// Workgroup (column tile t, K split s): 256 threads.  Lane l of wave w owns
// column t*32 + (l & 31) and the 16-k half h = l >> 5 of 32-k step q = w of
// each superblock (128 k) of the split.  Per superblock:
//   - the workgroup stages the 32 activation rows' 128 bytes (4 KiB, the
//     operand tile's superblock) in LDS, double-buffered;
//   - each lane loads its weight dword (16 offset codes u = w + 1 of its
//     column, k = 128 ks + 32 w + 16 h + j), unpacks it into four dwords of
//     four codes, and for each of the 32 rows reads the row's 16 activation
//     bytes of that k range (one LDS read, the same address for the 32 lanes
//     of a half-wave) and accumulates four v_dot4_i32_i8.
// The eight (wave, half) partials of the 32x32 tile meet in LDS; split 0
// subtracts the row sums (sum_k q u = sum_k q w + sum_k q), and every split
// adds its tile into acc_out with device-scope integer atomics (exact in any
// order; acc_out starts at zero).
#include "btl_act_row.h"
#include "btl_mfma.h"

namespace btl {

__global__ __launch_bounds__(256) void k_gemm_decode_dot4(const int8_t* xa, const int32_t* rowsum, int M, int KS,
                                                          int NT, int nsplit, const uint32_t* wdev, int32_t* acc_out,
                                                          int N) {
  __shared__ __attribute__((aligned(16))) int8_t s_a[2][4096];
  __shared__ int32_t s_red[8][32][33];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, c = lane & 31;
  const int t = blockIdx.x % NT, s = blockIdx.x / NT;
  const int sb0 = (s * KS) / nsplit, sb1 = ((s + 1) * KS) / nsplit;
  int32_t acc[32];
#pragma unroll
  for (int m = 0; m < 32; ++m) acc[m] = 0;
  // operand superblock sb: 4 KiB at xa + sb * 4096 (row block 0), one 16-byte
  // chunk per thread
  if (sb0 < sb1) *reinterpret_cast<v4i*>(s_a[0] + tid * 16) = ld128(xa + (int64_t)sb0 * 4096 + tid * 16);
  __syncthreads();
  for (int sb = sb0; sb < sb1; ++sb) {
    const int cur = (sb - sb0) & 1;
    v4i nxt = (v4i){0, 0, 0, 0};
    if (sb + 1 < sb1) nxt = ld128(xa + (int64_t)(sb + 1) * 4096 + tid * 16);
    const uint32_t d = wdev[(((int64_t)t * KS + sb) * 64 + lane) * 4 + w];
    const v4i u = unpack_b(d);
    const int8_t* a0 = s_a[cur] + (w * 64 + 32 * h) * 16;  // row m at a0 + 16 m
#pragma unroll
    for (int m = 0; m < 32; ++m) {
      const v4i a = *reinterpret_cast<const v4i*>(a0 + 16 * m);
      int32_t v = acc[m];
      v = __builtin_amdgcn_sdot4(a.x, u.x, v, false);
      v = __builtin_amdgcn_sdot4(a.y, u.y, v, false);
      v = __builtin_amdgcn_sdot4(a.z, u.z, v, false);
      v = __builtin_amdgcn_sdot4(a.w, u.w, v, false);
      acc[m] = v;
    }
    if (sb + 1 < sb1) *reinterpret_cast<v4i*>(s_a[cur ^ 1] + tid * 16) = nxt;
    __syncthreads();
  }
#pragma unroll
  for (int m = 0; m < 32; ++m) s_red[w * 2 + h][m][c] = acc[m];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int m = (tid >> 5) + 8 * k, col = tid & 31;
    int32_t v = 0;
#pragma unroll
    for (int g = 0; g < 8; ++g) v += s_red[g][m][col];
    if (m < M) {
      if (s == 0) v -= rowsum[m];
      atomicAdd(acc_out + (int64_t)m * N + t * 32 + col, v);
    }
  }
}

}  // namespace btl

using namespace btl;

extern "C" {

int btl_gemm_i8t2_dot4(const int8_t* xa, const int32_t* rowsum, int64_t M, int64_t K, int64_t N,
                       const uint32_t* wdev, int32_t* acc_out, btl_stream_t stream) {
  clear_error();
  if (M <= 0 || M > 32 || K <= 0 || K % 128 || N <= 0 || N % 32 || K > BTL_MAX_K)
    return set_error(BTL_ERR_SHAPE, "btl_gemm_i8t2_dot4: M=%lld (1..32), K=%lld (a multiple of 128), N=%lld "
                     "(a multiple of 32)", (long long)M, (long long)K, (long long)N);
  if (!xa || !rowsum || !wdev || !acc_out) return set_error(BTL_ERR_NULL, "btl_gemm_i8t2_dot4: null pointer");
  if (!aligned(xa, 16) || !aligned(rowsum, 4) || !aligned(wdev, 16) || !aligned(acc_out, 4))
    return set_error(BTL_ERR_ALIGN, "btl_gemm_i8t2_dot4: misaligned buffer");
  const int KS = (int)(K / 128), NT = (int)(N / 32);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess)
    return set_error(BTL_ERR_LAUNCH, "btl_gemm_i8t2_dot4: no device");
  // about two workgroups per CU, at least one superblock each
  int nsplit = (2 * cus + NT - 1) / NT;
  if (nsplit > KS) nsplit = KS;
  if (nsplit < 1) nsplit = 1;
  hipLaunchKernelGGL(k_gemm_decode_dot4, dim3(NT * nsplit), dim3(256), 0, (hipStream_t)stream, xa, rowsum, (int)M,
                     KS, NT, nsplit, wdev, acc_out, (int)N);
  return check_launch("dot4 GEMM");
}

}  // extern "C"
