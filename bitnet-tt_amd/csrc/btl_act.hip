// Activation prologue of a BitLinear: optional RMSNorm, per-token absmax int8
// quantisation, and the blocked layout the ternary GEMM consumes.
//
//   RMSNorm  (HF BitNetRMSNorm order; src/bitnet_tt/layers/bitlinear.py:433-461,
//            fused into the QKV launch at inference/generator_batch32.py:721-727):
//            r = 1/sqrt(sum(x^2)/K + eps); y = bf16(gamma * bf16(x * r))
//   quant    (src/bitnet_tt/utils/quantization.py:60-91):
//            a = max(max|y|, 1e-5); q = clip(rne(y * (127/a)), -128, 127)
//
// One workgroup (256 threads, 4 waves) per token row.  The sum of squares
// follows a fixed order so the statistic is reproducible bit for bit: thread
// t accumulates x^2 over the 8-element chunks t, t+256, ... in order, the 64
// lanes of a wave combine by an xor butterfly (offsets 32..1), and the four
// wave sums combine as (w0+w1)+(w2+w3).  Multiplies and adds are separately
// rounded (built with -ffp-contract=off); division and sqrt are correctly
// rounded.
//
// Quantised output layout (per 32-row block mb, 128-column superblock ks):
// byte (((mb*KS + ks)*4 + q)*64 + lane)*16 + p holds q[mb*32 + (lane & 31)]
// [ks*128 + q*32 + (lane >> 5)*16 + p] -- exactly the 16 bytes lane `lane`
// feeds to v_mfma_i32_32x32x32_i8 for k-step q, so one 1 KiB load per wave
// and k-step brings a whole A operand.  Rows >= M and columns >= K are zero.
#include <math.h>

#include "btl_common.h"

namespace btl {

constexpr int kActThreads = 256;
constexpr int kActMaxChunks = BTL_MAX_K / 8 / kActThreads;  // 8 chunks of 8 per thread

struct ActArgs {
  const uint16_t* x;
  int64_t ldx;
  int M, K, KS;
  const uint16_t* gamma;
  float norm_eps;
  float act_eps;
  int8_t* xa;
  float* a_dq;
  int32_t* rowsum;
  float* act_scale;  // optional [M] 127/a
  int8_t* xq_rm;     // optional [M, K] int8
  uint16_t* y_rm;    // optional [M, K] bf16 (the normalised y)
  uint32_t* zero_words;  // optional words cleared by block 0 (GEMM counters)
  int n_zero_words;
};

__device__ __forceinline__ int64_t xa_offset(int m, int k0, int KS) {
  const int mb = m >> 5, mr = m & 31;
  const int ks = k0 >> 7, qs = (k0 >> 5) & 3, h = (k0 >> 4) & 1, p0 = k0 & 15;
  return ((((int64_t)mb * KS + ks) * 4 + qs) * 64 + (h * 32 + mr)) * 16 + p0;
}

template <bool NORM, bool QUANT>
__global__ __launch_bounds__(kActThreads) void k_act_rows(ActArgs p) {
  const int m = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  __shared__ float s_sum[4];
  __shared__ float s_max[4];
  __shared__ int s_int[4];

  if (p.zero_words && m == 0)
    for (int i = tid; i < p.n_zero_words; i += kActThreads) p.zero_words[i] = 0u;

  const int nch = p.K >> 3;        // 8-element chunks holding data
  const int nchp = p.KS * 16;      // chunks up to the 128-column padding
  if (m >= p.M) {                  // padding row of the last 32-row block
    if (QUANT) {
      for (int c = tid; c < nchp; c += kActThreads)
        *reinterpret_cast<uint2*>(p.xa + xa_offset(m, 8 * c, p.KS)) = make_uint2(0u, 0u);
      if (tid == 0) {
        p.a_dq[m] = 0.0f;
        p.rowsum[m] = 0;
      }
    }
    return;
  }

  const uint16_t* xr = p.x + (int64_t)m * p.ldx;
  float v[kActMaxChunks][8];
#pragma unroll
  for (int i = 0; i < kActMaxChunks; ++i) {
    const int c = tid + kActThreads * i;
    if (c < nch) {
      const uint4 raw = *reinterpret_cast<const uint4*>(xr + 8 * c);
      const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[i][2 * j] = bf2f((uint16_t)(w4[j] & 0xffffu));
        v[i][2 * j + 1] = bf2f((uint16_t)(w4[j] >> 16));
      }
    }
  }

  if (NORM) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kActMaxChunks; ++i)
      if (tid + kActThreads * i < nch) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float sq = v[i][j] * v[i][j];
          s = s + sq;
        }
      }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_xor(s, off, 64);
    if (lane == 0) s_sum[wv] = s;
    __syncthreads();
    const float ss = (s_sum[0] + s_sum[1]) + (s_sum[2] + s_sum[3]);
    const float var = ss / (float)p.K;
    const float r = 1.0f / sqrtf(var + p.norm_eps);
#pragma unroll
    for (int i = 0; i < kActMaxChunks; ++i) {
      const int c = tid + kActThreads * i;
      if (c < nch) {
        uint4 graw = make_uint4(0u, 0u, 0u, 0u);
        if (p.gamma) graw = *reinterpret_cast<const uint4*>(p.gamma + 8 * c);
        const uint32_t g4[4] = {graw.x, graw.y, graw.z, graw.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float t = bf2f(f2bf(v[i][j] * r));
          if (p.gamma) {
            const float g = bf2f((uint16_t)((j & 1) ? (g4[j >> 1] >> 16) : (g4[j >> 1] & 0xffffu)));
            v[i][j] = bf2f(f2bf(g * t));
          } else {
            v[i][j] = t;
          }
        }
      }
    }
  }

  if (!QUANT || p.y_rm) {
    uint16_t* yr = p.y_rm + (int64_t)m * p.K;
#pragma unroll
    for (int i = 0; i < kActMaxChunks; ++i) {
      const int c = tid + kActThreads * i;
      if (c < nch) {
        uint4 o;
        o.x = (uint32_t)f2bf(v[i][0]) | ((uint32_t)f2bf(v[i][1]) << 16);
        o.y = (uint32_t)f2bf(v[i][2]) | ((uint32_t)f2bf(v[i][3]) << 16);
        o.z = (uint32_t)f2bf(v[i][4]) | ((uint32_t)f2bf(v[i][5]) << 16);
        o.w = (uint32_t)f2bf(v[i][6]) | ((uint32_t)f2bf(v[i][7]) << 16);
        *reinterpret_cast<uint4*>(yr + 8 * c) = o;
      }
    }
  }
  if (!QUANT) return;

  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kActMaxChunks; ++i)
    if (tid + kActThreads * i < nch) {
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[i][j]));
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if (lane == 0) s_max[wv] = amax;
  __syncthreads();
  float a = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
  a = a > p.act_eps ? a : p.act_eps;
  const float scale = 127.0f / a;

  int rs = 0;
#pragma unroll
  for (int i = 0; i < kActMaxChunks; ++i) {
    const int c = tid + kActThreads * i;
    if (c < nch) {
      uint32_t lo = 0u, hi = 0u;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float t = rintf(v[i][j] * scale);
        t = fminf(fmaxf(t, -128.0f), 127.0f);
        const int qi = (int)t;
        rs += qi;
        const uint32_t b = (uint32_t)(qi & 0xff);
        if (j < 4) lo |= b << (8 * j);
        else hi |= b << (8 * (j - 4));
      }
      *reinterpret_cast<uint2*>(p.xa + xa_offset(m, 8 * c, p.KS)) = make_uint2(lo, hi);
      if (p.xq_rm) *reinterpret_cast<uint2*>(p.xq_rm + (int64_t)m * p.K + 8 * c) = make_uint2(lo, hi);
    }
  }
  for (int c = nch + tid; c < nchp; c += kActThreads)
    *reinterpret_cast<uint2*>(p.xa + xa_offset(m, 8 * c, p.KS)) = make_uint2(0u, 0u);

#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) rs += __shfl_xor(rs, off, 64);
  if (lane == 0) s_int[wv] = rs;
  __syncthreads();
  if (tid == 0) {
    p.a_dq[m] = a / 127.0f;
    p.rowsum[m] = s_int[0] + s_int[1] + s_int[2] + s_int[3];
    if (p.act_scale) p.act_scale[m] = scale;
  }
}

// Launch helper shared with the fused entry point.
int launch_act(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma, float norm_eps,
               int8_t* xa, float* a_dq, int32_t* rowsum, float* act_scale, int8_t* xq_rm, uint16_t* y_rm,
               uint32_t* zero_words, int n_zero_words, hipStream_t stream) {
  ActArgs p;
  p.act_scale = act_scale;
  p.x = x;
  p.ldx = ldx;
  p.M = (int)M;
  p.K = (int)K;
  p.KS = (int)ksb(K);
  p.gamma = gamma;
  p.norm_eps = norm_eps;
  p.act_eps = 1e-5f;
  p.xa = xa;
  p.a_dq = a_dq;
  p.rowsum = rowsum;
  p.xq_rm = xq_rm;
  p.y_rm = y_rm;
  p.zero_words = zero_words;
  p.n_zero_words = n_zero_words;
  const unsigned rows = (unsigned)(mblocks(M) * 32);
  if (gamma)
    hipLaunchKernelGGL((k_act_rows<true, true>), dim3(rows), dim3(kActThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((k_act_rows<false, true>), dim3(rows), dim3(kActThreads), 0, stream, p);
  return check_launch("activation quantisation");
}

int check_act_args(const char* who, const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma) {
  if (!x) return set_error(BTL_ERR_NULL, "%s: x is NULL", who);
  if (M <= 0 || K <= 0) return set_error(BTL_ERR_SHAPE, "%s: M=%lld K=%lld", who, (long long)M, (long long)K);
  if (K % 32) return set_error(BTL_ERR_SHAPE, "%s: K=%lld must be a multiple of 32", who, (long long)K);
  if (K > BTL_MAX_K) return set_error(BTL_ERR_SHAPE, "%s: K=%lld > %d", who, (long long)K, BTL_MAX_K);
  if (M > (1 << 20)) return set_error(BTL_ERR_SHAPE, "%s: M=%lld too large", who, (long long)M);
  if (ldx < K || ldx % 8) return set_error(BTL_ERR_ALIGN, "%s: ldx=%lld must be >= K and a multiple of 8", who,
                                           (long long)ldx);
  if (!aligned(x, 16) || (gamma && !aligned(gamma, 16)))
    return set_error(BTL_ERR_ALIGN, "%s: x and gamma must be 16-byte aligned", who);
  return BTL_OK;
}

}  // namespace btl

using namespace btl;

extern "C" {

int btl_quant_absmax(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma, float norm_eps,
                     int8_t* xa, float* a_dq, int32_t* rowsum, float* act_scale, int8_t* xq_rm, uint16_t* y_rm,
                     btl_stream_t stream) {
  clear_error();
  int rc = check_act_args("btl_quant_absmax", x, M, K, ldx, gamma);
  if (rc) return rc;
  if (!xa || !a_dq || !rowsum) return set_error(BTL_ERR_NULL, "btl_quant_absmax: output pointer is NULL");
  if (!aligned(xa, 16) || !aligned(a_dq, 4) || !aligned(rowsum, 4) || (act_scale && !aligned(act_scale, 4)) ||
      (xq_rm && !aligned(xq_rm, 8)) ||
      (y_rm && !aligned(y_rm, 16)))
    return set_error(BTL_ERR_ALIGN, "btl_quant_absmax: misaligned output");
  return launch_act(x, M, K, ldx, gamma, norm_eps, xa, a_dq, rowsum, act_scale, xq_rm, y_rm, nullptr, 0,
                    (hipStream_t)stream);
}

int btl_rmsnorm(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma, float eps, uint16_t* y,
                btl_stream_t stream) {
  clear_error();
  int rc = check_act_args("btl_rmsnorm", x, M, K, ldx, gamma);
  if (rc) return rc;
  if (!y) return set_error(BTL_ERR_NULL, "btl_rmsnorm: y is NULL");
  if (!aligned(y, 16)) return set_error(BTL_ERR_ALIGN, "btl_rmsnorm: y must be 16-byte aligned");
  ActArgs p = {};
  p.x = x;
  p.ldx = ldx;
  p.M = (int)M;
  p.K = (int)K;
  p.KS = (int)ksb(K);
  p.gamma = gamma;
  p.norm_eps = eps;
  p.act_eps = 1e-5f;
  p.y_rm = y;
  hipLaunchKernelGGL((k_act_rows<true, false>), dim3((unsigned)M), dim3(kActThreads), 0, (hipStream_t)stream, p);
  return check_launch("btl_rmsnorm");
}

}  // extern "C"
