// Standalone activation prologue kernels: one or two waves per token row for
// the quantising prologue of batches of rows up to 8192 long, else one
// workgroup of 512 threads per row running the row computation of
// btl_act_row.h (RMSNorm, absmax int8 quantisation, blocked operand layout).  The fused decode kernel in
// btl_gemm.hip runs the same row computation inside the GEMM launch.
#include "btl_act_row.h"

namespace btl {

template <bool NORM, bool QUANT, int CPT>
__global__ __launch_bounds__(kActThreads) void k_act_rows(ActArgs p) {
  act_row<NORM, QUANT, false, CPT>(p, blockIdx.x, threadIdx.x);
}

// The quantising prologue with one wave per row (four rows a workgroup) or
// two (two rows): every row of a prefill batch in flight at once, with no
// barrier (one wave) or a barrier between two waves (the 512-thread row above
// spends most of its time in two block reductions over eight waves and runs a
// few hundred rows at a time).  The wave plays the eight waves of
// act_row in turn: lane l holds the chunks of threads l, l + 64, ..., l + 448
// of that row, so the sum of squares runs the same per-thread order, the same
// 64-lane butterfly per (virtual) wave and the same fixed combination of the
// eight wave sums -- bit for bit the statistic act_row computes.  The maximum
// and the row sum do not depend on the order.  Rows past M and columns past K
// are written as zeros, as act_row writes them.
constexpr int kActRowWaves = 4;  // waves a workgroup
// WPR waves per row (1 or 2): wave h of a row takes the virtual waves
// h * 8 / WPR .. and the two meet in LDS for the three row statistics.
template <bool NORM, int CPT, int WPR>
__global__ __launch_bounds__(64 * kActRowWaves) void k_act_rows_wave(ActArgs p) {
  constexpr int NV = kActWaves;  // the 512-thread row's waves
  constexpr int NL = NV / WPR;   // of them on this wave
  constexpr int RPW = kActRowWaves / WPR;
  __shared__ float s_ws[RPW][NV];
  __shared__ uint32_t s_mx[RPW][WPR];
  __shared__ int s_rsum[RPW][WPR];
  const int lane = threadIdx.x & 63, wi = threadIdx.x >> 6, r = wi / WPR, h = wi % WPR;
  // Workgroup b runs on XCD b % 8; XCD x takes a contiguous range of rows, so
  // the 32 rows of a row block, whose quantised bytes interleave in 16-byte
  // pieces, meet in one L2 instead of leaving partial lines in eight.
  const int per = (gridDim.x + 7) / 8;
  const int v = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (v >= (int)gridDim.x) return;
  const int m = v * RPW + r;
  const int nch = p.K >> 3, nchp = p.KS * 16;
  const bool pad = m >= p.M;  // padding row of the last 32-row block
  if (p.zero_words && m == 0 && h == 0)
    for (int i = lane; i < p.n_zero_words; i += 64) p.zero_words[i] = 0u;
  if (pad) {
    for (int c = h * 64 + lane; c < nchp; c += 64 * WPR) store8<false>(p.xa + xa_offset(m, 8 * c, p.KS), 0u, 0u);
    if (lane == 0 && h == 0) {
      p.a_dq[m] = 0.0f;
      if (p.rowsum) p.rowsum[m] = 0;
    }
    if (WPR == 1) return;  // with two waves a row it still takes part in the barriers
  }
  const uint16_t* xr = p.x + (int64_t)m * p.ldx;
  // chunk of (virtual wave w = h * NL + l, i): c = 64 w + lane + 512 i
  uint4 y[CPT][NL], graw[CPT][NL];
#pragma unroll
  for (int i = 0; i < CPT; ++i)
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      const int c = 64 * (h * NL + l) + lane + kActThreads * i;
      y[i][l] = !pad && c < nch ? *reinterpret_cast<const uint4*>(xr + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
      graw[i][l] = make_uint4(0u, 0u, 0u, 0u);
      if (NORM && p.gamma && !pad && c < nch) graw[i][l] = *reinterpret_cast<const uint4*>(p.gamma + 8 * c);
    }
  // With one chunk per thread and one wave per row, (i, l) blocks past the
  // row's chunks hold zeros in every lane: they are skipped (a wave-uniform
  // branch), which changes no bit -- a zero adds nothing to a sum of squares
  // or a maximum, and their chunks are not stored.  (Measured on MI355X:
  // M = 2048, K = 2560 7.4 -> 6.75 us; the branches cost more than they save
  // in the other instances, which keep the straight-line code.)
  auto live = [&](int i, int l) {
    return !(CPT == 1 && WPR == 1) || 64 * (h * NL + l) + kActThreads * i < nch;
  };
  if (NORM) {
    float ws[NL];
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        if (!live(i, l)) continue;
        const uint32_t w4[4] = {y[i][l].x, y[i][l].y, y[i][l].z, y[i][l].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // elements 2j, 2j+1 in order; zero chunks add zeros
          const float a = bf_lo(w4[j]), b = bf_hi(w4[j]);
          s = s + a * a;
          s = s + b * b;
        }
      }
      ws[l] = live(0, l) ? wave_xor_sum(s) : 0.0f;
    }
    float total;
    if constexpr (WPR == 1) {
      total = sum8_fixed(ws);
    } else {
      if (lane == 0)
#pragma unroll
        for (int l = 0; l < NL; ++l) s_ws[r][h * NL + l] = ws[l];
      __syncthreads();
      total = sum8_fixed(s_ws[r]);
    }
    const float rr = 1.0f / sqrtf(total / (float)p.K + p.norm_eps);
    // y = bf16(gamma * bf16(x * r)) (bf16(x * r) without gamma), kept as bf16 pairs
#pragma unroll
    for (int i = 0; i < CPT; ++i)
#pragma unroll
      for (int l = 0; l < NL; ++l) {
        if (!live(i, l)) continue;
        uint32_t w4[4] = {y[i][l].x, y[i][l].y, y[i][l].z, y[i][l].w};
        const uint32_t g4[4] = {graw[i][l].x, graw[i][l].y, graw[i][l].z, graw[i][l].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t t = f2bf_pair(bf_lo(w4[j]) * rr, bf_hi(w4[j]) * rr);
          w4[j] = p.gamma ? f2bf_pair(bf_lo(g4[j]) * bf_lo(t), bf_hi(g4[j]) * bf_hi(t)) : t;
        }
        y[i][l] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
      }
  }
  // a = max(max|y|, act_eps), as act_row takes it (fmaxf within the lane,
  // then the bit patterns across lanes)
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i)
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      if (!live(i, l)) continue;
      const uint32_t w4[4] = {y[i][l].x, y[i][l].y, y[i][l].z, y[i][l].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) amax = fmaxf(fmaxf(amax, fabsf(bf_lo(w4[j]))), fabsf(bf_hi(w4[j])));
    }
  uint32_t u = __float_as_uint(amax);
  u = max(u, xor_partner_u<32>(u));
  u = max(u, xor_partner_u<16>(u));
  u = max(u, xor_partner_u<8>(u));
  u = max(u, xor_partner_u<4>(u));
  u = max(u, xor_partner_u<2>(u));
  u = max(u, xor_partner_u<1>(u));
  if constexpr (WPR == 2) {
    if (lane == 0) s_mx[r][h] = u;
    __syncthreads();
    u = max(s_mx[r][0], s_mx[r][1]);
  }
  const float amx = __uint_as_float(u);
  const float a = amx > p.act_eps ? amx : p.act_eps;
  const float scale = 127.0f / a;
  if (lane == 0 && h == 0 && !pad) {
    p.a_dq[m] = a / 127.0f;
    if (p.act_scale) p.act_scale[m] = scale;
  }
  int rs = 0;
  if (!pad) {
#pragma unroll
    for (int i = 0; i < CPT; ++i)
#pragma unroll
      for (int l = 0; l < NL; ++l) {
        if (!live(i, l)) continue;
        const int c = 64 * (h * NL + l) + lane + kActThreads * i;
        if (c < nch) {
          const uint32_t w4[4] = {y[i][l].x, y[i][l].y, y[i][l].z, y[i][l].w};
          const float vv[8] = {bf_lo(w4[0]), bf_hi(w4[0]), bf_lo(w4[1]), bf_hi(w4[1]),
                               bf_lo(w4[2]), bf_hi(w4[2]), bf_lo(w4[3]), bf_hi(w4[3])};
          uint32_t lo, hi;
          quant8(vv, scale, lo, hi, rs);
          store_chunk<false>(p.xa, m, c, p.KS, lo, hi);
          if (p.xq_rm) *reinterpret_cast<uint2*>(p.xq_rm + (int64_t)m * p.K + 8 * c) = make_uint2(lo, hi);
          if (p.y_rm) *reinterpret_cast<uint4*>(p.y_rm + (int64_t)m * p.K + 8 * c) = y[i][l];
        }
      }
    for (int c = nch + h * 64 + lane; c < nchp; c += 64 * WPR) store8<false>(p.xa + xa_offset(m, 8 * c, p.KS), 0u, 0u);
  }
  if (!p.rowsum) return;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) rs += __shfl_xor(rs, off, 64);
  if constexpr (WPR == 2) {
    if (lane == 0) s_rsum[r][h] = rs;
    __syncthreads();
    rs = s_rsum[r][0] + s_rsum[r][1];
  }
  if (lane == 0 && h == 0 && !pad) p.rowsum[m] = rs;
}

template <bool NORM, bool QUANT>
static void launch_rows(unsigned rows, hipStream_t s, const ActArgs& p) {
  // rows is a multiple of 32 (whole row blocks) when quantising.  One wave
  // per row from 1024 rows, two from 256, the 512-thread row below that
  // (measured on MI355X, graph-timed: M = 2048, K = 2560 / 6912: 512-thread
  // rows 10.6 / 17.9 us in a BitLinear sequence, one wave 9.5 / 14.3 us;
  // M = 512: 512-thread rows 5.05 / 7.26 us, two waves 4.5 / 6.1 us, one wave
  // 6.0 / 9.2 us; M = 100: 512-thread rows 3.6 us, two waves 4.3 us).
  if (QUANT && act_cpt(p.K) <= 2 && rows >= 1024) {
    const dim3 grid(rows / kActRowWaves), block(64 * kActRowWaves);
    if (act_cpt(p.K) == 1)
      hipLaunchKernelGGL((k_act_rows_wave<NORM, 1, 1>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((k_act_rows_wave<NORM, 2, 1>), grid, block, 0, s, p);
    return;
  }
  if (QUANT && act_cpt(p.K) <= 2 && rows >= 256) {
    const dim3 grid(rows / (kActRowWaves / 2)), block(64 * kActRowWaves);
    if (act_cpt(p.K) == 1)
      hipLaunchKernelGGL((k_act_rows_wave<NORM, 1, 2>), grid, block, 0, s, p);
    else
      hipLaunchKernelGGL((k_act_rows_wave<NORM, 2, 2>), grid, block, 0, s, p);
    return;
  }
  switch (act_cpt(p.K)) {
    case 1: hipLaunchKernelGGL((k_act_rows<NORM, QUANT, 1>), dim3(rows), dim3(kActThreads), 0, s, p); break;
    case 2: hipLaunchKernelGGL((k_act_rows<NORM, QUANT, 2>), dim3(rows), dim3(kActThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((k_act_rows<NORM, QUANT, 4>), dim3(rows), dim3(kActThreads), 0, s, p); break;
  }
}

// Launch helper shared with the fused entry point.
int launch_act(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma, float norm_eps,
               int8_t* xa, float* a_dq, int32_t* rowsum, float* act_scale, int8_t* xq_rm, uint16_t* y_rm,
               uint32_t* zero_words, int n_zero_words, hipStream_t stream) {
  ActArgs p = {};
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
    launch_rows<true, true>(rows, stream, p);
  else
    launch_rows<false, true>(rows, stream, p);
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
  if (!xa || !a_dq) return set_error(BTL_ERR_NULL, "btl_quant_absmax: output pointer is NULL");
  if (!aligned(xa, 16) || !aligned(a_dq, 4) || (rowsum && !aligned(rowsum, 4)) || (act_scale && !aligned(act_scale, 4)) ||
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
  launch_rows<true, false>((unsigned)M, (hipStream_t)stream, p);
  return check_launch("btl_rmsnorm");
}

}  // extern "C"
