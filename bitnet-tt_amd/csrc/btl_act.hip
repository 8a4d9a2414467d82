// Standalone activation prologue kernel: one workgroup (256 threads) per
// token row, running the row computation of btl_act_row.h (RMSNorm, absmax
// int8 quantisation, blocked operand layout).  The fused decode kernel in
// btl_gemm.hip runs the same row computation inside the GEMM launch.
#include "btl_act_row.h"

namespace btl {

template <bool NORM, bool QUANT, int CPT>
__global__ __launch_bounds__(kActThreads) void k_act_rows(ActArgs p) {
  act_row<NORM, QUANT, false, CPT>(p, blockIdx.x, threadIdx.x);
}

template <bool NORM, bool QUANT>
static void launch_rows(unsigned rows, hipStream_t s, const ActArgs& p) {
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
