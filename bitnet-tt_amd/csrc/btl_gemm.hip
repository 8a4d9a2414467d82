// Ternary GEMM of the BitLinear path on gfx950:
//   acc[m,n] = sum_k q[m,k] * w[k,n]   (int8 activations, ternary weights, int32)
// followed by the scale epilogue (or the gate||up relu^2*up epilogue).
//
// Weights arrive as offset codes u = w + 1 in {0,1,2}, 2 bits each, already
// in MFMA operand order, so unpacking a dword of 16 codes into the four B
// operand dwords is one shift and one AND each.  The int8 MFMA then computes
// sum_k q*u, and the exact accumulator is recovered as
//   acc = sum_k q*u - sum_k q      (the row sum comes with the quantiser).
// |acc| <= 128*2*16384 < 2^31, so every step is exact.
//
// Decode (M <= 32): the whole activation block is one 32-row MFMA operand.
// A workgroup (4 waves) owns TPW column tiles of 32 and a slice of the K
// superblocks; each wave takes a quarter of that slice, issues all of its
// weight and activation loads up front (1 KiB per wave per load: fully
// coalesced), then runs the MFMAs.  The four wave partials meet in LDS.
// When K is split across workgroups (split-K), each writes its partial tile
// to the workspace and the last to arrive (atomic counter) sums them in a
// fixed order and runs the epilogue -- no spinning, no float atomics, the
// result is deterministic.
//
// Prefill (M > 32): 128x128 output tiles, one 64x64 quadrant per wave, A and
// B fragments loaded straight into registers (both operands are stored in
// MFMA order), the next superblock prefetched while the current one runs.
#include "btl_common.h"

namespace btl {

int launch_act(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma, float norm_eps,
               int8_t* xa, float* a_dq, int32_t* rowsum, float* act_scale, int8_t* xq_rm, uint16_t* y_rm,
               uint32_t* zero_words, int n_zero_words, hipStream_t stream);
int check_act_args(const char* who, const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma);

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const int8_t* xa;
  const float* a_dq;
  const int32_t* rowsum;
  const uint32_t* wdev;
  int M, KS, NT, N, n_out, Mb;
  int splitk, ngroups;
  float seg_scale[BTL_MAX_SEGMENTS];
  int seg_end[BTL_MAX_SEGMENTS];
  int nseg;
  const uint16_t* residual;
  uint16_t* out;
  int32_t* acc_out;
  int32_t* ws_part;
  uint32_t* ws_cnt;
};

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

__device__ __forceinline__ float seg_scale_of(const GemmArgs& p, int n) {
  float s = p.seg_scale[0];
#pragma unroll
  for (int i = 0; i + 1 < BTL_MAX_SEGMENTS; ++i)
    if (i + 1 < p.nseg && n >= p.seg_end[i]) s = p.seg_scale[i + 1];
  return s;
}

// Row of element r (0..15) of a lane's 32x32 MFMA accumulator.
__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// Epilogue for one accumulator element (acc already row-sum corrected).
__device__ __forceinline__ void epi_scale(const GemmArgs& p, int i, int n, int32_t acc) {
  if (p.acc_out) p.acc_out[(int64_t)i * p.N + n] = acc;
  const float f = seg_scale_of(p, n) * p.a_dq[i];
  uint16_t o = f2bf((float)acc * f);
  if (p.residual) o = f2bf(bf2f(p.residual[(int64_t)i * p.n_out + n]) + bf2f(o));
  p.out[(int64_t)i * p.n_out + n] = o;
}
__device__ __forceinline__ void epi_relu2(const GemmArgs& p, int i, int ng, int nu, int32_t ag, int32_t au) {
  if (p.acc_out) {
    p.acc_out[(int64_t)i * p.N + ng] = ag;
    p.acc_out[(int64_t)i * p.N + nu] = au;
  }
  const float ad = p.a_dq[i];
  const float g = bf2f(f2bf((float)ag * (seg_scale_of(p, ng) * ad)));
  const float u = bf2f(f2bf((float)au * (seg_scale_of(p, nu) * ad)));
  const float gr = g > 0.0f ? g : 0.0f;
  const float sq = bf2f(f2bf(gr * gr));
  p.out[(int64_t)i * p.n_out + ng] = f2bf(sq * u);
}

enum { EPI_SCALE = BTL_EPI_SCALE, EPI_RELU2 = BTL_EPI_RELU2_MUL };

// ------------------------------------------------------------- decode ----
template <int TPW, int NSB, int EPI>
__global__ __launch_bounds__(256) void k_gemm_decode(GemmArgs p) {
  static_assert(EPI != EPI_RELU2 || TPW == 2, "relu2 pairs a gate tile with its up tile");
  __shared__ int32_t red[4][TPW][16][64];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = blockIdx.x % p.ngroups;
  const int s = blockIdx.x / p.ngroups;

  int tile[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) tile[t] = (EPI == EPI_RELU2) ? (g + t * (p.NT >> 1)) : (g * TPW + t);

  const int sb0 = (s * p.KS) / p.splitk, sb1 = ((s + 1) * p.KS) / p.splitk;
  const int nsb = sb1 - sb0;
  const int wb = sb0 + (wv * nsb) / 4, we = sb0 + ((wv + 1) * nsb) / 4;

  v16i acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  for (int base = wb; base < we; base += NSB) {
    const int cnt = (we - base) < NSB ? (we - base) : NSB;
    v4i b[TPW][NSB];
    v4i a[NSB][4];
    // Loads for the whole pass go out before any MFMA; a slot past `cnt`
    // re-reads the pass's last superblock (valid address, cache hit).
#pragma unroll
    for (int i = 0; i < NSB; ++i) {
      const int sb = base + (i < cnt ? i : cnt - 1);
#pragma unroll
      for (int t = 0; t < TPW; ++t) b[t][i] = ld128(p.wdev + (((int64_t)tile[t] * p.KS + sb) * 64 + lane) * 4);
    }
#pragma unroll
    for (int i = 0; i < NSB; ++i) {
      const int sb = base + (i < cnt ? i : cnt - 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) a[i][q] = ld128(p.xa + (((int64_t)sb * 4 + q) * 64 + lane) * 16);
    }
#pragma unroll
    for (int i = 0; i < NSB; ++i) {
      if (i < cnt) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
          for (int t = 0; t < TPW; ++t) {
            const uint32_t d = (uint32_t)b[t][i][q];
            acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i][q], unpack_b(d), acc[t], 0, 0, 0);
          }
        }
      }
    }
  }

#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wv][t][r][lane] = acc[t][r];
  __syncthreads();

  // Thread (wv, lane) finishes accumulator rows r = wv + 4*rr of every tile.
  int32_t v[TPW][4];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int r = wv + 4 * rr;
      v[t][rr] = red[0][t][r][lane] + red[1][t][r][lane] + red[2][t][r][lane] + red[3][t][r][lane];
    }

  if (p.splitk > 1) {
    int32_t* part = p.ws_part + ((int64_t)(g * p.splitk + s) * TPW) * 1024;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        __hip_atomic_store(part + t * 1024 + (wv + 4 * rr) * 64 + lane, v[t][rr], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = atomicAdd(p.ws_cnt + g, 1u);
      s_last = (prev == (unsigned)(p.splitk - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        int32_t sum = 0;
        for (int ss = 0; ss < p.splitk; ++ss)
          sum += __hip_atomic_load(p.ws_part + ((int64_t)(g * p.splitk + ss) * TPW + t) * 1024 +
                                       (wv + 4 * rr) * 64 + lane,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v[t][rr] = sum;
      }
    if (tid == 0) __hip_atomic_store(p.ws_cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  const int j = lane & 31;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int i = acc_row(wv + 4 * rr, lane);
    if (i >= p.M) continue;
    const int32_t rs = p.rowsum[i];
    if (EPI == EPI_RELU2) {
      epi_relu2(p, i, tile[0] * 32 + j, tile[1] * 32 + j, v[0][rr] - rs, v[1][rr] - rs);
    } else {
#pragma unroll
      for (int t = 0; t < TPW; ++t) epi_scale(p, i, tile[t] * 32 + j, v[t][rr] - rs);
    }
  }
}

// ------------------------------------------------------------ prefill ----
// Workgroup tile: 4 row blocks x 4 column tiles (scale) or 2 gate tiles plus
// their 2 up tiles (relu2).  Wave (wm, wn) = (wv & 1, wv >> 1) owns row
// blocks 2*wm, 2*wm+1 and column slots 2*wn, 2*wn+1 (relu2: slot 0 = gate,
// slot 1 = matching up tile).
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_prefill(GemmArgs p) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv & 1, wn = wv >> 1;
  const int gm = blockIdx.y, gn = blockIdx.x;
  int mblk[2];
  bool mok[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    mblk[u] = gm * 4 + 2 * wm + u;
    mok[u] = mblk[u] < p.Mb;
    if (!mok[u]) mblk[u] = p.Mb - 1;
  }
  int tile[2];
  bool tok[2];
  if (EPI == EPI_RELU2) {
    const int half = p.NT >> 1;
    int gt = gn * 2 + wn;
    tok[0] = tok[1] = gt < half;
    if (gt >= half) gt = half - 1;
    tile[0] = gt;
    tile[1] = gt + half;
  } else {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      tile[u] = gn * 4 + 2 * wn + u;
      tok[u] = tile[u] < p.NT;
      if (!tok[u]) tile[u] = p.NT - 1;
    }
  }

  v16i acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  const int KS = p.KS;
  v4i a[2][4], b[2], an[2][4], bn[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    b[u] = ld128(p.wdev + (((int64_t)tile[u] * KS) * 64 + lane) * 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) a[u][q] = ld128(p.xa + ((((int64_t)mblk[u] * KS) * 4 + q) * 64 + lane) * 16);
  }
  for (int ks = 0; ks < KS; ++ks) {
    const int kn = (ks + 1 < KS) ? ks + 1 : ks;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      bn[u] = ld128(p.wdev + (((int64_t)tile[u] * KS + kn) * 64 + lane) * 4);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        an[u][q] = ld128(p.xa + ((((int64_t)mblk[u] * KS + kn) * 4 + q) * 64 + lane) * 16);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const v4i b0 = unpack_b((uint32_t)b[0][q]);
      const v4i b1 = unpack_b((uint32_t)b[1][q]);
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        acc[x][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[x][q], b0, acc[x][0], 0, 0, 0);
        acc[x][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[x][q], b1, acc[x][1], 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      b[u] = bn[u];
#pragma unroll
      for (int q = 0; q < 4; ++q) a[u][q] = an[u][q];
    }
  }

  const int j = lane & 31;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    if (!mok[x]) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = mblk[x] * 32 + acc_row(r, lane);
      if (i >= p.M) continue;
      const int32_t rs = p.rowsum[i];
      if (EPI == EPI_RELU2) {
        if (tok[0]) epi_relu2(p, i, tile[0] * 32 + j, tile[1] * 32 + j, acc[x][0][r] - rs, acc[x][1][r] - rs);
      } else {
#pragma unroll
        for (int u = 0; u < 2; ++u)
          if (tok[u]) epi_scale(p, i, tile[u] * 32 + j, acc[x][u][r] - rs);
      }
    }
  }
}

// ------------------------------------------------------------- planning --
static int nsb_bucket(int per_wave) {
  if (per_wave <= 2) return 2;
  if (per_wave <= 4) return 4;
  if (per_wave <= 6) return 6;
  return 8;
}

GemmPlan plan_gemm(int64_t M, int64_t K, int64_t N, int epilogue, int splitk_req) {
  GemmPlan pl = {};
  const int64_t KS = ksb(K), NT = N / 32;
  if (M > 32) {
    pl.prefill = true;
    pl.tpw = 0;
    pl.ngroups = 0;
    pl.splitk = 1;
    pl.ws_bytes = 0;
    return pl;
  }
  pl.prefill = false;
  pl.tpw = 2;
  if (epilogue == BTL_EPI_SCALE && NT % 2) pl.tpw = 1;
  if (epilogue == BTL_EPI_SCALE && NT <= 160) pl.tpw = 1;  // small N: spread tiles over more CUs
  pl.ngroups = (int)((epilogue == BTL_EPI_RELU2_MUL) ? NT / 2 : NT / pl.tpw);
  int sk = splitk_req;
  if (sk <= 0) {
    // Aim for about one workgroup per CU (256 CUs) without making a wave's
    // share of K smaller than one superblock.
    sk = (int)((256 + pl.ngroups / 2) / pl.ngroups);
    if (sk < 1) sk = 1;
  }
  const int max_sk = (int)(KS / 4 > 1 ? KS / 4 : 1);
  if (sk > max_sk) sk = max_sk;
  if (sk > 16) sk = 16;
  pl.splitk = sk;
  pl.ws_bytes = 0;
  if (sk > 1) {
    const int64_t cnt = round_up((int64_t)pl.ngroups * 4, 256);
    pl.ws_bytes = cnt + (int64_t)sk * pl.ngroups * pl.tpw * 4096;
  }
  return pl;
}

FusedLayout fused_layout(int64_t M, int64_t K, int64_t N, int epilogue, int splitk_req) {
  FusedLayout L;
  const int64_t rows = mblocks(M) * 32;
  L.xa = 0;
  L.a_dq = round_up(btl_act_bytes(M, K), 256);
  L.rowsum = L.a_dq + round_up(rows * 4, 256);
  L.gemm_ws = L.rowsum + round_up(rows * 4, 256);
  L.total = L.gemm_ws + plan_gemm(M, K, N, epilogue, splitk_req).ws_bytes;
  return L;
}

template <int TPW, int EPI>
static void launch_decode_nsb(int nsb, dim3 grid, hipStream_t s, const GemmArgs& a) {
  switch (nsb) {
    case 2: hipLaunchKernelGGL((k_gemm_decode<TPW, 2, EPI>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_gemm_decode<TPW, 4, EPI>), grid, dim3(256), 0, s, a); break;
    case 6: hipLaunchKernelGGL((k_gemm_decode<TPW, 6, EPI>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((k_gemm_decode<TPW, 8, EPI>), grid, dim3(256), 0, s, a); break;
  }
}

static int check_gemm_args(const char* who, int64_t M, int64_t K, int64_t N, const uint32_t* wdev,
                           const float* seg_scale, const int64_t* seg_end, int nseg, int epilogue,
                           const uint16_t* residual, const uint16_t* out) {
  if (!wdev || !out || !seg_scale) return set_error(BTL_ERR_NULL, "%s: null pointer", who);
  if (M <= 0 || K <= 0 || N <= 0) return set_error(BTL_ERR_SHAPE, "%s: M=%lld K=%lld N=%lld", who, (long long)M,
                                                   (long long)K, (long long)N);
  if (K % 32 || N % 32) return set_error(BTL_ERR_SHAPE, "%s: K=%lld and N=%lld must be multiples of 32", who,
                                         (long long)K, (long long)N);
  if (K > BTL_MAX_K) return set_error(BTL_ERR_SHAPE, "%s: K=%lld > %d", who, (long long)K, BTL_MAX_K);
  if (M > (1 << 20) || N > (1 << 24)) return set_error(BTL_ERR_SHAPE, "%s: M or N too large", who);
  if (epilogue != BTL_EPI_SCALE && epilogue != BTL_EPI_RELU2_MUL)
    return set_error(BTL_ERR_ARG, "%s: unknown epilogue %d", who, epilogue);
  if (epilogue == BTL_EPI_RELU2_MUL) {
    if (N % 64) return set_error(BTL_ERR_SHAPE, "%s: relu2 epilogue needs N=2F with F %% 32 == 0", who);
    if (residual) return set_error(BTL_ERR_ARG, "%s: residual is only supported with the scale epilogue", who);
  }
  if (nseg < 1 || nseg > BTL_MAX_SEGMENTS) return set_error(BTL_ERR_ARG, "%s: nseg=%d", who, nseg);
  if (nseg > 1 && !seg_end) return set_error(BTL_ERR_NULL, "%s: seg_end is NULL", who);
  if (nseg > 1) {
    int64_t prev = 0;
    for (int i = 0; i < nseg; ++i) {
      if (seg_end[i] <= prev || seg_end[i] % 32)
        return set_error(BTL_ERR_ARG, "%s: seg_end must increase in multiples of 32", who);
      prev = seg_end[i];
    }
    if (seg_end[nseg - 1] != N) return set_error(BTL_ERR_ARG, "%s: last seg_end must equal N", who);
  }
  if (!aligned(wdev, 16)) return set_error(BTL_ERR_ALIGN, "%s: wdev must be 16-byte aligned", who);
  if (!aligned(out, 4) || (residual && !aligned(residual, 4)))
    return set_error(BTL_ERR_ALIGN, "%s: out/residual must be 4-byte aligned", who);
  return BTL_OK;
}

static int launch_gemm(const int8_t* xa, const float* a_dq, const int32_t* rowsum, int64_t M, int64_t K, int64_t N,
                       const uint32_t* wdev, const float* seg_scale, const int64_t* seg_end, int nseg, int epilogue,
                       const uint16_t* residual, uint16_t* out, int32_t* acc_out, char* ws, const GemmPlan& pl,
                       hipStream_t s) {
  GemmArgs a = {};
  a.xa = xa;
  a.a_dq = a_dq;
  a.rowsum = rowsum;
  a.wdev = wdev;
  a.M = (int)M;
  a.KS = (int)ksb(K);
  a.NT = (int)(N / 32);
  a.N = (int)N;
  a.n_out = (int)(epilogue == BTL_EPI_RELU2_MUL ? N / 2 : N);
  a.Mb = (int)mblocks(M);
  a.nseg = nseg;
  for (int i = 0; i < BTL_MAX_SEGMENTS; ++i) {
    a.seg_scale[i] = i < nseg ? seg_scale[i] : 0.0f;
    a.seg_end[i] = i < nseg ? (int)(nseg > 1 ? seg_end[i] : N) : (int)N;
  }
  a.residual = residual;
  a.out = out;
  a.acc_out = acc_out;
  if (pl.prefill) {
    const int ngn = (epilogue == BTL_EPI_RELU2_MUL) ? (int)((a.NT / 2 + 1) / 2) : (a.NT + 3) / 4;
    dim3 grid((unsigned)ngn, (unsigned)((a.Mb + 3) / 4));
    if (epilogue == BTL_EPI_RELU2_MUL)
      hipLaunchKernelGGL((k_gemm_prefill<EPI_RELU2>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((k_gemm_prefill<EPI_SCALE>), grid, dim3(256), 0, s, a);
    return check_launch("ternary gemm (prefill)");
  }
  a.splitk = pl.splitk;
  a.ngroups = pl.ngroups;
  if (pl.splitk > 1) {
    a.ws_cnt = reinterpret_cast<uint32_t*>(ws);
    a.ws_part = reinterpret_cast<int32_t*>(ws + round_up((int64_t)pl.ngroups * 4, 256));
  }
  const int per_wg = (int)((a.KS + pl.splitk - 1) / pl.splitk);
  const int per_wave = (per_wg + 3) / 4;
  const int nsb = nsb_bucket(per_wave);
  dim3 grid((unsigned)(pl.ngroups * pl.splitk));
  if (epilogue == BTL_EPI_RELU2_MUL)
    launch_decode_nsb<2, EPI_RELU2>(nsb, grid, s, a);
  else if (pl.tpw == 2)
    launch_decode_nsb<2, EPI_SCALE>(nsb, grid, s, a);
  else
    launch_decode_nsb<1, EPI_SCALE>(nsb, grid, s, a);
  return check_launch("ternary gemm (decode)");
}

}  // namespace btl

using namespace btl;

extern "C" {

int btl_choose_splitk(int64_t M, int64_t K, int64_t N, int epilogue) {
  if (M <= 0 || K <= 0 || N <= 0 || N % 32) return 0;
  return plan_gemm(M, K, N, epilogue, 0).splitk;
}

int64_t btl_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int epilogue, int splitk) {
  if (M <= 0 || K <= 0 || N <= 0 || N % 32) return 0;
  return plan_gemm(M, K, N, epilogue, splitk).ws_bytes;
}

int64_t btl_fused_workspace_bytes(int64_t M, int64_t K, int64_t N, int epilogue, int splitk) {
  if (M <= 0 || K <= 0 || N <= 0 || N % 32) return 0;
  return fused_layout(M, K, N, epilogue, splitk).total;
}

int btl_gemm_i8t2(const int8_t* xa, const float* a_dq, const int32_t* rowsum, int64_t M, int64_t K, int64_t N,
                  const uint32_t* wdev, const float* seg_scale, const int64_t* seg_end, int nseg, int epilogue,
                  const uint16_t* residual, uint16_t* out, int32_t* acc_out, void* workspace, size_t workspace_bytes,
                  int splitk, btl_stream_t stream) {
  clear_error();
  int rc = check_gemm_args("btl_gemm_i8t2", M, K, N, wdev, seg_scale, seg_end, nseg, epilogue, residual, out);
  if (rc) return rc;
  if (!xa || !a_dq || !rowsum) return set_error(BTL_ERR_NULL, "btl_gemm_i8t2: activation pointer is NULL");
  if (!aligned(xa, 16) || !aligned(a_dq, 4) || !aligned(rowsum, 4) || (acc_out && !aligned(acc_out, 4)))
    return set_error(BTL_ERR_ALIGN, "btl_gemm_i8t2: misaligned activation or acc_out buffer");
  if (splitk < 0) return set_error(BTL_ERR_ARG, "btl_gemm_i8t2: splitk=%d", splitk);
  const GemmPlan pl = plan_gemm(M, K, N, epilogue, splitk);
  if (pl.ws_bytes > 0) {
    if (!workspace) return set_error(BTL_ERR_NULL, "btl_gemm_i8t2: split-K needs a workspace");
    if ((int64_t)workspace_bytes < pl.ws_bytes)
      return set_error(BTL_ERR_WORKSPACE, "btl_gemm_i8t2: workspace %zu < %lld bytes", workspace_bytes,
                       (long long)pl.ws_bytes);
    if (!aligned(workspace, 256)) return set_error(BTL_ERR_ALIGN, "btl_gemm_i8t2: workspace must be 256-byte aligned");
  }
  return launch_gemm(xa, a_dq, rowsum, M, K, N, wdev, seg_scale, seg_end, nseg, epilogue, residual, out, acc_out,
                     (char*)workspace, pl, (hipStream_t)stream);
}

int btl_bitlinear_fused(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma, float norm_eps,
                        const uint32_t* wdev, int64_t N, const float* seg_scale, const int64_t* seg_end, int nseg,
                        int epilogue, const uint16_t* residual, uint16_t* out, int32_t* acc_out, int8_t* xq_debug,
                        void* workspace, size_t workspace_bytes, int splitk, btl_stream_t stream) {
  clear_error();
  int rc = check_act_args("btl_bitlinear_fused", x, M, K, ldx, gamma);
  if (rc) return rc;
  rc = check_gemm_args("btl_bitlinear_fused", M, K, N, wdev, seg_scale, seg_end, nseg, epilogue, residual, out);
  if (rc) return rc;
  if (!workspace) return set_error(BTL_ERR_NULL, "btl_bitlinear_fused: workspace is NULL");
  if (!aligned(workspace, 256)) return set_error(BTL_ERR_ALIGN, "btl_bitlinear_fused: workspace must be 256-byte aligned");
  if (splitk < 0) return set_error(BTL_ERR_ARG, "btl_bitlinear_fused: splitk=%d", splitk);
  if ((acc_out && !aligned(acc_out, 4)) || (xq_debug && !aligned(xq_debug, 8)))
    return set_error(BTL_ERR_ALIGN, "btl_bitlinear_fused: misaligned debug output");
  const FusedLayout L = fused_layout(M, K, N, epilogue, splitk);
  if ((int64_t)workspace_bytes < L.total)
    return set_error(BTL_ERR_WORKSPACE, "btl_bitlinear_fused: workspace %zu < %lld bytes", workspace_bytes,
                     (long long)L.total);
  const GemmPlan pl = plan_gemm(M, K, N, epilogue, splitk);
  char* ws = (char*)workspace;
  hipStream_t s = (hipStream_t)stream;
  // The activation kernel also clears the split-K counters, so a workspace
  // left dirty by an interrupted call is repaired by the next one.
  rc = launch_act(x, M, K, ldx, gamma, norm_eps, (int8_t*)(ws + L.xa), (float*)(ws + L.a_dq),
                  (int32_t*)(ws + L.rowsum), nullptr, xq_debug, nullptr, pl.splitk > 1 ? (uint32_t*)(ws + L.gemm_ws) : nullptr,
                  pl.splitk > 1 ? pl.ngroups : 0, s);
  if (rc) return rc;
  return launch_gemm((const int8_t*)(ws + L.xa), (const float*)(ws + L.a_dq), (const int32_t*)(ws + L.rowsum), M, K,
                     N, wdev, seg_scale, seg_end, nseg, epilogue, residual, out, acc_out, ws + L.gemm_ws, pl, s);
}

}  // extern "C"
