// Activation prologue of a BitLinear for one token row: optional RMSNorm,
// per-token absmax int8 quantisation, and the blocked operand layout the
// ternary GEMM consumes.  Shared by the standalone activation kernel and the
// fused decode BitLinear kernel.
//
//   RMSNorm  (HF BitNetRMSNorm order; src/bitnet_tt/layers/bitlinear.py:433-461,
//            fused into the QKV launch at inference/generator_batch32.py:721-727):
//            r = 1/sqrt(sum(x^2)/K + eps); y = bf16(gamma * bf16(x * r))
//   quant    (src/bitnet_tt/utils/quantization.py:60-91):
//            a = max(max|y|, 1e-5); q = clip(rne(y * (127/a)), -128, 127)
//
// 512 threads (8 waves) work on a row.  The sum of squares follows a fixed
// order so the statistic is reproducible bit for bit: thread t accumulates
// x^2 over the 8-element chunks t, t+512, ... in order, the 64 lanes of a wave
// combine by an xor butterfly (offsets 32..1), and the eight wave sums
// combine as ((w0+w1)+(w2+w3))+((w4+w5)+(w6+w7)).  Multiplies and adds are
// separately rounded (built with -ffp-contract=off); division and sqrt are
// correctly rounded.
//
// Quantised output layout (per 32-row block mb, 128-column superblock ks):
// byte (((mb*KS + ks)*4 + q)*64 + lane)*16 + p holds q[mb*32 + (lane & 31)]
// [ks*128 + q*32 + (lane >> 5)*16 + p] -- exactly the 16 bytes lane `lane`
// feeds to v_mfma_i32_32x32x32_i8 for k-step q, so one 1 KiB load per wave
// and k-step brings a whole A operand.  Rows >= M and columns >= K are zero.
#pragma once

#include <math.h>

#include "btl_common.h"

namespace btl {

constexpr int kActThreads = 512;
constexpr int kActWaves = kActThreads / 64;
constexpr int kActMaxChunks = BTL_MAX_K / 8 / kActThreads;  // 4 chunks of 8 per thread

// Chunks of 8 elements per thread for a row of K (1, 2 or 4): the row code
// is instantiated per bucket so a thread's loops cover only chunks it can own.
inline int act_cpt(int64_t K) {
  const int64_t c = (K / 8 + kActThreads - 1) / kActThreads;
  return c <= 1 ? 1 : c <= 2 ? 2 : 4;
}

// Fixed combination order of the 8 wave partials (part of the numerics
// contract: the oracle restates it).
__device__ __forceinline__ float sum8_fixed(const float* s) {
  return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

struct ActArgs {
  const uint16_t* x;
  int64_t ldx;
  int M, K, KS;
  const uint16_t* gamma;
  float norm_eps;
  float act_eps;
  int8_t* xa;
  float* a_dq;
  int32_t* rowsum;       // optional [rows] sum_k q (the GEMM recomputes it)
  float* act_scale;      // optional [M] 127/a
  int8_t* xq_rm;         // optional [M, K] int8
  uint16_t* y_rm;        // optional [M, K] bf16 (the normalised y)
  uint32_t* zero_words;  // optional words cleared by row 0 (GEMM counters)
  int n_zero_words;
};

// Memory operations every workgroup of the device observes without an L2
// write-back: agent-scope relaxed atomics bypass the per-XCD L2.  Data is
// published as "coherent stores, wait for their acknowledgement, bump a
// counter"; a __threadfence() would instead write back every XCD's whole L2.
__device__ __forceinline__ void st_coherent(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_coherent(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_coherent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_coherent(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
  return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT));
}
// Waits until every memory operation this thread issued has completed.
__device__ __forceinline__ void wait_memory() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Workgroup barrier after this wave's LDS accesses have completed
// (lgkmcnt(0)), without the memory fence of __syncthreads, whose release part
// would also wait for every global load in flight (weights prefetched for a
// later phase, LDS-direct loads).  The compiler fences keep LDS instructions
// on their side of it; the explicit wait covers their results, which the
// compiler would otherwise be free to collect after the barrier.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ int64_t xa_offset(int m, int k0, int KS) {
  const int mb = m >> 5, mr = m & 31;
  const int ks = k0 >> 7, qs = (k0 >> 5) & 3, h = (k0 >> 4) & 1, p0 = k0 & 15;
  return ((((int64_t)mb * KS + ks) * 4 + qs) * 64 + (h * 32 + mr)) * 16 + p0;
}

// ---- cross-lane partners of the xor butterfly ------------------------------
// xor_partner<d>(v) is v of lane (lane ^ d), for d = 32, 16, 8, 4, 2, 1: the
// swaps of v_permlane32/16_swap for 32 and 16, DPP row/quad permutations for
// the rest (xor 8 = half-row mirror of the row mirror, xor 4 = quad reverse of
// the half-row mirror).  No LDS round trip, so a 64-lane butterfly costs a few
// ALU cycles per step instead of an LDS latency.
// Every permutation used here stays inside a row of 16 lanes with all rows and
// banks enabled, so no lane reads outside the wave and bound_ctrl changes
// nothing; with it set, the compiler folds the move into the consuming
// add / max (one v_*_dpp instead of a move and an ALU op).
template <int C>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, C, 0xF, 0xF, true);
}
template <int D>
__device__ __forceinline__ uint32_t xor_partner_u(uint32_t x) {
  static_assert(D == 32 || D == 16 || D == 8 || D == 4 || D == 2 || D == 1, "butterfly distance");
  const int lane = __lane_id();
  if (D == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return lane < 32 ? r[1] : r[0];
  } else if (D == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else if (D == 8) {
    return dpp_mov<0x141>(dpp_mov<0x140>(x));  // row_half_mirror(row_mirror)
  } else if (D == 4) {
    return dpp_mov<0x1B>(dpp_mov<0x141>(x));  // quad_perm(3,2,1,0)(row_half_mirror)
  } else if (D == 2) {
    return dpp_mov<0x4E>(x);  // quad_perm(2,3,0,1)
  } else {
    return dpp_mov<0xB1>(x);  // quad_perm(1,0,3,2)
  }
}
template <int D>
__device__ __forceinline__ float xor_partner(float v) {
  return __uint_as_float(xor_partner_u<D>(__float_as_uint(v)));
}

// Butterfly over the 64 lanes, partners at distance 32, 16, 8, 4, 2, 1 in this
// order (every lane ends with the same value).
__device__ __forceinline__ float wave_xor_sum(float s) {
  s = s + xor_partner<32>(s);
  s = s + xor_partner<16>(s);
  s = s + xor_partner<8>(s);
  s = s + xor_partner<4>(s);
  s = s + xor_partner<2>(s);
  s = s + xor_partner<1>(s);
  return s;
}

template <bool COHERENT>
__device__ __forceinline__ void store8(int8_t* p, uint32_t lo, uint32_t hi) {
  if (COHERENT)
    st_coherent(reinterpret_cast<uint64_t*>(p), (uint64_t)lo | ((uint64_t)hi << 32));
  else
    *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
}

// Stores the quantised chunk c (8 bytes lo|hi) of row m.  Chunks c and c^1
// (lanes t and t^1 of one wave) fill one 16-byte slot of the operand layout,
// so a wave's store instruction writes whole slots.  With COHERENT the store
// is an agent-scope atomic one (write-through to the memory side), emitted by
// the compiler, whose hazard checks cover its data registers (a hand-written
// 16-byte store in inline asm is invisible to them: a VALU write of the store
// data right after it corrupted the last lanes' bytes).
template <bool COHERENT>
__device__ __forceinline__ void store_chunk(int8_t* xa, int m, int c, int KS, uint32_t lo, uint32_t hi) {
  store8<COHERENT>(xa + xa_offset(m, 8 * c, KS), lo, hi);
}
// The fused decode kernel's own operand tile (rows m < 32, written and read
// inside one launch): the same 1 KiB block per 32-k step, but row m's 32
// bytes (both k-groups) at byte 32 m of the block, so a 128-byte line holds 4
// rows and a row's store of 64 chunks feeds 16 lines instead of 32 (the rows'
// stores are acknowledged sooner).  Chunks 4i .. 4i + 3 are 32 consecutive
// bytes of block i.
__device__ __forceinline__ int64_t fused_chunk_offset(int m, int c) {
  return (int64_t)(c >> 2) * 1024 + (m & 31) * 32 + (c & 3) * 8;
}
template <bool FUSED>
__device__ __forceinline__ int64_t operand_chunk_offset(int m, int c, int KS) {
  return FUSED ? fused_chunk_offset(m, c) : xa_offset(m, 8 * c, KS);
}

// ---- pieces of the row prologue shared by every kernel that runs it -------
// A row lives in registers as v[i][0..7] = elements 8c..8c+7 of chunk
// c = tid + kActThreads*i (512 threads: all eight waves of the row's block);
// only chunks c < nch hold data.

// 1/sqrt(sum(v^2)/K + eps) in the fixed order described above (one barrier).
template <int CPT>
__device__ __forceinline__ float row_rms_inv(const float (&v)[CPT][8], int nch, int K, float eps, int tid,
                                             float* s_sum) {
  const bool active = tid < kActThreads;
  const int lane = tid & 63, wv = tid >> 6;
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i)
    if (active && tid + kActThreads * i < nch) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sq = v[i][j] * v[i][j];
        s = s + sq;
      }
    }
  s = wave_xor_sum(s);
  if (active && lane == 0) s_sum[wv] = s;
  __syncthreads();
  const float ss = sum8_fixed(s_sum);
  const float var = ss / (float)K;
  return 1.0f / sqrtf(var + eps);
}

// The two bf16 halves of a word as floats.
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// A row's gains, bf16 pairs as loaded, as floats.
template <int CPT>
__device__ __forceinline__ void gains_to_floats(const uint4 (&graw)[CPT], float (&g)[CPT][8]) {
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const uint32_t g4[4] = {graw[i].x, graw[i].y, graw[i].z, graw[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      g[i][2 * j] = bf_lo(g4[j]);
      g[i][2 * j + 1] = bf_hi(g4[j]);
    }
  }
}

// y = bf16(g * bf16(x * r)), in place, with the gains as floats.  Each
// v_cvt_pk_bf16_f32 rounds two values, each exactly as f2bf.
template <int CPT>
__device__ __forceinline__ void row_apply_norm_f(float (&v)[CPT][8], const float (&g)[CPT][8], float r, int nch,
                                                 int tid) {
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    if (tid < kActThreads && c < nch) {
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const uint32_t t = f2bf_pair(v[i][j] * r, v[i][j + 1] * r);
        const uint32_t y = f2bf_pair(g[i][j] * bf_lo(t), g[i][j + 1] * bf_hi(t));
        v[i][j] = bf_lo(y);
        v[i][j + 1] = bf_hi(y);
      }
    }
  }
}

// y = bf16(gamma * bf16(x * r)) (or bf16(x * r) without gamma), in place.
template <int CPT>
__device__ __forceinline__ void row_apply_norm(float (&v)[CPT][8], const uint4 (&graw)[CPT], bool has_gamma,
                                               float r, int nch, int tid) {
  if (has_gamma) {
    float g[CPT][8];
    gains_to_floats<CPT>(graw, g);
    row_apply_norm_f<CPT>(v, g, r, nch, tid);
    return;
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    if (tid < kActThreads && c < nch) {
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const uint32_t t = f2bf_pair(v[i][j] * r, v[i][j + 1] * r);
        v[i][j] = bf_lo(t);
        v[i][j + 1] = bf_hi(t);
      }
    }
  }
}

// a = max(max|v|, act_eps) over the row (one barrier).  Past the thread's own
// elements the maxima are taken on the bit patterns: for non-negative floats
// the unsigned order is the float order, and integer max needs none of the
// NaN canonicalisation fmaxf adds to every step.
template <int CPT>
__device__ __forceinline__ float row_absmax(const float (&v)[CPT][8], int nch, float act_eps, int tid,
                                            float* s_max) {
  const bool active = tid < kActThreads;
  const int lane = tid & 63, wv = tid >> 6;
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i)
    if (active && tid + kActThreads * i < nch) {
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[i][j]));
    }
  uint32_t u = __float_as_uint(amax);
  u = max(u, xor_partner_u<32>(u));
  u = max(u, xor_partner_u<16>(u));
  u = max(u, xor_partner_u<8>(u));
  u = max(u, xor_partner_u<4>(u));
  u = max(u, xor_partner_u<2>(u));
  u = max(u, xor_partner_u<1>(u));
  uint32_t* s_maxu = reinterpret_cast<uint32_t*>(s_max);
  if (active && lane == 0) s_maxu[wv] = u;
  __syncthreads();
  uint32_t m = s_maxu[0];
#pragma unroll
  for (int w = 1; w < kActWaves; ++w) m = max(m, s_maxu[w]);
  const float a = __uint_as_float(m);
  return a > act_eps ? a : act_eps;
}

// Eight quantised values q = clip(rne(v * scale), -128, 127) packed
// little-endian into two words; rs += their sum.  Every caller passes
// scale = 127/a with a >= max|v| over the row (a = max(max|v|, 1e-5)), so
// |fl(v * scale)| <= 127 (1 + 2^-24)^2 < 127.5 for finite v and the clip never
// binds.  For |t| < 2^22, fl(t + 1.5 * 2^23) is 1.5 * 2^23 + rne(t) (ties to
// even, as rintf), whose bit pattern is 0x4B400000 + rne(t): its low byte is
// the two's complement int8 code.  v_perm_b32 gathers the four low bytes of a
// word, and v_dot4 against 0x01010101 sums its four signed bytes.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  return __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u) | __builtin_amdgcn_perm(b3, b2, 0x04000c0cu);
}
__device__ __forceinline__ void quant8(const float (&v)[8], float scale, uint32_t& lo, uint32_t& hi, int& rs) {
  uint32_t b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float t = v[j] * scale;
    b[j] = __float_as_uint(t + 12582912.0f);
  }
  lo = pack_low_bytes(b[0], b[1], b[2], b[3]);
  hi = pack_low_bytes(b[4], b[5], b[6], b[7]);
  rs = __builtin_amdgcn_sdot4((int)lo, 0x01010101, rs, false);
  rs = __builtin_amdgcn_sdot4((int)hi, 0x01010101, rs, false);
}

// Row m of the activation prologue.  Threads 0..255 do the work; any further
// threads of the block only take part in the barriers.  With COHERENT the
// quantised row and a_dq are written with coherent stores, the row into the
// fused decode kernel's own tile layout (for a consumer in the same launch).
template <bool NORM, bool QUANT, bool COHERENT, int CPT>
__device__ void act_row(const ActArgs& p, int m, int tid) {
  static_assert(CPT >= 1 && CPT <= kActMaxChunks, "chunks per thread");
  const bool active = tid < kActThreads;
  const int lane = tid & 63, wv = tid >> 6;
  __shared__ float s_sum[kActWaves];
  __shared__ float s_max[kActWaves];
  __shared__ int s_int[kActWaves];

  if (p.zero_words && m == 0 && active)
    for (int i = tid; i < p.n_zero_words; i += kActThreads) {
      if (COHERENT)
        st_coherent(p.zero_words + i, 0u);
      else
        p.zero_words[i] = 0u;
    }

  const int nch = p.K >> 3;    // 8-element chunks holding data
  const int nchp = p.KS * 16;  // chunks up to the 128-column padding
  if (m >= p.M) {              // padding row of the last 32-row block
    if (QUANT && active) {
      for (int c = tid; c < nchp; c += kActThreads)
        store8<COHERENT>(p.xa + operand_chunk_offset<COHERENT>(m, c, p.KS), 0u, 0u);
      if (tid == 0) {
        if (COHERENT)
          st_coherent(p.a_dq + m, 0.0f);
        else
          p.a_dq[m] = 0.0f;
        if (p.rowsum) p.rowsum[m] = 0;
      }
    }
    return;
  }

  const uint16_t* xr = p.x + (int64_t)m * p.ldx;
  float v[CPT][8];
  // gamma travels with x: both loads are in flight before the first barrier.
  uint4 graw[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    graw[i] = make_uint4(0u, 0u, 0u, 0u);
    if (NORM && p.gamma && active && c < nch) graw[i] = *reinterpret_cast<const uint4*>(p.gamma + 8 * c);
  }
  // all loads are issued before the first conversion waits for one
  uint4 raw[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    raw[i] = make_uint4(0u, 0u, 0u, 0u);
    if (active && c < nch) raw[i] = *reinterpret_cast<const uint4*>(xr + 8 * c);
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const uint32_t w4[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[i][2 * j] = bf2f((uint16_t)(w4[j] & 0xffffu));
      v[i][2 * j + 1] = bf2f((uint16_t)(w4[j] >> 16));
    }
  }

  if (NORM) {
    const float r = row_rms_inv<CPT>(v, nch, p.K, p.norm_eps, tid, s_sum);
    row_apply_norm<CPT>(v, graw, p.gamma != nullptr, r, nch, tid);
  }

  if (!QUANT || p.y_rm) {
    uint16_t* yr = p.y_rm + (int64_t)m * p.K;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + kActThreads * i;
      if (active && c < nch) {
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

  const float a = row_absmax<CPT>(v, nch, p.act_eps, tid, s_max);
  const float scale = 127.0f / a;
  if (tid == 0) {
    if (COHERENT)
      st_coherent(p.a_dq + m, a / 127.0f);
    else
      p.a_dq[m] = a / 127.0f;
    if (p.act_scale) p.act_scale[m] = scale;
  }

  int rs = 0;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    if (active && c < nch) {
      uint32_t lo, hi;
      quant8(v[i], scale, lo, hi, rs);
      store8<COHERENT>(p.xa + operand_chunk_offset<COHERENT>(m, c, p.KS), lo, hi);
      if (p.xq_rm) *reinterpret_cast<uint2*>(p.xq_rm + (int64_t)m * p.K + 8 * c) = make_uint2(lo, hi);
    }
  }
  if (active)
    for (int c = nch + tid; c < nchp; c += kActThreads)
      store8<COHERENT>(p.xa + operand_chunk_offset<COHERENT>(m, c, p.KS), 0u, 0u);

  if (!p.rowsum) return;  // the GEMM derives row sums from its operand
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) rs += __shfl_xor(rs, off, 64);
  if (active && lane == 0) s_int[wv] = rs;
  __syncthreads();
  if (tid == 0) {
    int32_t total = 0;
#pragma unroll
    for (int w = 0; w < kActWaves; ++w) total += s_int[w];
    if (COHERENT)
      st_coherent(p.rowsum + m, total);
    else
      p.rowsum[m] = total;
  }
}

}  // namespace btl
