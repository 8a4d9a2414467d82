// Decode attention between the fused QKV BitLinear and o_proj: RoPE on the new
// q and k rows, KV-cache update at each user's position, and scaled
// dot-product attention of every query head over its key-value head's cached
// positions [0, pos] (src/bitnet_tt/layers/attention.py:1040-1262: head split
// :1088-1096, RoPE :1103-1140, cache update :1153-1171, SDPA decode
// :1177-1231, head concat :1239-1254; frequencies utils/rope.py:7-23).
//
// Layout: qkv [B, (H + 2 Hkv) D] bf16 (Q heads, then K heads, then V heads);
// caches [B, Hkv, S, D] bf16 (the reference's KV-cache shape); output
// [B, H D] bf16 (heads concatenated, o_proj's input).  D = 128.
//
// One workgroup of 8 waves per (user, key-value head); a round covers 512
// cached positions, 64 per wave, and every wave issues all of its key and
// value loads (256 B per lane each) before computing, so a round is one
// memory round trip with 256 KiB in flight per CU (at the 2B shape, context
// 512, the whole context is one round).  Measured on MI355X, splitting the
// context over more workgroups (to use all 256 CUs) and merging their
// partials through the workspace was slower at this shape: the merge's
// store-acknowledge-count-reload chain costs more than the extra CUs gain.
//  - Scores: v_mfma_f32_16x16x32_bf16, the G rotated query rows (padded to
//    16 with zeros) against 16 cached key rows per MFMA (keys contiguous
//    along D, the contraction, so the B operands load straight from the
//    cache).
//  - Softmax: the running (online) form in fp32 per wave and head.
//  - Probability-weighted values: MFMA as well.  The wave's value rows go
//    to LDS (rows padded by 8 bytes, so the four position groups of an
//    operand read fall in different banks) and are read back as B operands
//    (8 positions of one dimension per lane); the probabilities enter as two
//    bf16 parts, p = hi + lo, which keeps them to ~16 bits.
//  - The waves' (max, sum, output) partials and the new position (rotated k,
//    v) merge in LDS in a fixed order.
#include <hip/hip_runtime.h>

#include "btl.h"
#include "btl_act_row.h"
#include "btl_common.h"
#include "btl_trace.h"

namespace btl {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kAtD = 128;                        // head dimension
constexpr int kAtWaves = 8;                      // waves per workgroup
constexpr int kAtPosWave = 64;                   // positions per wave and round
constexpr int kAtRound = kAtWaves * kAtPosWave;  // positions per round
constexpr int kAtMaxG = 4;                       // query heads per key-value head
constexpr int kAtVPitch = kAtD + 4;              // bf16 per LDS value row (8-byte pad)

struct AttnArgs {
  const uint16_t* qkv;
  int ldq;                 // elements per qkv row
  const int32_t* pos;      // [B] position of each user's new token
  const float* rcos;       // [S, D/2] cos of position x frequency i
  const float* rsin;       // [S, D/2]
  uint16_t* kc;            // [B, Hkv, S, D]
  uint16_t* vc;            // [B, Hkv, S, D]
  uint16_t* out;           // [B, H * D]
  int32_t* error;          // set when a position is outside [0, S)
  int B, H, Hkv, G, S;
  float scale;
  int adjacent;            // 1: RoPE pairs (2i, 2i+1); 0: (i, i + D/2)
};

// Rotates one pair (x0, x1) by the angle of frequency i at the position.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float& y0, float& y1) {
  y0 = x0 * c - x1 * s;
  y1 = x1 * c + x0 * s;
}

// Max and sum over the 16 lanes of a row (lanes 0..15 hold the values).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, xor_partner<8>(v));
  v = fmaxf(v, xor_partner<4>(v));
  v = fmaxf(v, xor_partner<2>(v));
  v = fmaxf(v, xor_partner<1>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
}
__device__ __forceinline__ float row16_sum(float v) {
  v = v + xor_partner<8>(v);
  v = v + xor_partner<4>(v);
  v = v + xor_partner<2>(v);
  v = v + xor_partner<1>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
}

__device__ __forceinline__ float wexp(float m, float M) { return m == -__builtin_inff() ? 0.0f : __expf(m - M); }

__global__ __launch_bounds__(64 * kAtWaves, 1) void k_decode_attention(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t s_q[kAtMaxG][kAtD];   // rotated query rows of the group
  __shared__ __attribute__((aligned(16))) uint16_t s_new[2][kAtD];       // the new k (rotated) and v rows
  __shared__ float s_snew[kAtMaxG];                                       // scores of the new position
  __shared__ __attribute__((aligned(16))) uint16_t s_p[kAtWaves][2][kAtMaxG][kAtPosWave];  // probabilities hi, lo
  __shared__ float s_ml[kAtWaves][kAtMaxG][2];                            // each wave's running max and sum
  // value rows of each wave's round; after the last round, each wave's
  // unnormalised output [G][D] fp32 (the LDS is reused)
  __shared__ __attribute__((aligned(16))) uint16_t s_v[kAtWaves][kAtPosWave][kAtVPitch];
  static_assert(sizeof(float) * kAtWaves * kAtMaxG * kAtD <= sizeof(uint16_t) * kAtWaves * kAtPosWave * kAtVPitch,
                "output partials fit in the value buffer");
  float (*s_o)[kAtMaxG][kAtD] = reinterpret_cast<float (*)[kAtMaxG][kAtD]>(&s_v[0][0][0]);

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  BTL_TRACE_AT(0);
  const int hk = blockIdx.x % p.Hkv;
  const int b = blockIdx.x / p.Hkv;
  const int G = p.G;
  const int pos = p.pos[b];
  const bool pos_ok = pos >= 0 && pos < p.S;
  if (!pos_ok && tid == 0 && hk == 0) st_coherent(p.error, 1);
  const int nold = pos_ok ? pos : 0;  // cached positions [0, nold); the new one is pos
  const int nrounds = (nold + kAtRound - 1) / kAtRound;
  const int pc = pos_ok ? pos : 0;
  const uint16_t* qrow = p.qkv + (int64_t)b * p.ldq;
  const int64_t kv_base = ((int64_t)b * p.Hkv + hk) * p.S;  // row index of (b, hk, position 0)
  const int half = kAtD / 2;
  const int r16 = lane & 15, grp = lane >> 4;

  // this wave's rows of round rd: positions rd*512 + 64 wv + [0, 64)
  uint4 kr[4][kAtD / 32];  // K operands: 4 blocks of 16 positions x 4 k-steps
  uint4 vr[16];            // value pieces: dims 8 r16 .. + 8 of row 4 t + grp
  auto load_round = [&](int rd) __attribute__((always_inline)) {
    const int base = rd * kAtRound + kAtPosWave * wv;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int row = min(base + 16 * blk + r16, p.S - 1);
      const uint16_t* kp = p.kc + (kv_base + row) * kAtD + 8 * grp;
#pragma unroll
      for (int ks = 0; ks < kAtD / 32; ++ks) kr[blk][ks] = *reinterpret_cast<const uint4*>(kp + 32 * ks);
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int row = min(base + 4 * t + grp, p.S - 1);
      vr[t] = *reinterpret_cast<const uint4*>(p.vc + (kv_base + row) * kAtD + 8 * r16);
    }
  };
  const bool wave_work = kAtPosWave * wv < nold;  // this wave has cached positions in round 0
  if (wave_work) load_round(0);
  BTL_TRACE_AT(1);

  // the new q, k, v rows: RoPE of the group's query rows and of the new k
  // row; the new rows go to LDS and to the caches (read by later calls)
  {
    const int i = tid & (half - 1);
    const int d0 = p.adjacent ? 2 * i : i, d1 = p.adjacent ? 2 * i + 1 : i + half;
    const float rc = p.rcos[pc * half + i], rs = p.rsin[pc * half + i];
    const int u = tid / half;  // 0..7: query rows 0..3, then the k row, then v
    if (u < kAtMaxG) {
      float y0 = 0.0f, y1 = 0.0f;
      if (u < G && pos_ok) {
        const uint16_t* q = qrow + (hk * G + u) * kAtD;
        rope_pair(bf2f(q[d0]), bf2f(q[d1]), rc, rs, y0, y1);
      }
      s_q[u][d0] = f2bf(y0);
      s_q[u][d1] = f2bf(y1);
    } else if (u == kAtMaxG) {
      const uint16_t* k = qrow + (p.H + hk) * kAtD;
      float y0, y1;
      rope_pair(bf2f(k[d0]), bf2f(k[d1]), rc, rs, y0, y1);
      const uint16_t k0 = f2bf(y0), k1 = f2bf(y1);
      s_new[0][d0] = k0;
      s_new[0][d1] = k1;
      if (pos_ok) {
        uint16_t* dst = p.kc + (kv_base + pos) * kAtD;
        dst[d0] = k0;
        dst[d1] = k1;
      }
    } else if (u == kAtMaxG + 1) {
      const int d = 2 * i;
      const uint32_t vnew = *reinterpret_cast<const uint32_t*>(qrow + (p.H + p.Hkv + hk) * kAtD + d);
      *reinterpret_cast<uint32_t*>(&s_new[1][d]) = vnew;
      if (pos_ok) *reinterpret_cast<uint32_t*>(p.vc + (kv_base + pos) * kAtD + d) = vnew;
    }
  }
  __syncthreads();
  BTL_TRACE_AT(2);
  if (wv < G) {  // score of the new position for head wv (lanes over D, fixed-order sum)
    const float d = bf2f(s_q[wv][2 * lane]) * bf2f(s_new[0][2 * lane]) +
                    bf2f(s_q[wv][2 * lane + 1]) * bf2f(s_new[0][2 * lane + 1]);
    const float sn = wave_xor_sum(d) * p.scale;
    if (lane == 0) s_snew[wv] = sn;
  }
  // query operands (A: row r16 = head, k-step ks: dims 32 ks + 8 grp ..)
  v8bf qa[kAtD / 32];
#pragma unroll
  for (int ks = 0; ks < kAtD / 32; ++ks) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (r16 < G) v = *reinterpret_cast<const uint4*>(&s_q[r16][32 * ks + 8 * grp]);
    qa[ks] = __builtin_bit_cast(v8bf, v);
  }

  // running softmax state of this wave, per head (lanes 0..15 hold the
  // output rows: acc o[m][j] = head j, dimension 16 m + r16)
  float mrun[kAtMaxG], lrun[kAtMaxG];
  v4f o[kAtD / 16];
#pragma unroll
  for (int g = 0; g < kAtMaxG; ++g) {
    mrun[g] = -__builtin_inff();
    lrun[g] = 0.0f;
  }
#pragma unroll
  for (int m = 0; m < kAtD / 16; ++m) o[m] = (v4f){0.f, 0.f, 0.f, 0.f};

  for (int rd = 0; rd < nrounds; ++rd) {
    const int base = rd * kAtRound + kAtPosWave * wv;
    if (base >= nold) break;  // wave-uniform: nothing cached from here on
    if (rd > 0) load_round(rd);
    // scores: 4 blocks of 16 positions
    v4f sc[4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      sc[blk] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kAtD / 32; ++ks)
        sc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], __builtin_bit_cast(v8bf, kr[blk][ks]), sc[blk], 0,
                                                          0, 0);
    }
    // value rows to LDS (rows past the context as zeros, whatever the cache
    // holds there: a zero probability times a non-finite value is NaN)
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const bool ok = base + 4 * t + grp < nold;
      const uint4 v = ok ? vr[t] : make_uint4(0u, 0u, 0u, 0u);
      uint2* dst = reinterpret_cast<uint2*>(&s_v[wv][4 * t + grp][8 * r16]);
      dst[0] = make_uint2(v.x, v.y);
      dst[1] = make_uint2(v.z, v.w);
    }
    // online softmax per head over the wave's 64 positions (lanes 0..15:
    // block blk's position 16 blk + lane)
#pragma unroll
    for (int g = 0; g < kAtMaxG; ++g) {
      float s4[4];
      float mx = -__builtin_inff();
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const bool ok = lane < 16 && base + 16 * blk + lane < nold;
        s4[blk] = ok ? sc[blk][g] * p.scale : -__builtin_inff();
        mx = fmaxf(mx, s4[blk]);
      }
      mx = row16_max(mx);
      const float mn = fmaxf(mrun[g], mx);
      const float alpha = wexp(mrun[g], mn);
      float sm = 0.0f;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const float e = wexp(s4[blk], mn);
        sm += e;
        if (lane < 16) {
          const uint16_t hi = f2bf(e);
          s_p[wv][0][g][16 * blk + lane] = hi;
          s_p[wv][1][g][16 * blk + lane] = f2bf(e - bf2f(hi));
        }
      }
      sm = row16_sum(sm);
      lrun[g] = lrun[g] * alpha + sm;
      mrun[g] = mn;
      // rows j of the output accumulators are heads: lanes 0..15 hold them
#pragma unroll
      for (int m = 0; m < kAtD / 16; ++m) o[m][g] *= alpha;
    }
    BTL_TRACE_AT(3);
    __builtin_amdgcn_wave_barrier();  // the wave's own LDS writes are read back by other lanes
    // probability-weighted values: 2 k-steps of 32 positions x 8 column
    // blocks of 16 dimensions, probabilities as hi + lo parts
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      v8bf pa[2];
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (r16 < G) v = *reinterpret_cast<const uint4*>(&s_p[wv][part][r16][32 * k2 + 8 * grp]);
        pa[part] = __builtin_bit_cast(v8bf, v);
      }
#pragma unroll
      for (int m = 0; m < kAtD / 16; ++m) {
        // B operand: dimension 16 m + r16 of positions 32 k2 + 8 grp + [0, 8)
        const uint16_t* col = &s_v[wv][32 * k2 + 8 * grp][16 * m + r16];
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = (uint32_t)col[(2 * e) * kAtVPitch] | ((uint32_t)col[(2 * e + 1) * kAtVPitch] << 16);
        const v8bf vb = __builtin_bit_cast(v8bf, make_uint4(w[0], w[1], w[2], w[3]));
        o[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[0], vb, o[m], 0, 0, 0);
        o[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[1], vb, o[m], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();  // reads done before the next round rewrites the buffers
  }
  BTL_TRACE_AT(4);

  // merge: every wave's partial, then the new position, in a fixed order
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < kAtMaxG; ++g) {
      s_ml[wv][g][0] = mrun[g];
      s_ml[wv][g][1] = lrun[g];
    }
  }
  __syncthreads();  // every wave is done with its value rows: s_o reuses them
  if (lane < 16) {
#pragma unroll
    for (int m = 0; m < kAtD / 16; ++m)
#pragma unroll
      for (int g = 0; g < kAtMaxG; ++g) s_o[wv][g][16 * m + lane] = o[m][g];
  }
  __syncthreads();
  {
    const int g = tid / kAtD, d = tid % kAtD;  // 512 threads: 4 heads x 128 dims
    if (g < G) {
      const float snew = s_snew[g];
      float M = snew;
#pragma unroll
      for (int w = 0; w < kAtWaves; ++w) M = fmaxf(M, s_ml[w][g][0]);
      const float wn = __expf(snew - M);
      float L = wn;
      float O = wn * bf2f(s_new[1][d]);
#pragma unroll
      for (int w = 0; w < kAtWaves; ++w) {
        const float ww = wexp(s_ml[w][g][0], M);
        L += ww * s_ml[w][g][1];
        O += ww * s_o[w][g][d];
      }
      const float inv = pos_ok ? 1.0f / L : 0.0f;
      p.out[(int64_t)b * p.H * kAtD + (hk * G + g) * kAtD + d] = f2bf(O * inv);
    }
  }
  BTL_TRACE_AT(5);
}

}  // namespace btl

using namespace btl;

BTL_TRACE_READ_FN(btl_trace_read_attention)

extern "C" {

int64_t btl_decode_attention_workspace_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t S) {
  if (B <= 0 || Hkv <= 0 || H <= 0 || H % Hkv || H / Hkv > kAtMaxG || S <= 0) return 0;
  return 256;  // the error word
}

int64_t btl_decode_attention_error_offset(int64_t B, int64_t Hkv) {
  (void)B;
  (void)Hkv;
  return 0;
}

int btl_decode_attention(const uint16_t* qkv, int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t S,
                         const int32_t* pos, const float* rope_cos, const float* rope_sin, int rope_adjacent,
                         float scale, uint16_t* k_cache, uint16_t* v_cache, uint16_t* out, void* workspace,
                         size_t workspace_bytes, btl_stream_t stream) {
  clear_error();
  if (D != kAtD) return set_error(BTL_ERR_SHAPE, "btl_decode_attention: head dim %lld (128 supported)", (long long)D);
  if (B <= 0 || B > 4096 || Hkv <= 0 || H <= 0 || H % Hkv || H / Hkv > kAtMaxG || S <= 0 || S > (1 << 20))
    return set_error(BTL_ERR_SHAPE, "btl_decode_attention: B=%lld H=%lld Hkv=%lld S=%lld (H/Hkv <= %d)",
                     (long long)B, (long long)H, (long long)Hkv, (long long)S, kAtMaxG);
  if (!qkv || !pos || !rope_cos || !rope_sin || !k_cache || !v_cache || !out || !workspace)
    return set_error(BTL_ERR_NULL, "btl_decode_attention: NULL pointer");
  if (!aligned(qkv, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(out, 16) ||
      !aligned(workspace, 256) || !aligned(pos, 4) || !aligned(rope_cos, 4) || !aligned(rope_sin, 4))
    return set_error(BTL_ERR_ALIGN, "btl_decode_attention: misaligned buffer");
  const int64_t need = btl_decode_attention_workspace_bytes(B, H, Hkv, S);
  if ((int64_t)workspace_bytes < need)
    return set_error(BTL_ERR_WORKSPACE, "btl_decode_attention: workspace %zu < %lld bytes", workspace_bytes,
                     (long long)need);
  AttnArgs a;
  a.qkv = qkv;
  a.ldq = (int)((H + 2 * Hkv) * D);
  a.pos = pos;
  a.rcos = rope_cos;
  a.rsin = rope_sin;
  a.kc = k_cache;
  a.vc = v_cache;
  a.out = out;
  a.B = (int)B;
  a.H = (int)H;
  a.Hkv = (int)Hkv;
  a.G = (int)(H / Hkv);
  a.S = (int)S;
  a.scale = scale;
  a.adjacent = rope_adjacent ? 1 : 0;
  a.error = reinterpret_cast<int32_t*>(workspace);
  const dim3 grid((unsigned)(B * Hkv));
  hipLaunchKernelGGL(k_decode_attention, grid, dim3(64 * kAtWaves), 0, (hipStream_t)stream, a);
  return check_launch("decode attention");
}

}  // extern "C"
