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
// One workgroup per (user, key-value head) streams the cached context in
// chunks of 128 positions, each wave taking 32 of them: the wave's K operands
// and value rows of the next chunk are in flight in registers while the
// current chunk is processed.  The prologue rotates the G = H / Hkv query
// rows of the group and the new k row (RoPE), which goes with the v row into
// the caches before the rows of the last chunk -- the one that holds it -- are
// read.  Scores come from
// v_mfma_f32_16x16x32_bf16 (the G query rows, padded to 16, against 16 cached
// key rows per MFMA; keys are contiguous along D, the contraction).  The
// softmax is the running (online) form in fp32: every wave derives the same
// chunk maximum, rescale factor and sum from the chunk's scores in LDS, so
// the waves' partial outputs share one scale and are summed in a fixed order
// at the end.  The probability-weighted value rows accumulate on the VALU
// (lanes over D, value rows read whole).
#include <hip/hip_runtime.h>

#include "btl.h"
#include "btl_act_row.h"
#include "btl_common.h"

namespace btl {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kAtD = 128;       // head dimension
constexpr int kAtChunk = 128;   // positions per workgroup
constexpr int kAtMaxG = 4;      // query heads per key-value head handled (one wave each)

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

// Cached rows of one chunk held in registers by a wave (its 32 positions):
// the K operands of its two 16-position MFMA blocks (4 k-steps each), and its
// value rows as 16-byte pieces: v[t] = dims 8 (lane & 15) .. + 8 of the row
// 4 t + (lane >> 4).
struct AttnChunkRegs {
  uint4 k[2][kAtD / 32];
  uint4 v[8];
};

__global__ __launch_bounds__(256, 1) void k_decode_attention(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t s_q[16][kAtD];   // MFMA A operand: G rotated query rows, rest 0
  __shared__ __attribute__((aligned(16))) uint16_t s_new[2][kAtD];  // the new k (rotated) and v rows
  __shared__ float s_pw[4][kAtMaxG][32];                             // each wave's probabilities of a chunk
  __shared__ float s_ml[4][kAtMaxG][2];                              // each wave's running max and sum
  __shared__ float s_o[4][kAtMaxG][kAtD];                            // each wave's unnormalised output
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int dg = lane & 15, rg = lane >> 4;  // value piece: dims 8 dg .. + 8 of rows rg + 4 t
  const int hk = blockIdx.x % p.Hkv;
  const int b = blockIdx.x / p.Hkv;
  const int G = p.G;
  const int pos = p.pos[b];
  const bool pos_ok = pos >= 0 && pos < p.S;
  if (!pos_ok && tid == 0 && hk == 0) st_coherent(p.error, 1);
  const int nold = pos_ok ? pos : 0;             // cached positions [0, nold); the new one is pos
  const int nch = (nold + kAtChunk - 1) / kAtChunk;
  const int pc = pos_ok ? pos : 0;
  const uint16_t* qrow = p.qkv + (int64_t)b * p.ldq;
  const int64_t kv_base = ((int64_t)b * p.Hkv + hk) * p.S;  // row index of (b, hk, position 0)
  const int half = kAtD / 2;

  // this wave's rows of chunk c: positions c*128 + 32 wv + [0, 32)
  auto load_chunk = [&](AttnChunkRegs& r, int c) __attribute__((always_inline)) {
    const int cc = c < nch ? c : (nch > 0 ? nch - 1 : 0);  // a valid chunk; extra ones are never used
    const int base = cc * kAtChunk + 32 * wv;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const int row = min(base + 16 * blk + (lane & 15), p.S - 1);
      const uint16_t* kr = p.kc + (kv_base + row) * kAtD + 8 * (lane >> 4);
#pragma unroll
      for (int ks = 0; ks < kAtD / 32; ++ks) r.k[blk][ks] = *reinterpret_cast<const uint4*>(kr + 32 * ks);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int row = min(base + 4 * t + rg, p.S - 1);
      r.v[t] = *reinterpret_cast<const uint4*>(p.vc + (kv_base + row) * kAtD + 8 * dg);
    }
  };

  // the rows of the first two chunks go out first (they never include the
  // new position), then the small loads of the new q, k, v rows
  AttnChunkRegs ra, rb;
  load_chunk(ra, 0);
  load_chunk(rb, 1);
  float qx0[4], qx1[4], rc, rs, kx0, kx1;
  uint32_t vnew;
  {
    const int i = tid & (half - 1);
    const int d0 = p.adjacent ? 2 * i : i, d1 = p.adjacent ? 2 * i + 1 : i + half;
    rc = p.rcos[pc * half + i];
    rs = p.rsin[pc * half + i];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = min((tid + 256 * u) / half, G - 1);
      const uint16_t* q = qrow + (hk * G + g) * kAtD;
      qx0[u] = bf2f(q[d0]);
      qx1[u] = bf2f(q[d1]);
    }
    const uint16_t* k = qrow + (p.H + hk) * kAtD;
    kx0 = bf2f(k[d0]);
    kx1 = bf2f(k[d1]);
    vnew = *reinterpret_cast<const uint32_t*>(qrow + (p.H + p.Hkv + hk) * kAtD + 2 * i);
  }
  // RoPE of the group's query rows (rows >= G stay 0) and of the new k row;
  // the new rows go to LDS and to the caches (read by later calls)
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = tid + 256 * u, g = t / half, i = t % half;
    const int d0 = p.adjacent ? 2 * i : i, d1 = p.adjacent ? 2 * i + 1 : i + half;
    float y0, y1;
    rope_pair(qx0[u], qx1[u], rc, rs, y0, y1);
    const bool live = g < G && pos_ok;
    s_q[g][d0] = live ? f2bf(y0) : (uint16_t)0;
    s_q[g][d1] = live ? f2bf(y1) : (uint16_t)0;
  }
  if (tid < half) {
    const int i = tid;
    const int d0 = p.adjacent ? 2 * i : i, d1 = p.adjacent ? 2 * i + 1 : i + half;
    float y0, y1;
    rope_pair(kx0, kx1, rc, rs, y0, y1);
    const uint16_t k0 = f2bf(y0), k1 = f2bf(y1);
    s_new[0][d0] = k0;
    s_new[0][d1] = k1;
    if (pos_ok) {
      uint16_t* dst = p.kc + (kv_base + pos) * kAtD;
      dst[d0] = k0;
      dst[d1] = k1;
    }
  } else if (tid < 2 * half) {
    const int d = 2 * (tid - half);
    *reinterpret_cast<uint32_t*>(&s_new[1][d]) = vnew;
    if (pos_ok) *reinterpret_cast<uint32_t*>(p.vc + (kv_base + pos) * kAtD + d) = vnew;
  }
  __syncthreads();

  // each wave: running softmax over its own positions, per head
  float m[kAtMaxG], l[kAtMaxG], o[kAtMaxG][8];
#pragma unroll
  for (int g = 0; g < kAtMaxG; ++g) {
    m[g] = -__builtin_inff();
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
  }

  auto process = [&](AttnChunkRegs& r, int c) __attribute__((always_inline)) {
    const int base = c * kAtChunk + 32 * wv;  // this wave's first position
    v4f acc[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      acc[blk] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kAtD / 32; ++ks) {
        const uint4 qa = *reinterpret_cast<const uint4*>(&s_q[lane & 15][32 * ks + 8 * (lane >> 4)]);
        acc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, qa),
                                                           __builtin_bit_cast(v8bf, r.k[blk][ks]), acc[blk], 0, 0, 0);
      }
    }
    // lanes 0..15: head g's scores of positions base + lane (block 0) and
    // base + 16 + lane (block 1); reduce over those 16 lanes
#pragma unroll
    for (int g = 0; g < kAtMaxG; ++g) {
      const bool ok0 = lane < 16 && base + lane < nold, ok1 = lane < 16 && base + 16 + lane < nold;
      const float s0 = ok0 ? acc[0][g] * p.scale : -__builtin_inff();
      const float s1 = ok1 ? acc[1][g] * p.scale : -__builtin_inff();
      // butterflies within each 16-lane row (DPP), then lane 0's row for all
      float mx = fmaxf(s0, s1);
      mx = fmaxf(mx, xor_partner<8>(mx));
      mx = fmaxf(mx, xor_partner<4>(mx));
      mx = fmaxf(mx, xor_partner<2>(mx));
      mx = fmaxf(mx, xor_partner<1>(mx));
      mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 0));
      const float mn = fmaxf(m[g], mx);
      const float alpha = m[g] == -__builtin_inff() ? 0.0f : __expf(m[g] - mn);
      const float e0 = ok0 ? __expf(s0 - mn) : 0.0f, e1 = ok1 ? __expf(s1 - mn) : 0.0f;
      float sm = e0 + e1;
      sm += xor_partner<8>(sm);
      sm += xor_partner<4>(sm);
      sm += xor_partner<2>(sm);
      sm += xor_partner<1>(sm);
      sm = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sm), 0));
      l[g] = l[g] * alpha + sm;
      m[g] = mn;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
      if (lane < 16) {
        s_pw[wv][g][lane] = e0;
        s_pw[wv][g][16 + lane] = e1;
      }
    }
    __builtin_amdgcn_wave_barrier();  // the wave's own LDS writes are read back by other lanes
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      // rows past the context count as zero (whatever the cache holds there)
      const bool vok = base + 4 * t + rg < nold;
      const uint32_t w4[4] = {vok ? r.v[t].x : 0u, vok ? r.v[t].y : 0u, vok ? r.v[t].z : 0u, vok ? r.v[t].w : 0u};
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = bf2f((uint16_t)(w4[e] & 0xffffu));
        v[2 * e + 1] = bf2f((uint16_t)(w4[e] >> 16));
      }
#pragma unroll
      for (int g = 0; g < kAtMaxG; ++g) {
        const float pe = s_pw[wv][g][4 * t + rg];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] += pe * v[e];
      }
    }
    __builtin_amdgcn_wave_barrier();  // reads done before the next chunk rewrites s_pw
  };

  for (int c = 0; c < nch; c += 2) {
    process(ra, c);
    load_chunk(ra, c + 2);
    if (c + 1 < nch) process(rb, c + 1);
    load_chunk(rb, c + 3);
  }

  // each wave's partial (row groups summed within the wave) into LDS
#pragma unroll
  for (int g = 0; g < kAtMaxG; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = o[g][e];
      x += xor_partner<16>(x);
      x += xor_partner<32>(x);
      o[g][e] = x;
    }
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < kAtMaxG; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_o[wv][g][8 * dg + e] = o[g][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < kAtMaxG; ++g) {
      s_ml[wv][g][0] = m[g];
      s_ml[wv][g][1] = l[g];
    }
  }
  __syncthreads();

  // wave g merges head g: the four waves' partials and the new position
  const int g = wv;
  if (g < G) {
    // score of the new position (lanes over D, fixed-order sum)
    float d = bf2f(s_q[g][2 * lane]) * bf2f(s_new[0][2 * lane]) + bf2f(s_q[g][2 * lane + 1]) * bf2f(s_new[0][2 * lane + 1]);
    const float snew = wave_xor_sum(d) * p.scale;
    float M = snew;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_ml[w][g][0]);
    const float wn = __expf(snew - M);
    float L = wn;
    float O0 = wn * bf2f(s_new[1][2 * lane]), O1 = wn * bf2f(s_new[1][2 * lane + 1]);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = s_ml[w][g][0];
      const float ww = mw == -__builtin_inff() ? 0.0f : __expf(mw - M);
      L += ww * s_ml[w][g][1];
      O0 += ww * s_o[w][g][2 * lane];
      O1 += ww * s_o[w][g][2 * lane + 1];
    }
    const float inv = pos_ok ? 1.0f / L : 0.0f;
    uint16_t* out = p.out + (int64_t)b * p.H * kAtD + (hk * G + g) * kAtD + 2 * lane;
    *reinterpret_cast<uint32_t*>(out) = (uint32_t)f2bf(O0 * inv) | ((uint32_t)f2bf(O1 * inv) << 16);
  }
}

}  // namespace btl

using namespace btl;

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
  char* ws = reinterpret_cast<char*>(workspace);
  a.error = reinterpret_cast<int32_t*>(ws);
  const dim3 grid((unsigned)(B * Hkv));
  hipLaunchKernelGGL(k_decode_attention, grid, dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("decode attention");
}

}  // extern "C"
