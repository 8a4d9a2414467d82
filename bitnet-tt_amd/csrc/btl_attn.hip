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
// One workgroup per (user, key-value head, chunk of 128 positions): it
// applies RoPE to the G = H / Hkv query rows of the group; the chunk that
// holds the user's position also writes the rotated k row and the v row into
// the caches.  Scores come from v_mfma_f32_16x16x32_bf16 (the G query rows,
// padded to 16, against 16 cached key rows per MFMA; keys are contiguous
// along D, the contraction), softmax runs in fp32 in a fixed order, and the
// probability-weighted sum of value rows runs on the VALU (a wave per query
// head, lanes over D, value rows read whole).  Chunks meet through a
// workspace: each writes (max, sum, unnormalised output) per head, and the
// last chunk of a (user, head group) to finish -- an atomic counter it resets
// -- combines them in chunk order and writes the output.
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
constexpr int kAtPart = 2 + kAtD;  // floats per head partial: max, sum, output

struct AttnArgs {
  const uint16_t* qkv;
  int ldq;                 // elements per qkv row
  const int32_t* pos;      // [B] position of each user's new token
  const float* rcos;       // [S, D/2] cos of position x frequency i
  const float* rsin;       // [S, D/2]
  uint16_t* kc;            // [B, Hkv, S, D]
  uint16_t* vc;            // [B, Hkv, S, D]
  uint16_t* out;           // [B, H * D]
  float* part;             // [B, Hkv, NS, G, kAtPart]
  uint32_t* count;         // [B, Hkv] chunks done (zero between calls)
  int32_t* error;          // set when a position is outside [0, S)
  int B, H, Hkv, G, S, NS;
  float scale;
  int adjacent;            // 1: RoPE pairs (2i, 2i+1); 0: (i, i + D/2)
};

// Rotates one pair (x0, x1) by the angle of frequency i at the position.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float& y0, float& y1) {
  y0 = x0 * c - x1 * s;
  y1 = x1 * c + x0 * s;
}

__global__ __launch_bounds__(256) void k_decode_attention(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t s_q[16][kAtD];  // MFMA A operand: G rotated query rows, rest 0
  __shared__ float s_p[kAtMaxG][kAtChunk];                          // scores, then exp(score - max)
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int sp = blockIdx.x % p.NS;
  const int hk = (blockIdx.x / p.NS) % p.Hkv;
  const int b = blockIdx.x / (p.NS * p.Hkv);
  const int G = p.G;
  const int pos = p.pos[b];
  const bool pos_ok = pos >= 0 && pos < p.S;
  const int last_pos = pos_ok ? pos : -1;
  const int s0 = sp * kAtChunk;
  const int s1 = min(s0 + kAtChunk, last_pos + 1);  // this chunk covers [s0, s1)
  if (!pos_ok && tid == 0 && sp == 0) st_coherent(p.error, 1);

  const uint16_t* qrow = p.qkv + (int64_t)b * p.ldq;
  const int64_t kv_base = ((int64_t)b * p.Hkv + hk) * p.S;  // row index of (b, hk, position 0)
  const int half = kAtD / 2;

  // rotated query rows of the group into LDS; the chunk holding the position
  // writes the rotated k row and the v row into the caches
  for (int t = tid; t < 16 * half; t += 256) {
    const int g = t / half, i = t % half;
    const int d0 = p.adjacent ? 2 * i : i, d1 = p.adjacent ? 2 * i + 1 : i + half;
    uint16_t o0 = 0, o1 = 0;
    if (g < G && pos_ok) {
      const uint16_t* q = qrow + (hk * G + g) * kAtD;
      float y0, y1;
      rope_pair(bf2f(q[d0]), bf2f(q[d1]), p.rcos[pos * half + i], p.rsin[pos * half + i], y0, y1);
      o0 = f2bf(y0);
      o1 = f2bf(y1);
    }
    s_q[g][d0] = o0;
    s_q[g][d1] = o1;
  }
  const bool owner = pos_ok && pos >= s0 && pos < s0 + kAtChunk;
  if (owner) {
    if (tid < half) {
      const int i = tid;
      const int d0 = p.adjacent ? 2 * i : i, d1 = p.adjacent ? 2 * i + 1 : i + half;
      const uint16_t* k = qrow + (p.H + hk) * kAtD;
      float y0, y1;
      rope_pair(bf2f(k[d0]), bf2f(k[d1]), p.rcos[pos * half + i], p.rsin[pos * half + i], y0, y1);
      uint16_t* dst = p.kc + (kv_base + pos) * kAtD;
      dst[d0] = f2bf(y0);
      dst[d1] = f2bf(y1);
    } else if (tid < 2 * half) {
      const int d = 2 * (tid - half);
      const uint32_t v = *reinterpret_cast<const uint32_t*>(qrow + (p.H + p.Hkv + hk) * kAtD + d);
      *reinterpret_cast<uint32_t*>(p.vc + (kv_base + pos) * kAtD + d) = v;
    }
    wait_memory();  // the rows are in L2 before this workgroup reads them back
  }
  __syncthreads();

  // scores: wave w takes position blocks of 16 from s0 + 16 w, step 64
  for (int blk = s0 + 16 * wv; blk < s1; blk += 64) {
    v4f acc = (v4f){0.f, 0.f, 0.f, 0.f};
    const int prow = blk + (lane & 15);
    const int prc = prow < s1 ? prow : s1 - 1;  // a valid row; its score is masked below
    const uint16_t* krow = p.kc + (kv_base + prc) * kAtD + 8 * (lane >> 4);
#pragma unroll
    for (int ks = 0; ks < kAtD / 32; ++ks) {
      const uint4 kb = *reinterpret_cast<const uint4*>(krow + 32 * ks);
      const uint4 qa = *reinterpret_cast<const uint4*>(&s_q[lane & 15][32 * ks + 8 * (lane >> 4)]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, qa), __builtin_bit_cast(v8bf, kb), acc,
                                                    0, 0, 0);
    }
    // lanes 0..15 hold rows 0..3 (the query heads) at column lane: position blk + lane
    if (lane < 16) {
#pragma unroll
      for (int g = 0; g < kAtMaxG; ++g)
        if (g < G) s_p[g][blk + lane - s0] = blk + lane < s1 ? acc[g] * p.scale : -__builtin_inff();
    }
  }
  __syncthreads();

  // softmax statistics and the weighted value sum: wave g = query head g
  const int g = wv;
  const int n = s1 - s0;  // positions of this chunk (may be <= 0)
  float m = -__builtin_inff(), l = 0.0f, o0 = 0.0f, o1 = 0.0f;
  if (g < G && n > 0) {
    float mx = -__builtin_inff();
    for (int j = lane; j < n; j += 64) mx = fmaxf(mx, s_p[g][j]);
    m = wave_xor_max(mx);
    float sum = 0.0f;
    for (int j = lane; j < n; j += 64) {
      const float e = __expf(s_p[g][j] - m);
      s_p[g][j] = e;
      sum += e;
    }
    l = wave_xor_sum(sum);
  }
  __syncthreads();  // exponentials visible to the whole wave (written by other lanes)
  if (g < G && n > 0) {
    const uint16_t* vrow = p.vc + (kv_base + s0) * kAtD + 2 * lane;
    for (int j = 0; j < n; ++j) {
      const uint32_t v = *reinterpret_cast<const uint32_t*>(vrow + (int64_t)j * kAtD);
      const float e = s_p[g][j];
      o0 += e * bf2f((uint16_t)(v & 0xffffu));
      o1 += e * bf2f((uint16_t)(v >> 16));
    }
  }

  const int64_t bh = (int64_t)b * p.Hkv + hk;
  auto write_out = [&](int gg, float v0, float v1) {
    uint16_t* o = p.out + (int64_t)b * p.H * kAtD + (hk * G + gg) * kAtD + 2 * lane;
    *reinterpret_cast<uint32_t*>(o) = (uint32_t)f2bf(v0) | ((uint32_t)f2bf(v1) << 16);
  };
  if (p.NS == 1) {
    if (g < G) {
      const float inv = l > 0.0f ? 1.0f / l : 0.0f;
      write_out(g, o0 * inv, o1 * inv);
    }
    return;
  }
  // publish this chunk's partials; the last chunk of (b, hk) combines
  if (g < G) {
    float* pp = p.part + ((bh * p.NS + sp) * G + g) * kAtPart;
    if (lane == 0) {
      st_coherent(pp, m);
      st_coherent(pp + 1, l);
    }
    st_coherent(pp + 2 + 2 * lane, o0);
    st_coherent(pp + 3 + 2 * lane, o1);
  }
  wait_memory();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(p.count + bh, 1u) + 1u == (uint32_t)p.NS;
  __syncthreads();
  if (!s_last) return;
  if (g < G) {
    float M = -__builtin_inff();
    for (int c = 0; c < p.NS; ++c) M = fmaxf(M, ld_coherent(p.part + ((bh * p.NS + c) * G + g) * kAtPart));
    float L = 0.0f, O0 = 0.0f, O1 = 0.0f;
    for (int c = 0; c < p.NS; ++c) {
      const float* pp = p.part + ((bh * p.NS + c) * G + g) * kAtPart;
      const float mc = ld_coherent(pp);
      if (mc == -__builtin_inff()) continue;  // an empty chunk
      const float w = __expf(mc - M);
      L += w * ld_coherent(pp + 1);
      O0 += w * ld_coherent(pp + 2 + 2 * lane);
      O1 += w * ld_coherent(pp + 3 + 2 * lane);
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    write_out(g, O0 * inv, O1 * inv);
  }
  if (tid == 0) st_coherent(p.count + bh, 0u);
}

}  // namespace btl

using namespace btl;

extern "C" {

int64_t btl_decode_attention_workspace_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t S) {
  if (B <= 0 || Hkv <= 0 || H <= 0 || H % Hkv || H / Hkv > kAtMaxG || S <= 0) return 0;
  const int64_t ns = (S + kAtChunk - 1) / kAtChunk;
  const int64_t counters = round_up(B * Hkv * 4 + 4, 256);  // counters, then the error word
  return counters + B * Hkv * ns * (H / Hkv) * kAtPart * 4;
}

int64_t btl_decode_attention_error_offset(int64_t B, int64_t Hkv) { return B * Hkv * 4; }

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
  a.NS = (int)((S + kAtChunk - 1) / kAtChunk);
  a.scale = scale;
  a.adjacent = rope_adjacent ? 1 : 0;
  char* ws = reinterpret_cast<char*>(workspace);
  a.count = reinterpret_cast<uint32_t*>(ws);
  a.error = reinterpret_cast<int32_t*>(ws + btl_decode_attention_error_offset(B, Hkv));
  a.part = reinterpret_cast<float*>(ws + round_up(B * Hkv * 4 + 4, 256));
  const dim3 grid((unsigned)(B * Hkv * a.NS));
  hipLaunchKernelGGL(k_decode_attention, grid, dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("decode attention");
}

}  // extern "C"
