// Decode attention between the fused QKV BitLinear and o_proj: RoPE on the new
// q and k rows, KV-cache update at each user's position, and scaled
// dot-product attention of every query head over its key-value head's cached
// positions [0, pos] (src/bitnet_tt/layers/attention.py:1040-1262).  The
// per-(user, key-value head) body is btl_attn_body.h, which the persistent
// decode step runs too.
//
// Layout: qkv [B, (H + 2 Hkv) D] bf16 (Q heads, then K heads, then V heads);
// caches [B, Hkv, S, D] bf16 (the reference's KV-cache shape); output
// [B, H D] bf16 (heads concatenated, o_proj's input).  D = 128.
//
// One workgroup of 8 waves per (user, key-value head).  Measured on MI355X,
// splitting the context over more workgroups (to use all 256 CUs) and
// merging their partials through the workspace was slower at the 2B shape:
// the merge's store-acknowledge-count-reload chain costs more than the extra
// CUs gain.
#include <hip/hip_runtime.h>

#include "btl.h"
#include "btl_attn_body.h"
#include "btl_common.h"
#include "btl_trace.h"

namespace btl {

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

__global__ __launch_bounds__(64 * kAtWaves, 1) void k_decode_attention(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) AttnSmem s;
  const int tid = threadIdx.x;
  BTL_TRACE_AT(0);
  AttnPair a;
  a.rcos = p.rcos;
  a.rsin = p.rsin;
  a.kc = p.kc;
  a.vc = p.vc;
  a.Hkv = p.Hkv;
  a.G = p.G;
  a.S = p.S;
  a.hk = blockIdx.x % p.Hkv;
  a.b = blockIdx.x / p.Hkv;
  a.pos = p.pos[a.b];
  a.scale = p.scale;
  a.adjacent = p.adjacent;
  a.tid = tid;
  if (!a.pos_ok() && tid == 0 && a.hk == 0) st_coherent(p.error, 1);
  AttnRound r;
  att_load_round(a, 0, r);
  BTL_TRACE_AT(1);
  // the new token's rows of the group: q rows hk G .. hk G + G - 1, k row hk, v row hk
  const uint16_t* qrow = p.qkv + (int64_t)a.b * p.ldq;
  if (tid < (kAtMaxG + 2) * (kAtD / 8)) {
    const int u = tid / (kAtD / 8), c = tid % (kAtD / 8);
    const int src = u < kAtMaxG ? a.hk * a.G + u : u == kAtMaxG ? p.H + a.hk : p.H + p.Hkv + a.hk;
    if (u >= kAtMaxG || u < a.G)
      *reinterpret_cast<uint4*>(&s.in[u][8 * c]) = *reinterpret_cast<const uint4*>(qrow + (int64_t)src * kAtD + 8 * c);
  }
  __syncthreads();
  BTL_TRACE_AT(2);
  const uint16_t o = att_body(a, s, r, true);
  if (tid < a.G * kAtD) p.out[(int64_t)a.b * p.H * kAtD + (a.hk * a.G) * kAtD + tid] = o;
  BTL_TRACE_AT(7);
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
