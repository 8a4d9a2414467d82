// Decode attention of one (user, key-value head) pair on one 512-thread
// workgroup, shared by the standalone decode-attention kernel and the
// persistent decode step (so both give the same bits).  The arithmetic
// follows src/bitnet_tt/layers/attention.py:1040-1262 (head split
// :1088-1096, RoPE :1103-1140, cache update :1153-1171, SDPA decode
// :1177-1231, head concat :1239-1254; frequencies utils/rope.py:7-23).
//
// Caches [B, Hkv, S, D] bf16; D = 128; G <= 4 query heads per key-value head.
// A round covers 512 cached positions, 64 per wave; every wave issues all of
// its key and value loads (256 B per lane each) before computing, so a round
// is one memory round trip (at context 512 the whole context is one round,
// and the caller may issue it before the new token's q, k, v exist).
//  - Scores: v_mfma_f32_16x16x32_bf16, the G rotated query rows (head g at
//    row 4 g, the other rows zero) against 16 cached key rows per MFMA (keys
//    contiguous along D, the contraction, so the B operands load straight
//    from the cache).  Row 4 g of the result lies in lane group g, so lane
//    16 g + j holds head g's score of position j of the block.
//  - Softmax: the running (online) form in fp32 per wave and head, every
//    head in its own lane group (one butterfly over 16 lanes serves all
//    heads).
//  - Probability-weighted values: MFMA as well.  The wave's value rows go
//    to LDS 32 at a time (rows padded by 8 bytes) and come back as B operands
//    (8 positions of one dimension per lane) through two transposing LDS
//    reads each; the probabilities enter as two bf16 parts, p = hi + lo,
//    which keeps them to ~16 bits.
//  - The waves' (max, sum, output) partials and the new position (rotated k,
//    v) merge in LDS in a fixed order.
#pragma once

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
constexpr int kAtVRows = 32;                     // value rows of a wave staged at once

struct AttnSmem {
  uint16_t in[kAtMaxG + 2][kAtD];                   // the new token's q rows, k row, v row (as produced)
  uint16_t q[kAtMaxG][kAtD];                        // rotated query rows
  uint16_t nw[2][kAtD];                             // the new k (rotated) and v rows
  float snew[kAtMaxG];                              // scores of the new position
  float ml[kAtWaves][kAtMaxG][2];                   // each wave's running max and sum
  uint16_t p[kAtWaves][2][kAtMaxG][kAtPosWave];     // probabilities hi, lo
  // 32 value rows of each wave; after the last round, each wave's
  // unnormalised output [G][D] fp32 (the LDS is reused)
  uint16_t v[kAtWaves][kAtVRows][kAtVPitch];
};
static_assert(sizeof(float) * kAtWaves * kAtMaxG * kAtD <= sizeof(uint16_t) * kAtWaves * kAtVRows * kAtVPitch,
              "output partials fit in the value buffer");

struct AttnPair {
  const float* rcos;  // [S, D/2] cos of position x frequency i
  const float* rsin;  // [S, D/2]
  uint16_t* kc;       // [B, Hkv, S, D]
  uint16_t* vc;
  int Hkv, G, S, b, hk, pos;
  float scale;
  int adjacent;  // 1: RoPE pairs (2i, 2i+1); 0: (i, i + D/2)
  // This thread's index in the workgroup.  A caller that runs the body inside
  // a longer loop passes an index the compiler cannot prove loop-invariant,
  // so that the per-lane offsets and masks derived from it are recomputed
  // (a few VALU operations) rather than held, or spilled, across the loop.
  int tid;
  __device__ __forceinline__ bool pos_ok() const { return pos >= 0 && pos < S; }
  __device__ __forceinline__ int nold() const { return pos_ok() ? pos : 0; }  // cached positions [0, nold)
  __device__ __forceinline__ int64_t kv_base() const { return ((int64_t)b * Hkv + hk) * S; }
};

// Rotates one pair (x0, x1) by the angle of frequency i at the position.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float& y0, float& y1) {
  y0 = x0 * c - x1 * s;
  y1 = x1 * c + x0 * s;
}

// Max and sum over each group of 16 lanes (an xor butterfly 8, 4, 2, 1:
// every lane of a group ends with its group's value).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, xor_partner<8>(v));
  v = fmaxf(v, xor_partner<4>(v));
  v = fmaxf(v, xor_partner<2>(v));
  v = fmaxf(v, xor_partner<1>(v));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v = v + xor_partner<8>(v);
  v = v + xor_partner<4>(v);
  v = v + xor_partner<2>(v);
  v = v + xor_partner<1>(v);
  return v;
}

__device__ __forceinline__ float wexp(float m, float M) { return m == -__builtin_inff() ? 0.0f : __expf(m - M); }

// ds_read_b64_tr_b16: in each group of 16 lanes, lane j receives, for
// r = 0..3, element j % 4 of the four 16-bit values that lane 4 r + j / 4
// addresses (measured on gfx950).  With lane 4 r + q addressing row r,
// columns 4 q .. 4 q + 3 of a row-major block, lane j gets column j of rows
// 0..3: a transposed 4 x 16 read.
typedef short v4s __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4s lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(__attribute__((address_space(3))) void*)p);
}

// A wave's key and value rows of round rd: K operands (4 blocks of 16
// positions x 4 k-steps) and value pieces (dims 8 r16 .. + 8 of row 4 t + grp).
struct AttnRound {
  uint4 kr[4][kAtD / 32];
  uint4 vr[16];
  float rc, rs;  // this thread's RoPE factors at the position (loaded with the first round)
};

// Buffer loads: the pair's rows [S][D] of a cache as one resource, so every
// load takes a 32-bit lane offset and an immediate (the k-steps and the value
// row groups), not a 64-bit address per load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t att_rows(const uint16_t* c, const AttnPair& a) {
  // the pair's base is the same in every lane: one scalar descriptor, no
  // per-lane (waterfall) resource loop around each load
  const uint64_t base = reinterpret_cast<uint64_t>(c + a.kv_base() * kAtD);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                           __builtin_amdgcn_readfirstlane(a.S * kAtD * 2), 0x00020000);
}
__device__ __forceinline__ uint4 att_ld(__amdgpu_buffer_rsrc_t r, int voff, int imm) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + imm, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ void att_load_round(const AttnPair& a, int rd, AttnRound& r) {
  const int lane = a.tid & 63, wv = __builtin_amdgcn_readfirstlane(a.tid >> 6);
  if (rd == 0) {  // the RoPE factors of frequency tid & 63 at the position, with the first round
    const int i = a.tid & (kAtD / 2 - 1), pc = a.pos_ok() ? a.pos : 0;
    r.rc = a.rcos[pc * (kAtD / 2) + i];
    r.rs = a.rsin[pc * (kAtD / 2) + i];
  }
  const int r16 = lane & 15, grp = lane >> 4;
  const int base = rd * kAtRound + kAtPosWave * wv;
  const __amdgpu_buffer_rsrc_t kc = att_rows(a.kc, a), vc = att_rows(a.vc, a);
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    const int row = min(base + 16 * blk + r16, a.S - 1);
    const int off = (row * kAtD + 8 * grp) * 2;
#pragma unroll
    for (int ks = 0; ks < kAtD / 32; ++ks) r.kr[blk][ks] = att_ld(kc, off, 64 * ks);
  }
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int row = min(base + 4 * t + grp, a.S - 1);
    r.vr[t] = att_ld(vc, (row * kAtD + 8 * r16) * 2, 0);
  }
}

// Everything after the first round's loads (att_load_round(a, 0, r), issued
// by the caller in every wave): RoPE of the group's query rows
// and the new k row (the new rows go to LDS and to the caches), scores,
// online softmax, probability-weighted values, merge.  s.in holds the new
// token's rows (q rows 0..G-1, k at kAtMaxG, v at kAtMaxG + 1) and every
// thread has passed a barrier since they were written.  Returns, for
// threads tid < G D (head tid / D, dimension tid % D), the bf16 output
// (zero for a position outside [0, S)); the other threads return 0.  Ends
// with every LDS access of the body complete (the caller may reuse s after
// a barrier).
// Measurement builds (-DBTL_TRACE) stamp events 3-6 (RoPE done, first
// round's softmax done, its values done, merge barriers passed) when trace is set.
__device__ __forceinline__ uint16_t att_body(const AttnPair& a, AttnSmem& s, AttnRound& r, bool trace = false) {
  const int tid = a.tid, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.G;
  const bool pos_ok = a.pos_ok();
  const int nold = a.nold();
  const int nrounds = (nold + kAtRound - 1) / kAtRound;
  const int64_t kvb = a.kv_base();
  const int half = kAtD / 2;
  const int r16 = lane & 15, grp = lane >> 4;
  {
    const int i = tid & (half - 1);
    const int d0 = a.adjacent ? 2 * i : i, d1 = a.adjacent ? 2 * i + 1 : i + half;
    const float rc = r.rc, rs = r.rs;
    const int u = tid / half;  // 0..7: query rows 0..3, then the k row, then v
    if (u < kAtMaxG) {
      float y0 = 0.0f, y1 = 0.0f;
      if (u < G && pos_ok) rope_pair(bf2f(s.in[u][d0]), bf2f(s.in[u][d1]), rc, rs, y0, y1);
      s.q[u][d0] = f2bf(y0);
      s.q[u][d1] = f2bf(y1);
    } else if (u == kAtMaxG) {
      float y0, y1;
      rope_pair(bf2f(s.in[kAtMaxG][d0]), bf2f(s.in[kAtMaxG][d1]), rc, rs, y0, y1);
      const uint16_t k0 = f2bf(y0), k1 = f2bf(y1);
      s.nw[0][d0] = k0;
      s.nw[0][d1] = k1;
      if (pos_ok) {
        uint16_t* dst = a.kc + (kvb + a.pos) * kAtD;
        dst[d0] = k0;
        dst[d1] = k1;
      }
    } else if (u == kAtMaxG + 1) {
      const int d = 2 * i;
      const uint32_t vnew = *reinterpret_cast<const uint32_t*>(&s.in[kAtMaxG + 1][d]);
      *reinterpret_cast<uint32_t*>(&s.nw[1][d]) = vnew;
      if (pos_ok) *reinterpret_cast<uint32_t*>(a.vc + (kvb + a.pos) * kAtD + d) = vnew;
    }
  }
  lds_barrier();  // the rotated rows are in LDS (the cache-row stores need no acknowledgement)
  if (trace) BTL_TRACE_AT(3);
  if (wv < G) {  // score of the new position for head wv (lanes over D, fixed-order sum)
    const float d = bf2f(s.q[wv][2 * lane]) * bf2f(s.nw[0][2 * lane]) +
                    bf2f(s.q[wv][2 * lane + 1]) * bf2f(s.nw[0][2 * lane + 1]);
    const float sn = wave_xor_sum(d) * a.scale;
    if (lane == 0) s.snew[wv] = sn;
  }
  // query operands (A: row 4 g = head g, k-step ks: dims 32 ks + 8 grp ..)
  const bool qrow = (r16 & 3) == 0 && (r16 >> 2) < G;
  v8bf qa[kAtD / 32];
#pragma unroll
  for (int ks = 0; ks < kAtD / 32; ++ks) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (qrow) v = *reinterpret_cast<const uint4*>(&s.q[r16 >> 2][32 * ks + 8 * grp]);
    qa[ks] = __builtin_bit_cast(v8bf, v);
  }

  // running softmax state of this wave for head gh = lane group (lanes
  // 16 gh + j; element 0 of the output accumulator o[m] is head gh,
  // dimension 16 m + j)
  const int gh = grp, j16 = r16;
  float mrun = -__builtin_inff(), lrun = 0.0f;
  v4f o[kAtD / 16];
#pragma unroll
  for (int m = 0; m < kAtD / 16; ++m) o[m] = (v4f){0.f, 0.f, 0.f, 0.f};

  for (int rd = 0; rd < nrounds; ++rd) {
    const int base = rd * kAtRound + kAtPosWave * wv;
    if (base >= nold) break;  // wave-uniform: nothing cached from here on
    if (rd > 0) att_load_round(a, rd, r);
    // scores: 4 blocks of 16 positions
    v4f sc[4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      sc[blk] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kAtD / 32; ++ks)
        sc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], __builtin_bit_cast(v8bf, r.kr[blk][ks]), sc[blk], 0,
                                                          0, 0);
    }
    // online softmax of head gh over the wave's 64 positions (lane
    // 16 gh + j: block blk's position 16 blk + j)
    {
      float s4[4];
      float mx = -__builtin_inff();
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const bool ok = gh < G && base + 16 * blk + j16 < nold;
        s4[blk] = ok ? sc[blk][0] * a.scale : -__builtin_inff();
        mx = fmaxf(mx, s4[blk]);
      }
      mx = row16_max(mx);
      const float mn = fmaxf(mrun, mx);
      const float alpha = wexp(mrun, mn);
      float sm = 0.0f;
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const float e = wexp(s4[blk], mn);
        sm += e;
        if (gh < G) {
          const uint16_t hi = f2bf(e);
          s.p[wv][0][gh][16 * blk + j16] = hi;
          s.p[wv][1][gh][16 * blk + j16] = f2bf(e - bf2f(hi));
        }
      }
      sm = row16_sum(sm);
      lrun = lrun * alpha + sm;
      mrun = mn;
#pragma unroll
      for (int m = 0; m < kAtD / 16; ++m) o[m][0] *= alpha;
    }
    if (rd == 0 && trace) BTL_TRACE_AT(4);
    // probability-weighted values: 2 k-steps of 32 positions x 8 column
    // blocks of 16 dimensions, probabilities as hi + lo parts; each k-step's
    // 32 value rows staged in LDS just before it (rows past the context as
    // zeros, whatever the cache holds there: a zero probability times a
    // non-finite value is NaN)
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int tt = 8 * k2 + t;
        const bool ok = base + 4 * tt + grp < nold;
        const uint4 v = ok ? r.vr[tt] : make_uint4(0u, 0u, 0u, 0u);
        uint2* dst = reinterpret_cast<uint2*>(&s.v[wv][4 * t + grp][8 * r16]);
        dst[0] = make_uint2(v.x, v.y);
        dst[1] = make_uint2(v.z, v.w);
      }
      __builtin_amdgcn_wave_barrier();  // the wave's own LDS writes are read back by other lanes
      v8bf pa[2];
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (qrow) v = *reinterpret_cast<const uint4*>(&s.p[wv][part][r16 >> 2][32 * k2 + 8 * grp]);
        pa[part] = __builtin_bit_cast(v8bf, v);
      }
#pragma unroll
      for (int m = 0; m < kAtD / 16; ++m) {
        // B operand: dimension 16 m + r16 of positions 32 k2 + 8 grp + [0, 8):
        // lane 4 r + q of the group reads row 8 grp + 4 h + r, dimensions
        // 16 m + 4 q .. + 3, for the halves h = 0, 1
        const int rr = r16 >> 2, qq = r16 & 3;
        const v4s lo = lds_read_tr16(&s.v[wv][8 * grp + rr][16 * m + 4 * qq]);
        const v4s hi = lds_read_tr16(&s.v[wv][8 * grp + 4 + rr][16 * m + 4 * qq]);
        typedef short v8s __attribute__((ext_vector_type(8)));
        const v8bf vb = __builtin_bit_cast(v8bf, (v8s){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w});
        o[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[0], vb, o[m], 0, 0, 0);
        o[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[1], vb, o[m], 0, 0, 0);
      }
      __builtin_amdgcn_wave_barrier();  // reads done before the buffers are rewritten
    }
  }

  // merge: every wave's partial, then the new position, in a fixed order
  if (j16 == 0) {
    s.ml[wv][gh][0] = mrun;
    s.ml[wv][gh][1] = lrun;
  }
  if (trace) BTL_TRACE_AT(5);
  lds_barrier();  // every wave is done with its value rows: the output partials reuse them
  float(*s_o)[kAtMaxG][kAtD] = reinterpret_cast<float(*)[kAtMaxG][kAtD]>(&s.v[0][0][0]);
  if (gh < G) {
#pragma unroll
    for (int m = 0; m < kAtD / 16; ++m) s_o[wv][gh][16 * m + j16] = o[m][0];
  }
  lds_barrier();
  if (trace) BTL_TRACE_AT(6);
  uint16_t res = 0;
  {
    const int g = tid / kAtD, d = tid % kAtD;  // 512 threads: 4 heads x 128 dims
    if (g < G) {
      const float snew = s.snew[g];
      float M = snew;
#pragma unroll
      for (int w = 0; w < kAtWaves; ++w) M = fmaxf(M, s.ml[w][g][0]);
      const float wn = __expf(snew - M);
      float L = wn;
      float O = wn * bf2f(s.nw[1][d]);
#pragma unroll
      for (int w = 0; w < kAtWaves; ++w) {
        const float ww = wexp(s.ml[w][g][0], M);
        L += ww * s.ml[w][g][1];
        O += ww * s_o[w][g][d];
      }
      const float inv = pos_ok ? 1.0f / L : 0.0f;
      res = f2bf(O * inv);
    }
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this thread's LDS reads are done
  return res;
}

}  // namespace btl
