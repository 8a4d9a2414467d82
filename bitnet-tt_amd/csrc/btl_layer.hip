// Persistent decode layer of a BitNet b1.58 model on gfx950: one launch runs
// every BitLinear from a layer's o_proj to the next layer's QKV.
//
// Per layer the reference decode loop (src/bitnet_tt/inference/
// generator_batch32.py:713-761) issues QKV -> attention -> o_proj (+residual)
// -> gate||up -> relu^2*up -> down (+residual).  Attention stays outside; the
// BitLinear work between two attentions runs here as one launch of
// one-workgroup-per-CU persistent kernel, in eight phases:
//
//   row 0   attn row m -> RMSNorm(attn_sub_norm) -> int8 row of xa[o]     WG m
//   o_proj  int32 partial sums over K slices                               all WGs
//   row 1   hidden[m] += bf16(sum * s * a); RMSNorm(post_attention) -> xa[gu]
//   gate_up relu(g)^2 * u -> ffn_h                                         all WGs
//   row 2   ffn_h row m -> RMSNorm(ffn_sub_norm) -> xa[down]
//   down    int32 partial sums over K slices
//   row 3   hidden[m] += bf16(sum * s * a); RMSNorm(next input_layernorm) -> xa[qkv]
//   qkv     qkv_out = bf16(acc * s_seg * a)                                (next layer)
//
// Arithmetic is exactly that of btl_bitlinear_fused (same row code, same
// epilogue expressions), so a layer launch is bit-identical to its four
// single-BitLinear launches.
//
// Each workgroup owns one unit (column tile or gate/up tile pair x K slice) of
// every BitLinear and loads the weights of all its units into registers at
// the start (each wave its own superblocks), so the 17 MB of a layer stream in
// while the first row phase runs, and every later phase only waits for data
// produced inside the launch.  Each workgroup keeps its own launch counter
// (the epoch); every hand-off carries a tag made of it and the BitLinear's
// index, so nothing ever needs clearing.  Two hand-offs per BitLinear:
//
//   row -> GEMM (the int8 tile, read by every GEMM workgroup): the row block
//     writes its row with device-coherent stores, waits for them, then sets
//     its row flag; GEMM workgroups poll the 32 flags and read the tile with
//     plain loads (it is written once per launch and read only after the
//     flags, and caches start clean at every kernel boundary), so each XCD's
//     L2 fetches it once.
//   GEMM -> row, relu^2*up values (27 KB per row): every 8-byte word carries
//     two bf16 and the 4-byte tag and is written with one device-coherent
//     store; the row block polls the words themselves.  The producer never
//     waits and there is no separate flag.
//   GEMM -> row, split-K partial sums of o_proj / down (sk x 10 KB per row,
//     too much to poll): coherent stores, wait, one done flag per workgroup;
//     the row block polls the flags, then reads its row with plain loads.
//
// Waits are bounded: a timeout sets the error word and the phase goes on, so
// every wave always exits.
#include "btl_act_row.h"
#include "btl_mfma.h"

namespace btl {

constexpr int kLayerWaves = 8;
constexpr int kLayerNSW = 3;        // superblocks per wave and BitLinear held in registers
constexpr int kLayerMaxSplit = 4;   // K slices of o_proj / down
constexpr int kLayerMaxGrid = 1024;
enum { L_O = 0, L_GU = 1, L_DOWN = 2, L_QKV = 3, kLayerOps = 4 };
enum { MODE_PART = 0, MODE_SCALE = 1, MODE_RELU2 = 2 };

// Workspace header (bytes): row flags, error word, done flags, per-workgroup epochs.
constexpr int64_t kLyRowFlag = 0;                                  // [4][32] words
constexpr int64_t kLyError = 1024;                                 // one word
constexpr int64_t kLyDoneFlag = 4096;                              // [4][kLayerMaxGrid] words
constexpr int64_t kLyEpoch = kLyDoneFlag + 4 * 4 * kLayerMaxGrid;  // [kLayerMaxGrid] words
constexpr int64_t kLyHeader = 65536;

struct LayerOp {
  const uint32_t* wdev;
  int K, KS, N, NT;
  int tpw, sk, ngroups, units;
  float seg_scale[BTL_MAX_SEGMENTS];
  int seg_end[BTL_MAX_SEGMENTS];
  int nseg;
  const uint16_t* gamma;  // RMSNorm gain of this BitLinear's input
  int8_t* xa;             // quantised input, MFMA A layout
  float* a_dq;            // [32] per-row dequantisation a/127
  int32_t* part;          // MODE_PART: [sk][32][N] partial sums
  uint64_t* ll;           // MODE_RELU2: [32][N/4] tagged bf16 pairs
  uint16_t* out;          // bf16 output (MODE_SCALE / MODE_RELU2)
};

struct LayerArgs {
  LayerOp op[kLayerOps];
  int nops;  // 4: with the next layer's QKV; 3: last layer
  int M;
  float eps;
  const uint16_t* attn;  // [M][K of o_proj]
  uint16_t* hidden;      // [M][H] residual stream, updated in place
  uint32_t* row_flag;    // [4][32]
  uint32_t* done_flag;   // [4][kLayerMaxGrid]
  uint32_t* epoch;       // [kLayerMaxGrid]
  uint32_t* error;
  unsigned spin_limit;
};

__device__ __forceinline__ float seg_scale_at(const LayerOp& op, int n) {
  float s = op.seg_scale[0];
#pragma unroll
  for (int i = 0; i + 1 < BTL_MAX_SEGMENTS; ++i)
    if (i + 1 < op.nseg && n >= op.seg_end[i]) s = op.seg_scale[i + 1];
  return s;
}

// Wave 0 polls words[0..n) until all equal `want`; then the whole block
// passes a barrier.
__device__ void wait_flags(const uint32_t* words, int n, uint32_t want, const LayerArgs& p) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    unsigned spins = 0;
    for (;;) {
      bool mine = true;
      for (int i = tid; i < n; i += 64) mine = mine & (ld_coherent(words + i) == want);
      if (__all(mine)) break;
      if (++spins > p.spin_limit) {
        if (tid == 0) st_coherent(p.error, 1u);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
}

// Unit of workgroup b in `op` (workgroups past the last unit alias unit 0 so
// their weight loads stay in bounds; they do no GEMM work).
struct Unit {
  int g, s, sb0, sb1;
};
__device__ __forceinline__ Unit unit_of(const LayerOp& op, int b) {
  const int u = b < op.units ? b : 0;
  Unit r;
  r.g = u % op.ngroups;
  r.s = u / op.ngroups;
  r.sb0 = r.s * op.KS / op.sk;
  r.sb1 = (r.s + 1) * op.KS / op.sk;
  return r;
}
__device__ __forceinline__ int unit_tile(const LayerOp& op, const Unit& u, int t) {
  return t == 0 ? u.g : u.g + (op.NT >> 1);  // relu2: gate tile g pairs with up tile g + F/32
}

// Weights of this wave's superblocks sb0 + wv + 8i.  Always kLayerNSW loads
// per tile (a slot past the slice re-reads its last superblock), so the
// number of loads in flight is fixed at compile time and later waits on other
// loads do not have to drain the weight stream.
template <int TPW>
__device__ __forceinline__ void load_weights(const LayerOp& op, int b, int wv, int lane, v4i (&w)[TPW][kLayerNSW]) {
  const Unit u = unit_of(op, b);
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int tile = unit_tile(op, u, t);
#pragma unroll
    for (int i = 0; i < kLayerNSW; ++i) {
      int sb = u.sb0 + wv + kLayerWaves * i;
      sb = sb < u.sb1 ? sb : u.sb1 - 1;
      w[t][i] = ld128(op.wdev + (((int64_t)tile * op.KS + sb) * 64 + lane) * 4);
    }
  }
}

__device__ __forceinline__ uint64_t tagged(uint32_t tag, uint32_t v) { return ((uint64_t)tag << 32) | v; }

// One BitLinear's GEMM phase on workgroup b: wait for the M row flags of the
// op, MFMA over this wave's superblocks, reduce the waves in LDS, subtract the
// K slice's row sums, then write the partial sums (and the done flag `done`)
// or the epilogue.
template <int TPW, int MODE>
__device__ void layer_gemm(const LayerArgs& p, const LayerOp& op, const v4i (&w)[TPW][kLayerNSW],
                           const uint32_t* flags, uint32_t want, uint32_t* done, int32_t* red,
                           int32_t (*red_rs)[32]) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, b = blockIdx.x;
  if (b >= op.units) return;
  wait_flags(flags, p.M, want, p);
  const Unit u = unit_of(op, b);
  int tile[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) tile[t] = unit_tile(op, u, t);

  v4i a[kLayerNSW][4];
#pragma unroll
  for (int i = 0; i < kLayerNSW; ++i) {
    const int sb = u.sb0 + wv + kLayerWaves * i;
    if (sb < u.sb1) {
#pragma unroll
      for (int q = 0; q < 4; ++q) a[i][q] = ld128(op.xa + ((sb * 4 + q) * 64 + lane) * 16);
    }
  }
  v16i acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  int32_t rs_lane = 0;
#pragma unroll
  for (int i = 0; i < kLayerNSW; ++i) {
    if (u.sb0 + wv + kLayerWaves * i < u.sb1) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int t = 0; t < TPW; ++t)
          acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i][q], unpack_b((uint32_t)w[t][i][q]), acc[t], 0, 0, 0);
        rs_lane = bytes_sum(a[i][q], rs_lane);
      }
    }
  }
  {
    const int32_t rs_row = rs_lane + (int32_t)xor_partner_u<32>((uint32_t)rs_lane);
    if (lane < 32) red_rs[wv][lane] = rs_row;
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[((wv * TPW + t) * 16 + r) * 64 + lane] = acc[t][r];
  __syncthreads();

  // Thread (wv, lane) finishes accumulator rows r = wv and wv + 8 of each tile.
  const int jc = lane & 31;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int r = wv + kLayerWaves * rr;
    const int i = acc_row(r, lane);
    int32_t rs = 0;
#pragma unroll
    for (int w2 = 0; w2 < kLayerWaves; ++w2) rs += red_rs[w2][i];
    int32_t v[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      int32_t sum = -rs;
#pragma unroll
      for (int w2 = 0; w2 < kLayerWaves; ++w2) sum += red[((w2 * TPW + t) * 16 + r) * 64 + lane];
      v[t] = sum;
    }
    if (MODE == MODE_PART) {
      if (i < p.M) {
#pragma unroll
        for (int t = 0; t < TPW; ++t) st_coherent(op.part + ((int64_t)u.s * 32 + i) * op.N + tile[t] * 32 + jc, v[t]);
      }
    } else if (MODE == MODE_RELU2) {
      const float ad = op.a_dq[i];
      const int ng = tile[0] * 32 + jc, nu = tile[1] * 32 + jc;
      const float gg = bf2f(f2bf((float)v[0] * (seg_scale_at(op, ng) * ad)));
      const float uu = bf2f(f2bf((float)v[1] * (seg_scale_at(op, nu) * ad)));
      const float gr = gg > 0.0f ? gg : 0.0f;
      const float sq = bf2f(f2bf(gr * gr));
      const uint32_t h = f2bf(sq * uu);
      // lanes jc, jc+1 hold the same row: the even lane stores both columns
      const uint32_t pair = h | (__shfl_down(h, 1, 64) << 16);
      if (i < p.M && (jc & 1) == 0) {
        *reinterpret_cast<uint32_t*>(op.out + (int64_t)i * (op.N >> 1) + ng) = pair;
        st_coherent(op.ll + (int64_t)i * (op.N >> 2) + (ng >> 1), tagged(want, pair));
      }
    } else {
      if (i < p.M) {
        const float ad = op.a_dq[i];
        const int n = tile[0] * 32 + jc;
        op.out[(int64_t)i * op.N + n] = f2bf((float)v[0] * (seg_scale_at(op, n) * ad));
      }
    }
  }
  if (MODE == MODE_PART) {
    wait_memory();
    __syncthreads();
    if (tid == 0) st_coherent(done + b, want);
  }
}

// Row phase tail: RMSNorm with the op's gain, absmax int8 quantisation into
// the op's xa, a_dq; then the row's flag.  Returns a/127 of the row.
template <int CPT>
__device__ float row_publish(const LayerArgs& p, const LayerOp& op, float (&v)[CPT][8], const uint4 (&graw)[CPT],
                             int m, uint32_t* flag, uint32_t want, float* s_sum, float* s_max) {
  const int tid = threadIdx.x;
  const int nch = op.K >> 3, nchp = op.KS * 16;
  const float r = row_rms_inv<CPT>(v, nch, op.K, p.eps, tid, s_sum);
  row_apply_norm<CPT>(v, graw, true, r, nch, tid);
  const float a = row_absmax<CPT>(v, nch, 1e-5f, tid, s_max);
  const float scale = 127.0f / a;
  const float ad = a / 127.0f;
  if (tid == 0) st_coherent(op.a_dq + m, ad);
  int rs = 0;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    if (tid < kActThreads && c < nch) {
      uint32_t lo, hi;
      quant8(v[i], scale, lo, hi, rs);
      store_chunk<true>(op.xa, m, c, op.KS, lo, hi);
    }
  }
  if (tid < kActThreads) {
    for (int c = nch + tid; c < nchp; c += kActThreads) store8<true>(op.xa + xa_offset(m, 8 * c, op.KS), 0u, 0u);
    wait_memory();  // only the row waves stored; the others may still have weight loads in flight
  }
  __syncthreads();
  if (tid == 0) st_coherent(flag, want);
  return ad;
}

// Polls the tagged words of one 8-element chunk: n8 groups of 8 words (one
// per K slice) are summed; returns when every tag equals `want` (or the spin
// limit is reached, which sets the error word).
__device__ __forceinline__ bool tags_ok(uint64_t d, uint32_t want) { return (uint32_t)(d >> 32) == want; }

// Loads 8-element chunks tid + 256i of a bf16 row into v, and the matching
// chunks of gamma.
template <int CPT>
__device__ __forceinline__ void load_row(const uint16_t* x, const uint16_t* gamma, int nch, float (&v)[CPT][8],
                                         uint4 (&graw)[CPT]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    graw[i] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < kActThreads && c < nch) graw[i] = *reinterpret_cast<const uint4*>(gamma + 8 * c);
  }
  // all loads are issued before the first conversion waits for one
  uint4 raw[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    raw[i] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < kActThreads && c < nch) raw[i] = *reinterpret_cast<const uint4*>(x + 8 * c);
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
}

// Residual epilogue of o_proj / down for row m: v = bf16(hid + bf16(sum_s part *
// (s_seg * ad))); hid and the hidden row in memory take the new values.  The
// caller has waited for the op's done flags.
template <int CPT>
__device__ __forceinline__ void row_residual(const LayerArgs& p, const LayerOp& op, int m, float ad,
                                             uint32_t (&hid)[CPT][4], float (&v)[CPT][8]) {
  const int tid = threadIdx.x;
  const int nch = op.N >> 3;
  // every slice's loads are in flight before the first add
  int4 raw[CPT][kLayerMaxSplit][2];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
#pragma unroll
    for (int s = 0; s < kLayerMaxSplit; ++s) {
      raw[i][s][0] = make_int4(0, 0, 0, 0);
      raw[i][s][1] = make_int4(0, 0, 0, 0);
      if (tid < kActThreads && c < nch && s < op.sk) {
        const int32_t* src = op.part + ((int64_t)s * 32 + m) * op.N + 8 * c;
        raw[i][s][0] = *reinterpret_cast<const int4*>(src);
        raw[i][s][1] = *reinterpret_cast<const int4*>(src + 4);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    if (tid < kActThreads && c < nch) {
      int32_t acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < kLayerMaxSplit; ++s) {
        acc[0] += raw[i][s][0].x;
        acc[1] += raw[i][s][0].y;
        acc[2] += raw[i][s][0].z;
        acc[3] += raw[i][s][0].w;
        acc[4] += raw[i][s][1].x;
        acc[5] += raw[i][s][1].y;
        acc[6] += raw[i][s][1].z;
        acc[7] += raw[i][s][1].w;
      }
      uint32_t o4[4];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int n = 8 * c + j;
        const uint16_t o = f2bf((float)acc[j] * (seg_scale_at(op, n) * ad));
        const uint16_t r = (uint16_t)((j & 1) ? (hid[i][j >> 1] >> 16) : (hid[i][j >> 1] & 0xffffu));
        const uint16_t h = f2bf(bf2f(r) + bf2f(o));
        v[i][j] = bf2f(h);
        if (j & 1)
          o4[j >> 1] |= (uint32_t)h << 16;
        else
          o4[j >> 1] = h;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) hid[i][j] = o4[j];
      *reinterpret_cast<uint4*>(p.hidden + (int64_t)m * op.N + 8 * c) = make_uint4(o4[0], o4[1], o4[2], o4[3]);
    }
  }
}

// Row m of the relu^2*up output from its tagged words (two bf16 per word).
template <int CPT>
__device__ __forceinline__ void load_row_tagged(const LayerArgs& p, const uint64_t* src, int nch, uint32_t want,
                                                float (&v)[CPT][8]) {
  const int tid = threadIdx.x;
  uint32_t pr[CPT][4];
  unsigned spins = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + kActThreads * i;
#pragma unroll
      for (int j = 0; j < 4; ++j) pr[i][j] = 0u;
      if (tid < kActThreads && c < nch) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint64_t d = ld_coherent(src + 4 * c + j);
          ok = ok & tags_ok(d, want);
          pr[i][j] = (uint32_t)d;
        }
      }
    }
    if (ok) break;
    if (++spins > p.spin_limit) {
      st_coherent(p.error, 1u);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[i][2 * j] = bf2f((uint16_t)(pr[i][j] & 0xffffu));
      v[i][2 * j + 1] = bf2f((uint16_t)(pr[i][j] >> 16));
    }
}

// Gain chunks tid + 256i of a row of K (zero past K).
template <int CPT>
__device__ __forceinline__ void load_gamma(const uint16_t* gamma, int nch, uint4 (&graw)[CPT]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + kActThreads * i;
    graw[i] = make_uint4(0u, 0u, 0u, 0u);
    if (gamma && tid < kActThreads && c < nch) graw[i] = *reinterpret_cast<const uint4*>(gamma + 8 * c);
  }
}

// CQ / CH / CF: 8-element chunks per thread of rows of the attention output,
// the hidden state and the FFN intermediate.
template <int CQ, int CH, int CF>
__global__ __launch_bounds__(512) void k_decode_layer(LayerArgs p) {
  __shared__ int32_t red[kLayerWaves * 2 * 16 * 64];
  __shared__ int32_t red_rs[kLayerWaves][32];
  __shared__ float s_sum[kActWaves];
  __shared__ float s_max[kActWaves];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, b = blockIdx.x;
  const uint32_t E = p.epoch[b];
  const bool row_block = b < p.M;
  const int m = b;
  const LayerOp& o = p.op[L_O];
  const LayerOp& gu = p.op[L_GU];
  const LayerOp& dn = p.op[L_DOWN];
  const LayerOp& qk = p.op[L_QKV];

  // Row phase 0 inputs and the gains of all row phases first, so they are
  // ahead of the weight stream.
  float v0[CQ][8];
  uint4 g0[CQ], g1[CH], g2[CF], g3[CH];
  uint32_t hid[CH][4];
  if (row_block) {
    load_row<CQ>(p.attn + (int64_t)m * o.K, o.gamma, o.K >> 3, v0, g0);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + kActThreads * i;
      if (tid < kActThreads && c < (o.N >> 3)) {
        const uint4 raw = *reinterpret_cast<const uint4*>(p.hidden + (int64_t)m * o.N + 8 * c);
        hid[i][0] = raw.x;
        hid[i][1] = raw.y;
        hid[i][2] = raw.z;
        hid[i][3] = raw.w;
      }
    }
    load_gamma<CH>(gu.gamma, gu.K >> 3, g1);
    load_gamma<CF>(dn.gamma, dn.K >> 3, g2);
    load_gamma<CH>(p.nops == 4 ? qk.gamma : nullptr, qk.K >> 3, g3);
  }
  // The row waves of a row block load their weights after publishing row 0
  // (their stores' wait would otherwise also wait for the weight stream).
  const bool defer = row_block && tid < kActThreads;
  v4i w_o[1][kLayerNSW], w_gu[2][kLayerNSW], w_dn[1][kLayerNSW], w_q[1][kLayerNSW];
  auto load_all = [&]() {
    load_weights<1>(o, b, wv, lane, w_o);
    load_weights<2>(gu, b, wv, lane, w_gu);
    load_weights<1>(dn, b, wv, lane, w_dn);
    load_weights<1>(qk, b, wv, lane, w_q);  // the host aliases o_proj here on the last layer
  };
  if (!defer) load_all();

  uint32_t* const rf = p.row_flag;
  uint32_t* const df = p.done_flag;
  auto want = [&](int j) { return (E << 3) | (uint32_t)(j + 1); };

  float ad = 0.0f;
  if (row_block) ad = row_publish<CQ>(p, o, v0, g0, m, rf + L_O * 32 + m, want(L_O), s_sum, s_max);
  if (defer) load_all();
  layer_gemm<1, MODE_PART>(p, o, w_o, rf + L_O * 32, want(L_O), df + L_O * kLayerMaxGrid, red, red_rs);

  if (row_block) {
    wait_flags(df + L_O * kLayerMaxGrid, o.units, want(L_O), p);
    float v1[CH][8];
    row_residual<CH>(p, o, m, ad, hid, v1);
    ad = row_publish<CH>(p, gu, v1, g1, m, rf + L_GU * 32 + m, want(L_GU), s_sum, s_max);
  }
  layer_gemm<2, MODE_RELU2>(p, gu, w_gu, rf + L_GU * 32, want(L_GU), nullptr, red, red_rs);

  if (row_block) {
    float v2[CF][8];
    load_row_tagged<CF>(p, gu.ll + (int64_t)m * (gu.N >> 2), dn.K >> 3, want(L_GU), v2);
    ad = row_publish<CF>(p, dn, v2, g2, m, rf + L_DOWN * 32 + m, want(L_DOWN), s_sum, s_max);
  }
  layer_gemm<1, MODE_PART>(p, dn, w_dn, rf + L_DOWN * 32, want(L_DOWN), df + L_DOWN * kLayerMaxGrid, red, red_rs);

  if (row_block) {
    wait_flags(df + L_DOWN * kLayerMaxGrid, dn.units, want(L_DOWN), p);
    float v3[CH][8];
    row_residual<CH>(p, dn, m, ad, hid, v3);
    if (p.nops == 4) row_publish<CH>(p, qk, v3, g3, m, rf + L_QKV * 32 + m, want(L_QKV), s_sum, s_max);
  }
  if (p.nops == 4) layer_gemm<1, MODE_SCALE>(p, qk, w_q, rf + L_QKV * 32, want(L_QKV), nullptr, red, red_rs);

  if (tid == 0) p.epoch[b] = E + 1;
}

// ---------------------------------------------------------------- host ----
static int layer_grid() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

struct LayerSizes {
  int64_t xa[kLayerOps], a_dq[kLayerOps], part_o, ll_gu, part_dn, total;
};

static LayerSizes layer_sizes(int64_t H, int64_t Q, int64_t F, int64_t NQKV) {
  LayerSizes z;
  const int64_t Ks[kLayerOps] = {Q, H, F, H};
  int64_t off = kLyHeader;
  for (int j = 0; j < kLayerOps; ++j) {
    z.xa[j] = off;
    off += round_up(32 * ksb(Ks[j]) * 128, 4096);
  }
  for (int j = 0; j < kLayerOps; ++j) {
    z.a_dq[j] = off;
    off += 256;
  }
  off = round_up(off, 4096);
  z.part_o = off;  // partial sums of o_proj: [kLayerMaxSplit][32][H]
  off += round_up((int64_t)kLayerMaxSplit * 32 * H * 4, 4096);
  z.ll_gu = off;  // tagged relu^2*up pairs: [32][F/2] words
  off += round_up((int64_t)32 * (F / 2) * 8, 4096);
  z.part_dn = off;  // partial sums of down
  off += round_up((int64_t)kLayerMaxSplit * 32 * H * 4, 4096);
  (void)NQKV;
  z.total = off;
  return z;
}

static int plan_op(LayerOp& op, const char* name, int64_t K, int64_t N, const btl_layer_weight_t* w, int mode,
                   int grid) {
  if (!w || !w->wdev) return set_error(BTL_ERR_NULL, "btl_decode_layer: %s weight is NULL", name);
  if (!w->gamma) return set_error(BTL_ERR_NULL, "btl_decode_layer: %s RMSNorm gain is NULL", name);
  if (!aligned(w->wdev, 16) || !aligned(w->gamma, 16))
    return set_error(BTL_ERR_ALIGN, "btl_decode_layer: %s weight / gain must be 16-byte aligned", name);
  if (w->nseg < 1 || w->nseg > BTL_MAX_SEGMENTS)
    return set_error(BTL_ERR_ARG, "btl_decode_layer: %s has %d segments", name, w->nseg);
  int64_t prev = 0;
  for (int i = 0; i < w->nseg; ++i) {
    if (w->seg_end[i] <= prev || w->seg_end[i] % 32)
      return set_error(BTL_ERR_ARG, "btl_decode_layer: %s segment ends must increase in multiples of 32", name);
    prev = w->seg_end[i];
  }
  if (prev != N) return set_error(BTL_ERR_ARG, "btl_decode_layer: %s last segment end %lld != N=%lld", name,
                                  (long long)prev, (long long)N);
  op.wdev = w->wdev;
  op.gamma = w->gamma;
  op.K = (int)K;
  op.KS = (int)ksb(K);
  op.N = (int)N;
  op.NT = (int)(N / 32);
  op.nseg = w->nseg;
  for (int i = 0; i < BTL_MAX_SEGMENTS; ++i) {
    op.seg_scale[i] = i < w->nseg ? w->seg_scale[i] : 0.0f;
    op.seg_end[i] = i < w->nseg ? (int)w->seg_end[i] : (int)N;
  }
  if (mode == MODE_RELU2) {
    op.tpw = 2;
    op.ngroups = op.NT / 2;
    op.sk = 1;
  } else {
    op.tpw = 1;
    op.ngroups = op.NT;
    op.sk = 1;
    if (mode == MODE_PART) {
      int sk = grid / op.ngroups;
      if (sk > kLayerMaxSplit) sk = kLayerMaxSplit;
      if (sk > op.KS) sk = op.KS;
      op.sk = sk < 1 ? 1 : sk;
    }
  }
  op.units = op.ngroups * op.sk;
  const int per_slice = (op.KS + op.sk - 1) / op.sk;
  if (op.units > grid || per_slice > kLayerWaves * kLayerNSW)
    return set_error(BTL_ERR_SHAPE,
                     "btl_decode_layer: %s (K=%lld, N=%lld) does not fit one workgroup per CU with weights in "
                     "registers (%d units, %d superblocks per slice)",
                     name, (long long)K, (long long)N, op.units, per_slice);
  return BTL_OK;
}

template <int CQ, int CH, int CF>
static void launch_layer(int grid, hipStream_t s, const LayerArgs& a) {
  hipLaunchKernelGGL((k_decode_layer<CQ, CH, CF>), dim3(grid), dim3(512), 0, s, a);
}

}  // namespace btl

using namespace btl;

extern "C" {

int64_t btl_decode_layer_workspace_bytes(int64_t M, int64_t H, int64_t Q, int64_t F, int64_t NQKV) {
  if (M <= 0 || M > 32 || H <= 0 || Q <= 0 || F <= 0 || NQKV < 0) return 0;
  return layer_sizes(H, Q, F, NQKV).total;
}

int64_t btl_decode_layer_error_offset(void) { return kLyError; }

int btl_decode_layer(int64_t M, int64_t H, int64_t Q, int64_t F, int64_t NQKV, const btl_layer_weight_t* o_proj,
                     const btl_layer_weight_t* gate_up, const btl_layer_weight_t* down,
                     const btl_layer_weight_t* next_qkv, float eps, const uint16_t* attn, uint16_t* hidden,
                     uint16_t* ffn_h, uint16_t* qkv_out, void* workspace, size_t workspace_bytes,
                     btl_stream_t stream) {
  clear_error();
  if (!attn || !hidden || !ffn_h || !workspace) return set_error(BTL_ERR_NULL, "btl_decode_layer: null pointer");
  if (next_qkv && !qkv_out) return set_error(BTL_ERR_NULL, "btl_decode_layer: next_qkv needs qkv_out");
  if (M <= 0 || M > 32) return set_error(BTL_ERR_SHAPE, "btl_decode_layer: M=%lld (1..32 decode rows)", (long long)M);
  if (H % 128 || Q % 128 || F % 128 || H > BTL_MAX_K || Q > BTL_MAX_K || F > BTL_MAX_K || (next_qkv && NQKV % 32) ||
      (next_qkv && NQKV <= 0))
    return set_error(BTL_ERR_SHAPE, "btl_decode_layer: H=%lld Q=%lld F=%lld must be multiples of 128 (<= %d), NQKV "
                     "a multiple of 32", (long long)H, (long long)Q, (long long)F, BTL_MAX_K);
  if (!aligned(attn, 16) || !aligned(hidden, 16) || !aligned(ffn_h, 16) || !aligned(workspace, 256) ||
      (qkv_out && !aligned(qkv_out, 4)))
    return set_error(BTL_ERR_ALIGN, "btl_decode_layer: buffers must be 16-byte aligned, workspace 256");
  const LayerSizes z = layer_sizes(H, Q, F, NQKV);
  if ((int64_t)workspace_bytes < z.total)
    return set_error(BTL_ERR_WORKSPACE, "btl_decode_layer: workspace %zu < %lld bytes", workspace_bytes,
                     (long long)z.total);
  const int cq = act_cpt(Q), ch = act_cpt(H), cf = act_cpt(F);
  // instances: small shapes, the 2B shapes (F = 6912), and K up to 16384
  const bool inst_small = cq == 1 && ch == 1 && cf == 1;
  const bool inst_2b = cq == 1 && ch == 1 && cf == 2;
  const bool inst_big = cq <= 2 && ch <= 2 && cf <= 4 && !inst_small && !inst_2b;
  if (!inst_small && !inst_2b && !inst_big)
    return set_error(BTL_ERR_SHAPE, "btl_decode_layer: no kernel instance for H=%lld Q=%lld F=%lld", (long long)H,
                     (long long)Q, (long long)F);
  const btl_layer_weight_t* ws_in[kLayerOps] = {o_proj, gate_up, down, next_qkv};
  const char* names[kLayerOps] = {"o_proj", "gate_up", "down", "next_qkv"};
  for (int j = 0; j < kLayerOps; ++j)
    if ((j < 3 || next_qkv) && (!ws_in[j] || !ws_in[j]->wdev || !ws_in[j]->gamma))
      return set_error(BTL_ERR_NULL, "btl_decode_layer: %s weight or RMSNorm gain is NULL", names[j]);
  const int grid = layer_grid();
  if (grid <= 0 || grid > kLayerMaxGrid) return set_error(BTL_ERR_LAUNCH, "btl_decode_layer: cannot size the grid");

  LayerArgs a = {};
  int rc = plan_op(a.op[L_O], "o_proj", Q, H, o_proj, MODE_PART, grid);
  if (!rc) rc = plan_op(a.op[L_GU], "gate_up", H, 2 * F, gate_up, MODE_RELU2, grid);
  if (!rc) rc = plan_op(a.op[L_DOWN], "down", F, H, down, MODE_PART, grid);
  if (!rc && next_qkv) rc = plan_op(a.op[L_QKV], "next_qkv", H, NQKV, next_qkv, MODE_SCALE, grid);
  if (rc) return rc;
  if (gate_up->nseg != 2 || gate_up->seg_end[0] != F)
    return set_error(BTL_ERR_ARG, "btl_decode_layer: gate_up needs two segments (gate | up) split at F");
  if (!next_qkv) {
    a.op[L_QKV] = a.op[L_O];  // weight loads stay in bounds; no QKV phase runs
    a.op[L_QKV].units = 0;
  }
  char* ws = (char*)workspace;
  for (int j = 0; j < kLayerOps; ++j) {
    a.op[j].xa = (int8_t*)(ws + z.xa[j]);
    a.op[j].a_dq = (float*)(ws + z.a_dq[j]);
    a.op[j].part = nullptr;
    a.op[j].ll = nullptr;
    a.op[j].out = nullptr;
  }
  a.op[L_O].part = (int32_t*)(ws + z.part_o);
  a.op[L_GU].ll = (uint64_t*)(ws + z.ll_gu);
  a.op[L_DOWN].part = (int32_t*)(ws + z.part_dn);
  a.op[L_GU].out = ffn_h;
  a.op[L_QKV].out = next_qkv ? qkv_out : nullptr;
  a.nops = next_qkv ? 4 : 3;
  a.M = (int)M;
  a.eps = eps;
  a.attn = attn;
  a.hidden = hidden;
  a.row_flag = (uint32_t*)(ws + kLyRowFlag);
  a.done_flag = (uint32_t*)(ws + kLyDoneFlag);
  a.error = (uint32_t*)(ws + kLyError);
  a.epoch = (uint32_t*)(ws + kLyEpoch);
  a.spin_limit = 1u << 17;
  hipStream_t s = (hipStream_t)stream;
  if (inst_2b)
    launch_layer<1, 1, 2>(grid, s, a);
  else if (inst_big)
    launch_layer<2, 2, 4>(grid, s, a);
  else
    launch_layer<1, 1, 1>(grid, s, a);
  return check_launch("decode layer");
}

}  // extern "C"
