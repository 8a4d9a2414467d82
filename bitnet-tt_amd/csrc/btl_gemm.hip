// Ternary GEMM of the BitLinear path on gfx950:
//   acc[m,n] = sum_k q[m,k] * w[k,n]   (int8 activations, ternary weights, int32)
// followed by the scale epilogue (or the gate||up relu^2*up epilogue).
//
// Weights arrive as offset codes u = w + 1 in {0,1,2}, 2 bits each, already
// in MFMA operand order, so unpacking a dword of 16 codes into the four B
// operand dwords is one shift and one AND each.  The int8 MFMA then computes
// sum_k q*u, and the exact accumulator is recovered as
//   acc = sum_k q*u - sum_k q
// with the row sum taken from the A operand in the same pass (v_dot4 of the
// operand bytes with 0x01010101; each K slice subtracts its own part), or,
// in prefill, from the row sums the activation kernel wrote when the caller
// passes them (the loop is then MFMAs and unpacking only).
// |acc| <= 128*2*16384 < 2^31, so every step is exact.
//
// Decode (M <= 32): the whole activation block is one 32-row MFMA operand.
// A workgroup (4 or 8 waves) owns TPW column tiles of 32 and a slice of the K
// superblocks; each wave takes its share of that slice, issues its weight
// loads and then its activation loads (1 KiB per wave per load: fully
// coalesced) before the first MFMA.  The wave partials meet in LDS.  When K
// is split across workgroups (split-K), each publishes its partial tile with
// coherent stores and the last to arrive (atomic counter) sums them and runs
// the epilogue -- no spinning, no float atomics, a deterministic result.
//
// Fused decode BitLinear (one launch): workgroups 0..31 run the activation
// prologue of one token row each (btl_act_row.h) and publish the quantised
// rows with coherent stores and one ready flag per row; the GEMM workgroups
// issue their weight loads first, then wait for the 32 flags (bounded spin),
// so weight streaming overlaps the prologue and a launch is saved.
//
// Prefill (M > 32): 128x256 output tiles, operands staged through LDS once
// per superblock and shared by the four waves (64x128 each).
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "btl_act_row.h"
#include "btl_mfma.h"
#include "btl_trace.h"

namespace btl {

int launch_act(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma, float norm_eps,
               int8_t* xa, float* a_dq, int32_t* rowsum, float* act_scale, int8_t* xq_rm, uint16_t* y_rm,
               uint32_t* zero_words, int n_zero_words, hipStream_t stream);
int check_act_args(const char* who, const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma);

struct GemmArgs {
  const int8_t* xa;
  const float* a_dq;
  const int32_t* rowsum;  // optional [M] sum_k q (prefill: else summed from the tile's operand)
  const uint32_t* wdev;
  int M, KS, NT, N, n_out, Mb;
  int splitk, ngroups;
  int mh;  // fused decode: 1, or 2 workgroups per column group, one per 16-row half
  int half16;  // fused decode, M <= 16: one workgroup per column group on the 16-row body
  int xa_bytes;
  float seg_scale[BTL_MAX_SEGMENTS];
  int seg_end[BTL_MAX_SEGMENTS];
  int nseg;
  const uint16_t* residual;
  uint16_t* out;
  int32_t* acc_out;
  int32_t* ws_part;
  uint32_t* ws_cnt;
};

// Producer/consumer handshake of the fused decode kernel: launch counters,
// so no call has to reset anything for the next one.
//   ready[m] (own 128-byte line each): the number of launches whose row m
//          activation block has published its row.  Block m reads it when it
//          starts and stores one more once the row is out.
//   seen[j], j < kGemmSlots (packed words): the number of launches the GEMM
//          slot has taken part in.  GEMM block g reads seen[g] when it starts,
//          so e = seen[g] + 1 names this launch; it waits until every ready
//          word has reached e, then stores e into the slots g, g + ngemm, ...
//          so that slots beyond this launch's grid keep the count too.
// Every completed launch leaves all ready and seen words at the same count
// (zero-filled = no launch yet), whatever grid sizes share the workspace.
struct FusedSync {
  uint32_t* words;  // handshake words
  uint32_t* err;    // sticky error word (the workspace's own, or the caller's)
  int nact;         // activation workgroups (32)
  int ngemm;        // GEMM workgroups (at most kGemmSlots)
  unsigned spin_limit;
};
constexpr int kSyncStride = 32;   // words: 128 bytes
constexpr int kReadyStride = kSyncStride;
constexpr int kGemmSlots = 512;   // bound on the GEMM workgroups of one launch
enum { kErrorWord = 32, kSeenLine = 33 };  // in 128-byte lines; ready words from line 0
__device__ __forceinline__ uint32_t* sync_word(const FusedSync& fs, int w) { return fs.words + w * kSyncStride; }
__device__ __forceinline__ uint32_t* ready_word(const FusedSync& fs, int m) { return fs.words + m * kReadyStride; }
__device__ __forceinline__ uint32_t* seen_word(const FusedSync& fs, int j) {
  return fs.words + kSeenLine * kSyncStride + j;
}

__device__ __forceinline__ float seg_scale_of(const GemmArgs& p, int n) {
  float s = p.seg_scale[0];
#pragma unroll
  for (int i = 0; i + 1 < BTL_MAX_SEGMENTS; ++i)
    if (i + 1 < p.nseg && n >= p.seg_end[i]) s = p.seg_scale[i + 1];
  return s;
}

// Epilogue for one accumulator element (acc already row-sum corrected);
// ad = a_dq of the row, res = the residual element (used when p.residual).
// Callers load ad and res ahead: a load inside the store loop would cost a
// memory round trip per element.
__device__ __forceinline__ void epi_scale(const GemmArgs& p, int i, int n, int32_t acc, float ad, uint16_t res) {
  if (p.acc_out) p.acc_out[(int64_t)i * p.N + n] = acc;
  const float f = seg_scale_of(p, n) * ad;
  uint16_t o = f2bf((float)acc * f);
  if (p.residual) o = f2bf(bf2f(res) + bf2f(o));
  p.out[(int64_t)i * p.n_out + n] = o;
}
// Residual element (i, n) with the row clamped into range (for loads issued
// before the row check).
__device__ __forceinline__ uint16_t residual_at(const GemmArgs& p, int i, int n) {
  if (!p.residual) return 0;
  const int ic = i < p.M ? i : p.M - 1;
  return p.residual[(int64_t)ic * p.n_out + n];
}
__device__ __forceinline__ void epi_relu2(const GemmArgs& p, int i, int ng, int nu, int32_t ag, int32_t au,
                                          float ad) {
  if (p.acc_out) {
    p.acc_out[(int64_t)i * p.N + ng] = ag;
    p.acc_out[(int64_t)i * p.N + nu] = au;
  }
  const float g = bf2f(f2bf((float)ag * (seg_scale_of(p, ng) * ad)));
  const float u = bf2f(f2bf((float)au * (seg_scale_of(p, nu) * ad)));
  const float gr = g > 0.0f ? g : 0.0f;
  const float sq = bf2f(f2bf(gr * gr));
  p.out[(int64_t)i * p.n_out + ng] = f2bf(sq * u);
}

enum { EPI_SCALE = BTL_EPI_SCALE, EPI_RELU2 = BTL_EPI_RELU2_MUL };

// ------------------------------------------------------------- decode ----
// Poll wave of a fused GEMM workgroup: wait until the activation rows this
// workgroup reads (all of them, or row half h when mh = 2) carry this
// launch's number, then record the number in the workgroup's seen slots.
// A bounded spin: on time-out the error word is set and the wave goes on.
__device__ __forceinline__ void wait_rows_ready(const FusedSync& fs, int bid, int mh, int h, int lane) {
  const uint32_t e = ld_coherent(seen_word(fs, bid)) + 1u;  // this launch's number
  unsigned n = 0;
  for (;;) {
    const bool mine = lane >= fs.nact || (mh == 2 && (lane >> 4) != h) ||
                      (int32_t)(ld_coherent(ready_word(fs, lane)) - e) >= 0;
    if (__all(mine)) break;
    if (++n > fs.spin_limit) {
      if (lane == 0) st_coherent(fs.err, 1u);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  // after the wait: stores count in the same wait counter as the polls
  for (int j = bid + lane * fs.ngemm; j < kGemmSlots; j += 64 * fs.ngemm) st_coherent(seen_word(fs, j), e);
}

// GEMM workgroup of the decode path.  With FUSED the activations come from
// workgroups of the same launch: wait for them after the weight loads of the
// first pass are in flight, and read activations and scales coherently.
template <int TPW, int NSB, int EPI, int WAVES, bool FUSED>
__device__ void gemm_decode_wg(const GemmArgs& p, int bid, const FusedSync& fs) {
  static_assert(EPI != EPI_RELU2 || TPW == 2, "relu2 pairs a gate tile with its up tile");
  static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves");
  constexpr int RR = 16 / WAVES;  // accumulator rows finished per thread and tile
  __shared__ int32_t red[WAVES][TPW][16][64];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = bid % p.ngroups;
  const int s = bid / p.ngroups;

  int tile[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) tile[t] = (EPI == EPI_RELU2) ? (g + t * (p.NT >> 1)) : (g * TPW + t);

  const int sb0 = (s * p.KS) / p.splitk, sb1 = ((s + 1) * p.KS) / p.splitk;
  const int nsb = sb1 - sb0;
  // In the fused kernel the last wave only polls the ready flags: with no
  // weight loads of its own in flight, a poll returns as soon as the flag
  // lands (loads complete in issue order).  The other waves share K.
  constexpr int KW = FUSED ? WAVES - 1 : WAVES;
  const int wb = wv < KW ? sb0 + (wv * nsb) / KW : sb1;
  const int we = wv < KW ? sb0 + ((wv + 1) * nsb) / KW : sb1;


  v16i acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  // A slot past a pass's count re-reads the pass's last superblock (valid
  // address, cache hit); only the first `cnt` slots feed MFMAs.
  v4i b[TPW][NSB];
  auto load_b = [&](int base, int cnt) {
#pragma unroll
    for (int i = 0; i < NSB; ++i) {
      const int sb = base + (i < cnt ? i : cnt - 1);
#pragma unroll
      for (int t = 0; t < TPW; ++t) b[t][i] = ld128(p.wdev + (((int64_t)tile[t] * p.KS + sb) * 64 + lane) * 4);
    }
  };

  if (wb < we) load_b(wb, (we - wb) < NSB ? (we - wb) : NSB);
  // The residual is an input of the launch: fetch it now, behind the weights.
  uint16_t res_pre[TPW][RR];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int rr = 0; rr < RR; ++rr)
      res_pre[t][rr] = EPI == EPI_SCALE ? residual_at(p, acc_row(wv + WAVES * rr, lane), tile[t] * 32 + (lane & 31)) : 0;
  float ad_pre[RR];
  if (FUSED) {
    // Every thread of the workgroup reaches this barrier, with or without work.
    if (wv == WAVES - 1) wait_rows_ready(fs, bid, 1, 0, lane);
    __syncthreads();
    // Scales of the rows this thread finishes, loaded with the activations.
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) ad_pre[rr] = ld_coherent(p.a_dq + acc_row(wv + WAVES * rr, lane));
  }

  // Row sums from v_dot4 on the A bytes (an MFMA against an all-ones operand
  // instead measured 0.7 us slower per gate||up launch: this body's MFMAs
  // set its pace).
  int32_t rs_lane = 0;  // sum of this lane's A bytes (row lane & 31, half lane >> 5)
  for (int base = wb; base < we; base += NSB) {
    const int cnt = (we - base) < NSB ? (we - base) : NSB;
    if (base != wb) load_b(base, cnt);
    v4i a[NSB][4];
#pragma unroll
    for (int i = 0; i < NSB; ++i) {
      const int sb = base + (i < cnt ? i : cnt - 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // lane l: row l & 31, k-group l >> 5 (the fused kernel's own tile
        // holds a row's 32 bytes of a step together, fused_chunk_offset)
        const int off = FUSED ? (sb * 4 + q) * 1024 + (lane & 31) * 32 + (lane >> 5) * 16
                              : ((sb * 4 + q) * 64 + lane) * 16;
        // plain loads in both kernels: the tile is written once per launch
        // (by this launch's activation blocks, before their ready flags) and
        // caches start clean at every kernel boundary, so each XCD's L2
        // fetches it once for all of its CUs
        a[i][q] = ld128(p.xa + off);
      }
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
          rs_lane = bytes_sum(a[i][q], rs_lane);
        }
      }
    }
  }
  __shared__ int32_t red_rs[WAVES][32];
  {
    const int32_t rs_row = rs_lane + (int32_t)xor_partner_u<32>((uint32_t)rs_lane);
    if (lane < 32) red_rs[wv][lane] = rs_row;
  }

#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wv][t][r][lane] = acc[t][r];
  __syncthreads();

  // Thread (wv, lane) finishes accumulator rows r = wv + WAVES*rr of every
  // tile, minus this K slice's part of the row sum.
  int32_t v[TPW][RR];
#pragma unroll
  for (int rr = 0; rr < RR; ++rr) {
    const int r = wv + WAVES * rr;
    const int i = acc_row(r, lane);
    int32_t rs = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) rs += red_rs[w][i];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      int32_t sum = -rs;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) sum += red[w][t][r][lane];
      v[t][rr] = sum;
    }
  }

  if (p.splitk > 1) {
    // Publish this slice's partial tile; the last slice to arrive sums all
    // of them (integers: any order gives the same result) and finishes.
    int32_t* part = p.ws_part + ((int64_t)(g * p.splitk + s) * TPW) * 1024;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int rr = 0; rr < RR; ++rr) st_coherent(part + t * 1024 + (wv + WAVES * rr) * 64 + lane, v[t][rr]);
    wait_memory();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = atomicAdd(p.ws_cnt + g, 1u);
      s_last = (prev == (unsigned)(p.splitk - 1));
    }
    __syncthreads();
    if (!s_last) return;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int rr = 0; rr < RR; ++rr) {
        int32_t sum = v[t][rr];
        for (int ss = 0; ss < p.splitk; ++ss)
          if (ss != s)
            sum += ld_coherent(p.ws_part + ((int64_t)(g * p.splitk + ss) * TPW + t) * 1024 +
                               (wv + WAVES * rr) * 64 + lane);
        v[t][rr] = sum;
      }
    if (tid == 0) st_coherent(p.ws_cnt + g, 0u);
  }

  const int j = lane & 31;
  float ad_row[RR];
#pragma unroll
  for (int rr = 0; rr < RR; ++rr) ad_row[rr] = FUSED ? ad_pre[rr] : p.a_dq[acc_row(wv + WAVES * rr, lane)];
#pragma unroll
  for (int rr = 0; rr < RR; ++rr) {
    const int i = acc_row(wv + WAVES * rr, lane);
    if (i >= p.M) continue;
    const float ad = ad_row[rr];
    if (EPI == EPI_RELU2) {
      epi_relu2(p, i, tile[0] * 32 + j, tile[1] * 32 + j, v[0][rr], v[1][rr], ad);
    } else {
#pragma unroll
      for (int t = 0; t < TPW; ++t) epi_scale(p, i, tile[t] * 32 + j, v[t][rr], ad, res_pre[t][rr]);
    }
  }
}

// GEMM workgroup of a fused row-half launch (mh = 2, or half16 for M <= 16
// with every workgroup on h = 0): rows 16h..16h+15 of
// the token tile against TPW column tiles of 32 (scale epilogue: tiles
// g*TPW ..; relu2: gate tile g and its up tile), on
// v_mfma_i32_16x16x64_i8, two MFMAs (columns 0-15 and 16-31) per tile and
// 64 k.  A 32-row MFMA would spend half its cycles on the other half's rows.
//  * A: lane l takes row 16h + (l & 15), k-group l >> 4 of a 64-k step
//    straight from the fused kernel's tile: k-group G of step p is 32-k step
//    2p + (G >> 1), half G & 1, i.e. the 16 bytes at 32 row + 16 (G & 1) of
//    that step's block (fused_chunk_offset).
//  * B: the device layout gives lane l column l & 31, half l >> 5 of each
//    32-k step.  A 32-lane swap and then a 16-lane swap of the packed words
//    of steps 2p and 2p+1 give, in 16-lane rows r of (step, lanes),
//    [2p.r0 | 2p.r2 | 2p+1.r0 | 2p+1.r2] (columns 0-15) and
//    [2p.r1 | 2p.r3 | 2p+1.r1 | 2p+1.r3] (columns 16-31): lane l then holds
//    column (l & 15) (+16) with the k-group of its A operand.
//  * C: lane l, element j is row 4 (l >> 4) + j, column l & 15.
template <int TPW, int NSB, int EPI, int WAVES>
__device__ void gemm_decode_half(const GemmArgs& p, int bid, const FusedSync& fs) {
  static_assert(EPI == EPI_SCALE ? (TPW == 1 || TPW == 2) : TPW == 2, "tiles per workgroup");
  static_assert(WAVES * 64 == 512, "one output element per thread and tile");
  __shared__ int32_t red[WAVES][TPW][8][64];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // The two halves of a group are 8 workgroups apart, so that round-robin
  // dispatch puts them on one XCD and its L2 fetches the group's weights
  // once.  Past the last whole block of 8 groups they pair up r apart.
  const int g8 = p.ngroups & ~7;
  int g, h;
  if (p.half16) {  // M <= 16: one workgroup per group, rows 0..15
    g = bid;
    h = 0;
  } else if (bid < 2 * g8) {
    g = ((bid >> 4) << 3) | (bid & 7);
    h = (bid >> 3) & 1;
  } else {
    const int i = bid - 2 * g8, r = p.ngroups - g8;
    g = g8 + i % r;
    h = i / r;
  }
  int tile[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    constexpr int HP = TPW / 2;  // relu2: gate tiles t < HP, up tiles t >= HP
    tile[t] = EPI == EPI_RELU2 ? (t < HP ? g * HP + t : (p.NT >> 1) + g * HP + (t - HP)) : g * TPW + t;
  }
  // the last wave only polls (as in gemm_decode_wg); the others share K
  constexpr int KW = WAVES - 1;
  const int wb = wv < KW ? (wv * p.KS) / KW : p.KS;
  const int we = wv < KW ? ((wv + 1) * p.KS) / KW : p.KS;

  v4i b[TPW][NSB];
  auto load_b = [&](int base, int cnt) {
#pragma unroll
    for (int i = 0; i < NSB; ++i) {
      const int sb = base + (i < cnt ? i : cnt - 1);
#pragma unroll
      for (int t = 0; t < TPW; ++t) b[t][i] = ld128(p.wdev + (((int64_t)tile[t] * p.KS + sb) * 64 + lane) * 4);
    }
  };
  // The swaps above, in place: words 2p and 2p + 1 then hold columns 0-15 and
  // 16-31 of 64-k step p.
  auto regroup_b = [&]() {
#pragma unroll
    for (int i = 0; i < NSB; ++i)
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          const auto s32 =
              __builtin_amdgcn_permlane32_swap((uint32_t)b[t][i][2 * pp], (uint32_t)b[t][i][2 * pp + 1], false, false);
          const auto s16 = __builtin_amdgcn_permlane16_swap(s32[0], s32[1], false, false);
          b[t][i][2 * pp] = (int)s16[0];
          b[t][i][2 * pp + 1] = (int)s16[1];
        }
  };
  // The first weights are regrouped while the flags are awaited.
  if (wb < we) {
    load_b(wb, (we - wb) < NSB ? (we - wb) : NSB);
    regroup_b();
  }

  // the output elements this thread finishes: row 16h + er, column ec of every tile
  const int er = tid >> 5, ec = tid & 31;
  const int row = 16 * h + er;
  uint16_t res[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) res[t] = EPI == EPI_SCALE ? residual_at(p, row, tile[t] * 32 + ec) : 0;
  if (wv == WAVES - 1) wait_rows_ready(fs, bid, 2, h, lane);
  __syncthreads();
  const float ad = ld_coherent(p.a_dq + row);

  v4i acc[TPW][2];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t][0] = acc[t][1] = (v4i){0, 0, 0, 0};
  // Row sums on the matrix pipe, which has room here (the 2-bit unpack keeps
  // the VALU busier): A against an all-ones operand, every column of row r
  // holding sum_k q[r][k].
  const v4i ones = (v4i){0x01010101, 0x01010101, 0x01010101, 0x01010101};
  v4i acc_rs = (v4i){0, 0, 0, 0};
  const int a_off = (16 * h + (lane & 15)) * 32 + ((lane >> 4) & 1) * 16;  // row, k-group in a step's block
  const int a_step = lane >> 5;
  for (int base = wb; base < we; base += NSB) {
    const int cnt = (we - base) < NSB ? (we - base) : NSB;
    if (base != wb) {
      load_b(base, cnt);
      regroup_b();
    }
    v4i a[NSB][2];
#pragma unroll
    for (int i = 0; i < NSB; ++i) {
      const int sb = base + (i < cnt ? i : cnt - 1);
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) a[i][pp] = ld128(p.xa + (sb * 4 + 2 * pp + a_step) * 1024 + a_off);
    }
#pragma unroll
    for (int i = 0; i < NSB; ++i) {
      if (i < cnt) {
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
          for (int t = 0; t < TPW; ++t) {
            acc[t][0] =
                __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][pp], unpack_b((uint32_t)b[t][i][2 * pp]), acc[t][0], 0, 0, 0);
            acc[t][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][pp], unpack_b((uint32_t)b[t][i][2 * pp + 1]),
                                                              acc[t][1], 0, 0, 0);
          }
          acc_rs = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][pp], ones, acc_rs, 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      red[wv][t][j][lane] = acc[t][0][j] - acc_rs[j];
      red[wv][t][4 + j][lane] = acc[t][1][j] - acc_rs[j];
    }
  __syncthreads();
  const int reg = 4 * (ec >> 4) + (er & 3), src = 16 * (er >> 2) + (ec & 15);
  int32_t v[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    int32_t sum = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) sum += red[w][t][reg][src];
    v[t] = sum;
  }
  if (row >= p.M) return;
  if constexpr (EPI == EPI_RELU2) {
#pragma unroll
    for (int u = 0; u < TPW / 2; ++u) epi_relu2(p, row, tile[u] * 32 + ec, tile[u + TPW / 2] * 32 + ec, v[u], v[u + TPW / 2], ad);
  } else {
#pragma unroll
    for (int t = 0; t < TPW; ++t) epi_scale(p, row, tile[t] * 32 + ec, v[t], ad, res[t]);
  }
}

template <int TPW, int NSB, int EPI, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_gemm_decode(GemmArgs p) {
  gemm_decode_wg<TPW, NSB, EPI, WAVES, false>(p, blockIdx.x, FusedSync{});
}

// One launch per decode BitLinear: blocks [0, nact) quantise the token rows,
// blocks [nact, nact + ngemm) run the GEMM.  Activation blocks come first in
// dispatch order, so they never wait behind GEMM blocks.
template <int TPW, int NSB, int EPI, bool NORM, int CPT, bool HALF>
__global__ __launch_bounds__(512) void k_bitlinear_decode(GemmArgs p, ActArgs a, FusedSync fs) {
  if ((int)blockIdx.x < fs.nact) {
    uint32_t* ready = ready_word(fs, (int)blockIdx.x);
    const uint32_t e = threadIdx.x == 0 ? ld_coherent(ready) + 1u : 0u;  // read while the row loads
    act_row<NORM, true, true, CPT>(a, blockIdx.x, threadIdx.x);
    wait_memory();
    __syncthreads();
    if (threadIdx.x == 0) st_coherent(ready, e);
    return;
  }
  if constexpr (HALF)
    gemm_decode_half<TPW, NSB, EPI, 8>(p, blockIdx.x - fs.nact, fs);
  else
    gemm_decode_wg<TPW, NSB, EPI, 8, true>(p, blockIdx.x - fs.nact, fs);
}

// ------------------------------------------------------------ prefill ----
// Workgroup tile: 4 row blocks (128 rows) x 8 column tiles (256 columns); for
// relu2 the 8 slots are 4 gate tiles and their 4 up tiles, so the workgroup
// finishes 128 columns of relu(g)^2*u.  Each superblock (128 of K) of the
// activation tile (16 KiB: 4 row blocks x 4 k-steps) and of the packed
// weights (8 KiB: 8 tiles) is staged in LDS as 24 chunks of 1 KiB, six per
// wave, each one global_load_lds_dwordx4 (lane i's 16 bytes land at chunk +
// 16i), so staging costs no registers.  ST stages rotate (3 for 128-row
// tiles, 4 for 64-row tiles): one barrier per superblock, after the wave's
// own loads of it have landed (vmcnt), also marks the previous stage as read
// by every wave, and that stage is refilled right after it with the
// superblock ST - 1 ahead.  The four waves form a WR x (4/WR) grid: wave
// (wm, wn) = (wv % WR, wv / WR) computes the RB/WR row blocks from
// (RB/WR)*wm against US = 2*WR column slots: US*wn.. (scale), or US/2 gate
// slots from (US/2)*wn with the up slots 4 above them (relu2: a column's gate
// and up tiles stay in one wave).  With WR = 1 a wave covers every row block,
// so each unpacked weight operand feeds RB MFMAs.
//
// Tile order is XCD-aware: workgroup b runs on XCD b % 8, so tiles are
// numbered in groups of kPfGroupRows row tiles (column tiles inner) and XCD x
// takes the contiguous range [x*per, (x+1)*per) of that order -- a compact
// block of about kPfGroupRows row tiles x per/kPfGroupRows column tiles whose
// operands (a few MB) stay in that XCD's L2.
constexpr int kPfXcds = 8;
constexpr int kPfGroupRows = 4;
constexpr int kPfCT = 8;      // column tiles of 32 per workgroup
// Row blocks of 32 per workgroup: 4 (128 rows), or 2 (64 rows, each wave one
// row block) when 128-row tiles would leave CUs idle.

template <int EPI>
__device__ __forceinline__ int pf_tile(const GemmArgs& p, int gn, int slot) {
  if (EPI == EPI_RELU2) {
    const int half = p.NT >> 1;
    const int g = gn * 4 + (slot & 3);
    return (slot < 4 ? 0 : half) + (g < half ? g : half - 1);
  }
  const int t = gn * kPfCT + slot;
  return t < p.NT ? t : p.NT - 1;
}

// s_waitcnt with only the vector-memory count constrained (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
#define BTL_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// Waits until at most min(later, S - 1) superblocks' worth (PW loads each) of
// this wave's direct-to-LDS loads are outstanding (the immediate of s_waitcnt
// is a compile-time constant, hence the recursion).
template <int PW, int S>
__device__ __forceinline__ void pf_wait(int later) {
  if constexpr (S > 1) {
    if (later >= S - 1) {
      BTL_WAIT_VMCNT((S - 1) * PW);
      return;
    }
    pf_wait<PW, S - 1>(later);
  } else {
    BTL_WAIT_VMCNT(0);
  }
}

template <int RB, int WR>
struct PfShape {
  static_assert(RB == 2 || RB == 4, "64- or 128-row tiles");
  static_assert(WR == 1 || WR == 2, "waves along the rows");
  static constexpr int rb = RB;                  // row blocks of 32 per workgroup
  static constexpr int xr = RB / WR;             // row blocks per wave
  static constexpr int us = 2 * WR;              // column slots per wave
  static constexpr int chunks = RB * 4 + kPfCT;  // 1 KiB chunks per stage
  static constexpr int per_wave = chunks / 4;
  // Stages in flight: the 128-row tile's 24 KiB stages fit three times for two
  // workgroups per CU; the 64-row tile's 16 KiB stages four times.
  static constexpr int stages = RB == 4 ? 3 : 4;
};

// Issues this wave's direct-to-LDS loads of superblock ks (a plain function:
// a lambda here keeps the host compiler from emitting the kernel's stub).
template <int NC, int ST>
__device__ __forceinline__ void pf_issue(int8_t* stage_base, int stage_bytes, const int8_t* const* src, const int* step,
                                         int ks, int wv) {
  int8_t* dst = stage_base + (ks % ST) * stage_bytes + wv * NC * 1024;
#pragma unroll
  for (int i = 0; i < NC; ++i) __builtin_amdgcn_global_load_lds(src[i] + (int64_t)ks * step[i], dst + i * 1024, 16, 0, 0);
}

// PRS: the row sums come in p.rowsum (the activation kernel's); without it
// one wave per row block sums that block's operand bytes in the loop.
// SK (with PRS): p.splitk workgroups share each tile, superblocks split
// evenly; each publishes its raw partial sums (coherent stores, then a
// per-tile arrival counter) and the last to arrive adds the others' partials
// -- integers, so any order gives the same result -- and runs the epilogue.
// Nothing waits on another workgroup.
template <int RB, int WR>
constexpr int pf_partial_qwords() {  // 64-bit words of one workgroup's partial tile
  return 4 * PfShape<RB, WR>::xr * PfShape<RB, WR>::us * 8 * 64;
}
template <int EPI, int RB, int WR, bool PRS, bool SK>
__global__ __launch_bounds__(256, 2) void k_gemm_prefill(GemmArgs p, int ngm, int ngn) {
  static_assert(!SK || PRS, "split-K sums raw partials and subtracts the given row sums once");
  constexpr int ST = PfShape<RB, WR>::stages;
  constexpr int kPfRB = PfShape<RB, WR>::rb;
  constexpr int XR = PfShape<RB, WR>::xr;
  constexpr int US = PfShape<RB, WR>::us;
  constexpr int HU = US / 2;  // relu2: gate (and up) slots per wave
  constexpr int kPfChunks = PfShape<RB, WR>::chunks;
  constexpr int kPfChunksPerWave = PfShape<RB, WR>::per_wave;
  // One LDS object: the stage buffers, then a_dq and the row sums of the
  // tile's rows, then the split-K arrival flag.
  __shared__ __attribute__((aligned(16))) int8_t lds[ST * kPfChunks * 1024 + kPfRB * 32 * 8 + 16];
  int* s_last = reinterpret_cast<int*>(lds + ST * kPfChunks * 1024 + kPfRB * 32 * 8);
  int8_t (*stage)[kPfChunks * 1024] = reinterpret_cast<int8_t (*)[kPfChunks * 1024]>(lds);
  float* s_adq = reinterpret_cast<float*>(lds + ST * kPfChunks * 1024);
  int32_t* s_rs = reinterpret_cast<int32_t*>(lds + ST * kPfChunks * 1024 + kPfRB * 32 * 4);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // wave-uniform as far as the compiler knows (a branch on wn then costs no
  // select over both sides)
  const int wm = __builtin_amdgcn_readfirstlane(wv % WR), wn = __builtin_amdgcn_readfirstlane(wv / WR);
  const int ntiles = ngm * ngn;
  const int nsplit = SK ? p.splitk : 1;
  const int nunits = ntiles * nsplit;  // a tile's splits are consecutive units
  const int per = (nunits + kPfXcds - 1) / kPfXcds;
  const int unit = (int)(blockIdx.x % kPfXcds) * per + (int)(blockIdx.x / kPfXcds);
  if (unit >= nunits) return;
  const int t = unit / nsplit, sp = unit % nsplit;
  const int grp = t / (kPfGroupRows * ngn);            // group of kPfGroupRows row tiles
  const int rows_in = min(kPfGroupRows, ngm - grp * kPfGroupRows);
  const int r = t - grp * kPfGroupRows * ngn;
  const int gm = grp * kPfGroupRows + r % rows_in;
  const int gn = r / rows_in;
  // this workgroup's superblocks [sb0, sb0 + KS) of the p.KS
  const int sb0 = SK ? (sp * p.KS) / nsplit : 0;
  const int KS = SK ? ((sp + 1) * p.KS) / nsplit - sb0 : p.KS;
  const int KSall = p.KS;  // row stride of the operand layouts

  // Global source of this wave's chunks at superblock 0; a superblock
  // advances activation chunks by 4 KiB and weight chunks by 1 KiB.
  const int8_t* src[kPfChunksPerWave];
  int step[kPfChunksPerWave];
#pragma unroll
  for (int i = 0; i < kPfChunksPerWave; ++i) {
    const int c = wv * kPfChunksPerWave + i;
    if (c < kPfRB * 4) {
      int mb = gm * kPfRB + (c >> 2);
      mb = mb < p.Mb ? mb : p.Mb - 1;
      src[i] = p.xa + ((((int64_t)mb * KSall + sb0) * 4 + (c & 3)) * 64 + lane) * 16;
      step[i] = 4096;
    } else {
      const int tile = pf_tile<EPI>(p, gn, c - kPfRB * 4);
      src[i] = reinterpret_cast<const int8_t*>(p.wdev) + (((int64_t)tile * KSall + sb0) * 64 + lane) * 16;
      step[i] = 1024;
    }
  }
  int slot[US];
#pragma unroll
  for (int u = 0; u < US; ++u) slot[u] = (EPI == EPI_RELU2) ? ((u < HU ? 0 : 4) + HU * wn + u % HU) : (US * wn + u);

  v16i acc[XR][US];
#pragma unroll
  for (int x = 0; x < XR; ++x)
#pragma unroll
    for (int u = 0; u < US; ++u) acc[x][u] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  // Row sums (!PRS): each row block of the tile is summed by one wave: wave
  // (wm, wn) takes its row block XR*wm + wn when wn < XR.
  int32_t rs_lane = 0;

  const int row_mine = gm * kPfRB * 32 + (tid & (kPfRB * 32 - 1));
  const float adq_mine = p.a_dq[min(row_mine, p.Mb * 32 - 1)];
  if (PRS) rs_lane = p.rowsum[min(row_mine, p.M - 1)];  // rows past M are not stored
#pragma unroll
  for (int k = 0; k < ST; ++k)
    if (k < KS) pf_issue<kPfChunksPerWave, ST>(lds, kPfChunks * 1024, src, step, k, wv);
  BTL_TRACE_AT(0);
  for (int ks = 0; ks < KS; ++ks) {
    // Superblocks of this wave in flight: ks .. ks + ST - 1 at ks = 0, then
    // ks .. ks + ST - 2 (the refill of a freed stage is issued one iteration
    // after its reads); ks has landed once the rest are all that is left.
    pf_wait<kPfChunksPerWave, ST>(min(ks == 0 ? ST - 1 : ST - 2, KS - 1 - ks));
    if (ks < 5) BTL_TRACE_AT(1 + 2 * ks);
    // every wave's loads of ks have landed and every wave is done reading
    // stage (ks - 1) % ST, which is refilled with superblock ks - 1 + ST
    lds_barrier();
    if (ks < 5) BTL_TRACE_AT(2 + 2 * ks);
    if (ks >= 1 && ks - 1 + ST < KS)
      pf_issue<kPfChunksPerWave, ST>(lds, kPfChunks * 1024, src, step, ks - 1 + ST, wv);
    const int8_t* buf = stage[ks % ST];
    v4i bw[US];
#pragma unroll
    for (int u = 0; u < US; ++u) bw[u] = *reinterpret_cast<const v4i*>(buf + (kPfRB * 4 + slot[u]) * 1024 + lane * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v4i a[XR];
#pragma unroll
      for (int x = 0; x < XR; ++x) a[x] = *reinterpret_cast<const v4i*>(buf + ((XR * wm + x) * 4 + q) * 1024 + lane * 16);
#pragma unroll
      for (int u = 0; u < US; ++u) {
        const v4i b = unpack_b((uint32_t)bw[u][q]);
#pragma unroll
        for (int x = 0; x < XR; ++x) acc[x][u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[x], b, acc[x][u], 0, 0, 0);
      }
      if (!PRS) {
#pragma unroll
        for (int x = 0; x < XR; ++x)
          if (x == wn) rs_lane = bytes_sum(a[x], rs_lane);  // wn is uniform across the wave
      }
    }
    if (ks == KS - 1) BTL_TRACE_AT(13);
  }

  if (SK && nsplit > 1) {
    // Publish this split's partial tile: lane-contiguous 64-bit words
    // (registers r, r + 1 of accumulator (x, u)), one block per split.
    constexpr int kQ = pf_partial_qwords<RB, WR>();
    uint64_t* const part = reinterpret_cast<uint64_t*>(p.ws_part);
    uint64_t* const mine = part + (int64_t)(t * nsplit + sp) * kQ;
#pragma unroll
    for (int x = 0; x < XR; ++x)
#pragma unroll
      for (int u = 0; u < US; ++u)
#pragma unroll
        for (int r2 = 0; r2 < 8; ++r2)
          st_coherent(mine + (((wv * XR + x) * US + u) * 8 + r2) * 64 + lane,
                      (uint64_t)(uint32_t)acc[x][u][2 * r2] | ((uint64_t)(uint32_t)acc[x][u][2 * r2 + 1] << 32));
    wait_memory();
    __syncthreads();  // the whole partial is out before the arrival is counted
    if (tid == 0) *s_last = atomicAdd(p.ws_cnt + t, 1u) == (unsigned)(nsplit - 1);
    __syncthreads();
    if (!*s_last) return;
    // Last to arrive: every other split's partial is out (its counter
    // increment followed its acknowledged stores); add them.
    for (int o = 0; o < nsplit; ++o) {
      if (o == sp) continue;
      const uint64_t* const other = part + (int64_t)(t * nsplit + o) * kQ;
#pragma unroll
      for (int x = 0; x < XR; ++x)
#pragma unroll
        for (int u = 0; u < US; ++u)
#pragma unroll
          for (int r2 = 0; r2 < 8; ++r2) {
            const uint64_t v = ld_coherent(other + (((wv * XR + x) * US + u) * 8 + r2) * 64 + lane);
            acc[x][u][2 * r2] += (int32_t)(uint32_t)v;
            acc[x][u][2 * r2 + 1] += (int32_t)(uint32_t)(v >> 32);
          }
    }
    if (tid == 0) st_coherent(p.ws_cnt + t, 0u);  // the workspace is left clean for the next call
  }

  // Epilogue in two passes through LDS (the stage buffers are free now):
  // each wave writes its scaled bf16 values (relu^2*u for relu2) into the
  // workgroup's output tile, then all threads write whole rows with 16-byte
  // stores, adding the residual read the same way.
  if (PRS) {
    if (tid < kPfRB * 32) s_rs[tid] = rs_lane;  // loaded at the start with a_dq
  } else {
    const int32_t rs_row = rs_lane + (int32_t)xor_partner_u<32>((uint32_t)rs_lane);  // lanes l, l+32: halves of row l & 31
    if (lane < 32 && wn < XR) s_rs[(XR * wm + wn) * 32 + lane] = rs_row;
  }
  if (tid < kPfRB * 32) s_adq[tid] = adq_mine;  // loaded at the start; stored now, after the stage loads
  __syncthreads();  // s_rs, s_adq visible; every wave is done with the stage buffers
  int8_t* tile_lds = &stage[0][0];
  constexpr int kOutCols = (EPI == EPI_RELU2) ? kPfCT * 16 : kPfCT * 32;  // output columns of the tile
  constexpr int kPitch = kOutCols * 2 + 16;  // bytes per row; halves of a wave land 16 banks apart
  static_assert(kPfRB * 32 * kPitch <= ST * kPfChunks * 1024, "output tile fits in the stage buffers");
  const int j = lane & 31;
  // weight scale per slot: segment ends are multiples of 32, so one per tile
  float sw[US];
#pragma unroll
  for (int u = 0; u < US; ++u) {
    if (EPI == EPI_RELU2) {
      const int half = p.NT >> 1;
      const int g = min(gn * 4 + HU * wn + u % HU, half - 1);
      sw[u] = seg_scale_of(p, (u < HU ? g : g + half) * 32);
    } else {
      sw[u] = seg_scale_of(p, min(gn * kPfCT + slot[u], p.NT - 1) * 32);
    }
  }
#pragma unroll
  for (int x = 0; x < XR; ++x) {
    float ad[16];
    int32_t rsr[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      ad[r] = s_adq[(XR * wm + x) * 32 + acc_row(r, lane)];
      rsr[r] = s_rs[(XR * wm + x) * 32 + acc_row(r, lane)];
    }
    if (p.acc_out) {  // exact accumulators (debug output)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = gm * kPfRB * 32 + (XR * wm + x) * 32 + acc_row(r, lane);
        if (i >= p.M) continue;
#pragma unroll
        for (int u = 0; u < US; ++u) {
          int t;
          if (EPI == EPI_RELU2) {
            const int g = gn * 4 + HU * wn + u % HU;
            t = g < (p.NT >> 1) ? (u < HU ? g : g + (p.NT >> 1)) : -1;
          } else {
            t = gn * kPfCT + slot[u] < p.NT ? gn * kPfCT + slot[u] : -1;
          }
          if (t >= 0) p.acc_out[(int64_t)i * p.N + t * 32 + j] = acc[x][u][r] - rsr[r];
        }
      }
    }
    // Row block x of this wave: lane l holds column j of rows acc_row(r, l)
    // = 8*(r/4) + 4*(l/32) + r%4, so a column's rows sit at constant offsets
    // from one base per slot, and rows r, r + 1 share one conversion.
    int8_t* const base_x = tile_lds + ((XR * wm + x) * 32 + 4 * (lane >> 5)) * kPitch + j * 2;
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const int off0 = (8 * (r >> 2) + (r & 3)) * kPitch, off1 = off0 + kPitch;
      if (EPI == EPI_RELU2) {
#pragma unroll
        for (int u = 0; u < HU; ++u) {
          int8_t* const bu = base_x + (HU * wn + u) * 64;
          const uint32_t g2 = f2bf_pair((float)(acc[x][u][r] - rsr[r]) * (sw[u] * ad[r]),
                                        (float)(acc[x][u][r + 1] - rsr[r + 1]) * (sw[u] * ad[r + 1]));
          const uint32_t u2 = f2bf_pair((float)(acc[x][u + HU][r] - rsr[r]) * (sw[u + HU] * ad[r]),
                                        (float)(acc[x][u + HU][r + 1] - rsr[r + 1]) * (sw[u + HU] * ad[r + 1]));
          const float g0 = fmaxf(bf2f((uint16_t)g2), 0.0f), g1 = fmaxf(bf2f((uint16_t)(g2 >> 16)), 0.0f);
          const uint32_t sq = f2bf_pair(g0 * g0, g1 * g1);
          const uint32_t o = f2bf_pair(bf2f((uint16_t)sq) * bf2f((uint16_t)u2),
                                       bf2f((uint16_t)(sq >> 16)) * bf2f((uint16_t)(u2 >> 16)));
          *reinterpret_cast<uint16_t*>(bu + off0) = (uint16_t)o;
          *reinterpret_cast<uint16_t*>(bu + off1) = (uint16_t)(o >> 16);
        }
      } else {
#pragma unroll
        for (int u = 0; u < US; ++u) {
          int8_t* const bu = base_x + slot[u] * 64;
          const uint32_t o = f2bf_pair((float)(acc[x][u][r] - rsr[r]) * (sw[u] * ad[r]),
                                       (float)(acc[x][u][r + 1] - rsr[r + 1]) * (sw[u] * ad[r + 1]));
          *reinterpret_cast<uint16_t*>(bu + off0) = (uint16_t)o;
          *reinterpret_cast<uint16_t*>(bu + off1) = (uint16_t)(o >> 16);
        }
      }
    }
  }
  BTL_TRACE_AT(11);
  lds_barrier();  // the output tile is complete
  constexpr int kChunksPerRow = kOutCols / 8;
  constexpr int kPerThread = kPfRB * 32 * kChunksPerRow / 256;
  const int col_base = gn * kOutCols;
  const int n_cols = (EPI == EPI_RELU2) ? (p.NT >> 1) * 32 : p.NT * 32;  // == p.n_out
  uint4 res[kPerThread];
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int c = tid + 256 * k;
    const int i = gm * kPfRB * 32 + c / kChunksPerRow;
    const int col = col_base + (c % kChunksPerRow) * 8;
    res[k] = make_uint4(0u, 0u, 0u, 0u);
    if (EPI == EPI_SCALE && p.residual && i < p.M && col < n_cols)
      res[k] = *reinterpret_cast<const uint4*>(p.residual + (int64_t)i * p.n_out + col);
  }
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int c = tid + 256 * k;
    const int il = c / kChunksPerRow;
    const int i = gm * kPfRB * 32 + il;
    const int col = col_base + (c % kChunksPerRow) * 8;
    if (i >= p.M || col >= n_cols) continue;
    uint4 o = *reinterpret_cast<const uint4*>(tile_lds + il * kPitch + (c % kChunksPerRow) * 16);
    if (EPI == EPI_SCALE && p.residual) {
      uint32_t ow[4] = {o.x, o.y, o.z, o.w};
      const uint32_t rw[4] = {res[k].x, res[k].y, res[k].z, res[k].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = f2bf(bf2f((uint16_t)(rw[e] & 0xffffu)) + bf2f((uint16_t)(ow[e] & 0xffffu)));
        const uint32_t hi = f2bf(bf2f((uint16_t)(rw[e] >> 16)) + bf2f((uint16_t)(ow[e] >> 16)));
        ow[e] = lo | (hi << 16);
      }
      o = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
    *reinterpret_cast<uint4*>(p.out + (int64_t)i * p.n_out + col) = o;
  }
  BTL_TRACE_AT(14);
}

// ------------------------------------------------- prefill, wide tiles ----
// Two workgroups per CU (four waves each, one per SIMD) and an output tile
// sized so that the grid is about two tiles per CU: 64 rows (two row blocks)
// x CT column tiles, CT = ceil(NT / (2 CUs / row tiles)).  At M = 2048 on 256
// CUs that is 32 row tiles x 16 column groups (CT = 14, 8, 5 for N = 6912,
// 3840, 2560), so every CU gets about the same share where 128x256 tiles
// leave some CUs one tile and others two.  The two workgroups of a CU run
// independently, so one's barrier and LDS waits overlap the other's MFMAs.
// Every wave covers both row blocks (each unpacked weight operand feeds two
// MFMAs); wave w takes column span w / WQ of 4 / WQ and k-step group w % WQ
// of each superblock:
//   WQ = 1: span w of 4, all four k-steps;
//   WQ = 2: span w / 2 of 2, k-steps 2 (w % 2) and 2 (w % 2) + 1;
//   WQ = 4: all CT tiles, k-step w;
// whichever gives the smallest per-wave share; spans differ by at most one
// tile.  k-step partials are added in LDS at the end (integers: any order
// gives the same sums).
// Staging as in k_gemm_prefill (global_load_lds, ST rotating stages, one
// barrier per superblock), with up to 8 stages.  A stage holds the 8
// activation chunks (chunk rb*4 + k-step) and up to 4*CTW/WQ weight chunks;
// wave w loads chunks w, w + 4, ...; chunks a tile does not have become
// 4-byte loads into a pad line, so every wave has the same number of loads in
// flight and waits on one vmcnt.  (Measured on MI355X: reading the next
// superblock's operands during the MFMAs, or spreading the refill loads
// between them, is slower -- more registers, and the other workgroup of the
// CU already fills those gaps; one workgroup of eight waves per CU is slower
// too, its barriers stall all four SIMDs at once.)
// Epilogue per row block: the waves put their raw sums into LDS in MFMA
// layout ([tile][register][lane]; k-step groups added with LDS atomics);
// then each thread converts 8 consecutive columns of a row (row sum, weight
// scale x a_dq, bf16, + residual) and writes them with one 16-byte store,
// consecutive threads along the row.
constexpr int kWideLds = 76 * 1024;  // two workgroups a CU
constexpr int kWideMaxStages = 8;
constexpr int kWideGroupRows = 8;  // XCD order: groups of 8 row tiles, column groups inner
constexpr int kWideResWords = 16 * 64 + 8;  // epilogue words per column tile (padded)

template <int CTW, int WQ>
struct WideShape {
  static constexpr int qw = 4 / WQ;                        // k-steps per superblock per wave
  static constexpr int ctmax = CTW * 4 / WQ;               // column tiles a tile may have
  static constexpr int pw = 2 + (ctmax + 3) / 4;           // loads per wave per stage
  static constexpr int stage_bytes = (8 + ctmax) * 1024 + 256;  // + the pad line
  static constexpr int st = kWideLds / stage_bytes < kWideMaxStages ? kWideLds / stage_bytes : kWideMaxStages;
  static constexpr int kpt = (32 * 4 * ctmax + 255) / 256;  // epilogue chunks per thread and row block
  static_assert((st - 1) * pw < 64, "vmcnt immediate");
  static_assert(st >= 3, "pipeline depth");
  // column tiles whose epilogue sums fit in the stage buffers
  static constexpr int ctfit = st * stage_bytes / (kWideResWords * 4) < ctmax ? st * stage_bytes / (kWideResWords * 4)
                                                                             : ctmax;
};

// Wave wv's loads of superblock ks: chunk wv + 4i of the stage; loads
// i < nreal are real, the rest pad loads.
template <int PW>
__device__ __forceinline__ void wide_issue(int8_t* stage, int8_t* pad, const int8_t* const* src, const int* step,
                                           int nreal, int ks, int wv) {
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    if (i < nreal)
      __builtin_amdgcn_global_load_lds(src[i] + (int64_t)ks * step[i], stage + (wv + 4 * i) * 1024, 16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds(src[0] + (int64_t)ks * step[0], pad, 4, 0, 0);
  }
}

template <int QW>
__device__ __forceinline__ void wide_read_b(const int8_t* p, uint32_t (&d)[QW]) {
  if constexpr (QW == 4) {
    const v4i v = *reinterpret_cast<const v4i*>(p);
    d[0] = (uint32_t)v.x, d[1] = (uint32_t)v.y, d[2] = (uint32_t)v.z, d[3] = (uint32_t)v.w;
  } else if constexpr (QW == 2) {
    typedef int v2i __attribute__((ext_vector_type(2)));
    const v2i v = *reinterpret_cast<const v2i*>(p);
    d[0] = (uint32_t)v.x, d[1] = (uint32_t)v.y;
  } else {
    d[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

// Operands of one superblock for a wave with NC column tiles: the
// activation k-steps of its group (both row blocks) and its weight dwords.
template <int NC, int QW>
struct WideOps {
  v4i a[QW][2];
  uint32_t bw[NC > 0 ? NC : 1][QW];
};

template <int NC, int QW>
__device__ __forceinline__ void wide_read_ops(const int8_t* buf, int qg, int slot0, int lane, WideOps<NC, QW>& o) {
  if constexpr (NC > 0) {
#pragma unroll
    for (int q = 0; q < QW; ++q) {
      o.a[q][0] = *reinterpret_cast<const v4i*>(buf + (qg * QW + q) * 1024 + lane * 16);
      o.a[q][1] = *reinterpret_cast<const v4i*>(buf + (4 + qg * QW + q) * 1024 + lane * 16);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) wide_read_b<QW>(buf + slot0 + c * 1024 + lane * 16 + qg * QW * 4, o.bw[c]);
  }
}

template <int NC, int CTW, int QW>
__device__ __forceinline__ void wide_mfma(v16i (&acc)[2][CTW], const WideOps<NC, QW>& o) {
  if constexpr (NC > 0) {
#pragma unroll
    for (int q = 0; q < QW; ++q) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const v4i b = unpack_b(o.bw[c][q]);
        acc[0][c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[q][0], b, acc[0][c], 0, 0, 0);
        acc[1][c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[q][1], b, acc[1][c], 0, 0, 0);
      }
    }
  }
}

// The superblock loop of a wave with NC column tiles (NC <= CTW), its first
// tile at LDS offset slot0 of a stage; the first ST superblocks are issued.
template <int NC, int CTW, int WQ>
__device__ __forceinline__ void wide_loop(v16i (&acc)[2][CTW], int8_t* lds, int8_t* pad, const int8_t* const* src,
                                          const int* step, int nreal, int KS, int wv, int qg, int slot0, int lane) {
  using S = WideShape<CTW, WQ>;
  constexpr int ST = S::st, SB = S::stage_bytes, PW = S::pw, QW = S::qw;
  for (int ks = 0; ks < KS; ++ks) {
    pf_wait<PW, ST>(min(ks == 0 ? ST - 1 : ST - 2, KS - 1 - ks));
    // every wave's loads of ks have landed and every wave is done reading
    // stage (ks - 1) % ST, which is refilled with superblock ks - 1 + ST
    lds_barrier();
    if (ks < 2) BTL_TRACE_AT(1 + ks);
    if (ks == KS / 2) BTL_TRACE_AT(3);
    if (ks >= 1 && ks - 1 + ST < KS) wide_issue<PW>(lds + ((ks - 1) % ST) * SB, pad, src, step, nreal, ks - 1 + ST, wv);
    WideOps<NC, QW> o;
    wide_read_ops<NC, QW>(lds + (ks % ST) * SB, qg, slot0, lane, o);
    wide_mfma<NC, CTW, QW>(acc, o);
  }
}

// The loop unrolled over the wave's range size nct (0 <= nct <= CTW).
template <int N, int CTW, int WQ>
__device__ __forceinline__ void wide_dispatch(int nct, v16i (&acc)[2][CTW], int8_t* lds, int8_t* pad,
                                              const int8_t* const* src, const int* step, int nreal, int KS, int wv,
                                              int qg, int slot0, int lane) {
  if constexpr (N == 0) {
    wide_loop<0, CTW, WQ>(acc, lds, pad, src, step, nreal, KS, wv, qg, slot0, lane);
  } else {
    if (nct == N)
      wide_loop<N, CTW, WQ>(acc, lds, pad, src, step, nreal, KS, wv, qg, slot0, lane);
    else
      wide_dispatch<N - 1, CTW, WQ>(nct, acc, lds, pad, src, step, nreal, KS, wv, qg, slot0, lane);
  }
}

// Scale epilogue with the row sums given (p.rowsum).  CT <= WideShape::ctfit.
template <int CTW, int WQ>
__global__ __launch_bounds__(256, 2) void k_gemm_wide(GemmArgs p, int ngm, int ngn, int CT) {
  using S = WideShape<CTW, WQ>;
  constexpr int ST = S::st, SB = S::stage_bytes, PW = S::pw, KPT = S::kpt;
  __shared__ __attribute__((aligned(16))) int8_t lds[ST * SB + 64 * 8 + S::ctmax * 4];
  float* s_adq = reinterpret_cast<float*>(lds + ST * SB);
  int32_t* s_rs = reinterpret_cast<int32_t*>(lds + ST * SB + 64 * 4);
  float* s_sw = reinterpret_cast<float*>(lds + ST * SB + 64 * 8);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // SIMD s = wv % 4 takes k-step group qg of column span [lo, hi); its two
  // waves take the two halves of the span.
  const int qg = wv % WQ, part = wv / WQ, nparts = 4 / WQ;
  const int ntiles = ngm * ngn;
  const int per = (ntiles + kPfXcds - 1) / kPfXcds;
  const int t = (int)(blockIdx.x % kPfXcds) * per + (int)(blockIdx.x / kPfXcds);
  if (t >= ntiles) return;
  const int grp = t / (kWideGroupRows * ngn);
  const int rows_in = min(kWideGroupRows, ngm - grp * kWideGroupRows);
  const int rt = t - grp * kWideGroupRows * ngn;
  const int gm = grp * kWideGroupRows + rt % rows_in;
  const int gn = rt / rows_in;
  const int KS = p.KS;
  const int CTg = min(CT, p.NT - gn * CT);  // this tile's column tiles (the last group may have fewer)

  // Sources: i = 0, 1 the activation chunk of row block i, k-step wv; i >= 2
  // weight tile wv + 4 (i - 2) of the tile (clamped into the matrix).
  const int8_t* src[PW];
  int step[PW];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    if (i < 2) {
      const int mb = min(gm * 2 + i, p.Mb - 1);
      src[i] = p.xa + ((((int64_t)mb * KS) * 4 + wv) * 64 + lane) * 16;
      step[i] = 4096;
    } else {
      const int tile = min(gn * CT + wv + 4 * (i - 2), p.NT - 1);
      src[i] = reinterpret_cast<const int8_t*>(p.wdev) + (((int64_t)tile * KS) * 64 + lane) * 16;
      step[i] = 1024;
    }
  }
  const int nreal = 2 + (CTg > wv ? (CTg - wv + 3) / 4 : 0);
  int8_t* const pad = lds + SB - 256;  // pad line of stage 0 (never read)

  // This wave's column tiles [c0, c0 + nct)
  const int c0 = part * CTg / nparts, nct = (part + 1) * CTg / nparts - c0;

  v16i acc[2][CTW];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int c = 0; c < CTW; ++c) acc[x][c] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  const int row_mine = gm * 64 + (tid & 63);
  const float adq_mine = p.a_dq[min(row_mine, p.Mb * 32 - 1)];
  const int32_t rs_mine = p.rowsum[min(row_mine, p.M - 1)];
#pragma unroll
  for (int k = 0; k < ST; ++k)
    if (k < KS) wide_issue<PW>(lds + k * SB, pad, src, step, nreal, k, wv);
  BTL_TRACE_AT(0);
#ifdef BTL_TRACE
  if (tid == 0 && blockIdx.x < (unsigned)kTraceBlocks) g_trace[blockIdx.x][15][0] = __builtin_amdgcn_s_memtime();
#endif
  wide_dispatch<CTW, CTW, WQ>(nct, acc, lds, pad, src, step, nreal, KS, wv, qg, (8 + c0) * 1024, lane);
  BTL_TRACE_AT(13);
#ifdef BTL_TRACE
  if (tid == 0 && blockIdx.x < (unsigned)kTraceBlocks) g_trace[blockIdx.x][15][13] = __builtin_amdgcn_s_memtime();
#endif

  if (tid < 64) {
    s_adq[tid] = adq_mine;
    s_rs[tid] = rs_mine;
  }
  if (tid < CTg) s_sw[tid] = seg_scale_of(p, (gn * CT + tid) * 32);
  __syncthreads();  // every wave is done with the stage buffers
  int32_t* const R = reinterpret_cast<int32_t*>(lds);
  const int nch = CTg * 4;  // 16-byte output chunks per row
  const float inv_nch = 1.0f / (float)nch;
  const int n_cols = p.NT * 32;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    // chunk k = tid + 256 j: row il = k / nch (exact in float: k < 2^13,
    // nch <= 256), column chunk cc = k - il * nch
    int il_[KPT], cc_[KPT];
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int k = tid + 256 * j;
      il_[j] = (int)(((float)k + 0.5f) * inv_nch);
      cc_[j] = k - il_[j] * nch;
    }
    uint4 res[KPT];
    if (p.residual) {
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int i = min(gm * 64 + x * 32 + il_[j], p.M - 1);
        const int col = min(gn * CT * 32 + cc_[j] * 8, n_cols - 8);
        res[j] = il_[j] < 32 ? *reinterpret_cast<const uint4*>(p.residual + (int64_t)i * p.n_out + col)
                             : make_uint4(0u, 0u, 0u, 0u);
      }
    }
    if (x) __syncthreads();  // the previous row block's sums have been read
    if (qg == 0) {
#pragma unroll
      for (int c = 0; c < CTW; ++c)
        if (c < nct)
#pragma unroll
          for (int r = 0; r < 16; ++r) R[(c0 + c) * kWideResWords + r * 64 + lane] = acc[x][c][r];
    }
    if (WQ > 1) {
      __syncthreads();
      if (qg != 0) {
#pragma unroll
        for (int c = 0; c < CTW; ++c)
          if (c < nct)
#pragma unroll
            for (int r = 0; r < 16; ++r) atomicAdd(&R[(c0 + c) * kWideResWords + r * 64 + lane], acc[x][c][r]);
      }
    }
    __syncthreads();
    if (x == 0) BTL_TRACE_AT(11);
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int il = il_[j], cc = cc_[j], ct = cc >> 2, jq = cc & 3;
      if (il >= 32) break;
      const int i = gm * 64 + x * 32 + il;
      const int col = (gn * CT + ct) * 32 + jq * 8;
      if (i >= p.M || col >= n_cols) continue;
      // row il of the block: lane half (il >> 2) & 1, register 4 (il >> 3) + (il & 3)
      const int32_t* s = R + ct * kWideResWords + (((il >> 3) << 2) | (il & 3)) * 64 + ((il >> 2) & 1) * 32 + jq * 8;
      const v4i v0 = *reinterpret_cast<const v4i*>(s);
      const v4i v1 = *reinterpret_cast<const v4i*>(s + 4);
      const int32_t rs = s_rs[x * 32 + il];
      const float f = s_sw[ct] * s_adq[x * 32 + il];
      const int32_t e[8] = {v0.x - rs, v0.y - rs, v0.z - rs, v0.w - rs, v1.x - rs, v1.y - rs, v1.z - rs, v1.w - rs};
      uint32_t o[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) o[h] = f2bf_pair((float)e[2 * h] * f, (float)e[2 * h + 1] * f);
      if (p.acc_out) {
        int32_t* const ao = p.acc_out + (int64_t)i * p.N + col;
        *reinterpret_cast<v4i*>(ao) = (v4i){e[0], e[1], e[2], e[3]};
        *reinterpret_cast<v4i*>(ao + 4) = (v4i){e[4], e[5], e[6], e[7]};
      }
      if (p.residual) {
        const uint32_t rw[4] = {res[j].x, res[j].y, res[j].z, res[j].w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint32_t lo = f2bf(bf2f((uint16_t)(rw[h] & 0xffffu)) + bf2f((uint16_t)(o[h] & 0xffffu)));
          const uint32_t hi = f2bf(bf2f((uint16_t)(rw[h] >> 16)) + bf2f((uint16_t)(o[h] >> 16)));
          o[h] = lo | (hi << 16);
        }
      }
      *reinterpret_cast<uint4*>(p.out + (int64_t)i * p.n_out + col) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  BTL_TRACE_AT(14);
}

// ------------------------------------------------------------- planning --
// Waves per standalone decode workgroup: 8 (two per SIMD) unless
// BTL_DECODE_WAVES=4.  The fused kernel always runs 8.
static int decode_waves() {
  static const int w = [] {
    const char* e = getenv("BTL_DECODE_WAVES");
    return (e && atoi(e) == 4) ? 4 : 8;
  }();
  return w;
}

// Compute units of the current device (256 on MI355X), cached per device
// (any thread may fill an entry; every writer stores the same value).  Host
// code without a GPU (size queries) plans for 256.
static int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (!cus) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
      (void)hipGetLastError();
      cus = 256;
    }
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

static int nsb_bucket(int per_wave) {
  if (per_wave <= 2) return 2;
  if (per_wave <= 4) return 4;
  if (per_wave <= 6) return 6;
  return 8;
}

constexpr int kFusedActBlocks = 32;
constexpr int64_t kSyncBytes = 8192;  // handshake words of the fused decode kernel
static_assert((kSeenLine * kSyncStride + kGemmSlots) * 4 <= kSyncBytes, "handshake words overflow");

// max_wgs: cap on workgroups (the fused kernel keeps every block resident).
static GemmPlan plan_decode(int64_t K, int64_t N, int epilogue, int splitk_req, int waves, int max_wgs) {
  GemmPlan pl = {};
  const int64_t KS = ksb(K), NT = N / 32;
  pl.prefill = false;
  pl.waves = waves;
  pl.tpw = 2;
  if (epilogue == BTL_EPI_SCALE && (NT % 2 || NT <= 160)) pl.tpw = 1;  // small N: spread tiles over more CUs
  pl.ngroups = (int)((epilogue == BTL_EPI_RELU2_MUL) ? NT / 2 : NT / pl.tpw);
  int sk = splitk_req;
  if (sk <= 0) {
    // About one workgroup per CU, without making a wave's share of K
    // smaller than one superblock.
    sk = (int)((max_wgs + pl.ngroups / 2) / pl.ngroups);
    if (sk < 1) sk = 1;
    while (sk > 1 && (int64_t)sk * pl.ngroups > max_wgs) --sk;
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

// Prefill tiling: 128-row tiles unless they would leave CUs idle, then
// 64-row tiles; a 64-row grid smaller than the CU count splits K (kernels
// given row sums only) up to about one workgroup per CU, at least 4
// superblocks each.  Measured on MI355X at M = 512: K = 6912, N = 2560
// 32.7 -> 21.7 us (3 splits); two workgroups per CU instead is slower at
// every shape (the finishing workgroup reads S - 1 partials of 64 KiB).
struct PfGrid {
  int rb, ngm, ngn, splitk;
};
static PfGrid pf_grid(int64_t M, int64_t K, int64_t N, int epilogue) {
  PfGrid g;
  const int Mb = (int)mblocks(M), NT = (int)(N / 32), KS = (int)ksb(K);
  g.ngn = (epilogue == BTL_EPI_RELU2_MUL) ? (NT / 2 + 3) / 4 : (NT + kPfCT - 1) / kPfCT;
  const int cus = device_cus();
  g.rb = ((Mb + 3) / 4) * g.ngn >= cus ? 4 : 2;
  g.ngm = (Mb + g.rb - 1) / g.rb;
  const int ntiles = g.ngm * g.ngn;
  g.splitk = 1;
  if (g.rb == 2 && ntiles <= cus) {
    int sk = cus / ntiles;
    if (sk > KS / 4) sk = KS / 4;
    if (sk > 8) sk = 8;
    g.splitk = sk > 1 ? sk : 1;
  }
  return g;
}

GemmPlan plan_gemm(int64_t M, int64_t K, int64_t N, int epilogue, int splitk_req) {
  if (M > 32) {
    GemmPlan pl = {};
    pl.prefill = true;
    const PfGrid g = pf_grid(M, K, N, epilogue);
    pl.splitk = g.splitk;
    pl.ngroups = g.ngm * g.ngn;  // tiles: one arrival counter each
    pl.ws_bytes = 0;
    if (g.splitk > 1)
      pl.ws_bytes = round_up((int64_t)pl.ngroups * 4, 256) +
                    (int64_t)pl.ngroups * g.splitk * pf_partial_qwords<2, 1>() * 8;
    return pl;
  }
  return plan_decode(K, N, epilogue, splitk_req, decode_waves(), device_cus());
}

// Fused plan: the GEMM blocks plus the activation blocks fit on the device
// at once.  fused = false when the shape needs more GEMM blocks than that.
static GemmPlan plan_fused(int64_t M, int64_t K, int64_t N, int epilogue, int splitk_req) {
  if (M > 32) return plan_gemm(M, K, N, epilogue, splitk_req);
  const int max_wgs = device_cus() - kFusedActBlocks;
  // No split by default: the workgroups' weights are in flight long before
  // the activations are, so a longer K per workgroup costs little, while the
  // split-K hand-off costs a memory round trip or two (measured on MI355X at
  // the 2B shapes: o_proj 8.6 us unsplit vs 9.6 us split in two).
  if (splitk_req <= 0) splitk_req = 1;
  GemmPlan pl = plan_decode(K, N, epilogue, splitk_req, 8, max_wgs);
  pl.fused = (int64_t)pl.ngroups * pl.splitk <= max_wgs && pl.ngroups * pl.splitk <= kGemmSlots && act_cpt(K) <= 4;
  // Two workgroups per column group, one per 16-row half, where both fit
  // (for the scale epilogue, doubling the column tiles of a group if that
  // makes them fit): each reads half of the activation tile after the
  // hand-off and runs 16-row MFMAs.  Measured on MI355X at the 2B shapes:
  // down 11.05 -> 9.6 us, o_proj 7.95 -> 7.1 us, QKV (two tiles a group)
  // 7.98 -> 7.62 us.
  pl.mh = 1;
  if (pl.fused && M > 16 && pl.splitk == 1) {
    const int NT = (int)(N / 32);
    auto fits = [&](int ng) { return 2 * ng <= max_wgs && 2 * ng <= kGemmSlots; };
    if (fits(pl.ngroups)) {
      pl.mh = 2;
    } else if (epilogue == BTL_EPI_SCALE && pl.tpw == 1 && NT % 2 == 0 && fits(NT / 2)) {
      pl.tpw = 2;
      pl.ngroups = NT / 2;
      pl.mh = 2;
    }
    // Not for gate||up: four tiles a workgroup (two gate/up pairs) measured
    // 9.9 us against 8.95 us for the whole-tile workgroups at 2560 -> 2 x 6912.
    // The 16-row MFMA halves the MFMA time per unpacked weight dword, so the
    // 2-bit unpack on the VALU then sets the pace.
  } else if (pl.fused && M <= 16 && pl.splitk == 1) {
    // Every row in the first half: one workgroup per column group runs the
    // 16-row body on it, so no MFMA or operand fetch is spent on the 16
    // padding rows of the whole-tile body.
    pl.half16 = true;
  }
  return pl;
}

FusedLayout fused_layout(int64_t M, int64_t K, int64_t N, int epilogue, int splitk_req) {
  FusedLayout L;
  const int64_t rows = mblocks(M) * 32;
  L.xa = kSyncBytes;
  L.a_dq = L.xa + round_up(btl_act_bytes(M, K), 256);
  L.rowsum = L.a_dq + round_up(rows * 4, 256);
  L.gemm_ws = L.rowsum + round_up(rows * 4, 256);
  const GemmPlan pf = plan_fused(M, K, N, epilogue, splitk_req);
  const GemmPlan pg = plan_gemm(M, K, N, epilogue, splitk_req);
  L.total = L.gemm_ws + (pf.ws_bytes > pg.ws_bytes ? pf.ws_bytes : pg.ws_bytes);
  return L;
}

template <int TPW, int EPI, int WAVES>
static void launch_decode_nsb(int nsb, dim3 grid, hipStream_t s, const GemmArgs& a) {
  const dim3 block(64 * WAVES);
  switch (nsb) {
    case 2: hipLaunchKernelGGL((k_gemm_decode<TPW, 2, EPI, WAVES>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_gemm_decode<TPW, 4, EPI, WAVES>), grid, block, 0, s, a); break;
    case 6: hipLaunchKernelGGL((k_gemm_decode<TPW, 6, EPI, WAVES>), grid, block, 0, s, a); break;
    default:  // 8 superblocks a pass (6 where 8 would spill, see decode_nsb)
      hipLaunchKernelGGL((k_gemm_decode<TPW, (WAVES == 8 && TPW == 2) ? 6 : 8, EPI, WAVES>), grid, block, 0, s, a);
      break;
  }
}

// The fused kernel's workgroups wait on each other: the instance launches
// only if the device (the stream's CUs) holds the whole grid at once.
template <int TPW, int EPI, bool NORM, int CPT, bool HALF>
static int launch_fused_nsb(int nsb, dim3 grid, hipStream_t s, const GemmArgs& g, const ActArgs& a,
                            const FusedSync& fs) {
  void (*k)(GemmArgs, ActArgs, FusedSync);
  switch (nsb) {
    case 2: k = k_bitlinear_decode<TPW, 2, EPI, NORM, CPT, HALF>; break;
    case 4: k = k_bitlinear_decode<TPW, 4, EPI, NORM, CPT, HALF>; break;
    case 6: k = k_bitlinear_decode<TPW, 6, EPI, NORM, CPT, HALF>; break;
    default: k = k_bitlinear_decode<TPW, TPW == 2 ? 6 : 8, EPI, NORM, CPT, HALF>; break;
  }
  const int rc = check_coresident_launch("fused decode BitLinear", reinterpret_cast<const void*>(k), 512, grid.x, s);
  if (rc) return rc;
  hipLaunchKernelGGL(k, grid, dim3(512), 0, s, g, a, fs);
  return BTL_OK;
}

// Superblocks per pass: the slice's share per wave, bucketed.  Two waves per
// SIMD leave 256 registers a wave: 2 tiles x 8 superblocks would spill, so
// such slices run as passes of 6.
static int decode_nsb(const GemmPlan& pl, int64_t KS, int epilogue) {
  const int per_wg = (int)((KS + pl.splitk - 1) / pl.splitk);
  const int work_waves = pl.fused ? pl.waves - 1 : pl.waves;  // the fused kernel's last wave polls
  const int per_wave = (per_wg + work_waves - 1) / work_waves;
  int nsb = nsb_bucket(per_wave);
  if (pl.waves == 8 && (pl.tpw == 2 || epilogue == BTL_EPI_RELU2_MUL) && nsb > 6) nsb = 6;
  return nsb;
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
  if (M > 32 && (!aligned(out, 16) || (residual && !aligned(residual, 16))))
    return set_error(BTL_ERR_ALIGN, "%s: out/residual must be 16-byte aligned for M > 32", who);
  return BTL_OK;
}

static GemmArgs gemm_args(const int8_t* xa, const float* a_dq, const int32_t* rowsum, int64_t M, int64_t K,
                          int64_t N, const uint32_t* wdev, const float* seg_scale, const int64_t* seg_end, int nseg,
                          int epilogue, const uint16_t* residual, uint16_t* out, int32_t* acc_out, char* ws,
                          const GemmPlan& pl) {
  GemmArgs a = {};
  a.xa = xa;
  a.a_dq = a_dq;
  a.rowsum = pl.prefill ? rowsum : nullptr;  // the decode kernels sum their operand
  a.wdev = wdev;
  a.M = (int)M;
  a.KS = (int)ksb(K);
  a.NT = (int)(N / 32);
  a.N = (int)N;
  a.n_out = (int)(epilogue == BTL_EPI_RELU2_MUL ? N / 2 : N);
  a.Mb = (int)mblocks(M);
  a.xa_bytes = (int)btl_act_bytes(M, K);
  a.nseg = nseg;
  for (int i = 0; i < BTL_MAX_SEGMENTS; ++i) {
    a.seg_scale[i] = i < nseg ? seg_scale[i] : 0.0f;
    a.seg_end[i] = i < nseg ? (int)(nseg > 1 ? seg_end[i] : N) : (int)N;
  }
  a.residual = residual;
  a.out = out;
  a.acc_out = acc_out;
  a.splitk = pl.splitk;
  a.mh = pl.mh == 2 ? 2 : 1;
  a.half16 = pl.half16 ? 1 : 0;
  a.ngroups = pl.ngroups;
  if (pl.splitk > 1) {  // decode split-K, or prefill split-K (per tile)
    a.ws_cnt = reinterpret_cast<uint32_t*>(ws);
    a.ws_part = reinterpret_cast<int32_t*>(ws + round_up((int64_t)pl.ngroups * 4, 256));
  }
  return a;
}

// Wide-tile plan (k_gemm_wide): 64-row tiles and CT column tiles, about two
// tiles per CU; WQ the split (1, 2 or 4 k-step groups) whose busiest wave has
// the fewest MFMAs (ties: the smaller WQ, fewer partial sums), CTW the
// largest wave range rounded up to an instantiated size (2, 3, 5; WQ = 1:
// 2, 3, 4).  Used for the scale epilogue with the row sums given, from M = 256,
// while the ranges fit (N <= 8192 at M = 2048); BTL_PREFILL_WIDE=0 turns it
// off (the 128x256 / 64x256 kernel then runs).
struct WidePlan {
  int ngm, ngn, ct, ctw, wq;
};
// k-step x column-tile MFMA pairs per superblock of the busiest wave, and the
// largest wave range, for CT tiles split the k_gemm_wide way.
static int wide_simd_load(int ct, int wq, int* ctw) {
  const int parts = 4 / wq, span = (ct + parts - 1) / parts;
  *ctw = span;
  return span * (4 / wq);
}
template <int WQ>
static int wide_ctfit_wq(int ctw) {
  return ctw <= 2 ? WideShape<2, WQ>::ctfit
                  : (ctw == 3 ? WideShape<3, WQ>::ctfit : WideShape<WQ == 1 ? 4 : 5, WQ>::ctfit);
}
static int wide_ctfit(int wq, int ctw) {
  return wq == 4 ? wide_ctfit_wq<4>(ctw) : (wq == 2 ? wide_ctfit_wq<2>(ctw) : wide_ctfit_wq<1>(ctw));
}
static bool wide_plan(int64_t M, int64_t K, int64_t N, int epilogue, bool prs, WidePlan* w) {
  const char* e = getenv("BTL_PREFILL_WIDE");
  if (e && e[0] == '0') return false;
  if (epilogue != BTL_EPI_SCALE || !prs || M < 256) return false;
  const int Mb = (int)mblocks(M), NT = (int)(N / 32);
  const int cus = device_cus();
  w->ngm = (Mb + 1) / 2;
  if (w->ngm > 2 * cus) return false;
  const int ngn_t = 2 * cus / w->ngm;
  w->ct = (NT + ngn_t - 1) / ngn_t;
  if (w->ct > 40) return false;
  w->ngn = (NT + w->ct - 1) / w->ct;
  // A grid well short of two tiles per CU with a long K runs faster as the
  // split-K 64-row tiles (measured on MI355X at M = 512, K = 6912, N = 2560:
  // 320 wide tiles 23.0-24.5 us, 64x256 tiles split in 3 22.0 us).
  if (w->ngm * w->ngn * 2 < 3 * cus && ksb(K) > 32) return false;
  int best = -1;
  for (int wq = 1; wq <= 4; wq *= 2) {
    int need;
    const int load = wide_simd_load(w->ct, wq, &need);
    // instantiated: CTW 2..5 (WQ = 1: 2..4; five tiles a wave with four
    // k-steps of operands held twice would spill)
    if (need > (wq == 1 ? 4 : 5) || w->ct > wide_ctfit(wq, need < 2 ? 2 : (need == 4 && wq != 1 ? 5 : need)))
      continue;
    if (best < 0 || load < best) {
      best = load;
      w->wq = wq;
      w->ctw = need < 2 ? 2 : (need == 4 && wq != 1 ? 5 : need);
    }
  }
  return best >= 0;
}

template <int WQ>
static void launch_wide_wq(int ctw, dim3 grid, hipStream_t s, const GemmArgs& a, int ngm, int ngn, int ct) {
  switch (ctw) {
    case 2: hipLaunchKernelGGL((k_gemm_wide<2, WQ>), grid, dim3(256), 0, s, a, ngm, ngn, ct); break;
    case 3: hipLaunchKernelGGL((k_gemm_wide<3, WQ>), grid, dim3(256), 0, s, a, ngm, ngn, ct); break;
    default:  // 4 (WQ = 1) or 5; the plan never takes four tiles with WQ = 2 or 4
      hipLaunchKernelGGL((k_gemm_wide<WQ == 1 ? 4 : 5, WQ>), grid, dim3(256), 0, s, a, ngm, ngn, ct);
      break;
  }
}

static void launch_wide(const WidePlan& w, hipStream_t s, const GemmArgs& a) {
  const int per = (w.ngm * w.ngn + kPfXcds - 1) / kPfXcds;
  const dim3 grid((unsigned)(per * kPfXcds));
  if (w.wq == 4)
    launch_wide_wq<4>(w.ctw, grid, s, a, w.ngm, w.ngn, w.ct);
  else if (w.wq == 2)
    launch_wide_wq<2>(w.ctw, grid, s, a, w.ngm, w.ngn, w.ct);
  else
    launch_wide_wq<1>(w.ctw, grid, s, a, w.ngm, w.ngn, w.ct);
}

template <int EPI>
static void launch_prefill_epi(bool prs, int rb, bool sk, dim3 grid, hipStream_t s, const GemmArgs& a, int ngm,
                               int ngn) {
  if (!prs) {
    if (rb == 4)
      hipLaunchKernelGGL((k_gemm_prefill<EPI, 4, 2, false, false>), grid, dim3(256), 0, s, a, ngm, ngn);
    else
      hipLaunchKernelGGL((k_gemm_prefill<EPI, 2, 1, false, false>), grid, dim3(256), 0, s, a, ngm, ngn);
  } else if (rb == 4) {
    hipLaunchKernelGGL((k_gemm_prefill<EPI, 4, 2, true, false>), grid, dim3(256), 0, s, a, ngm, ngn);
  } else if (sk) {
    hipLaunchKernelGGL((k_gemm_prefill<EPI, 2, 1, true, true>), grid, dim3(256), 0, s, a, ngm, ngn);
  } else {
    hipLaunchKernelGGL((k_gemm_prefill<EPI, 2, 1, true, false>), grid, dim3(256), 0, s, a, ngm, ngn);
  }
}

static int launch_gemm(const GemmArgs& a, int epilogue, const GemmPlan& pl, hipStream_t s) {
  if (pl.prefill) {
    WidePlan w;
    const int64_t K = (int64_t)a.KS * 128;
    if (wide_plan(a.M, K, a.N, epilogue, a.rowsum != nullptr, &w) && aligned(a.acc_out, 16)) {
      launch_wide(w, s, a);
      return check_launch("ternary gemm (prefill, wide tiles)");
    }
    const PfGrid g = pf_grid(a.M, (int64_t)a.KS * 128, a.N, epilogue);
    const int ngm = g.ngm, ngn = g.ngn, rb = g.rb;
    // split-K runs with the given row sums (partials are raw sums; the row sum
    // is subtracted once, by the workgroup that finishes the tile)
    const bool sk = a.rowsum && a.splitk > 1;
    GemmArgs b = a;
    if (!sk) b.splitk = 1;
    const int per = (ngm * ngn * b.splitk + kPfXcds - 1) / kPfXcds;
    dim3 grid((unsigned)(per * kPfXcds));
    // Every wave takes two row blocks, so each unpacked weight operand feeds
    // two MFMAs: 64-row tiles run the 1 x 4 wave grid (2 column slots per
    // wave), 128-row tiles the 2 x 2 grid (4 slots).  Measured on MI355X at
    // the 2B shapes, one row block per wave is 5-9 % slower (VALU unpacking
    // that does not overlap the MFMAs) and four per wave ~10 % slower (LDS
    // reads and 237 VGPRs).
    if (epilogue == BTL_EPI_RELU2_MUL)
      launch_prefill_epi<EPI_RELU2>(a.rowsum != nullptr, rb, sk, grid, s, b, ngm, ngn);
    else
      launch_prefill_epi<EPI_SCALE>(a.rowsum != nullptr, rb, sk, grid, s, b, ngm, ngn);
    return check_launch("ternary gemm (prefill)");
  }
  const int nsb = decode_nsb(pl, a.KS, epilogue);
  dim3 grid((unsigned)(pl.ngroups * pl.splitk));
  if (pl.waves == 8) {
    if (epilogue == BTL_EPI_RELU2_MUL)
      launch_decode_nsb<2, EPI_RELU2, 8>(nsb, grid, s, a);
    else if (pl.tpw == 2)
      launch_decode_nsb<2, EPI_SCALE, 8>(nsb, grid, s, a);
    else
      launch_decode_nsb<1, EPI_SCALE, 8>(nsb, grid, s, a);
  } else {
    if (epilogue == BTL_EPI_RELU2_MUL)
      launch_decode_nsb<2, EPI_RELU2, 4>(nsb, grid, s, a);
    else if (pl.tpw == 2)
      launch_decode_nsb<2, EPI_SCALE, 4>(nsb, grid, s, a);
    else
      launch_decode_nsb<1, EPI_SCALE, 4>(nsb, grid, s, a);
  }
  return check_launch("ternary gemm (decode)");
}

template <bool NORM, int CPT>
static int launch_fused_epi(int epilogue, const GemmPlan& pl, int nsb, dim3 grid, hipStream_t s, const GemmArgs& g,
                            const ActArgs& a, const FusedSync& fs) {
  if (pl.mh == 2 || pl.half16) {
    if (epilogue == BTL_EPI_RELU2_MUL) return launch_fused_nsb<2, EPI_RELU2, NORM, CPT, true>(nsb, grid, s, g, a, fs);
    if (pl.tpw == 2) return launch_fused_nsb<2, EPI_SCALE, NORM, CPT, true>(nsb, grid, s, g, a, fs);
    return launch_fused_nsb<1, EPI_SCALE, NORM, CPT, true>(nsb, grid, s, g, a, fs);
  }
  if (epilogue == BTL_EPI_RELU2_MUL) return launch_fused_nsb<2, EPI_RELU2, NORM, CPT, false>(nsb, grid, s, g, a, fs);
  if (pl.tpw == 2) return launch_fused_nsb<2, EPI_SCALE, NORM, CPT, false>(nsb, grid, s, g, a, fs);
  return launch_fused_nsb<1, EPI_SCALE, NORM, CPT, false>(nsb, grid, s, g, a, fs);
}

// Rows of 1, 2 or 4 chunks of 8 per thread (K <= 4096, 8192, 16384).
template <bool NORM>
static int launch_fused(int cpt, int epilogue, const GemmPlan& pl, int nsb, dim3 grid, hipStream_t s,
                        const GemmArgs& g, const ActArgs& a, const FusedSync& fs) {
  if (cpt <= 1) return launch_fused_epi<NORM, 1>(epilogue, pl, nsb, grid, s, g, a, fs);
  if (cpt <= 2) return launch_fused_epi<NORM, 2>(epilogue, pl, nsb, grid, s, g, a, fs);
  return launch_fused_epi<NORM, 4>(epilogue, pl, nsb, grid, s, g, a, fs);
}


// Argument checks shared by both fused entry points.
static int check_fused_args(const char* who, const uint16_t* x, int64_t M, int64_t K, int64_t ldx,
                            const uint16_t* gamma, const uint32_t* wdev, int64_t N, const float* seg_scale,
                            const int64_t* seg_end, int nseg, int epilogue, const uint16_t* residual,
                            const uint16_t* out, const int32_t* acc_out, const int8_t* xq_debug, int splitk) {
  int rc = check_act_args(who, x, M, K, ldx, gamma);
  if (rc) return rc;
  rc = check_gemm_args(who, M, K, N, wdev, seg_scale, seg_end, nseg, epilogue, residual, out);
  if (rc) return rc;
  if (splitk < 0) return set_error(BTL_ERR_ARG, "%s: splitk=%d", who, splitk);
  if ((acc_out && !aligned(acc_out, 4)) || (xq_debug && !aligned(xq_debug, 8)))
    return set_error(BTL_ERR_ALIGN, "%s: misaligned debug output", who);
  return BTL_OK;
}

// ---- the static scratch of btl_bitlinear_fused_noalloc ---------------------
// A workspace the library owns for callers that cannot allocate: one copy
// per device (each GPU the library runs on holds it until the process ends),
// zero at load and cleared once more by the first call on a device.  Calls
// on one device share it and leave its launch counters consistent for the
// next call; calls that overlap on one device race on it.
constexpr int64_t kNoAllocScratchBytes = BTL_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static_assert(kNoAllocScratchBytes % 256 == 0, "scratch size");

__global__ __launch_bounds__(256) void k_zero_words(uint4* p, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

constexpr int kMaxDevices = 64;
static std::atomic<char*> g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of this device's scratch (hipGetSymbolAddress once per
// device, with that device current); the first call also clears it on the
// caller's stream, ahead of the call's own kernels.
static int noalloc_scratch(char** out, hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return set_error(BTL_ERR_LAUNCH, "btl_bitlinear_fused_noalloc: no current device (or device id >= %d)",
                     kMaxDevices);
  }
  char* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p) {
    *out = p;
    return BTL_OK;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !addr) {
      (void)hipGetLastError();
      return set_error(BTL_ERR_LAUNCH, "btl_bitlinear_fused_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                       dev, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(k_zero_words, dim3(256), dim3(256), 0, stream, reinterpret_cast<uint4*>(addr),
                       (int64_t)(kNoAllocScratchBytes / 16));
    const int rc = check_launch("btl_bitlinear_fused_noalloc: scratch clear");
    if (rc) return rc;
    p = static_cast<char*>(addr);
    g_scratch[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return BTL_OK;
}

// Shared by btl_bitlinear_fused and btl_bitlinear_fused_noalloc: arguments
// checked, workspace sized and aligned; err: the sticky error word the
// fused kernel's bounded waits set (inside the workspace unless the caller
// gives one).
static int bitlinear_fused_impl(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma,
                                float norm_eps, const uint32_t* wdev, int64_t N, const float* seg_scale,
                                const int64_t* seg_end, int nseg, int epilogue, const uint16_t* residual,
                                uint16_t* out, int32_t* acc_out, int8_t* xq_debug, char* ws, const FusedLayout& L,
                                uint32_t* err, int splitk, btl_stream_t stream) {
  hipStream_t s = (hipStream_t)stream;
  int8_t* xa = (int8_t*)(ws + L.xa);
  float* a_dq = (float*)(ws + L.a_dq);

  const GemmPlan pf = plan_fused(M, K, N, epilogue, splitk);
  if (pf.fused) {
    ActArgs a = {};
    a.x = x;
    a.ldx = ldx;
    a.M = (int)M;
    a.K = (int)K;
    a.KS = (int)ksb(K);
    a.gamma = gamma;
    a.norm_eps = norm_eps;
    a.act_eps = 1e-5f;
    a.xa = xa;
    a.a_dq = a_dq;
    a.rowsum = nullptr;
    a.xq_rm = xq_debug;
    // Row 0 also clears the split-K counters, so a workspace left dirty by an
    // interrupted call is repaired by the next one.
    a.zero_words = pf.splitk > 1 ? (uint32_t*)(ws + L.gemm_ws) : nullptr;
    a.n_zero_words = pf.splitk > 1 ? pf.ngroups : 0;
    const GemmArgs g = gemm_args(xa, a_dq, nullptr, M, K, N, wdev, seg_scale, seg_end, nseg, epilogue, residual, out,
                                 acc_out, ws + L.gemm_ws, pf);
    FusedSync fs;
    fs.words = (uint32_t*)ws;
    fs.err = err ? err : fs.words + kErrorWord * kSyncStride;
    fs.nact = kFusedActBlocks;
    fs.ngemm = pf.ngroups * pf.splitk * g.mh;
    fs.spin_limit = 1u << 20;
    const int nsb = decode_nsb(pf, ksb(K), epilogue);
    const dim3 grid((unsigned)(kFusedActBlocks + fs.ngemm));
    const int cpt = act_cpt(K);
    const int rc = gamma ? launch_fused<true>(cpt, epilogue, pf, nsb, grid, s, g, a, fs)
                         : launch_fused<false>(cpt, epilogue, pf, nsb, grid, s, g, a, fs);
    if (rc == BTL_OK) return check_launch("fused decode BitLinear");
    // Not co-resident on this stream's CUs: the two-launch path below (the
    // activation kernel, then the GEMM) computes the same bits without any
    // wait between workgroups.
    clear_error();
  }

  const GemmPlan pl = plan_gemm(M, K, N, epilogue, splitk);
  // The prefill GEMM takes the row sums from the activation kernel, which
  // has them in registers anyway; the decode GEMM sums its own operand.
  int32_t* rowsum = pl.prefill ? (int32_t*)(ws + L.rowsum) : nullptr;
  const int rc = launch_act(x, M, K, ldx, gamma, norm_eps, xa, a_dq, rowsum, nullptr, xq_debug, nullptr,
                  pl.splitk > 1 ? (uint32_t*)(ws + L.gemm_ws) : nullptr, pl.splitk > 1 ? pl.ngroups : 0, s);
  if (rc) return rc;
  const GemmArgs g = gemm_args(xa, a_dq, rowsum, M, K, N, wdev, seg_scale, seg_end, nseg, epilogue, residual, out,
                               acc_out, ws + L.gemm_ws, pl);
  return launch_gemm(g, epilogue, pl, s);
}

}  // namespace btl

using namespace btl;

extern "C" {

int btl_gemm_tiling(int64_t M, int64_t K, int64_t N, int epilogue, int rowsum_given, int32_t* info) {
  if (!info) return set_error(BTL_ERR_NULL, "btl_gemm_tiling: info is NULL");
  if (M <= 0 || K <= 0 || N <= 0 || N % 32 || K % 32)
    return set_error(BTL_ERR_SHAPE, "btl_gemm_tiling: M=%lld K=%lld N=%lld", (long long)M, (long long)K, (long long)N);
  for (int i = 0; i < 6; ++i) info[i] = 0;
  WidePlan w;
  if (M <= 32) {
    const GemmPlan pl = plan_gemm(M, K, N, epilogue, 0);
    info[0] = 0, info[1] = 32, info[2] = pl.tpw, info[3] = pl.splitk;
  } else if (wide_plan(M, K, N, epilogue, rowsum_given != 0, &w)) {
    info[0] = 2, info[1] = 64, info[2] = w.ct, info[3] = 1, info[4] = w.wq, info[5] = w.ctw;
  } else {
    const PfGrid g = pf_grid(M, K, N, epilogue);
    info[0] = 1, info[1] = g.rb * 32, info[2] = kPfCT, info[3] = rowsum_given ? g.splitk : 1;
  }
  return BTL_OK;
}

int btl_choose_splitk(int64_t M, int64_t K, int64_t N, int epilogue) {
  if (M <= 0 || K <= 0 || N <= 0 || N % 32) return 0;
  return plan_gemm(M, K, N, epilogue, 0).splitk;
}

int64_t btl_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int epilogue, int splitk) {
  if (M <= 0 || K <= 0 || N <= 0 || N % 32) return 0;
  return plan_gemm(M, K, N, epilogue, splitk).ws_bytes;
}

int64_t btl_fused_error_offset(void) { return (int64_t)kErrorWord * kSyncStride * 4; }

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
  if (!xa || !a_dq) return set_error(BTL_ERR_NULL, "btl_gemm_i8t2: activation pointer is NULL");
  if (!aligned(xa, 16) || !aligned(a_dq, 4) || (rowsum && !aligned(rowsum, 4)) || (acc_out && !aligned(acc_out, 4)))
    return set_error(BTL_ERR_ALIGN, "btl_gemm_i8t2: misaligned activation, rowsum or acc_out buffer");
  if (splitk < 0) return set_error(BTL_ERR_ARG, "btl_gemm_i8t2: splitk=%d", splitk);
  const GemmPlan pl = plan_gemm(M, K, N, epilogue, splitk);
  if (pl.ws_bytes > 0) {
    if (!workspace) return set_error(BTL_ERR_NULL, "btl_gemm_i8t2: split-K needs a workspace");
    if ((int64_t)workspace_bytes < pl.ws_bytes)
      return set_error(BTL_ERR_WORKSPACE, "btl_gemm_i8t2: workspace %zu < %lld bytes", workspace_bytes,
                       (long long)pl.ws_bytes);
    if (!aligned(workspace, 256)) return set_error(BTL_ERR_ALIGN, "btl_gemm_i8t2: workspace must be 256-byte aligned");
  }
  const GemmArgs a = gemm_args(xa, a_dq, rowsum, M, K, N, wdev, seg_scale, seg_end, nseg, epilogue, residual, out,
                               acc_out, (char*)workspace, pl);
  return launch_gemm(a, epilogue, pl, (hipStream_t)stream);
}

int btl_bitlinear_fused(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma, float norm_eps,
                        const uint32_t* wdev, int64_t N, const float* seg_scale, const int64_t* seg_end, int nseg,
                        int epilogue, const uint16_t* residual, uint16_t* out, int32_t* acc_out, int8_t* xq_debug,
                        void* workspace, size_t workspace_bytes, int splitk, btl_stream_t stream) {
  clear_error();
  int rc = check_fused_args("btl_bitlinear_fused", x, M, K, ldx, gamma, wdev, N, seg_scale, seg_end, nseg, epilogue,
                            residual, out, acc_out, xq_debug, splitk);
  if (rc) return rc;
  if (!workspace) return set_error(BTL_ERR_NULL, "btl_bitlinear_fused: workspace is NULL");
  if (!aligned(workspace, 256)) return set_error(BTL_ERR_ALIGN, "btl_bitlinear_fused: workspace must be 256-byte aligned");
  const FusedLayout L = fused_layout(M, K, N, epilogue, splitk);
  if ((int64_t)workspace_bytes < L.total)
    return set_error(BTL_ERR_WORKSPACE, "btl_bitlinear_fused: workspace %zu < %lld bytes", workspace_bytes,
                     (long long)L.total);
  return bitlinear_fused_impl(x, M, K, ldx, gamma, norm_eps, wdev, N, seg_scale, seg_end, nseg, epilogue, residual,
                              out, acc_out, xq_debug, (char*)workspace, L, nullptr, splitk, stream);
}

int btl_bitlinear_fused_noalloc(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma,
                                float norm_eps, const uint32_t* wdev, int64_t N, const float* seg_scale,
                                const int64_t* seg_end, int nseg, int epilogue, const uint16_t* residual,
                                uint16_t* out, int32_t* acc_out, int8_t* xq_debug, uint32_t* error_word, int splitk,
                                btl_stream_t stream) {
  clear_error();
  int rc = check_fused_args("btl_bitlinear_fused_noalloc", x, M, K, ldx, gamma, wdev, N, seg_scale, seg_end, nseg,
                            epilogue, residual, out, acc_out, xq_debug, splitk);
  if (rc) return rc;
  if (error_word && !aligned(error_word, 4))
    return set_error(BTL_ERR_ALIGN, "btl_bitlinear_fused_noalloc: error_word must be 4-byte aligned");
  const FusedLayout L = fused_layout(M, K, N, epilogue, splitk);
  if (L.total > kNoAllocScratchBytes)
    return set_error(BTL_ERR_WORKSPACE,
                     "btl_bitlinear_fused_noalloc: M=%lld K=%lld N=%lld needs %lld bytes of scratch, more than the "
                     "library's static %lld (use btl_bitlinear_fused with a workspace)",
                     (long long)M, (long long)K, (long long)N, (long long)L.total, (long long)kNoAllocScratchBytes);
  char* ws = nullptr;
  rc = noalloc_scratch(&ws, (hipStream_t)stream);
  if (rc) return rc;
  return bitlinear_fused_impl(x, M, K, ldx, gamma, norm_eps, wdev, N, seg_scale, seg_end, nseg, epilogue, residual,
                              out, acc_out, xq_debug, ws, L, error_word, splitk, stream);
}

}  // extern "C"

BTL_TRACE_READ_FN(btl_trace_read_gemm)
