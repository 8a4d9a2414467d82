// The BitLinear portion of a whole batch-32 decode step of a BitNet b1.58
// model as one persistent launch on gfx950 (every layer's QKV, o_proj,
// gate||up and down; src/bitnet_tt/inference/generator_batch32.py:713-761).
//
// Roles.  One workgroup per CU, 512 threads.
//   Row workgroups 0..31: one token row each.  A row workgroup keeps its row
//     of the residual stream (hidden) in registers for the whole step and runs
//     every elementwise stage of that row: residual adds, RMSNorm, per-token
//     absmax int8 quantisation into the GEMM's operand tile, publication.
//   GEMM workgroups 32..: one unit (column tiles x row half) of each
//     BitLinear.  The weights of a unit are loaded into registers one
//     BitLinear ahead (while the GEMMs of the current one wait for their
//     operand tile), so no weight load is on the hand-off chain.
//   With the decode attention (the ATT instances, btl_decode_step_full), the
//     last M * Hkv GEMM workgroups also take one (user, key-value head)
//     attention item each per layer, between QKV and o_proj: they issue the
//     item's cached keys and values when they reach the layer, poll the
//     user's QKV words, run the attention body shared with
//     btl_decode_attention, and publish the heads' outputs as tagged words,
//     which the user's row workgroup polls for its o_proj stage.  QKV units
//     cover all 32 rows of two column tiles in these instances, so that at
//     the 2B shape no attention unit has QKV work.
//
// Per layer (BitLinear j = QKV, O, GU, DN):
//   row:  y = RMSNorm(h; input_layernorm) -> int8 tile[QKV]                 publish
//   GEMM: qkv = bf16(acc * s_seg * a)                       -> tagged words, qkv_out
//   row:  wait for row m of qkv (the attention of that user needs exactly it;
//         the BitLinear portion reads its output from the attention stand-in
//         buffer), y = RMSNorm(attn; attn_sub_norm) -> tile[O]               publish
//   GEMM: o = bf16(acc * s * a)                                -> tagged words
//   row:  h = bf16(h + o); y = RMSNorm(h; post_attention_layernorm) -> tile[GU]
//   GEMM: relu(g)^2 * u (gate tile and up tile in one unit)    -> tagged words, ffn_h
//   row:  y = RMSNorm(r; ffn_sub_norm) -> tile[DN]
//   GEMM: d = bf16(acc * s * a)                                -> tagged words
//   row:  h = bf16(h + d), next layer.
// The arithmetic is that of btl_bitlinear_fused (same row code, same epilogue
// expressions), so the step is bit-identical to the 120 single-BitLinear
// launches.
//
// Hand-offs (every one crosses XCDs; a coherent hop costs ~0.45 us each way):
//   row -> GEMM: the row's int8 operand bytes with device-coherent 8-byte
//     stores, then, without waiting for their acknowledgement, the row's flag
//     (one tagged word: a/127; the units sum the operand bytes they read for
//     the weight codes' offset themselves, so the row stage ends with no
//     reduction of its own).  A
//     GEMM unit polls the flags of its 16 (or 32) rows, then reads its operand
//     tile with L1-bypassing loads and checks it: between two uses every row
//     overwrites its slice of a tile with the sentinel byte 0x80, which no
//     quantised value takes (|q| <= 127), so operand bytes that have not landed
//     yet are recognised and read again.
//   GEMM -> row: 8-byte words holding two bf16 outputs and a 32-bit tag, each
//     one device-coherent store; the row workgroup polls the words it needs
//     (the data is its own flag: no acknowledgement wait, no flag hop).
// Tags and flags carry (launch epoch << 8 | layer*4 + BitLinear), the epoch
// being a per-workgroup launch counter kept in the workspace, so nothing is
// ever cleared.  Every wait is bounded: a wait that runs out sets the error
// word, and a workgroup that has seen an error stops waiting, so the launch
// always ends (with invalid outputs).
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "btl_act_row.h"
#include "btl_attn_body.h"
#include "btl_mfma.h"
#include "btl_trace.h"

namespace btl {

constexpr int kStepRows = 32;       // row workgroups (token rows)
constexpr int kStepWaves = 8;
constexpr int kStepPollWave = 7;    // the GEMM workgroup's wave that polls the row flags (then computes)
constexpr int kStepMaxGrid = 1024;
constexpr int kStepWSlots = 7;      // weight registers (16 B each) per wave and buffer
enum { S_QKV = 0, S_O = 1, S_GU = 2, S_DN = 3, kStepOps = 4 };

// Workspace: header, op table, then one hand-off region (operand tiles, row
// flags, tagged output words) that every layer reuses.  Reuse is safe by the
// dependency chain: row m clears (sentinel) and later overwrites its slice of
// tile j only after it has received all of its outputs of (l, j) -- and every
// unit that reads row m's slice of tile (l, j) or polls its flag writes row
// m's outputs of (l, j) only after those reads -- and a GEMM unit overwrites
// the tagged words of (l+1, j) only after every row it covers has published
// (l+1, j), which each row does after reading its words of (l, j).
//
// Operand tile layout.  A tile holds the A operands of the 32-row MFMA in
// 1 KiB blocks, one per 32-k step: row r's 16 bytes of k-group g (k 16 g ..
// 16 g + 15 of the step) at byte 32 r + 16 g of the block, so a 128-byte
// line holds 32 bytes of each of 4 rows.  A wave's operand load (a 16-byte
// piece per lane, of 32 rows or, in a 16-row unit, of 16 rows and two steps)
// reads whole lines, and a row's store of 64 chunks of 8 bytes writes 32
// bytes into each of 16 lines.  (The lane order of the MFMA operand itself,
// row l & 31 and k-group l >> 5 in lane l, would put 8 rows' 16-byte pieces
// in a line: every row store then fed twice the lines, and the row flags,
// which follow the stores to memory, landed 0.2-0.5 us later.)
//
// Operand tiles between uses.  Row m writes its slice of tile j for (l, j)
// (8-byte coherent stores, no acknowledgement wait).  Right after publishing
// (l, j + 1), when it has all of its outputs of (l, j), it clears a share of
// tile j to the sentinel in whole lines: 1/16 of the lines that hold its
// 16-row half's bytes (every unit of that half, 16-row or 32-row, has then
// read them).  Every row stage starts with a wait for all of the row's
// earlier memory operations (microseconds old by then, so it costs nothing),
// and the stage's barriers put every thread's wait before thread 0's flag,
// so a clear is performed before the row publishes anything later, and the
// next flag of tile j of every row of the same half causally follows it
// (through that half's units of the BitLinears in between, which wait for
// this row's flags).  A row of the other half may run ahead, but it never
// writes lines of this half.  A unit that has seen the flags of (l + 1, j)
// therefore reads, for every 8-byte piece, either the sentinel or the new
// bytes, never bytes of (l, j); seeing the sentinel it waits for the piece
// and reads again.  Tiles start
// (btl_decode_step_prepare) and end (the last row stage clears the last tile)
// every launch as the sentinel.
constexpr int64_t kStEpoch = 0;          // [kStepMaxGrid] u32
constexpr int64_t kStError = 4096;       // u32
constexpr int64_t kStTable = 8192;       // StepOp[L][4]
constexpr int kStepMaxLayers = 64;

struct StepOp {
  const uint32_t* wdev;
  const uint16_t* gamma;
  float seg_scale[BTL_MAX_SEGMENTS];
  int seg_end[BTL_MAX_SEGMENTS];
  int nseg;
  int pad[3];
};
static_assert(sizeof(StepOp) == 64, "op table entry");
// The KV caches of each layer (device addresses: key cache, value cache),
// for the instances that run the decode attention between QKV and o_proj
// (copied in by btl_decode_step_attention_prepare).
constexpr int64_t kStAttn = kStTable + (int64_t)kStepMaxLayers * kStepOps * sizeof(StepOp);
constexpr int64_t kStHeader = kStAttn + (int64_t)kStepMaxLayers * 16;

// GEMM unit shapes.  gate||up units cover all 32 rows (v_mfma_i32_32x32x32_i8:
// each unpacked weight dword feeds one MFMA) with a gate tile and its up
// tile.  QKV, o_proj and down run 16-row halves (v_mfma_i32_16x16x64_i8), so
// that a unit reads half of its operand tile: QKV with two adjacent column
// tiles per unit (its 120 tiles make 120 units), o_proj and down with one.
// With the decode attention (A = true) QKV units cover all 32 rows of two
// adjacent tiles (60 units at the 2B shape), so that the attention can run on
// units with no QKV work.  Every unit covers all of K and writes bf16 outputs
// (two per tagged word).
enum { MODE_SCALE = 0, MODE_RELU2 = 1 };
template <int J, bool A = false>
struct OpShape;
template <bool A>
struct OpShape<S_QKV, A> {
  static constexpr int TPW = 2, HALF = A ? 0 : 1, MODE = MODE_SCALE;
};
template <bool A>
struct OpShape<S_O, A> {
  static constexpr int TPW = 1, HALF = 1, MODE = MODE_SCALE;
};
template <bool A>
struct OpShape<S_GU, A> {
  static constexpr int TPW = 2, HALF = 0, MODE = MODE_RELU2;
};
template <bool A>
struct OpShape<S_DN, A> {
  static constexpr int TPW = 1, HALF = 1, MODE = MODE_SCALE;
};

struct StepArgs {
  const StepOp* ops;  // [L][4] (in the workspace)
  int L, M, H, F, NQKV;
  int KSH, KSF;       // superblocks of K = H and K = F
  float eps;
  const uint16_t* attn;  // [M][H] o_proj input (attention output stand-in)
  uint16_t* hidden;      // [M][H] in/out
  uint16_t* qkv_out;     // [M][NQKV]
  uint16_t* ffn_h;       // [M][F]
  uint32_t* epoch;
  uint32_t* error;
  char* layers;          // the hand-off region
  int64_t off_xa[kStepOps], off_flag, off_out[kStepOps];
  unsigned spin_limit;
  // Decode attention between QKV and o_proj (the ATT instances): per layer
  // the caches [M][Hkv][S][128] (kv: [L][2] in the workspace), each user's
  // position, the RoPE tables [S][64], the score scale; the attention output
  // goes to the rows as tagged words (off_att) and to the caller (attn_out).
  const uint64_t* kv;
  const int32_t* pos;
  const float* rcos;
  const float* rsin;
  uint16_t* attn_out;
  int64_t off_att;
  int Hkv, G, S, adjacent;
  float scale;
};

// Operand-tile byte between two uses: -128, which absmax quantisation never
// produces.  A 16-bit lane of an operand dword holding quantised bytes is
// >= -127 * 256 = -32512; one of a cleared 8-byte piece is 0x8080 = -32640.
constexpr uint32_t kTileSentinel = 0x80808080u;

__device__ __forceinline__ uint32_t step_tag(uint32_t E, int l, int j) { return (E << 8) | (uint32_t)(l * 4 + j); }

// Measurement builds (-DBTL_TRACE) time-stamp the phases of one layer.
#ifndef BTL_STEP_TRACE_LAYER
#define BTL_STEP_TRACE_LAYER 10
#endif
#define STEP_TRACE(l, ev)                              \
  do {                                                 \
    if ((l) == BTL_STEP_TRACE_LAYER) BTL_TRACE_AT(ev); \
  } while (0)

__device__ __forceinline__ char* layer_base(const StepArgs& p, int) { return p.layers; }
// Byte offset of chunk c (operand bytes 8c .. 8c + 7) of row m in a tile (the
// layout above): chunks 4i .. 4i + 3 of a row are 32 consecutive bytes of
// block i.
__host__ __device__ __forceinline__ int64_t tile_chunk_offset(int m, int c) {
  return (int64_t)(c >> 2) * 1024 + (m & 31) * 32 + (c & 3) * 8;
}
__device__ __forceinline__ int8_t* tile_of(const StepArgs& p, int l, int j) {
  return reinterpret_cast<int8_t*>(layer_base(p, l) + p.off_xa[j]);
}
// Row m's flag of (l, j), on its own 128-byte line: one word, tag << 32 | the
// bits of a/127.
__device__ __forceinline__ uint64_t* flag_of(const StepArgs& p, int l, int j, int m) {
  return reinterpret_cast<uint64_t*>(layer_base(p, l) + p.off_flag) + (j * 32 + m) * 16;
}
// Tagged output words of BitLinear j: bf16 pairs [32][N_out / 2].
__device__ __forceinline__ uint64_t* out_of(const StepArgs& p, int l, int j) {
  return reinterpret_cast<uint64_t*>(layer_base(p, l) + p.off_out[j]);
}
// Tagged words of the attention output (ATT instances): bf16 pairs [32][H / 2].
__device__ __forceinline__ uint64_t* att_of(const StepArgs& p) {
  return reinterpret_cast<uint64_t*>(p.layers + p.off_att);
}

// Loads of an operand tile.  Every layer reuses the tile's addresses, and a
// CU's L1 may still hold lines it read one layer earlier, so the loads are
// device-scope (sc1): they bypass the L1 and read the L2, which the rows'
// device-coherent stores keep current.  Lane offset in a VGPR, the rest in an
// SGPR.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const int8_t* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(base), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ v4i ld_tile(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 16));
}

__device__ __forceinline__ float op_seg_scale(const StepOp& op, int n) {
  float s = op.seg_scale[0];
#pragma unroll
  for (int i = 0; i + 1 < BTL_MAX_SEGMENTS; ++i)
    if (i + 1 < op.nseg && n >= op.seg_end[i]) s = op.seg_scale[i + 1];
  return s;
}

// Bounded wait state of a workgroup: once any wait anywhere ran out, the
// error word is set and waits end early.
struct WaitState {
  bool dead;
  bool reread;  // take the operand re-read path every time (set by a test through the workspace)
};
// The error word names the first wait that ran out: kind (1 row words, 2 row
// flags, 3 operand tile, 4 an attention unit's QKV words; 5: a user's
// position outside [0, S)) | (layer*4 + BitLinear) << 8 | workgroup << 16.
enum { WAIT_WORDS = 1, WAIT_FLAGS = 2, WAIT_TILE = 3, WAIT_ATT_WORDS = 4, BAD_POSITION = 5 };
__device__ __forceinline__ void set_error_word(const StepArgs& p, int kind, uint32_t want) {
  uint32_t expected = 0u;
  const uint32_t code = (uint32_t)kind | ((want & 0xffu) << 8) | (blockIdx.x << 16);
  __hip_atomic_compare_exchange_strong(p.error, &expected, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool should_stop(const StepArgs& p, unsigned n, WaitState& ws, int kind, uint32_t want) {
  if (n > p.spin_limit) {
    set_error_word(p, kind, want);
    ws.dead = true;
    return true;
  }
  if ((n & 255u) == 255u && ld_coherent(p.error) != 0u) {
    ws.dead = true;
    return true;
  }
  return false;
}

// ------------------------------------------------------------------ rows ----
// Chunk c = tid + 512 i of a row holds its elements 8c .. 8c + 7.

// Sleep between two polls of a bounded wait (s_sleep units of 64 clocks).
#ifndef BTL_STEP_POLL_SLEEP
#define BTL_STEP_POLL_SLEEP 1
#endif

// One poll round: this thread's words, all of them, unconditionally (a chunk
// past the row's end reads the last chunk, and nothing takes it), as 16-byte
// loads that bypass the L1, two words each.  A word is written by one 8-byte
// store (two bf16 outputs and their tag), and an aligned 16-byte load is one
// access to one cache line, so each word it returns is either the old or the
// new one, never a mix; the words of one load may differ in age, and each is
// taken only once its own tag shows.  Loads under per-word lane masks would
// let the register allocator reuse a destination before the round ends, and
// the wait that reuse needs would split the round into several memory round
// trips.
template <int C>
__device__ __forceinline__ void issue_words(const uint64_t* row, int nch, uint64_t (&d)[C][4]) {
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(row), (short)0, nch * 32, 0x00020000);
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = min(tid + kActThreads * i, nch - 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const v4i t = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, c * 32 + h * 16, 0, 16));
      d[i][2 * h] = (uint64_t)(uint32_t)t.x | ((uint64_t)(uint32_t)t.y << 32);
      d[i][2 * h + 1] = (uint64_t)(uint32_t)t.z | ((uint64_t)(uint32_t)t.w << 32);
    }
  }
}
// Takes the words of a round (issued for `pend`) that carry the tag.
template <int C>
__device__ __forceinline__ void take_words(const uint64_t (&d)[C][4], unsigned pend, uint32_t want, unsigned& pending,
                                           uint32_t (&pr)[C][4]) {
#pragma unroll
  for (int i = 0; i < C; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if ((pend & pending & (1u << (4 * i + k))) && (uint32_t)(d[i][k] >> 32) == want) {
        pr[i][k] = (uint32_t)d[i][k];
        pending &= ~(1u << (4 * i + k));
      }
}

// Waits for the tagged bf16-pair words of row m of an output with `ncols`
// columns and returns this thread's chunks as bf16 pairs (pr[i][0..3]).  Each
// thread polls its own words until each has shown the tag.  One round is in
// flight at a time (a second round in flight doubles the polling traffic, which
// slows the stores being waited for more than it speeds up their detection);
// every load of a round is issued before any tag of it is checked.
template <int C>
__device__ void wait_row_words(const StepArgs& p, const uint64_t* row, int ncols, uint32_t want, uint32_t (&pr)[C][4],
                               WaitState& ws) {
  const int tid = threadIdx.x;
  const int nch = ncols >> 3;
  unsigned pending = 0u;  // bit 4i + k: word k of chunk i still to read
#pragma unroll
  for (int i = 0; i < C; ++i) {
#pragma unroll
    for (int k = 0; k < 4; ++k) pr[i][k] = 0u;
    if (tid + kActThreads * i < nch) pending |= 0xFu << (4 * i);
  }
  if (!pending || ws.dead) return;
  unsigned n = 0;
  while (true) {
    uint64_t d[C][4];
    const unsigned pend = pending;
    issue_words<C>(row, nch, d);
    take_words<C>(d, pend, want, pending, pr);
    if (!pending || should_stop(p, ++n, ws, WAIT_WORDS, want)) break;
    __builtin_amdgcn_s_sleep(BTL_STEP_POLL_SLEEP);
  }
}

template <int C>
__device__ __forceinline__ void load_gain(const uint16_t* gamma, int nch, float (&g)[C][8]) {
  const int tid = threadIdx.x;
  uint4 raw[C];
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = tid + kActThreads * i;
    raw[i] = make_uint4(0u, 0u, 0u, 0u);
    if (c < nch) {
      const v4i t = ldg128(gamma + 8 * c);
      raw[i] = make_uint4((uint32_t)t.x, (uint32_t)t.y, (uint32_t)t.z, (uint32_t)t.w);
    }
  }
  gains_to_floats<C>(raw, g);
}

template <int C>
__device__ __forceinline__ void pairs_to_floats(const uint32_t (&pr)[C][4], float (&v)[C][8]) {
#pragma unroll
  for (int i = 0; i < C; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[i][2 * k] = bf2f((uint16_t)(pr[i][k] & 0xffffu));
      v[i][2 * k + 1] = bf2f((uint16_t)(pr[i][k] >> 16));
    }
}

// RMSNorm with gain g, absmax int8 quantisation into the tile of (l, j), then
// the row's flag (a/127), issued right behind the operand stores with no
// wait for their acknowledgement (a GEMM unit checks the bytes it
// reads against the sentinel).  Rows m >= M publish zeros.  The same row code
// as btl_bitlinear_fused.  K is a multiple of 128 (checked on the host), so
// the row's chunks fill its slice of the tile.
template <int C>
__device__ void publish_row(const StepArgs& p, int l, int j, int m, int K, float (&v)[C][8],
                            const float (&g)[C][8], uint32_t want, float* s_sum, float* s_max) {
  const int tid = threadIdx.x;
  const int nch = K >> 3;
  int8_t* xa = tile_of(p, l, j);
  float adq = 0.0f;
  int rs = 0;
  uint32_t qlo[C], qhi[C];
#pragma unroll
  for (int i = 0; i < C; ++i) qlo[i] = qhi[i] = 0u;
  if (m < p.M) {
    const float r = row_rms_inv<C>(v, nch, K, p.eps, tid, s_sum);
    row_apply_norm_f<C>(v, g, r, nch, tid);
    const float a = row_absmax<C>(v, nch, 1e-5f, tid, s_max);
    const float scale = 127.0f / a;
    adq = a / 127.0f;
#pragma unroll
    for (int i = 0; i < C; ++i)
      if (tid + kActThreads * i < nch) quant8(v[i], scale, qlo[i], qhi[i], rs);
  }
  (void)rs;  // the GEMM units sum the operand bytes they read
  // The operand bytes go out last: nothing after them in this stage reuses
  // their registers or waits on the vector-memory counter.
#pragma unroll
  for (int i = 0; i < C; ++i) {
    const int c = tid + kActThreads * i;
    if (c < nch) st_coherent(reinterpret_cast<uint64_t*>(xa + tile_chunk_offset(m, c)), (uint64_t)qlo[i] | ((uint64_t)qhi[i] << 32));
  }
  // Thread 0 sets the flag right behind its own operand stores, with no
  // barrier for the other waves' (a barrier there measured 1 % slower per
  // step): a unit that reads a piece before it lands sees the sentinel.  The
  // reductions' barriers above already order the tile clear that follows
  // after the threads that polled the row's words; a row past the batch
  // skips them, so it takes a barrier here instead.
  if (m >= p.M) lds_barrier();
  if (tid == 0) st_coherent(flag_of(p, l, j, m), ((uint64_t)want << 32) | __float_as_uint(adq));
}

// Row m's share of a tile back to the sentinel, in whole 128-byte lines (a
// wave's store instruction writes four full lines).  The share lies in lines
// that hold operand bytes of row m's 16-row half only: in each 1 KiB k-step
// block, lines 0-3 hold rows 0-15 and lines 4-7 rows 16-31.  The 16 rows of
// a half split their half's 16 KS lines into shares of KS lines (16 KS 8-byte
// pieces each), so the 32 shares cover the tile once.  Every clear being by half is what
// orders it before the tile's next write: the next write of those lines is
// by rows of the same half, and each of them publishes it only after
// receiving outputs of units of that half which waited for row m's flag of a
// later BitLinear (or, for gate||up, of units that waited for every row).
__host__ __device__ __forceinline__ int64_t clear_piece_offset(int m, int KS, int pc) {
  const int li = (m & 15) * KS + (pc >> 4);
  return (int64_t)(li >> 2) * 1024 + (m >> 4) * 512 + (li & 3) * 128 + (pc & 15) * 8;
}
template <int CP>
__device__ __forceinline__ void clear_tile_share(int8_t* xa, int m, int KS) {
  const int tid = threadIdx.x, npieces = KS * 16;
#pragma unroll
  for (int i = 0; i < CP; ++i) {
    const int pc = tid + kActThreads * i;
    if (pc < npieces)
      st_coherent(reinterpret_cast<uint64_t*>(xa + clear_piece_offset(m, KS, pc)),
                  ((uint64_t)kTileSentinel << 32) | kTileSentinel);
  }
}

// h = bf16(h + o) for this thread's chunk (one chunk per thread), o the
// BitLinear's bf16 outputs as pairs: the residual epilogue of
// btl_bitlinear_fused.
__device__ __forceinline__ void residual_add(uint32_t (&hid)[4], const uint32_t (&o)[4], bool live) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t s = f2bf_pair(bf_lo(hid[k]) + bf_lo(o[k]), bf_hi(hid[k]) + bf_hi(o[k]));
    hid[k] = live ? s : 0u;
  }
}

// CF: chunks per thread of a row of F (a row of H, and of the QKV output,
// is one chunk per thread: H, NQKV <= 4096).  Each stage: wait for the row's
// words of the previous BitLinear, then for every earlier memory operation of
// this thread (the last tile clear among them), publish, then clear the
// previous BitLinear's tile slice, whose readers are all done.
template <int CF, bool ATT>
__device__ void step_row(const StepArgs& p, const StepOp* sops, int m, uint32_t E, float* s_sum, float* s_max) {
  constexpr int CH = 1;
  const int tid = threadIdx.x;
  const bool live = m < p.M;
  const int nh = p.H >> 3, nf = p.F >> 3;
  WaitState ws{false, false};
  uint32_t hid[CH][4];
  {
    uint4 raw = make_uint4(0u, 0u, 0u, 0u);
    if (live && tid < nh) raw = *reinterpret_cast<const uint4*>(p.hidden + (int64_t)m * p.H + 8 * tid);
    hid[0][0] = raw.x;
    hid[0][1] = raw.y;
    hid[0][2] = raw.z;
    hid[0][3] = raw.w;
  }
  // gains of the next QKV stage: loaded ahead, during the wait before it
  float g_qkv[CH][8];
  load_gain<CH>(sops[S_QKV].gamma, nh, g_qkv);
  for (int l = 0; l < p.L; ++l) {
    const StepOp* ops = sops + l * kStepOps;
    // ---- QKV: RMSNorm(h; input_layernorm)
    {
      float v[CH][8];
      pairs_to_floats<CH>(hid, v);
      STEP_TRACE(l, 0);
      publish_row<CH>(p, l, S_QKV, m, p.H, v, g_qkv, step_tag(E, l, S_QKV), s_sum, s_max);
      STEP_TRACE(l, 1);
      if (l > 0) clear_tile_share<CF>(tile_of(p, l - 1, S_DN), m, p.KSF);
    }
    // ---- O: RMSNorm(attn; attn_sub_norm) of the user's attention output row
    {
      float g[CH][8];
      load_gain<CH>(ops[S_O].gamma, nh, g);
      uint32_t pr[CH][4];
      if (ATT) {
        // the row from the attention units of this user's key-value heads,
        // which read all of the user's QKV row first.  A row past the batch
        // has no attention units: it waits for its QKV row itself (the tile
        // clear below needs every QKV unit of its half done) and takes zeros.
        if (live) {
          wait_row_words<CH>(p, att_of(p) + (int64_t)m * (p.H >> 1), p.H, step_tag(E, l, 0), pr, ws);
        } else {
          wait_row_words<CH>(p, out_of(p, l, S_QKV) + (int64_t)m * (p.NQKV >> 1), p.NQKV, step_tag(E, l, S_QKV), pr,
                             ws);
#pragma unroll
          for (int k = 0; k < 4; ++k) pr[0][k] = 0u;
        }
        wait_memory();
        STEP_TRACE(l, 2);
      } else {
        // the attention output stand-in (an input of the step, loaded before
        // the wait) once the user's QKV row, which attention would read, is in
        uint4 raw = make_uint4(0u, 0u, 0u, 0u);
        if (live && tid < nh) raw = *reinterpret_cast<const uint4*>(p.attn + (int64_t)m * p.H + 8 * tid);
        wait_row_words<CH>(p, out_of(p, l, S_QKV) + (int64_t)m * (p.NQKV >> 1), p.NQKV, step_tag(E, l, S_QKV), pr,
                           ws);
        wait_memory();
        STEP_TRACE(l, 2);
        pr[0][0] = raw.x;
        pr[0][1] = raw.y;
        pr[0][2] = raw.z;
        pr[0][3] = raw.w;
      }
      float v[CH][8];
      pairs_to_floats<CH>(pr, v);
      publish_row<CH>(p, l, S_O, m, p.H, v, g, step_tag(E, l, S_O), s_sum, s_max);
      STEP_TRACE(l, 3);
      clear_tile_share<CH>(tile_of(p, l, S_QKV), m, p.KSH);
    }
    // ---- GU: h = bf16(h + o); RMSNorm(h; post_attention_layernorm)
    {
      float g[CH][8];
      load_gain<CH>(ops[S_GU].gamma, nh, g);
      uint32_t pr[CH][4];
      wait_row_words<CH>(p, out_of(p, l, S_O) + (int64_t)m * (p.H >> 1), p.H, step_tag(E, l, S_O), pr, ws);
      wait_memory();
      STEP_TRACE(l, 4);
      residual_add(hid[0], pr[0], live);
      float v[CH][8];
      pairs_to_floats<CH>(hid, v);
      publish_row<CH>(p, l, S_GU, m, p.H, v, g, step_tag(E, l, S_GU), s_sum, s_max);
      STEP_TRACE(l, 5);
      clear_tile_share<CH>(tile_of(p, l, S_O), m, p.KSH);
    }
    // ---- DN: RMSNorm(relu(g)^2 * u; ffn_sub_norm)
    {
      float g[CF][8];
      load_gain<CF>(ops[S_DN].gamma, nf, g);
      uint32_t pr[CF][4];
      wait_row_words<CF>(p, out_of(p, l, S_GU) + (int64_t)m * (p.F >> 1), p.F, step_tag(E, l, S_GU), pr, ws);
      wait_memory();
      STEP_TRACE(l, 6);
      float v[CF][8];
      pairs_to_floats<CF>(pr, v);
      publish_row<CF>(p, l, S_DN, m, p.F, v, g, step_tag(E, l, S_DN), s_sum, s_max);
      STEP_TRACE(l, 7);
      clear_tile_share<CH>(tile_of(p, l, S_GU), m, p.KSH);
    }
    // ---- h = bf16(h + d)
    {
      if (l + 1 < p.L) load_gain<CH>(sops[(l + 1) * kStepOps + S_QKV].gamma, nh, g_qkv);
      uint32_t pr[CH][4];
      wait_row_words<CH>(p, out_of(p, l, S_DN) + (int64_t)m * (p.H >> 1), p.H, step_tag(E, l, S_DN), pr, ws);
      wait_memory();
      residual_add(hid[0], pr[0], live);
    }
  }
  // The last tile back to the sentinel: every launch leaves all tiles so.
  // Threads with no output words of their own (tid >= H/8) skip the wait
  // above, so they must not clear before the threads that poll have all of
  // the row's words (every other clear sits behind publish_row's barriers).
  lds_barrier();
  clear_tile_share<CF>(tile_of(p, p.L - 1, S_DN), m, p.KSF);
  if (live && tid < nh)
    *reinterpret_cast<uint4*>(p.hidden + (int64_t)m * p.H + 8 * tid) =
        make_uint4(hid[0][0], hid[0][1], hid[0][2], hid[0][3]);
}

// ------------------------------------------------------------------ GEMM ----
__device__ __forceinline__ int op_n(const StepArgs& p, int j) {  // output columns of the GEMM
  return j == S_QKV ? p.NQKV : j == S_GU ? 2 * p.F : p.H;
}
__device__ __forceinline__ int op_ks(const StepArgs& p, int j) { return j == S_DN ? p.KSF : p.KSH; }
template <int J, bool A = false>
__device__ __forceinline__ int op_units(const StepArgs& p) {
  const int NT = op_n(p, J) / 32;
  return J == S_GU ? NT / 2 : OpShape<J, A>::HALF ? 2 * NT / OpShape<J, A>::TPW : NT / OpShape<J, A>::TPW;
}

// Unit u of BitLinear J: its first tile (GU: the gate tile; the up tile is
// F/32 further) and, for 16-row units, its row half h.  Units take groups of
// TPW adjacent tiles (GU: one gate/up pair); the two halves of a 16-row group
// are 8 workgroups apart, so round-robin dispatch puts them on one XCD and
// its L2 fetches their weights once.
template <int J, bool A = false>
__device__ __forceinline__ void unit_of(const StepArgs& p, int u, int& tile0, int& h) {
  const int NG = op_n(p, J) / 32 / (OpShape<J, A>::HALF ? OpShape<J, A>::TPW : 1);
  h = 0;
  if (!OpShape<J, A>::HALF) {
    tile0 = J == S_GU ? u : u * OpShape<J, A>::TPW;
    return;
  }
  const int g8 = NG & ~7;
  int g;
  if (u < 2 * g8) {
    g = ((u >> 4) << 3) | (u & 7);
    h = (u >> 3) & 1;
  } else {
    const int i = u - 2 * g8, rem = NG - g8;
    g = g8 + i % rem;
    h = i / rem;
  }
  tile0 = g * OpShape<J, A>::TPW;
}
template <int J>
__device__ __forceinline__ int unit_tile(const StepArgs& p, int tile0, int t) {
  if (J == S_GU) return t == 0 ? tile0 : tile0 + op_n(p, J) / 64;  // the up tile F/32 after the gate tile
  return tile0 + t;
}

// This wave's superblocks of [sb0, sb1): waves w and w + 4 share a SIMD, so
// the first (n % 8) waves take one more (0-3 before 4-7) and every SIMD gets
// the same share.
__device__ __forceinline__ void wave_ks(int sb0, int sb1, int wv, int& wb, int& we) {
  const int n = sb1 - sb0, base = n / kStepWaves, rem = n % kStepWaves;
  wb = sb0 + wv * base + (wv < rem ? wv : rem);
  we = wb + base + (wv < rem ? 1 : 0);
}

// Weights of this wave's superblocks of unit u of BitLinear J into w
// (slot t * NSW + i); slots past the wave's range re-read its last superblock.
// Every slot the BitLinear reads is written (zeros where the unit or wave has
// no work), so the buffer's previous contents are dead from here on and its
// registers free in between (the decode attention runs there).
template <int J, int NSW, bool A = false>
__device__ __forceinline__ void load_unit_weights(const StepArgs& p, const StepOp* sops, int l, int u,
                                                  v4i (&w)[kStepWSlots]) {
  static_assert(OpShape<J, A>::TPW * NSW <= kStepWSlots, "weight slots");
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int KS = op_ks(p, J);
  int tile0 = 0, h = 0, wb = 0, we = 0;
  const bool unit = u < op_units<J, A>(p);
  if (unit) {
    unit_of<J, A>(p, u, tile0, h);
    wave_ks(0, KS, wv, wb, we);
  }
  const bool work = unit && wb < we;
  const uint32_t* wdev = sops[l * kStepOps + J].wdev;
#pragma unroll
  for (int t = 0; t < OpShape<J, A>::TPW; ++t) {
    const int tile = unit_tile<J>(p, tile0, t);
#pragma unroll
    for (int i = 0; i < NSW; ++i) {
      const int sb = wb + i < we ? wb + i : we - 1;
      w[t * NSW + i] = work ? ldg128(wdev + (((int64_t)tile * KS + sb) * 64 + lane) * 4) : (v4i){0, 0, 0, 0};
    }
  }
}

// Poll wave: wait for the flags of rows [r0, r0 + n) of (l, j), n <= 32, lane
// r reading row r0 + r; the a/127 they carry go to s_adq[0 .. n).
__device__ void wait_flags(const StepArgs& p, int l, int j, int r0, int n, uint32_t want, float* s_adq,
                           WaitState& ws) {
  const int r = threadIdx.x & 63;
  const bool act = r < n;
  unsigned k = 0;
  uint64_t f = 0;
  while (!ws.dead) {
    if (act) f = ld_coherent(flag_of(p, l, j, r0 + r));
    const bool ok = !act || (uint32_t)(f >> 32) == want;
    if (__all(ok)) break;
    if (should_stop(p, ++k, ws, WAIT_FLAGS, want)) break;
    __builtin_amdgcn_s_sleep(BTL_STEP_POLL_SLEEP);
  }
  if (act) s_adq[r] = __uint_as_float((uint32_t)f);
}

// Running minimum of the operand dwords read, as signed 32-bit integers (one
// v_min3_i32 per 16-byte slot).  Dwords 0 and 2 of a slot each lie in one
// 8-byte piece, written (data or sentinel) by one 8-byte store.  A data
// dword's top byte is a quantised value, at least -127, so the dword is at
// least 0x81000000 as an integer; the sentinel dword 0x80808080 is below it.
__device__ __forceinline__ uint32_t slot_min(uint32_t mn, const v4i& a) {
  return (uint32_t)min(min((int)mn, a.x), a.z);
}
__device__ __forceinline__ bool slot_stale(uint32_t mn) { return (int)mn < (int)0x81000000u; }
// Rare path of an operand read that found the sentinel: polls the two 8-byte
// pieces of one 16-byte slot (dwords 0 and 2, 4-byte loads that bypass the L1)
// until neither is the sentinel, or the error word is set, or the wait runs
// out (which sets it).  The slot is then read again in full.  (Reading every
// operand again in one round instead, until none is the sentinel, keeps more
// registers live across the loop: the instance with the decode attention then
// spills, 914 against 873 us per step.)
__device__ __forceinline__ void wait_tile_piece(const StepArgs& p, __amdgpu_buffer_rsrc_t xa, int off, unsigned& n,
                                                WaitState& ws, uint32_t want) {
  while (!ws.dead) {
    const uint32_t d0 = __builtin_amdgcn_raw_buffer_load_b32(xa, off, 0, 16);
    const uint32_t d2 = __builtin_amdgcn_raw_buffer_load_b32(xa, off + 8, 0, 16);
    if (!slot_stale((uint32_t)min((int)d0, (int)d2))) break;
    if (++n > p.spin_limit) set_error_word(p, WAIT_TILE, want);
    if (n > p.spin_limit || ld_coherent(p.error) != 0u) {
      ws.dead = true;
      break;
    }
    __builtin_amdgcn_s_sleep(BTL_STEP_POLL_SLEEP);
  }
}
// One BitLinear J of layer l on GEMM workgroup gi: wait for the operand
// tile's rows, MFMA against the weights held in w, reduce the waves in LDS,
// epilogue (tagged bf16 pairs), then issue the next BitLinear's weights into wn.
// The packed weight words of a 16-row unit regrouped in place for
// v_mfma_i32_16x16x64_i8: a 32-lane and then a 16-lane swap of the words of
// 32-k steps 2p and 2p + 1 give lane l column (l & 15) (word 2p) and column
// 16 + (l & 15) (word 2p + 1), each with k-group l >> 4 of the 64-k step.
template <int TPW, int NSW>
__device__ __forceinline__ void regroup_half_weights(v4i (&w)[kStepWSlots]) {
#pragma unroll
  for (int s = 0; s < TPW * NSW; ++s)
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const auto s32 = __builtin_amdgcn_permlane32_swap((uint32_t)w[s][2 * pp], (uint32_t)w[s][2 * pp + 1], false,
                                                        false);
      const auto s16 = __builtin_amdgcn_permlane16_swap(s32[0], s32[1], false, false);
      w[s][2 * pp] = (int)s16[0];
      w[s][2 * pp + 1] = (int)s16[1];
    }
}

template <int J, int NSW, int NJ, int NNSW, bool A>
__device__ void step_gemm_op(const StepArgs& p, const StepOp* sops, int l, int gi, uint32_t E,
                             v4i (&w)[kStepWSlots], v4i (&wn)[kStepWSlots], int nl, int32_t* lds,
                             WaitState& ws) {
  constexpr int TPW = OpShape<J, A>::TPW, MODE = OpShape<J, A>::MODE;
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (gi >= op_units<J, A>(p)) {
    if (nl < p.L) load_unit_weights<NJ, NNSW, A>(p, sops, nl, gi, wn);
    return;
  }
  const StepOp& op = sops[l * kStepOps + J];
  int tile0, h, wb, we;
  unit_of<J, A>(p, gi, tile0, h);
  wave_ks(0, op_ks(p, J), wv, wb, we);
  const int cnt = we - wb;
  const uint32_t want = step_tag(E, l, J);
  int32_t* red = lds;                                // reductions
  float* s_adq = reinterpret_cast<float*>(lds + kStepWaves * 2 * 16 * 64);  // [32] a/127 from the flags
  constexpr int NR = OpShape<J, A>::HALF ? 16 : 32;  // rows of the unit
  // A 16-row unit's weight words are regrouped for its MFMA before the flags
  // are awaited (they were loaded during the previous hand-off).
  if constexpr (OpShape<J, A>::HALF) regroup_half_weights<TPW, NSW>(w);
  if (wv == kStepPollWave) wait_flags(p, l, J, 16 * h, NR, want, s_adq, ws);
  lds_barrier();  // the rows' flags are in (no wait for loads in flight)
  STEP_TRACE(l, 8 + 2 * J);
  const __amdgpu_buffer_rsrc_t xa = tile_rsrc(tile_of(p, l, J), 32 * op_ks(p, J) * 128);
  uint64_t* outw = out_of(p, l, J);
  const int n_out = J == S_QKV ? p.NQKV : J == S_GU ? p.F : p.H;

  if constexpr (OpShape<J, A>::HALF) {
    // ---- rows 16h .. 16h + 15 on v_mfma_i32_16x16x64_i8, two MFMAs (columns
    // 0-15, 16-31) per 64 k.  A: lane l takes row 16h + (l & 15), k-group l >> 4
    // of the 64-k step straight from the tile (32-k step 2p + (G >> 1), half
    // G & 1).  B: the regrouped packed words 2p and 2p + 1 (columns 0-15 and
    // 16-31).  C: lane l, element j is row 4 (l >> 4) + j, column l & 15.
    const int er = tid >> 5, ec = tid & 31;
    const int row = 16 * h + er;
    float sc[TPW];  // LDS reads, early: off the epilogue's path
#pragma unroll
    for (int t = 0; t < TPW; ++t) sc[t] = op_seg_scale(op, unit_tile<J>(p, tile0, t) * 32 + ec);
    const float ad = s_adq[er];
    // lane l: row 16h + (l & 15), k-group (l >> 4) & 1 of 32-k step 2p + (l >> 5)
    const int a_voff = (lane >> 5) * 1024 + (16 * h + (lane & 15)) * 32 + ((lane >> 4) & 1) * 16;
    // Operand loads, then the MFMAs as the data arrives, each operand's
    // 16-bit lanes folded into a running minimum on the way.  A piece that
    // still held the sentinel had not landed: then (rarely) the wave waits for
    // its pieces, reads them and its weights again, and redoes the MFMAs.
    // One more MFMA per operand, against all-ones bytes, gives the wave's
    // share of each row's sum of quantised values in every column of
    // acc_rs (the weight codes are value + 1); the body waits on its 2-bit
    // unpack on the VALU more than on the MFMAs, so this one runs in their
    // shadow.
    v4i a[NSW][2];
    // Every wave issues NSW superblocks of loads (one past its range reads the
    // tile's first 16 bytes in every lane, one line), so all waves count the
    // same loads and each MFMA waits only for its own operands.
    auto load = [&]() {
#pragma unroll
      for (int i = 0; i < NSW; ++i) {
        const bool mine = i < cnt;
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
          a[i][pp] = ld_tile(xa, mine ? a_voff : 0, mine ? ((wb + i) * 4 + 2 * pp) * 1024 : 0);
        __builtin_amdgcn_sched_barrier(0);  // superblocks in order: the first MFMAs wait for the first loads
      }
    };
    v4i acc[TPW][2], acc_rs;
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    auto mfma = [&](const v4i (&ww)[kStepWSlots]) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) acc[t][0] = acc[t][1] = (v4i){0, 0, 0, 0};
      acc_rs = (v4i){0, 0, 0, 0};
      uint32_t mn = 0x7fffffffu;
#pragma unroll
      for (int i = 0; i < NSW; ++i)
        if (i < cnt)
#pragma unroll
          for (int pp = 0; pp < 2; ++pp) {
            mn = slot_min(mn, a[i][pp]);
            acc_rs = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][pp], ones, acc_rs, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < TPW; ++t) {
              const v4i& g = ww[t * NSW + i];
              acc[t][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][pp], unpack_b((uint32_t)g[2 * pp]), acc[t][0],
                                                                0, 0, 0);
              acc[t][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][pp], unpack_b((uint32_t)g[2 * pp + 1]),
                                                                acc[t][1], 0, 0, 0);
            }
          }
      return mn;
    };
    load();
    if (__any(slot_stale(mfma(w))) || ws.reread) {
      unsigned tries = 0;
      for (int i = 0; i < cnt; ++i)
        for (int pp = 0; pp < 2; ++pp)
          wait_tile_piece(p, xa, a_voff + ((wb + i) * 4 + 2 * pp) * 1024, tries, ws, want);
      load();
      v4i wr[kStepWSlots];
      load_unit_weights<J, NSW, A>(p, sops, l, gi, wr);
      regroup_half_weights<TPW, NSW>(wr);
      (void)mfma(wr);
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        red[((wv * TPW + t) * 8 + q) * 64 + lane] = acc[t][0][q] - acc_rs[q];
        red[((wv * TPW + t) * 8 + 4 + q) * 64 + lane] = acc[t][1][q] - acc_rs[q];
      }
    lds_barrier();
    const int reg = 4 * (ec >> 4) + (er & 3), src = 16 * (er >> 2) + (ec & 15);
    int32_t sum[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      sum[t] = 0;
#pragma unroll
      for (int v2 = 0; v2 < kStepWaves; ++v2) sum[t] += red[((v2 * TPW + t) * 8 + reg) * 64 + src];
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int n = unit_tile<J>(p, tile0, t) * 32 + ec;
      const uint32_t o = f2bf((float)sum[t] * (sc[t] * ad));
      const uint32_t pair = o | (xor_partner_u<1>(o) << 16);  // lanes ec, ec+1 share the row (a DPP swap)
      if ((ec & 1) == 0) {
        st_coherent(outw + (int64_t)row * (n_out >> 1) + (n >> 1), ((uint64_t)want << 32) | pair);
        if (J == S_QKV && row < p.M) *reinterpret_cast<uint32_t*>(p.qkv_out + (int64_t)row * p.NQKV + n) = pair;
      }
    }
    // LDS free for the next BitLinear; the barrier after the stores keeps
    // them ahead of every wave's next weight loads (1 % faster per step than
    // the stores after it)
    lds_barrier();
  } else {
    // ---- all 32 rows on v_mfma_i32_32x32x32_i8 ----
    const int jc = lane & 31;
    // segment scales: LDS reads of the op table, issued early, off the epilogue's path
    const float sc0 = op_seg_scale(op, tile0 * 32 + jc);
    const float sc1 = TPW == 1 ? sc0 : op_seg_scale(op, unit_tile<J>(p, tile0, 1) * 32 + jc);
    float ad_r[2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) ad_r[rr] = s_adq[acc_row(wv + kStepWaves * rr, lane)];
    // Operand loads, MFMAs with the sentinel fold, and the rare re-read, as
    // in the 16-row body, and the row sums from an MFMA against all-ones
    // bytes as there (v_dot4 on the operand bytes instead, on the VALU that
    // the unpack already keeps busy, measured 1 % slower per step).  Lane l:
    // row l & 31, k-group l >> 5.
    const int a_voff = (lane & 31) * 32 + (lane >> 5) * 16;
    v4i a[NSW][4];
    auto load = [&]() {  // NSW superblocks in every wave, as in the 16-row body
#pragma unroll
      for (int i = 0; i < NSW; ++i) {
        const bool mine = i < cnt;
#pragma unroll
        for (int q = 0; q < 4; ++q) a[i][q] = ld_tile(xa, mine ? a_voff : 0, mine ? ((wb + i) * 4 + q) * 1024 : 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    v16i acc[TPW], acc_rs;
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    auto mfma = [&](const v4i (&ww)[kStepWSlots]) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) acc[t] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
      acc_rs = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
      uint32_t mn = 0x7fffffffu;
#pragma unroll
      for (int i = 0; i < NSW; ++i)
        if (i < cnt)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            mn = slot_min(mn, a[i][q]);
            acc_rs = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i][q], ones, acc_rs, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < TPW; ++t)
              acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i][q], unpack_b((uint32_t)ww[t * NSW + i][q]), acc[t],
                                                             0, 0, 0);
          }
      return mn;
    };
    load();
    if (__any(slot_stale(mfma(w))) || ws.reread) {
      unsigned tries = 0;
      for (int i = 0; i < cnt; ++i)
        for (int q = 0; q < 4; ++q) wait_tile_piece(p, xa, a_voff + ((wb + i) * 4 + q) * 1024, tries, ws, want);
      load();
      v4i wr[kStepWSlots];
      load_unit_weights<J, NSW, A>(p, sops, l, gi, wr);
      (void)mfma(wr);
    }
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((wv * TPW + t) * 16 + r) * 64 + lane] = acc[t][r] - acc_rs[r];
    lds_barrier();
    // thread (wv, lane) finishes rows acc_row(wv + 8 rr, lane), column lane & 31, of every tile
    int32_t v[TPW][2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int r = wv + kStepWaves * rr;
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        int32_t sum = 0;
#pragma unroll
        for (int v2 = 0; v2 < kStepWaves; ++v2) sum += red[((v2 * TPW + t) * 16 + r) * 64 + lane];
        v[t][rr] = sum;
      }
    }
    // Every load of this BitLinear has been consumed; settling the counter
    // here, before the first store, keeps the compiler from placing a wait
    // (for the stores' acknowledgements too) between the two rows' stores.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int i = acc_row(wv + kStepWaves * rr, lane);
      // scale mode: one output per tile; relu2 mode: one from the gate/up pair
      constexpr int NO = MODE == MODE_SCALE ? TPW : 1;
#pragma unroll
      for (int t = 0; t < NO; ++t) {
        const int n = unit_tile<J>(p, tile0, t) * 32 + jc;
        uint32_t o;
        if (MODE == MODE_SCALE) {
          o = f2bf((float)v[t][rr] * ((t == 0 ? sc0 : sc1) * ad_r[rr]));
        } else {
          const float gg = bf2f(f2bf((float)v[0][rr] * (sc0 * ad_r[rr])));
          const float uu = bf2f(f2bf((float)v[TPW - 1][rr] * (sc1 * ad_r[rr])));
          const float gr = gg > 0.0f ? gg : 0.0f;
          const float sq = bf2f(f2bf(gr * gr));
          o = f2bf(sq * uu);
        }
        const uint32_t pair = o | (xor_partner_u<1>(o) << 16);  // lanes jc, jc+1 share the row (a DPP swap)
        if ((jc & 1) == 0) {
          st_coherent(outw + (int64_t)i * (n_out >> 1) + (n >> 1), ((uint64_t)want << 32) | pair);
          // the caller's copy: the same pair as one 4-byte store
          if (J == S_QKV && i < p.M) *reinterpret_cast<uint32_t*>(p.qkv_out + (int64_t)i * p.NQKV + n) = pair;
          if (J == S_GU && i < p.M) *reinterpret_cast<uint32_t*>(p.ffn_h + (int64_t)i * p.F + n) = pair;
        }
      }
    }
    // LDS free for the next BitLinear.  The barrier also keeps every wave's
    // output stores ahead of any wave's loads of the next weights in the CU's
    // memory pipeline (two reduction areas without it measured 1 % slower;
    // the barrier before the stores instead of after them, 0.2 %).
    lds_barrier();
  }
  STEP_TRACE(l, 9 + 2 * J);
  // The next BitLinear's weights, issued after this one's last wait: its
  // hand-off takes longer than the loads, and no wait here covers them.
  if (nl < p.L) load_unit_weights<NJ, NNSW, A>(p, sops, nl, gi, wn);
}

// ------------------------------------------------------------ attention ----
// LDS words of the attention instances' GEMM workgroups, above the attention's
// LDS: the unit index (read back each layer) and a zero (read by the attention).
constexpr int kStepIdxInt = 20400;
// Decode attention of user b = ai / Hkv and key-value head hk = ai % Hkv (ATT
// instances; src/bitnet_tt/inference/generator_batch32.py:728-746), item ai of
// the layer, run by a GEMM workgroup between its QKV and o_proj units.  The
// first round of the pair's cached keys and values does not depend on this
// step, so its loads are issued first; then the new token's rows (the group's G query heads, its
// key and value head) come in as row b's tagged QKV output words, and the
// body shared with btl_decode_attention runs on the workgroup (the same code,
// so the same bits).  Its G x 128 outputs leave as tagged bf16 pairs, which
// row b's workgroup polls for its o_proj stage, and as the caller's copy.
__device__ void step_attention(const StepArgs& p, int l, int ai, uint32_t E, int32_t* lds, WaitState& ws) {
  if (ai < 0 || ai >= p.M * p.Hkv) return;
  const int tid = threadIdx.x;
  AttnSmem& s = *reinterpret_cast<AttnSmem*>(lds);
  AttnPair a;
  a.rcos = p.rcos;
  a.rsin = p.rsin;
  a.kc = reinterpret_cast<uint16_t*>(p.kv[2 * l]);
  a.vc = reinterpret_cast<uint16_t*>(p.kv[2 * l + 1]);
  a.Hkv = p.Hkv;
  a.G = p.G;
  a.S = p.S;
  a.b = ai / p.Hkv;
  a.hk = ai % p.Hkv;
  a.pos = p.pos[a.b];
  a.scale = p.scale;
  a.adjacent = p.adjacent;
  // the thread index plus a zero read back from LDS on every call: the body's
  // per-lane values are recomputed in each layer rather than kept (spilled)
  // across the layer loop
  a.tid = tid + *reinterpret_cast<volatile int32_t*>(lds + kStepIdxInt + 1);
  if (!a.pos_ok() && tid == 0) set_error_word(p, BAD_POSITION, (uint32_t)(l * 4 + S_O));
  AttnRound r;
  att_load_round(a, 0, r);
  STEP_TRACE(l, 0);
  // the new rows: thread t < 6 x 64 takes word t % 64 (two values) of row
  // segment t / 64 (query rows 0..G-1, the key row at kAtMaxG, the value row
  // at kAtMaxG + 1)
  const uint32_t want = step_tag(E, l, S_QKV);
  const uint64_t* row = out_of(p, l, S_QKV) + (int64_t)a.b * (p.NQKV >> 1);
  const int Hq = p.G * p.Hkv;
  if (tid < (kAtMaxG + 2) * (kAtD / 2)) {
    const int u = tid / (kAtD / 2), w = tid % (kAtD / 2);
    if (u >= kAtMaxG || u < p.G) {
      const int head = u < kAtMaxG ? a.hk * p.G + u : u == kAtMaxG ? Hq + a.hk : Hq + p.Hkv + a.hk;
      const uint64_t* wp = row + head * (kAtD / 2) + w;
      unsigned n = 0;
      uint64_t v = 0;
      while (!ws.dead) {
        v = ld_coherent(wp);
        if ((uint32_t)(v >> 32) == want) break;
        if (should_stop(p, ++n, ws, WAIT_ATT_WORDS, want)) break;
        __builtin_amdgcn_s_sleep(BTL_STEP_POLL_SLEEP);
      }
      *reinterpret_cast<uint32_t*>(&s.in[u][2 * w]) = (uint32_t)v;
    }
  }
  lds_barrier();  // the new rows are in LDS (the cache loads stay in flight)
  STEP_TRACE(l, 1);
  const uint32_t o = att_body(a, s, r, l == BTL_STEP_TRACE_LAYER);
  const uint32_t pair = o | (xor_partner_u<1>(o) << 16);  // dims d, d + 1 of a head (a DPP lane swap)
  if (tid < p.G * kAtD && (tid & 1) == 0) {
    const int col = a.hk * p.G * kAtD + tid;  // heads hk G + tid / 128, dimension tid % 128
    st_coherent(att_of(p) + (int64_t)a.b * (p.H >> 1) + (col >> 1), ((uint64_t)step_tag(E, l, 0) << 32) | pair);
    *reinterpret_cast<uint32_t*>(p.attn_out + (int64_t)a.b * p.H + col) = pair;
  }
  STEP_TRACE(l, 7);
  lds_barrier();  // the LDS is the next BitLinear's again
}


// The first GEMM unit with an attention item: the items take the last M * Hkv
// units, which at the 2B shape (160 items, 60 QKV units of 224) have no QKV
// work, so each issues its cached keys and values at the start of the layer.
__device__ __forceinline__ int step_first_att(const StepArgs& p) {
  return (int)gridDim.x - kStepRows - p.M * p.Hkv;
}

// NQ: superblocks per wave of a unit of QKV, O and GU (K = H); NDN: of DN (K = F).
template <int NQ, int NDN, bool ATT>
__device__ void step_gemm(const StepArgs& p, const StepOp* sops, int gi, uint32_t E, int32_t* lds) {
  // Word kStError + 64 of the workspace: bit 0 makes every GEMM unit take the
  // re-read path of its sentinel check (a test of that rare path; the results
  // are the same bits).
  WaitState ws{false, (__builtin_amdgcn_readfirstlane(p.error[16]) & 1u) != 0u};
  v4i wa[kStepWSlots], wb[kStepWSlots];
  load_unit_weights<S_QKV, NQ, ATT>(p, sops, 0, gi, wa);
  if (threadIdx.x == 0) {
    lds[kStepIdxInt] = gi;
    lds[kStepIdxInt + 1] = 0;  // the attention body's opaque zero
  }
  lds_barrier();
  for (int l = 0; l < p.L; ++l) {
    // The unit index is read back from LDS each layer (a value the compiler
    // cannot see through), so that the per-unit offsets derived from it are
    // recomputed (a few scalar and VALU operations) rather than kept live
    // across the layer loop: 194 VGPRs instead of 225 without the attention
    // (702 -> 690 us per step), and room for the attention body with it.
    gi = __builtin_amdgcn_readfirstlane(*reinterpret_cast<volatile int32_t*>(lds + kStepIdxInt));
    // An attention unit loads its o_proj weights after the attention (whose
    // key and value rows take the registers meanwhile): o_proj's operands
    // arrive microseconds later, through the rows' o_proj stage.
    const int ai = ATT ? gi - step_first_att(p) : -1;
    const bool att_unit = ai >= 0;
    step_gemm_op<S_QKV, NQ, S_O, NQ, ATT>(p, sops, l, gi, E, wa, wb, att_unit ? p.L : l, lds, ws);
    if (att_unit) {
      step_attention(p, l, ai, E, lds, ws);
      load_unit_weights<S_O, NQ, ATT>(p, sops, l, gi, wb);
    }
    step_gemm_op<S_O, NQ, S_GU, NQ, ATT>(p, sops, l, gi, E, wb, wa, l, lds, ws);
    step_gemm_op<S_GU, NQ, S_DN, NDN, ATT>(p, sops, l, gi, E, wa, wb, l, lds, ws);
    step_gemm_op<S_DN, NDN, S_QKV, NQ, ATT>(p, sops, l, gi, E, wb, wa, l + 1, lds, ws);
  }
}

template <int CF, int NQ, int NDN, bool ATT>
__global__ __launch_bounds__(512) void k_decode_step(StepArgs p) {
  // GEMM: reductions [8][2][16][64] int32 and 32 a/127; rows: 16 words.  The op table
  // (up to 16 KiB) is copied into LDS above them, so reading a weight address or a
  // scale is an LDS read, never a vector memory load waited for with the weight
  // stream.  96 KiB in all: more than half of a CU's LDS, so no CU ever holds two
  // workgroups of the launch.
  __shared__ __attribute__((aligned(16))) int32_t lds[24576];
  constexpr int kTableInts = kStepMaxLayers * kStepOps * (int)sizeof(StepOp) / 4;
  static_assert(kStepWaves * 2 * 16 * 64 + 32 + kTableInts <= 24576 && kStepWaves * 2 * 16 * 64 + 32 <= kStepIdxInt,
                "LDS layout");
  static_assert(sizeof(AttnSmem) <= (24576 - kTableInts) * 4, "the attention body's LDS below the op table");
  static_assert(kStepIdxInt * 4 >= (int)sizeof(AttnSmem) && kStepIdxInt + 2 <= 24576 - kTableInts,
                "the unit index and zero words between the attention's LDS and the op table");
  StepOp* sops = reinterpret_cast<StepOp*>(lds + (24576 - kTableInts));
  {
    const uint4* src = reinterpret_cast<const uint4*>(p.ops);
    uint4* dst = reinterpret_cast<uint4*>(sops);
    const int n16 = p.L * kStepOps * (int)sizeof(StepOp) / 16;
    for (int i = threadIdx.x; i < n16; i += blockDim.x) dst[i] = src[i];
  }
  __syncthreads();
  const int b = blockIdx.x;
  const uint32_t E = p.epoch[b] + 1u;  // this launch (written by the previous launch of the step)
  if (b < kStepRows) {
    float* f = reinterpret_cast<float*>(lds);
    step_row<CF, ATT>(p, sops, b, E, f, f + kActWaves);
  } else {
    step_gemm<NQ, NDN, ATT>(p, sops, b - kStepRows, E, lds);
  }
  if (threadIdx.x == 0) p.epoch[b] = E;
}

// ------------------------------------------------------- hand-off floor ----
// The step's launch structure with no arithmetic, for measurement: per
// BitLinear the row workgroups wait for every word of their row of the
// previous BitLinear's output (as the step does), then set their flag; each
// GEMM unit waits for its rows' flags (as the step does), then writes its
// tagged words (zero payload) in the step's store pattern.  No weight,
// operand tile, gain or norm is touched and nothing is computed, so its time
// is the latency floor that the chain of 120 dependent hand-off pairs sets.
template <int CF>
__device__ void floor_row(const StepArgs& p, int m, uint32_t E) {
  WaitState ws{false, false};
  for (int l = 0; l < p.L; ++l)
    for (int j = 0; j < kStepOps; ++j) {
      if (l > 0 || j > 0) {  // the words this row stage waits for in the step
        const int pj = j > 0 ? j - 1 : S_DN, pl = j > 0 ? l : l - 1;
        const int ncols = pj == S_QKV ? p.NQKV : pj == S_GU ? p.F : p.H;
        uint32_t pr[CF][4];
        if (pj == S_GU)
          wait_row_words<CF>(p, out_of(p, pl, pj) + (int64_t)m * (ncols >> 1), ncols, step_tag(E, pl, pj), pr, ws);
        else
          wait_row_words<1>(p, out_of(p, pl, pj) + (int64_t)m * (ncols >> 1), ncols, step_tag(E, pl, pj),
                            reinterpret_cast<uint32_t(&)[1][4]>(pr), ws);
      }
      __syncthreads();
      if (threadIdx.x == 0) st_coherent(flag_of(p, l, j, m), (uint64_t)step_tag(E, l, j) << 32);
    }
  uint32_t pr[1][4];  // the last down projection's words end the row's step
  wait_row_words<1>(p, out_of(p, p.L - 1, S_DN) + (int64_t)m * (p.H >> 1), p.H, step_tag(E, p.L - 1, S_DN), pr, ws);
}

template <int J>
__device__ __forceinline__ void floor_gemm_op(const StepArgs& p, int l, int gi, uint32_t E, float* s_adq,
                                              WaitState& ws) {
  if (gi >= op_units<J>(p)) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  int tile0, h;
  unit_of<J>(p, gi, tile0, h);
  const uint32_t want = step_tag(E, l, J);
  constexpr int NR = OpShape<J>::HALF ? 16 : 32;
  if (wv == kStepPollWave) wait_flags(p, l, J, 16 * h, NR, want, s_adq, ws);
  lds_barrier();
  uint64_t* outw = out_of(p, l, J);
  const int n_out = J == S_QKV ? p.NQKV : J == S_GU ? p.F : p.H;
  if constexpr (OpShape<J>::HALF) {
    const int er = tid >> 5, ec = tid & 31, row = 16 * h + er;
#pragma unroll
    for (int t = 0; t < OpShape<J>::TPW; ++t) {
      const int n = unit_tile<J>(p, tile0, t) * 32 + ec;
      if ((ec & 1) == 0) st_coherent(outw + (int64_t)row * (n_out >> 1) + (n >> 1), (uint64_t)want << 32);
    }
  } else {
    const int jc = lane & 31, n = tile0 * 32 + jc;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int i = acc_row(wv + kStepWaves * rr, lane);
      if ((jc & 1) == 0) st_coherent(outw + (int64_t)i * (n_out >> 1) + (n >> 1), (uint64_t)want << 32);
    }
  }
}

template <int CF>
__global__ __launch_bounds__(512) void k_decode_step_floor(StepArgs p) {
  __shared__ float s_adq[32];
  const int b = blockIdx.x;
  const uint32_t E = p.epoch[b] + 1u;
  if (b < kStepRows) {
    floor_row<CF>(p, b, E);
  } else {
    WaitState ws{false, false};
    for (int l = 0; l < p.L; ++l) {
      floor_gemm_op<S_QKV>(p, l, b - kStepRows, E, s_adq, ws);
      floor_gemm_op<S_O>(p, l, b - kStepRows, E, s_adq, ws);
      floor_gemm_op<S_GU>(p, l, b - kStepRows, E, s_adq, ws);
      floor_gemm_op<S_DN>(p, l, b - kStepRows, E, s_adq, ws);
    }
  }
  if (threadIdx.x == 0) p.epoch[b] = E;
}

// ---------------------------------------------------------------- host ----
struct StepSizes {
  int64_t off_xa[kStepOps], tiles_end, off_flag, off_out[kStepOps], off_att, layer_bytes, total;
};

static StepSizes step_sizes(int64_t H, int64_t F, int64_t NQKV) {
  StepSizes z;
  const int64_t Ks[kStepOps] = {H, H, H, F};
  // tagged words (bf16 pairs) a row workgroup reads back
  const int64_t words[kStepOps] = {NQKV / 2, H / 2, F / 2, H / 2};
  int64_t off = 0;
  for (int j = 0; j < kStepOps; ++j) {
    z.off_xa[j] = off;
    off += round_up(32 * ksb(Ks[j]) * 128, 4096);
  }
  z.tiles_end = off;
  z.off_flag = off;
  off += kStepOps * 32 * 128;
  for (int j = 0; j < kStepOps; ++j) {
    z.off_out[j] = off;
    off += round_up(32 * words[j] * 8, 4096);
  }
  z.off_att = off;  // the attention output's tagged words (ATT instances)
  off += round_up(32 * (H / 2) * 8, 4096);
  z.layer_bytes = round_up(off, 65536);
  z.total = kStHeader + z.layer_bytes;
  return z;
}

static int step_grid() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

// The step's instance for F (the down projection's row chunks per thread),
// with or without the decode attention.
static void (*step_kernel_fn(int64_t F, bool att))(StepArgs) {
  const int cf = act_cpt(F);
  if (cf == 1) return att ? k_decode_step<1, 3, 7, true> : k_decode_step<1, 3, 7, false>;
  if (cf == 2) return att ? k_decode_step<2, 3, 7, true> : k_decode_step<2, 3, 7, false>;
  return nullptr;
}
static const void* step_kernel(int64_t F, bool floor, bool att = false) {
  const int cf = act_cpt(F);
  if (floor) return cf == 1 ? reinterpret_cast<const void*>(k_decode_step_floor<1>)
                            : reinterpret_cast<const void*>(k_decode_step_floor<2>);
  return reinterpret_cast<const void*>(step_kernel_fn(F, att));
}

static int step_check_shape(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L) {
  if (M <= 0 || M > 32) return set_error(BTL_ERR_SHAPE, "btl_decode_step: M=%lld (1..32 decode rows)", (long long)M);
  if (L <= 0 || L > kStepMaxLayers)
    return set_error(BTL_ERR_SHAPE, "btl_decode_step: L=%lld layers (1..%d)", (long long)L, kStepMaxLayers);
  if (H % 128 || F % 128 || NQKV % 64 || H <= 0 || F <= 0 || NQKV <= 0)
    return set_error(BTL_ERR_SHAPE, "btl_decode_step: H=%lld and F=%lld must be multiples of 128, NQKV=%lld of 64",
                     (long long)H, (long long)F, (long long)NQKV);
  if (H > 4096 || NQKV > 4096 || F > 8192)
    return set_error(BTL_ERR_SHAPE, "btl_decode_step: H=%lld NQKV=%lld (<= 4096), F=%lld (<= 8192) exceed the kernel's "
                     "row registers", (long long)H, (long long)NQKV, (long long)F);
  // weights per wave within the register slots: ceil(KS / 8) superblocks per tile, <= 3 for K = H
  // (two tiles for gate||up), <= 7 for K = F
  if ((ksb(H) + 7) / 8 > 3 || (ksb(F) + 7) / 8 > 7)
    return set_error(BTL_ERR_SHAPE, "btl_decode_step: H=%lld or F=%lld too large for the weight registers",
                     (long long)H, (long long)F);
  const int grid = step_grid();
  const int64_t units = std::max({NQKV / 32, 2 * (H / 32), F / 32});  // QKV and O, DN (two row halves), GU
  if (grid <= kStepRows || grid > kStepMaxGrid || units > grid - kStepRows)
    return set_error(BTL_ERR_SHAPE, "btl_decode_step: %lld GEMM units do not fit %d workgroups", (long long)units,
                     grid - kStepRows);
  return BTL_OK;
}

static StepArgs step_args(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L, float eps, uint16_t* hidden,
                          uint16_t* qkv_out, uint16_t* ffn_h, char* ws, const StepSizes& z) {
  StepArgs a = {};
  a.ops = reinterpret_cast<const StepOp*>(ws + kStTable);
  a.L = (int)L;
  a.M = (int)M;
  a.H = (int)H;
  a.F = (int)F;
  a.NQKV = (int)NQKV;
  a.KSH = (int)ksb(H);
  a.KSF = (int)ksb(F);
  a.eps = eps;
  a.hidden = hidden;
  a.qkv_out = qkv_out;
  a.ffn_h = ffn_h;
  a.epoch = reinterpret_cast<uint32_t*>(ws + kStEpoch);
  a.error = reinterpret_cast<uint32_t*>(ws + kStError);
  a.layers = ws + kStHeader;
  for (int j = 0; j < kStepOps; ++j) {
    a.off_xa[j] = z.off_xa[j];
    a.off_out[j] = z.off_out[j];
  }
  a.off_flag = z.off_flag;
  a.spin_limit = 1u << 18;
  return a;
}

static int launch_step(const StepArgs& a, int64_t F, bool att, const char* who, hipStream_t s) {
  void (*k)(StepArgs) = step_kernel_fn(F, att);
  if (!k) return set_error(BTL_ERR_SHAPE, "%s: no kernel instance for F=%lld", who, (long long)F);
  const int grid = step_grid();
  const int rc = check_coresident_launch(who, reinterpret_cast<const void*>(k), 512, grid, s);
  if (rc) return rc;
  hipLaunchKernelGGL(k, dim3(grid), dim3(512), 0, s, a);
  return check_launch(who);
}

}  // namespace btl

using namespace btl;

extern "C" {

int64_t btl_decode_step_workspace_bytes(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L) {
  if (M <= 0 || M > 32 || H <= 0 || F <= 0 || NQKV <= 0 || L <= 0 || L > kStepMaxLayers) return 0;
  return step_sizes(H, F, NQKV).total;
}

int64_t btl_decode_step_error_offset(void) { return kStError; }

int btl_decode_step_clear_share(int m, int64_t KS, int64_t* offsets, int64_t n) {
  clear_error();
  if (!offsets) return set_error(BTL_ERR_NULL, "btl_decode_step_clear_share: null offsets");
  if (m < 0 || m >= kStepRows || KS < 1 || KS > 128 || n < 0)
    return set_error(BTL_ERR_ARG, "btl_decode_step_clear_share: m=%d (0..31), KS=%lld (1..128), n=%lld", m,
                     (long long)KS, (long long)n);
  for (int64_t pc = 0; pc < n && pc < 16 * KS; ++pc) offsets[pc] = clear_piece_offset(m, (int)KS, (int)pc);
  return BTL_OK;
}

int btl_decode_step_prepare(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L,
                            const btl_layer_weight_t* weights, void* workspace, size_t workspace_bytes) {
  clear_error();
  int rc = step_check_shape(M, H, F, NQKV, L);
  if (rc) return rc;
  if (!weights || !workspace) return set_error(BTL_ERR_NULL, "btl_decode_step_prepare: null pointer");
  // every workgroup of the launch waits on others: the device must hold the grid at once
  rc = check_coresident_launch("btl_decode_step_prepare", step_kernel(F, false), 512, step_grid(), nullptr);
  if (rc) return rc;
  if (!aligned(workspace, 256)) return set_error(BTL_ERR_ALIGN, "btl_decode_step_prepare: workspace must be 256-byte aligned");
  const StepSizes z = step_sizes(H, F, NQKV);
  if ((int64_t)workspace_bytes < z.total)
    return set_error(BTL_ERR_WORKSPACE, "btl_decode_step_prepare: workspace %zu < %lld bytes", workspace_bytes,
                     (long long)z.total);
  static const char* names[kStepOps] = {"qkv", "o_proj", "gate_up", "down"};
  const int64_t Ns[kStepOps] = {NQKV, H, 2 * F, H};
  StepOp table[kStepMaxLayers * kStepOps];
  memset(table, 0, sizeof(table));
  for (int64_t l = 0; l < L; ++l)
    for (int j = 0; j < kStepOps; ++j) {
      const btl_layer_weight_t& w = weights[l * kStepOps + j];
      if (!w.wdev || !w.gamma)
        return set_error(BTL_ERR_NULL, "btl_decode_step_prepare: layer %lld %s weight or gain is NULL", (long long)l,
                         names[j]);
      if (!aligned(w.wdev, 16) || !aligned(w.gamma, 16))
        return set_error(BTL_ERR_ALIGN, "btl_decode_step_prepare: layer %lld %s weight / gain must be 16-byte aligned",
                         (long long)l, names[j]);
      if (w.nseg < 1 || w.nseg > BTL_MAX_SEGMENTS)
        return set_error(BTL_ERR_ARG, "btl_decode_step_prepare: layer %lld %s has %d segments", (long long)l, names[j],
                         w.nseg);
      int64_t prev = 0;
      for (int i = 0; i < w.nseg; ++i) {
        if (w.seg_end[i] <= prev || w.seg_end[i] % 32)
          return set_error(BTL_ERR_ARG, "btl_decode_step_prepare: layer %lld %s segment ends must increase in "
                           "multiples of 32", (long long)l, names[j]);
        prev = w.seg_end[i];
      }
      if (prev != Ns[j])
        return set_error(BTL_ERR_ARG, "btl_decode_step_prepare: layer %lld %s last segment end %lld != N=%lld",
                         (long long)l, names[j], (long long)prev, (long long)Ns[j]);
      if (j == S_GU && (w.nseg != 2 || w.seg_end[0] != F))
        return set_error(BTL_ERR_ARG, "btl_decode_step_prepare: layer %lld gate_up needs two segments split at F",
                         (long long)l);
      StepOp& op = table[l * kStepOps + j];
      op.wdev = w.wdev;
      op.gamma = w.gamma;
      op.nseg = w.nseg;
      for (int i = 0; i < BTL_MAX_SEGMENTS; ++i) {
        op.seg_scale[i] = i < w.nseg ? w.seg_scale[i] : 0.0f;
        op.seg_end[i] = i < w.nseg ? (int)w.seg_end[i] : (int)Ns[j];
      }
    }
  if (hipMemcpy((char*)workspace + kStTable, table, sizeof(StepOp) * L * kStepOps, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(BTL_ERR_LAUNCH, "btl_decode_step_prepare: copying the op table failed");
  }
  // operand tiles start every launch as the sentinel (a launch leaves them so)
  if (hipMemset((char*)workspace + kStHeader, (int)(kTileSentinel & 0xffu), (size_t)z.tiles_end) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(BTL_ERR_LAUNCH, "btl_decode_step_prepare: resetting the operand tiles failed");
  }
  return BTL_OK;
}

int btl_decode_step(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L, float eps, const uint16_t* attn,
                    uint16_t* hidden, uint16_t* qkv_out, uint16_t* ffn_h, void* workspace, size_t workspace_bytes,
                    btl_stream_t stream) {
  clear_error();
  int rc = step_check_shape(M, H, F, NQKV, L);
  if (rc) return rc;
  if (!attn || !hidden || !qkv_out || !ffn_h || !workspace) return set_error(BTL_ERR_NULL, "btl_decode_step: null pointer");
  if (!aligned(attn, 16) || !aligned(hidden, 16) || !aligned(workspace, 256) || !aligned(qkv_out, 4) ||
      !aligned(ffn_h, 4))
    return set_error(BTL_ERR_ALIGN, "btl_decode_step: attn/hidden must be 16-byte aligned, qkv_out/ffn_h 4, workspace 256");
  const StepSizes z = step_sizes(H, F, NQKV);
  if ((int64_t)workspace_bytes < z.total)
    return set_error(BTL_ERR_WORKSPACE, "btl_decode_step: workspace %zu < %lld bytes", workspace_bytes,
                     (long long)z.total);
  StepArgs a = step_args(M, H, F, NQKV, L, eps, hidden, qkv_out, ffn_h, (char*)workspace, z);
  a.attn = attn;
  return launch_step(a, F, false, "btl_decode_step", (hipStream_t)stream);
}

int btl_decode_step_attention_prepare(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L,
                                      const uint16_t* const* k_caches, const uint16_t* const* v_caches,
                                      void* workspace, size_t workspace_bytes) {
  clear_error();
  int rc = step_check_shape(M, H, F, NQKV, L);
  if (rc) return rc;
  if (!k_caches || !v_caches || !workspace)
    return set_error(BTL_ERR_NULL, "btl_decode_step_attention_prepare: null pointer");
  if (!aligned(workspace, 256))
    return set_error(BTL_ERR_ALIGN, "btl_decode_step_attention_prepare: workspace must be 256-byte aligned");
  const StepSizes z = step_sizes(H, F, NQKV);
  if ((int64_t)workspace_bytes < z.total)
    return set_error(BTL_ERR_WORKSPACE, "btl_decode_step_attention_prepare: workspace %zu < %lld bytes",
                     workspace_bytes, (long long)z.total);
  uint64_t table[2 * kStepMaxLayers];
  for (int64_t l = 0; l < L; ++l) {
    if (!k_caches[l] || !v_caches[l])
      return set_error(BTL_ERR_NULL, "btl_decode_step_attention_prepare: layer %lld cache is NULL", (long long)l);
    if (!aligned(k_caches[l], 16) || !aligned(v_caches[l], 16))
      return set_error(BTL_ERR_ALIGN, "btl_decode_step_attention_prepare: layer %lld cache must be 16-byte aligned",
                       (long long)l);
    table[2 * l] = reinterpret_cast<uint64_t>(k_caches[l]);
    table[2 * l + 1] = reinterpret_cast<uint64_t>(v_caches[l]);
  }
  if (hipMemcpy((char*)workspace + kStAttn, table, 16 * L, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(BTL_ERR_LAUNCH, "btl_decode_step_attention_prepare: copying the cache table failed");
  }
  return BTL_OK;
}

int btl_decode_step_full(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L, float eps, int64_t Hkv, int64_t S,
                         const int32_t* pos, const float* rope_cos, const float* rope_sin, int rope_adjacent,
                         float scale, uint16_t* hidden, uint16_t* qkv_out, uint16_t* attn_out, uint16_t* ffn_h,
                         void* workspace, size_t workspace_bytes, btl_stream_t stream) {
  clear_error();
  int rc = step_check_shape(M, H, F, NQKV, L);
  if (rc) return rc;
  const int64_t Hq = H / kAtD;
  if (H % kAtD || Hkv <= 0 || Hq % Hkv || Hq / Hkv > kAtMaxG || NQKV != H + 2 * Hkv * kAtD || S <= 0 ||
      S > (1 << 20))
    return set_error(BTL_ERR_SHAPE,
                     "btl_decode_step_full: H=%lld (128-wide heads), Hkv=%lld (at most %d query heads each), "
                     "NQKV=%lld (must be H + 2 Hkv 128), S=%lld",
                     (long long)H, (long long)Hkv, kAtMaxG, (long long)NQKV, (long long)S);
  if (M * Hkv > step_grid() - kStepRows)
    return set_error(BTL_ERR_SHAPE, "btl_decode_step_full: %lld attention units do not fit %d workgroups",
                     (long long)(M * Hkv), step_grid() - kStepRows);
  if (!pos || !rope_cos || !rope_sin || !hidden || !qkv_out || !attn_out || !ffn_h || !workspace)
    return set_error(BTL_ERR_NULL, "btl_decode_step_full: null pointer");
  if (!aligned(hidden, 16) || !aligned(workspace, 256) || !aligned(qkv_out, 4) || !aligned(ffn_h, 4) ||
      !aligned(attn_out, 4) || !aligned(pos, 4) || !aligned(rope_cos, 4) || !aligned(rope_sin, 4))
    return set_error(BTL_ERR_ALIGN, "btl_decode_step_full: hidden must be 16-byte aligned, the other buffers 4, "
                     "workspace 256");
  const StepSizes z = step_sizes(H, F, NQKV);
  if ((int64_t)workspace_bytes < z.total)
    return set_error(BTL_ERR_WORKSPACE, "btl_decode_step_full: workspace %zu < %lld bytes", workspace_bytes,
                     (long long)z.total);
  StepArgs a = step_args(M, H, F, NQKV, L, eps, hidden, qkv_out, ffn_h, (char*)workspace, z);
  a.kv = reinterpret_cast<const uint64_t*>((char*)workspace + kStAttn);
  a.pos = pos;
  a.rcos = rope_cos;
  a.rsin = rope_sin;
  a.attn_out = attn_out;
  a.off_att = z.off_att;
  a.Hkv = (int)Hkv;
  a.G = (int)(Hq / Hkv);
  a.S = (int)S;
  a.adjacent = rope_adjacent ? 1 : 0;
  a.scale = scale;
  return launch_step(a, F, true, "btl_decode_step_full", (hipStream_t)stream);
}

int btl_decode_step_floor(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L, void* workspace,
                          size_t workspace_bytes, btl_stream_t stream) {
  clear_error();
  int rc = step_check_shape(M, H, F, NQKV, L);
  if (rc) return rc;
  if (!workspace) return set_error(BTL_ERR_NULL, "btl_decode_step_floor: null workspace");
  if (!aligned(workspace, 256)) return set_error(BTL_ERR_ALIGN, "btl_decode_step_floor: workspace must be 256-byte aligned");
  const StepSizes z = step_sizes(H, F, NQKV);
  if ((int64_t)workspace_bytes < z.total)
    return set_error(BTL_ERR_WORKSPACE, "btl_decode_step_floor: workspace %zu < %lld bytes", workspace_bytes,
                     (long long)z.total);
  char* ws = (char*)workspace;
  StepArgs a = {};
  a.L = (int)L;
  a.M = (int)M;
  a.H = (int)H;
  a.F = (int)F;
  a.NQKV = (int)NQKV;
  a.KSH = (int)ksb(H);
  a.KSF = (int)ksb(F);
  a.epoch = reinterpret_cast<uint32_t*>(ws + kStEpoch);
  a.error = reinterpret_cast<uint32_t*>(ws + kStError);
  a.layers = ws + kStHeader;
  for (int j = 0; j < kStepOps; ++j) {
    a.off_xa[j] = z.off_xa[j];
    a.off_out[j] = z.off_out[j];
  }
  a.off_flag = z.off_flag;
  a.spin_limit = 1u << 18;
  const int grid = step_grid();
  hipStream_t s = (hipStream_t)stream;
  rc = check_coresident_launch("btl_decode_step_floor", step_kernel(F, true), 512, grid, s);
  if (rc) return rc;
  if (act_cpt(F) == 1)
    hipLaunchKernelGGL((k_decode_step_floor<1>), dim3(grid), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((k_decode_step_floor<2>), dim3(grid), dim3(512), 0, s, a);
  return check_launch("decode step floor");
}

}  // extern "C"

BTL_TRACE_READ_FN(btl_trace_read_step)
