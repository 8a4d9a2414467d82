// LM head of the decode step: logits = RMSNorm(hidden) @ W^T with W the bf16
// [vocab, hidden] head matrix, and the greedy token of every row
// (src/bitnet_tt/model/bitnet.py:139-215 loads the head,
// src/bitnet_tt/inference/generator_batch32.py:768-811 runs final norm and
// head, :1170-1174 takes the argmax).  The final RMSNorm is btl_rmsnorm.
//
// The head is 656 MB of bf16 at the 2B shape, more bytes than every BitLinear
// of a step together, so the kernel is a weight stream:
//  * the weights are repacked once into MFMA operand order: 16 vocab rows x
//    32 k per KiB, lane l holding W[row l & 15][k0 + 8 (l >> 4) .. + 8], so a
//    wave's operand is one coalesced 16-byte load per lane;
//  * one workgroup per CU walks pairs of neighbouring vocab tiles of 16 rows;
//    its eight waves split K, each keeping its slice of the (up to 32)
//    normalised rows in registers for the whole launch, and run
//    v_mfma_f32_16x16x32_bf16 (one or two 16-row blocks);
//  * the fp32 logits wait in LDS and are written in whole lines after the
//    weight stream;
//  * the loads of the next tile are issued before the previous tile's partial
//    sums are reduced through LDS, so the reduction runs under them;
//  * every thread keeps the best (value, first index) of its two rows; the
//    rows' bests meet in a device-scope 64-bit atomicMax, and the last
//    workgroup to finish turns the keys into token ids and clears them.
#include <hip/hip_runtime.h>

#include "btl.h"
#include "btl_act_row.h"
#include "btl_common.h"
#include "btl_mfma.h"

namespace btl {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kLmWaves = 8;
constexpr int kLmMaxRows = 32;
constexpr int kLmLgTiles = 32;  // tiles of logits a workgroup holds in LDS before writing them out

struct LmArgs {
  const uint16_t* xn;  // [M, K] bf16, normalised rows
  int M, K, V, VT, KS32;
  const uint4* w;     // device layout, VT x KS32 x 64 lanes x 16 bytes
  float* logits;      // [M, V] (LOGITS launches)
  int32_t* tokens;    // [M]
  uint64_t* keys;     // [32] in the workspace (zero between calls)
  uint32_t* count;    // workgroups done (zero between calls)
};

// Total order of float bits as unsigned (larger float -> larger key).
__device__ __forceinline__ uint32_t float_order(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// RB row blocks of 16 (M <= 16 RB), NB k32 steps per wave (K <= 256 NB).
// Tiles are 16 vocab rows, taken in pairs of neighbours: a workgroup takes
// pairs blockIdx.x + j * gridDim.x, tiles 2 pair and 2 pair + 1 one after the
// other.  It keeps two tiles in flight (register sets b0 and b1): while one
// tile's partial sums are reduced, the next one's loads are outstanding and
// the one after is issued as soon as its registers are free.  The loop body
// is straight-line (tiles past the end are clamped to a valid tile and their
// results dropped) so that every wait counts exactly the loads it needs.
// The logits (LOGITS) collect in LDS, up to kLmLgTiles tiles, and leave in
// whole 128-byte lines of a row (the two tiles of a pair) once the workgroup's
// weight stream is done (or the buffer is full): stored tile by tile, 64 bytes
// in each of 32 rows, the 16 MB of logits of 32 rows cost the stream 18 us.
template <int RB, int NB, bool LOGITS>
__global__ __launch_bounds__(512, 1) void k_lm_head(LmArgs p) {
  __shared__ float red[kLmWaves][RB][4][64];
  __shared__ float lgb[LOGITS ? kLmLgTiles : 1][RB * 16][16];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int G = gridDim.x;
  const int P = (p.VT + 1) >> 1;                                 // tile pairs
  const int mine_p = (P - (int)blockIdx.x + G - 1) / G;          // >= 1: the grid is at most P
  const int last_pair = (int)blockIdx.x + (mine_p - 1) * G;
  const int mine = 2 * mine_p - (2 * last_pair + 1 < p.VT ? 0 : 1);  // the last pair of an odd VT holds one tile

  v8bf a[RB][NB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r = rb * 16 + (lane & 15);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int k = (wv * NB + j) * 32 + 8 * (lane >> 4);
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (r < p.M && k < p.K) v = *reinterpret_cast<const uint4*>(p.xn + (int64_t)r * p.K + k);
      a[rb][j] = __builtin_bit_cast(v8bf, v);
    }
  }

  // the element of each tile this thread reduces: (rb, i, l) of the waves' accumulators
  const bool reducer = tid < RB * 256;
  const int e_l = tid & 63, e_i = (tid >> 6) & 3, e_rb = (tid >> 8) < RB ? (tid >> 8) : RB - 1;
  const int row = e_rb * 16 + 4 * (e_l >> 4) + e_i;
  float best = -__builtin_inff();
  int bidx = -1;

  auto tile_of = [&](int i) {
    const int c = i < mine ? i : mine - 1;
    return 2 * ((int)blockIdx.x + (c >> 1) * G) + (c & 1);
  };
  auto issue = [&](uint4 (&b)[NB], int t) {
    const uint4* src = p.w + ((int64_t)t * p.KS32 + wv * NB) * 64 + lane;
#pragma unroll
    for (int j = 0; j < NB; ++j) b[j] = src[j * 64];
  };
  auto consume = [&](const uint4 (&b)[NB], int i) {
    v4f acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rb][j], __builtin_bit_cast(v8bf, b[j]), acc[rb], 0, 0, 0);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wv][rb][q][lane] = acc[rb][q];
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kLmWaves; ++w) s += red[w][e_rb][e_i][e_l];
    __syncthreads();
    const int col = tile_of(i) * 16 + (e_l & 15);
    const bool ok = reducer && i < mine && row < p.M && col < p.V;
    if (LOGITS && reducer && i < mine) lgb[i % kLmLgTiles][row][e_l & 15] = s;
    if (ok && s > best) best = s, bidx = col;  // a thread's columns only grow: ties keep the first
  };
  // Logits of tiles c0 .. c0 + cnt - 1 (c0 even) from LDS: a wave writes two
  // rows of one pair, 32 consecutive columns each.
  auto flush = [&](int c0, int cnt) {
    __syncthreads();
    const int cc = tid & 31, r0 = tid >> 5;
    for (int pc = 0; pc < cnt; pc += 2) {
      const int c = pc + (cc >> 4);
      const int col = tile_of(c0 + c) * 16 + (cc & 15);
#pragma unroll
      for (int r = r0; r < RB * 16; r += 16)
        if (c < cnt && r < p.M && col < p.V) p.logits[(int64_t)r * p.V + col] = lgb[c][r][cc & 15];
    }
    __syncthreads();
  };
  auto after = [&](int i) {  // uniform: every thread calls flush at the same tiles
    if (LOGITS && i < mine && ((i + 1) % kLmLgTiles == 0 || i + 1 == mine))
      flush(i - i % kLmLgTiles, i % kLmLgTiles + 1);
  };

  uint4 b0[NB], b1[NB];
  issue(b0, tile_of(0));
  issue(b1, tile_of(1));
  for (int i = 0; i < mine; i += 2) {
    consume(b0, i);
    issue(b0, tile_of(i + 2));
    after(i);
    consume(b1, i + 1);
    issue(b1, tile_of(i + 3));
    after(i + 1);
  }

  // best of each row over the 16 lanes that hold its columns
  uint64_t key = bidx >= 0 ? ((uint64_t)float_order(best) << 32) | (0xffffffffu - (uint32_t)bidx) : 0u;
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) {
    const uint64_t o = __shfl_xor(key, off, 64);
    key = o > key ? o : key;
  }
  if (reducer && (e_l & 15) == 0 && row < p.M && key)
    __hip_atomic_fetch_max(p.keys + row, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  wait_memory();  // this workgroup's maxima are performed before it counts itself done
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(p.count, 1u) + 1u == gridDim.x;
  __syncthreads();
  if (!s_last) return;
  if (tid < p.M) {
    const uint64_t k = ld_coherent(p.keys + tid);
    p.tokens[tid] = k ? (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffu)) : -1;
    st_coherent(p.keys + tid, (uint64_t)0);
  }
  if (tid == 0) st_coherent(p.count, 0u);
}

// W [V, K] bf16 row-major -> device layout (zero rows past V, zero k past K).
__global__ void k_lm_head_repack(const uint16_t* w, int V, int K, int KS32, int64_t total, uint4* out) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= total) return;
  const int lane = (int)(g & 63);
  const int64_t blk = g >> 6;
  const int s = (int)(blk % KS32);
  const int vt = (int)(blk / KS32);
  const int row = vt * 16 + (lane & 15);
  const int k = s * 32 + 8 * (lane >> 4);
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (row < V && k < K) v = *reinterpret_cast<const uint4*>(w + (int64_t)row * K + k);
  out[g] = v;
}

// k32 steps per wave: the smallest supported count covering K.
static int lm_nb(int64_t K) {
  static const int kNB[] = {1, 2, 4, 6, 8, 10, 12};
  const int need = (int)((K + 255) / 256);
  for (int nb : kNB)
    if (nb >= need) return nb;
  return 0;
}

template <int RB, int NB>
static void launch_lm(bool logits, dim3 grid, hipStream_t s, const LmArgs& a) {
  if (logits)
    hipLaunchKernelGGL((k_lm_head<RB, NB, true>), grid, dim3(64 * kLmWaves), 0, s, a);
  else
    hipLaunchKernelGGL((k_lm_head<RB, NB, false>), grid, dim3(64 * kLmWaves), 0, s, a);
}

template <int NB>
static void launch_lm_nb(int rb, bool logits, dim3 grid, hipStream_t s, const LmArgs& a) {
  if (rb == 1)
    launch_lm<1, NB>(logits, grid, s, a);
  else
    launch_lm<2, NB>(logits, grid, s, a);
}

static int check_lm_shape(const char* who, int64_t V, int64_t K) {
  if (V <= 0 || V > (int64_t)1 << 30 || K <= 0 || K % 16)
    return set_error(BTL_ERR_SHAPE, "%s: V=%lld K=%lld (K a multiple of 16 required)", who, (long long)V, (long long)K);
  if (!lm_nb(K)) return set_error(BTL_ERR_SHAPE, "%s: K=%lld > %d", who, (long long)K, 12 * 256);
  return 0;
}

}  // namespace btl

using namespace btl;

extern "C" {

int64_t btl_lm_head_weight_bytes(int64_t V, int64_t K) {
  if (V <= 0 || K <= 0 || K % 16 || !lm_nb(K)) return 0;
  return (V + 15) / 16 * (int64_t)lm_nb(K) * kLmWaves * 1024;
}

int64_t btl_lm_head_workspace_bytes(void) { return 512; }

int btl_lm_head_repack(const uint16_t* w, int64_t V, int64_t K, uint16_t* wdev, btl_stream_t stream) {
  clear_error();
  int rc = check_lm_shape("btl_lm_head_repack", V, K);
  if (rc) return rc;
  if (!w || !wdev) return set_error(BTL_ERR_NULL, "btl_lm_head_repack: NULL pointer");
  if (!aligned(w, 16) || !aligned(wdev, 16)) return set_error(BTL_ERR_ALIGN, "btl_lm_head_repack: 16-byte alignment");
  const int KS32 = lm_nb(K) * kLmWaves;
  const int64_t total = (V + 15) / 16 * KS32 * 64;
  hipLaunchKernelGGL(k_lm_head_repack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, w,
                     (int)V, (int)K, KS32, total, reinterpret_cast<uint4*>(wdev));
  return check_launch("lm head repack");
}

int btl_lm_head(const uint16_t* xn, int64_t M, int64_t K, int64_t V, const uint16_t* wdev, float* logits,
                int32_t* tokens, void* workspace, size_t workspace_bytes, btl_stream_t stream) {
  clear_error();
  int rc = check_lm_shape("btl_lm_head", V, K);
  if (rc) return rc;
  if (M <= 0 || M > kLmMaxRows) return set_error(BTL_ERR_SHAPE, "btl_lm_head: M=%lld (1..32 rows)", (long long)M);
  if (!xn || !wdev || !tokens || !workspace) return set_error(BTL_ERR_NULL, "btl_lm_head: NULL pointer");
  if (!aligned(xn, 16) || !aligned(wdev, 16) || !aligned(tokens, 4) || (logits && !aligned(logits, 4)) ||
      !aligned(workspace, 256))
    return set_error(BTL_ERR_ALIGN, "btl_lm_head: misaligned buffer");
  if ((int64_t)workspace_bytes < btl_lm_head_workspace_bytes())
    return set_error(BTL_ERR_WORKSPACE, "btl_lm_head: workspace %zu < %lld bytes", workspace_bytes,
                     (long long)btl_lm_head_workspace_bytes());
  LmArgs a;
  a.xn = xn;
  a.M = (int)M;
  a.K = (int)K;
  a.V = (int)V;
  a.VT = (int)((V + 15) / 16);
  const int nb = lm_nb(K);
  a.KS32 = nb * kLmWaves;
  a.w = reinterpret_cast<const uint4*>(wdev);
  a.logits = logits;
  a.tokens = tokens;
  a.keys = reinterpret_cast<uint64_t*>(workspace);
  a.count = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(workspace) + 256);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const int pairs = (a.VT + 1) / 2;
  const dim3 grid((unsigned)(pairs < cus ? pairs : cus));
  hipStream_t s = (hipStream_t)stream;
  const int rb = M <= 16 ? 1 : 2;
  const bool lg = logits != nullptr;
  switch (nb) {
    case 1: launch_lm_nb<1>(rb, lg, grid, s, a); break;
    case 2: launch_lm_nb<2>(rb, lg, grid, s, a); break;
    case 4: launch_lm_nb<4>(rb, lg, grid, s, a); break;
    case 6: launch_lm_nb<6>(rb, lg, grid, s, a); break;
    case 8: launch_lm_nb<8>(rb, lg, grid, s, a); break;
    case 10: launch_lm_nb<10>(rb, lg, grid, s, a); break;
    default: launch_lm_nb<12>(rb, lg, grid, s, a); break;
  }
  return check_launch("lm head");
}

}  // extern "C"
