// Load-time weight preparation on the GPU:
//   * absmean ternary quantisation with numpy's float32 mean order
//     (src/bitnet_tt/utils/quantization.py:15-57),
//   * the reference's 2-bit tile format (src/bitnet_tt/kernels/pack.py:101-191),
//   * the repack of that format into the layout the GEMM streams.
// All of it is integer/byte work bound by memory traffic; none of it runs in
// the decode step.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "btl_act_row.h"
#include "btl_common.h"

namespace btl {

// ---------------------------------------------------------------- errors --
static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}
void clear_error() { g_err[0] = 0; }
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(BTL_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return BTL_OK;
}

// ------------------------------------------------------- co-residency --
// Kernels whose workgroups wait on each other (the fused decode BitLinear,
// the persistent step) need the whole grid resident at once.  The capacity
// is the kernel's occupancy (workgroups per CU at its block size, from its
// registers and LDS) times the CUs the stream may use (its CU mask, when the
// runtime reports one, else the device's CU count).  Occupancy per kernel
// and block size is cached (fixed by the compiled code object).
int coresident_check(const char* who, int64_t grid, int64_t per_cu, int64_t cus) {
  if (per_cu <= 0 || cus <= 0)
    return set_error(BTL_ERR_LAUNCH, "%s: the device holds no workgroup of this kernel (%lld per CU, %lld CUs)", who,
                     (long long)per_cu, (long long)cus);
  if (grid > per_cu * cus)
    return set_error(BTL_ERR_LAUNCH,
                     "%s: %lld workgroups that wait on each other, but only %lld fit at once (%lld per CU x %lld CUs)",
                     who, (long long)grid, (long long)(per_cu * cus), (long long)per_cu, (long long)cus);
  return BTL_OK;
}

int stream_cus(hipStream_t s) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  uint32_t mask[32];  // up to 1024 CUs
  const uint32_t words = (uint32_t)((cus + 31) / 32);
  if (words <= 32 && hipExtStreamGetCUMask(s, words, mask) == hipSuccess) {
    int n = 0;
    for (uint32_t i = 0; i < words; ++i) n += __builtin_popcount(mask[i]);
    if (n > 0 && n < cus) cus = n;
  } else {
    (void)hipGetLastError();
  }
  return cus;
}

int kernel_per_cu(const void* kernel, int threads) {
  struct Entry {
    const void* k;
    int dev, threads, per_cu;
  };
  static Entry cache[128];
  static int used = 0;
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  std::lock_guard<std::mutex> lk(mu);
  for (int i = 0; i < used; ++i)
    if (cache[i].k == kernel && cache[i].dev == dev && cache[i].threads == threads) return cache[i].per_cu;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (used < 128) cache[used++] = Entry{kernel, dev, threads, n};
  return n;
}

int check_coresident_launch(const char* who, const void* kernel, int threads, int64_t grid, hipStream_t s) {
  return coresident_check(who, grid, kernel_per_cu(kernel, threads), stream_cus(s));
}

// ------------------------------------------------- numpy-order abs-sum --
// numpy reduces a float32 array in buffered blocks of 8192 elements; each
// block is summed pairwise: blocks of < 8 sequentially, blocks of <= 128 with
// eight strided accumulators combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7))
// plus a sequential tail, larger blocks split at n/2 rounded down to a
// multiple of 8.  One thread reproduces that tree for one 8192-block.
__device__ float pw_leaf_abs(const float* a, int n) {
  if (n < 8) {
    float r = 0.0f;
    for (int i = 0; i < n; ++i) r += fabsf(a[i]);
    return r;
  }
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = fabsf(a[j]);
  int i = 8;
  for (; i < n - (n % 8); i += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] += fabsf(a[i + j]);
  }
  float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) res += fabsf(a[i]);
  return res;
}

__device__ float pw_abs(const float* a, int n) {
  // Post-order walk of the split tree with an explicit stack (depth <= 8
  // for n <= 8192).
  int off[12], len[12], stage[12];
  float left[12];
  int sp = 0;
  off[0] = 0;
  len[0] = n;
  stage[0] = 0;
  float res = 0.0f;
  bool have = false;
  for (;;) {
    if (!have) {
      const int o = off[sp], l = len[sp];
      if (l <= 128) {
        res = pw_leaf_abs(a + o, l);
        have = true;
        if (--sp < 0) return res;
        continue;
      }
      int n2 = l / 2;
      n2 -= n2 % 8;
      stage[sp] = 1;
      ++sp;
      off[sp] = o;
      len[sp] = n2;
      stage[sp] = 0;
    } else if (stage[sp] == 1) {
      left[sp] = res;
      stage[sp] = 2;
      const int o = off[sp], l = len[sp];
      int n2 = l / 2;
      n2 -= n2 % 8;
      ++sp;
      off[sp] = o + n2;
      len[sp] = l - n2;
      stage[sp] = 0;
      have = false;
    } else {
      res = left[sp] + res;
      if (--sp < 0) return res;
    }
  }
}

// Blocks b0, b0 + 1, ... one thread each (the partial last block).
__global__ void k_wq_block_sums(const float* __restrict__ w, int64_t n, float* __restrict__ part, int64_t b0) {
  const int64_t b = b0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t start = b * 8192;
  if (start >= n) return;
  const int len = (int)((n - start) < 8192 ? (n - start) : 8192);
  part[b] = pw_abs(w + start, len);
}

// Full 8192-blocks, one wave each.  The split tree of 8192 is balanced (every
// split at n / 2, a multiple of 8) down to 64 leaves of 128: lane j sums leaf j
// (elements 128 j .. 128 j + 127) as pw_leaf_abs does, and each of the six
// levels above adds adjacent subtrees, one xor butterfly step (float addition
// is commutative, so which lane of a pair holds the left subtree does not
// matter).  The same sums as the one-thread walk, in a 64th of the passes.
__global__ __launch_bounds__(256) void k_wq_block_sums_wave(const float* __restrict__ w, int64_t nfull,
                                                            float* __restrict__ part) {
  const int64_t b = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (b >= nfull) return;  // wave-uniform
  const float4* a = reinterpret_cast<const float4*>(w + b * 8192 + lane * 128);
  float r[8];
  {
    const float4 x0 = a[0], x1 = a[1];
    r[0] = fabsf(x0.x), r[1] = fabsf(x0.y), r[2] = fabsf(x0.z), r[3] = fabsf(x0.w);
    r[4] = fabsf(x1.x), r[5] = fabsf(x1.y), r[6] = fabsf(x1.z), r[7] = fabsf(x1.w);
  }
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    const float4 x0 = a[2 * i], x1 = a[2 * i + 1];
    r[0] += fabsf(x0.x), r[1] += fabsf(x0.y), r[2] += fabsf(x0.z), r[3] += fabsf(x0.w);
    r[4] += fabsf(x1.x), r[5] += fabsf(x1.y), r[6] += fabsf(x1.z), r[7] += fabsf(x1.w);
  }
  float v = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  v = v + xor_partner<1>(v);
  v = v + xor_partner<2>(v);
  v = v + xor_partner<4>(v);
  v = v + xor_partner<8>(v);
  v = v + xor_partner<16>(v);
  v = v + xor_partner<32>(v);
  if (lane == 0) part[b] = v;
}

// The blocks' sums in block order (numpy adds its buffered blocks one after
// another): 256 threads stage up to 8192 partials at a time in LDS, and
// thread 0 adds them in order, four per LDS read.
__global__ __launch_bounds__(256) void k_wq_finalize(const float* __restrict__ part, int64_t nblocks, int64_t n,
                                                     float eps, float* __restrict__ scale_out) {
  __shared__ __attribute__((aligned(16))) float sp[8192];
  const int tid = threadIdx.x;
  float acc = 0.0f;
  for (int64_t b0 = 0; b0 < nblocks; b0 += 8192) {
    const int cnt = nblocks - b0 < 8192 ? (int)(nblocks - b0) : 8192;
    for (int i = tid; i < cnt; i += 256) sp[i] = part[b0 + i];
    __syncthreads();
    if (tid == 0) {
      const float4* s4 = reinterpret_cast<const float4*>(sp);
      int i = 0;
#pragma unroll 8
      for (; i + 4 <= cnt; i += 4) {
        const float4 q = s4[i >> 2];
        acc += q.x;
        acc += q.y;
        acc += q.z;
        acc += q.w;
      }
      for (; i < cnt; ++i) acc += sp[i];
    }
    __syncthreads();
  }
  if (tid != 0) return;
  // numpy: float32(float64(sum) / float64(count)), then np.maximum(., eps).
  float mean = (float)((double)acc / (double)n);
  scale_out[0] = mean > eps ? mean : eps;
}

__global__ void k_wq_quant(const float* __restrict__ w, int64_t n, const float* __restrict__ scale,
                           int8_t* __restrict__ q) {
  const float s = scale[0];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float r = rintf(w[i] / s);  // correctly rounded division (HIP default)
    r = fminf(fmaxf(r, -1.0f), 1.0f);
    q[i] = (int8_t)(int)r;
  }
}

// ------------------------------------------------------ reference tiles --
// Element (r, c) of a 32x32 tile sits at face position
// p = 256*(2*[r>=16] + [c>=16]) + 16*(r%16) + (c%16), byte p/4, bits
// 7-2*(p%4) .. 6-2*(p%4) (pack.py:53-98).
__device__ __forceinline__ uint32_t tern_code(int8_t v) { return v == 1 ? 1u : (v == -1 ? 2u : 0u); }
__device__ __forceinline__ int tern_value(uint32_t c) { return c == 1u ? 1 : (c == 2u ? -1 : 0); }

__global__ void k_pack_tiles(const int8_t* __restrict__ w, int64_t out_f, int64_t in_f, int64_t nt_n,
                             int64_t nbytes, uint8_t* __restrict__ packed) {
  const int64_t byte = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (byte >= nbytes) return;
  const int64_t t = byte >> 8;
  const int pb = (int)(byte & 255);
  const int64_t kt = t / nt_n, nt = t % nt_n;
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = 4 * pb + i;
    const int f = p >> 8, rr = (p >> 4) & 15, cc = p & 15;
    const int64_t k = kt * 32 + 16 * (f >> 1) + rr;
    const int64_t n = nt * 32 + 16 * (f & 1) + cc;
    const int8_t v = (k < in_f && n < out_f) ? w[n * in_f + k] : (int8_t)0;
    out |= tern_code(v) << (6 - 2 * i);
  }
  packed[byte] = (uint8_t)out;
}

__global__ void k_unpack_tiles(const uint8_t* __restrict__ packed, int64_t in_f, int64_t out_f, int64_t nt_n,
                               int64_t nbytes, int8_t* __restrict__ w_kn) {
  const int64_t byte = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (byte >= nbytes) return;
  const int64_t t = byte >> 8;
  const int pb = (int)(byte & 255);
  const int64_t kt = t / nt_n, nt = t % nt_n;
  const uint32_t b = packed[byte];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = 4 * pb + i;
    const int f = p >> 8, rr = (p >> 4) & 15, cc = p & 15;
    const int64_t k = kt * 32 + 16 * (f >> 1) + rr;
    const int64_t n = nt * 32 + 16 * (f & 1) + cc;
    if (k < in_f && n < out_f) w_kn[k * out_f + n] = (int8_t)tern_value((b >> (6 - 2 * i)) & 3u);
  }
}

// ------------------------------------------------------- device layout --
// Word ((nt*KS + ks)*64 + lane)*4 + q holds the offset codes u = w + 1 of
// column nt*32 + (lane & 31), rows k = ks*128 + q*32 + (lane >> 5)*16 + j,
// code j at bit 8*(j & 3) + 2*(j >> 2): (word >> 2r) & 0x03030303 is then
// the MFMA B operand dword r (bytes = rows 4r..4r+3 of the lane's 16).
// Rows k >= K carry u = 1 (weight 0).
__global__ void k_repack(const uint8_t* __restrict__ packed, int64_t K, int64_t N, int64_t KS, int64_t nwords,
                         uint32_t* __restrict__ wdev) {
  const int64_t wi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (wi >= nwords) return;
  const int q = (int)(wi & 3);
  const int lane = (int)((wi >> 2) & 63);
  const int64_t sbi = wi >> 8;  // nt*KS + ks
  const int64_t nt = sbi / KS, ks = sbi % KS;
  const int64_t nt_n = N / 32;
  const int c = lane & 31;
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int64_t k = ks * 128 + q * 32 + (lane >> 5) * 16 + j;
    uint32_t u = 1u;
    if (k < K) {
      const int r = (int)(k & 31);
      const int64_t t = (k >> 5) * nt_n + nt;
      const int p = 256 * (2 * (r >> 4) + (c >> 4)) + 16 * (r & 15) + (c & 15);
      const uint32_t code = (packed[t * 256 + (p >> 2)] >> (6 - 2 * (p & 3))) & 3u;
      u = (uint32_t)(tern_value(code) + 1);
    }
    word |= u << (8 * (j & 3) + 2 * (j >> 2));
  }
  wdev[wi] = word;
}

static unsigned grid_for(int64_t n, int block) { return (unsigned)((n + block - 1) / block); }

}  // namespace btl

using namespace btl;

extern "C" {

const char* btl_last_error(void) { return g_err; }
int btl_version(void) { return 200; }

int btl_check_coresident(int64_t grid, int64_t per_cu, int64_t cus) {
  clear_error();
  return coresident_check("btl_check_coresident", grid, per_cu, cus);
}

int64_t btl_packed_tile_count(int64_t in_f, int64_t out_f) {
  if (in_f <= 0 || out_f <= 0) return 0;
  return ((in_f + 31) / 32) * ((out_f + 31) / 32);
}
int64_t btl_packed_dram_bytes(int64_t in_f, int64_t out_f) { return btl_packed_tile_count(in_f, out_f) * 256; }
int64_t btl_devlayout_words(int64_t K, int64_t N) {
  if (K <= 0 || N <= 0 || N % 32) return 0;
  return (N / 32) * ksb(K) * 256;
}
int64_t btl_act_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0) return 0;
  return mblocks(M) * ksb(K) * 4096;
}

int64_t btl_weight_quant_scratch_bytes(int64_t n) {
  if (n <= 0) return 0;
  return ((n + 8191) / 8192) * (int64_t)sizeof(float);
}

int btl_weight_quant_ternary(const float* w, int64_t n, float eps, int8_t* q, float* scale_out, void* scratch,
                             size_t scratch_bytes, btl_stream_t stream) {
  clear_error();
  if (!w || !q || !scale_out || !scratch) return set_error(BTL_ERR_NULL, "btl_weight_quant_ternary: null pointer");
  if (n <= 0) return set_error(BTL_ERR_SHAPE, "btl_weight_quant_ternary: n=%lld", (long long)n);
  if (!aligned(scratch, 4) || !aligned(scale_out, 4) || !aligned(w, 4))
    return set_error(BTL_ERR_ALIGN, "btl_weight_quant_ternary: float buffers must be 4-byte aligned");
  if ((int64_t)scratch_bytes < btl_weight_quant_scratch_bytes(n))
    return set_error(BTL_ERR_WORKSPACE, "btl_weight_quant_ternary: scratch %zu < %lld", scratch_bytes,
                     (long long)btl_weight_quant_scratch_bytes(n));
  hipStream_t s = (hipStream_t)stream;
  const int64_t nb = (n + 8191) / 8192, nfull = n / 8192;
  float* part = (float*)scratch;
  // full blocks one wave each (float4 loads: w 16-byte aligned), else one thread a block
  if (aligned(w, 16)) {
    if (nfull > 0) hipLaunchKernelGGL(k_wq_block_sums_wave, dim3(grid_for(nfull * 64, 256)), dim3(256), 0, s, w, nfull, part);
    if (nb > nfull) hipLaunchKernelGGL(k_wq_block_sums, dim3(1), dim3(64), 0, s, w, n, part, nfull);
  } else {
    hipLaunchKernelGGL(k_wq_block_sums, dim3(grid_for(nb, 64)), dim3(64), 0, s, w, n, part, (int64_t)0);
  }
  hipLaunchKernelGGL(k_wq_finalize, dim3(1), dim3(256), 0, s, part, nb, n, eps, scale_out);
  const int64_t blocks = grid_for(n, 256) < 65536 ? grid_for(n, 256) : 65536;
  hipLaunchKernelGGL(k_wq_quant, dim3((unsigned)blocks), dim3(256), 0, s, w, n, scale_out, q);
  return check_launch("btl_weight_quant_ternary");
}

int btl_pack_tiles(const int8_t* w, int64_t out_f, int64_t in_f, uint8_t* packed, btl_stream_t stream) {
  clear_error();
  if (!w || !packed) return set_error(BTL_ERR_NULL, "btl_pack_tiles: null pointer");
  if (out_f <= 0 || in_f <= 0) return set_error(BTL_ERR_SHAPE, "btl_pack_tiles: shape (%lld, %lld)",
                                                (long long)out_f, (long long)in_f);
  const int64_t nbytes = btl_packed_dram_bytes(in_f, out_f);
  const int64_t nt_n = (out_f + 31) / 32;
  hipLaunchKernelGGL(k_pack_tiles, dim3(grid_for(nbytes, 256)), dim3(256), 0, (hipStream_t)stream, w, out_f, in_f,
                     nt_n, nbytes, packed);
  return check_launch("btl_pack_tiles");
}

int btl_unpack_tiles(const uint8_t* packed, int64_t in_f, int64_t out_f, int8_t* w_kn, btl_stream_t stream) {
  clear_error();
  if (!w_kn || !packed) return set_error(BTL_ERR_NULL, "btl_unpack_tiles: null pointer");
  if (out_f <= 0 || in_f <= 0) return set_error(BTL_ERR_SHAPE, "btl_unpack_tiles: shape (%lld, %lld)",
                                                (long long)in_f, (long long)out_f);
  const int64_t nbytes = btl_packed_dram_bytes(in_f, out_f);
  const int64_t nt_n = (out_f + 31) / 32;
  hipLaunchKernelGGL(k_unpack_tiles, dim3(grid_for(nbytes, 256)), dim3(256), 0, (hipStream_t)stream, packed, in_f,
                     out_f, nt_n, nbytes, w_kn);
  return check_launch("btl_unpack_tiles");
}

int btl_repack(const uint8_t* packed, int64_t K, int64_t N, uint32_t* wdev, btl_stream_t stream) {
  clear_error();
  if (!packed || !wdev) return set_error(BTL_ERR_NULL, "btl_repack: null pointer");
  if (K <= 0 || N <= 0 || K % 32 || N % 32)
    return set_error(BTL_ERR_SHAPE, "btl_repack: K=%lld N=%lld must be positive multiples of 32", (long long)K,
                     (long long)N);
  if (K > BTL_MAX_K) return set_error(BTL_ERR_SHAPE, "btl_repack: K=%lld > %d", (long long)K, BTL_MAX_K);
  if (!aligned(wdev, 16)) return set_error(BTL_ERR_ALIGN, "btl_repack: wdev must be 16-byte aligned");
  const int64_t nwords = btl_devlayout_words(K, N);
  hipLaunchKernelGGL(k_repack, dim3(grid_for(nwords, 256)), dim3(256), 0, (hipStream_t)stream, packed, K, N, ksb(K),
                     nwords, wdev);
  return check_launch("btl_repack");
}

}  // extern "C"
