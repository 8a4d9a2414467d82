/*
 * btl_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, CPU-only restatement of the BitLinear hot path of bitnet-tt
 * (2-bit packed ternary weights, absmean weight quantisation, per-token int8
 * absmax activation quantisation, RMSNorm prologue, int32 accumulation,
 * scale epilogue, relu^2*up).  It is the checker that the HIP kernels are
 * compared against; nothing in the product links or calls it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the bitnet-tt repository root).  Third-party semantics (numpy's float32
 * reduction order, HuggingFace BitNet) are cited by their published behaviour.
 *
 * Parity pins (see tests/test_oracle_pins.py):
 *   - codes / byte packing / face order / tile order: the reference's own
 *     known answers (tests/test_ternary_kernel.py:31-170), brute force over all
 *     81 ternary 4-tuples, bijectivity;
 *   - weight scale: bit-exact against numpy's np.mean(np.abs(W)) on many shapes;
 *   - activation quant: closed-form special cases (exact +-absmax -> +-127,
 *     zero rows, ties to even) and tests/test_bitlinear.py:70-97,
 *     tests/test_model.py:91-102;
 *   - int32 GEMM: I@W = W, all-ones -> row sums, brute force in int64;
 *   - RMSNorm: blocked-order fp32 statistic within 2 ulp of the double one.
 * Parity unpinned: none of the functions below (the blocked fp32 RMS order is a
 * stated contract of this build, pinned against the double-precision statistic
 * by an error bound rather than by a reference vector).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* bf16 helpers (round-to-nearest-even, NaN kept quiet)               */
/* ------------------------------------------------------------------ */
static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = ((uint32_t)h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
void orc_f32_to_bf16(const float* x, int64_t n, uint16_t* y) {
  for (int64_t i = 0; i < n; ++i) y[i] = f32_to_bf16(x[i]);
}
void orc_bf16_to_f32(const uint16_t* x, int64_t n, float* y) {
  for (int64_t i = 0; i < n; ++i) y[i] = bf16_to_f32(x[i]);
}

/* ------------------------------------------------------------------ */
/* 2-bit codes: src/bitnet_tt/kernels/pack.py:31-50                   */
/* -1 -> 0b10, 0 -> 0b00, +1 -> 0b01; decode 0b11 -> 0                */
/* (kernels/device/reader_ternary_in1.cpp:43-56 LUT).                 */
/* ------------------------------------------------------------------ */
static inline uint8_t enc1(int8_t v) { return v == 1 ? 1u : (v == -1 ? 2u : 0u); }
static inline int8_t dec1(uint8_t c) { return c == 1u ? 1 : (c == 2u ? -1 : 0); }

void orc_encode_ternary(const int8_t* v, int64_t n, uint8_t* codes) { /* pack.py:37-42 */
  for (int64_t i = 0; i < n; ++i) codes[i] = enc1(v[i]);
}
void orc_decode_ternary(const uint8_t* codes, int64_t n, int8_t* v) { /* pack.py:45-50 */
  for (int64_t i = 0; i < n; ++i) v[i] = dec1(codes[i]);
}
/* pack.py:53-63: groups of 4 codes, first code in bits 7:6 (MSB first). */
void orc_pack_4_to_byte(const uint8_t* codes, int64_t ncodes, uint8_t* out) {
  for (int64_t b = 0; b < ncodes / 4; ++b)
    out[b] = (uint8_t)(((codes[4 * b] & 3u) << 6) | ((codes[4 * b + 1] & 3u) << 4) |
                       ((codes[4 * b + 2] & 3u) << 2) | (codes[4 * b + 3] & 3u));
}
/* pack.py:66-76 */
void orc_unpack_byte_to_4(const uint8_t* in, int64_t nbytes, uint8_t* codes) {
  for (int64_t b = 0; b < nbytes; ++b) {
    codes[4 * b + 0] = (in[b] >> 6) & 3u;
    codes[4 * b + 1] = (in[b] >> 4) & 3u;
    codes[4 * b + 2] = (in[b] >> 2) & 3u;
    codes[4 * b + 3] = in[b] & 3u;
  }
}
/* pack.py:79-86: 32x32 tile -> faces f0 (r<16,c<16), f1 (r<16,c>=16),
 * f2 (r>=16,c<16), f3 (r>=16,c>=16), each row-major 16x16. */
void orc_tile_to_faces(const int8_t* tile, int8_t* faces) {
  for (int f = 0; f < 4; ++f)
    for (int rr = 0; rr < 16; ++rr)
      for (int cc = 0; cc < 16; ++cc)
        faces[f * 256 + rr * 16 + cc] = tile[(16 * (f / 2) + rr) * 32 + 16 * (f % 2) + cc];
}
/* pack.py:89-98 */
void orc_faces_to_tile(const int8_t* faces, int8_t* tile) {
  for (int f = 0; f < 4; ++f)
    for (int rr = 0; rr < 16; ++rr)
      for (int cc = 0; cc < 16; ++cc)
        tile[(16 * (f / 2) + rr) * 32 + 16 * (f % 2) + cc] = faces[f * 256 + rr * 16 + cc];
}
/* pack.py:194-203 */
int64_t orc_packed_tile_count(int64_t in_f, int64_t out_f) {
  return ((in_f + 31) / 32) * ((out_f + 31) / 32);
}
int64_t orc_packed_dram_bytes(int64_t in_f, int64_t out_f) {
  return orc_packed_tile_count(in_f, out_f) * 256;
}
/* pack.py:101-155: quantised (out_f, in_f) int8 -> transpose to (in_f, out_f)
 * -> zero-pad to 32 -> tiles in row-major (tile-row = in/K, tile-col = out/N)
 * order -> faces -> codes -> 4 per byte.  `packed` holds tile_count*256 bytes. */
void orc_pack_ternary_tilized(const int8_t* wq, int64_t out_f, int64_t in_f, uint8_t* packed) {
  int64_t kt_n = (in_f + 31) / 32, nt_n = (out_f + 31) / 32;
  int8_t tile[1024], faces[1024];
  uint8_t codes[1024];
  int64_t t = 0;
  for (int64_t kt = 0; kt < kt_n; ++kt)
    for (int64_t nt = 0; nt < nt_n; ++nt, ++t) {
      for (int r = 0; r < 32; ++r)
        for (int c = 0; c < 32; ++c) {
          int64_t k = kt * 32 + r, n = nt * 32 + c;
          tile[r * 32 + c] = (k < in_f && n < out_f) ? wq[n * in_f + k] : 0;
        }
      orc_tile_to_faces(tile, faces);
      orc_encode_ternary(faces, 1024, codes);
      orc_pack_4_to_byte(codes, 1024, packed + t * 256);
    }
}
/* pack.py:158-191 (values only; the per-tile scale multiply is applied by the
 * Python wrapper): packed tiles -> (in_f, out_f) int8. */
void orc_unpack_ternary_tilized(const uint8_t* packed, int64_t in_f, int64_t out_f, int8_t* wt) {
  int64_t kt_n = (in_f + 31) / 32, nt_n = (out_f + 31) / 32;
  int8_t tile[1024], faces[1024];
  uint8_t codes[1024];
  int64_t t = 0;
  for (int64_t kt = 0; kt < kt_n; ++kt)
    for (int64_t nt = 0; nt < nt_n; ++nt, ++t) {
      orc_unpack_byte_to_4(packed + t * 256, 256, codes);
      orc_decode_ternary(codes, 1024, faces);
      orc_faces_to_tile(faces, tile);
      for (int r = 0; r < 32; ++r)
        for (int c = 0; c < 32; ++c) {
          int64_t k = kt * 32 + r, n = nt * 32 + c;
          if (k < in_f && n < out_f) wt[k * out_f + n] = tile[r * 32 + c];
        }
    }
}

/* ------------------------------------------------------------------ */
/* Weight quantisation: src/bitnet_tt/utils/quantization.py:15-57     */
/* scale = max(mean(|W|), eps) computed the way numpy computes a       */
/* float32 mean: add.reduce in buffered blocks of 8192 elements, each  */
/* block summed pairwise (8 accumulators for blocks <= 128, halves     */
/* rounded down to a multiple of 8 above), blocks added in order into  */
/* a float32 accumulator, then float32(double(sum) / double(n)).       */
/* ------------------------------------------------------------------ */
static float pairwise_f32(const float* a, int64_t n) {
  if (n < 8) {
    float r = 0.0f;
    for (int64_t i = 0; i < n; ++i) r += a[i];
    return r;
  }
  if (n <= 128) {
    float r[8];
    int64_t i;
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    for (i = 8; i < n - (n % 8); i += 8)
      for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
  }
  int64_t n2 = n / 2;
  n2 -= n2 % 8;
  return pairwise_f32(a, n2) + pairwise_f32(a + n2, n - n2);
}
float orc_sum_f32_numpy(const float* a, int64_t n) {
  float acc = 0.0f;
  for (int64_t i = 0; i < n; i += 8192) acc += pairwise_f32(a + i, (n - i) < 8192 ? (n - i) : 8192);
  return acc;
}
/* quantization.py:15-29 */
float orc_compute_weight_scale(const float* w, int64_t n, float eps) {
  float* tmp = (float*)malloc((size_t)n * sizeof(float));
  for (int64_t i = 0; i < n; ++i) tmp[i] = fabsf(w[i]);
  float s = orc_sum_f32_numpy(tmp, n);
  free(tmp);
  float mean = (float)((double)s / (double)n);
  return mean > eps ? mean : eps; /* np.maximum(scale, eps) in float32 */
}
/* quantization.py:32-57: q = clip(round_half_even(W / s), -1, 1) */
float orc_weight_quant_ternary(const float* w, int64_t n, float eps, int8_t* q) {
  float s = orc_compute_weight_scale(w, n, eps);
  for (int64_t i = 0; i < n; ++i) {
    float r = rintf(w[i] / s);
    q[i] = (int8_t)(r > 1.0f ? 1 : (r < -1.0f ? -1 : (int)r));
  }
  return s;
}

/* ------------------------------------------------------------------ */
/* Activation quantisation: quantization.py:60-91 (== HF ActQuant,     */
/* transformers/integrations/bitnet.py:232-237): per row,              */
/* a = max(max|x|, eps); scale = 127/a (float32);                      */
/* q = clip(round_half_even(x * scale), -128, 127).                    */
/* The dequantisation factor used by this build's epilogue is          */
/* a_dq = a / 127 (float32).                                           */
/* ------------------------------------------------------------------ */
void orc_act_quant_absmax(const float* x, int64_t rows, int64_t k, float eps, int8_t* q,
                          float* scale, float* a_dq, int32_t* rowsum) {
  for (int64_t m = 0; m < rows; ++m) {
    const float* xr = x + m * k;
    float a = 0.0f;
    for (int64_t i = 0; i < k; ++i) {
      float v = fabsf(xr[i]);
      if (v > a) a = v;
    }
    if (!(a > eps)) a = eps;
    float s = 127.0f / a;
    int32_t rs = 0;
    for (int64_t i = 0; i < k; ++i) {
      float r = rintf(xr[i] * s);
      r = r > 127.0f ? 127.0f : (r < -128.0f ? -128.0f : r);
      q[m * k + i] = (int8_t)r;
      rs += (int32_t)r;
    }
    if (scale) scale[m] = s;
    if (a_dq) a_dq[m] = a / 127.0f;
    if (rowsum) rowsum[m] = rs;
  }
}

/* ------------------------------------------------------------------ */
/* RMSNorm: HF BitNetRMSNorm.forward (modeling_bitnet.py:53-58), used   */
/* by the reference as input_layernorm / ffn_sub_norm / attn_sub_norm   */
/* (layers/bitlinear.py:433-461, layers/ffn.py:180,                    */
/* inference/generator_batch32.py:721-727):                             */
/*   r = 1/sqrt(mean(x^2) + eps);  y = bf16(gamma * bf16(x * r)).       */
/* order 0: sum of squares in double, r rounded once to float32.        */
/* order 1: this build's fixed fp32 order -- 512 partial sums, partial  */
/* t adding x^2 (rounded) over 8-element chunks c = t, t+512, ...;      */
/* partials combined by the xor butterfly over 64 lanes (offsets        */
/* 32..1) inside each of 8 groups, then                                 */
/* ((g0+g1)+(g2+g3))+((g4+g5)+(g6+g7));                                 */
/* var = ss / K, r = 1/sqrt(var + eps) with correctly rounded ops.      */
/* ------------------------------------------------------------------ */
static float rms_inv_blocked(const float* x, int64_t k, float eps) {
  float part[512];
  int64_t nchunk = k / 8;
  for (int t = 0; t < 512; ++t) {
    float s = 0.0f;
    for (int64_t c = t; c < nchunk; c += 512)
      for (int j = 0; j < 8; ++j) {
        float v = x[c * 8 + j];
        float sq = v * v;
        s = s + sq;
      }
    part[t] = s;
  }
  float grp[8];
  for (int g = 0; g < 8; ++g) {
    float v[64], nv[64];
    for (int l = 0; l < 64; ++l) v[l] = part[g * 64 + l];
    for (int off = 32; off >= 1; off >>= 1) {
      for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ off];
      memcpy(v, nv, sizeof(v));
    }
    grp[g] = v[0];
  }
  float ss = ((grp[0] + grp[1]) + (grp[2] + grp[3])) + ((grp[4] + grp[5]) + (grp[6] + grp[7]));
  float var = ss / (float)k;
  float d = sqrtf(var + eps);
  return 1.0f / d;
}
static float rms_inv_double(const float* x, int64_t k, float eps) {
  double s = 0.0;
  for (int64_t i = 0; i < k; ++i) s += (double)x[i] * (double)x[i];
  return (float)(1.0 / sqrt(s / (double)k + (double)eps));
}
float orc_rms_inv(const float* x, int64_t k, float eps, int order) {
  return order == 1 ? rms_inv_blocked(x, k, eps) : rms_inv_double(x, k, eps);
}
void orc_rmsnorm_bf16(const uint16_t* x, const uint16_t* gamma, int64_t rows, int64_t k, float eps,
                      int order, uint16_t* y) {
  float* xf = (float*)malloc((size_t)k * sizeof(float));
  for (int64_t m = 0; m < rows; ++m) {
    for (int64_t i = 0; i < k; ++i) xf[i] = bf16_to_f32(x[m * k + i]);
    float r = orc_rms_inv(xf, k, eps, order);
    for (int64_t i = 0; i < k; ++i) {
      float t = bf16_to_f32(f32_to_bf16(xf[i] * r));
      y[m * k + i] = gamma ? f32_to_bf16(bf16_to_f32(gamma[i]) * t) : f32_to_bf16(t);
    }
  }
  free(xf);
}

/* ------------------------------------------------------------------ */
/* int32 accumulation: the exact contraction that ternary_matmul        */
/* performs (layers/bitlinear.py:336-341; kernels/device/               */
/* ternary_mm_compute.cpp:31-56 accumulates over Kt per output tile).   */
/* xq [M,K] int8, w [K,N] int8 ternary -> acc [M,N] int32.              */
/* ------------------------------------------------------------------ */
void orc_gemm_i8t(const int8_t* xq, const int8_t* w_kn, int64_t m_n, int64_t k_n, int64_t n_n,
                  int32_t* acc) {
  for (int64_t m = 0; m < m_n; ++m) {
    int32_t* row = acc + m * n_n;
    for (int64_t n = 0; n < n_n; ++n) row[n] = 0;
    for (int64_t k = 0; k < k_n; ++k) {
      int32_t xv = xq[m * k_n + k];
      if (!xv) continue;
      const int8_t* wr = w_kn + k * n_n;
      for (int64_t n = 0; n < n_n; ++n) row[n] += xv * (int32_t)wr[n];
    }
  }
}

/* Epilogue: out = bf16((float)acc * (s_w[segment(n)] * a_dq[m])).
 * Per-segment weight scales follow the fused QKV / gate||up builders
 * (layers/attention.py:481-506, layers/ffn.py:22-34); the single-segment
 * case is Linear's post-multiply (layers/bitlinear.py:351-352).
 * seg_end[i] is the exclusive column bound of segment i. */
void orc_scale_bf16(const int32_t* acc, int64_t m_n, int64_t n_n, const float* a_dq,
                    const float* seg_scale, const int64_t* seg_end, int nseg, uint16_t* out) {
  for (int64_t m = 0; m < m_n; ++m)
    for (int64_t n = 0; n < n_n; ++n) {
      int s = 0;
      while (s < nseg - 1 && n >= seg_end[s]) ++s;
      float f = seg_scale[s] * a_dq[m];
      out[m * n_n + n] = f32_to_bf16((float)acc[m * n_n + n] * f);
    }
}
/* layers/ffn.py:164-170 (ReLU then SQUARE on gate, times up), with the
 * bf16 materialisation of each intermediate as in HF's BitNetMLP:
 * h = bf16(bf16(relu(g)^2) * u). */
void orc_relu2_mul_bf16(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* h) {
  for (int64_t i = 0; i < n; ++i) {
    float gv = bf16_to_f32(g[i]);
    gv = gv > 0.0f ? gv : 0.0f;
    float sq = bf16_to_f32(f32_to_bf16(gv * gv));
    h[i] = f32_to_bf16(sq * bf16_to_f32(u[i]));
  }
}
/* Residual add of the decode loop (inference/generator_batch32.py:749, 756). */
void orc_add_bf16(const uint16_t* a, const uint16_t* b, int64_t n, uint16_t* y) {
  for (int64_t i = 0; i < n; ++i) y[i] = f32_to_bf16(bf16_to_f32(a[i]) + bf16_to_f32(b[i]));
}

/* ------------------------------------------------------------------ */
/* This build's device weight layout (not a reference format): the     */
/* checker for the repack kernel.  W [K,N] ternary, Kp = 128*ceil(K/128),*/
/* N % 32 == 0.  Word ((nt*KS + ks)*64 + lane)*4 + q holds 16 offset    */
/* codes u = w+1 for column nt*32 + (lane & 31) and rows                 */
/* k = ks*128 + q*32 + (lane >> 5)*16 + j, j = 0..15, code j at bit      */
/* 8*(j & 3) + 2*(j >> 2); rows k >= K hold u = 1 (zero weight).        */
/* ------------------------------------------------------------------ */
void orc_devlayout_encode(const int8_t* w_kn, int64_t k_n, int64_t n_n, uint32_t* dev) {
  int64_t ks_n = (k_n + 127) / 128, nt_n = n_n / 32;
  for (int64_t nt = 0; nt < nt_n; ++nt)
    for (int64_t ks = 0; ks < ks_n; ++ks)
      for (int lane = 0; lane < 64; ++lane)
        for (int q = 0; q < 4; ++q) {
          uint32_t word = 0;
          int64_t n = nt * 32 + (lane & 31);
          for (int j = 0; j < 16; ++j) {
            int64_t k = ks * 128 + q * 32 + (lane >> 5) * 16 + j;
            uint32_t u = (k < k_n) ? (uint32_t)(w_kn[k * n_n + n] + 1) : 1u;
            word |= u << (8 * (j & 3) + 2 * (j >> 2));
          }
          dev[((nt * ks_n + ks) * 64 + lane) * 4 + q] = word;
        }
}
void orc_devlayout_decode(const uint32_t* dev, int64_t k_n, int64_t n_n, int8_t* w_kn) {
  int64_t ks_n = (k_n + 127) / 128, nt_n = n_n / 32;
  for (int64_t nt = 0; nt < nt_n; ++nt)
    for (int64_t ks = 0; ks < ks_n; ++ks)
      for (int lane = 0; lane < 64; ++lane)
        for (int q = 0; q < 4; ++q) {
          uint32_t word = dev[((nt * ks_n + ks) * 64 + lane) * 4 + q];
          int64_t n = nt * 32 + (lane & 31);
          for (int j = 0; j < 16; ++j) {
            int64_t k = ks * 128 + q * 32 + (lane >> 5) * 16 + j;
            if (k < k_n) w_kn[k * n_n + n] = (int8_t)((int)((word >> (8 * (j & 3) + 2 * (j >> 2))) & 3u) - 1);
          }
        }
}
