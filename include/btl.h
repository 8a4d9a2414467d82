/*
 * btl.h -- C ABI of the MI355X (gfx950) BitLinear library (libbtl.so).
 *
 * The library is the drop-in for bitnet-tt's ternary-matmul path: the op
 * `ttnn.experimental.ternary_matmul(a, b, use_packed_ternary=True,
 * norm_weight=..., norm_epsilon=...)` called from
 * src/bitnet_tt/layers/bitlinear.py:336-341 and
 * src/bitnet_tt/inference/generator_batch32.py:721-727, its weight packing
 * (src/bitnet_tt/kernels/pack.py:101-191) and the quantisers of
 * src/bitnet_tt/utils/quantization.py:15-91.  Every entry point takes plain
 * device pointers, sizes and a hipStream_t; nothing allocates device memory
 * and every launch is ordered on the given stream, so the calls can be
 * recorded into a HIP graph.  A non-zero return is an error code and
 * btl_last_error() describes it (per calling thread).
 *
 * Data types: bf16 tensors are passed as uint16_t bit patterns.
 */
#ifndef BTL_H_
#define BTL_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* btl_stream_t; /* == hipStream_t */

/* ---- status codes ---------------------------------------------------- */
enum {
  BTL_OK = 0,
  BTL_ERR_NULL = 1,      /* a required pointer is NULL                  */
  BTL_ERR_SHAPE = 2,     /* sizes outside what the kernels support      */
  BTL_ERR_ALIGN = 3,     /* pointer or leading dimension misaligned     */
  BTL_ERR_WORKSPACE = 4, /* workspace smaller than btl_*_workspace_bytes */
  BTL_ERR_ARG = 5,       /* other invalid argument (mode, segments ...)  */
  BTL_ERR_LAUNCH = 6     /* the HIP runtime rejected a launch           */
};

/* ---- epilogue modes of the GEMM ------------------------------------- */
enum {
  /* out[m,n] = bf16(acc[m,n] * (seg_scale[seg(n)] * a_dq[m]))
   * [+ residual[m,n] in bf16 when residual != NULL].
   * Replaces ternary_matmul + Linear's multiply(out, weight_scale)
   * (src/bitnet_tt/layers/bitlinear.py:336-352). */
  BTL_EPI_SCALE = 0,
  /* N = 2F (gate||up, src/bitnet_tt/layers/ffn.py:22-34); with
   * g = bf16(acc[m,n] * s0 * a_dq[m]), u = bf16(acc[m,F+n] * s1 * a_dq[m]):
   * out[m,n] = bf16(bf16(relu(g)^2) * u), out is [M, F]
   * (src/bitnet_tt/layers/ffn.py:140-170). */
  BTL_EPI_RELU2_MUL = 1
};

#define BTL_MAX_SEGMENTS 4
#define BTL_MAX_K 16384

/* Co-residency rule of the kernels whose workgroups wait on each other
 * (btl_bitlinear_fused's one-launch decode path, btl_decode_step and its
 * floor): `grid` workgroups must fit on the device at once, per_cu (the
 * kernel's occupancy at its block size) x cus (the CUs the stream may use:
 * its CU mask, else all).  Returns BTL_OK, or BTL_ERR_LAUNCH with a message.
 * The library applies it with the queried values before every such launch:
 * the fused entry point then takes its two-launch path (same bits), the step
 * refuses (btl_decode_step_prepare and btl_decode_step return the error).
 * No counterpart in the reference (its op surfaces failures as RuntimeError,
 * src/bitnet_tt/layers/bitlinear.py:329-330); exported so that the rule can
 * be checked without a device. */
int btl_check_coresident(int64_t grid, int64_t per_cu, int64_t cus);

/* Last error message of the calling thread ("" if none). */
const char* btl_last_error(void);
/* ABI version (major*100 + minor). */
int btl_version(void);

/* ---- sizes (host only, never touch the GPU) ---------------------------
 * btl_packed_tile_count: src/bitnet_tt/kernels/pack.py:194-198.
 * btl_packed_dram_bytes: src/bitnet_tt/kernels/pack.py:201-203.
 * btl_devlayout_words:   uint32 words of the device weight layout of a
 *                        K x N ternary matrix (N % 32 == 0).
 * btl_act_bytes:         bytes of the quantised-activation buffer (32-row
 *                        blocks x 128-column superblocks, int8).
 * btl_gemm_workspace_bytes / btl_fused_workspace_bytes: workspace that
 *   btl_gemm_i8t2 / btl_bitlinear_fused need for the given shape and
 *   split-K factor (0 = the library's choice).                            */
int64_t btl_packed_tile_count(int64_t in_features, int64_t out_features);
int64_t btl_packed_dram_bytes(int64_t in_features, int64_t out_features);
int64_t btl_devlayout_words(int64_t K, int64_t N);
int64_t btl_act_bytes(int64_t M, int64_t K);
int btl_choose_splitk(int64_t M, int64_t K, int64_t N, int epilogue);
/* The tiling btl_gemm_i8t2 runs for a shape (no counterpart in the reference:
 * a planning query for benchmarks and tests).  rowsum_given: the caller
 * passes the row sums (the prefill BitLinear does).  info[6] = {kind (0
 * decode, 1 prefill 128x256 / 64x256 tiles, 2 prefill wide tiles), rows per
 * tile, column tiles of 32 per tile (kind 1: slots; relu2 pairs gate and up),
 * split-K factor, k-step groups (kind 2), column tiles per wave (kind 2)}.
 * The answer describes a call whose acc_out is NULL or 16-byte aligned: the
 * wide tiles store accumulators 16 bytes at a time, so a call with an acc_out
 * aligned to 4 bytes only runs the kind-1 tiles instead. */
int btl_gemm_tiling(int64_t M, int64_t K, int64_t N, int epilogue, int rowsum_given, int32_t* info);
int64_t btl_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int epilogue, int splitk);
int64_t btl_fused_workspace_bytes(int64_t M, int64_t K, int64_t N, int epilogue, int splitk);

/* ---- weight preparation (load time) ---------------------------------- */

/* Absmean ternary quantisation of a float32 latent weight with n elements
 * (src/bitnet_tt/utils/quantization.py:15-57):
 *   scale = max(mean(|W|), eps) with numpy's float32 summation order,
 *   q = clip(round_half_even(W / scale), -1, 1).
 * scratch: >= btl_weight_quant_scratch_bytes(n) bytes of device memory.
 * scale_out: device pointer to one float.                                  */
int64_t btl_weight_quant_scratch_bytes(int64_t n);
int btl_weight_quant_ternary(const float* w, int64_t n, float eps, int8_t* q, float* scale_out,
                             void* scratch, size_t scratch_bytes, btl_stream_t stream);

/* pack_ternary_tilized (src/bitnet_tt/kernels/pack.py:101-155): quantised
 * (out_features, in_features) int8 -> 2-bit tiles of the transposed matrix,
 * tile t = kt*Nt + nt, faces f0..f3, codes {0:00,+1:01,-1:10}, MSB first,
 * 256 bytes per tile.  packed: btl_packed_dram_bytes(in, out) bytes.     */
int btl_pack_tiles(const int8_t* w_outin, int64_t out_features, int64_t in_features, uint8_t* packed,
                   btl_stream_t stream);

/* unpack_ternary_tilized values (src/bitnet_tt/kernels/pack.py:158-191):
 * packed tiles -> (in_features, out_features) int8 in {-1,0,+1}
 * (code 0b11 decodes to 0, kernels/device/reader_ternary_in1.cpp:43-56). */
int btl_unpack_tiles(const uint8_t* packed, int64_t in_features, int64_t out_features, int8_t* w_kn,
                     btl_stream_t stream);

/* Repack the reference tile layout into the device layout the GEMM streams
 * (replaces the BFP2 mantissa repack of src/bitnet_tt/layers/bitlinear.py:
 * 221-248 / 272-297).  K = in_features (K % 32 == 0), N = out_features
 * (N % 32 == 0).  wdev: btl_devlayout_words(K, N) words.                  */
int btl_repack(const uint8_t* packed, int64_t K, int64_t N, uint32_t* wdev, btl_stream_t stream);

/* ---- activations ----------------------------------------------------- */

/* Per-token absmax int8 quantisation (src/bitnet_tt/utils/quantization.py:
 * 60-91), optionally preceded by RMSNorm with gain gamma
 * (HF BitNetRMSNorm order; src/bitnet_tt/layers/bitlinear.py:433-461):
 *   y = gamma ? bf16(gamma * bf16(x / sqrt(mean(x^2) + norm_eps))) : x
 *   a = max(max|y|, 1e-5); q = clip(rne(y * (127/a)), -128, 127)
 * Outputs: xa (btl_act_bytes(M,K), blocked layout the GEMM reads),
 * a_dq[32*ceil(M/32)] = a/127, optional rowsum[32*ceil(M/32)] = sum_k q,
 * optional act_scale[M] = 127/a (the scale quantization.py returns),
 * optional xq_rowmajor [M,K] int8 and y_rowmajor [M,K] bf16.
 * x is [M,K] with row stride ldx elements (ldx % 8 == 0).                */
int btl_quant_absmax(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma,
                     float norm_eps, int8_t* xa, float* a_dq, int32_t* rowsum, float* act_scale,
                     int8_t* xq_rowmajor, uint16_t* y_rowmajor, btl_stream_t stream);

/* RMSNorm alone (src/bitnet_tt/layers/bitlinear.py:356-461): y [M,K] bf16. */
int btl_rmsnorm(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma, float eps,
                uint16_t* y, btl_stream_t stream);

/* ---- the ternary GEMM ------------------------------------------------ */

/* acc[m,n] = sum_k q[m,k] * w[k,n] in int32 (exact), then the epilogue.
 * xa/a_dq as produced by btl_quant_absmax for the same M, K; rowsum:
 * optional [M] sum_k q, its rowsum output -- with it the M > 32 kernels skip
 * summing the operand themselves (NULL: they do; M <= 32 ignores it).
 * seg_scale/seg_end: host arrays of nseg (1..4) weight scales and exclusive
 * column ends (multiples of 32, last == N) -- per-projection scales of the
 * fused QKV / gate||up weights (src/bitnet_tt/layers/attention.py:481-506,
 * src/bitnet_tt/layers/ffn.py:22-34).  out: [M, N] (SCALE) or [M, N/2]
 * (RELU2_MUL) bf16; residual: optional [M, N] bf16 (SCALE only; may equal
 * out).  acc_out: optional [M, N] int32 copy of the exact accumulators.
 * splitk: 0 = library's choice (M <= 32); for M > 32 the library splits K
 * itself when the tile grid is smaller than the CU count and rowsum is
 * given.  workspace: btl_gemm_workspace_bytes(...) bytes (split-K partials
 * and counters; 0 for shapes that never split); its counters must be zero
 * before the first call and are left zero by every completed call.        */
int btl_gemm_i8t2(const int8_t* xa, const float* a_dq, const int32_t* rowsum, int64_t M, int64_t K, int64_t N, const uint32_t* wdev,
                  const float* seg_scale, const int64_t* seg_end, int nseg, int epilogue, const uint16_t* residual, uint16_t* out, int32_t* acc_out, void* workspace,
                  size_t workspace_bytes, int splitk, btl_stream_t stream);

/* The decode GEMM on the VALU (v_dot4_i32_i8) instead of MFMA: a measured
 * alternative, with no counterpart in the reference, kept to show the cost of
 * that formulation on MI355X (bench.py times it beside btl_gemm_i8t2).
 * acc_out[M, N] (int32, zero-filled by the caller) += the exact accumulators
 * of q @ w, q the int8 operand tile xa of btl_quant_absmax, w the device
 * layout, rowsum[M] = sum_k q.  M <= 32, K a multiple of 128, N of 32. */
int btl_gemm_i8t2_dot4(const int8_t* xa, const int32_t* rowsum, int64_t M, int64_t K, int64_t N,
                       const uint32_t* wdev, int32_t* acc_out, btl_stream_t stream);

/* Byte offset, inside a btl_bitlinear_fused workspace, of the 32-bit word
 * that is non-zero when a bounded wait of the single-launch decode kernel
 * ran out (the outputs of that call are then invalid).  The first 8192 bytes
 * of the workspace hold that kernel's launch counters; they must be zero
 * before the first call (a zero-filled workspace), and every completed call
 * leaves them ready for the next one, whatever shapes share the workspace.
 * A wait can only run out when the launch's workgroups are not all resident
 * at once (another kernel holding CUs); after that, zero-fill the workspace
 * again before reusing it. */
int64_t btl_fused_error_offset(void);

/* One BitLinear launch sequence: [RMSNorm(gamma) ->] absmax quant -> ternary
 * GEMM -> epilogue.  This is ternary_matmul(x, W, norm_weight=gamma,
 * norm_epsilon=eps) followed by the scale multiply
 * (src/bitnet_tt/inference/generator_batch32.py:721-727;
 * src/bitnet_tt/layers/bitlinear.py:309-353).  Arguments as above;
 * xq_debug [M,K] int8 optional.  workspace: btl_fused_workspace_bytes(...),
 * zero-filled once before first use.  For M <= 32 (decode) the whole
 * sequence is one launch: 32 workgroups quantise the token rows while the
 * GEMM workgroups already stream their weights. */
int btl_bitlinear_fused(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma,
                        float norm_eps, const uint32_t* wdev, int64_t N, const float* seg_scale,
                        const int64_t* seg_end, int nseg, int epilogue, const uint16_t* residual, uint16_t* out,
                        int32_t* acc_out, int8_t* xq_debug, void* workspace, size_t workspace_bytes, int splitk,
                        btl_stream_t stream);

/* Same as btl_bitlinear_fused, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference: it exists for those
 * callers only.  Instead of a caller workspace it uses a scratch array the
 * library holds in static device memory, BTL_NOALLOC_SCRATCH_BYTES per device
 * (each GPU the library runs on keeps its copy until the process ends); it
 * calls no allocating routine.  Shapes whose workspace
 * (btl_fused_workspace_bytes) exceeds that size are rejected with
 * BTL_ERR_WORKSPACE; every decode shape (M <= 32, K <= 16384, N <= 16384,
 * either epilogue) without a split-K request fits (the largest needs
 * 2,630,656 bytes).  error_word: optional device uint32 the caller owns;
 * a bounded wait that runs out stores a non-zero value there (the call's
 * outputs are then invalid; the library never clears it).  Every call on a
 * device shares that device's scratch and leaves it ready for the next call;
 * calls that overlap on one device (concurrent streams or threads) race on
 * it and must be serialised by the caller.  The first call on a device
 * clears the scratch with a kernel on `stream`. */
#define BTL_NOALLOC_SCRATCH_BYTES (3 << 20)
int btl_bitlinear_fused_noalloc(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* gamma,
                                float norm_eps, const uint32_t* wdev, int64_t N, const float* seg_scale,
                                const int64_t* seg_end, int nseg, int epilogue, const uint16_t* residual,
                                uint16_t* out, int32_t* acc_out, int8_t* xq_debug, uint32_t* error_word, int splitk,
                                btl_stream_t stream);

/* ---- persistent decode step ------------------------------------------- */

/* One BitLinear weight of the decode step: device layout (btl_repack), its
 * per-segment scales with exclusive column ends (host values), and the
 * RMSNorm gain applied to the BitLinear's input (bf16, device). */
typedef struct {
  const uint32_t* wdev;
  float seg_scale[BTL_MAX_SEGMENTS];
  int64_t seg_end[BTL_MAX_SEGMENTS];
  int nseg;
  const uint16_t* gamma;
} btl_layer_weight_t;

/* The BitLinear portion of a whole decode step as one launch: for every
 * layer l, QKV (RMSNorm(hidden; input_layernorm), output to qkv_out), o_proj
 * (RMSNorm(attn; attn_sub_norm), residual into hidden), gate||up (RMSNorm;
 * relu(g)^2*u into ffn_h), down (RMSNorm(ffn_h; ffn_sub_norm), residual into
 * hidden) -- src/bitnet_tt/inference/generator_batch32.py:713-761, with the
 * attention between QKV and o_proj replaced by the `attn` input (the same
 * buffer for every layer).  o_proj's row stage starts only after that row's
 * QKV output exists, as attention would.  Each BitLinear is the arithmetic of
 * btl_bitlinear_fused (bit-identical results).
 *
 * weights: [L][4] = qkv, o_proj, gate_up, down of each layer, with the gain
 * of the RMSNorm in front of each (qkv: three segments ending at Q, Q+KV,
 * NQKV; gate_up: two segments split at F).  Shapes: M <= 32 rows, H = the
 * attention width (o_proj is H -> H), H and F multiples of 128, H <= 3072,
 * F <= 7168, NQKV <= 4096 (a multiple of 64), L <= 64, and the GEMM units
 * max(NQKV/32, H/16, F/32) at most the CU count minus 32 (224 on a 256-CU
 * MI355X).  attn [M,H], hidden [M,H] (in/out), qkv_out
 * [M,NQKV] and ffn_h [M,F] bf16 (the last layer's values).
 *
 * Workspace (256-byte aligned): btl_decode_step_workspace_bytes(...) bytes,
 * zero-filled once, then prepared with btl_decode_step_prepare (which copies
 * the weight table into it and sets its operand tiles to their between-use
 * state, synchronously: not under graph capture) and used only by
 * btl_decode_step calls on one device and one stream.  One workgroup per CU
 * waits on the others: nothing else may hold the GPU's CUs during the launch
 * (a wait that runs out sets the word at btl_decode_step_error_offset and the
 * outputs are invalid; the workspace must then be zero-filled and prepared
 * again before the next btl_decode_step).  The error word names the first
 * failure: bits 0-7 the kind (1 row words, 2 row flags, 3 operand tile, 4 an
 * attention unit's QKV words, 5 a position outside the cache), bits 8-15
 * layer x 4 + BitLinear, bits 16-31 the workgroup. */
int64_t btl_decode_step_workspace_bytes(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L);
int64_t btl_decode_step_error_offset(void);
int btl_decode_step_prepare(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L,
                            const btl_layer_weight_t* weights, void* workspace, size_t workspace_bytes);
int btl_decode_step(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L, float eps, const uint16_t* attn,
                    uint16_t* hidden, uint16_t* qkv_out, uint16_t* ffn_h, void* workspace, size_t workspace_bytes,
                    btl_stream_t stream);

/* The whole decode step, attention included, as one launch: per layer
 * QKV -> decode attention -> o_proj -> gate||up -> down, as
 * src/bitnet_tt/inference/generator_batch32.py:713-761 runs it (attention
 * :728-746, the body of src/bitnet_tt/layers/attention.py:1040-1262).  The
 * attention of each (user, key-value head) runs on one GEMM workgroup between
 * its QKV and o_proj units, with the same code as btl_decode_attention (the
 * same bits); the rows' o_proj stage reads its output.  Same shapes as
 * btl_decode_step with the attention width H = Hq x 128 (Hq query heads of
 * 128, Hq / Hkv <= 4 per key-value head, NQKV = H + 2 Hkv 128) and M x Hkv
 * attention units within the GEMM workgroups.  The caches are [M][Hkv][S][128]
 * bf16 per layer, their addresses copied into the workspace by
 * btl_decode_step_attention_prepare (synchronously: not under graph capture;
 * again whenever they move); pos [M] int32 (device), the RoPE tables
 * [S][64] fp32 (rope_adjacent: pairs (2i, 2i+1), else (i, i+64)) and the score
 * scale as for btl_decode_attention.  Writes hidden (in/out), the last
 * layer's qkv_out [M][NQKV], attn_out [M][H] and ffn_h [M][F], and each
 * layer's cache row at pos.  A position outside [0, S) sets the error word
 * (kind 5) and the outputs are invalid.  The workspace is btl_decode_step's,
 * prepared by btl_decode_step_prepare as well. */
int btl_decode_step_attention_prepare(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L,
                                      const uint16_t* const* k_caches, const uint16_t* const* v_caches,
                                      void* workspace, size_t workspace_bytes);
int btl_decode_step_full(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L, float eps, int64_t Hkv, int64_t S,
                         const int32_t* pos, const float* rope_cos, const float* rope_sin, int rope_adjacent,
                         float scale, uint16_t* hidden, uint16_t* qkv_out, uint16_t* attn_out, uint16_t* ffn_h,
                         void* workspace, size_t workspace_bytes, btl_stream_t stream);

/* Measurement aid with no counterpart in the reference: btl_decode_step's
 * launch structure with no arithmetic.  The same workgroups, waits and
 * hand-off stores (row workgroups wait for every word of their row of the
 * previous BitLinear's output and set their flags; GEMM units wait for their
 * rows' flags and write their tagged output words), but no weight, operand
 * tile, gain or norm is read and nothing is computed: the launch time is the
 * latency floor of the step's 4L dependent hand-off pairs.  Same shapes and
 * workspace as btl_decode_step (it may be interleaved with btl_decode_step
 * calls on that workspace; it needs no btl_decode_step_prepare); writes only
 * the workspace. */
int btl_decode_step_floor(int64_t M, int64_t H, int64_t F, int64_t NQKV, int64_t L, void* workspace,
                          size_t workspace_bytes, btl_stream_t stream);

/* Test hook with no counterpart in the reference: the byte offsets (from an
 * operand tile's base) of the 16*KS 8-byte pieces that row m (0..31) of
 * btl_decode_step writes back to the between-use sentinel after a tile's
 * readers are done, for a tile of KS 128-column superblocks (1..128): the
 * same function the kernel calls.  Writes min(n, 16*KS) offsets; returns
 * BTL_OK or BTL_ERR_ARG / BTL_ERR_NULL.  Host only (no device call). */
int btl_decode_step_clear_share(int m, int64_t KS, int64_t* offsets, int64_t n);

/* ---- LM head (final norm is btl_rmsnorm) ------------------------------
 * Replaces the head matmul of src/bitnet_tt/inference/generator_batch32.py:
 * 768-811 (ttnn.matmul of the normed hidden state with the head weight that
 * src/bitnet_tt/model/bitnet.py:139-215 loads) and its argmax (:1170-1174,
 * ttnn.argmax over the vocabulary).
 *
 * btl_lm_head_weight_bytes: bytes of the head in the device layout (16 vocab
 *   rows x 32 k per KiB in MFMA operand order, K padded to a multiple of 256;
 *   0 for unsupported shapes: K % 16 != 0 or K > 3072).
 * btl_lm_head_repack: W [V,K] bf16 row-major (the HF / reference (vocab,
 *   hidden) matrix) -> the device layout.
 * btl_lm_head_workspace_bytes: workspace of btl_lm_head.  Its first 384
 *   bytes (argmax keys and a done counter) must be zero before the first call
 *   and every completed call leaves them zero; the rest is scratch. */
int64_t btl_lm_head_weight_bytes(int64_t V, int64_t K);
int64_t btl_lm_head_workspace_bytes(void);
int btl_lm_head_repack(const uint16_t* w, int64_t V, int64_t K, uint16_t* wdev, btl_stream_t stream);

/* logits[M,V] fp32 = xn[M,K] (bf16, the normalised rows) @ W^T, accumulated
 * in fp32 (MFMA bf16); tokens[M] int32 = the first index of each row's
 * largest logit (NaNs ignored).  M <= 32.  logits may be NULL. */
int btl_lm_head(const uint16_t* xn, int64_t M, int64_t K, int64_t V, const uint16_t* wdev, float* logits,
                int32_t* tokens, void* workspace, size_t workspace_bytes, btl_stream_t stream);

/* ---- decode attention between QKV and o_proj --------------------------
 * Replaces the decode attention of src/bitnet_tt/layers/attention.py:
 * 1040-1262 (nlp_create_qkv_heads_decode, rotary_embedding_llama,
 * paged_update_cache, scaled_dot_product_attention_decode,
 * nlp_concat_heads_decode), called from generator_batch32.py:739-746.
 *
 * qkv [B, (H + 2 Hkv) D] bf16 (the fused QKV output: Q heads, K heads, V
 * heads), pos [B] int32 on the device (each user's new position), rope_cos /
 * rope_sin [S, D/2] fp32 = cos / sin of position x theta^(-2i/D)
 * (utils/rope.py:7-23), k_cache / v_cache [B, Hkv, S, D] bf16.  RoPE pairs
 * (2i, 2i+1) when rope_adjacent (Q/K weights permuted as attention.py:
 * 462-478 does) else (i, i + D/2).  Writes the rotated k row and the v row
 * at pos into the caches, then out [B, H D] bf16 = softmax(scale q k^T) v over
 * positions [0, pos], query head h reading key-value head h / (H / Hkv).
 * D = 128, H / Hkv <= 4.  The workspace holds one int32 at
 * btl_decode_attention_error_offset (zero-filled before the first call): it
 * becomes non-zero when a position is outside [0, S) (that user's output is
 * then zero and its caches are not written). */
int64_t btl_decode_attention_workspace_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t S);
int64_t btl_decode_attention_error_offset(int64_t B, int64_t Hkv);
int btl_decode_attention(const uint16_t* qkv, int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t S,
                         const int32_t* pos, const float* rope_cos, const float* rope_sin, int rope_adjacent,
                         float scale, uint16_t* k_cache, uint16_t* v_cache, uint16_t* out, void* workspace,
                         size_t workspace_bytes, btl_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* BTL_H_ */
