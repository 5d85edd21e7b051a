/*
 * q4dec.h -- C ABI of the MI355X (gfx950) Qwen3-0.6B Q4 decode library
 * (libq4dec.so).
 *
 * Conventions (all entry points):
 *   - Every pointer is a device pointer owned by the caller, except the
 *     q4d_model_t / q4d_layer_t / q4d_matrix_t / q4d_kv_cache_t descriptor
 *     structs themselves, which live in host memory and are read on the host.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Calls are stream-ordered and asynchronous: no allocation and no host
 *     synchronisation happen inside.  Scratch memory is the caller's
 *     workspace (q4d_workspace_bytes / q4d_workspace_init).
 *   - Shapes, alignment, token ids and context lengths that the host can see
 *     are validated before any launch; a failing call returns a negative
 *     Q4D_ERR_* code and launches nothing (no memory traffic).  Values that
 *     only exist on the device (token ids and positions fed back from an
 *     earlier step) are range-checked by the kernels, which then skip the
 *     out-of-range work and set the workspace status word (q4d_read_status).
 *   - fp16 buffers are passed as uint16_t* (IEEE binary16 bit patterns).
 *
 * The Q4 weight format is the reference's (Source/Q4_FORMAT.md:75-140):
 * row-major [rows, cols/2] uint8, two signed int4 per byte with the even
 * column in the low nibble; uint16 Q2.14 scales [rows, cols/64].
 *
 * Reference interfaces replaced (paths in Tyler913/LLM_Accelerator):
 *   q4d_linear           <- manual_linear_from_weight
 *                           (Qwen3-0.6B-Base/python_each_module/common.py:137-145)
 *                           and the integer Q4 GEMV contract (Source/Q4_FORMAT.md:155-190)
 *   q4d_lm_head_argmax_batch <- q4d_lm_head_argmax per row of a batch
 *   q4d_gemm             <- manual_linear_from_weight over many activation rows
 *                           (x [B, S, K], common.py:137-145), for prefill and batched decode
 *   q4d_rms_norm         <- manual_rms_norm (common.py:129-134)
 *   q4d_qk_norm_rope     <- manual_rms_norm over heads + manual_rope_cos_sin +
 *                           manual_apply_rope (common.py:155-183, 258-268)
 *   q4d_kv_append        <- append_cache (common.py:186-189) with the physical
 *                           [layer][K/V][head][pos][dim] order of
 *                           23_export_kv_cache_append_vectors.py:64-84
 *   q4d_cached_attention <- manual_repeat_kv + manual_cached_attention
 *                           (common.py:192-228)
 *   q4d_embedding        <- embedding_table[token]
 *                           (10_validate_full_run_one_token.py:31)
 *   q4d_lm_head_argmax   <- final manual_rms_norm + LM head + argmax
 *                           (10_validate_full_run_one_token.py:52-56) with the
 *                           lowest-index tie rule of
 *                           56_export_persistent_multitoken_layer_golden.py:860
 *   q4d_decoder_layer    <- manual_decoder_layer_cached (common.py:231-298)
 *   q4d_run_one_token    <- run_manual_one_token
 *                           (10_validate_full_run_one_token.py:17-56) and the
 *                           hardware step qot_run_token
 *                           (FPGA_Project/software/qmap_one_token_runtime/
 *                            qmap_one_token_runtime.h:368-392)
 *   Q4D_ERR_*            <- QOT_ERR_* (qmap_one_token_runtime.h:17-29)
 */
#ifndef Q4DEC_H
#define Q4DEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; 0..-10 keep the meaning of QOT_ERR_* (qmap_one_token_runtime.h:17-29). */
enum {
  Q4D_OK = 0,
  Q4D_ERR_BUSY = -1,
  Q4D_ERR_BAD_LAYER = -2,
  Q4D_ERR_BAD_TABLE = -3,    /* bad model/weight descriptor */
  Q4D_ERR_BAD_ADDR = -4,     /* misaligned pointer */
  Q4D_ERR_TIMEOUT = -5,
  Q4D_ERR_STATUS = -6,       /* device-side status word reported an error */
  Q4D_ERR_NULL = -7,
  Q4D_ERR_BAD_TOKEN = -8,
  Q4D_ERR_CAPACITY = -9,     /* workspace too small / batch too large */
  Q4D_ERR_CONTEXT = -10,     /* position outside [0, max_ctx) */
  Q4D_ERR_SHAPE = -11,       /* unsupported or inconsistent shape */
  Q4D_ERR_LAUNCH = -12,      /* HIP launch error */
  Q4D_ERR_DTYPE = -13
};

/* Device status word bits (q4d_read_status). */
enum {
  Q4D_STATUS_BAD_TOKEN = 1,
  Q4D_STATUS_BAD_POSITION = 2,
  /* XCD-split decode layer only (no reference counterpart): the workgroups of one kv
   * head (blockIdx % 8 equal) did not all run on one XCD, or an exchange between them
   * did not complete within 20 ms (the results of that call are not valid). */
  Q4D_STATUS_XCD_MAP = 4,
  Q4D_STATUS_SYNC_TIMEOUT = 8
};

enum { Q4D_F16 = 0, Q4D_F32 = 1, Q4D_BF16 = 2 };

typedef struct q4d_matrix {
  const uint8_t* w;   /* [rows, cols/2] packed int4 */
  const uint16_t* s;  /* [rows, cols/64] Q2.14 */
  int32_t rows;
  int32_t cols;
} q4d_matrix_t;

/* Attribute names follow the HF layer object read by common.py:245-296. */
typedef struct q4d_layer {
  q4d_matrix_t q_proj, k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj;
  const float* input_layernorm;           /* [hidden] */
  const float* post_attention_layernorm;  /* [hidden] */
  const float* q_norm;                    /* [head_dim] */
  const float* k_norm;                    /* [head_dim] */
} q4d_layer_t;

typedef struct q4d_model {
  int32_t hidden_size;        /* 1024 */
  int32_t intermediate_size;  /* 3072 */
  int32_t num_layers;         /* 28 */
  int32_t num_q_heads;        /* 16 */
  int32_t num_kv_heads;       /* 8 */
  int32_t head_dim;           /* 128 */
  int32_t vocab_size;         /* 151936 */
  int32_t max_ctx;            /* rows of the RoPE tables and KV capacity */
  float rms_norm_eps;         /* 1e-6 */
  float attn_scaling;         /* head_dim ** -0.5 */
  const q4d_layer_t* layers;  /* host array [num_layers] */
  q4d_matrix_t embed_tokens;  /* tied embedding / LM head [vocab, hidden] */
  const float* final_norm;    /* [hidden] */
  const float* rope_cos;      /* [max_ctx, head_dim/2] fp32, cos(pos * inv_freq) */
  const float* rope_sin;      /* [max_ctx, head_dim/2] fp32 */
} q4d_model_t;

/* fp16 KV cache, [num_layers][2 (K,V)][batch][num_kv_heads][max_ctx][head_dim]. */
typedef struct q4d_kv_cache {
  uint16_t* data;
  int32_t num_layers;
  int32_t batch;
  int32_t num_kv_heads;
  int32_t max_ctx;
  int32_t head_dim;
} q4d_kv_cache_t;

/* ---- library / workspace ------------------------------------------------ */
int q4d_version(void);
const char* q4d_status_string(int code);
/* Bytes of workspace needed by the fused entry points for `batch` sequences. */
size_t q4d_workspace_bytes(const q4d_model_t* model, int32_t batch);
/* Zero the workspace counters, exchange flags and status word (call once after
 * allocation, and again to clear a status word that reported an error).  With batch 1
 * it also runs the XCD-split plan's one-time device check (q4d_set_decode_plan), which
 * synchronises `stream` the first time on each device. */
int q4d_workspace_init(void* ws, size_t ws_bytes, const q4d_model_t* model, int32_t batch, void* stream);
/* Precision of fp32 activations inside the GEMVs: 2 (default) = each value
 * enters as an fp16 hi + fp16 lo pair (~22 significant bits); 1 = rounded to
 * fp16.  Process-wide; set it before launching work. */
int q4d_set_activation_precision(int32_t mode);
/* Kernel plan of the batch-1 decode layer (q4d_decoder_layer, q4d_run_one_token*; no
 * reference counterpart, the arithmetic is the same): Q4D_DECODE_XCD (default) runs a
 * layer as two launches split over the GPU's eight XCDs, one kv head per XCD, with the
 * XCD's workgroups exchanging data through its L2; Q4D_DECODE_STAGED runs the five
 * per-stage launches of q4d_layer_stage.  XCD applies to the Qwen3-0.6B shape (hidden
 * 1024, 16/8 heads of 128, intermediate 3072), max_ctx <= 32768 and activation
 * precision 2, on a device that passes a one-time check (at least 256 CUs, one 320-thread
 * workgroup of each XCD-split kernel fits on a CU, and a probe launch of 256 workgroups
 * places workgroups b, b + 8, b + 16, ... on one XCD and the eight residues on eight
 * XCDs, as an unpartitioned MI355X does); other models and devices run staged.  The
 * check runs in q4d_workspace_init (batch 1) or at the first decode call, synchronises
 * the stream once, and is skipped (staged plan, not cached) while the stream is being
 * captured into a graph.  Process-wide; set it before capturing graphs.  Returns the
 * previous plan. */
enum { Q4D_DECODE_XCD = 0, Q4D_DECODE_STAGED = 1 };
int q4d_set_decode_plan(int32_t plan);
/* The plan a batch-1 decode call with `model` runs on the current device now
 * (Q4D_DECODE_XCD or Q4D_DECODE_STAGED); runs the device check if it has not run yet.
 * No reference counterpart. */
int q4d_decode_plan_active(const q4d_model_t* model, void* stream);
/* Test hook of the device check (no reference counterpart): mode 1 reports every device
 * as unsuitable, so the staged plan runs; mode 0 (default) restores the check.  Returns
 * the previous mode. */
int q4d_diag_set_xcd_check(int32_t mode);
/* Copy the device status word into *out (synchronises `stream`). */
int q4d_read_status(const void* ws, size_t ws_bytes, const q4d_model_t* model, int32_t batch,
                    int32_t* out, void* stream);

/* ---- primitive ops ------------------------------------------------------- */
/* y[m, :] = W x[m, :] for m < batch.  x: [batch, cols] (x_dtype), y: [batch, rows] (y_dtype).
 * Supported cols: 1024, 2048, 3072; rows even. */
int q4d_linear(const q4d_matrix_t* w, const void* x, int32_t x_dtype, void* y, int32_t y_dtype,
               int32_t batch, void* stream);
/* No counterpart in the reference (it applies one matrix per call,
 * manual_linear_from_weight, common.py:137-145): q4d_linear over `count` independent matrices of one shape, each with
 * its own activations and output, up to 64 per launch: w is a host array of count
 * descriptors (equal rows and cols), x and y host arrays of count device pointers as in
 * q4d_linear.  Each y[i] equals q4d_linear(&w[i], x[i], ...) bit for bit.  Every descriptor
 * and pointer is checked before the first launch: a call that returns an error has written
 * no output.  For callers that
 * apply many small matrices at once (expert or adapter weights), where one launch per matrix
 * would cost more than its bytes. */
int q4d_linear_group(const q4d_matrix_t* w, const void* const* x, int32_t x_dtype, void* const* y, int32_t y_dtype,
                     int32_t batch, int32_t count, void* stream);
/* y = x * rsqrt(mean(x^2) + eps) * gamma over the last dim (fp32 in). */
int q4d_rms_norm(const float* x, const float* gamma, float eps, int32_t rows, int32_t dim,
                 void* y, int32_t y_dtype, void* stream);
/* Per-head RMSNorm with gamma, then rotate-half RoPE at positions[b].
 * x: fp32 [batch, heads, head_dim] (in place allowed); positions: device int32 [batch]. */
int q4d_qk_norm_rope(const float* x, float* y, const float* gamma, float eps, int32_t batch,
                     int32_t heads, int32_t head_dim, const float* rope_cos, const float* rope_sin,
                     int32_t max_ctx, const int32_t* positions, int32_t* status, void* stream);
/* RoPE only: y[b,h,:] = x*cos[b] + rotate_half(x)*sin[b] (common.py:148-152,173-183).
 * x, y: fp32 [batch, heads, head_dim]; cos, sin: fp32 [batch, head_dim] (full width). */
int q4d_apply_rope(const float* x, float* y, const float* cos, const float* sin, int32_t batch,
                   int32_t heads, int32_t head_dim, void* stream);
/* manual_apply_rope over a sequence (common.py:173-183, as 04_validate_qk_norm_rope.py:59-60
 * calls it for a whole prompt): y[b,h,s,:] = x*cos[b,s] + rotate_half(x)*sin[b,s].
 * x, y: fp32 [batch, heads, seq, head_dim] (y must not alias x); cos, sin: fp32
 * [batch, seq, head_dim].  q4d_apply_rope is the seq = 1 case. */
int q4d_apply_rope_seq(const float* x, float* y, const float* cos, const float* sin, int32_t batch,
                       int32_t heads, int32_t seq, int32_t head_dim, void* stream);
/* manual_rotate_half (common.py:148-152): y = cat(-x[..., d/2:], x[..., :d/2]) per row.
 * x, y: fp32 [rows, head_dim], not aliased. */
int q4d_rotate_half(const float* x, float* y, int64_t rows, int32_t head_dim, void* stream);
/* manual_causal_attention (common.py:201-216; called by 06_validate_attention.py:71):
 * out = softmax(q k^T * scaling + causal mask) v per head, GQA with q head h reading kv head
 * h / (q_heads / kv_heads) (manual_repeat_kv, common.py:192-198, without the copy).
 * q, out: fp32 [batch, q_heads, seq, head_dim]; k, v: fp32 [batch, kv_heads, seq,
 * head_dim]; head_dim 128; 16-byte aligned.  The operands are rounded to fp16 (q with
 * scaling folded in) for the MFMA flash-attention kernel of q4d_prefill, which keeps
 * the probabilities in fp16 and accumulates in fp32; the softmax weights are not
 * materialised.  ws: q4d_causal_attention_workspace_bytes(batch, q_heads, kv_heads, seq)
 * bytes, 256-byte aligned. */
size_t q4d_causal_attention_workspace_bytes(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t seq);
int q4d_causal_attention(const float* q, const float* k, const float* v, float* out, int32_t batch,
                         int32_t q_heads, int32_t kv_heads, int32_t seq, int32_t head_dim, float scaling,
                         void* ws, size_t ws_bytes, void* stream);
/* Write k, v (fp32 [batch, kv_heads, head_dim]) into layer `layer` of the cache at positions[b];
 * either of k / v may be NULL to leave that plane untouched. */
int q4d_kv_append(const q4d_kv_cache_t* kv, int32_t layer, const float* k, const float* v,
                  const int32_t* positions, int32_t* status, void* stream);
/* GQA decode attention over cache positions [0, positions[b]] of `layer`.
 * q: fp32 [batch, q_heads, head_dim] already normed/roped; out: fp16 [batch, q_heads*head_dim]. */
int q4d_cached_attention(const q4d_model_t* model, const q4d_kv_cache_t* kv, int32_t layer,
                         const float* q, const int32_t* positions, void* out, int32_t out_dtype,
                         void* ws, size_t ws_bytes, void* stream);
/* hidden[b, :] = dequant(embed_tokens[tokens[b], :]) (fp32). */
int q4d_embedding(const q4d_matrix_t* table, const int32_t* tokens, int32_t batch, float* hidden,
                  int32_t* status, void* stream);
/* Final RMSNorm + tied LM head + argmax (lowest index wins ties).
 * hidden: fp32 [1, hidden]; out_token int32 [1]; out_score fp32 [1] (the winning logit);
 * logits: optional fp32 [vocab] (NULL to skip). */
int q4d_lm_head_argmax(const q4d_model_t* model, const float* hidden, int32_t* out_token,
                       float* out_score, float* logits, void* ws, size_t ws_bytes, void* stream);

/* Batched q4d_lm_head_argmax: final RMSNorm, LM head on MFMA (hidden rounded to fp16,
 * Q4 tiles dequantised to fp16, fp32 accumulation) and a two-stage argmax per row
 * (lowest index wins ties).  hidden fp32 [batch, hidden]; out_tokens int32 [batch];
 * out_scores fp32 [batch]; logits optional fp32 [batch, vocab].  vocab % 128 == 0. */
int q4d_lm_head_argmax_batch(const q4d_model_t* model, const float* hidden, int32_t batch,
                             int32_t* out_tokens, float* out_scores, float* logits, void* ws,
                             size_t ws_bytes, void* stream);

/* y[m, :] = W x[m, :] for m < M on MFMA, for many activation rows sharing the weights
 * (prefill, batched decode): x fp16 [M, cols]; y [M, rows] in y_dtype; if resid is not
 * NULL, y (fp32) = resid + W x (resid may alias y).  Q4 tiles are dequantised to fp16
 * (one rounding of q*scale) and accumulated in fp32.  rows % 128 == 0, cols % 64 == 0. */
int q4d_gemm(const q4d_matrix_t* w, const uint16_t* x, int32_t M, void* y, int32_t y_dtype,
             const float* resid, void* stream);
/* q4d_gemm with the K dimension split over `ksplit` blocks per output tile
 * (1..16, at most cols / 64; 0 = chosen for the shape), for few activation
 * rows where the output tiles alone leave the device idle: each split's fp32
 * tile goes to `part` (ksplit x M x rows floats, 16-byte aligned), then the
 * splits are added in order.  Same result as q4d_gemm up to the grouping of
 * the fp32 sums.  No counterpart in the reference; it is the batched-decode
 * projection path of q4d_decode_batch, exported for callers with scratch. */
int q4d_gemm_splitk(const q4d_matrix_t* w, const uint16_t* x, int32_t M, void* y, int32_t y_dtype,
                    const float* resid, float* part, size_t part_bytes, int32_t ksplit, void* stream);

/* Integer Q4 GEMV of the reference's fixed-point path, exact:
 *   y_q26[n]    = sum_g scale[n,g] * sum_{j<64} x[64g+j] * q[n,64g+j]   (int64, Q26)
 *   y_q12_12[n] = sat24(y_q26[n] >> 14)  (arithmetic shift, signed 24-bit saturation)
 * x_int: Q12.12 (or Q4.12) activations as int32 in 24-bit signed range, [cols], 16-byte
 * aligned; either output may be NULL; *saturated (may be NULL) is incremented once per
 * saturated row.  cols % 64 == 0, cols <= 3072.
 * Replaces compute_q4_gemv_q26 + q26_to_q12_12
 * (Qwen3-0.6B-Base/python_each_module/28_export_mlp_gate_up_vectors.py:124-138) and
 * q4_gemv_from_ints (13_export_q4_gemv_vectors.py:138-154). */
int q4d_linear_q26(const q4d_matrix_t* w, const int32_t* x_int, int64_t* y_q26, int32_t* y_q12_12,
                   int32_t* saturated, void* stream);

/* Argmax over n int64 scores: the highest, and among equal scores the lowest index (the
 * streamed LM-head scan, 56_export_persistent_multitoken_layer_golden.py:766-798,860). */
int q4d_argmax_q26(const int64_t* scores, int32_t n, int32_t* out_token, int64_t* out_score, void* stream);

/* ---- fused decode ---------------------------------------------------------- */
/* One cached decoder layer (batch 1): hidden_out = layer(hidden_in); appends
 * K/V at positions[0] of the cache.  hidden_in and hidden_out may alias. */
int q4d_decoder_layer(const q4d_model_t* model, int32_t layer, const float* hidden_in,
                      float* hidden_out, const q4d_kv_cache_t* kv, const int32_t* positions,
                      void* ws, size_t ws_bytes, void* stream);
/* One stage of a decoder layer (batch 1), in the order q4d_decoder_layer runs them.  The
 * stages follow the per-layer QMAP stage boundaries of the hardware path
 * (qot_layer_qmap_bases_t, qmap_one_token_runtime.h:31-42):
 *   Q4D_STAGE_QKV       input RMSNorm + q|k|v projection      -> workspace qkv
 *   Q4D_STAGE_ATTENTION q/k RMSNorm + RoPE + KV append + split-K GQA attention -> workspace
 *                       chunk partials (max, sum, partial output per 128-position chunk)
 *   Q4D_STAGE_O_PROJ    merge of the chunk partials + o_proj + residual:
 *                       hidden_out = hidden_in + W_o attn
 *   Q4D_STAGE_GATE_UP   post-attention RMSNorm(hidden_out) + gate/up + SiLU*up -> workspace act
 *   Q4D_STAGE_DOWN      down_proj + residual: hidden_out += W_d act
 * Running the five stages in order equals one q4d_decoder_layer call. */
enum { Q4D_STAGE_QKV = 0, Q4D_STAGE_ATTENTION = 1, Q4D_STAGE_O_PROJ = 2, Q4D_STAGE_GATE_UP = 3,
       Q4D_STAGE_DOWN = 4 };
int q4d_layer_stage(const q4d_model_t* model, int32_t layer, int32_t stage, const float* hidden_in,
                    float* hidden_out, const q4d_kv_cache_t* kv, const int32_t* positions, void* ws,
                    size_t ws_bytes, void* stream);
/* Embedding -> all layers -> final norm -> LM head argmax for tokens[0] at
 * positions[0] (batch 1).  Writes next_token[0] and score[0]; logits optional. */
int q4d_run_one_token(const q4d_model_t* model, const int32_t* tokens, const int32_t* positions,
                      const q4d_kv_cache_t* kv, int32_t* next_token, float* score, float* logits,
                      void* ws, size_t ws_bytes, void* stream);
/* q4d_run_one_token followed by the greedy feedback of q4d_advance, in the same
 * launches: the LM head's last block also sets tokens[0] = next_token[0], positions[0] += 1
 * and, if hist_tokens is not NULL and *hist_count < hist_capacity, records the token and
 * score at index *hist_count and increments it.  The embedding of tokens[0] is built inside
 * layer 0's q|k|v launch, so a step is two launches fewer than q4d_run_one_token +
 * q4d_advance, with the same results bit for bit.  The generation loop it replaces feeds the
 * argmax back as the next input (10_validate_full_run_one_token.py:135-172; on the board
 * qot_decode_token_ids, qmap_one_token_runtime.h:399-497). */
int q4d_run_one_token_feedback(const q4d_model_t* model, int32_t* tokens, int32_t* positions,
                               const q4d_kv_cache_t* kv, int32_t* next_token, float* score, float* logits,
                               int32_t* hist_tokens, float* hist_scores, int32_t* hist_count,
                               int32_t hist_capacity, void* ws, size_t ws_bytes, void* stream);
/* q4d_run_one_token without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops or harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Its scratch is a 4 MiB device array
 * inside the library, one per GPU, held until the process ends; the call allocates
 * nothing.  Models whose batch-1 workspace (q4d_workspace_bytes(model, 1)) exceeds
 * 4 MiB are rejected with Q4D_ERR_CAPACITY (Qwen3-0.6B shapes: max_ctx <= 27328).
 * status: device int32[1], caller-owned and caller-cleared; the step ORs its
 * Q4D_STATUS_* bits into it.  All calls on one GPU share that GPU's scratch, so calls
 * that overlap on one GPU (two streams, two threads) race; serialise them.  Results
 * equal q4d_run_one_token's bit for bit. */
int q4d_run_one_token_noalloc(const q4d_model_t* model, const int32_t* tokens, const int32_t* positions,
                              const q4d_kv_cache_t* kv, int32_t* next_token, float* score, float* logits,
                              int32_t* status, void* stream);
/* One decode step for `batch` independent sequences (batched decode): tokens[b] at
 * positions[b] (device int32 [batch], each sequence its own position) through embedding,
 * all layers (projections as MFMA GEMMs over the batch, GQA attention per sequence) and the
 * LM head; writes next_tokens[b], scores[b] and, if logits is not NULL, logits
 * [batch, vocab] (fp32).  Activations enter each projection as fp16.  The KV cache must
 * have batch >= `batch`; the workspace is sized by q4d_workspace_bytes(model, batch).
 * No counterpart in the reference (its decode is batch 1); per sequence it computes
 * run_manual_one_token (10_validate_full_run_one_token.py:17-56). */
int q4d_decode_batch(const q4d_model_t* model, const int32_t* tokens, const int32_t* positions,
                     int32_t batch, const q4d_kv_cache_t* kv, int32_t* next_tokens, float* scores,
                     float* logits, void* ws, size_t ws_bytes, void* stream);
/* Bytes of workspace q4d_prefill needs for up to `max_tokens` tokens per call. */
size_t q4d_prefill_workspace_bytes(const q4d_model_t* model, int32_t max_tokens);
/* Prefill: n_tokens tokens (device int32 [n_tokens]) of sequence `seq` of the cache at positions
 * start_pos .. start_pos + n_tokens - 1, through embedding, all layers and the LM head of the last
 * token.  Appends the K/V rows of every position (attention over [0, position] for each token) and
 * writes next_token[0] / score[0] (and logits [vocab] if not NULL) for the last token.  Equals
 * n_tokens consecutive run_manual_one_token steps
 * (10_validate_full_run_one_token.py:17-56, driven as in :81-135) with the projections as MFMA
 * GEMMs (activations rounded to fp16) and causal attention on MFMA (q and probabilities in fp16).
 * Positions must satisfy start_pos + n_tokens <= max_ctx (Q4D_ERR_CONTEXT otherwise). */
int q4d_prefill(const q4d_model_t* model, const int32_t* tokens, int32_t n_tokens, int32_t start_pos,
                int32_t seq, const q4d_kv_cache_t* kv, int32_t* next_token, float* score, float* logits,
                void* ws, size_t ws_bytes, void* stream);
/* Advance a device-resident decode loop: tokens[0] = next_token[0], positions[0] += 1, and,
 * if hist_tokens is not NULL and *hist_count < hist_capacity, record next_token[0] and score[0]
 * at index *hist_count and increment it.  Lets a captured graph replay q4d_run_one_token
 * without host round trips (the device form of qot_decode_token_ids,
 * qmap_one_token_runtime.h:399+). */
int q4d_advance(int32_t* tokens, int32_t* positions, const int32_t* next_token, const float* score,
                int32_t* hist_tokens, float* hist_scores, int32_t* hist_count, int32_t hist_capacity,
                void* stream);
/* q4d_advance with the decode session's stop rules on the device (qot_session.c:41-60, in
 * this order after each generated token: end-of-text, end-of-turn, new-token budget, context
 * cap).  stop_state: device int32[8] = {done, stop reason (Q4D_SESSION_STOP_*), generated
 * count, max new tokens, end-of-text id or -1, end-of-turn id or -1, max context, 0}; the
 * caller sets it before the first generated token.  Once done nothing advances, so further
 * replayed steps recompute the last step unchanged; the host reads `done` between replays. */
int q4d_advance_session(int32_t* tokens, int32_t* positions, const int32_t* next_token, const float* score,
                        int32_t* hist_tokens, float* hist_scores, int32_t* hist_count, int32_t hist_capacity,
                        int32_t* stop_state, void* stream);

/* ---- fixed-point (RTL-exact) decode ------------------------------------------
 * The integer arithmetic of the reference's FPGA datapath, bit for bit
 * (Qwen3-0.6B-Base/python_each_module/56_export_persistent_multitoken_layer_golden.py:468-561
 * and the stage exporters it loads, :862-875).  Formats (56_...:1087-1095):
 *   hidden state / layer output   signed 24-bit Q14.10 in int32
 *   norm, projection, RoPE, attention and MLP values   signed 24-bit Q12.12 in int32
 *   gammas Q8.7 and RoPE cos/sin Q1.15 in int16; scores Q24.24 int64; probabilities
 *   unsigned Q0.16; LM-head logits Q26 int64.
 * Shifts are arithmetic (floor); every stage output saturates to signed 24 bits.
 * The Q4 matrices are those of q4d_model_t (same layout); the KV cache holds int32 Q12.12
 * words in the reference's physical order [layer][K/V][kv_head][position][dim]
 * (23_export_kv_cache_append_vectors.py:64-84).  Batch 1, max_ctx <= 4096. */
typedef struct q4d_fixed_layer {
  const int16_t* input_gamma;  /* [hidden] Q8.7 */
  const int16_t* post_gamma;   /* [hidden] Q8.7 */
  const int16_t* q_gamma;      /* [head_dim] Q8.7 */
  const int16_t* k_gamma;      /* [head_dim] Q8.7 */
} q4d_fixed_layer_t;

typedef struct q4d_fixed_model {
  const q4d_model_t* base;          /* shapes, layers[l].*_proj and the tied embed_tokens (Q4);
                                       its float norm/RoPE pointers are not read */
  const q4d_fixed_layer_t* layers;  /* host array [base->num_layers] */
  const int16_t* final_gamma;       /* [hidden] Q8.7 */
  const int16_t* rope_cos;          /* [base->max_ctx, head_dim] Q1.15 (54_export_rope_runtime_table.py) */
  const int16_t* rope_sin;          /* [base->max_ctx, head_dim] Q1.15 */
  int32_t score_scale_q0_31;        /* round(head_dim**-0.5 * 2**31) (56_...:449-451) */
} q4d_fixed_model_t;

typedef struct q4d_fixed_kv {
  int32_t* data;  /* [num_layers][2][num_kv_heads][max_ctx][head_dim] int32 Q12.12 */
  int32_t num_layers;
  int32_t num_kv_heads;
  int32_t max_ctx;
  int32_t head_dim;
} q4d_fixed_kv_t;

/* Saturation / status counters of the fixed-point workspace (q4d_fixed_read_counts),
 * one per stage, as in the per-position "saturation" record of 56_...:634-650. */
enum {
  Q4D_FX_STATUS = 0,  /* device status bits (Q4D_STATUS_*) */
  Q4D_FX_SAT_INPUT_NORM = 1, Q4D_FX_SAT_QKV = 2, Q4D_FX_SAT_QK_NORM = 3, Q4D_FX_SAT_ROPE = 4,
  Q4D_FX_SAT_ATTENTION = 5, Q4D_FX_SAT_O_PROJ = 6, Q4D_FX_SAT_POST_RESIDUAL = 7,
  Q4D_FX_SAT_POST_NORM = 8, Q4D_FX_SAT_GATE = 9, Q4D_FX_SAT_UP = 10, Q4D_FX_SAT_SILU = 11,
  Q4D_FX_SAT_MLP_HIDDEN = 12, Q4D_FX_SAT_DOWN = 13, Q4D_FX_SAT_LAYER_RESIDUAL = 14,
  Q4D_FX_SAT_FINAL_NORM = 15, Q4D_FX_COUNTS = 16
};

/* Host only (no device access): the exp LUT (n_exp = 257: round(exp(-i/16) * 2**20),
 * 46_export_chained_attention_score_value_vectors.py:88-93) and the sigmoid LUT
 * (n_sigmoid = 1025: round(sigmoid(-8 + i/64) * 2**16) clipped to 65535,
 * 29_export_mlp_silu_mul_vectors.py:77-83). */
int q4d_fixed_tables(int32_t* exp_lut, int32_t n_exp, int32_t* sigmoid_lut, int32_t n_sigmoid);
/* Workspace of the fixed-point decode (256-byte aligned); init uploads the LUTs and clears
 * the counters. */
size_t q4d_fixed_workspace_bytes(const q4d_fixed_model_t* model);
int q4d_fixed_workspace_init(void* ws, size_t ws_bytes, const q4d_fixed_model_t* model, void* stream);
/* Copies the first n (<= Q4D_FX_COUNTS) counters to host memory, each summed over the
 * workspace's 64 stripes of counter words (synchronises the stream). */
int q4d_fixed_read_counts(const void* ws, size_t ws_bytes, int32_t* counts, int32_t n, void* stream);

/* Stage entry points (device buffers; the fused calls below run the same device code). */
/* Integer RMSNorm of `rows` vectors of `dim` elements.  kind 0 = hidden (Q14.10 in,
 * mean >> 10, eps 1, 2**26 / rms, output >> 21; 17_export_rmsnorm_fixed_vectors.py:108-150,
 * 27_...:110-149, 32_...:101-141), kind 1 = head (Q12.12 in, mean >> 7, eps 17, 2**28 / rms,
 * output >> 23; 22_export_qk_norm_rope_fixed_vectors.py:127-166; dim must be 128).
 * stats (may be NULL): int64 [rows][6] = sum_squares, mean_square, sqrt_radicand, rms,
 * inv_rms, saturated elements. */
int q4d_fixed_rms_norm(const int32_t* x, const int16_t* gamma, int32_t rows, int32_t dim, int32_t kind,
                       int32_t* y, int64_t* stats, void* stream);
/* Per-head q/k RMSNorm then RoPE of one position (22_...:169-212): q [q_heads,128],
 * k [kv_heads,128] Q12.12; cos/sin: the position's Q1.15 table row [128].  q_norm / k_norm
 * (may be NULL) receive the normalised heads.  With q_gamma and k_gamma both NULL the norm
 * is skipped and the inputs are rotated as given (fixed_rope_reference alone, 18_...). */
int q4d_fixed_qk_norm_rope(const int32_t* q, const int32_t* k, int32_t q_heads, int32_t kv_heads,
                           const int16_t* q_gamma, const int16_t* k_gamma, const int16_t* cos_row,
                           const int16_t* sin_row, int32_t* q_rope, int32_t* k_rope, int32_t* q_norm,
                           int32_t* k_norm, void* stream);
/* Attention of one token over cache positions 0 .. cache_length-1 of `layer`
 * (attention_score_value, 56_...:347-381): raw[h,p] = q_h . k_p (int64), scaled =
 * (raw * score_scale) >> 31, LUT softmax (46_...:96-121), out = sat24((sum_p prob * v) >> 16).
 * q_rope [q_heads,128]; exp_lut: device int32 [257] (q4d_fixed_tables).  raw, scaled
 * (int64), lut_index, prob (int32) [q_heads, cache_length] may be NULL.  ws: 256-byte
 * aligned scratch of q4d_fixed_attention_workspace_bytes(q_heads, kv->max_ctx) bytes (scores
 * and chunk maxima between the two launches). */
size_t q4d_fixed_attention_workspace_bytes(int32_t q_heads, int32_t max_ctx);
int q4d_fixed_attention(const q4d_fixed_kv_t* kv, int32_t layer, int32_t q_heads, int32_t cache_length,
                        const int32_t* q_rope, int32_t score_scale_q0_31, const int32_t* exp_lut,
                        int32_t* out, int64_t* raw, int64_t* scaled, int32_t* lut_index, int32_t* prob,
                        void* ws, size_t ws_bytes, void* stream);
/* Writes k [kv_heads,128] and v [kv_heads,128] at positions[0] of `layer` (23_...:64-84). */
int q4d_fixed_kv_append(const q4d_fixed_kv_t* kv, int32_t layer, const int32_t* positions,
                        const int32_t* k, const int32_t* v, void* stream);
/* SwiGLU of the fixed path (29_export_mlp_silu_mul_vectors.py:86-93, 56_...:547-556):
 * index = gate on the 1/64 grid of [-8, 8]; silu = sat24((gate * lut[index]) >> 16);
 * hidden = sat24((silu * up) >> 12).  sigmoid_lut: device int32 [1025]; lut_index,
 * sigmoid, silu_gate may be NULL. */
int q4d_fixed_silu_mul(const int32_t* gate, const int32_t* up, int32_t n, const int32_t* sigmoid_lut,
                       int32_t* hidden, int32_t* lut_index, int32_t* sigmoid, int32_t* silu_gate,
                       void* stream);
/* out = sat24(hidden + (x >> 2)): a Q12.12 branch output onto the Q14.10 residual stream
 * (56_...:530-533, 558-561). */
int q4d_fixed_residual_add(const int32_t* hidden, const int32_t* x, int32_t n, int32_t* out, void* stream);
/* Q14.10 embedding rows of the tied Q4 table: (q * scale) >> 4 (56_...:214-221). */
int q4d_fixed_embedding(const q4d_matrix_t* table, const int32_t* tokens, int32_t n, int32_t* hidden,
                        void* stream);
/* Integer Q4 projection of one activation vector (compute_matrix_outputs,
 * 21_export_qmap_qkv_projection_image.py:163-191; projection, 56_...:300-317):
 * y[r] = sat24((sum_g s[r,g] * sum_{k in g} q[r,k] * x[k]) >> 14), Q12.12 in and out.
 * x: device int32 [w->cols], w->cols in {1024, 2048, 3072}.  With input_gamma (device
 * int16 Q8.7 [1024]) non-NULL, x is the Q14.10 hidden state and passes through the hidden
 * RMSNorm first, as in the fused input-norm + q|k|v projection.  y: device int32
 * [w->rows], not overlapping x.  Saturations are not counted. */
int q4d_fixed_q4_gemv(const q4d_matrix_t* w, const int32_t* x, const int16_t* input_gamma, int32_t* y,
                      void* stream);

/* One fixed-point decoder layer at positions[0] (run_fixed_layer, 56_...:468-561): input
 * norm + q|k|v, q/k norm + RoPE + KV append + attention, o_proj + residual, post norm +
 * gate/up + SiLU*up, down + residual.  hidden_in / hidden_out: Q14.10 [hidden]; may alias. */
int q4d_fixed_decoder_layer(const q4d_fixed_model_t* model, int32_t layer, const int32_t* hidden_in,
                            int32_t* hidden_out, const q4d_fixed_kv_t* kv, const int32_t* positions,
                            void* ws, size_t ws_bytes, void* stream);
/* Embedding, every layer, final RMSNorm and the full-vocabulary tied-Q4 LM-head scan
 * (56_...:684-798): next_token[0] = the highest Q26 logit, lowest row on ties;
 * score[0] its Q26 value; logits (int64 [vocab]) optional; hidden_out (Q14.10 [hidden],
 * the last layer's output) optional. */
int q4d_fixed_run_one_token(const q4d_fixed_model_t* model, const int32_t* tokens, const int32_t* positions,
                            const q4d_fixed_kv_t* kv, int32_t* next_token, int64_t* score, int64_t* logits,
                            int32_t* hidden_out, void* ws, size_t ws_bytes, void* stream);

/* ---- decode session (host state machine) ------------------------------------
 * Serial prompt prefill, greedy feedback, stop reasons and the context cap, one
 * model invocation per q4d_session_step: the state machine and event stream of the
 * board session loop qot_session (FPGA_Project/software/qmap_prompt_demo/qot_session.h,
 * qot_session.c:101-276), with the context cap and vocabulary size as parameters
 * (the board fixes QOT_MAX_CONTEXT = 256, QOT_VOCAB_SIZE = 151936) and the runner
 * being one GPU decode step.  Host memory only; the runners synchronise their stream. */
#define Q4D_SESSION_DEFAULT_EOS_TOKEN_ID 151643u    /* QOT_SESSION_DEFAULT_EOS_TOKEN_ID */
#define Q4D_SESSION_DEFAULT_IM_END_TOKEN_ID 151645u /* QOT_SESSION_DEFAULT_IM_END_TOKEN_ID */
enum { Q4D_SESSION_ERR_STATE = -100 };              /* QOT_SESSION_ERR_STATE */
enum {
  Q4D_SESSION_STATE_UNINITIALIZED = 0, Q4D_SESSION_STATE_IDLE, Q4D_SESSION_STATE_PREFILL,
  Q4D_SESSION_STATE_DECODE, Q4D_SESSION_STATE_STOPPING, Q4D_SESSION_STATE_DONE, Q4D_SESSION_STATE_ERROR
};
enum {
  Q4D_SESSION_STOP_NONE = 0, Q4D_SESSION_STOP_EOS, Q4D_SESSION_STOP_IM_END, Q4D_SESSION_STOP_MAX_NEW,
  Q4D_SESSION_STOP_CONTEXT, Q4D_SESSION_STOP_HW_ERROR
};
enum {
  Q4D_SESSION_EVENT_NONE = 0, Q4D_SESSION_EVENT_PREFILL, Q4D_SESSION_EVENT_TOKEN, Q4D_SESSION_EVENT_DONE,
  Q4D_SESSION_EVENT_ERROR
};

/* Result of one model invocation (qot_result_t's status / token_id / score_q26). */
typedef struct q4d_token_result {
  uint32_t status;    /* device status word (0 = ok) */
  uint32_t token_id;  /* argmax of the logits */
  float score;        /* its logit (float path) */
  int32_t reserved;
  int64_t score_q26;  /* its Q26 score (fixed-point path) */
} q4d_token_result_t;

/* One full-model token invocation (qot_session_runner_fn without the board handles). */
typedef int (*q4d_session_runner_fn)(void* runner_context, uint32_t input_token_id, uint32_t position,
                                     q4d_token_result_t* result);

typedef struct q4d_session_options {
  uint32_t max_new_tokens;
  uint32_t eos_token_id;
  uint32_t im_end_token_id;
  uint32_t stop_on_eos;
  uint32_t stop_on_im_end;
} q4d_session_options_t;

typedef struct q4d_session_event {
  int32_t kind;         /* Q4D_SESSION_EVENT_* */
  int32_t stop_reason;  /* Q4D_SESSION_STOP_* */
  uint32_t input_token_id;
  uint32_t input_position;
  uint32_t prompt_tokens_consumed;
  uint32_t generated_index;
  int32_t error_code;
  q4d_token_result_t result;
} q4d_session_event_t;

typedef struct q4d_session {
  uint32_t start_position, max_context, vocab_size;
  q4d_session_runner_fn runner;
  void* runner_context;
  const uint32_t* prompt;  /* caller's, valid until DONE or ERROR */
  uint32_t prompt_count, prompt_index, next_position, pending_token, generated_count;
  q4d_session_options_t options;
  q4d_token_result_t last_result;
  int32_t last_error;
  int32_t state;        /* Q4D_SESSION_STATE_* */
  int32_t stop_reason;  /* Q4D_SESSION_STOP_* */
} q4d_session_t;

/* Runner contexts.  io: caller's device int32[8], 16-byte aligned (token, position, next
 * token, -, score).  The float runner also reads the workspace status word. */
typedef struct q4d_gpu_runner {
  const q4d_model_t* model;
  const q4d_kv_cache_t* kv;
  void* ws;
  size_t ws_bytes;
  void* stream;
  int32_t* io;
} q4d_gpu_runner_t;
typedef struct q4d_fixed_runner {
  const q4d_fixed_model_t* model;
  const q4d_fixed_kv_t* kv;
  void* ws;
  size_t ws_bytes;
  void* stream;
  int32_t* io;
} q4d_fixed_runner_t;

/* qot_session_default_options: max_new 1, stop on EOS 151643 and <|im_end|> 151645. */
void q4d_session_default_options(q4d_session_options_t* options);
/* qot_session_init (qot_session.c:101-123); Q4D_ERR_CONTEXT if start_position >= max_context. */
int q4d_session_init(q4d_session_t* session, uint32_t start_position, uint32_t max_context, uint32_t vocab_size,
                     q4d_session_runner_fn runner, void* runner_context);
/* qot_session_begin (qot_session.c:125-172). */
int q4d_session_begin(q4d_session_t* session, const uint32_t* prompt_token_ids, uint32_t prompt_token_count,
                      const q4d_session_options_t* options);
/* qot_session_step (qot_session.c:174-245): at most one runner call, one event. */
int q4d_session_step(q4d_session_t* session, q4d_session_event_t* event);
void q4d_session_reset(q4d_session_t* session);
int q4d_session_is_terminal(const q4d_session_t* session);
const char* q4d_session_state_name(int32_t state);
const char* q4d_session_stop_reason_name(int32_t reason);
/* Runners to pass to q4d_session_init with a q4d_gpu_runner_t / q4d_fixed_runner_t context:
 * one q4d_run_one_token / q4d_fixed_run_one_token step (the board's qot_run_token). */
int q4d_session_gpu_runner(void* runner_context, uint32_t input_token_id, uint32_t position,
                           q4d_token_result_t* result);
int q4d_session_fixed_runner(void* runner_context, uint32_t input_token_id, uint32_t position,
                             q4d_token_result_t* result);

/* ---- float -> Q4 weight conversion ------------------------------------------
 * The reference's quantizer (quantize_weight_q4, 13_export_q4_gemv_vectors.py:101-135;
 * the same rule in 26_...:126-145, 28_...:103-121, 30_...:103-121, 33_...:95-113) for a
 * device matrix: per 64-column group absmax, code = rint(fp32(absmax / 7) * 2^14)
 * round-half-even, 1 for a nonzero group that rounds to 0; q = clip(rint(w / (code /
 * 2^14)), -8, 7), packed two per byte with the even column in the low nibble.
 * weight: device fp32 (Q4D_F32) or bf16 (Q4D_BF16) [rows, ld], row-major, cols a
 * multiple of 64, ld >= cols; packed: device uint8 [rows, cols/2]; scale: device uint16
 * [rows, cols/64].  status: device int32 [2] that the caller zeroes first; the kernel
 * adds the number of groups whose code exceeds 65535 (the reference raises "Q4 scale does
 * not fit unsigned 16-bit Q2.14") to status[0] and of groups holding a non-finite value to
 * status[1]; those groups' outputs are not meaningful. */
int q4d_quantize_q4(const void* weight, int32_t dtype, int64_t ld, int32_t rows, int32_t cols, uint8_t* packed,
                    uint16_t* scale, int32_t* status, void* stream);
/* The same conversion for `count` matrices of one shape, dtype and row pitch (the
 * reference converts a checkpoint's matrices one quantize_weight_q4 call each, 56_...:241-291):
 * weights[i], packed[i], scales[i] are device pointers as in q4d_quantize_q4, passed in HOST
 * arrays of count entries.  Up to 64 matrices go in one launch (more are split into launches
 * of 64); the codes and scales equal count separate q4d_quantize_q4 calls bit for bit, and
 * status[0] / status[1] receive the bad-group counts summed over all the matrices. */
int q4d_quantize_q4_batch(const void* const* weights, int32_t dtype, int64_t ld, int32_t rows, int32_t cols,
                          int32_t count, uint8_t* const* packed, uint16_t* const* scales, int32_t* status,
                          void* stream);

/* ---- diagnostics --------------------------------------------------------------
 * No counterpart in the reference; for measurement.  Launches n dependent kernels on
 * `stream`, kernel i with grid (grid_x[i], grid_y[i]) of block[i] threads (a multiple of
 * 64, at most 1024), each doing one global read of the previous kernel's 4 KB output and
 * (block 0) writing its own: the launch floor of a chain of kernels with those grids.
 * grid_x, grid_y, block: host arrays of n (1..4096); buf: device, 2048 floats, 16-byte
 * aligned. */
int q4d_diag_launch_chain(const int32_t* grid_x, const int32_t* grid_y, const int32_t* block, int32_t n,
                          float* buf, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q4DEC_H */
