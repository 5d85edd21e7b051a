// Host-side internals shared by the libq4dec translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/q4dec.h"

namespace q4d {

// Decode attention splits the context into chunks of this many positions
// (kAttnChunkLong when the consumer merges the partials); workspace partials
// are sized for the shorter chunk.
constexpr int kAttnChunk = 64;
constexpr int kAttnChunkLong = 128;
// Upper bound on the LM-head grid (one partial argmax per block).
constexpr int kLmMaxBlocks = 2048;
// XCD-split batch-1 layer (q4d_xcd.hip): one kv head per XCD, 32 workgroups per XCD,
// attention chunk records of (max, sum, 2 pad, o[128]) floats.
constexpr int kXcdGroups = 8;
constexpr int kXcdBlocks = 32;
constexpr int kXcdApRec = 132;
constexpr int kXcdInter = 3072;

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// fp16 activations of at most 64 rows in 32-column chunks ("tiled"): element (m, k) at
// ((k / 32) * 64 + m) * 32 + k % 32, so 16 rows x 32 columns (one MFMA operand fragment
// set) are 1 KB of contiguous memory.  The batched decode step (2 <= batch <= 64) keeps
// the GEMMs' fp16 inputs this way; kF16Tiled is the y_dtype / out_dtype code of the
// kernels that write it.
constexpr int kXtRows = 64;
constexpr int kF16Tiled = 0x100;
__host__ __device__ inline size_t xt_index(int m, int k) {
  return ((size_t)(k >> 5) * kXtRows + m) * 32 + (k & 31);
}
inline bool xt_batch(int batch) { return batch > 1 && batch <= kXtRows; }

// The streaming LM head's two-level argmax hand-off: blocks g, g + 8, ... fold their
// best (score, index) key into group key g (u64 at byte 128 g) and count in on group
// counter g (int32 at 1024 + 128 g); the last block of each group counts in on the top
// counter (int32 at 2048).  Each word has a 128-byte line of its own.
constexpr int kLmGroups = 8;
constexpr size_t kLmHandBytes = 2048 + 128;

// Byte offsets of the regions of a caller-provided workspace.
struct WsLayout {
  size_t status;     // int32[64]: [0] = status bits
  size_t counters;   // int32[batch * kv_heads] attention split counters
  size_t lm_hand;    // LM-head argmax hand-off, kLmHandBytes (zeroed with the counters)
  size_t xflags;     // u32 [8][32] exchange flags of the XCD-split layer (zeroed with the counters)
  size_t hidden;     // f32 [batch, hidden]          residual stream
  size_t qkv;        // f32 [batch, (qh + 2 kvh) * d] raw q|k|v projections
  size_t qrope;      // f32 [batch, qh * d]          q after norm + RoPE (primitive path)
  size_t attn;       // f32 [batch, qh * d]          attention output (o_proj input)
  size_t act;        // f32 [batch, intermediate]    silu(gate) * up
  size_t part_ml;    // f32 [batch, qh, nsplit, 2]   split max / sum
  size_t part_acc;   // f32 [batch, qh, nsplit, d]   split partial outputs
  size_t xh;         // f16 [batch, max(hidden, qh*d, intermediate)]  MFMA-path activations
  size_t row_score;  // f32 [batch, vocab/128]  batched LM-head argmax partials
  size_t row_idx;    // i32 [batch, vocab/128]
  size_t gemm_part;  // f32 [8][batch][max(q|k|v rows, 2 x intermediate)] split-K partial tiles
  size_t gemm_part_floats;
  // XCD-split batch-1 layer (q4d_xcd.hip)
  size_t xqkv;       // f32 [8][512]      each XCD's raw q|k|v rows
  size_t xap;        // f32 [8][32][2][kXcdApRec] attention chunk partials
  size_t xac;        // f32 [8][384]      each XCD's SwiGLU activations
  size_t xpo;        // f32 [8][hidden]   o_proj split-K partials
  size_t xpd;        // f32 [8][hidden]   down split-K partials
  size_t xhx;        // f32 [hidden]      layer input (residual base of launch B)
  size_t xhx2;       // f32 [hidden]      post-attention state (residual base of the next layer)
  size_t total;
  int nsplit_max;
};

inline WsLayout ws_layout(const q4d_model_t* m, int batch) {
  WsLayout L{};
  const size_t A = 256;
  const int d = m->head_dim, qh = m->num_q_heads, kvh = m->num_kv_heads;
  L.nsplit_max = (m->max_ctx + kAttnChunk - 1) / kAttnChunk;
  const int xrows = xt_batch(batch) ? kXtRows : batch;  // rows of the fp16 GEMM inputs
  size_t o = 0;
  L.status = o;   o = align_up(o + 64 * 4, A);
  L.counters = o; o = align_up(o + (size_t)(batch * kvh) * 4, A);
  L.lm_hand = o;  o = align_up(o + kLmHandBytes, A);
  L.xflags = o;   o = align_up(o + (size_t)kXcdGroups * kXcdBlocks * 4, A);
  L.hidden = o;   o = align_up(o + (size_t)batch * m->hidden_size * 4, A);
  L.qkv = o;      o = align_up(o + (size_t)batch * (qh + 2 * kvh) * d * 4, A);
  L.qrope = o;    o = align_up(o + (size_t)batch * qh * d * 4, A);
  L.attn = o;     o = align_up(o + (size_t)(batch > xrows ? batch : xrows) * qh * d * 4, A);
  L.act = o;      o = align_up(o + (size_t)(batch > xrows ? batch : xrows) * m->intermediate_size * 4, A);
  L.part_ml = o;  o = align_up(o + (size_t)batch * qh * L.nsplit_max * 2 * 4, A);
  L.part_acc = o; o = align_up(o + (size_t)batch * qh * L.nsplit_max * d * 4, A);
  int wmax = m->hidden_size;
  if (qh * d > wmax) wmax = qh * d;
  if (m->intermediate_size > wmax) wmax = m->intermediate_size;
  const size_t nparts = (size_t)(m->vocab_size + 127) / 128;
  L.xh = o;        o = align_up(o + (size_t)xrows * wmax * 2, A);
  L.row_score = o; o = align_up(o + (size_t)batch * nparts * 4, A);
  L.row_idx = o;   o = align_up(o + (size_t)batch * nparts * 4, A);
  {
    const size_t w1 = (size_t)(qh + 2 * kvh) * d, w2 = 2 * (size_t)m->intermediate_size;
    L.gemm_part_floats = 8 * (size_t)batch * (w1 > w2 ? w1 : w2);
    L.gemm_part = o; o = align_up(o + L.gemm_part_floats * 4, A);
  }
  {
    const size_t hs = (size_t)m->hidden_size * 4;
    L.xqkv = o; o = align_up(o + (size_t)kXcdGroups * 4 * d * 4, A);
    L.xap = o;  o = align_up(o + (size_t)kXcdGroups * kXcdBlocks * 2 * kXcdApRec * 4, A);
    L.xac = o;  o = align_up(o + (size_t)m->intermediate_size * 4, A);
    L.xpo = o;  o = align_up(o + kXcdGroups * hs, A);
    L.xpd = o;  o = align_up(o + kXcdGroups * hs, A);
    L.xhx = o;  o = align_up(o + hs, A);
    L.xhx2 = o; o = align_up(o + hs, A);
  }
  L.total = o;
  return L;
}

template <class T>
inline T* ws_ptr(void* ws, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

inline bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline int check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? Q4D_OK : Q4D_ERR_LAUNCH;
}

// ---- GEMV launcher ---------------------------------------------------------
// X_ATTN: fp32 activations merged in the prologue from split-K decode-attention
// partials (part_ml / part_acc of the attention kernel run with merge = 0).
// X_EMB: RMSNorm of the tied Q4 embedding row of token emb_token[0] (the first
// layer's q|k|v projection of a one-token step); block 0 also writes the fp32 row
// to emb_out (the residual stream), and an id outside the table gives zeros and
// sets Q4D_STATUS_BAD_TOKEN in emb_status, as the embedding kernel does.
enum XMode { X_F16 = 0, X_F32 = 1, X_RMS = 2, X_ATTN = 3, X_EMB = 4 };
enum EpMode { EP_F16 = 0, EP_F32 = 1, EP_RESID = 2, EP_SWIGLU = 3, EP_ARGMAX = 4, EP_ROPE = 5 };

struct GemvArgs {
  // Up to three row segments stacked into one logical [rows, K] matrix.
  const uint8_t* w[3];
  const uint16_t* s[3];
  int seg_end[3];   // cumulative row ends
  int nseg;
  int rows;         // logical rows (PAIR mode: rows of each of the two segments)
  int cols;         // K
  // Activations.
  const void* x;        // X_F16: fp16 [batch, K]; X_F32 / X_RMS: fp32 [batch, K]
  // X_RMS in the streaming LM head only: x is x + x_parts[0] + ... + x_parts[7]
  // (fp32 [8][K], summed in this order, as the XCD-split layer forms its output);
  // block 0 stores that sum to x_out when x_out is set.
  const float* x_parts;
  float* x_out;
  const float* gamma;   // X_RMS
  float eps;            // X_RMS
  // Epilogue.
  void* y;              // output (see EpMode)
  const float* resid;   // EP_RESID: y = resid + W x
  // EP_ARGMAX.
  float* logits;        // optional
  char* lm_hand;        // kLmHandBytes, zero before the first launch; reset by the last block
  int* out_token;
  float* out_score;
  int batch;
  // X_ATTN: chunk partials [batch][heads][nsplit_max] of (max, sum) and [head_dim]
  const float* part_ml;
  const float* part_acc;
  const int32_t* positions;  // device [batch]: the attended positions are 0 .. positions[b]
  int nsplit_max;
  int attn_chunk;            // positions per chunk
  // X_EMB.
  const int32_t* emb_token;  // device [1]
  const uint8_t* emb_w;      // tied table codes [emb_vocab, K/2] and Q2.14 scales [emb_vocab, K/64]
  const uint16_t* emb_s;
  int emb_vocab;
  float* emb_out;            // block 0 writes the fp32 embedding row here
  int32_t* emb_status;
  // EP_ARGMAX with greedy feedback (adv_tokens set): the last block also stores the
  // token as the next input, advances the position and records the history, as
  // advance_kernel does.
  int32_t* adv_tokens;
  int32_t* adv_positions;
  int32_t* hist_tokens;      // optional
  float* hist_scores;        // optional
  int32_t* hist_count;
  int hist_cap;
};

// Validates geometry, picks the kernel instance and launches.  Returns Q4D_*.
int launch_gemv(const GemvArgs& a, int xmode, int epmode, bool pair, hipStream_t stream);
// count independent [rows, cols] matrices with their own activations and outputs, up to 64
// per launch (plain linear modes only: X_F16 / X_F32 in, EP_F16 / EP_F32 out).
int launch_gemv_group(int rows, int cols, int batch, const uint8_t* const* w, const uint16_t* const* s,
                      const void* const* x, void* const* y, int count, int xm, int xp, int ep, hipStream_t st);

// ---- other launchers ---------------------------------------------------------
int launch_rms_norm(const float* x, const float* gamma, float eps, int rows, int dim, void* y,
                    int y_dtype, hipStream_t stream);
int launch_embedding(const q4d_matrix_t* t, const int32_t* tokens, int batch, float* hidden,
                     int32_t* status, hipStream_t stream);
int launch_qk_norm_rope(const float* x, float* y, const float* gamma, float eps, int batch,
                        int heads, int head_dim, const float* cosT, const float* sinT, int max_ctx,
                        const int32_t* positions, int32_t* status, hipStream_t stream);
int launch_kv_append(const q4d_kv_cache_t* kv, int layer, const float* k, const float* v,
                     const int32_t* positions, int32_t* status, hipStream_t stream);

struct AttnArgs {
  // fused = 1: q/k/v are raw projections in `qkv` ([batch, (qh+2kvh)*d]); the
  // kernel applies q/k RMSNorm + RoPE and appends k/v to the cache.
  // fused = 0: q is ready ([batch, qh*d], normed, roped); cache already holds pos.
  int fused;
  // merge = 1: the last block of each (kv head, sequence) merges the chunk
  // partials into `out`.  merge = 0: partials only (`chunk` = 64 or 128 positions
  // per chunk), merged by the consumer (the o_proj GEMV with X_ATTN).
  int merge;
  int chunk;
  const float* qkv;
  const float* q;
  const float* q_gamma;
  const float* k_gamma;
  float eps;
  float scaling;
  const float* rope_cos;
  const float* rope_sin;
  uint16_t* kcache;  // layer's K plane: [batch][kvh][max_ctx][d]
  uint16_t* vcache;
  const int32_t* positions;
  int batch, qh, kvh, d, max_ctx, nsplit_max;
  float* part_ml;
  float* part_acc;
  int* counters;
  void* out;
  int out_dtype;
  int32_t* status;
};
int launch_attention(const AttnArgs& a, hipStream_t stream);

// ---- XCD-split batch-1 decoder layer (q4d_xcd.hip) -----------------------------
struct XcdBufs {
  uint32_t* flags;  // [8][32]
  float* qkv;       // [8][512]
  float* ap;        // [8][32][2][kXcdApRec]
  float* ac;        // [8][384]
  float* po;        // [8][1024]
  float* pd;        // [8][1024]
  float* hx;        // [1024] layer input
  float* hx2;       // [1024] post-attention state
  int32_t* status;
};
struct XcdAttnArgs {
  const uint8_t *qw, *kw, *vw, *ow;
  const uint16_t *qs, *ks, *vs, *os;
  const float* in_gamma;
  const float* q_gamma;
  const float* k_gamma;
  float eps;
  float qscale;            // attention scaling * log2(e)
  const float* rope_cos;   // [max_ctx][64]
  const float* rope_sin;
  uint16_t* kcache;        // the layer's K plane [kv_heads][max_ctx][128] (one sequence)
  uint16_t* vcache;
  const int32_t* positions;
  int max_ctx;
  // layer input: 0 = hx2 + the 8 down partials of the previous layer, 1 = hin,
  // 2 = the embedding row of emb_token[0]
  int in_mode;
  const float* hin;
  const int32_t* emb_token;
  const uint8_t* emb_w;
  const uint16_t* emb_s;
  int emb_vocab;
  XcdBufs x;
};
struct XcdMlpArgs {
  const uint8_t *gw, *uw, *dw;
  const uint16_t *gs, *us, *ds;
  const float* post_gamma;
  float eps;
  XcdBufs x;
};
// 16-position groups per thread of launch A for a KV capacity (0: unsupported, > 4096).
int xcd_npt(int max_ctx);
// Whether the current device suits the XCD-split launches (checked once per device;
// see q4d_decode_plan_active).  xcd_set_check_mode(1) reports every device as
// unsuitable, 0 restores the check (q4d_diag_set_xcd_check); returns the previous mode.
bool xcd_device_ok(hipStream_t st);
int xcd_set_check_mode(int mode);
int launch_xcd_attn(const XcdAttnArgs& a, hipStream_t st);
int launch_xcd_mlp(const XcdMlpArgs& a, hipStream_t st);
// out = hx2 + sum of the 8 down partials.
int launch_xcd_finalize(const XcdBufs& x, float* out, hipStream_t st);

// ---- Q4 GEMM on MFMA (prefill / batched decode) ------------------------------
// Prefill's per-head work on the q|k|v projections (q/k RMSNorm, RoPE, K/V append)
// and its causal attention: the q|k|v GEMM's EP_ROPE epilogue and
// launch_prefill_attention.
struct PrefillArgs {
  const float* q_gamma;
  const float* k_gamma;
  float eps;
  float qscale;            // attention scaling * log2(e), folded into q
  const float* rope_cos;   // [max_ctx][head_dim / 2]
  const float* rope_sin;
  uint16_t* kcache;        // K plane of the layer and sequence: [kvh][max_ctx][head_dim] fp16
  uint16_t* vcache;
  _Float16* q16;           // [qh][n][head_dim] normed, roped, pre-scaled q
  _Float16* out;           // [n][qh * head_dim] attention output
  int n, p0, qh, kvh, max_ctx;
};
struct GemmArgs {
  const uint8_t* w[3];
  const uint16_t* s[3];
  int seg_end[3];
  int nseg;
  int N;               // output columns (PAIR: rows of each of gate / up)
  int K;
  int M;               // activation rows
  const uint16_t* x;   // fp16 [M, K]
  void* y;             // output [M, ldy]
  int ldy;
  const float* resid;  // EP_RESID: y = resid + X W^T (fp32, [M, ldy])
  float* logits;       // EP_ARGMAX: optional [M, N]
  float* part_score;   // EP_ARGMAX: [M, N/128]
  int* part_idx;
  // Split-K (not for EP_ARGMAX): with `part` set, launch_gemm may split the K
  // steps over ksplit blocks per output tile when the tiles alone would not
  // fill the device; each writes its fp32 tile to part[z][M][N (PAIR: 2N)]
  // and a reduction kernel sums the splits in order and applies the
  // epilogue.  part_cap = floats available at `part`.  ksplit = 0 lets
  // launch_gemm choose (ksplit = 1: no split).
  float* part;
  size_t part_cap;
  int ksplit;
  int defer_reduce;  // with a split, leave the partials for launch_splitk_resid_norm
  // skinny: with M <= 64 the skinny kernel may run (its sums are grouped differently
  // from the tiled kernels', so callers that compare against those opt out: prefill
  // chunks must equal one call bit for bit).  x_tiled: X in the tiled layout (xt_index);
  // y_tiled: the fp16 output of EP_SWIGLU, and xn of launch_splitk_resid_norm, written
  // tiled (both only through the skinny kernel).
  int skinny;
  int x_tiled;
  int y_tiled;
  int* ksplit_used;  // optional: receives the split launch_gemm ran (1: the epilogue was applied)
  // EP_ROPE (prefill q|k|v, no split): the 128 columns of an output tile are one
  // head, q heads then k heads then v heads; q rows go normed, roped and scaled to
  // rope.q16, k rows normed and roped and v rows as they are to the cache planes
  // at positions rope.p0 + m.  y is not written.
  PrefillArgs rope;
};
constexpr int kGemmMaxSplit = 16;
// Compute units of the current device (cached per process; 256 on MI355X).
int device_cus();
int launch_gemm(const GemmArgs& a, int ep, bool pair, hipStream_t st);
// The deferred reduction of an EP_RESID split GEMM fused with the RMSNorm that follows it:
// y = resid + sum_z part[z] (fp32, in order of z), then xn = fp16(y * rsqrt(mean(y^2) + eps)
// * gamma) per row.  N % 4 == 0, N <= 4096.
int launch_splitk_resid_norm(const GemmArgs& a, int ksplit, const float* gamma, float eps, uint16_t* xn,
                             hipStream_t st);
int launch_argmax_rows(const float* part_score, const int* part_idx, int nparts, int M, int32_t* out_token,
                       float* out_score, hipStream_t st);

// ---- integer Q4 GEMV of the fixed-point path (q4d_int.hip) ------------------
int launch_gemv_q26(const q4d_matrix_t* w, const int32_t* x, int64_t* y_q26, int32_t* y_q12, int32_t* saturated,
                    hipStream_t st);
int launch_argmax_q26(const int64_t* scores, int n, int32_t* tok, int64_t* score, hipStream_t st);

// ---- prefill (many tokens of one sequence) ---------------------------------------
int launch_prefill_attention(const PrefillArgs& a, hipStream_t st);

// Prefill workspace: the single-token layout (status, counters, LM-head argmax)
// followed by the per-token buffers.
// K splits of the prefill o_proj / down GEMMs (N = hidden gives too few output tiles to
// keep two blocks on every CU); fixed, so a row's sums do not depend on the token count.
constexpr int kPrefillSplit = 2;

struct PrefillLayout {
  WsLayout base;
  size_t hidden;  // f32 [n][hidden]
  size_t xh;      // f16 [n][max(hidden, intermediate)]
  size_t q16;     // f16 [qh][n][d]
  size_t attn;    // f16 [n][qh * d]
  size_t act;     // f16 [n][intermediate]
  size_t part;    // f32 [2][n][hidden]: split-K partials of the o_proj / down GEMMs
  size_t total;
};

inline PrefillLayout prefill_layout(const q4d_model_t* m, int n) {
  PrefillLayout P{};
  P.base = ws_layout(m, 1);
  const size_t A = 256;
  const int d = m->head_dim, qh = m->num_q_heads;
  const int wx = m->hidden_size > m->intermediate_size ? m->hidden_size : m->intermediate_size;
  size_t o = align_up(P.base.total, A);
  P.hidden = o; o = align_up(o + (size_t)n * m->hidden_size * 4, A);
  P.xh = o;     o = align_up(o + (size_t)n * wx * 2, A);
  P.q16 = o;    o = align_up(o + (size_t)qh * n * d * 2, A);
  P.attn = o;   o = align_up(o + (size_t)n * qh * d * 2, A);
  P.act = o;    o = align_up(o + (size_t)n * m->intermediate_size * 2, A);
  P.part = o;   o = align_up(o + (size_t)kPrefillSplit * n * m->hidden_size * 4, A);
  P.total = o;
  return P;
}

int launch_fill_i32(int32_t* p, int32_t v, size_t n, hipStream_t stream);
int launch_chain(const int32_t* grid_x, const int32_t* grid_y, const int32_t* block, int n, float* buf,
                 hipStream_t stream);
int launch_advance_session(int32_t* tokens, int32_t* positions, const int32_t* next_token, const float* score,
                           int32_t* hist_tokens, float* hist_scores, int32_t* hist_count, int32_t hist_capacity,
                           int32_t* stop, hipStream_t stream);
int launch_advance(int32_t* tokens, int32_t* positions, const int32_t* next_token, const float* score,
                   int32_t* hist_tokens, float* hist_scores, int32_t* hist_count, int32_t hist_capacity,
                   hipStream_t stream);
int launch_apply_rope(const float* x, float* y, const float* cosv, const float* sinv, int batch, int heads,
                      int seq, int head_dim, hipStream_t stream);
int launch_rotate_half(const float* x, float* y, long long rows, int head_dim, hipStream_t stream);
// Causal GQA attention over fp32 q [batch, qh, seq, 128], k / v [batch, kvh, seq, 128]
// -> fp32 out [batch, qh, seq, 128] through prefill_attn_kernel (q4d_prefill.hip);
// ws holds the fp16 operands (causal_attention_ws_bytes).
size_t causal_attention_ws_bytes(int batch, int qh, int kvh, int seq);
int launch_causal_attention(const float* q, const float* k, const float* v, float* out, int batch, int qh,
                            int kvh, int seq, float scaling, void* ws, hipStream_t st);

}  // namespace q4d
