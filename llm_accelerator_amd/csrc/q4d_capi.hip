// extern "C" entry points of libq4dec.so: host-side validation, then
// stream-ordered launches.  See include/q4dec.h for the contract.
#include <string.h>

#include <mutex>

#include "q4d_internal.h"

// Device scratch of q4d_run_one_token_noalloc (see noalloc_scratch below).
constexpr size_t kNoallocScratchBytes = size_t(4) << 20;
constexpr int kNoallocClearWords = 1024;  // status, counters, LM-head hand-off and exchange flags (4 KB)
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace q4d {
int launch_gemv_xp(const GemvArgs& a, int xm, int xp, int ep, bool pair, hipStream_t st);
}

using namespace q4d;

namespace {

// Activation precision inside the fused decode: 2 = fp32 activations enter
// each GEMV as hi+lo fp16 halves (about 22 significant bits), 1 = rounded to fp16.
int g_act_precision = 2;
int g_decode_plan = Q4D_DECODE_XCD;

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

int check_matrix(const q4d_matrix_t* m, int rows, int cols) {
  if (!m || !m->w || !m->s) return Q4D_ERR_NULL;
  if (m->rows != rows || m->cols != cols) return Q4D_ERR_BAD_TABLE;
  if (!aligned(m->w, 16) || !aligned(m->s, 4)) return Q4D_ERR_BAD_ADDR;
  return Q4D_OK;
}

int check_model(const q4d_model_t* m) {
  if (!m || !m->layers || !m->final_norm || !m->rope_cos || !m->rope_sin) return Q4D_ERR_NULL;
  if (m->hidden_size != 1024 || m->head_dim != 128 || m->num_kv_heads <= 0 ||
      m->num_q_heads != 2 * m->num_kv_heads)
    return Q4D_ERR_SHAPE;
  const int qd = m->num_q_heads * m->head_dim, kd = m->num_kv_heads * m->head_dim;
  if (qd != 1024 && qd != 2048 && qd != 3072) return Q4D_ERR_SHAPE;
  const int I = m->intermediate_size;
  if (I != 1024 && I != 2048 && I != 3072) return Q4D_ERR_SHAPE;
  if (m->num_layers <= 0 || m->max_ctx <= 0 || m->vocab_size <= 0 || (m->vocab_size & 1)) return Q4D_ERR_SHAPE;
  if (kd % 2) return Q4D_ERR_SHAPE;
  int rc;
  if ((rc = check_matrix(&m->embed_tokens, m->vocab_size, m->hidden_size))) return rc;
  for (int l = 0; l < m->num_layers; ++l) {
    const q4d_layer_t& L = m->layers[l];
    if ((rc = check_matrix(&L.q_proj, qd, 1024)) || (rc = check_matrix(&L.k_proj, kd, 1024)) ||
        (rc = check_matrix(&L.v_proj, kd, 1024)) || (rc = check_matrix(&L.o_proj, 1024, qd)) ||
        (rc = check_matrix(&L.gate_proj, I, 1024)) || (rc = check_matrix(&L.up_proj, I, 1024)) ||
        (rc = check_matrix(&L.down_proj, 1024, I)))
      return rc == Q4D_ERR_BAD_TABLE ? Q4D_ERR_BAD_LAYER : rc;
    if (!L.input_layernorm || !L.post_attention_layernorm || !L.q_norm || !L.k_norm) return Q4D_ERR_NULL;
    if (!aligned(L.input_layernorm, 16) || !aligned(L.post_attention_layernorm, 16)) return Q4D_ERR_BAD_ADDR;
  }
  if (!aligned(m->final_norm, 16)) return Q4D_ERR_BAD_ADDR;
  return Q4D_OK;
}

int check_kv(const q4d_kv_cache_t* kv, const q4d_model_t* m, int batch) {
  if (!kv || !kv->data) return Q4D_ERR_NULL;
  if (kv->num_layers != m->num_layers || kv->num_kv_heads != m->num_kv_heads || kv->head_dim != m->head_dim ||
      kv->max_ctx != m->max_ctx)
    return Q4D_ERR_SHAPE;
  if (kv->batch < batch || batch <= 0) return Q4D_ERR_CAPACITY;
  if (!aligned(kv->data, 16)) return Q4D_ERR_BAD_ADDR;
  return Q4D_OK;
}

int check_ws(const void* ws, size_t bytes, const q4d_model_t* m, int batch) {
  if (!ws) return Q4D_ERR_NULL;
  if (!aligned(ws, 256)) return Q4D_ERR_BAD_ADDR;
  if (bytes < ws_layout(m, batch).total) return Q4D_ERR_CAPACITY;
  return Q4D_OK;
}

void kv_planes(const q4d_kv_cache_t* kv, int layer, uint16_t** kp, uint16_t** vp) {
  const size_t plane = (size_t)kv->batch * kv->num_kv_heads * kv->max_ctx * kv->head_dim;
  *kp = kv->data + (size_t)layer * 2 * plane;
  *vp = *kp + plane;
}

GemvArgs one_matrix(const q4d_matrix_t* w, int batch) {
  GemvArgs a;
  memset(&a, 0, sizeof(a));
  a.w[0] = w->w;
  a.s[0] = w->s;
  a.seg_end[0] = w->rows;
  a.nseg = 1;
  a.rows = w->rows;
  a.cols = w->cols;
  a.batch = batch;
  return a;
}

// Greedy feedback of a one-token step, stored by the LM head's last block (the
// work of q4d_advance without its launch).
struct Feedback {
  int32_t* tokens;
  int32_t* positions;
  int32_t* hist_tokens;
  float* hist_scores;
  int32_t* hist_count;
  int32_t hist_capacity;
};

bool xcd_eligible(const q4d_model_t* m, hipStream_t st);
int run_layer_xcd(const q4d_model_t* m, int l, int in_mode, const float* hin, const int32_t* emb_tokens,
                  float* hout, const q4d_kv_cache_t* kv, const int32_t* positions, void* ws, const WsLayout& W,
                  int32_t* status, hipStream_t st);

// One decoder layer, batch 1 (common.py:231-298), five launches; `only`
// selects a single stage (Q4D_STAGE_*) or -1 for all.  With `emb_tokens` the
// layer's input is the embedding row of emb_tokens[0], built in the q|k|v
// launch's prologue, which also stores it to hout (the residual stream; hin
// must then be hout).
int run_layer(const q4d_model_t* m, int l, const float* hin, float* hout, const q4d_kv_cache_t* kv,
              const int32_t* positions, void* ws, const WsLayout& W, hipStream_t st, int only = -1,
              int32_t* status = nullptr, const int32_t* emb_tokens = nullptr) {
  if (only < 0 && xcd_eligible(m, st)) {
    int32_t* stw = status ? status : ws_ptr<int32_t>(ws, W.status);
    return emb_tokens ? run_layer_xcd(m, l, 2, nullptr, emb_tokens, hout, kv, positions, ws, W, stw, st)
                      : run_layer_xcd(m, l, 1, hin, nullptr, hout, kv, positions, ws, W, stw, st);
  }
  const q4d_layer_t& L = m->layers[l];
  const int xp = g_act_precision;
  float* qkv = ws_ptr<float>(ws, W.qkv);
  float* attn = ws_ptr<float>(ws, W.attn);
  float* act = ws_ptr<float>(ws, W.act);
  int rc;

  // 1. input RMSNorm fused into the q|k|v projection
  GemvArgs a;
  memset(&a, 0, sizeof(a));
  a.w[0] = L.q_proj.w; a.s[0] = L.q_proj.s;
  a.w[1] = L.k_proj.w; a.s[1] = L.k_proj.s;
  a.w[2] = L.v_proj.w; a.s[2] = L.v_proj.s;
  a.seg_end[0] = L.q_proj.rows;
  a.seg_end[1] = a.seg_end[0] + L.k_proj.rows;
  a.seg_end[2] = a.seg_end[1] + L.v_proj.rows;
  a.nseg = 3;
  a.rows = a.seg_end[2];
  a.cols = 1024;
  a.x = hin;
  a.gamma = L.input_layernorm;
  a.eps = m->rms_norm_eps;
  a.y = qkv;
  a.batch = 1;
  int xm = X_RMS;
  if (emb_tokens) {
    if (hin != hout) return Q4D_ERR_SHAPE;
    a.x = nullptr;
    a.emb_token = emb_tokens;
    a.emb_w = m->embed_tokens.w;
    a.emb_s = m->embed_tokens.s;
    a.emb_vocab = m->embed_tokens.rows;
    a.emb_out = hout;
    a.emb_status = status ? status : ws_ptr<int32_t>(ws, W.status);
    xm = X_EMB;
  }
  if ((only < 0 || only == Q4D_STAGE_QKV) && (rc = launch_gemv_xp(a, xm, xp, EP_F32, false, st))) return rc;

  // 2. q/k norm + RoPE + KV append + attention + split merge
  AttnArgs t;
  memset(&t, 0, sizeof(t));
  t.fused = 1;
  t.qkv = qkv;
  t.q_gamma = L.q_norm;
  t.k_gamma = L.k_norm;
  t.eps = m->rms_norm_eps;
  t.scaling = m->attn_scaling;
  t.rope_cos = m->rope_cos;
  t.rope_sin = m->rope_sin;
  kv_planes(kv, l, &t.kcache, &t.vcache);
  t.positions = positions;
  t.batch = 1;
  t.qh = m->num_q_heads;
  t.kvh = m->num_kv_heads;
  t.d = m->head_dim;
  t.max_ctx = m->max_ctx;
  t.nsplit_max = W.nsplit_max;
  t.part_ml = ws_ptr<float>(ws, W.part_ml);
  t.part_acc = ws_ptr<float>(ws, W.part_acc);
  t.counters = ws_ptr<int>(ws, W.counters);
  t.out = attn;
  t.out_dtype = Q4D_F32;
  t.status = status ? status : ws_ptr<int32_t>(ws, W.status);
  t.merge = 0;  // partials only: merged by the o_proj prologue
  // 64-position chunks give twice the attention blocks; the o_proj prologue merges
  // up to 8 chunks in one batch of loads, so they are used while 8 cover max_ctx
  t.chunk = (m->max_ctx + kAttnChunk - 1) / kAttnChunk <= 8 ? kAttnChunk : kAttnChunkLong;
  if ((only < 0 || only == Q4D_STAGE_ATTENTION) && (rc = launch_attention(t, st))) return rc;

  // 3. merge the attention partials, o_proj + residual
  a = one_matrix(&L.o_proj, 1);
  a.part_ml = t.part_ml;
  a.part_acc = t.part_acc;
  a.positions = positions;
  a.nsplit_max = W.nsplit_max;
  a.attn_chunk = t.chunk;
  a.y = hout;
  a.resid = hin;
  if ((only < 0 || only == Q4D_STAGE_O_PROJ) && (rc = launch_gemv_xp(a, X_ATTN, xp, EP_RESID, false, st)))
    return rc;

  // 4. post-attention RMSNorm + gate/up + SwiGLU
  memset(&a, 0, sizeof(a));
  a.w[0] = L.gate_proj.w; a.s[0] = L.gate_proj.s;
  a.w[1] = L.up_proj.w;   a.s[1] = L.up_proj.s;
  a.seg_end[0] = L.gate_proj.rows;
  a.seg_end[1] = 2 * L.gate_proj.rows;
  a.nseg = 2;
  a.rows = L.gate_proj.rows;
  a.cols = 1024;
  a.x = hout;
  a.gamma = L.post_attention_layernorm;
  a.eps = m->rms_norm_eps;
  a.y = act;
  a.batch = 1;
  if ((only < 0 || only == Q4D_STAGE_GATE_UP) && (rc = launch_gemv_xp(a, X_RMS, xp, EP_SWIGLU, true, st)))
    return rc;

  // 5. down_proj + residual (in place on hout)
  a = one_matrix(&L.down_proj, 1);
  a.x = act;
  a.y = hout;
  a.resid = hout;
  if (only < 0 || only == Q4D_STAGE_DOWN) return launch_gemv_xp(a, X_F32, xp, EP_RESID, false, st);
  return Q4D_OK;
}

// The XCD-split layer (q4d_xcd.hip) covers the Qwen3-0.6B shape at activation precision 2,
// on a device that passes its placement check (xcd_device_ok); anything else runs staged.
bool xcd_eligible(const q4d_model_t* m, hipStream_t st) {
  return g_decode_plan == Q4D_DECODE_XCD && g_act_precision == 2 && m->hidden_size == 1024 &&
         m->intermediate_size == kXcdInter && m->num_q_heads == 2 * kXcdGroups && m->num_kv_heads == kXcdGroups &&
         m->head_dim == 128 && xcd_npt(m->max_ctx) > 0 && xcd_device_ok(st);
}

XcdBufs xcd_bufs(void* ws, const WsLayout& W, int32_t* status) {
  XcdBufs x;
  x.flags = ws_ptr<uint32_t>(ws, W.xflags);
  x.qkv = ws_ptr<float>(ws, W.xqkv);
  x.ap = ws_ptr<float>(ws, W.xap);
  x.ac = ws_ptr<float>(ws, W.xac);
  x.po = ws_ptr<float>(ws, W.xpo);
  x.pd = ws_ptr<float>(ws, W.xpd);
  x.hx = ws_ptr<float>(ws, W.xhx);
  x.hx2 = ws_ptr<float>(ws, W.xhx2);
  x.status = status;
  return x;
}

// One decoder layer, batch 1, as the two XCD-split launches.  Input: in_mode 1 = hin,
// 2 = the embedding row of emb_tokens[0], 0 = the previous layer of the same step
// (its post-attention state and down partials in the workspace).  With hout set, the
// layer output is also formed there (otherwise the next layer's launch A forms it).
int run_layer_xcd(const q4d_model_t* m, int l, int in_mode, const float* hin, const int32_t* emb_tokens,
                  float* hout, const q4d_kv_cache_t* kv, const int32_t* positions, void* ws, const WsLayout& W,
                  int32_t* status, hipStream_t st) {
  const q4d_layer_t& L = m->layers[l];
  const XcdBufs xb = xcd_bufs(ws, W, status);
  XcdAttnArgs a;
  memset(&a, 0, sizeof(a));
  a.qw = L.q_proj.w; a.qs = L.q_proj.s;
  a.kw = L.k_proj.w; a.ks = L.k_proj.s;
  a.vw = L.v_proj.w; a.vs = L.v_proj.s;
  a.ow = L.o_proj.w; a.os = L.o_proj.s;
  a.in_gamma = L.input_layernorm;
  a.q_gamma = L.q_norm;
  a.k_gamma = L.k_norm;
  a.eps = m->rms_norm_eps;
  a.qscale = m->attn_scaling * 1.4426950408889634f;
  a.rope_cos = m->rope_cos;
  a.rope_sin = m->rope_sin;
  kv_planes(kv, l, &a.kcache, &a.vcache);
  a.positions = positions;
  a.max_ctx = m->max_ctx;
  a.in_mode = in_mode;
  a.hin = hin;
  a.emb_token = emb_tokens;
  a.emb_w = m->embed_tokens.w;
  a.emb_s = m->embed_tokens.s;
  a.emb_vocab = m->embed_tokens.rows;
  a.x = xb;
  int rc = launch_xcd_attn(a, st);
  if (rc) return rc;
  XcdMlpArgs b;
  memset(&b, 0, sizeof(b));
  b.gw = L.gate_proj.w; b.gs = L.gate_proj.s;
  b.uw = L.up_proj.w;   b.us = L.up_proj.s;
  b.dw = L.down_proj.w; b.ds = L.down_proj.s;
  b.post_gamma = L.post_attention_layernorm;
  b.eps = m->rms_norm_eps;
  b.x = xb;
  if ((rc = launch_xcd_mlp(b, st))) return rc;
  return hout ? launch_xcd_finalize(xb, hout, st) : Q4D_OK;
}

// With parts set, the LM head's input is hidden + parts[0] + ... + parts[7] (the
// XCD-split layer's output), which it also stores to hidden_out when that is set.
int run_lm_head(const q4d_model_t* m, const float* hidden, int32_t* tok, float* score, float* logits,
                void* ws, const WsLayout& W, hipStream_t st, const Feedback* fb = nullptr,
                const float* parts = nullptr, float* hidden_out = nullptr) {
  GemvArgs a = one_matrix(&m->embed_tokens, 1);
  a.x = hidden;
  a.x_parts = parts;
  a.x_out = hidden_out;
  a.gamma = m->final_norm;
  a.eps = m->rms_norm_eps;
  a.logits = logits;
  a.lm_hand = ws_ptr<char>(ws, W.lm_hand);
  a.out_token = tok;
  a.out_score = score;
  if (fb) {
    a.adv_tokens = fb->tokens;
    a.adv_positions = fb->positions;
    a.hist_tokens = fb->hist_tokens;
    a.hist_scores = fb->hist_scores;
    a.hist_count = fb->hist_count;
    a.hist_cap = fb->hist_capacity;
  }
  return launch_gemv_xp(a, X_RMS, g_act_precision, EP_ARGMAX, false, st);
}

// Embedding -> all layers -> LM head argmax for one token (batch 1), the launches of
// q4d_run_one_token: the embedding is built inside layer 0's q|k|v launch, and
// with `fb` the LM head also stores the greedy feedback.  `status` receives the
// device-side status bits.
int run_token(const q4d_model_t* m, const int32_t* tokens, const int32_t* positions, const q4d_kv_cache_t* kv,
              int32_t* next_token, float* score, float* logits, void* ws, const WsLayout& W, int32_t* status,
              hipStream_t st, const Feedback* fb = nullptr) {
  float* hidden = ws_ptr<float>(ws, W.hidden);
  int rc;
  if (xcd_eligible(m, st)) {
    // layer l > 0 takes its input from the previous layer's launches directly; the LM
    // head's prologue forms the last layer's output (stored in `hidden` as well)
    for (int l = 0; l < m->num_layers; ++l)
      if ((rc = run_layer_xcd(m, l, l == 0 ? 2 : 0, nullptr, tokens, nullptr, kv, positions, ws, W, status, st)))
        return rc;
    const XcdBufs xb = xcd_bufs(ws, W, status);
    return run_lm_head(m, xb.hx2, next_token, score, logits, ws, W, st, fb, xb.pd, hidden);
  }
  for (int l = 0; l < m->num_layers; ++l)
    if ((rc = run_layer(m, l, hidden, hidden, kv, positions, ws, W, st, -1, status, l == 0 ? tokens : nullptr)))
      return rc;
  return run_lm_head(m, hidden, next_token, score, logits, ws, W, st, fb);
}

// Scratch of q4d_run_one_token_noalloc, for callers that cannot allocate: a
// workspace of this library's layout in a device array (one copy per GPU, zero
// from module load).  Host code never uses the array's name as an address: each
// device's address comes from hipGetSymbolAddress, once per device, below.
// Every call on one GPU shares that GPU's copy; calls that overlap on one GPU race.
int noalloc_scratch(hipStream_t st, void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return Q4D_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return Q4D_ERR_LAUNCH;
    // the counters, the LM-head hand-off region and the exchange flags start at zero (the
    // kernels leave them as the next launch expects); cleared once here with a fill kernel
    // in case the module's zero fill is not relied on
    const int rc = launch_fill_i32(static_cast<int32_t*>(p), 0, kNoallocClearWords, st);
    if (rc) return rc;
    ptrs[dev] = p;
  }
  *out = ptrs[dev];
  return Q4D_OK;
}

}  // namespace

extern "C" {

int q4d_version(void) { return 1; }

const char* q4d_status_string(int code) {
  switch (code) {
    case Q4D_OK: return "ok";
    case Q4D_ERR_BUSY: return "busy";
    case Q4D_ERR_BAD_LAYER: return "bad layer descriptor";
    case Q4D_ERR_BAD_TABLE: return "bad weight descriptor";
    case Q4D_ERR_BAD_ADDR: return "misaligned pointer";
    case Q4D_ERR_TIMEOUT: return "timeout";
    case Q4D_ERR_STATUS: return "device status error";
    case Q4D_ERR_NULL: return "null pointer";
    case Q4D_ERR_BAD_TOKEN: return "token id outside the vocabulary";
    case Q4D_ERR_CAPACITY: return "workspace or cache capacity exceeded";
    case Q4D_ERR_CONTEXT: return "position outside the context";
    case Q4D_ERR_SHAPE: return "unsupported shape";
    case Q4D_ERR_LAUNCH: return "kernel launch failed";
    case Q4D_ERR_DTYPE: return "unsupported dtype";
    default: return "unknown status";
  }
}

int q4d_set_decode_plan(int32_t plan) {
  if (plan != Q4D_DECODE_XCD && plan != Q4D_DECODE_STAGED) return Q4D_ERR_SHAPE;
  const int prev = g_decode_plan;
  g_decode_plan = plan;
  return prev;
}

int q4d_set_activation_precision(int32_t mode) {
  if (mode != 1 && mode != 2) return Q4D_ERR_DTYPE;
  g_act_precision = mode;
  return Q4D_OK;
}

size_t q4d_workspace_bytes(const q4d_model_t* model, int32_t batch) {
  if (!model || batch <= 0) return 0;
  return ws_layout(model, batch).total;
}

int q4d_workspace_init(void* ws, size_t ws_bytes, const q4d_model_t* model, int32_t batch, void* stream) {
  if (!model) return Q4D_ERR_NULL;
  int rc = check_ws(ws, ws_bytes, model, batch);
  if (rc) return rc;
  const WsLayout W = ws_layout(model, batch);
  // the XCD-split plan's one-time device check runs here, before any decode call
  // (and before a caller captures decode steps into a graph)
  if (batch == 1) xcd_device_ok(as_stream(stream));
  // status block and counters are contiguous at the start of the workspace
  return launch_fill_i32(ws_ptr<int32_t>(ws, 0), 0, W.hidden / 4, as_stream(stream));
}

int q4d_decode_plan_active(const q4d_model_t* model, void* stream) {
  if (!model) return Q4D_ERR_NULL;
  return xcd_eligible(model, as_stream(stream)) ? Q4D_DECODE_XCD : Q4D_DECODE_STAGED;
}

int q4d_diag_set_xcd_check(int32_t mode) {
  if (mode != 0 && mode != 1) return Q4D_ERR_SHAPE;
  return xcd_set_check_mode(mode);
}

int q4d_read_status(const void* ws, size_t ws_bytes, const q4d_model_t* model, int32_t batch, int32_t* out,
                    void* stream) {
  if (!model || !out) return Q4D_ERR_NULL;
  int rc = check_ws(ws, ws_bytes, model, batch);
  if (rc) return rc;
  const WsLayout W = ws_layout(model, batch);
  if (hipMemcpyAsync(out, static_cast<const char*>(ws) + W.status, 4, hipMemcpyDeviceToHost,
                     as_stream(stream)) != hipSuccess)
    return Q4D_ERR_LAUNCH;
  return hipStreamSynchronize(as_stream(stream)) == hipSuccess ? Q4D_OK : Q4D_ERR_LAUNCH;
}

int q4d_linear(const q4d_matrix_t* w, const void* x, int32_t x_dtype, void* y, int32_t y_dtype, int32_t batch,
               void* stream) {
  if (!w) return Q4D_ERR_NULL;
  int rc = check_matrix(w, w->rows, w->cols);
  if (rc) return rc;
  if (x_dtype != Q4D_F16 && x_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  if (y_dtype != Q4D_F16 && y_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  if (batch <= 0) return Q4D_ERR_SHAPE;
  GemvArgs a = one_matrix(w, batch);
  a.x = x;
  a.y = y;
  return launch_gemv_xp(a, x_dtype == Q4D_F16 ? X_F16 : X_F32, x_dtype == Q4D_F16 ? 1 : g_act_precision,
                        y_dtype == Q4D_F16 ? EP_F16 : EP_F32, false, as_stream(stream));
}

int q4d_linear_group(const q4d_matrix_t* w, const void* const* x, int32_t x_dtype, void* const* y, int32_t y_dtype,
                     int32_t batch, int32_t count, void* stream) {
  if (!w || !x || !y) return Q4D_ERR_NULL;
  if (count <= 0 || batch <= 0) return Q4D_ERR_SHAPE;
  if (x_dtype != Q4D_F16 && x_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  if (y_dtype != Q4D_F16 && y_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  // every descriptor and pointer is checked before the first launch, so a call that
  // returns an error has written no output
  for (int i = 0; i < count; ++i) {
    const int rc = check_matrix(&w[i], w[0].rows, w[0].cols);
    if (rc) return rc;
    if (!x[i] || !y[i]) return Q4D_ERR_NULL;
    if (!aligned(x[i], 16)) return Q4D_ERR_BAD_ADDR;
  }
  constexpr int kChunk = 64;  // descriptors unpacked per step
  const uint8_t* wp[kChunk];
  const uint16_t* sp[kChunk];
  for (int i0 = 0; i0 < count; i0 += kChunk) {
    const int n = count - i0 < kChunk ? count - i0 : kChunk;
    for (int k = 0; k < n; ++k) {
      wp[k] = w[i0 + k].w;
      sp[k] = w[i0 + k].s;
    }
    const int rc = launch_gemv_group(w[0].rows, w[0].cols, batch, wp, sp, x + i0, y + i0, n,
                                     x_dtype == Q4D_F16 ? X_F16 : X_F32, x_dtype == Q4D_F16 ? 1 : g_act_precision,
                                     y_dtype == Q4D_F16 ? EP_F16 : EP_F32, as_stream(stream));
    if (rc) return rc;
  }
  return Q4D_OK;
}

int q4d_rms_norm(const float* x, const float* gamma, float eps, int32_t rows, int32_t dim, void* y,
                 int32_t y_dtype, void* stream) {
  if (!x || !gamma || !y) return Q4D_ERR_NULL;
  if (rows <= 0 || dim <= 0) return Q4D_ERR_SHAPE;
  if (y_dtype != Q4D_F16 && y_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  return launch_rms_norm(x, gamma, eps, rows, dim, y, y_dtype, as_stream(stream));
}

int q4d_qk_norm_rope(const float* x, float* y, const float* gamma, float eps, int32_t batch, int32_t heads,
                     int32_t head_dim, const float* rope_cos, const float* rope_sin, int32_t max_ctx,
                     const int32_t* positions, int32_t* status, void* stream) {
  if (!x || !y || !gamma || !rope_cos || !rope_sin || !positions || !status) return Q4D_ERR_NULL;
  if (batch <= 0 || heads <= 0 || max_ctx <= 0) return Q4D_ERR_SHAPE;
  return launch_qk_norm_rope(x, y, gamma, eps, batch, heads, head_dim, rope_cos, rope_sin, max_ctx, positions,
                             status, as_stream(stream));
}

int q4d_kv_append(const q4d_kv_cache_t* kv, int32_t layer, const float* k, const float* v,
                  const int32_t* positions, int32_t* status, void* stream) {
  if (!kv || !kv->data || (!k && !v) || !positions || !status) return Q4D_ERR_NULL;
  if (layer < 0 || layer >= kv->num_layers) return Q4D_ERR_BAD_LAYER;
  if (kv->batch <= 0 || kv->num_kv_heads <= 0 || kv->max_ctx <= 0 || kv->head_dim <= 0) return Q4D_ERR_SHAPE;
  return launch_kv_append(kv, layer, k, v, positions, status, as_stream(stream));
}

int q4d_cached_attention(const q4d_model_t* model, const q4d_kv_cache_t* kv, int32_t layer, const float* q,
                         const int32_t* positions, void* out, int32_t out_dtype, void* ws, size_t ws_bytes,
                         void* stream) {
  if (!model || !q || !positions || !out) return Q4D_ERR_NULL;
  if (model->head_dim != 128 || model->num_q_heads != 2 * model->num_kv_heads) return Q4D_ERR_SHAPE;
  if (out_dtype != Q4D_F16 && out_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  int rc;
  if (!kv) return Q4D_ERR_NULL;
  if (layer < 0 || layer >= kv->num_layers) return Q4D_ERR_BAD_LAYER;
  if ((rc = check_kv(kv, model, kv->batch))) return rc;
  if ((rc = check_ws(ws, ws_bytes, model, kv->batch))) return rc;
  const WsLayout W = ws_layout(model, kv->batch);
  AttnArgs t;
  memset(&t, 0, sizeof(t));
  t.fused = 0;
  t.q = q;
  t.scaling = model->attn_scaling;
  kv_planes(kv, layer, &t.kcache, &t.vcache);
  t.positions = positions;
  t.batch = kv->batch;
  t.qh = model->num_q_heads;
  t.kvh = model->num_kv_heads;
  t.d = model->head_dim;
  t.max_ctx = model->max_ctx;
  t.nsplit_max = W.nsplit_max;
  t.part_ml = ws_ptr<float>(ws, W.part_ml);
  t.part_acc = ws_ptr<float>(ws, W.part_acc);
  t.counters = ws_ptr<int>(ws, W.counters);
  t.out = out;
  t.out_dtype = out_dtype;
  t.status = ws_ptr<int32_t>(ws, W.status);
  t.merge = 1;
  return launch_attention(t, as_stream(stream));
}

int q4d_embedding(const q4d_matrix_t* table, const int32_t* tokens, int32_t batch, float* hidden,
                  int32_t* status, void* stream) {
  if (!table || !tokens || !hidden) return Q4D_ERR_NULL;
  int rc = check_matrix(table, table->rows, table->cols);
  if (rc) return rc;
  if (batch <= 0 || table->cols % 64) return Q4D_ERR_SHAPE;
  return launch_embedding(table, tokens, batch, hidden, status, as_stream(stream));
}

int q4d_lm_head_argmax(const q4d_model_t* model, const float* hidden, int32_t* out_token, float* out_score,
                       float* logits, void* ws, size_t ws_bytes, void* stream) {
  if (!model || !hidden || !out_token || !out_score || !model->final_norm) return Q4D_ERR_NULL;
  int rc = check_matrix(&model->embed_tokens, model->vocab_size, model->hidden_size);
  if (rc) return rc;
  if (model->hidden_size != 1024 || (model->vocab_size & 1)) return Q4D_ERR_SHAPE;
  if ((rc = check_ws(ws, ws_bytes, model, 1))) return rc;
  return run_lm_head(model, hidden, out_token, out_score, logits, ws, ws_layout(model, 1), as_stream(stream));
}

int q4d_decoder_layer(const q4d_model_t* model, int32_t layer, const float* hidden_in, float* hidden_out,
                      const q4d_kv_cache_t* kv, const int32_t* positions, void* ws, size_t ws_bytes,
                      void* stream) {
  if (!hidden_in || !hidden_out || !positions) return Q4D_ERR_NULL;
  int rc = check_model(model);
  if (rc) return rc;
  if (layer < 0 || layer >= model->num_layers) return Q4D_ERR_BAD_LAYER;
  if ((rc = check_kv(kv, model, 1))) return rc;
  if (kv->batch != 1) return Q4D_ERR_CAPACITY;
  if ((rc = check_ws(ws, ws_bytes, model, 1))) return rc;
  return run_layer(model, layer, hidden_in, hidden_out, kv, positions, ws, ws_layout(model, 1), as_stream(stream));
}

int q4d_gemm(const q4d_matrix_t* w, const uint16_t* x, int32_t M, void* y, int32_t y_dtype, const float* resid,
             void* stream) {
  if (!w) return Q4D_ERR_NULL;
  int rc = check_matrix(w, w->rows, w->cols);
  if (rc) return rc;
  if (y_dtype != Q4D_F16 && y_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  if (resid && y_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.w[0] = w->w;
  a.s[0] = w->s;
  a.seg_end[0] = w->rows;
  a.nseg = 1;
  a.N = w->rows;
  a.K = w->cols;
  a.M = M;
  a.x = x;
  a.y = y;
  a.ldy = w->rows;
  a.resid = resid;
  return launch_gemm(a, resid ? EP_RESID : (y_dtype == Q4D_F16 ? EP_F16 : EP_F32), false, as_stream(stream));
}

int q4d_linear_q26(const q4d_matrix_t* w, const int32_t* x_int, int64_t* y_q26, int32_t* y_q12_12,
                   int32_t* saturated, void* stream) {
  if (!w || !x_int || (!y_q26 && !y_q12_12)) return Q4D_ERR_NULL;
  if (!w->w || !w->s) return Q4D_ERR_NULL;
  if (w->rows <= 0 || w->cols <= 0 || w->cols % 64 || w->cols > 3072) return Q4D_ERR_SHAPE;
  if (!aligned(w->w, 16) || !aligned(w->s, 2) || !aligned(x_int, 16)) return Q4D_ERR_BAD_ADDR;
  if ((y_q26 && !aligned(y_q26, 8)) || (y_q12_12 && !aligned(y_q12_12, 4))) return Q4D_ERR_BAD_ADDR;
  return launch_gemv_q26(w, x_int, y_q26, y_q12_12, saturated, as_stream(stream));
}

int q4d_argmax_q26(const int64_t* scores, int32_t n, int32_t* out_token, int64_t* out_score, void* stream) {
  if (!scores || !out_token || !out_score) return Q4D_ERR_NULL;
  if (n <= 0) return Q4D_ERR_SHAPE;
  if (!aligned(scores, 8) || !aligned(out_score, 8)) return Q4D_ERR_BAD_ADDR;
  return launch_argmax_q26(scores, n, out_token, out_score, as_stream(stream));
}

int q4d_gemm_splitk(const q4d_matrix_t* w, const uint16_t* x, int32_t M, void* y, int32_t y_dtype,
                    const float* resid, float* part, size_t part_bytes, int32_t ksplit, void* stream) {
  if (!w || !part) return Q4D_ERR_NULL;
  int rc = check_matrix(w, w->rows, w->cols);
  if (rc) return rc;
  if (y_dtype != Q4D_F16 && y_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  if (resid && y_dtype != Q4D_F32) return Q4D_ERR_DTYPE;
  if (ksplit < 0 || ksplit > kGemmMaxSplit || (ksplit > 0 && ksplit > w->cols / 64)) return Q4D_ERR_SHAPE;
  if (!aligned(part, 16)) return Q4D_ERR_BAD_ADDR;
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.w[0] = w->w;
  a.s[0] = w->s;
  a.seg_end[0] = w->rows;
  a.nseg = 1;
  a.N = w->rows;
  a.K = w->cols;
  a.M = M;
  a.x = x;
  a.y = y;
  a.ldy = w->rows;
  a.resid = resid;
  a.part = part;
  a.part_cap = part_bytes / 4;
  a.ksplit = ksplit;
  a.skinny = ksplit == 0;  // the library chooses: the skinny kernel for M <= 64
  return launch_gemm(a, resid ? EP_RESID : (y_dtype == Q4D_F16 ? EP_F16 : EP_F32), false, as_stream(stream));
}

// Final RMSNorm (to fp16) + LM head GEMM with per-row argmax partials over
// 128-column blocks + one wave per row reducing them.
static int run_lm_head_batch(const q4d_model_t* model, const float* hidden, int batch, int32_t* next_tokens,
                             float* scores, float* logits, void* ws, const WsLayout& W, hipStream_t st) {
  const int H = model->hidden_size;
  uint16_t* xh = ws_ptr<uint16_t>(ws, W.xh);
  int rc = launch_rms_norm(hidden, model->final_norm, model->rms_norm_eps, batch, H, xh, Q4D_F16, st);
  if (rc) return rc;
  GemmArgs g;
  memset(&g, 0, sizeof(g));
  g.w[0] = model->embed_tokens.w;
  g.s[0] = model->embed_tokens.s;
  g.seg_end[0] = model->vocab_size;
  g.nseg = 1;
  g.N = model->vocab_size;
  g.K = H;
  g.M = batch;
  g.x = xh;
  g.logits = logits;
  g.part_score = ws_ptr<float>(ws, W.row_score);
  g.part_idx = ws_ptr<int>(ws, W.row_idx);
  if ((rc = launch_gemm(g, EP_ARGMAX, false, st))) return rc;
  return launch_argmax_rows(g.part_score, g.part_idx, model->vocab_size / 128, batch, next_tokens, scores, st);
}

int q4d_decode_batch(const q4d_model_t* model, const int32_t* tokens, const int32_t* positions, int32_t batch,
                     const q4d_kv_cache_t* kv, int32_t* next_tokens, float* scores, float* logits, void* ws,
                     size_t ws_bytes, void* stream) {
  if (!tokens || !positions || !next_tokens || !scores) return Q4D_ERR_NULL;
  int rc = check_model(model);
  if (rc) return rc;
  if (batch <= 0) return Q4D_ERR_SHAPE;
  if ((rc = check_kv(kv, model, batch))) return rc;
  if ((rc = check_ws(ws, ws_bytes, model, batch))) return rc;
  if (model->vocab_size % 128) return Q4D_ERR_SHAPE;
  const WsLayout W = ws_layout(model, batch);
  hipStream_t st = as_stream(stream);
  const int H = model->hidden_size, qd = model->num_q_heads * model->head_dim;
  const int I = model->intermediate_size;
  float* hidden = ws_ptr<float>(ws, W.hidden);
  uint16_t* xh = ws_ptr<uint16_t>(ws, W.xh);
  float* qkv = ws_ptr<float>(ws, W.qkv);
  uint16_t* attn = ws_ptr<uint16_t>(ws, W.attn);
  uint16_t* act = ws_ptr<uint16_t>(ws, W.act);
  int32_t* status = ws_ptr<int32_t>(ws, W.status);
  float* part = ws_ptr<float>(ws, W.gemm_part);  // split-K tiles of the M = batch GEMMs
  // the GEMMs' fp16 inputs (xh, attn, act) in the tiled layout for 2..64 sequences
  const int xt = xt_batch(batch) ? 1 : 0;
  const int xdt = xt ? kF16Tiled : Q4D_F16;
  if ((rc = launch_embedding(&model->embed_tokens, tokens, batch, hidden, status, st))) return rc;
  // the first layer's input RMSNorm; later ones come out of the previous layer's down
  // projection, whose split-K reduction and residual run fused with it
  if ((rc = launch_rms_norm(hidden, model->layers[0].input_layernorm, model->rms_norm_eps, batch, H, xh, xdt, st)))
    return rc;
  // o_proj / down + residual, then the RMSNorm that follows (gamma): the split-K sums,
  // the residual and the norm as one kernel when the GEMM was split
  auto resid_then_norm = [&](GemmArgs& g, const float* gamma) -> int {
    int ks = 1;
    g.defer_reduce = 1;
    g.ksplit_used = &ks;
    g.skinny = 1;
    g.x_tiled = xt;
    int r = launch_gemm(g, EP_RESID, false, st);
    if (r) return r;
    g.y_tiled = xt;
    if (ks > 1) return launch_splitk_resid_norm(g, ks, gamma, model->rms_norm_eps, xh, st);
    return launch_rms_norm(hidden, gamma, model->rms_norm_eps, batch, H, xh, xdt, st);
  };
  for (int l = 0; l < model->num_layers; ++l) {
    const q4d_layer_t& L = model->layers[l];
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.w[0] = L.q_proj.w; g.s[0] = L.q_proj.s;
    g.w[1] = L.k_proj.w; g.s[1] = L.k_proj.s;
    g.w[2] = L.v_proj.w; g.s[2] = L.v_proj.s;
    g.seg_end[0] = L.q_proj.rows;
    g.seg_end[1] = g.seg_end[0] + L.k_proj.rows;
    g.seg_end[2] = g.seg_end[1] + L.v_proj.rows;
    g.nseg = 3;
    g.N = g.seg_end[2];
    g.K = H;
    g.M = batch;
    g.x = xh;
    g.skinny = 1;
    g.x_tiled = xt;
    g.y = qkv;
    g.ldy = g.N;
    g.part = part; g.part_cap = W.gemm_part_floats;
    if ((rc = launch_gemm(g, EP_F32, false, st))) return rc;

    AttnArgs t;
    memset(&t, 0, sizeof(t));
    t.fused = 1;
    t.qkv = qkv;
    t.q_gamma = L.q_norm;
    t.k_gamma = L.k_norm;
    t.eps = model->rms_norm_eps;
    t.scaling = model->attn_scaling;
    t.rope_cos = model->rope_cos;
    t.rope_sin = model->rope_sin;
    kv_planes(kv, l, &t.kcache, &t.vcache);
    t.positions = positions;
    t.batch = batch;
    t.qh = model->num_q_heads;
    t.kvh = model->num_kv_heads;
    t.d = model->head_dim;
    t.max_ctx = model->max_ctx;
    t.nsplit_max = W.nsplit_max;
    t.part_ml = ws_ptr<float>(ws, W.part_ml);
    t.part_acc = ws_ptr<float>(ws, W.part_acc);
    t.counters = ws_ptr<int>(ws, W.counters);
    t.out = attn;
    t.out_dtype = xdt;
    t.status = status;
    t.merge = 1;
    if ((rc = launch_attention(t, st))) return rc;

    memset(&g, 0, sizeof(g));
    g.w[0] = L.o_proj.w; g.s[0] = L.o_proj.s;
    g.seg_end[0] = H;
    g.nseg = 1;
    g.N = H; g.K = qd; g.M = batch;
    g.x = attn; g.y = hidden; g.ldy = H; g.resid = hidden;
    g.part = part; g.part_cap = W.gemm_part_floats;
    if ((rc = resid_then_norm(g, L.post_attention_layernorm))) return rc;

    memset(&g, 0, sizeof(g));
    g.w[0] = L.gate_proj.w; g.s[0] = L.gate_proj.s;
    g.w[1] = L.up_proj.w;   g.s[1] = L.up_proj.s;
    g.seg_end[0] = I; g.seg_end[1] = 2 * I;
    g.nseg = 2;
    g.N = I; g.K = H; g.M = batch;
    g.x = xh; g.y = act; g.ldy = I;
    g.skinny = 1;
    g.x_tiled = g.y_tiled = xt;
    g.part = part; g.part_cap = W.gemm_part_floats;
    if ((rc = launch_gemm(g, EP_SWIGLU, true, st))) return rc;

    memset(&g, 0, sizeof(g));
    g.w[0] = L.down_proj.w; g.s[0] = L.down_proj.s;
    g.seg_end[0] = H;
    g.nseg = 1;
    g.N = H; g.K = I; g.M = batch;
    g.x = act; g.y = hidden; g.ldy = H; g.resid = hidden;
    g.part = part; g.part_cap = W.gemm_part_floats;
    if (l + 1 < model->num_layers) {
      if ((rc = resid_then_norm(g, model->layers[l + 1].input_layernorm))) return rc;
    } else {
      g.skinny = 1;
      g.x_tiled = xt;
      if ((rc = launch_gemm(g, EP_RESID, false, st))) return rc;
    }
  }
  return run_lm_head_batch(model, hidden, batch, next_tokens, scores, logits, ws, W, st);
}

int q4d_lm_head_argmax_batch(const q4d_model_t* model, const float* hidden, int32_t batch, int32_t* out_tokens,
                             float* out_scores, float* logits, void* ws, size_t ws_bytes, void* stream) {
  if (!hidden || !out_tokens || !out_scores) return Q4D_ERR_NULL;
  if (!model) return Q4D_ERR_NULL;
  int rc = check_matrix(&model->embed_tokens, model->vocab_size, model->hidden_size);
  if (rc) return rc;
  if (!model->final_norm) return Q4D_ERR_NULL;
  if (batch <= 0 || model->vocab_size % 128) return Q4D_ERR_SHAPE;
  if ((rc = check_ws(ws, ws_bytes, model, batch))) return rc;
  return run_lm_head_batch(model, hidden, batch, out_tokens, out_scores, logits, ws, ws_layout(model, batch),
                           as_stream(stream));
}

int q4d_layer_stage(const q4d_model_t* model, int32_t layer, int32_t stage, const float* hidden_in,
                    float* hidden_out, const q4d_kv_cache_t* kv, const int32_t* positions, void* ws,
                    size_t ws_bytes, void* stream) {
  if (stage < Q4D_STAGE_QKV || stage > Q4D_STAGE_DOWN) return Q4D_ERR_SHAPE;
  if (!hidden_in || !hidden_out || !positions) return Q4D_ERR_NULL;
  int rc = check_model(model);
  if (rc) return rc;
  if (layer < 0 || layer >= model->num_layers) return Q4D_ERR_BAD_LAYER;
  if ((rc = check_kv(kv, model, 1))) return rc;
  if (kv->batch != 1) return Q4D_ERR_CAPACITY;
  if ((rc = check_ws(ws, ws_bytes, model, 1))) return rc;
  return run_layer(model, layer, hidden_in, hidden_out, kv, positions, ws, ws_layout(model, 1),
                   as_stream(stream), stage);
}

int q4d_run_one_token(const q4d_model_t* model, const int32_t* tokens, const int32_t* positions,
                      const q4d_kv_cache_t* kv, int32_t* next_token, float* score, float* logits, void* ws,
                      size_t ws_bytes, void* stream) {
  if (!tokens || !positions || !next_token || !score) return Q4D_ERR_NULL;
  int rc = check_model(model);
  if (rc) return rc;
  if ((rc = check_kv(kv, model, 1))) return rc;
  if (kv->batch != 1) return Q4D_ERR_CAPACITY;
  if ((rc = check_ws(ws, ws_bytes, model, 1))) return rc;
  const WsLayout W = ws_layout(model, 1);
  return run_token(model, tokens, positions, kv, next_token, score, logits, ws, W, ws_ptr<int32_t>(ws, W.status),
                   as_stream(stream));
}

int q4d_run_one_token_feedback(const q4d_model_t* model, int32_t* tokens, int32_t* positions,
                               const q4d_kv_cache_t* kv, int32_t* next_token, float* score, float* logits,
                               int32_t* hist_tokens, float* hist_scores, int32_t* hist_count,
                               int32_t hist_capacity, void* ws, size_t ws_bytes, void* stream) {
  if (!tokens || !positions || !next_token || !score) return Q4D_ERR_NULL;
  if (hist_tokens && (!hist_count || hist_capacity < 0)) return Q4D_ERR_NULL;
  int rc = check_model(model);
  if (rc) return rc;
  if ((rc = check_kv(kv, model, 1))) return rc;
  if (kv->batch != 1) return Q4D_ERR_CAPACITY;
  if ((rc = check_ws(ws, ws_bytes, model, 1))) return rc;
  const WsLayout W = ws_layout(model, 1);
  const Feedback fb = {tokens, positions, hist_tokens, hist_scores, hist_count, hist_capacity};
  return run_token(model, tokens, positions, kv, next_token, score, logits, ws, W, ws_ptr<int32_t>(ws, W.status),
                   as_stream(stream), &fb);
}

int q4d_run_one_token_noalloc(const q4d_model_t* model, const int32_t* tokens, const int32_t* positions,
                              const q4d_kv_cache_t* kv, int32_t* next_token, float* score, float* logits,
                              int32_t* status, void* stream) {
  if (!tokens || !positions || !next_token || !score || !status) return Q4D_ERR_NULL;
  int rc = check_model(model);
  if (rc) return rc;
  if ((rc = check_kv(kv, model, 1))) return rc;
  if (kv->batch != 1) return Q4D_ERR_CAPACITY;
  if (!aligned(status, 4)) return Q4D_ERR_BAD_ADDR;
  const WsLayout W = ws_layout(model, 1);
  if (W.total > kNoallocScratchBytes || W.hidden > kNoallocClearWords * 4) return Q4D_ERR_CAPACITY;
  hipStream_t st = as_stream(stream);
  void* ws = nullptr;
  if ((rc = noalloc_scratch(st, &ws))) return rc;
  return run_token(model, tokens, positions, kv, next_token, score, logits, ws, W, status, st);
}

size_t q4d_prefill_workspace_bytes(const q4d_model_t* model, int32_t max_tokens) {
  if (!model || max_tokens <= 0) return 0;
  return prefill_layout(model, max_tokens).total;
}

int q4d_prefill(const q4d_model_t* model, const int32_t* tokens, int32_t n_tokens, int32_t start_pos,
                int32_t seq, const q4d_kv_cache_t* kv, int32_t* next_token, float* score, float* logits, void* ws,
                size_t ws_bytes, void* stream) {
  if (!tokens || !next_token || !score) return Q4D_ERR_NULL;
  int rc = check_model(model);
  if (rc) return rc;
  if (n_tokens <= 0) return Q4D_ERR_SHAPE;
  if ((rc = check_kv(kv, model, 1))) return rc;
  if (seq < 0 || seq >= kv->batch) return Q4D_ERR_CAPACITY;
  if (start_pos < 0 || (long long)start_pos + n_tokens > model->max_ctx) return Q4D_ERR_CONTEXT;
  if (!ws) return Q4D_ERR_NULL;
  if (!aligned(ws, 256)) return Q4D_ERR_BAD_ADDR;
  const PrefillLayout P = prefill_layout(model, n_tokens);
  if (ws_bytes < P.total) return Q4D_ERR_CAPACITY;
  hipStream_t st = as_stream(stream);
  const int n = n_tokens, H = model->hidden_size, I = model->intermediate_size;
  const int qh = model->num_q_heads, kvh = model->num_kv_heads, d = model->head_dim;
  float* hidden = ws_ptr<float>(ws, P.hidden);
  uint16_t* xh = ws_ptr<uint16_t>(ws, P.xh);
  uint16_t* act = ws_ptr<uint16_t>(ws, P.act);
  if ((rc = launch_embedding(&model->embed_tokens, tokens, n, hidden, ws_ptr<int32_t>(ws, P.base.status), st)))
    return rc;
  const size_t seq_off = (size_t)seq * kvh * kv->max_ctx * d;
  for (int l = 0; l < model->num_layers; ++l) {
    const q4d_layer_t& L = model->layers[l];
    // input RMSNorm -> fp16 (layers after the first get it from the previous down GEMM's
    // fused reduction), then q|k|v as one three-segment GEMM whose epilogue applies the
    // q/k RMSNorm and RoPE and appends K/V for all n positions
    if (l == 0 && (rc = launch_rms_norm(hidden, L.input_layernorm, model->rms_norm_eps, n, H, xh, Q4D_F16, st)))
      return rc;
    PrefillArgs pa;
    memset(&pa, 0, sizeof(pa));
    pa.q_gamma = L.q_norm;
    pa.k_gamma = L.k_norm;
    pa.eps = model->rms_norm_eps;
    pa.qscale = model->attn_scaling * 1.4426950408889634f;
    pa.rope_cos = model->rope_cos;
    pa.rope_sin = model->rope_sin;
    uint16_t *kp, *vp;
    kv_planes(kv, l, &kp, &vp);
    pa.kcache = kp + seq_off;
    pa.vcache = vp + seq_off;
    pa.q16 = ws_ptr<_Float16>(ws, P.q16);
    pa.out = ws_ptr<_Float16>(ws, P.attn);
    pa.n = n; pa.p0 = start_pos; pa.qh = qh; pa.kvh = kvh; pa.max_ctx = model->max_ctx;
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.w[0] = L.q_proj.w; g.s[0] = L.q_proj.s;
    g.w[1] = L.k_proj.w; g.s[1] = L.k_proj.s;
    g.w[2] = L.v_proj.w; g.s[2] = L.v_proj.s;
    g.seg_end[0] = L.q_proj.rows;
    g.seg_end[1] = g.seg_end[0] + L.k_proj.rows;
    g.seg_end[2] = g.seg_end[1] + L.v_proj.rows;
    g.nseg = 3;
    g.N = g.seg_end[2]; g.K = H; g.M = n;
    g.x = xh;
    g.rope = pa;
    if ((rc = launch_gemm(g, EP_ROPE, false, st))) return rc;

    // causal GQA attention over positions [0, start_pos + n)
    if ((rc = launch_prefill_attention(pa, st))) return rc;

    // o_proj + residual, post-attention RMSNorm, gate/up + SwiGLU, down + residual
    memset(&g, 0, sizeof(g));
    g.w[0] = L.o_proj.w; g.s[0] = L.o_proj.s;
    g.seg_end[0] = H; g.nseg = 1;
    g.N = H; g.K = qh * d; g.M = n;
    g.x = ws_ptr<uint16_t>(ws, P.attn); g.y = hidden; g.ldy = H; g.resid = hidden;
    g.part = ws_ptr<float>(ws, P.part); g.part_cap = (size_t)kPrefillSplit * n * H; g.ksplit = kPrefillSplit;
    g.defer_reduce = 1;  // split sums + residual + post-attention RMSNorm in one pass
    if ((rc = launch_gemm(g, EP_RESID, false, st))) return rc;
    if ((rc = launch_splitk_resid_norm(g, kPrefillSplit, L.post_attention_layernorm, model->rms_norm_eps,
                                       xh, st)))
      return rc;
    memset(&g, 0, sizeof(g));
    g.w[0] = L.gate_proj.w; g.s[0] = L.gate_proj.s;
    g.w[1] = L.up_proj.w;   g.s[1] = L.up_proj.s;
    g.seg_end[0] = I; g.seg_end[1] = 2 * I; g.nseg = 2;
    g.N = I; g.K = H; g.M = n;
    g.x = xh; g.y = act; g.ldy = I;
    if ((rc = launch_gemm(g, EP_SWIGLU, true, st))) return rc;
    memset(&g, 0, sizeof(g));
    g.w[0] = L.down_proj.w; g.s[0] = L.down_proj.s;
    g.seg_end[0] = H; g.nseg = 1;
    g.N = H; g.K = I; g.M = n;
    g.x = act; g.y = hidden; g.ldy = H; g.resid = hidden;
    g.part = ws_ptr<float>(ws, P.part); g.part_cap = (size_t)kPrefillSplit * n * H; g.ksplit = kPrefillSplit;
    if (l + 1 < model->num_layers) {  // split sums + residual + the next layer's input RMSNorm
      g.defer_reduce = 1;
      if ((rc = launch_gemm(g, EP_RESID, false, st))) return rc;
      if ((rc = launch_splitk_resid_norm(g, kPrefillSplit, model->layers[l + 1].input_layernorm,
                                         model->rms_norm_eps, xh, st)))
        return rc;
    } else if ((rc = launch_gemm(g, EP_RESID, false, st))) {
      return rc;
    }
  }
  // final RMSNorm + LM head + argmax for the last token
  return run_lm_head(model, hidden + (size_t)(n - 1) * H, next_token, score, logits, ws, P.base, st);
}

int q4d_advance(int32_t* tokens, int32_t* positions, const int32_t* next_token, const float* score,
                int32_t* hist_tokens, float* hist_scores, int32_t* hist_count, int32_t hist_capacity,
                void* stream) {
  if (!tokens || !positions || !next_token) return Q4D_ERR_NULL;
  if (hist_tokens && (!hist_count || !score || hist_capacity < 0)) return Q4D_ERR_NULL;
  return launch_advance(tokens, positions, next_token, score, hist_tokens, hist_scores, hist_count,
                        hist_capacity, as_stream(stream));
}

int q4d_advance_session(int32_t* tokens, int32_t* positions, const int32_t* next_token, const float* score,
                        int32_t* hist_tokens, float* hist_scores, int32_t* hist_count, int32_t hist_capacity,
                        int32_t* stop_state, void* stream) {
  if (!tokens || !positions || !next_token || !stop_state) return Q4D_ERR_NULL;
  if (hist_tokens && (!hist_count || !score || hist_capacity < 0)) return Q4D_ERR_NULL;
  if (!aligned(stop_state, 4)) return Q4D_ERR_BAD_ADDR;
  return launch_advance_session(tokens, positions, next_token, score, hist_tokens, hist_scores, hist_count,
                                hist_capacity, stop_state, as_stream(stream));
}

int q4d_apply_rope(const float* x, float* y, const float* cos, const float* sin, int32_t batch, int32_t heads,
                   int32_t head_dim, void* stream) {
  return q4d_apply_rope_seq(x, y, cos, sin, batch, heads, 1, head_dim, stream);
}

int q4d_apply_rope_seq(const float* x, float* y, const float* cos, const float* sin, int32_t batch, int32_t heads,
                       int32_t seq, int32_t head_dim, void* stream) {
  if (!x || !y || !cos || !sin) return Q4D_ERR_NULL;
  if (batch <= 0 || heads <= 0 || seq <= 0 || head_dim <= 0 || (head_dim & 1)) return Q4D_ERR_SHAPE;
  return launch_apply_rope(x, y, cos, sin, batch, heads, seq, head_dim, as_stream(stream));
}

int q4d_rotate_half(const float* x, float* y, int64_t rows, int32_t head_dim, void* stream) {
  if (!x || !y) return Q4D_ERR_NULL;
  if (rows <= 0 || head_dim <= 0 || (head_dim & 1) || rows > (int64_t(1) << 40) / head_dim) return Q4D_ERR_SHAPE;
  return launch_rotate_half(x, y, rows, head_dim, as_stream(stream));
}

size_t q4d_causal_attention_workspace_bytes(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t seq) {
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || seq <= 0) return 0;
  return causal_attention_ws_bytes(batch, q_heads, kv_heads, seq);
}

int q4d_causal_attention(const float* q, const float* k, const float* v, float* out, int32_t batch,
                         int32_t q_heads, int32_t kv_heads, int32_t seq, int32_t head_dim, float scaling, void* ws,
                         size_t ws_bytes, void* stream) {
  if (!q || !k || !v || !out || !ws) return Q4D_ERR_NULL;
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || seq <= 0 || q_heads % kv_heads || q_heads > 65535)
    return Q4D_ERR_SHAPE;
  if (head_dim != 128) return Q4D_ERR_SHAPE;
  if ((long long)batch * q_heads * seq * head_dim > (1LL << 40)) return Q4D_ERR_SHAPE;
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16) || !aligned(ws, 256))
    return Q4D_ERR_BAD_ADDR;
  if (ws_bytes < causal_attention_ws_bytes(batch, q_heads, kv_heads, seq)) return Q4D_ERR_CAPACITY;
  return launch_causal_attention(q, k, v, out, batch, q_heads, kv_heads, seq, scaling, ws, as_stream(stream));
}

int q4d_diag_launch_chain(const int32_t* grid_x, const int32_t* grid_y, const int32_t* block, int32_t n,
                          float* buf, void* stream) {
  if (!grid_x || !grid_y || !block || !buf) return Q4D_ERR_NULL;
  if (n <= 0 || n > 4096) return Q4D_ERR_SHAPE;
  if (!aligned(buf, 16)) return Q4D_ERR_BAD_ADDR;
  for (int i = 0; i < n; ++i)
    if (grid_x[i] < 1 || grid_x[i] > 65535 || grid_y[i] < 1 || grid_y[i] > 65535 || block[i] < 64 ||
        block[i] > 1024 || block[i] % 64)
      return Q4D_ERR_SHAPE;
  return launch_chain(grid_x, grid_y, block, n, buf, as_stream(stream));
}

}  // extern "C"
