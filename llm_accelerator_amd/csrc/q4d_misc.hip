// Small decode kernels: RMSNorm, per-head RMSNorm + RoPE, KV append, Q4
// embedding gather, fills and the device-side decode-loop advance.
#include <math.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

// manual_rms_norm (reference common.py:129-134): one block per row.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* x, const float* gamma, float eps,
                                                       int dim, void* y, int y_dtype) {
  __shared__ float sred[4];
  const int row = blockIdx.x, t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const float* xr = x + (size_t)row * dim;
  float ss = 0.f;
  for (int i = t; i < dim; i += 256) ss = fmaf(xr[i], xr[i], ss);
  ss = wave_sum(ss);
  if (lane == 0) sred[wid] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf(((sred[0] + sred[1]) + (sred[2] + sred[3])) / (float)dim + eps);
  for (int i = t; i < dim; i += 256) {
    const float v = (xr[i] * inv) * gamma[i];
    if (y_dtype == Q4D_F16)
      static_cast<_Float16*>(y)[(size_t)row * dim + i] = (_Float16)v;
    else if (y_dtype == kF16Tiled)
      static_cast<_Float16*>(y)[xt_index(row, i)] = (_Float16)v;
    else
      static_cast<float*>(y)[(size_t)row * dim + i] = v;
  }
}

int launch_rms_norm(const float* x, const float* gamma, float eps, int rows, int dim, void* y,
                    int y_dtype, hipStream_t stream) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), 0, stream, x, gamma, eps, dim, y, y_dtype);
  return check_launch();
}

// Per-head RMSNorm with gamma then rotate-half RoPE (common.py:148-183,
// 258-268).  One block of head_dim (= 128) threads per (batch, head).
__global__ __launch_bounds__(128) void qk_norm_rope_kernel(const float* x, float* y, const float* gamma,
                                                           float eps, int heads, const float* cosT,
                                                           const float* sinT, int max_ctx,
                                                           const int32_t* positions, int32_t* status) {
  constexpr int D = 128;
  __shared__ float sred[2];
  __shared__ float sv[D];
  const int bh = blockIdx.x, b = bh / heads;
  const int d = threadIdx.x, lane = d & 63, wid = d >> 6;
  const int pos = positions[b];
  if (pos < 0 || pos >= max_ctx) {
    if (d == 0) atomicOr(status, Q4D_STATUS_BAD_POSITION);
    return;
  }
  const float v = x[(size_t)bh * D + d];
  const float ss = wave_sum(v * v);
  if (lane == 0) sred[wid] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((sred[0] + sred[1]) / (float)D + eps);
  const float vn = (v * inv) * gamma[d];
  sv[d] = vn;
  __syncthreads();
  const float rot = d < 64 ? -sv[d + 64] : sv[d - 64];
  const float c = cosT[(size_t)pos * (D / 2) + (d & 63)];
  const float s = sinT[(size_t)pos * (D / 2) + (d & 63)];
  y[(size_t)bh * D + d] = vn * c + rot * s;
}

int launch_qk_norm_rope(const float* x, float* y, const float* gamma, float eps, int batch, int heads,
                        int head_dim, const float* cosT, const float* sinT, int max_ctx,
                        const int32_t* positions, int32_t* status, hipStream_t stream) {
  if (head_dim != 128) return Q4D_ERR_SHAPE;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(batch * heads), dim3(128), 0, stream, x, y, gamma, eps,
                     heads, cosT, sinT, max_ctx, positions, status);
  return check_launch();
}

// append_cache (common.py:186-189) into [layer][K/V][batch][head][pos][dim].
__global__ __launch_bounds__(128) void kv_append_kernel(uint16_t* kplane, uint16_t* vplane, const float* k,
                                                        const float* v, int kvh, int max_ctx, int head_dim,
                                                        const int32_t* positions, int32_t* status) {
  const int bh = blockIdx.x, b = bh / kvh;
  const int pos = positions[b];
  if (pos < 0 || pos >= max_ctx) {
    if (threadIdx.x == 0) atomicOr(status, Q4D_STATUS_BAD_POSITION);
    return;
  }
  const size_t dst = ((size_t)bh * max_ctx + pos) * head_dim;
  for (int d = threadIdx.x; d < head_dim; d += 128) {
    if (k) reinterpret_cast<_Float16*>(kplane)[dst + d] = (_Float16)k[(size_t)bh * head_dim + d];
    if (v) reinterpret_cast<_Float16*>(vplane)[dst + d] = (_Float16)v[(size_t)bh * head_dim + d];
  }
}

int launch_kv_append(const q4d_kv_cache_t* kv, int layer, const float* k, const float* v,
                     const int32_t* positions, int32_t* status, hipStream_t stream) {
  const size_t plane = (size_t)kv->batch * kv->num_kv_heads * kv->max_ctx * kv->head_dim;
  uint16_t* kp = kv->data + (size_t)layer * 2 * plane;
  hipLaunchKernelGGL(kv_append_kernel, dim3(kv->batch * kv->num_kv_heads), dim3(128), 0, stream, kp,
                     kp + plane, k, v, kv->num_kv_heads, kv->max_ctx, kv->head_dim, positions, status);
  return check_launch();
}

// Tied Q4 embedding row -> fp32 hidden: W = q * scale / 2^14 (exact), the
// float form of reference 49_export_q4_embedding_vectors.py:99-101.
__global__ __launch_bounds__(256) void embedding_kernel(const uint8_t* w, const uint16_t* s, int vocab,
                                                        int cols, const int32_t* tokens, float* hidden,
                                                        int32_t* status) {
  const int b = blockIdx.x;
  const int tok = tokens[b];
  float* out = hidden + (size_t)b * cols;
  if (tok < 0 || tok >= vocab) {
    if (threadIdx.x == 0 && status) atomicOr(status, Q4D_STATUS_BAD_TOKEN);
    for (int c = threadIdx.x; c < cols; c += 256) out[c] = 0.f;
    return;
  }
  const uint8_t* row = w + (size_t)tok * (cols / 2);
  const uint16_t* sr = s + (size_t)tok * (cols / 64);
  for (int c = threadIdx.x; c < cols / 2; c += 256) {
    const uint32_t byte = row[c];
    const float sc = scale_q2_14(sr[(2 * c) >> 6]);
    const int lo = (int)(byte & 0xF) - ((byte & 0x8) ? 16 : 0);
    const int hi = (int)(byte >> 4) - ((byte & 0x80) ? 16 : 0);
    out[2 * c] = (float)lo * sc;
    out[2 * c + 1] = (float)hi * sc;
  }
}

int launch_embedding(const q4d_matrix_t* t, const int32_t* tokens, int batch, float* hidden,
                     int32_t* status, hipStream_t stream) {
  hipLaunchKernelGGL(embedding_kernel, dim3(batch), dim3(256), 0, stream, t->w, t->s, t->rows, t->cols,
                     tokens, hidden, status);
  return check_launch();
}

__global__ void fill_i32_kernel(int32_t* p, int32_t v, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = v;
}

int launch_fill_i32(int32_t* p, int32_t v, size_t n, hipStream_t stream) {
  const int blocks = (int)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
  hipLaunchKernelGGL(fill_i32_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, stream, p, v, n);
  return check_launch();
}

// Launch-floor probe: a kernel that only reads the previous launch's 4 KB output (one
// dependent global load per thread) and, in block 0, writes its own (in + 1).  A chain
// of these with the grids of a decode step measures what the launches cost without
// their work.
__global__ void chain_kernel(const float* __restrict__ in, float* __restrict__ out) {
  const int t = threadIdx.x;
  if (blockIdx.x == 0 && blockIdx.y == 0) {
    for (int i = t; i < 1024; i += blockDim.x) out[i] = in[i] + 1.0f;
  } else {
    const float v = in[t & 1023];
    if (v != v) out[t & 1023] = v;  // never taken for finite data; keeps the read
  }
}

int launch_chain(const int32_t* grid_x, const int32_t* grid_y, const int32_t* block, int n, float* buf,
                 hipStream_t stream) {
  for (int i = 0; i < n; ++i) {
    const float* in = buf + (i & 1) * 1024;
    float* out = buf + ((i + 1) & 1) * 1024;
    hipLaunchKernelGGL(chain_kernel, dim3(grid_x[i], grid_y[i]), dim3(block[i]), 0, stream, in, out);
  }
  return check_launch();
}

__global__ void advance_kernel(int32_t* tokens, int32_t* positions, const int32_t* next_token,
                               const float* score, int32_t* hist_tokens, float* hist_scores,
                               int32_t* hist_count, int32_t hist_capacity) {
  if (threadIdx.x == 0) {
    const int32_t nt = next_token[0];
    tokens[0] = nt;
    positions[0] += 1;
    if (hist_tokens) {
      const int32_t c = hist_count[0];
      if (c < hist_capacity) {
        hist_tokens[c] = nt;
        if (hist_scores) hist_scores[c] = score[0];
        hist_count[0] = c + 1;
      }
    }
  }
}

// The advance step with the decode session's stop rules applied on the device
// (qot_session.c:41-60 checks them in this order after every generated token):
// end-of-text, end-of-turn, the new-token budget, the context cap.  stop: int32[8] =
// done, stop reason, generated count, max new tokens, end-of-text id (-1: off),
// end-of-turn id (-1: off), max context, unused.  Once done, nothing moves: a
// replayed step recomputes the last row with the same token and position.
__global__ void advance_session_kernel(int32_t* tokens, int32_t* positions, const int32_t* next_token,
                                       const float* score, int32_t* hist_tokens, float* hist_scores,
                                       int32_t* hist_count, int32_t hist_capacity, int32_t* stop) {
  if (threadIdx.x != 0 || stop[0]) return;
  const int32_t nt = next_token[0];
  if (hist_tokens) {
    const int32_t c = hist_count[0];
    if (c < hist_capacity) {
      hist_tokens[c] = nt;
      if (hist_scores) hist_scores[c] = score[0];
      hist_count[0] = c + 1;
    }
  }
  const int32_t gen = stop[2] + 1;
  stop[2] = gen;
  int32_t why = Q4D_SESSION_STOP_NONE;
  if (stop[4] >= 0 && nt == stop[4]) why = Q4D_SESSION_STOP_EOS;
  else if (stop[5] >= 0 && nt == stop[5]) why = Q4D_SESSION_STOP_IM_END;
  else if (gen >= stop[3]) why = Q4D_SESSION_STOP_MAX_NEW;
  else if (positions[0] + 1 >= stop[6]) why = Q4D_SESSION_STOP_CONTEXT;
  if (why != Q4D_SESSION_STOP_NONE) {
    stop[1] = why;
    stop[0] = 1;
    return;
  }
  tokens[0] = nt;
  positions[0] += 1;
}

int launch_advance_session(int32_t* tokens, int32_t* positions, const int32_t* next_token, const float* score,
                           int32_t* hist_tokens, float* hist_scores, int32_t* hist_count, int32_t hist_capacity,
                           int32_t* stop, hipStream_t stream) {
  hipLaunchKernelGGL(advance_session_kernel, dim3(1), dim3(64), 0, stream, tokens, positions, next_token, score,
                     hist_tokens, hist_scores, hist_count, hist_capacity, stop);
  return check_launch();
}

int launch_advance(int32_t* tokens, int32_t* positions, const int32_t* next_token, const float* score,
                   int32_t* hist_tokens, float* hist_scores, int32_t* hist_count, int32_t hist_capacity,
                   hipStream_t stream) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, stream, tokens, positions, next_token, score,
                     hist_tokens, hist_scores, hist_count, hist_capacity);
  return check_launch();
}

// y = x * cos + rotate_half(x) * sin (common.py:148-152, 173-183) for x [batch, heads,
// seq, head_dim] and cos / sin [batch, seq, head_dim]; one block per (batch, head, position).
__global__ __launch_bounds__(128) void apply_rope_kernel(const float* x, float* y, const float* cosv,
                                                         const float* sinv, int heads, int seq, int head_dim) {
  const int r = blockIdx.x, sp = r % seq, b = r / seq / heads, half = head_dim / 2;
  const float* xr = x + (size_t)r * head_dim;
  const float* cr = cosv + ((size_t)b * seq + sp) * head_dim;
  const float* sr = sinv + ((size_t)b * seq + sp) * head_dim;
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
    const float rot = d < half ? -xr[d + half] : xr[d - half];
    y[(size_t)r * head_dim + d] = xr[d] * cr[d] + rot * sr[d];
  }
}

int launch_apply_rope(const float* x, float* y, const float* cosv, const float* sinv, int batch, int heads,
                      int seq, int head_dim, hipStream_t stream) {
  if (x == y) return Q4D_ERR_SHAPE;  // rotate_half reads the other half of the row
  const long long rows = (long long)batch * heads * seq;
  if (rows > 0x7fffffffLL) return Q4D_ERR_SHAPE;
  hipLaunchKernelGGL(apply_rope_kernel, dim3((unsigned)rows), dim3(128), 0, stream, x, y, cosv, sinv, heads, seq,
                     head_dim);
  return check_launch();
}

// y = cat(-x[..., half:], x[..., :half]) per row of head_dim (common.py:148-152).
__global__ __launch_bounds__(256) void rotate_half_kernel(const float* x, float* y, long long n, int head_dim) {
  const int half = head_dim / 2;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    const int d = (int)(i % head_dim);
    y[i] = d < half ? -x[i + half] : x[i - half];
  }
}

int launch_rotate_half(const float* x, float* y, long long rows, int head_dim, hipStream_t stream) {
  if (x == y) return Q4D_ERR_SHAPE;
  const long long n = rows * head_dim;
  const long long blocks = (n + 255) / 256;
  hipLaunchKernelGGL(rotate_half_kernel, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, stream,
                     x, y, n, head_dim);
  return check_launch();
}

}  // namespace q4d
