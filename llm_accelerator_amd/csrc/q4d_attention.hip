// GQA decode attention over an fp16 KV cache (gfx950, wave64).
//
// Follows manual_repeat_kv + manual_cached_attention (reference
// Qwen3-0.6B-Base/python_each_module/common.py:192-228): q head h reads kv
// head h / (q_heads / kv_heads); scores = q.k * scaling; softmax in fp32;
// out = softmax . v.  The cache plane of one layer is
// [batch][kv_head][max_ctx][head_dim] fp16 so each head streams contiguously.
//
// Grid (split, kv_head, batch); one 256-thread block handles the two q heads
// of one kv head over kAttnChunk (= 64) consecutive positions:
//   * scores: 16 lanes per position (16 B of K each), 4 positions per wave;
//   * softmax of the chunk in one wave per head (exp2 with log2e folded into q);
//   * P.V: each wave takes every 4th position, lanes own 2 dims;
//   * the (max, sum, partial output) of the chunk goes to the workspace and
//     the last block of a (batch, kv head) to arrive merges all chunks.
// With fused = 1 the block first applies the per-head q/k RMSNorm and RoPE of
// common.py:258-268 to the raw projections and the block owning the last
// chunk appends the new K/V row (append_cache, common.py:186-189).
#include <math.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

static_assert(kAttnChunk == kWave, "softmax uses one lane per position");

__global__ __launch_bounds__(256) void attn_decode_kernel(const AttnArgs a) {
  constexpr int D = 128;
  const int s = blockIdx.x, j = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int pos = a.positions[b];
  if (pos < 0 || pos >= a.max_ctx) {
    if (s == 0 && j == 0 && t == 0) atomicOr(a.status, Q4D_STATUS_BAD_POSITION);
    return;
  }
  const int T = pos + 1;
  const int nsplit = (T + kAttnChunk - 1) / kAttnChunk;
  if (s >= nsplit) return;
  const int start = s * kAttnChunk;
  const int n = min(T, start + kAttnChunk) - start;

  __shared__ float sq[2][D];
  __shared__ float sk[D];
  __shared__ float sred[8];
  __shared__ float ssc[2][kAttnChunk];
  __shared__ float sml[2][2];
  __shared__ float spv[4][2][D];
  __shared__ int s_last;

  const int hh = t >> 7;  // which of the two q heads (threads 0-127 / 128-255)
  const int d = t & (D - 1);
  const int h = j * 2 + hh;
  const int qkv_stride = (a.qh + 2 * a.kvh) * D;
  const float qscale = a.scaling * 1.4426950408889634f;  // fold log2(e) for exp2
  const size_t plane_off = ((size_t)(b * a.kvh + j) * a.max_ctx) * D;
  uint16_t* kb = a.kcache + plane_off;
  uint16_t* vb = a.vcache + plane_off;

  if (a.fused) {
    const float c = a.rope_cos[(size_t)pos * (D / 2) + (d & 63)];
    const float sn = a.rope_sin[(size_t)pos * (D / 2) + (d & 63)];
    // q: per-head RMSNorm (common.py:260) then RoPE (common.py:267-268)
    const float qv = a.qkv[(size_t)b * qkv_stride + h * D + d];
    const float ss = wave_sum(qv * qv);
    if (lane == 0) sred[wid] = ss;
    __syncthreads();
    const float qinv = 1.0f / sqrtf((sred[2 * hh] + sred[2 * hh + 1]) / (float)D + a.eps);
    const float qn = (qv * qinv) * a.q_gamma[d];
    sq[hh][d] = qn;
    __syncthreads();
    const float qrot = d < 64 ? -sq[hh][d + 64] : sq[hh][d - 64];
    const float qr = qn * c + qrot * sn;
    __syncthreads();
    sq[hh][d] = qr * qscale;

    if (s == nsplit - 1) {  // block-uniform: this chunk holds position pos
      // threads 0-127: new k (norm + RoPE); threads 128-255: new v
      const float kv = a.qkv[(size_t)b * qkv_stride + (a.qh + hh * a.kvh + j) * D + d];
      const float ks = wave_sum(kv * kv);
      if (lane == 0) sred[4 + wid] = ks;
      __syncthreads();
      const float kinv = 1.0f / sqrtf((sred[4] + sred[5]) / (float)D + a.eps);
      const float kn = (kv * kinv) * a.k_gamma[d];
      if (hh == 0) sk[d] = kn;
      __syncthreads();
      if (hh == 0) {
        const float krot = d < 64 ? -sk[d + 64] : sk[d - 64];
        const float kr = kn * c + krot * sn;
        reinterpret_cast<_Float16*>(kb)[(size_t)pos * D + d] = (_Float16)kr;
      } else {
        reinterpret_cast<_Float16*>(vb)[(size_t)pos * D + d] = (_Float16)kv;
      }
      __threadfence_block();
    }
  } else {
    sq[hh][d] = a.q[((size_t)b * a.qh + h) * D + d] * qscale;
  }
  __syncthreads();

  // ---- scores: 16 lanes per position, 8 dims per lane --------------------------
  const int sub = lane & 15;
  float q0[8], q1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    q0[e] = sq[0][sub * 8 + e];
    q1[e] = sq[1][sub * 8 + e];
  }
  for (int p0 = wid * 4; p0 < n; p0 += 16) {
    const int p = p0 + (lane >> 4);
    float s0 = 0.f, s1 = 0.f;
    if (p < n) {
      const u32x4 kk = *reinterpret_cast<const u32x4*>(kb + (size_t)(start + p) * D + sub * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // copy the element out first: bit-casting a vector element expression
        // directly reads element 0 with this compiler
        const uint32_t ke = kk[e];
        const h2 k2 = __builtin_bit_cast(h2, ke);
        const float ka = (float)k2.x, kc = (float)k2.y;
        s0 = fmaf(q0[2 * e], ka, s0);
        s0 = fmaf(q0[2 * e + 1], kc, s0);
        s1 = fmaf(q1[2 * e], ka, s1);
        s1 = fmaf(q1[2 * e + 1], kc, s1);
      }
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) {
      s0 += shfl_xor_f(s0, m);
      s1 += shfl_xor_f(s1, m);
    }
    if (sub == 0 && p < n) {
      ssc[0][p] = s0;
      ssc[1][p] = s1;
    }
  }
  __syncthreads();

  // ---- chunk softmax (one wave per head, one lane per position) -----------------
  if (wid < 2) {
    const float sc = lane < n ? ssc[wid][lane] : -INFINITY;
    const float m = wave_max(sc);
    const float e = lane < n ? exp2f(sc - m) : 0.f;
    const float l = wave_sum(e);
    if (lane < n) ssc[wid][lane] = e;
    if (lane == 0) {
      sml[wid][0] = m;
      sml[wid][1] = l;
    }
  }
  __syncthreads();

  // ---- P.V: wave takes positions wid, wid+4, ...; lane owns dims 2l, 2l+1 ------
  float a00 = 0.f, a01 = 0.f, a10 = 0.f, a11 = 0.f;
#pragma unroll 4
  for (int p = wid; p < n; p += 4) {
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(vb + (size_t)(start + p) * D + 2 * lane);
    const h2 v2 = __builtin_bit_cast(h2, vv);
    const float v0 = (float)v2.x, v1 = (float)v2.y;
    const float e0 = ssc[0][p], e1 = ssc[1][p];
    a00 = fmaf(e0, v0, a00);
    a01 = fmaf(e0, v1, a01);
    a10 = fmaf(e1, v0, a10);
    a11 = fmaf(e1, v1, a11);
  }
  spv[wid][0][2 * lane] = a00;
  spv[wid][0][2 * lane + 1] = a01;
  spv[wid][1][2 * lane] = a10;
  spv[wid][1][2 * lane + 1] = a11;
  __syncthreads();
  const float acc = (spv[0][hh][d] + spv[1][hh][d]) + (spv[2][hh][d] + spv[3][hh][d]);

  // ---- publish the chunk partial; the last block per (batch, kv head) merges ----
  const size_t pbase = (size_t)(b * a.qh + h) * a.nsplit_max;
  a.part_acc[(pbase + s) * D + d] = acc;
  if (d == 0) {
    a.part_ml[(pbase + s) * 2 + 0] = sml[hh][0];
    a.part_ml[(pbase + s) * 2 + 1] = sml[hh][1];
  }
  __threadfence();
  __syncthreads();
  int* counter = a.counters + b * a.kvh + j;
  if (t == 0) s_last = (atomicAdd(counter, 1) == nsplit - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  float M = -INFINITY;
  for (int i = 0; i < nsplit; ++i) M = fmaxf(M, a.part_ml[(pbase + i) * 2]);
  float Lsum = 0.f, o = 0.f;
  for (int i = 0; i < nsplit; ++i) {
    const float w = exp2f(a.part_ml[(pbase + i) * 2] - M);
    Lsum = fmaf(a.part_ml[(pbase + i) * 2 + 1], w, Lsum);
    o = fmaf(a.part_acc[(pbase + i) * D + d], w, o);
  }
  const float r = o / Lsum;
  const size_t oi = ((size_t)b * a.qh + h) * D + d;
  if (a.out_dtype == Q4D_F16)
    static_cast<_Float16*>(a.out)[oi] = (_Float16)r;
  else
    static_cast<float*>(a.out)[oi] = r;
  if (t == 0) *counter = 0;
}

int launch_attention(const AttnArgs& a, hipStream_t stream) {
  const int nsplit = a.nsplit_max;
  dim3 grid(nsplit, a.kvh, a.batch);
  hipLaunchKernelGGL(attn_decode_kernel, grid, dim3(256), 0, stream, a);
  return check_launch();
}

}  // namespace q4d
