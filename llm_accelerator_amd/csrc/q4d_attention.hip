// GQA decode attention over an fp16 KV cache (gfx950, wave64).
//
// Follows manual_repeat_kv + manual_cached_attention (reference
// Qwen3-0.6B-Base/python_each_module/common.py:192-228): q head h reads kv
// head h / (q_heads / kv_heads); scores = q.k * scaling; softmax in fp32;
// out = softmax . v.  The cache plane of one layer is
// [batch][kv_head][max_ctx][head_dim] fp16 so each head streams contiguously.
//
// Two kernels (split-K over the context, flash-decoding style):
//  1. attn_split_kernel, grid (split, kv_head, batch), 256 threads: the two q
//     heads of one kv head over kAttnChunk (= 64) positions.  Thread t owns
//     dims 8*(t%16)..+7 of positions t/16 + 16*i (i < 4) for both K and V and
//     issues its eight 16-byte loads together, so a chunk costs one memory
//     round trip.  Scores are 8-dim partial dots reduced over the 16 lanes of
//     a position; the chunk softmax runs in one wave per head (exp2, log2e
//     folded into q); P.V accumulates 16 values per thread.  The chunk's
//     (max, sum, partial output) goes to the workspace.
//  2. attn_merge_kernel, grid (kv_head, batch): rescales and sums the chunk
//     partials.  The kernel boundary orders the two, so no device-scope fence
//     (an L2 write-back on this part) is needed.
// With fused = 1 the split kernel first applies the per-head q/k RMSNorm and
// RoPE of common.py:258-268 to the raw projections; the block owning the
// last chunk appends the new K/V row (append_cache, common.py:186-189) and
// takes that position from LDS instead of reading back its own global write.
#include <math.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

static_assert(kAttnChunk == 64, "thread mapping assumes 64 positions per chunk");

__device__ __forceinline__ void unpack8(const u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t we = w[e];
    const h2 v = __builtin_bit_cast(h2, we);
    f[2 * e] = (float)v.x;
    f[2 * e + 1] = (float)v.y;
  }
}

__global__ __launch_bounds__(256) void attn_split_kernel(const AttnArgs a) {
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
  // positions below `cached` are read from the cache; in fused mode the new
  // position pos is produced here
  const int cached = a.fused ? pos : T;

  __shared__ float sq[2][D];
  __shared__ float sk[D];
  __shared__ uint16_t snew[2][D];  // fp16 bits of the appended k (roped) and v
  __shared__ float sred[8];
  __shared__ float ssc[2][kAttnChunk];
  __shared__ float sml[2][2];
  __shared__ float spv[4][2][D];

  const size_t plane_off = ((size_t)(b * a.kvh + j) * a.max_ctx) * D;
  uint16_t* kb = a.kcache + plane_off;
  uint16_t* vb = a.vcache + plane_off;

  // ---- issue every K/V load of this chunk first ------------------------------
  const int sub = t & 15;  // dims 8*sub .. 8*sub+7
  const int pr = t >> 4;   // positions pr + 16*i
  u32x4 kr[4], vr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = start + pr + 16 * i;
    if (p < cached) {
      kr[i] = *reinterpret_cast<const u32x4*>(kb + (size_t)p * D + sub * 8);
      vr[i] = *reinterpret_cast<const u32x4*>(vb + (size_t)p * D + sub * 8);
    } else {
      kr[i] = u32x4{0u, 0u, 0u, 0u};
      vr[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }

  const int hh = t >> 7;  // which of the two q heads (threads 0-127 / 128-255)
  const int d = t & (D - 1);
  const int h = j * 2 + hh;
  const float qscale = a.scaling * 1.4426950408889634f;  // fold log2(e) for exp2
  const bool last = (s == nsplit - 1);                   // block-uniform: holds pos

  if (a.fused) {
    const int qkv_stride = (a.qh + 2 * a.kvh) * D;
    const float c = a.rope_cos[(size_t)pos * (D / 2) + (d & 63)];
    const float sn = a.rope_sin[(size_t)pos * (D / 2) + (d & 63)];
    const float qv = a.qkv[(size_t)b * qkv_stride + h * D + d];
    // threads 0-127: new k; threads 128-255: new v (only the last chunk)
    const float kv = last ? a.qkv[(size_t)b * qkv_stride + (a.qh + hh * a.kvh + j) * D + d] : 0.f;
    // q: per-head RMSNorm (common.py:260) then RoPE (common.py:267-268)
    const float qs = wave_sum(qv * qv);
    const float ks = wave_sum(kv * kv);
    if (lane == 0) {
      sred[wid] = qs;
      sred[4 + wid] = ks;
    }
    __syncthreads();
    const float qinv = 1.0f / sqrtf((sred[2 * hh] + sred[2 * hh + 1]) / (float)D + a.eps);
    const float qn = (qv * qinv) * a.q_gamma[d];
    sq[hh][d] = qn;
    float kn = 0.f;
    if (last && hh == 0) {
      const float kinv = 1.0f / sqrtf((sred[4] + sred[5]) / (float)D + a.eps);
      kn = (kv * kinv) * a.k_gamma[d];
      sk[d] = kn;
    }
    __syncthreads();
    const float qrot = d < 64 ? -sq[hh][d + 64] : sq[hh][d - 64];
    const float qrope = qn * c + qrot * sn;
    if (last) {
      _Float16 nv;
      if (hh == 0) {
        const float krot = d < 64 ? -sk[d + 64] : sk[d - 64];
        nv = (_Float16)(kn * c + krot * sn);
      } else {
        nv = (_Float16)kv;
      }
      const uint16_t bits = __builtin_bit_cast(uint16_t, nv);
      snew[hh][d] = bits;
      (hh == 0 ? kb : vb)[(size_t)pos * D + d] = bits;
    }
    __syncthreads();
    sq[hh][d] = qrope * qscale;
  } else {
    sq[hh][d] = a.q[((size_t)b * a.qh + h) * D + d] * qscale;
  }
  __syncthreads();
  if (a.fused && last) {
    // the appended position comes from LDS (same fp16 bits as stored)
    const int ip = pos - start - pr;
    if (ip >= 0 && (ip & 15) == 0) {
      const int i = ip >> 4;
      const u32x4 kn4 = *reinterpret_cast<const u32x4*>(&snew[0][sub * 8]);
      const u32x4 vn4 = *reinterpret_cast<const u32x4*>(&snew[1][sub * 8]);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        if (ii == i) {
          kr[ii] = kn4;
          vr[ii] = vn4;
        }
    }
  }

  // ---- scores: 8-dim partial dots reduced over the 16 lanes of a position ------
  float q0[8], q1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    q0[e] = sq[0][sub * 8 + e];
    q1[e] = sq[1][sub * 8 + e];
  }
  float sc0[4], sc1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float kf[8];
    unpack8(kr[i], kf);
    float x0 = 0.f, x1 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x0 = fmaf(q0[e], kf[e], x0);
      x1 = fmaf(q1[e], kf[e], x1);
    }
    sc0[i] = x0;
    sc1[i] = x1;
  }
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc0[i] += shfl_xor_f(sc0[i], m);
      sc1[i] += shfl_xor_f(sc1[i], m);
    }
  if (sub == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = pr + 16 * i;
      if (p < n) {
        ssc[0][p] = sc0[i];
        ssc[1][p] = sc1[i];
      }
    }
  }
  __syncthreads();

  // ---- chunk softmax (one wave per head, one lane per position) -----------------
  if (wid < 2) {
    const float sc = lane < n ? ssc[wid][lane] : -INFINITY;
    const float m = wave_max(sc);
    const float e = lane < n ? exp2f(sc - m) : 0.f;
    const float l = wave_sum(e);
    ssc[wid][lane] = e;
    if (lane == 0) {
      sml[wid][0] = m;
      sml[wid][1] = l;
    }
  }
  __syncthreads();

  // ---- P.V on the registers loaded at the start --------------------------------
  float o0[8], o1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o0[e] = o1[e] = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = pr + 16 * i;
    const float e0 = p < n ? ssc[0][p] : 0.f;
    const float e1 = p < n ? ssc[1][p] : 0.f;
    float vf[8];
    unpack8(vr[i], vf);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o0[e] = fmaf(e0, vf[e], o0[e]);
      o1[e] = fmaf(e1, vf[e], o1[e]);
    }
  }
  // lanes l, l^16, l^32, l^48 hold the same dims for different positions
#pragma unroll
  for (int m = 16; m <= 32; m <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o0[e] += shfl_xor_f(o0[e], m);
      o1[e] += shfl_xor_f(o1[e], m);
    }
  if (lane < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      spv[wid][0][sub * 8 + e] = o0[e];
      spv[wid][1][sub * 8 + e] = o1[e];
    }
  }
  __syncthreads();
  const float acc = (spv[0][hh][d] + spv[1][hh][d]) + (spv[2][hh][d] + spv[3][hh][d]);

  // ---- publish the chunk partial --------------------------------------------------
  const size_t pbase = (size_t)(b * a.qh + h) * a.nsplit_max;
  a.part_acc[(pbase + s) * D + d] = acc;
  if (d == 0) {
    a.part_ml[(pbase + s) * 2 + 0] = sml[hh][0];
    a.part_ml[(pbase + s) * 2 + 1] = sml[hh][1];
  }
}

// Merge the chunk partials of the two q heads of one kv head.
__global__ __launch_bounds__(256) void attn_merge_kernel(const AttnArgs a) {
  constexpr int D = 128;
  const int j = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int pos = a.positions[b];
  if (pos < 0 || pos >= a.max_ctx) return;  // reported by the split kernel
  const int nsplit = (pos + kAttnChunk) / kAttnChunk;
  const int hh = t >> 7, d = t & (D - 1), h = j * 2 + hh;
  const size_t pbase = (size_t)(b * a.qh + h) * a.nsplit_max;
  // single pass with a running maximum; loads of different chunks independent
  float M = -INFINITY, L = 0.f, o = 0.f;
#pragma unroll 4
  for (int i = 0; i < nsplit; ++i) {
    const float mi = a.part_ml[(pbase + i) * 2];
    const float li = a.part_ml[(pbase + i) * 2 + 1];
    const float ai = a.part_acc[(pbase + i) * D + d];
    const float Mn = fmaxf(M, mi);
    const float so = M == -INFINITY ? 0.f : exp2f(M - Mn);
    const float si = exp2f(mi - Mn);
    L = L * so + li * si;
    o = o * so + ai * si;
    M = Mn;
  }
  const float r = o / L;
  const size_t oi = ((size_t)b * a.qh + h) * D + d;
  if (a.out_dtype == Q4D_F16)
    static_cast<_Float16*>(a.out)[oi] = (_Float16)r;
  else
    static_cast<float*>(a.out)[oi] = r;
}

int launch_attention(const AttnArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(attn_split_kernel, dim3(a.nsplit_max, a.kvh, a.batch), dim3(256), 0, stream, a);
  hipLaunchKernelGGL(attn_merge_kernel, dim3(a.kvh, a.batch), dim3(256), 0, stream, a);
  return check_launch();
}

}  // namespace q4d
