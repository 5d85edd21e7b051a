// GQA decode attention over an fp16 KV cache (gfx950, wave64).
//
// Follows manual_repeat_kv + manual_cached_attention (reference
// Qwen3-0.6B-Base/python_each_module/common.py:192-228): q head h reads kv
// head h / (q_heads / kv_heads); scores = q.k * scaling; softmax in fp32;
// out = softmax . v.  The cache plane of one layer is
// [batch][kv_head][max_ctx][head_dim] fp16 so each head streams contiguously.
//
// One kernel, split-K over the context (flash-decoding style): grid
// (chunk, kv_head, batch), 256 threads per block; a block takes the two q
// heads of one kv head over CH (64 or 128) positions.
//  - Thread t owns dims 8*(t%16)..+7 of positions t/16 + 16*i (i < CH/16) for
//    both K and V and issues all its 16-byte loads first, so a chunk costs
//    one memory round trip.
//  - Waves 0/1 prepare q head 2j / 2j+1, waves 2/3 the new k / v row: lane l
//    holds dims l and l + 64, which are also each other's rotate-half
//    partner, so the per-head RMSNorm (common.py:258-262) and RoPE
//    (common.py:264-268) need no block-wide exchange.  With fused = 0 the q
//    heads arrive ready.
//  - Scores are 8-dim partial dots reduced over the 16 lanes of a position
//    (DPP); the chunk softmax runs in one wave per head (exp2, log2e folded
//    into q); P.V partials are reduced over positions through LDS.
//  - merge = 1 (64-position chunks): the chunk's (max, sum, partial output)
//    is published with device-scope atomic stores; after they complete the
//    block counts in on a per-(kv head, sequence) counter, and the block that
//    completes the count merges all chunks, reading them back with
//    device-scope atomic loads.  The counter atomic is issued only after the
//    stores are performed, so no fence (an L2 write-back on this part) and no
//    second launch is needed.
//  - merge = 0 (128-position chunks, the batch-1 decode layer): the partials
//    are plain stores and the next kernel (the o_proj GEMV) merges them in its
//    prologue, which removes the store / count / reload round trips from the
//    critical path.
// The block owning the new position appends its K/V row (append_cache,
// common.py:186-189) and takes that row from LDS rather than from its own
// global write.  Barriers that only order LDS traffic are LDS-only, so no
// wave waits for the append stores to be acknowledged.
#include <math.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

static_assert(kAttnChunk == 64 && kAttnChunkLong == 128, "thread mapping assumes 64 or 128 positions per chunk");

namespace {

// Merged head output element oi = (sequence * q heads + head) * head_dim + dim, as fp32,
// fp16, or fp16 in the tiled layout (row = sequence, column = head * head_dim + dim).
__device__ __forceinline__ void store_out(const AttnArgs& a, size_t oi, float r) {
  if (a.out_dtype == kF16Tiled) {
    const size_t w = (size_t)a.qh * a.d;
    static_cast<_Float16*>(a.out)[xt_index((int)(oi / w), (int)(oi % w))] = (_Float16)r;
  } else if (a.out_dtype == Q4D_F16) {
    static_cast<_Float16*>(a.out)[oi] = (_Float16)r;
  } else {
    static_cast<float*>(a.out)[oi] = r;
  }
}

__device__ __forceinline__ void unpack8(const u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t we = w[e];
    const h2 v = __builtin_bit_cast(h2, we);
    f[2 * e] = (float)v.x;
    f[2 * e + 1] = (float)v.y;
  }
}

// Max over each 16-lane row (every lane of the row receives it).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp_f<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  return fmaxf(v, dpp_f<kDppRowMirror>(v));
}

// Whole-wave sum / max, returned in every lane.
__device__ __forceinline__ float wave_sum_all(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_dpp(v)), 63));
}
__device__ __forceinline__ float wave_max_all(float v) {
  v = row16_max(v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Max / sum over the four 16-lane rows of a wave (every lane receives it):
// v_permlane16_swap pairs rows 0-1 and 2-3, v_permlane32_swap the two halves.
__device__ __forceinline__ float rows_max(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t a0 = a[0], a1 = a[1];
  const float s = fmaxf(__builtin_bit_cast(float, a0), __builtin_bit_cast(float, a1));
  const uint32_t w = __builtin_bit_cast(uint32_t, s);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  const uint32_t b0 = b[0], b1 = b[1];
  return fmaxf(__builtin_bit_cast(float, b0), __builtin_bit_cast(float, b1));
}
__device__ __forceinline__ float rows_sum(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t a0 = a[0], a1 = a[1];
  const float s = __builtin_bit_cast(float, a0) + __builtin_bit_cast(float, a1);
  const uint32_t w = __builtin_bit_cast(uint32_t, s);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  const uint32_t b0 = b[0], b1 = b[1];
  return __builtin_bit_cast(float, b0) + __builtin_bit_cast(float, b1);
}

__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The argument block's fields, loaded as one batch of scalar loads at kernel entry
// (left to itself the compiler interleaved the field loads with the position read
// and the control flow around it: four dependent scalar round trips before the
// first K/V load).
__device__ __forceinline__ void attn_preload(const AttnArgs& a) {
  asm volatile("" ::"s"(a.fused), "s"(a.merge), "s"(a.chunk), "s"(a.qkv), "s"(a.q), "s"(a.q_gamma),
               "s"(a.k_gamma), "s"(a.eps), "s"(a.scaling), "s"(a.rope_cos), "s"(a.rope_sin), "s"(a.kcache),
               "s"(a.vcache), "s"(a.positions), "s"(a.batch), "s"(a.qh), "s"(a.kvh), "s"(a.d), "s"(a.max_ctx),
               "s"(a.nsplit_max), "s"(a.part_ml), "s"(a.part_acc), "s"(a.counters), "s"(a.out), "s"(a.out_dtype),
               "s"(a.status));
}

// CH positions per chunk (64 or 128); thread t owns positions t/16 + 16 i, i < CH/16.
template <int CH>
__global__ __launch_bounds__(256) void attn_kernel(const AttnArgs a) {
  attn_preload(a);
  constexpr int D = 128;
  constexpr int NPT = CH / 16;  // positions per thread
  const int s = blockIdx.x, j = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, lane = t & 63;
  const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
  const int pos = a.positions[b];
  if (pos < 0 || pos >= a.max_ctx) {
    if (s == 0 && j == 0 && t == 0) atomicOr(a.status, Q4D_STATUS_BAD_POSITION);
    return;
  }
  const int T = pos + 1;
  const int nsplit = (T + CH - 1) / CH;
  if (s >= nsplit) return;
  const int start = s * CH;
  const int n = min(T, start + CH) - start;
  // positions below `cached` are read from the cache; in fused mode the new
  // position pos is produced here
  const int cached = a.fused ? pos : T;
  const bool last = (s == nsplit - 1);  // block-uniform: holds pos

  __shared__ float sq[2][D];
  __shared__ uint16_t snew[2][D];  // fp16 bits of the appended k (roped) and v
  __shared__ float ssc[2][CH];
  __shared__ float sml[2][2];
  __shared__ float spv[16][2][D];  // P.V partials per position row group
  __shared__ int s_last;

  const size_t plane_off = ((size_t)(b * a.kvh + j) * a.max_ctx) * D;
  uint16_t* kb = a.kcache + plane_off;
  uint16_t* vb = a.vcache + plane_off;

  // ---- the q / new k / new v inputs of this wave go out first ---------------
  // (vmcnt retires in issue order: issued after the K/V loads, the RMSNorm and
  // RoPE below could not start before the K/V chunk had arrived)
  // Waves 0/1 take q head 2j / 2j+1, wave 2 the new k row, wave 3 the new v
  // row; lane l holds dims l and l + 64.
  const float qscale = a.scaling * 1.4426950408889634f;  // fold log2(e) for exp2
  const int qkv_stride = (a.qh + 2 * a.kvh) * D;
  const bool qk_wave = a.fused ? (wid < 2 || (last && wid == 2)) : (wid < 2);
  const bool v_wave = a.fused && last && wid == 3;
  // Every wave loads unconditionally (pointers chosen by wave-uniform selects;
  // unused roles read valid memory): loads behind role branches make the
  // compiler wait for them at the join, before the K/V loads are issued.
  const float* row;
  const float* gam;
  const float* ctab;
  const float* stab;
  if (a.fused) {
    const float* src = a.qkv + (size_t)b * qkv_stride;
    const int ridx = wid < 2 ? j * 2 + wid : (wid == 2 ? a.qh + j : a.qh + a.kvh + j);
    row = src + (size_t)ridx * D;
    gam = wid < 2 ? a.q_gamma : a.k_gamma;
    ctab = a.rope_cos + (size_t)pos * (D / 2);
    stab = a.rope_sin + (size_t)pos * (D / 2);
  } else {
    row = a.q + ((size_t)b * a.qh + j * 2 + (wid < 2 ? wid : 1)) * D;
    gam = ctab = stab = row;
  }
  const float x0 = row[lane], x1 = row[lane + 64];
  const float g0 = gam[lane], g1 = gam[lane + 64];
  const float c = ctab[lane], sn = stab[lane];
  // keep these loads ahead of the K/V loads (vmcnt retires in issue order)
  __builtin_amdgcn_sched_barrier(0);

  // ---- then every K/V load of this chunk ------------------------------------
  const int sub = t & 15;  // dims 8*sub .. 8*sub+7
  const int pr = t >> 4;   // positions pr + 16*i
  // Rows past the cached ones are loaded from the last cached row (or row 0)
  // instead of being guarded: a guarded load makes the compiler wait for each
  // load before issuing the next.  Those positions get zero softmax weight
  // and the row holds finite cached values; position pos (fused mode) is
  // replaced from LDS below.
  u32x4 kr[NPT], vr[NPT];
  const int plast = cached > 0 ? cached - 1 : 0;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    int p = start + pr + 16 * i;
    p = p < cached ? p : plast;
    kr[i] = *reinterpret_cast<const u32x4*>(kb + (size_t)p * D + sub * 8);
    vr[i] = *reinterpret_cast<const u32x4*>(vb + (size_t)p * D + sub * 8);
  }

  // ---- per-head RMSNorm (common.py:258-262) + rotate-half RoPE (264-268) -------
  if (a.fused && qk_wave) {
    const float ss = wave_sum_all(fmaf(x0, x0, x1 * x1));
    const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
    const float n0 = (x0 * inv) * g0, n1 = (x1 * inv) * g1;
    // rotate_half: dim d < 64 takes -x[d + 64], dim d >= 64 takes x[d - 64]
    const float r0 = n0 * c + (-n1) * sn;
    const float r1 = n1 * c + n0 * sn;
    if (wid < 2) {
      sq[wid][lane] = r0 * qscale;
      sq[wid][lane + 64] = r1 * qscale;
    } else {
      const uint16_t b0 = __builtin_bit_cast(uint16_t, (_Float16)r0);
      const uint16_t b1 = __builtin_bit_cast(uint16_t, (_Float16)r1);
      snew[0][lane] = b0;
      snew[0][lane + 64] = b1;
      kb[(size_t)pos * D + lane] = b0;
      kb[(size_t)pos * D + lane + 64] = b1;
    }
  } else if (v_wave) {
    const uint16_t b0 = __builtin_bit_cast(uint16_t, (_Float16)x0);
    const uint16_t b1 = __builtin_bit_cast(uint16_t, (_Float16)x1);
    snew[1][lane] = b0;
    snew[1][lane + 64] = b1;
    vb[(size_t)pos * D + lane] = b0;
    vb[(size_t)pos * D + lane + 64] = b1;
  } else if (qk_wave) {
    sq[wid][lane] = x0 * qscale;
    sq[wid][lane + 64] = x1 * qscale;
  }
  block_sync_lds();
  if (a.fused && last) {
    // the appended position comes from LDS (same fp16 bits as stored)
    const int ip = pos - start - pr;
    if (ip >= 0 && (ip & 15) == 0) {
      const int i = ip >> 4;
      const u32x4 kn4 = *reinterpret_cast<const u32x4*>(&snew[0][sub * 8]);
      const u32x4 vn4 = *reinterpret_cast<const u32x4*>(&snew[1][sub * 8]);
#pragma unroll
      for (int ii = 0; ii < NPT; ++ii)
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
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    float kf[8];
    unpack8(kr[i], kf);
    float x0 = 0.f, x1 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x0 = fmaf(q0[e], kf[e], x0);
      x1 = fmaf(q1[e], kf[e], x1);
    }
    x0 = row16_sum(x0);
    x1 = row16_sum(x1);
    const int p = pr + 16 * i;
    if (sub == 0 && p < n) {
      ssc[0][p] = x0;
      ssc[1][p] = x1;
    }
  }
  block_sync_lds();

  // ---- chunk softmax (one wave per head, one lane per position) -----------------
  if (wid < 2) {
    float sc[CH / 64];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < CH / 64; ++k) {
      const int p = lane + 64 * k;
      sc[k] = p < n ? ssc[wid][p] : -INFINITY;
      mx = fmaxf(mx, sc[k]);
    }
    const float m = wave_max_all(mx);
    float es = 0.f;
#pragma unroll
    for (int k = 0; k < CH / 64; ++k) {
      const int p = lane + 64 * k;
      const float e = p < n ? exp2f(sc[k] - m) : 0.f;
      ssc[wid][p] = e;
      es += e;
    }
    const float l = wave_sum_all(es);
    if (lane == 0) {
      sml[wid][0] = m;
      sml[wid][1] = l;
    }
  }
  block_sync_lds();

  // ---- P.V on the registers loaded at the start --------------------------------
  float o0[8], o1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o0[e] = o1[e] = 0.f;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int p = pr + 16 * i;
    const float e0 = p < n ? ssc[0][p] : 0.f;
    const float e1 = p < n ? ssc[1][p] : 0.f;
    // rows past the chunk stand in for absent positions: zero them rather than weight an
    // Inf or NaN bit pattern of a row not yet written by 0
    const u32x4 vq = p < n ? vr[i] : u32x4{0u, 0u, 0u, 0u};
    float vf[8];
    unpack8(vq, vf);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o0[e] = fmaf(e0, vf[e], o0[e]);
      o1[e] = fmaf(e1, vf[e], o1[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; e += 4) {
    *reinterpret_cast<f32x4*>(&spv[pr][0][sub * 8 + e]) = f32x4{o0[e], o0[e + 1], o0[e + 2], o0[e + 3]};
    *reinterpret_cast<f32x4*>(&spv[pr][1][sub * 8 + e]) = f32x4{o1[e], o1[e + 1], o1[e + 2], o1[e + 3]};
  }
  block_sync_lds();
  const int hh = t >> 7, d = t & (D - 1), h = j * 2 + hh;
  float acc = 0.f;
#pragma unroll
  for (int g = 0; g < 16; ++g) acc += spv[g][hh][d];

  // ---- publish the chunk partial, count in; the last block merges ---------------
  const size_t pbase = (size_t)(b * a.qh + h) * a.nsplit_max;
  if (!a.merge) {
    // partials for the consumer; the kernel boundary makes them visible
    a.part_acc[(pbase + s) * D + d] = acc;
    if (d == 0) {
      a.part_ml[(pbase + s) * 2 + 0] = sml[hh][0];
      a.part_ml[(pbase + s) * 2 + 1] = sml[hh][1];
    }
    return;
  }
  if (nsplit == 1) {
    const float r = acc / sml[hh][1];
    const size_t oi = ((size_t)b * a.qh + h) * D + d;
    store_out(a, oi, r);
    return;
  }
  store_dev(&a.part_acc[(pbase + s) * D + d], acc);
  if (d == 0) {
    store_dev(&a.part_ml[(pbase + s) * 2 + 0], sml[hh][0]);
    store_dev(&a.part_ml[(pbase + s) * 2 + 1], sml[hh][1]);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are performed
  __syncthreads();                 // ... and every other thread's
  int* counter = a.counters + b * a.kvh + j;
  if (t == 0) s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
  __syncthreads();
  if (!s_last) return;

  // running maximum over the chunk partials; the device-scope loads of up to
  // kMergeBatch chunks are issued together (atomic loads are not reordered,
  // so a load-then-use loop would pay one memory round trip per chunk)
  constexpr int kMergeBatch = 8;
  float M = -INFINITY, L = 0.f, o = 0.f;
  for (int i0 = 0; i0 < nsplit; i0 += kMergeBatch) {
    float mi[kMergeBatch], li[kMergeBatch], ai[kMergeBatch];
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const int i = min(i0 + k, nsplit - 1);
      mi[k] = load_dev(&a.part_ml[(pbase + i) * 2]);
      li[k] = load_dev(&a.part_ml[(pbase + i) * 2 + 1]);
      ai[k] = load_dev(&a.part_acc[(pbase + i) * D + d]);
    }
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      if (i0 + k >= nsplit) break;
      const float Mn = fmaxf(M, mi[k]);
      const float so = M == -INFINITY ? 0.f : exp2f(M - Mn);
      const float si = exp2f(mi[k] - Mn);
      L = L * so + li[k] * si;
      o = o * so + ai[k] * si;
      M = Mn;
    }
  }
  const float r = o / L;
  const size_t oi = ((size_t)b * a.qh + h) * D + d;
  store_out(a, oi, r);
  if (t == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
}

// Long-context variant of attn_kernel<64> with merge = 1 (batched decode,
// q4d_cached_attention): a block covers one of nsplit nearly equal parts of the
// T = pos + 1 positions (nsplit = ceil(T / span), parts of whole 64-position
// sub-chunks) as consecutive sub-chunks, with the next sub-chunk's K/V loads
// in flight while the current one is used.  Each wave keeps its own online
// softmax (running maximum M and sum L per head; its output accumulators are
// rescaled by 2^(M_old - M_new) when M grows) over its 16 positions of every
// sub-chunk, so the sub-chunk loop has no barrier; the four waves' states are
// merged once after the span.  K/V are read with non-temporal loads (read once
// per step).  The launcher sizes `span` for about two blocks per CU over the
// batch's (sequence, kv head) pairs: a few long contiguous K/V streams per CU
// read HBM faster than many short ones (64 x 4097 positions, 28 layers: eight
// 576-position spans per head, 5 resident blocks per CU and 32-position
// sub-chunks took 6.35 ms per step; equal parts 6.27; one block per head with
// 64-position sub-chunks 5.48).  Same prologue and partial format as
// attn_kernel<64>; thread t owns dims 8 (t % 16) .. +7 of positions t / 16 + 16 i.
__global__ __launch_bounds__(256) void attn_span_kernel(const AttnArgs a, int span) {
  attn_preload(a);
  constexpr int D = 128, CH = 64, NPT = CH / 16;
  const int s = blockIdx.x, j = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, lane = t & 63;
  const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
  const int pos = a.positions[b];
  if (pos < 0 || pos >= a.max_ctx) {
    if (s == 0 && j == 0 && t == 0) atomicOr(a.status, Q4D_STATUS_BAD_POSITION);
    return;
  }
  const int T = pos + 1;
  const int nsplit = (T + span - 1) / span;
  if (s >= nsplit) return;
  const int nsub_all = (T + CH - 1) / CH;
  const int start = (s * nsub_all / nsplit) * CH;
  const int end = min(T, ((s + 1) * nsub_all / nsplit) * CH);
  const int nsub = (end - start + CH - 1) / CH;
  const int cached = a.fused ? pos : T;
  const bool last = (s == nsplit - 1);  // block-uniform: holds pos

  __shared__ float sq[2][D];
  __shared__ uint16_t snew[2][D];
  __shared__ float swml[4][2][2];  // each wave's (M, L) per head after the span
  __shared__ float spv[16][2][D];
  __shared__ int s_last;

  const size_t plane_off = ((size_t)(b * a.kvh + j) * a.max_ctx) * D;
  uint16_t* kb = a.kcache + plane_off;
  uint16_t* vb = a.vcache + plane_off;

  // ---- q / new k / new v rows first (as attn_kernel) ----------------------------
  const float qscale = a.scaling * 1.4426950408889634f;
  const int qkv_stride = (a.qh + 2 * a.kvh) * D;
  const bool qk_wave = a.fused ? (wid < 2 || (last && wid == 2)) : (wid < 2);
  const bool v_wave = a.fused && last && wid == 3;
  const float* row;
  const float* gam;
  const float* ctab;
  const float* stab;
  if (a.fused) {
    const float* src = a.qkv + (size_t)b * qkv_stride;
    const int ridx = wid < 2 ? j * 2 + wid : (wid == 2 ? a.qh + j : a.qh + a.kvh + j);
    row = src + (size_t)ridx * D;
    gam = wid < 2 ? a.q_gamma : a.k_gamma;
    ctab = a.rope_cos + (size_t)pos * (D / 2);
    stab = a.rope_sin + (size_t)pos * (D / 2);
  } else {
    row = a.q + ((size_t)b * a.qh + j * 2 + (wid < 2 ? wid : 1)) * D;
    gam = ctab = stab = row;
  }
  const float x0 = row[lane], x1 = row[lane + 64];
  const float g0 = gam[lane], g1 = gam[lane + 64];
  const float c = ctab[lane], sn = stab[lane];
  __builtin_amdgcn_sched_barrier(0);

  // ---- K/V of sub-chunk 0 (rows at or past `cached` read the last cached row:
  // unconditional loads, zero softmax weight; position pos comes from LDS)
  const int sub = t & 15, pr = t >> 4;
  const int plast = cached > 0 ? cached - 1 : 0;
  u32x4 kr[NPT], vr[NPT], kn[NPT], vn[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    int p = start + pr + 16 * i;
    p = p < cached ? p : plast;
    kr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kb + (size_t)p * D + sub * 8));
    vr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vb + (size_t)p * D + sub * 8));
  }

  // ---- per-head RMSNorm (common.py:258-262) + rotate-half RoPE (264-268) -------
  if (a.fused && qk_wave) {
    const float ss = wave_sum_all(fmaf(x0, x0, x1 * x1));
    const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
    const float n0 = (x0 * inv) * g0, n1 = (x1 * inv) * g1;
    const float r0 = n0 * c + (-n1) * sn;
    const float r1 = n1 * c + n0 * sn;
    if (wid < 2) {
      sq[wid][lane] = r0 * qscale;
      sq[wid][lane + 64] = r1 * qscale;
    } else {
      const uint16_t b0 = __builtin_bit_cast(uint16_t, (_Float16)r0);
      const uint16_t b1 = __builtin_bit_cast(uint16_t, (_Float16)r1);
      snew[0][lane] = b0;
      snew[0][lane + 64] = b1;
      kb[(size_t)pos * D + lane] = b0;
      kb[(size_t)pos * D + lane + 64] = b1;
    }
  } else if (v_wave) {
    const uint16_t b0 = __builtin_bit_cast(uint16_t, (_Float16)x0);
    const uint16_t b1 = __builtin_bit_cast(uint16_t, (_Float16)x1);
    snew[1][lane] = b0;
    snew[1][lane + 64] = b1;
    vb[(size_t)pos * D + lane] = b0;
    vb[(size_t)pos * D + lane + 64] = b1;
  } else if (qk_wave) {
    sq[wid][lane] = x0 * qscale;
    sq[wid][lane + 64] = x1 * qscale;
  }
  block_sync_lds();
  float q0[8], q1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    q0[e] = sq[0][sub * 8 + e];
    q1[e] = sq[1][sub * 8 + e];
  }

  float o0[8], o1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o0[e] = o1[e] = 0.f;
  // each wave runs its own online softmax over its 16 positions of every sub-chunk
  // (running maximum M and sum L per head), so the sub-chunk loop has no barrier;
  // the four waves' states merge once after the span
  float M0 = -INFINITY, L0 = 0.f, M1 = -INFINITY, L1 = 0.f;
  for (int sc = 0; sc < nsub; ++sc) {
    const int base = start + sc * CH;
    const int n = min(end - base, CH);
    // the next sub-chunk's K/V go out now (the last iteration re-reads its
    // own rows: unconditional loads keep the compiler from waiting on them)
    const int nb = sc + 1 < nsub ? base + CH : base;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      int p = nb + pr + 16 * i;
      p = p < cached ? p : plast;
      kn[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kb + (size_t)p * D + sub * 8));
      vn[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vb + (size_t)p * D + sub * 8));
    }
    if (a.fused && last) {
      const int ip = pos - base - pr;
      if (ip >= 0 && ip < CH && (ip & 15) == 0) {
        const int i = ip >> 4;
        const u32x4 kn4 = *reinterpret_cast<const u32x4*>(&snew[0][sub * 8]);
        const u32x4 vn4 = *reinterpret_cast<const u32x4*>(&snew[1][sub * 8]);
#pragma unroll
        for (int ii = 0; ii < NPT; ++ii)
          if (ii == i) {
            kr[ii] = kn4;
            vr[ii] = vn4;
          }
      }
    }
    // scores: 8-dim partial dots reduced over the 16 lanes of a position
    float y0[NPT], y1[NPT];
    float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      float kf[8];
      unpack8(kr[i], kf);
      float u0 = 0.f, u1 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u0 = fmaf(q0[e], kf[e], u0);
        u1 = fmaf(q1[e], kf[e], u1);
      }
      u0 = row16_sum(u0);
      u1 = row16_sum(u1);
      const bool ok = pr + 16 * i < n;
      y0[i] = ok ? u0 : -INFINITY;
      y1[i] = ok ? u1 : -INFINITY;
      m0 = fmaxf(m0, y0[i]);
      m1 = fmaxf(m1, y1[i]);
    }
    m0 = rows_max(m0);
    m1 = rows_max(m1);
    const float Mn0 = fmaxf(M0, m0), Mn1 = fmaxf(M1, m1);
    float e0[NPT], e1[NPT], s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const bool ok = pr + 16 * i < n;
      e0[i] = ok ? exp2f(y0[i] - Mn0) : 0.f;
      e1[i] = ok ? exp2f(y1[i] - Mn1) : 0.f;
      s0 += e0[i];
      s1 += e1[i];
    }
    s0 = rows_sum(s0);
    s1 = rows_sum(s1);
    const float sc0 = M0 == -INFINITY ? 0.f : exp2f(M0 - Mn0);
    const float sc1 = M1 == -INFINITY ? 0.f : exp2f(M1 - Mn1);
    L0 = fmaf(L0, sc0, s0);
    L1 = fmaf(L1, sc1, s1);
    M0 = Mn0;
    M1 = Mn1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o0[e] *= sc0;
      o1[e] *= sc1;
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int p = pr + 16 * i;
      const u32x4 vq = p < n ? vr[i] : u32x4{0u, 0u, 0u, 0u};  // as in attn_kernel
      float vf[8];
      unpack8(vq, vf);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o0[e] = fmaf(e0[i], vf[e], o0[e]);
        o1[e] = fmaf(e1[i], vf[e], o1[e]);
      }
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      kr[i] = kn[i];
      vr[i] = vn[i];
    }
  }
  if (lane == 0) {
    swml[wid][0][0] = M0;
    swml[wid][0][1] = L0;
    swml[wid][1][0] = M1;
    swml[wid][1][1] = L1;
  }
#pragma unroll
  for (int e = 0; e < 8; e += 4) {
    *reinterpret_cast<f32x4*>(&spv[pr][0][sub * 8 + e]) = f32x4{o0[e], o0[e + 1], o0[e + 2], o0[e + 3]};
    *reinterpret_cast<f32x4*>(&spv[pr][1][sub * 8 + e]) = f32x4{o1[e], o1[e + 1], o1[e + 2], o1[e + 3]};
  }
  block_sync_lds();
  const int hh = t >> 7, d = t & (D - 1), h = j * 2 + hh;
  float Mb = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) Mb = fmaxf(Mb, swml[w][hh][0]);
  float acc = 0.f, Lb = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float mw = swml[w][hh][0];
    const float sw = mw == -INFINITY ? 0.f : exp2f(mw - Mb);
    Lb = fmaf(swml[w][hh][1], sw, Lb);
    float part = 0.f;
#pragma unroll
    for (int g = 4 * w; g < 4 * w + 4; ++g) part += spv[g][hh][d];
    acc = fmaf(part, sw, acc);
  }

  // ---- publish the split partial, count in; the last block merges (as attn_kernel)
  const size_t pbase = (size_t)(b * a.qh + h) * a.nsplit_max;
  if (nsplit == 1) {
    const float r = acc / Lb;
    const size_t oi = ((size_t)b * a.qh + h) * D + d;
    store_out(a, oi, r);
    return;
  }
  store_dev(&a.part_acc[(pbase + s) * D + d], acc);
  if (d == 0) {
    store_dev(&a.part_ml[(pbase + s) * 2 + 0], Mb);
    store_dev(&a.part_ml[(pbase + s) * 2 + 1], Lb);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are performed
  __syncthreads();                 // ... and every other thread's
  int* counter = a.counters + b * a.kvh + j;
  if (t == 0) s_last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
  __syncthreads();
  if (!s_last) return;
  constexpr int kMergeBatch = 8;
  float Mx = -INFINITY, Lx = 0.f, o = 0.f;
  for (int i0 = 0; i0 < nsplit; i0 += kMergeBatch) {
    float mi[kMergeBatch], li[kMergeBatch], ai[kMergeBatch];
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const int i = min(i0 + k, nsplit - 1);
      mi[k] = load_dev(&a.part_ml[(pbase + i) * 2]);
      li[k] = load_dev(&a.part_ml[(pbase + i) * 2 + 1]);
      ai[k] = load_dev(&a.part_acc[(pbase + i) * D + d]);
    }
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      if (i0 + k >= nsplit) break;
      const float Mn = fmaxf(Mx, mi[k]);
      const float so = Mx == -INFINITY ? 0.f : exp2f(Mx - Mn);
      const float si = exp2f(mi[k] - Mn);
      Lx = Lx * so + li[k] * si;
      o = o * so + ai[k] * si;
      Mx = Mn;
    }
  }
  const float r = o / Lx;
  const size_t oi = ((size_t)b * a.qh + h) * D + d;
  store_out(a, oi, r);
  if (t == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
}

}  // namespace

int launch_attention(const AttnArgs& a, hipStream_t stream) {
  if (!a.part_ml || !a.part_acc || (a.merge && !a.counters)) return Q4D_ERR_NULL;
  if (a.merge) {
    // contexts past kSpanSplits x 64 positions: spans of several 64-position
    // sub-chunks, at most kSpanSplits per head, as many as make about two blocks
    // per CU over the (sequence, kv head) pairs
    constexpr int kSpanSplits = 8;
    const int nch = (a.max_ctx + kAttnChunk - 1) / kAttnChunk;
    if (nch <= kSpanSplits) {
      hipLaunchKernelGGL(attn_kernel<kAttnChunk>, dim3(a.nsplit_max, a.kvh, a.batch), dim3(256), 0, stream, a);
    } else {
      const int pairs = a.batch * a.kvh;
      const int ns = max(1, min(kSpanSplits, (2 * device_cus() + pairs - 1) / pairs));
      const int span = kAttnChunk * ((nch + ns - 1) / ns);
      const int nsplit = (a.max_ctx + span - 1) / span;
      hipLaunchKernelGGL(attn_span_kernel, dim3(nsplit, a.kvh, a.batch), dim3(256), 0, stream, a, span);
    }
  } else if (a.chunk == kAttnChunk) {
    const int ns = (a.max_ctx + kAttnChunk - 1) / kAttnChunk;
    hipLaunchKernelGGL(attn_kernel<kAttnChunk>, dim3(ns, a.kvh, a.batch), dim3(256), 0, stream, a);
  } else {
    const int ns = (a.max_ctx + kAttnChunkLong - 1) / kAttnChunkLong;
    hipLaunchKernelGGL(attn_kernel<kAttnChunkLong>, dim3(ns, a.kvh, a.batch), dim3(256), 0, stream, a);
  }
  return check_launch();
}

}  // namespace q4d
