// Batch-1 decode layer in two launches, split over MI355X's eight XCDs (gfx950, wave64).
//
// Same arithmetic as manual_decoder_layer_cached (reference
// Qwen3-0.6B-Base/python_each_module/common.py:231-298) for the Qwen3-0.6B shape
// (hidden 1024, 16 q heads, 8 kv heads, head_dim 128, intermediate 3072).
//
// The five-launch layer of q4d_gemv.hip / q4d_attention.hip pays a dependent kernel
// boundary (completion, L2 write-back, dispatch, argument loads: ~1.6 us) at each of
// its five stages.  Here each XCD owns one kv head, the way tensor parallelism splits
// a layer over devices:
//   launch A: x = layer input -> input RMSNorm -> the XCD's 512 q|k|v rows (its two q
//             heads, its k and v heads) -> q/k RMSNorm, RoPE, K/V append -> GQA
//             attention over the context, split among the XCD's 32 blocks -> chunk
//             merge -> o_proj over the XCD's 256 input columns: a split-K partial of
//             all 1024 outputs, po[xcd].
//   launch B: x' = x + sum of the 8 o_proj partials -> post-attention RMSNorm -> the
//             XCD's 384 gate and 384 up rows -> SwiGLU -> down over the XCD's 384 input
//             columns: a split-K partial, pd[xcd].
// The next layer's launch A (after the last layer: the LM head's prologue in a
// one-token step, xcd_finalize for a single layer call) forms
// x'' = x' + sum of the 8 down partials, summed in XCD order so every XCD gets the
// same bits.
//
// Inside a launch, the 32 workgroups of one XCD exchange data through that XCD's L2:
// plain stores, then one flag word per workgroup (a plain store after the data stores
// are acknowledged), polled with agent-scope (sc1) loads, which read the line the
// stores left in the L2 (0.45 us for a 32-workgroup exchange on MI355X, against
// ~1.6 us for a kernel boundary).  Data crosses XCDs only at launch boundaries.
// Dispatch deals workgroups to the XCDs round-robin, so workgroups b, b + 8, ... share
// one XCD (which one can rotate from launch to launch); each flag carries the XCC_ID
// hardware register of its writer, and a group found on more than one XCD is
// reported as Q4D_STATUS_XCD_MAP.  Every wait is bounded (20 ms of the 100 MHz
// real-time clock) and reports Q4D_STATUS_SYNC_TIMEOUT instead of hanging.  The 32 workgroups of an
// XCD fit on its 32 CUs together, so all of them are resident while they wait.
//
// Flags count exchanges: at kernel entry every workgroup of an XCD reads the same
// count e0 (all of them made the same number of exchanges before), and exchange k
// publishes e0 + k.  q4d_workspace_init zeroes them.
//
// Each workgroup has four compute waves and one exchange wave.  The compute waves
// issue every weight and K/V load of the launch at entry and consume the exchanged
// data from LDS; the exchange wave (no weight loads in flight) does the stores, the
// flag traffic and the loads of exchanged data, so a wait never queues behind
// weight loads (vector loads retire in issue order).
#include <math.h>

#include <mutex>

#include "q4d_device.h"
#include "q4d_gemv_dev.h"
#include "q4d_internal.h"

namespace q4d {

namespace {

constexpr int kXThreads = 320;   // four compute waves + the exchange wave
constexpr int kH = 1024, kD = 128;
constexpr int kGI = kXcdInter / kXcdGroups;  // 384 intermediate dims per XCD
constexpr unsigned long long kSpinTicks = 2000000ull;  // 20 ms of s_memrealtime (100 MHz)

static_assert(kXcdGroups == 8 && kXcdBlocks == 32, "one kv head per XCD, 32 workgroups per XCD");

__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xfu;
}

__device__ __forceinline__ uint32_t ld_sc1_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte agent-scope (sc1) load at byte offset `off` of a buffer resource.
__device__ __forceinline__ f32x4 ld_sc1_v4(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));
}

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// Flag words hold (exchange count << 4) | XCC id of the writer.  Exchange wave only:
// publish arrival number `cnt` of workgroup j and wait for the XCD's 32 workgroups
// (count compared modulo 2^28); the data stores this wave made before are
// acknowledged first.  A flag written from another XCD than this one means the
// dispatch did not keep the group on one XCD (reported; its exchanges then time out).
__device__ __forceinline__ void xcd_arrive_wait(uint32_t* f, int j, uint32_t cnt, uint32_t xcc, int lane,
                                                int32_t* status) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const uint32_t word = (cnt << 4) | xcc;
  if (lane == 0) asm volatile("global_store_dword %0, %1, off" ::"v"(f + j), "v"(word) : "memory");
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  while (true) {
    const uint32_t v = lane < kXcdBlocks ? ld_sc1_u32(f + lane) : word;
    const bool arrived = (int)(((v >> 4) - cnt) << 4) >= 0;
    if (__all(arrived)) {
      if (__any((v & 0xfu) != xcc) && lane == 0) atomicOr(status, Q4D_STATUS_XCD_MAP);
      break;
    }
    if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) {
      if (lane == 0) atomicOr(status, Q4D_STATUS_SYNC_TIMEOUT);
      break;
    }
  }
}

// x[e..e+3] = base + p[0] + p[1] + ... + p[7] (this summation order everywhere).
__device__ __forceinline__ f32x4 sum_partials(const float* base, const float* parts, int e) {
  f32x4 v = ld4(base + e);
  f32x4 p[kXcdGroups];
#pragma unroll
  for (int g = 0; g < kXcdGroups; ++g) p[g] = ld4(parts + g * kH + e);
#pragma unroll
  for (int g = 0; g < kXcdGroups; ++g) v = v + p[g];
  return v;
}

__device__ __forceinline__ void prep_vals(float (&v)[4], int q, uint32_t* ph, uint32_t* pl, float2* sm);

// fp16 hi/lo pairs in dequant order (see act_prepare in q4d_gemv_dev.h) for work
// item q (< K / 4) of a K-vector in LDS: chunk c = q / 8 holds columns 32c..32c+31,
// and the 8 items of a chunk are 8 consecutive lanes, which sum the chunk.
// v = (x * inv) * gamma when gamma is given, else x.
__device__ __forceinline__ void prep_item(const float* sx, int q, bool norm, float inv, const f32x4 g4, uint32_t* ph,
                                          uint32_t* pl, float2* sm) {
  const int c = q >> 3, m = (q & 7) >> 1, i0 = (q & 1) * 2;
  const int ea = c * 32 + m * 8 + i0, eb = ea + 4;
  float v[4] = {sx[ea], sx[eb], sx[ea + 1], sx[eb + 1]};
  if (norm) {
    v[0] = (v[0] * inv) * g4[0];
    v[1] = (v[1] * inv) * g4[1];
    v[2] = (v[2] * inv) * g4[2];
    v[3] = (v[3] * inv) * g4[3];
  }
  prep_vals(v, q, ph, pl, sm);
}

// The conversion of prep_item for the values v = {x[ea], x[eb], x[ea + 1], x[eb + 1]}
// of work item q.
__device__ __forceinline__ void prep_vals(float (&v)[4], int q, uint32_t* ph, uint32_t* pl, float2* sm) {
  const int c = q >> 3, m = (q & 7) >> 1, i0 = (q & 1) * 2;
  _Float16 h[4], l[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    asm("" : "+v"(v[k]));  // one rounded fp32 value feeds hi, lo and the sums
    h[k] = (_Float16)v[k];
    l[k] = (_Float16)(v[k] - (float)h[k]);
  }
  float sh = ((float)h[0] + (float)h[1]) + ((float)h[2] + (float)h[3]);
  float sl = ((float)l[0] + (float)l[1]) + ((float)l[2] + (float)l[3]);
  *reinterpret_cast<u32x2*>(&ph[c * 16 + m * 4 + i0]) = u32x2{pack_h2(h[0], h[1]), pack_h2(h[2], h[3])};
  *reinterpret_cast<u32x2*>(&pl[c * 16 + m * 4 + i0]) = u32x2{pack_h2(l[0], l[1]), pack_h2(l[2], l[3])};
  sh += dpp_f<kDppQuadSwap1>(sh);
  sh += dpp_f<kDppQuadSwap2>(sh);
  sh += dpp_f<kDppRowHalfMirror>(sh);
  sl += dpp_f<kDppQuadSwap1>(sl);
  sl += dpp_f<kDppQuadSwap2>(sl);
  sl += dpp_f<kDppRowHalfMirror>(sl);
  if ((q & 7) == 0) sm[c] = make_float2(8.f * sh, 8.f * sl);
}

// The gamma values prep_item(q) multiplies by.
__device__ __forceinline__ f32x4 prep_gamma(const float* gamma, int q) {
  const int c = q >> 3, m = (q & 7) >> 1, i0 = (q & 1) * 2;
  const int ea = c * 32 + m * 8 + i0, eb = ea + 4;
  return f32x4{gamma[ea], gamma[eb], gamma[ea + 1], gamma[eb + 1]};
}

__device__ __forceinline__ void load_chunk(const uint32_t* ph, const uint32_t* pl, const float2* sm, int c, XChunk& xh,
                                           XChunk& xl) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x4 a = reinterpret_cast<const u32x4*>(&ph[c * 16])[k];
    const u32x4 b = reinterpret_cast<const u32x4*>(&pl[c * 16])[k];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xh.p[4 * k + e] = __builtin_bit_cast(h2, (uint32_t)a[e]);
      xl.p[4 * k + e] = __builtin_bit_cast(h2, (uint32_t)b[e]);
    }
  }
  const float2 s = sm[c];
  xh.sum8 = s.x;
  xl.sum8 = s.y;
}

// 16 bytes of codes and the 32-bit word holding the Q2.14 scale of u16 index sidx.
struct WChunk {
  u32x4 w;
  uint32_t s;
  int sh;
};
__device__ __forceinline__ WChunk load_w(const uint8_t* w, size_t woff, const uint16_t* s, size_t sidx) {
  WChunk r;
  // codes as non-temporal loads, read once per step (one layer at ctx 512 from HBM:
  // 15.38 -> 14.84 us); the scale words stay ordinary loads: workgroups of an XCD
  // share their lines, and as non-temporal loads the layer took 15.66 us
  r.w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w + woff));
  r.s = *reinterpret_cast<const uint32_t*>(s + (sidx & ~(size_t)1));
  r.sh = (int)(sidx & 1) * 16;
  return r;
}
__device__ __forceinline__ float wdot(const WChunk& c, const XChunk& xh, const XChunk& xl) {
  return chunk_dot_hl(c.w, xh, xl) * scale_q2_14((c.s >> c.sh) & 0xFFFFu);
}

__device__ __forceinline__ float row16_max_f(float v) {
  v = fmaxf(v, dpp_f<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp_f<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  return fmaxf(v, dpp_f<kDppRowMirror>(v));
}
__device__ __forceinline__ float wave_max_bcast(float v) {
  v = row16_max_f(v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ void unpack8h(const u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const h2 v = __builtin_bit_cast(h2, (uint32_t)w[e]);
    f[2 * e] = (float)v.x;
    f[2 * e + 1] = (float)v.y;
  }
}

// Attention chunking for context T = pos + 1: nA = min(32, ceil(T / 16)) workgroups
// of ceil(T / nA) positions (at most 16 while T <= 512).
// Group-loop instances (groups of 16 positions per chunk) from which a chunk of more than
// one group is scored by four waves (even / odd groups) instead of two.
constexpr int kXcdSplitMinGroups = 4;

__device__ __forceinline__ void attn_split(int T, int& nA, int& chunk) {
  nA = min(kXcdBlocks, (T + 15) / 16);
  chunk = (T + nA - 1) / nA;
}

// Max / sum over each 32-lane half, in every lane of the half.
__device__ __forceinline__ float half_max(float v) {
  v = row16_max_f(v);
  const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float l1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float h1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (threadIdx.x & 32) ? fmaxf(hi, h1) : fmaxf(lo, l1);
}
__device__ __forceinline__ float half_sum(float v) {
  v = row16_sum(v);
  const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float l1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float h1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (threadIdx.x & 32) ? hi + h1 : lo + l1;
}

// The layer input x[4t .. 4t+3] for compute thread t: the loads (issued first) and the value.
struct XIn {
  f32x4 v[1 + kXcdGroups];
  uint32_t codes, scode;
};
__device__ __forceinline__ void xin_issue(int mode, const float* base, const float* parts, const float* hin,
                                          const int32_t* emb_token, const uint8_t* emb_w, const uint16_t* emb_s,
                                          int emb_vocab, int e, XIn& r, bool& ok) {
  ok = true;
  if (mode == 0) {
    r.v[0] = ld4(base + e);
#pragma unroll
    for (int g = 0; g < kXcdGroups; ++g) r.v[1 + g] = ld4(parts + g * kH + e);
  } else if (mode == 1) {
    r.v[0] = ld4(hin + e);
  } else {
    const int tok = emb_token[0];
    ok = tok >= 0 && tok < emb_vocab;
    const size_t row = ok ? (size_t)tok : 0;
    r.codes = *reinterpret_cast<const uint16_t*>(emb_w + row * (kH / 2) + e / 2);
    r.scode = emb_s[row * (kH / 64) + e / 64];
  }
}
__device__ __forceinline__ f32x4 xin_value(int mode, const XIn& r, bool ok) {
  if (mode == 0) {
    f32x4 v = r.v[0];
#pragma unroll
    for (int g = 0; g < kXcdGroups; ++g) v = v + r.v[1 + g];  // the order of sum_partials
    return v;
  }
  if (mode == 1) return r.v[0];
  // the embedding row, q * scale exactly as the embedding kernel computes it
  f32x4 v;
  const float sc = scale_q2_14(r.scode);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int nib = (int)((r.codes >> (4 * k)) & 0xFu);
    v[k] = ok ? (float)(nib - ((nib & 0x8) ? 16 : 0)) * sc : 0.0f;
  }
  return v;
}

// The argument blocks' fields, loaded as one batch of scalar loads at kernel entry
// (left to itself the compiler loads fields where the control flow first needs them:
// the argument pointer of the position, the position, then the rest, three dependent
// scalar round trips before the first load of the layer input).
__device__ __forceinline__ void xcd_bufs_preload(const XcdBufs& x) {
  asm volatile("" ::"s"(x.flags), "s"(x.qkv), "s"(x.ap), "s"(x.ac), "s"(x.po), "s"(x.pd), "s"(x.hx), "s"(x.hx2),
               "s"(x.status));
}
__device__ __forceinline__ void xcd_attn_preload(const XcdAttnArgs& a) {
  asm volatile("" ::"s"(a.qw), "s"(a.kw), "s"(a.vw), "s"(a.ow), "s"(a.qs), "s"(a.ks), "s"(a.vs), "s"(a.os),
               "s"(a.in_gamma), "s"(a.q_gamma), "s"(a.k_gamma), "s"(a.eps), "s"(a.qscale), "s"(a.rope_cos),
               "s"(a.rope_sin), "s"(a.kcache), "s"(a.vcache), "s"(a.positions), "s"(a.max_ctx), "s"(a.in_mode),
               "s"(a.hin), "s"(a.emb_token), "s"(a.emb_w), "s"(a.emb_s), "s"(a.emb_vocab));
  xcd_bufs_preload(a.x);
}
__device__ __forceinline__ void xcd_mlp_preload(const XcdMlpArgs& a) {
  asm volatile("" ::"s"(a.gw), "s"(a.uw), "s"(a.dw), "s"(a.gs), "s"(a.us), "s"(a.ds), "s"(a.post_gamma),
               "s"(a.eps));
  xcd_bufs_preload(a.x);
}

// ---------------------------------------------------------------------------
// Launch A: input, q|k|v, attention, o_proj partial.  NPT = 16-position groups of a
// workgroup's chunk (chunk <= 16 * NPT); MODE = the input mode (XcdAttnArgs::in_mode),
// a template parameter so that every compute wave issues the same loads in the same
// order whatever the mode: the wait for the input then covers the input loads only.
template <int NPT, int MODE>
__global__ __launch_bounds__(kXThreads) void xcd_attn_kernel(const XcdAttnArgs a) {
  constexpr int D = kD;
  xcd_attn_preload(a);
  const int b = blockIdx.x, g = b & (kXcdGroups - 1), j = b >> 3;
  const int t = threadIdx.x, lane = t & 63;
  const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
  const XcdBufs& X = a.x;

  // ---- the loads that do not depend on the position go out first: the layer input,
  // then the weights (vector loads retire in issue order).  Every wave issues the same
  // loads, the exchange wave with wave 0's addresses (tc, wc) and without using them:
  // loads issued under a wave condition make the compiler's wait for the input cover
  // the loads issued after it as well. ----
  const int tc = t & 255, wc = wid & 3;
  // the position through the constant address space: a scalar load issued here, whose
  // wait the compiler places at the first use (after the input is formed)
  const int pos = *(const __attribute__((address_space(4))) int32_t*)(a.positions);
  XIn xin;
  bool tok_ok = true;
  WChunk wq[2], wo;
  f32x4 g4;
  {
    xin_issue(MODE, X.hx2, X.pd, a.hin, a.emb_token, a.emb_w, a.emb_s, a.emb_vocab, 4 * tc, xin, tok_ok);
    g4 = prep_gamma(a.in_gamma, tc);
    // q|k|v rows 16j .. 16j+15 of the XCD's 512 (one matrix per workgroup)
    const int R0 = 16 * j;
    const uint8_t* wm;
    const uint16_t* sm_;
    int rb;
    if (R0 < 2 * D) {
      wm = a.qw; sm_ = a.qs; rb = 2 * D * g + R0;
    } else if (R0 < 3 * D) {
      wm = a.kw; sm_ = a.ks; rb = D * g + R0 - 2 * D;
    } else {
      wm = a.vw; sm_ = a.vs; rb = D * g + R0 - 3 * D;
    }
    const int c = lane & 31, hf = lane >> 5;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int row = rb + 4 * wc + 2 * p + hf;
      wq[p] = load_w(wm, (size_t)row * (kH / 2) + 16 * c, sm_, (size_t)row * (kH / 64) + (c >> 1));
    }
    // o_proj rows 32j + t/8, columns 256g + 32 (t % 8) .. +31
    {
      const int ro = 32 * j + (tc >> 3), c8 = tc & 7;
      wo = load_w(a.ow, (size_t)ro * (2 * kH / 2) + 128 * g + 16 * c8, a.os,
                  (size_t)ro * (2 * kH / 64) + 4 * g + (c8 >> 1));
    }
  }

  const int T = pos + 1;
  int nA, chunk;
  attn_split(T, nA, chunk);
  const bool attn_active = j < nA;
  const int cstart = j * chunk, cend = min(T, cstart + chunk), cn = cend - cstart;

  __shared__ alignas(16) float sx[kH];
  __shared__ alignas(16) uint32_t ph[kH / 2];
  __shared__ alignas(16) uint32_t pl[kH / 2];
  __shared__ float2 sm[kH / 32];
  __shared__ float sred[4];
  __shared__ float sres[16];
  __shared__ alignas(16) float sqkv[4 * D];
  __shared__ alignas(16) float sq[2][D];
  __shared__ alignas(16) float sodd[2][4 + D];  // odd groups' softmax state (long chunks)
  __shared__ alignas(16) uint16_t snew[2][D];
  __shared__ float swt[2][kXcdBlocks];
  __shared__ alignas(16) float spart[4][2 * D];
  __shared__ alignas(16) uint32_t ph2[2 * D / 2];
  __shared__ alignas(16) uint32_t pl2[2 * D / 2];
  __shared__ float2 sm2[2 * D / 32];

  uint32_t* flags = X.flags + g * kXcdBlocks;
  uint32_t e0 = 0, xcc = 0, fl = 0;

  // ---- the layer input: every workgroup forms all of it (XCD 0, workgroup 0 keeps
  // it as the residual base of launch B) ----
  if (wid < 4) {
    const f32x4 xv = xin_value(MODE, xin, tok_ok);
    *reinterpret_cast<f32x4*>(&sx[4 * t]) = xv;
    if (b == 0) *reinterpret_cast<f32x4*>(X.hx + 4 * t) = xv;
    if (MODE == 2 && !tok_ok && b == 0 && t == 0) atomicOr(X.status, Q4D_STATUS_BAD_TOKEN);
    float ss = fmaf(xv[0], xv[0], fmaf(xv[1], xv[1], fmaf(xv[2], xv[2], xv[3] * xv[3])));
    ss = wave_sum_bcast(ss);
    if (lane == 0) sred[wid] = ss;
  }
  block_sync_lds();

  // ---- the position (checked here: every load before this is independent of it),
  // then the RoPE rows and the K/V rows of the chunk ----
  if (pos < 0 || pos >= a.max_ctx) {
    if (b == 0 && t == 0) atomicOr(X.status, Q4D_STATUS_BAD_POSITION);
    return;  // uniform over the grid: no workgroup enters an exchange
  }
  float nx0 = 0.f, nx1 = 0.f, rc = 0.f, rs = 0.f;
  // attention waves (0, 1: q head 2g + wid): for K, lane = 4 p + quarter (position p of
  // a 16-position group, dims 32 quarter .. +31); for V, lane holds dims 2 lane, 2 lane + 1
  // of each of the group's 16 positions, so P.V needs no sum across lanes
  const int ap = lane >> 2, aq = lane & 3;
  u32x4 kr[4];
  uint32_t vv[16];
  const uint16_t* kb = a.kcache + (size_t)g * a.max_ctx * D;
  const uint16_t* vb = a.vcache + (size_t)g * a.max_ctx * D;
  const int plast = pos > 0 ? pos - 1 : 0;

  {
    {
      const float* gam = wc < 2 ? a.q_gamma : a.k_gamma;
      nx0 = gam[lane];
      nx1 = gam[lane + 64];
      rc = a.rope_cos[(size_t)pos * (D / 2) + lane];
      rs = a.rope_sin[(size_t)pos * (D / 2) + lane];
    }
    // the first 16 positions of the chunk (rows at or past pos load the last cached
    // row; pos itself is replaced from LDS and rows past the chunk are masked).  Every
    // wave issues them and only waves 0 and 1 use them: issued under a wave condition,
    // the compiler's waits for the weights loaded before them would cover them as well.
    {
      int p = cstart + ap;
      p = p < pos ? p : plast;
#pragma unroll
      for (int k = 0; k < 4; ++k) kr[k] = *reinterpret_cast<const u32x4*>(kb + (size_t)p * D + 32 * aq + 8 * k);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int pv = cstart + i < pos ? cstart + i : plast;
        vv[i] = *reinterpret_cast<const uint32_t*>(vb + (size_t)pv * D + 2 * lane);
      }
    }
  }

  // the exchange flag, read by every wave (the exchange wave uses it): a load issued by
  // one wave only shared a register with the compute waves' code and made them wait
  // for every load before the RMSNorm
  xcc = xcc_id();
  fl = ld_sc1_u32(flags + j);

  // ---- input RMSNorm -> hi/lo pairs ----
  if (wid < 4) {
    const float inv = 1.0f / sqrtf(((sred[0] + sred[1]) + (sred[2] + sred[3])) / (float)kH + a.eps);
    prep_item(sx, t, true, inv, g4, ph, pl, sm);
  }
  block_sync_lds();

  // ---- q|k|v dot products: wave w, pass p, half hf -> row 4w + 2p + hf ----
  if (wid < 4) {
    XChunk xh, xl;
    load_chunk(ph, pl, sm, lane & 31, xh, xl);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const float v = half_wave_sum_dpp(wdot(wq[p], xh, xl));
      if ((lane & 31) == 31) sres[4 * wid + 2 * p + (lane >> 5)] = v;
    }
  }
  block_sync_lds();

  if (wid == 4) {
    // ---- exchange 1: the XCD's raw q|k|v ----
    e0 = __builtin_amdgcn_readfirstlane(fl) >> 4;
    if (lane < 16) X.qkv[g * 4 * D + 16 * j + lane] = sres[lane];
    xcd_arrive_wait(flags, j, e0 + 1, xcc, lane, X.status);
    const Rsrc rq = make_rsrc(X.qkv + g * 4 * D, 4 * D * 4);
#pragma unroll
    for (int k = 0; k < 2; ++k)
      *reinterpret_cast<f32x4*>(&sqkv[4 * (lane + 64 * k)]) = ld_sc1_v4(rq, (uint32_t)(lane + 64 * k) * 16);
  }
  block_sync_lds();

  // ---- q/k RMSNorm (common.py:258-262), RoPE (264-268), K/V append (186-189) ----
  // wave 0/1: q head 2g / 2g+1, wave 2: k, wave 3: v; lane l holds dims l and l + 64
  if (wid < 4) {
    const float x0 = sqkv[wid * D + lane], x1 = sqkv[wid * D + lane + 64];
    if (wid < 3) {
      const float ss = wave_sum_bcast(fmaf(x0, x0, x1 * x1));
      const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
      const float n0 = (x0 * inv) * nx0, n1 = (x1 * inv) * nx1;
      const float r0 = n0 * rc + (-n1) * rs;
      const float r1 = n1 * rc + n0 * rs;
      if (wid < 2) {
        sq[wid][lane] = r0 * a.qscale;
        sq[wid][lane + 64] = r1 * a.qscale;
      } else {
        const uint16_t b0 = __builtin_bit_cast(uint16_t, (_Float16)r0);
        const uint16_t b1 = __builtin_bit_cast(uint16_t, (_Float16)r1);
        snew[0][lane] = b0;
        snew[0][lane + 64] = b1;
        if (j == 0) {
          uint16_t* kp = a.kcache + ((size_t)g * a.max_ctx + pos) * D;
          kp[lane] = b0;
          kp[lane + 64] = b1;
        }
      }
    } else {
      const uint16_t b0 = __builtin_bit_cast(uint16_t, (_Float16)x0);
      const uint16_t b1 = __builtin_bit_cast(uint16_t, (_Float16)x1);
      snew[1][lane] = b0;
      snew[1][lane + 64] = b1;
      if (j == 0) {
        uint16_t* vp = a.vcache + ((size_t)g * a.max_ctx + pos) * D;
        vp[lane] = b0;
        vp[lane + 64] = b1;
      }
    }
  }
  block_sync_lds();

  // ---- attention of q head 2g + (wid & 1) over this workgroup's chunk: scores over the
  // 4 quarter lanes of a position, an online softmax over the 16-position groups, P.V
  // with each lane owning two dims of the head.  Waves 0 and 1 take every group, except in
  // chunks of more than one group in the instances of kXcdSplitMinGroups groups and up: there
  // waves 0 and 1 take the even groups and waves 2 and 3 the odd ones, whose softmax state
  // then merges into waves 0 and 1 through LDS.  `split` is uniform over the workgroup
  // (cn is the workgroup's chunk), so the barrier it adds is too ----
  const bool split = NPT >= kXcdSplitMinGroups && cn > 16;
  float M = -INFINITY, L = 0.f, o0 = 0.f, o1 = 0.f;
  if ((wid < 2 || (split && wid < 4)) && attn_active) {
    float q[32];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&sq[wid & 1][32 * aq + 4 * k]);
      q[4 * k] = v[0]; q[4 * k + 1] = v[1]; q[4 * k + 2] = v[2]; q[4 * k + 3] = v[3];
    }
    for (int i = split ? (wid >> 1) : 0; i < NPT; i += split ? 2 : 1) {
      // groups past the chunk add nothing (every score masked): with room for long
      // contexts, stop at the chunk's end (wave-uniform) instead of running all NPT
      if (NPT >= 4 && 16 * i >= cn) break;
      const int pl_ = 16 * i + ap;  // position within the chunk
      const int gb = cstart + 16 * i;  // first position of the group
      if (i > 0) {
        int p = cstart + pl_;
        p = p < pos ? p : plast;
#pragma unroll
        for (int k = 0; k < 4; ++k) kr[k] = *reinterpret_cast<const u32x4*>(kb + (size_t)p * D + 32 * aq + 8 * k);
#pragma unroll
        for (int ii = 0; ii < 16; ++ii) {
          const int pv = gb + ii < pos ? gb + ii : plast;
          vv[ii] = *reinterpret_cast<const uint32_t*>(vb + (size_t)pv * D + 2 * lane);
        }
      }
      if (cstart + pl_ == pos) {
#pragma unroll
        for (int k = 0; k < 4; ++k) kr[k] = *reinterpret_cast<const u32x4*>(&snew[0][32 * aq + 8 * k]);
      }
      if (gb <= pos && pos < gb + 16) vv[pos - gb] = *reinterpret_cast<const uint32_t*>(&snew[1][2 * lane]);
      float sc = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float kf[8];
        unpack8h(kr[k], kf);
#pragma unroll
        for (int e = 0; e < 8; ++e) sc = fmaf(q[8 * k + e], kf[e], sc);
      }
      sc += dpp_f<kDppQuadSwap1>(sc);
      sc += dpp_f<kDppQuadSwap2>(sc);
      const bool valid = pl_ < cn;
      sc = valid ? sc : -INFINITY;
      const float mg = wave_max_bcast(sc);
      const float Mn = fmaxf(M, mg);
      const float so = M == -INFINITY ? 0.f : exp2f(M - Mn);
      const float e = valid ? exp2f(sc - Mn) : 0.f;  // the same in the 4 lanes of a position
      L = L * so + wave_sum_bcast(aq == 0 ? e : 0.f);
      o0 *= so;
      o1 *= so;
#pragma unroll
      for (int ii = 0; ii < 16; ++ii) {
        const float ei = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), 4 * ii));
        // rows past pos stand in for absent positions (at pos 0 a row not yet written):
        // their zero weight must not meet an Inf or NaN bit pattern
        const h2 v = __builtin_bit_cast(h2, gb + ii <= pos ? vv[ii] : 0u);
        o0 = fmaf(ei, (float)v.x, o0);
        o1 = fmaf(ei, (float)v.y, o1);
      }
      M = Mn;
    }
    if (split && wid >= 2) {
      *reinterpret_cast<float2*>(&sodd[wid & 1][4 + 2 * lane]) = make_float2(o0, o1);
      if (lane == 0) {
        sodd[wid & 1][0] = M;
        sodd[wid & 1][1] = L;
      }
    }
  }
  if (split) block_sync_lds();
  if (wid < 2 && attn_active) {
    if (split) {
      // the odd groups' state (a split chunk has at least two groups, so it holds scores)
      const float Mb = sodd[wid][0], Lb = sodd[wid][1];
      const float2 ob = *reinterpret_cast<const float2*>(&sodd[wid][4 + 2 * lane]);
      const float Mn = fmaxf(M, Mb);  // group 0 is never empty: M is finite
      const float sa = exp2f(M - Mn);
      const float sb = Mb == -INFINITY ? 0.f : exp2f(Mb - Mn);
      L = L * sa + Lb * sb;
      o0 = o0 * sa + ob.x * sb;
      o1 = o1 * sa + ob.y * sb;
      M = Mn;
    }
    float* rec = X.ap + (size_t)((g * kXcdBlocks + j) * 2 + wid) * kXcdApRec;
    *reinterpret_cast<float2*>(rec + 4 + 2 * lane) = make_float2(o0, o1);
    if (lane == 0) *reinterpret_cast<f32x4*>(rec) = f32x4{M, L, 0.f, 0.f};
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // acknowledged before the exchange wave's flag
  }
  block_sync_lds();

  // ---- exchange 2: the chunk partials, then their merge (flash-decoding combine) ----
  if (wid == 4) xcd_arrive_wait(flags, j, e0 + 2, xcc, lane, X.status);
  block_sync_lds();
  {
    // the exchange wave turns the chunk maxima and sums into weights
    // w_j = 2^(m_j - M) / sum_k 2^(m_k - M) l_k (lane = chunk + 32 * head); meanwhile
    // compute thread t loads dims 4 (t % 32) of head (t % 64) / 32 of the chunks
    // t / 64, t / 64 + 4, ... (up to 8 loads in flight per thread)
    const Rsrc rap = make_rsrc(X.ap + (size_t)g * kXcdBlocks * 2 * kXcdApRec, kXcdBlocks * 2 * kXcdApRec * 4);
    f32x4 ov[kXcdBlocks / 4];
    const int v = t & 63, hh = v >> 5, rg = t >> 6;
    if (wid == 4) {
      const int jj = lane & 31, h = lane >> 5;
      const bool valid = jj < nA;
      const uint32_t off = (uint32_t)((min(jj, nA - 1) * 2 + h) * kXcdApRec) * 4;
      const float m = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rap, off, 0, 16));
      const float l = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rap, off + 4, 0, 16));
      const float mv = valid ? m : -INFINITY;
      const float Mh = half_max(mv);
      const float w = valid ? exp2f(mv - Mh) : 0.f;
      const float Lh = half_sum(w * (valid ? l : 0.f));
      swt[h][jj] = w / Lh;
    } else {
#pragma unroll
      for (int k = 0; k < kXcdBlocks / 4; ++k) {
        const int jj = min(rg + 4 * k, nA - 1);
        ov[k] = ld_sc1_v4(rap, (uint32_t)((jj * 2 + hh) * kXcdApRec + 4 + 4 * (v & 31)) * 4);
      }
    }
    block_sync_lds();
    if (wid < 4) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < kXcdBlocks / 4; ++k) {
        const int jj = rg + 4 * k;
        const float w = jj < nA ? swt[hh][jj] : 0.f;
        acc += w * ov[k];
      }
      *reinterpret_cast<f32x4*>(&spart[rg][4 * v]) = acc;
    }
    block_sync_lds();
    // the merged 256-dim output is the sum of the 4 rows of spart, in row order
    if (wid == 0) {
      float v[4];
      const int c = lane >> 3, m = (lane & 7) >> 1, i0 = (lane & 1) * 2;
      const int ea = c * 32 + m * 8 + i0, eb = ea + 4;
      const int ix[4] = {ea, eb, ea + 1, eb + 1};
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = ((spart[0][ix[k]] + spart[1][ix[k]]) + spart[2][ix[k]]) + spart[3][ix[k]];
      prep_vals(v, lane, ph2, pl2, sm2);
    }
  }
  block_sync_lds();

  // ---- o_proj split-K partial: rows 32j + t/8, the XCD's 256 columns ----
  if (wid < 4) {
    XChunk xh, xl;
    load_chunk(ph2, pl2, sm2, t & 7, xh, xl);
    float v = wdot(wo, xh, xl);
    v += dpp_f<kDppQuadSwap1>(v);
    v += dpp_f<kDppQuadSwap2>(v);
    v += dpp_f<kDppRowHalfMirror>(v);
    if ((t & 7) == 0) X.po[g * kH + 32 * j + (t >> 3)] = v;
  }
}

// ---------------------------------------------------------------------------
// Launch B: x' = x + o_proj partials, post-attention RMSNorm, gate/up, SwiGLU, down partial.
__global__ __launch_bounds__(kXThreads) void xcd_mlp_kernel(const XcdMlpArgs a) {
  xcd_mlp_preload(a);
  const int b = blockIdx.x, g = b & (kXcdGroups - 1), j = b >> 3;
  const int t = threadIdx.x, lane = t & 63;
  const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
  const XcdBufs& X = a.x;

  __shared__ alignas(16) float sx[kH];
  __shared__ alignas(16) uint32_t ph[kH / 2];
  __shared__ alignas(16) uint32_t pl[kH / 2];
  __shared__ float2 sm[kH / 32];
  __shared__ float sred[4];
  __shared__ float sgu[24];
  __shared__ alignas(16) float sac[kGI];
  __shared__ alignas(16) uint32_t ph2[kGI / 2];
  __shared__ alignas(16) uint32_t pl2[kGI / 2];
  __shared__ float2 sm2[kGI / 32];

  uint32_t* flags = X.flags + g * kXcdBlocks;
  uint32_t e0 = 0, xcc = 0, fl = 0;
  XIn xin;
  bool tok_ok = true;
  WChunk wg[3], wd[2];
  f32x4 g4 = {0.f, 0.f, 0.f, 0.f};

  if (wid == 4) {
    xcc = xcc_id();
    fl = ld_sc1_u32(flags + j);
  } else {
    xin_issue(0, X.hx, X.po, nullptr, nullptr, nullptr, nullptr, 0, 4 * t, xin, tok_ok);
    g4 = prep_gamma(a.post_gamma, t);
    // gate/up: wave w, pass p, half hf -> row r = 6w + 2p + hf of the workgroup's 24
    // (r < 12: gate row 384g + 12j + r; else up row 384g + 12j + r - 12)
    const int c = lane & 31, hf = lane >> 5;
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const int r = 6 * wid + 2 * p + hf;
      const bool up = r >= 12;
      const int n = kGI * g + 12 * j + (up ? r - 12 : r);
      wg[p] = load_w(up ? a.uw : a.gw, (size_t)n * (kH / 2) + 16 * c, up ? a.us : a.gs,
                     (size_t)n * (kH / 64) + (c >> 1));
    }
    // down: pass p, row 32j + 16p + t/16, chunk t%16 (< 12) of the XCD's 384 columns
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int rd = 32 * j + 16 * p + (t >> 4), c16 = min(t & 15, 11);
      wd[p] = load_w(a.dw, (size_t)rd * (3 * kH / 2) + (kGI / 2) * g + 16 * c16, a.ds,
                     (size_t)rd * (3 * kH / 64) + (kGI / 64) * g + (c16 >> 1));
    }
  }

  // ---- x' = x + the 8 o_proj partials, formed by every workgroup (XCD 0, workgroup 0
  // keeps it as the residual base of the next layer) ----
  if (wid < 4) {
    const f32x4 xv = xin_value(0, xin, true);
    *reinterpret_cast<f32x4*>(&sx[4 * t]) = xv;
    if (b == 0) *reinterpret_cast<f32x4*>(X.hx2 + 4 * t) = xv;
    float ss = fmaf(xv[0], xv[0], fmaf(xv[1], xv[1], fmaf(xv[2], xv[2], xv[3] * xv[3])));
    ss = wave_sum_bcast(ss);
    if (lane == 0) sred[wid] = ss;
  }
  block_sync_lds();

  if (wid < 4) {
    const float inv = 1.0f / sqrtf(((sred[0] + sred[1]) + (sred[2] + sred[3])) / (float)kH + a.eps);
    prep_item(sx, t, true, inv, g4, ph, pl, sm);
  }
  block_sync_lds();

  if (wid < 4) {
    XChunk xh, xl;
    load_chunk(ph, pl, sm, lane & 31, xh, xl);
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const float v = half_wave_sum_dpp(wdot(wg[p], xh, xl));
      if ((lane & 31) == 31) sgu[6 * wid + 2 * p + (lane >> 5)] = v;
    }
  }
  block_sync_lds();

  if (wid == 4) {
    // ---- SwiGLU (common.py:288-292), exchange 1: the XCD's 384 activations ----
    e0 = __builtin_amdgcn_readfirstlane(fl) >> 4;
    if (lane < 12) {
      const float gv = sgu[lane], uv = sgu[12 + lane];
      X.ac[g * kGI + 12 * j + lane] = (gv / (1.0f + expf(-gv))) * uv;
    }
    xcd_arrive_wait(flags, j, e0 + 1, xcc, lane, X.status);
    const Rsrc ra = make_rsrc(X.ac + g * kGI, kGI * 4);
    for (int v = lane; v < kGI / 4; v += 64)
      *reinterpret_cast<f32x4*>(&sac[4 * v]) = ld_sc1_v4(ra, (uint32_t)v * 16);
  }
  block_sync_lds();
  if (t < kGI / 4) prep_item(sac, t, false, 1.f, g4, ph2, pl2, sm2);
  block_sync_lds();

  // ---- down split-K partial ----
  if (wid < 4) {
    const int c16 = t & 15;
    XChunk xh, xl;
    load_chunk(ph2, pl2, sm2, min(c16, 11), xh, xl);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      float v = c16 < 12 ? wdot(wd[p], xh, xl) : 0.f;
      v = row16_sum(v);
      if (c16 == 0) X.pd[g * kH + 32 * j + 16 * p + (t >> 4)] = v;
    }
  }
}

// out = hx2 + sum of the 8 down partials (the layer output after the last layer).
__global__ __launch_bounds__(256) void xcd_finalize_kernel(const float* hx2, const float* pd, float* out) {
  const int e = 4 * threadIdx.x;
  *reinterpret_cast<f32x4*>(out + e) = sum_partials(hx2, pd, e);
}

// Placement probe of the device check: workgroup b of a grid shaped like the XCD-split
// launches writes 0x100 | the XCC_ID register of the XCD it ran on.  No waits.
constexpr int kProbeBlocks = kXcdGroups * kXcdBlocks;
__device__ uint32_t g_xcc_probe[kProbeBlocks];

__global__ __launch_bounds__(64) void xcc_probe_kernel(uint32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = 0x100u | xcc_id();
}

template <int NPT>
bool attn_kernels_fit(int dev) {
  const void* fns[3] = {reinterpret_cast<const void*>(&xcd_attn_kernel<NPT, 0>),
                        reinterpret_cast<const void*>(&xcd_attn_kernel<NPT, 1>),
                        reinterpret_cast<const void*>(&xcd_attn_kernel<NPT, 2>)};
  (void)dev;
  for (const void* f : fns) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, kXThreads, 0) != hipSuccess || n < 1) return false;
  }
  return true;
}

// The device facts the XCD-split launches rely on: at least 8 x 32 CUs, one 320-thread
// workgroup of every launch fits on a CU, and a 256-workgroup grid deals workgroups
// b, b + 8, b + 16, ... to one XCD, with the 8 residues on 8 different XCDs.
bool xcd_device_probe(int dev, hipStream_t st) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < kXcdGroups * kXcdBlocks)
    return false;
  if (!attn_kernels_fit<1>(dev) || !attn_kernels_fit<2>(dev) || !attn_kernels_fit<4>(dev) ||
      !attn_kernels_fit<8>(dev) || !attn_kernels_fit<16>(dev) || !attn_kernels_fit<32>(dev) ||
      !attn_kernels_fit<64>(dev))
    return false;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&xcd_mlp_kernel), kXThreads,
                                                   0) != hipSuccess ||
      n < 1)
    return false;
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_xcc_probe)) != hipSuccess || !p) return false;
  uint32_t* dp = static_cast<uint32_t*>(p);
  uint32_t h[kProbeBlocks];
  hipLaunchKernelGGL(xcc_probe_kernel, dim3(kProbeBlocks), dim3(64), 0, st, dp);
  if (hipGetLastError() != hipSuccess) return false;
  if (hipMemcpyAsync(h, dp, sizeof(h), hipMemcpyDeviceToHost, st) != hipSuccess) return false;
  if (hipStreamSynchronize(st) != hipSuccess) return false;
  unsigned seen = 0;
  for (int b = 0; b < kProbeBlocks; ++b) {
    if (!(h[b] & 0x100u) || (h[b] & 0xfu) != (h[b & (kXcdGroups - 1)] & 0xfu)) return false;
    if (b < kXcdGroups) seen |= 1u << (h[b] & 0xfu);
  }
  return __builtin_popcount(seen) == kXcdGroups;
}

}  // namespace

namespace {
std::mutex g_check_mu;
int g_check_mode = 0;                 // 1: report every device as unsuitable
constexpr int kMaxDevices = 64;
int8_t g_check_state[kMaxDevices] = {};  // per device: 0 unknown, 1 suitable, -1 not
}  // namespace

// Per-device answer of xcd_device_probe, found once (not while `st` is being captured
// into a graph: the probe synchronises; the plan then falls back without caching).
bool xcd_device_ok(hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lock(g_check_mu);
  if (g_check_mode == 1) return false;
  if (g_check_state[dev]) return g_check_state[dev] > 0;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
  g_check_state[dev] = xcd_device_probe(dev, st) ? 1 : -1;
  return g_check_state[dev] > 0;
}

int xcd_set_check_mode(int mode) {
  std::lock_guard<std::mutex> lock(g_check_mu);
  const int prev = g_check_mode;
  g_check_mode = mode;
  return prev;
}

int xcd_npt(int max_ctx) {
  const int cm = max(16, (max_ctx + kXcdBlocks - 1) / kXcdBlocks);
  const int n = (cm + 15) / 16;
  return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : n <= 8 ? 8 : n <= 16 ? 16 : n <= 32 ? 32 : n <= 64 ? 64 : 0;
}

template <int NPT>
void launch_xcd_attn_npt(const XcdAttnArgs& a, hipStream_t st) {
  const dim3 grid(kXcdGroups * kXcdBlocks), block(kXThreads);
  switch (a.in_mode) {
    case 0: hipLaunchKernelGGL((xcd_attn_kernel<NPT, 0>), grid, block, 0, st, a); break;
    case 1: hipLaunchKernelGGL((xcd_attn_kernel<NPT, 1>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((xcd_attn_kernel<NPT, 2>), grid, block, 0, st, a); break;
  }
}

int launch_xcd_attn(const XcdAttnArgs& a, hipStream_t st) {
  if (a.in_mode < 0 || a.in_mode > 2) return Q4D_ERR_SHAPE;
  switch (xcd_npt(a.max_ctx)) {
    case 1: launch_xcd_attn_npt<1>(a, st); break;
    case 2: launch_xcd_attn_npt<2>(a, st); break;
    case 4: launch_xcd_attn_npt<4>(a, st); break;
    case 8: launch_xcd_attn_npt<8>(a, st); break;
    case 16: launch_xcd_attn_npt<16>(a, st); break;
    case 32: launch_xcd_attn_npt<32>(a, st); break;
    case 64: launch_xcd_attn_npt<64>(a, st); break;
    default: return Q4D_ERR_CAPACITY;
  }
  return check_launch();
}

int launch_xcd_mlp(const XcdMlpArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(xcd_mlp_kernel, dim3(kXcdGroups * kXcdBlocks), dim3(kXThreads), 0, st, a);
  return check_launch();
}

int launch_xcd_finalize(const XcdBufs& x, float* out, hipStream_t st) {
  hipLaunchKernelGGL(xcd_finalize_kernel, dim3(1), dim3(256), 0, st, x.hx2, x.pd, out);
  return check_launch();
}

}  // namespace q4d
