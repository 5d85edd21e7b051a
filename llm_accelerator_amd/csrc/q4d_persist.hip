// Persistent batch-1 decode kernel (gfx950): a run of up to
// kPersistMaxLayers decoder layers (common.py:231-298) in one launch.
//
// Each layer is five phases, the stages of the multi-kernel path:
//   qkv     input RMSNorm + q|k|v GEMV                       (all blocks)
//   attn    q/k RMSNorm + RoPE + KV append + attention over a (kv head,
//           128-position chunk) unit, partials out           (blocks 0 .. 8 x chunks)
//   o_proj  merge of the chunk partials + o_proj + residual  (kOprojBlocks blocks
//                                                             after the attention ones)
//   gate_up post-attention RMSNorm + gate/up + SwiGLU        (all blocks)
//   down    down_proj + residual                             (all blocks)
// A phase needs the whole output of the one before it, produced by other
// blocks.  Between kernels that dependency costs a launch (~1.6 us in a HIP
// graph) plus a memory round trip for the weights; here a block issues the
// loads of its next phase's weights (and, for attention, of its K/V chunk)
// first and only then waits for its inputs, so the weight round trip hides
// behind the wait.
//
// Exchange: every value a phase hands to another block is one 64-bit word
// (tag << 32 | fp32 bits) written with a device-scope atomic store; the
// consumer polls its words with device-scope atomic loads until each tag
// equals this launch's tag.  64-bit accesses are single-copy atomic, so a
// word with the right tag holds the right value; no counters, fences or
// barriers across blocks are needed.  Each layer of the launch has its own
// words (no reuse within a launch), and the tag is a per-block launch
// counter kept in the workspace, so words left by earlier launches carry
// older tags.  The chunk partials are the exception: each o_proj block
// reads all of them, so polling them word by word would multiply that
// traffic; an attention unit stores them as plain fp32 words, waits until
// its stores are performed, and then sets one tagged flag, which the o_proj
// blocks poll before reading the partials once.
//
// Every wait is bounded: a poll that spins kSpinLimit times sets
// Q4D_STATUS_SYNC_TIMEOUT and a block-wide abort flag, after which the block
// stops waiting, so every wave always reaches the end of the kernel.  The
// host launches the kernel only when the occupancy query shows all
// kPersistBlocks blocks can be resident at once (each block waits only for
// work of blocks that are running).
//
// Arithmetic per output element is that of the multi-kernel path: the same
// tile loads, dequant dot products, activation staging and reduction orders
// (q4d_gemv_dev.h) and the same attention and merge formulas.
#include <math.h>

#include "q4d_device.h"
#include "q4d_gemv_dev.h"
#include "q4d_internal.h"

namespace q4d {

namespace {

constexpr int kNW = kPersistWaves;
constexpr int kNT = kNW * 64;
constexpr int kOprojBlocks = 32;  // blocks of the o_proj phase (each reads every chunk partial)
constexpr int kOprojBlock0 = 8 * kPersistChunks;  // ... placed after the attention blocks
constexpr int kSpinLimit = 1 << 20;
constexpr int kD = 128;
constexpr int kPartFloats = kD + 4;  // 128 partial output dims, max, sum, 2 pad (16-byte rows)

static_assert(kPersistBlocks * kNW >= 2048, "q|k|v: one 2-row tile per wave");
static_assert(kPersistBlocks * 12 >= 1536, "gate/up: one tile pair per wave of the first 12");
static_assert(kPersistBlocks * 4 >= 512, "down: one tile per 3-wave team of the first 4");
static_assert(kOprojBlocks * 8 * 2 == 512, "o_proj: two tiles per 2-wave team");
static_assert(kOprojBlock0 + kOprojBlocks <= kPersistBlocks, "attention and o_proj on separate blocks");

// ---- tagged exchange words ------------------------------------------------------
__device__ __forceinline__ uint64_t tload(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tstore(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_ok(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ float tval(uint64_t w) { return __uint_as_float((uint32_t)w); }

struct Sync {
  uint32_t tag;
  int32_t* status;
  int* abort;  // LDS flag: this block already gave up waiting once
};

// Spin until every word w[k] = *addr(k) carries the tag (bounded).  All N
// loads go out together; a stale set is re-read whole (no per-word branches,
// so the loops unroll and nothing is indexed dynamically).
template <int N, class F>
__device__ __forceinline__ void tpoll(F addr, uint64_t (&w)[N], const Sync& sy) {
  // Gate: while the producers are still busy only lane 0 of the wave polls
  // (its first word), so waves that arrive early do not flood the memory
  // system with polls of the whole vector.  Called by whole waves.
  const int lane = threadIdx.x & 63;
  for (int spins = 0;; ++spins) {
    uint64_t g = (uint64_t)sy.tag << 32;
    if (lane == 0) g = tload(addr(0));
    if (__builtin_amdgcn_readfirstlane((int)tag_ok(g, sy.tag))) break;
    if (spins >= kSpinLimit) {
      atomicOr(sy.status, Q4D_STATUS_SYNC_TIMEOUT);
      *reinterpret_cast<volatile int*>(sy.abort) = 1;
      break;
    }
    if (*reinterpret_cast<volatile int*>(sy.abort)) break;
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int k = 0; k < N; ++k) w[k] = tload(addr(k));
  for (int spins = 0;; ++spins) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ok &= tag_ok(w[k], sy.tag);
    if (ok) break;
    if (spins >= kSpinLimit) {
      atomicOr(sy.status, Q4D_STATUS_SYNC_TIMEOUT);
      *reinterpret_cast<volatile int*>(sy.abort) = 1;
      break;
    }
    if (*reinterpret_cast<volatile int*>(sy.abort)) break;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < N; ++k) w[k] = tload(addr(k));
  }
}

__device__ __forceinline__ f32x4 tpoll4(const uint64_t* p, const Sync& sy) {
  uint64_t w[4];
  tpoll([p](int k) { return p + k; }, w, sy);
  return f32x4{tval(w[0]), tval(w[1]), tval(w[2]), tval(w[3])};
}

__device__ __forceinline__ float tpoll1(const uint64_t* p, const Sync& sy) {
  uint64_t w[1];
  tpoll([p](int) { return p; }, w, sy);
  return tval(w[0]);
}

// One wave: spin until flags[0 .. n) all carry the tag (n <= 64, bounded).
__device__ __forceinline__ void wave_poll_flags(const uint64_t* flags, int n, const Sync& sy) {
  const int lane = threadIdx.x & 63;
  const uint64_t* p = flags + (lane < n ? lane : n - 1);
  uint64_t w = tload(p);
  for (int spins = 0;; ++spins) {
    if (__all(tag_ok(w, sy.tag))) break;
    if (spins >= kSpinLimit) {
      atomicOr(sy.status, Q4D_STATUS_SYNC_TIMEOUT);
      *reinterpret_cast<volatile int*>(sy.abort) = 1;
      break;
    }
    if (*reinterpret_cast<volatile int*>(sy.abort)) break;
    __builtin_amdgcn_s_sleep(1);
    w = tload(p);
  }
}

__device__ __forceinline__ void fstore(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// threadIdx.x behind an empty asm: each phase recomputes its lane addresses
// instead of the compiler hoisting them all out of the layer loop (where
// they no longer fit in registers and go to scratch).
__device__ __forceinline__ int phase_tid() {
  int t = threadIdx.x;
  __asm__ volatile("" : "+v"(t));
  return t;
}

__device__ __forceinline__ uint64_t* layer_words(const PersistArgs& a, int li) {
  return a.xbuf + (size_t)li * kPxLayerWords;
}
// fp32 chunk partials of head h, chunk c: [128 dims, max, sum, pad, pad]
__device__ __forceinline__ float* layer_parts(const PersistArgs& a, int li) {
  return reinterpret_cast<float*>(layer_words(a, li) + kPxPart);
}

// ---- phase 1: input RMSNorm + q|k|v ------------------------------------------------
template <int XP>
__device__ __forceinline__ void phase_qkv(const PersistArgs& a, const PLayer& L, int li, const Sync& sy,
                                          ActLds<1024, kNW, X_RMS, XP>& s) {
  constexpr int K = 1024, NP = 2048;  // 4096 rows = q 2048 | k 1024 | v 1024
  const int tid = phase_tid();
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = wid * gridDim.x + blockIdx.x;
  const int tt = tile < NP ? tile : NP - 1;
  const Rsrc rw0 = make_rsrc(L.w[0], 2048u * (K / 2)), rs0 = make_rsrc(L.s[0], 2048u * (K / 32));
  const Rsrc rw1 = make_rsrc(L.w[1], 1024u * (K / 2)), rs1 = make_rsrc(L.s[1], 1024u * (K / 32));
  const Rsrc rw2 = make_rsrc(L.w[2], 1024u * (K / 2)), rs2 = make_rsrc(L.s[2], 1024u * (K / 32));
  const int e0 = 2048, e1 = 3072;
  const LaneOff lo = lane_off<K>(0, lane);
  const TileData A = load_tile<K>(tt, lo, SEG_RS);

  ActRegs<K, kNW, X_RMS, XP> ar;
  if (wid < 4) {  // 256 threads own the 256 four-float vectors of the hidden state
    const int t = tid;
    ar.g[0] = reinterpret_cast<const f32x4*>(L.in_norm)[t];
    if (li == 0)
      ar.x[0] = reinterpret_cast<const f32x4*>(a.h_in)[t];
    else
      ar.x[0] = tpoll4(layer_words(a, li - 1) + kPxH2 + 4 * t, sy);
  }
  block_sync_lds();  // the previous phase's LDS reads are done
  act_prepare<K, kNW, X_RMS, XP>(a.eps, ar, s);
  XChunk xh, xl;
  act_chunk(s, lane & 31, xh, xl);
  __builtin_amdgcn_sched_barrier(0);
  const float v = tile_rows<XP>(A, lo.sshift, xh, xl);
  if ((lane & 31) == 31 && tile < NP) tstore(layer_words(a, li) + kPxQkv + 2 * tile + (lane >> 5), v, sy.tag);
}

// ---- phase 2: attention over one (kv head, chunk) unit -----------------------------
struct AttnLds {
  float sq[2][kD];
  uint16_t snew[2][kD];  // fp16 bits of the appended k (roped) and v
  float ssc[2][kAttnChunkLong];
  float sml[2][2];
  float spv[16][2][kD];  // P.V partials per position row group
};

__device__ __forceinline__ void unpack8(const u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t we = w[e];
    const h2 v = __builtin_bit_cast(h2, we);
    f[2 * e] = (float)v.x;
    f[2 * e + 1] = (float)v.y;
  }
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp_f<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  return fmaxf(v, dpp_f<kDppRowMirror>(v));
}
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

// Waves 0-3 run the unit (the thread mapping of attn_kernel<128> in
// q4d_attention.hip); waves 4-15 only take part in the block barriers.
__device__ __forceinline__ void phase_attn(const PersistArgs& a, const PLayer& L, int li, int pos, const Sync& sy,
                                           AttnLds& s) {
  constexpr int D = kD, CH = kAttnChunkLong, NPT = CH / 16;
  const int T = pos + 1;
  const int ns = (T + CH - 1) / CH;
  const int u = blockIdx.x;
  if (u >= 8 * ns) return;  // block-uniform: no unit for this block
  const int j = u & 7, c = u >> 3;
  const int t = phase_tid(), lane = t & 63;
  const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
  const bool act = wid < 4;
  const int start = c * CH;
  const int n = min(T, start + CH) - start;
  const bool last = (c == ns - 1);  // holds position pos
  uint16_t* kb = a.kcache + (size_t)li * a.layer_stride + (size_t)j * a.max_ctx * D;
  uint16_t* vb = kb + a.kind_stride;

  // ---- every K/V load of the chunk first (positions below pos come from the
  // cache; rows past them are loaded from the last cached row and get zero
  // weight; position pos is replaced from LDS below)
  const int sub = t & 15, pr = (t >> 4) & 15;
  u32x4 kr[NPT], vr[NPT];
  const int plast = pos > 0 ? pos - 1 : 0;
  if (act) {
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      int p = start + pr + 16 * i;
      p = p < pos ? p : plast;
      kr[i] = *reinterpret_cast<const u32x4*>(kb + (size_t)p * D + sub * 8);
      vr[i] = *reinterpret_cast<const u32x4*>(vb + (size_t)p * D + sub * 8);
    }
  }

  // ---- raw q (waves 0/1: heads 2j, 2j+1), new k (wave 2) and v (wave 3) rows;
  // lane l holds dims l and l + 64
  const float qscale = a.scaling * 1.4426950408889634f;  // log2(e) folded in for exp2
  float x0 = 0.f, x1 = 0.f, g0 = 0.f, g1 = 0.f, cs = 0.f, sn = 0.f;
  if (act) {
    const float* gam = wid < 2 ? L.q_norm : L.k_norm;
    g0 = gam[lane];
    g1 = gam[lane + 64];
    cs = a.rope_cos[(size_t)pos * (D / 2) + lane];
    sn = a.rope_sin[(size_t)pos * (D / 2) + lane];
    const int ridx = wid < 2 ? 2 * j + wid : (wid == 2 ? 16 + j : 24 + j);
    const uint64_t* row = layer_words(a, li) + kPxQkv + ridx * D + lane;
    uint64_t w[2];
    tpoll([row](int k) { return row + 64 * k; }, w, sy);
    x0 = tval(w[0]);
    x1 = tval(w[1]);
  }
  const bool qk_wave = wid < 2 || (last && wid == 2);
  const bool v_wave = last && wid == 3;
  // per-head RMSNorm (common.py:258-262) + rotate-half RoPE (common.py:264-268)
  if (qk_wave) {
    const float ss = wave_sum_all(fmaf(x0, x0, x1 * x1));
    const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
    const float n0 = (x0 * inv) * g0, n1 = (x1 * inv) * g1;
    const float r0 = n0 * cs + (-n1) * sn;
    const float r1 = n1 * cs + n0 * sn;
    if (wid < 2) {
      s.sq[wid][lane] = r0 * qscale;
      s.sq[wid][lane + 64] = r1 * qscale;
    } else {
      const uint16_t b0 = __builtin_bit_cast(uint16_t, (_Float16)r0);
      const uint16_t b1 = __builtin_bit_cast(uint16_t, (_Float16)r1);
      s.snew[0][lane] = b0;
      s.snew[0][lane + 64] = b1;
      kb[(size_t)pos * D + lane] = b0;  // append_cache (common.py:186-189)
      kb[(size_t)pos * D + lane + 64] = b1;
    }
  } else if (v_wave) {
    const uint16_t b0 = __builtin_bit_cast(uint16_t, (_Float16)x0);
    const uint16_t b1 = __builtin_bit_cast(uint16_t, (_Float16)x1);
    s.snew[1][lane] = b0;
    s.snew[1][lane + 64] = b1;
    vb[(size_t)pos * D + lane] = b0;
    vb[(size_t)pos * D + lane + 64] = b1;
  }
  block_sync_lds();
  if (act && last) {
    const int ip = pos - start - pr;
    if (ip >= 0 && (ip & 15) == 0) {
      const int i = ip >> 4;
      const u32x4 kn4 = *reinterpret_cast<const u32x4*>(&s.snew[0][sub * 8]);
      const u32x4 vn4 = *reinterpret_cast<const u32x4*>(&s.snew[1][sub * 8]);
#pragma unroll
      for (int ii = 0; ii < NPT; ++ii)
        if (ii == i) {
          kr[ii] = kn4;
          vr[ii] = vn4;
        }
    }
  }

  // ---- scores: 8-dim partial dots reduced over the 16 lanes of a position
  if (act) {
    float q0[8], q1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      q0[e] = s.sq[0][sub * 8 + e];
      q1[e] = s.sq[1][sub * 8 + e];
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      float kf[8];
      unpack8(kr[i], kf);
      float y0 = 0.f, y1 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y0 = fmaf(q0[e], kf[e], y0);
        y1 = fmaf(q1[e], kf[e], y1);
      }
      y0 = row16_sum(y0);
      y1 = row16_sum(y1);
      const int p = pr + 16 * i;
      if (sub == 0 && p < n) {
        s.ssc[0][p] = y0;
        s.ssc[1][p] = y1;
      }
    }
  }
  block_sync_lds();

  // ---- chunk softmax (one wave per head, two positions per lane)
  if (wid < 2) {
    float sc[CH / 64];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < CH / 64; ++k) {
      const int p = lane + 64 * k;
      sc[k] = p < n ? s.ssc[wid][p] : -INFINITY;
      mx = fmaxf(mx, sc[k]);
    }
    const float m = wave_max_all(mx);
    float es = 0.f;
#pragma unroll
    for (int k = 0; k < CH / 64; ++k) {
      const int p = lane + 64 * k;
      const float e = p < n ? exp2f(sc[k] - m) : 0.f;
      s.ssc[wid][p] = e;
      es += e;
    }
    const float l = wave_sum_all(es);
    if (lane == 0) {
      s.sml[wid][0] = m;
      s.sml[wid][1] = l;
    }
  }
  block_sync_lds();

  // ---- P.V on the registers loaded at the start
  if (act) {
    float o0[8], o1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o0[e] = o1[e] = 0.f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int p = pr + 16 * i;
      const float e0 = p < n ? s.ssc[0][p] : 0.f;
      const float e1 = p < n ? s.ssc[1][p] : 0.f;
      float vf[8];
      unpack8(vr[i], vf);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o0[e] = fmaf(e0, vf[e], o0[e]);
        o1[e] = fmaf(e1, vf[e], o1[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      *reinterpret_cast<f32x4*>(&s.spv[pr][0][sub * 8 + e]) = f32x4{o0[e], o0[e + 1], o0[e + 2], o0[e + 3]};
      *reinterpret_cast<f32x4*>(&s.spv[pr][1][sub * 8 + e]) = f32x4{o1[e], o1[e + 1], o1[e + 2], o1[e + 3]};
    }
  }
  block_sync_lds();
  if (act) {
    const int hh = t >> 7, d = t & (D - 1), h = 2 * j + hh;
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) acc += s.spv[g][hh][d];
    float* part = layer_parts(a, li) + (size_t)(h * kPersistChunks + c) * kPartFloats;
    fstore(part + d, acc);
    if (d == 0) {
      fstore(part + kD, s.sml[hh][0]);
      fstore(part + kD + 1, s.sml[hh][1]);
    }
  }
  // every wave's partial stores are performed (the barrier waits for them),
  // then the unit's flag tells the o_proj blocks the partials are complete
  __syncthreads();
  if (t == 0) tstore(layer_words(a, li) + kPxFlags + u, 0.f, sy.tag);
}

// ---- phase 3: merge of the chunk partials + o_proj + residual ------------------------
// Dims d .. d + 3 of head h merged over its ns chunks (read once, after the
// unit flags): running maximum M over the chunk maxima m_c, then
// sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c.  The reads are 128-bit
// buffer loads with the device-coherent cache policy, all issued before any
// is used: chunks 0-3 unconditionally, 4-7 under one block-uniform branch
// (loads under a condition are merged at its join with a wait for all of
// them, so more branches would cost a round trip each).  Chunks past ns
// re-read chunk ns - 1 and are masked out.
__device__ __forceinline__ f32x4 merge_parts(const float* parts, int h, int ns, int d) {
  constexpr int kSc1 = 16;  // cache policy: device-coherent (as the agent-scope atomic loads)
  const Rsrc r = make_rsrc(parts, 16u * kPersistChunks * kPartFloats * 4);
  const uint32_t base = (uint32_t)(h * kPersistChunks) * kPartFloats * 4;
  f32x4 acc[kPersistChunks];
  f32x4 ml[kPersistChunks];  // (max, sum, pad, pad)
  static_assert(kPersistChunks == 8, "two batches of four chunks");
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = ml[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto load = [&](int c) {
    const uint32_t off = base + (uint32_t)(c < ns ? c : ns - 1) * kPartFloats * 4;
    acc[c] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)d * 4, off, kSc1));
    ml[c] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, 0u, off + kD * 4, kSc1));
  };
  // one branch: its join waits for everything issued so far, once
#pragma unroll
  for (int c = 0; c < 4; ++c) load(c);
  if (ns > 4) {
#pragma unroll
    for (int c = 4; c < 8; ++c) load(c);
  }
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < kPersistChunks; ++c)
    if (c < ns) M = fmaxf(M, ml[c][0]);
  float Ls = 0.f;
  f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < kPersistChunks; ++c) {
    const float wgt = c < ns ? exp2f(ml[c][0] - M) : 0.f;
    Ls = fmaf(wgt, ml[c][1], Ls);
    o += wgt * acc[c];
  }
  return o * (1.0f / Ls);
}

template <int XP>
__device__ __forceinline__ void phase_oproj(const PersistArgs& a, const PLayer& L, int li, int pos, const Sync& sy,
                                            ActLds<2048, kNW, X_F32, XP>& s, float* s_part) {
  constexpr int K = 2048, KS = 2, TEAMS = kNW / KS, U = 2, NB = kOprojBlocks;
  const int b = (int)blockIdx.x - kOprojBlock0;
  if (b < 0 || b >= NB) return;  // block-uniform
  const int tid = phase_tid();
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int team = wid / KS, ks = wid % KS, r = lane >> 5;
  const Rsrc rw = make_rsrc(L.w[3], 1024u * (K / 2)), rs = make_rsrc(L.s[3], 1024u * (K / 32));
  const LaneOff lo = lane_off<K>(ks, lane);
  TileData A[U];
  int tl[U];
#pragma unroll
  for (int uu = 0; uu < U; ++uu) {
    tl[uu] = (uu * TEAMS + team) * NB + b;  // 0 .. 511
    A[uu] = load_rows<K>(rw, rs, 2 * tl[uu], lo);
  }
  // residual rows of this lane (the hidden state entering the layer)
  float res[U];
#pragma unroll
  for (int uu = 0; uu < U; ++uu) {
    const int row = 2 * tl[uu] + r;
    res[uu] = li == 0 ? a.h_in[row] : tpoll1(layer_words(a, li - 1) + kPxH2 + row, sy);
  }
  // wait for the attention units' flags (one wave), then every thread t < 512
  // merges dims 4t .. 4t + 3 (head t / 32) of the attention output
  const int ns = pos / kAttnChunkLong + 1;
  if (wid == 0) wave_poll_flags(layer_words(a, li) + kPxFlags, 8 * ns, sy);
  block_sync_lds();
  ActRegs<K, kNW, X_F32, XP> ar;
  if (wid < 8) {
    const int t = tid, h = t >> 5, d = (t & 31) * 4;
    ar.x[0] = merge_parts(layer_parts(a, li), h, ns, d);
  }
  block_sync_lds();
  act_prepare<K, kNW, X_F32, XP>(a.eps, ar, s);
  XChunk xh, xl;
  act_chunk(s, ks * 32 + (lane & 31), xh, xl);
  __builtin_amdgcn_sched_barrier(0);
  float rsum[U];
#pragma unroll
  for (int uu = 0; uu < U; ++uu) rsum[uu] = tile_rows<XP>(A[uu], lo.sshift, xh, xl);
  const bool owner = (lane & 31) == 31;
  if (owner) {
#pragma unroll
    for (int uu = 0; uu < U; ++uu) s_part[((uu * TEAMS + team) * KS + ks) * 2 + r] = rsum[uu];
  }
  block_sync_lds();
  if (ks == 0 && owner) {
#pragma unroll
    for (int uu = 0; uu < U; ++uu) {
      float v = s_part[((uu * TEAMS + team) * KS) * 2 + r];
#pragma unroll
      for (int k = 1; k < KS; ++k) v += s_part[((uu * TEAMS + team) * KS + k) * 2 + r];
      tstore(layer_words(a, li) + kPxH1 + 2 * tl[uu] + r, res[uu] + v, sy.tag);
    }
  }
}

// ---- phase 4: post-attention RMSNorm + gate/up + SwiGLU -------------------------------
template <int XP>
__device__ __forceinline__ void phase_gateup(const PersistArgs& a, const PLayer& L, int li, const Sync& sy,
                                             ActLds<1024, kNW, X_RMS, XP>& s) {
  constexpr int K = 1024, NP = 1536;  // row pairs of each 3072 x 1024 matrix
  const int tid = phase_tid();
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = wid * gridDim.x + blockIdx.x;
  const int tt = tile < NP ? tile : NP - 1;
  const Rsrc rwg = make_rsrc(L.w[4], 3072u * (K / 2)), rsg = make_rsrc(L.s[4], 3072u * (K / 32));
  const Rsrc rwu = make_rsrc(L.w[5], 3072u * (K / 2)), rsu = make_rsrc(L.s[5], 3072u * (K / 32));
  const LaneOff lo = lane_off<K>(0, lane);
  const TileData A = load_rows<K>(rwg, rsg, 2 * tt, lo);
  const TileData G = load_rows<K>(rwu, rsu, 2 * tt, lo);
  ActRegs<K, kNW, X_RMS, XP> ar;
  if (wid < 4) {
    const int t = tid;
    ar.g[0] = reinterpret_cast<const f32x4*>(L.post_norm)[t];
    ar.x[0] = tpoll4(layer_words(a, li) + kPxH1 + 4 * t, sy);
  }
  block_sync_lds();
  act_prepare<K, kNW, X_RMS, XP>(a.eps, ar, s);
  XChunk xh, xl;
  act_chunk(s, lane & 31, xh, xl);
  __builtin_amdgcn_sched_barrier(0);
  const float g = tile_rows<XP>(A, lo.sshift, xh, xl);
  const float up = tile_rows<XP>(G, lo.sshift, xh, xl);
  if ((lane & 31) == 31 && tile < NP)
    tstore(layer_words(a, li) + kPxAct + 2 * tile + (lane >> 5), (g / (1.0f + expf(-g))) * up, sy.tag);
}

// ---- phase 5: down_proj + residual ---------------------------------------------------
template <int XP>
__device__ __forceinline__ void phase_down(const PersistArgs& a, const PLayer& L, int li, const Sync& sy,
                                           ActLds<3072, kNW, X_F32, XP>& s, float* s_part) {
  constexpr int K = 3072, KS = 3, NP = 512, TEAMS = kNW / KS;  // 5 teams; wave 15 has none
  const int tid = phase_tid();
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int team = wid / KS, ks = wid % KS, r = lane >> 5;
  const int tile = team * gridDim.x + blockIdx.x;
  const bool has = team < TEAMS && tile < NP;
  const int tt = tile < NP ? tile : NP - 1;
  const Rsrc rw = make_rsrc(L.w[6], 1024u * (K / 2)), rs = make_rsrc(L.s[6], 1024u * (K / 32));
  const LaneOff lo = lane_off<K>(ks, lane);
  const TileData A = load_rows<K>(rw, rs, 2 * tt, lo);
  const float res = tpoll1(layer_words(a, li) + kPxH1 + 2 * tt + r, sy);
  ActRegs<K, kNW, X_F32, XP> ar;
  if (wid < 12) {  // 768 threads own the 768 vectors of the SwiGLU activation
    ar.x[0] = tpoll4(layer_words(a, li) + kPxAct + 4 * tid, sy);
  }
  block_sync_lds();
  act_prepare<K, kNW, X_F32, XP>(a.eps, ar, s);
  XChunk xh, xl;
  act_chunk(s, ks * 32 + (lane & 31), xh, xl);
  __builtin_amdgcn_sched_barrier(0);
  const float p = tile_rows<XP>(A, lo.sshift, xh, xl);
  const bool owner = (lane & 31) == 31;
  if (owner && team < TEAMS) s_part[(team * KS + ks) * 2 + r] = p;
  block_sync_lds();
  if (ks == 0 && owner && has) {
    float v = s_part[(team * KS) * 2 + r];
#pragma unroll
    for (int k = 1; k < KS; ++k) v += s_part[(team * KS + k) * 2 + r];
    const int row = 2 * tile + r;
    const float out = res + v;
    tstore(layer_words(a, li) + kPxH2 + row, out, sy.tag);
    if (li == a.nl - 1) a.h_out[row] = out;  // read by the next kernel
  }
}

template <int XP>
union PersistLds {
  ActLds<1024, kNW, X_RMS, XP> a1;
  ActLds<2048, kNW, X_F32, XP> a2;
  ActLds<3072, kNW, X_F32, XP> a3;
  AttnLds at;
};

template <int XP>
__global__ __launch_bounds__(kNT) void persist_kernel(const PersistArgs a) {
  __shared__ PersistLds<XP> sm;
  __shared__ float s_part[64];
  __shared__ int s_abort;
  if (threadIdx.x == 0) s_abort = 0;
  __syncthreads();
  Sync sy;
  sy.tag = (uint32_t)a.seq[blockIdx.x] + 1u;
  sy.status = a.status;
  sy.abort = &s_abort;
  const int pos = a.positions[0];
  if (pos >= 0 && pos < a.max_ctx) {
    for (int li = 0; li < a.nl; ++li) {
      const PLayer& L = a.L[li];
      phase_qkv<XP>(a, L, li, sy, sm.a1);
      phase_attn(a, L, li, pos, sy, sm.at);
      phase_oproj<XP>(a, L, li, pos, sy, sm.a2, s_part);
      phase_gateup<XP>(a, L, li, sy, sm.a1);
      phase_down<XP>(a, L, li, sy, sm.a3, s_part);
    }
  } else if (blockIdx.x == 0 && threadIdx.x == 0) {
    atomicOr(a.status, Q4D_STATUS_BAD_POSITION);
  }
  if (threadIdx.x == 0) a.seq[blockIdx.x] = (int32_t)sy.tag;  // the next launch's tags follow this one's
}

// Resident blocks per CU for the kernel (0 on error), cached per device.
int residency(int xp) {
  static int cache[2][64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int& c = cache[xp - 1][dev];
  if (c == 0) {
    int occ = 0, cus = 0;
    const hipError_t e1 = xp == 2 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, persist_kernel<2>, kNT, 0)
                                  : hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, persist_kernel<1>, kNT, 0);
    const hipError_t e2 = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    c = (e1 == hipSuccess && e2 == hipSuccess) ? occ * cus : -1;
  }
  return c;
}

}  // namespace

bool persist_eligible(const q4d_model_t* m) {
  if (m->hidden_size != 1024 || m->intermediate_size != 3072 || m->num_q_heads != 16 || m->num_kv_heads != 8 ||
      m->head_dim != 128 || m->max_ctx > kPersistMaxCtx)
    return false;
  return residency(1) >= kPersistBlocks && residency(2) >= kPersistBlocks;
}

int launch_persist(const PersistArgs& a, int xp, hipStream_t st) {
  if (a.nl < 1 || a.nl > kPersistMaxLayers || a.max_ctx > kPersistMaxCtx) return Q4D_ERR_SHAPE;
  if (residency(xp) < kPersistBlocks) return Q4D_ERR_LAUNCH;
  if (xp == 2)
    hipLaunchKernelGGL(persist_kernel<2>, dim3(kPersistBlocks), dim3(kNT), 0, st, a);
  else
    hipLaunchKernelGGL(persist_kernel<1>, dim3(kPersistBlocks), dim3(kNT), 0, st, a);
  return check_launch();
}

}  // namespace q4d
