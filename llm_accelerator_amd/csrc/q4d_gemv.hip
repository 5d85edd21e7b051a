// Fused Q4 dequant-GEMV for gfx950 (wave64).
//
// Two kernels share one activation prologue and one dequant trick
// (q4d_device.h):
//
// gemv_kernel (one-shot; the decode-layer projections).  Tile: one wave
// covers 2 rows x 1024 columns.  Lane l reads the 16-byte chunk (l % 32) of
// row (l / 32), i.e. 32 columns, and the 32-bit word holding that chunk's
// Q2.14 scale, so every lane issues one 128-bit weight load per tile.  A
// matrix with K = 2048 or 3072 gives each row pair KS = K / 1024 waves of one
// block (one 1024-column slice each); their row sums are added through LDS
// in slice order (deterministic).  The gate/up pair of the MLP is two tiles
// per wave (the same two rows of each matrix).  Each wave takes U tiles and
// issues all their loads before consuming any.
//
// lm_kernel (streaming; the 151936 x 1024 LM head with fused argmax).  One
// resident grid; each wave walks 4-row tiles grid-stride in stages of U
// tiles with two stages in flight (ping-pong register sets, unconditional
// reloads in the steady state).  16 lanes cover a row: lane l of row l / 16
// holds the chunks at columns 32 (l % 16) and 512 + 32 (l % 16), so both
// loads are fully coalesced and a row is reduced over 16 lanes.  The hi and
// lo activation products share one accumulator per nibble position.  This
// halves the reduction and scale work per byte of the 2-row tile, which
// matters because between its prologue and its argmax hand-off the kernel
// keeps the SIMDs' VALU nearly saturated (4 waves per SIMD at ~130 VALU
// instructions per 2 KB tile), while the table streams at ~6.8 TB/s; the
// fixed phases around that (activation prologue, argmax hand-off) cost ~8 µs.
//
// Loads are buffer loads: the matrix base is a wave-uniform resource, the
// tile's row offset a scalar and the lane's offset a per-lane constant, so no
// per-load address arithmetic is spent.  Wave indices are scalar
// (readfirstlane) and tile indices are clamped into the matrix instead of
// guarded, so no load sits behind a divergent branch.  Activation loads go
// out first (vmcnt retires in issue order, so waiting for the activations
// leaves the weights in flight).
//
// Activations are prepared once per block in LDS: the block stages x (and
// gamma), computes the RMSNorm where asked, and converts the vector into the
// fp16 pair order the dequant trick consumes (hi, and lo = x - hi for ~22-bit
// activations), with per-chunk sums; each lane then reads its ready chunks.
// Doing this conversion per lane instead costs ~400 VALU instructions per
// wave and dominated the decode-size GEMVs.
//
// Prologues: fp16 x, fp32 x, RMSNorm of an fp32 hidden vector (reference
// common.py:129-134), or RMSNorm of the tied Q4 embedding row of a token id read
// on the device (the first layer of a one-token step; its block 0 also stores
// the row as the residual stream).  Epilogues: fp16/fp32 store, residual add
// (common.py:284,297), SwiGLU over the gate/up pair (common.py:293-295), and
// LM-head argmax with the lowest-index tie rule
// (56_export_persistent_multitoken_layer_golden.py:860).  The argmax is
// finished without fences, in two levels: each block folds its best (score,
// index) into the 64-bit key of its group (blocks g, g + 8, ...) with a
// device-scope atomicMax, waits for it to complete, then counts in on its
// group's counter; the last block of a group counts in on the top counter, and
// the last of those reads the eight group keys with device-scope loads (every
// read goes to the coherence point).  With greedy feedback that block also
// stores the token as the next step's input, advances the position and
// records the history (what advance_kernel does as a launch of its own).
// Weights and scales are read with non-temporal loads, and a wave's issue
// priority falls as it progresses, so the waves of a SIMD finish together.
#include <math.h>
#include <string.h>

#include "q4d_device.h"
#include "q4d_internal.h"
#include "q4d_gemv_dev.h"

namespace q4d {

namespace {

constexpr int kSlice = 1024;       // columns per wave tile
constexpr int kLmBlocksPerCU = 4;  // resident blocks per CU for the streaming kernel
constexpr int kLmStage = 1;        // 4-row tiles per stage of the streaming kernel
constexpr int kLmWaves = 16;       // waves per block of the streaming kernel
constexpr int kAttnMergeWaves = 8;   // waves per block of the GEMV merging attention partials
// Issue this thread's activation (and gamma) loads.
template <int K, int NWB, int XM, int XP>
__device__ __forceinline__ void act_load(const GemvArgs& a, int bat, ActRegs<K, NWB, XM, XP>& r) {
  using R = ActRegs<K, NWB, XM, XP>;
  if constexpr (XM == X_ATTN) return;  // chunk partials: attn_issue / attn_finish
  if constexpr (XM == X_EMB) {
    // vector v = columns 4v .. 4v+3: two bytes of codes and its group's scale code
    // of the token's row (row 0 stands in for an id outside the table)
    const int tok = __builtin_amdgcn_readfirstlane(a.emb_token[0]);
    const size_t row = (tok >= 0 && tok < a.emb_vocab) ? (size_t)tok : 0;
#pragma unroll
    for (int i = 0; i < R::XPT; ++i) {
      const int v = threadIdx.x + i * NWB * 64;
      if (v < R::XV) {
        r.ec[i] = *reinterpret_cast<const uint16_t*>(a.emb_w + row * (K / 2) + 2 * v);
        r.es[i] = a.emb_s[row * (K / 64) + v / 16];
        r.g[i] = reinterpret_cast<const f32x4*>(a.gamma)[v];
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < R::XPT; ++i) {
    const int v = threadIdx.x + i * NWB * 64;
    if (v < R::XV) {
      r.x[i] = reinterpret_cast<const f32x4*>(static_cast<const char*>(a.x) +
                                              (size_t)bat * K * (XM == X_F16 ? 2 : 4))[v];
      if constexpr (XM == X_RMS) r.g[i] = reinterpret_cast<const f32x4*>(a.gamma)[v];
    }
  }
}

// X_EMB: the embedding row from the codes act_load fetched, q * scale / 2^14
// exactly as embedding_kernel computes it; block 0 stores it as the residual
// stream and reports an id outside the table.
template <int K, int NWB, int XP>
__device__ __forceinline__ void emb_convert(const GemvArgs& a, ActRegs<K, NWB, X_EMB, XP>& r) {
  using R = ActRegs<K, NWB, X_EMB, XP>;
  const int tok = __builtin_amdgcn_readfirstlane(a.emb_token[0]);
  const bool ok = tok >= 0 && tok < a.emb_vocab;
  const bool writer = blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
  for (int i = 0; i < R::XPT; ++i) {
    const int v = threadIdx.x + i * NWB * 64;
    if (v < R::XV) {
      const float sc = scale_q2_14(r.es[i]);
      f32x4 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int nib = (int)((r.ec[i] >> (4 * e)) & 0xFu);
        x[e] = ok ? (float)(nib - ((nib & 0x8) ? 16 : 0)) * sc : 0.0f;
      }
      r.x[i] = x;
      if (writer) reinterpret_cast<f32x4*>(a.emb_out)[v] = x;
    }
  }
  if (writer && !ok && threadIdx.x == 0 && a.emb_status) atomicOr(a.emb_status, Q4D_STATUS_BAD_TOKEN);
}

// X_ATTN: the attention output for this thread's vectors, merged from the
// split-K chunk partials of the decode-attention kernel (merge = 0): running
// maximum M over the chunks' maxima m_i, then sum_i 2^(m_i - M) acc_i over
// sum_i 2^(m_i - M) l_i (the flash-decoding combine, as the attention kernel's
// own merge does it).  The loads of up to kMergeBatch chunks go out together.
constexpr int kMergeBatch = 8;

// One batch of kMergeBatch chunks of partials for dims d..d+3 of one head:
// the loads (issued on their own so they can go out before the weights) and
// the fold into the running (M, L, o).
struct MergeLoads {
  float2 ml[kMergeBatch];
  f32x4 ac[kMergeBatch];
};

__device__ __forceinline__ void merge_issue(const GemvArgs& a, size_t base, int d, int c0, MergeLoads& m) {
  constexpr int D = 128;
  // addresses clamp to the workspace, not to ns: ns comes from a device
  // load, and addresses depending on it would wait for that load first
#pragma unroll
  for (int k = 0; k < kMergeBatch; ++k) {
    const int c = c0 + k < a.nsplit_max ? c0 + k : a.nsplit_max - 1;
    m.ml[k] = *reinterpret_cast<const float2*>(a.part_ml + (base + c) * 2);
    m.ac[k] = *reinterpret_cast<const f32x4*>(a.part_acc + (base + c) * D + d);
  }
}

__device__ __forceinline__ void merge_fold(const MergeLoads& m, int c0, int ns, float& M, float& L, f32x4& o) {
  // chunks past ns are masked with selects, not branches: a branch lets the
  // compiler sink their loads into it, behind a wait for everything in flight
  float mk[kMergeBatch], lk[kMergeBatch];
  f32x4 ac[kMergeBatch];
  float Mn = M;
#pragma unroll
  for (int k = 0; k < kMergeBatch; ++k) {
    const bool valid = c0 + k < ns;
    mk[k] = valid ? m.ml[k].x : -INFINITY;
    lk[k] = valid ? m.ml[k].y : 0.f;
    ac[k] = valid ? m.ac[k] : f32x4{0.f, 0.f, 0.f, 0.f};
    Mn = fmaxf(Mn, mk[k]);
  }
  const float so = M == -INFINITY ? 0.f : exp2f(M - Mn);
  L *= so;
  o *= so;
#pragma unroll
  for (int k = 0; k < kMergeBatch; ++k) {
    const float wgt = exp2f(mk[k] - Mn);  // 0 for masked chunks
    L = fmaf(wgt, lk[k], L);
    o += wgt * ac[k];
  }
  M = Mn;
}

// X_ATTN activations: the first batch of chunk partials of this thread's
// vectors is loaded by attn_issue (before the weights), the merge runs in
// attn_finish (after the weights are issued); further batches, past
// kMergeBatch chunks, load and fold in turn.
template <int K, int NWB>
struct AttnPre {
  static constexpr int XV = K / 4, NT = NWB * 64, XPT = (XV + NT - 1) / NT;
  MergeLoads m[XPT];
  int pos;
};

template <int K, int NWB>
__device__ __forceinline__ void attn_issue(const GemvArgs& a, int bat, AttnPre<K, NWB>& p) {
  using P = AttnPre<K, NWB>;
  constexpr int D = 128;
  p.pos = a.positions[bat];
#pragma unroll
  for (int i = 0; i < P::XPT; ++i) {
    const int v = threadIdx.x + i * P::NT;
    const int vc = P::XV % P::NT != 0 && v >= P::XV ? P::XV - 1 : v;
    const int h = (4 * vc) / D, d = (4 * vc) % D;
    const size_t base = ((size_t)bat * (K / D) + h) * a.nsplit_max;
    merge_issue(a, base, d, 0, p.m[i]);
  }
}

template <int K, int NWB>
__device__ __forceinline__ void attn_finish(const GemvArgs& a, int bat, const AttnPre<K, NWB>& p,
                                            f32x4 (&xr)[(K / 4 + NWB * 64 - 1) / (NWB * 64)]) {
  using P = AttnPre<K, NWB>;
  constexpr int D = 128;
  int ns = (p.pos + a.attn_chunk) / a.attn_chunk;  // chunks holding positions 0..pos
  ns = ns < 1 ? 1 : (ns > a.nsplit_max ? a.nsplit_max : ns);
#pragma unroll
  for (int i = 0; i < P::XPT; ++i) {
    const int v = threadIdx.x + i * P::NT;
    if (P::XV % P::NT != 0 && v >= P::XV) continue;
    const int h = (4 * v) / D, d = (4 * v) % D;
    const size_t base = ((size_t)bat * (K / D) + h) * a.nsplit_max;
    float M = -INFINITY, L = 0.f;
    f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
    merge_fold(p.m[i], 0, ns, M, L, o);
    for (int c0 = kMergeBatch; c0 < ns; c0 += kMergeBatch) {
      MergeLoads m;
      merge_issue(a, base, d, c0, m);
      merge_fold(m, c0, ns, M, L, o);
    }
    xr[i] = o * (1.0f / L);
  }
}

// ---- one-shot kernel ----------------------------------------------------------
template <int KS, int NWB, int XM, int XP, int EP, bool PAIR, int U>
__device__ __forceinline__ void gemv_body(const GemvArgs& a) {
  constexpr int K = KS * kSlice;
  constexpr int TEAMS = NWB / KS;
  static_assert(NWB % KS == 0, "a block holds whole teams");
  static_assert(!PAIR || KS == 1, "gate/up pairs need K = 1024");
  static_assert(XM != X_F16 || XP == 1, "fp16 activations have no lo part");
  static_assert(EP != EP_ARGMAX, "the argmax epilogue lives in lm_kernel");
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int team = wid / KS;
  const int ks = wid % KS;
  const int bat = blockIdx.y;

  __shared__ ActLds<K, NWB, XM, XP> s_act;
  __shared__ float s_part[U * TEAMS * KS * 2];

  const int NP = a.rows / 2;  // tiles (row pairs; PAIR: of each matrix)

  // ---- activation loads go out first, then every weight load -----------------
  ActRegs<K, NWB, XM, XP> ar;
  act_load(a, bat, ar);
  AttnPre<K, NWB> ap;
  if constexpr (XM == X_ATTN) {
    attn_issue<K, NWB>(a, bat, ap);
    __builtin_amdgcn_sched_barrier(0);
  }

  const int e0 = a.seg_end[0], e1 = a.seg_end[1];
  const Rsrc rw0 = make_rsrc(a.w[0], (uint32_t)e0 * (K / 2));
  const Rsrc rs0 = make_rsrc(a.s[0], (uint32_t)e0 * (K / 32));
  const Rsrc rw1 = make_rsrc(a.w[1], (uint32_t)(PAIR ? e0 : e1 - e0) * (K / 2));
  const Rsrc rs1 = make_rsrc(a.s[1], (uint32_t)(PAIR ? e0 : e1 - e0) * (K / 32));
  const Rsrc rw2 = make_rsrc(a.w[2], (uint32_t)(a.seg_end[2] - e1) * (K / 2));
  const Rsrc rs2 = make_rsrc(a.s[2], (uint32_t)(a.seg_end[2] - e1) * (K / 32));
  const LaneOff lo = lane_off<K>(ks, lane);

  TileData A[U], G[PAIR ? U : 1];
  const int base = blockIdx.x * TEAMS + team;
  const int step = gridDim.x * TEAMS;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int t = base + u * step;
    t = t < NP ? t : NP - 1;
    if constexpr (PAIR) {
      A[u] = load_rows<K>(rw0, rs0, 2 * t, lo);  // gate rows
      G[u] = load_rows<K>(rw1, rs1, 2 * t, lo);  // up rows
    } else {
      A[u] = load_tile<K>(t, lo, SEG_RS);
    }
  }
  // the residual rows this lane may own, fetched with the weights rather than
  // after the reduction (that would add a dependent memory round trip)
  float res_pre[EP == EP_RESID ? U : 1];
  if constexpr (EP == EP_RESID) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = base + u * step;
      res_pre[u] = a.resid[(size_t)bat * a.rows + 2 * (t < NP ? t : NP - 1) + (lane >> 5)];
    }
  }
  // the attention partials were loaded before the weights, so the merge can
  // start as soon as they arrive (vmcnt retires in issue order); the barrier
  // keeps the scheduler from moving weight loads behind the merge arithmetic
  if constexpr (XM == X_ATTN) {
    __builtin_amdgcn_sched_barrier(0);
    attn_finish<K, NWB>(a, bat, ap, ar.x);
  }

  if constexpr (XM == X_EMB) emb_convert(a, ar);
  act_prepare(a.eps, ar, s_act);
  XChunk xh, xl;
  act_chunk(s_act, ks * 32 + (lane & 31), xh, xl);
  // keep the activation reads ahead of the first weight use: left to itself
  // the scheduler hoists weight arithmetic above them, so the wave would wait
  // for the weights first and build the activations afterwards
  __builtin_amdgcn_sched_barrier(0);

  const bool owner = (lane & 31) == 31;
  const int r = lane >> 5;
  float rs[U], rg[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    rs[u] = tile_rows<XP>(A[u], lo.sshift, xh, xl);
    if constexpr (PAIR) rg[u] = tile_rows<XP>(G[u], lo.sshift, xh, xl);
  }
  if constexpr (KS > 1) {
    if (owner) {
#pragma unroll
      for (int u = 0; u < U; ++u) s_part[((u * TEAMS + team) * KS + ks) * 2 + r] = rs[u];
    }
    __syncthreads();
    if (ks != 0) return;
    if (owner) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float v = s_part[((u * TEAMS + team) * KS) * 2 + r];
#pragma unroll
        for (int k = 1; k < KS; ++k) v += s_part[((u * TEAMS + team) * KS + k) * 2 + r];
        rs[u] = v;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int t = base + u * step;
    if (t >= NP) break;
    const float v = rs[u];
    if (owner) {
      const size_t o = (size_t)bat * a.rows + 2 * t + r;
      if constexpr (EP == EP_SWIGLU) {
        static_cast<float*>(a.y)[o] = (v / (1.0f + expf(-v))) * rg[u];
      } else if constexpr (EP == EP_F16) {
        static_cast<_Float16*>(a.y)[o] = (_Float16)v;
      } else if constexpr (EP == EP_F32) {
        static_cast<float*>(a.y)[o] = v;
      } else if constexpr (EP == EP_RESID) {
        static_cast<float*>(a.y)[o] = res_pre[u] + v;
      }
    }
  }
}

template <int KS, int NWB, int XM, int XP, int EP, bool PAIR, int U>
__global__ __launch_bounds__(NWB * 64) void gemv_kernel(const GemvArgs a) {
  gemv_body<KS, NWB, XM, XP, EP, PAIR, U>(a);
}

// Grouped plain linear: blockIdx.z picks one of up to kGemvGroupMax independent matrices of
// one shape, each with its own activations and output (the pointers sit in the argument
// block and are read through the kernarg segment pointer, so the runtime index does not
// copy the block to scratch); within a matrix the work is gemv_kernel's, so each output
// equals a launch of its own bit for bit.
constexpr int kGemvGroupMax = 64;

struct GemvGroupArgs {
  GemvArgs a;  // the shared geometry (segment 0 only; its pointers unused)
  const uint8_t* w[kGemvGroupMax];
  const uint16_t* s[kGemvGroupMax];
  const void* x[kGemvGroupMax];
  void* y[kGemvGroupMax];
};

// Row pairs per wave of the grouped kernel: a launch over many matrices streams, so each
// wave takes several pairs (the activation staging and the reduction are per block).
constexpr int kGroupU = 4;
constexpr int kGroupWaves = 8;  // waves per block at K = 1024

template <int KS, int NWB, int XM, int XP, int EP>
__global__ __launch_bounds__(NWB * 64) void gemv_group_kernel(const GemvGroupArgs G) {
  typedef __attribute__((address_space(4))) const GemvGroupArgs* KernargPtr;
  const KernargPtr P = (KernargPtr)__builtin_amdgcn_kernarg_segment_ptr();
  const int g = blockIdx.z;
  GemvArgs a = G.a;
  const uint8_t* w = P->w[g];
  const uint16_t* sc = P->s[g];
  a.w[0] = a.w[1] = a.w[2] = w;
  a.s[0] = a.s[1] = a.s[2] = sc;
  a.x = P->x[g];
  a.y = P->y[g];
  gemv_body<KS, NWB, XM, XP, EP, false, kGroupU>(a);
}

// ---- streaming LM-head kernel -------------------------------------------------
// One 4-row tile for one lane: two weight chunks (512 columns apart) and the
// scale word of one of their groups (the neighbour lane holds the other).
struct Tile4 {
  u32x4 w0, w1;
  uint32_t s;
};

// sum_j q_j x_j over one 32-column chunk times the chunk's scale code, hi and
// lo products in shared accumulators.  s8 = (8 * sum of hi + lo) * 2^-14.
template <int XP>
__device__ __forceinline__ float chunk_scaled(const u32x4 w, const XChunk& h, const XChunk& l, float s8,
                                              float code) {
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    // shift first, then xor+and in one 3-input op each (5 VALU per word)
    const uint32_t v = w[m], t = v >> 8;
    const uint32_t m0 = (v ^ 0x88888888u) & 0x000F000Fu, m1 = (v ^ 0x88888888u) & 0x00F000F0u;
    const uint32_t m2 = (t ^ 0x00888888u) & 0x000F000Fu, m3 = (t ^ 0x00888888u) & 0x00F000F0u;
    a = dot2(m0, h.p[4 * m + 0], a);
    b = dot2(m1, h.p[4 * m + 1], b);
    a = dot2(m2, h.p[4 * m + 2], a);
    b = dot2(m3, h.p[4 * m + 3], b);
    if constexpr (XP == 2) {
      a = dot2(m0, l.p[4 * m + 0], a);
      b = dot2(m1, l.p[4 * m + 1], b);
      a = dot2(m2, l.p[4 * m + 2], a);
      b = dot2(m3, l.p[4 * m + 3], b);
    }
  }
  // (2^24 a + 2^20 b - 8 sum x) * code * 2^-14
  return code * fmaf(fmaf(a, 16.f, b), 64.f, -s8);
}

// s_setprio with a wave-uniform runtime level (the instruction takes an immediate).
__device__ __forceinline__ void set_prio(int p) {
  if (p >= 3)
    __builtin_amdgcn_s_setprio(3);
  else if (p == 2)
    __builtin_amdgcn_s_setprio(2);
  else if (p == 1)
    __builtin_amdgcn_s_setprio(1);
  else
    __builtin_amdgcn_s_setprio(0);
}

template <int XP, int U, int NWB, bool PARTS>
__global__ __launch_bounds__(NWB * 64) void lm_kernel(const GemvArgs a) {
  constexpr int K = 1024;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  __shared__ ActLds<K, NWB, X_RMS, XP> s_act;
  __shared__ unsigned long long s_key[NWB];

  const int R = a.rows;
  const int NT4 = (R + 3) / 4;  // 4-row tiles; the last one is moved back to rows R-4..R-1

  ActRegs<K, NWB, X_RMS, XP> ar;
  act_load(a, 0, ar);
  static_assert(ActRegs<K, NWB, X_RMS, XP>::XPT == 1, "one activation vector per thread");
  f32x4 pp[PARTS ? kXcdGroups : 1];
  if constexpr (PARTS) {
    if (threadIdx.x < K / 4) {
#pragma unroll
      for (int g = 0; g < kXcdGroups; ++g) pp[g] = reinterpret_cast<const f32x4*>(a.x_parts + g * K)[threadIdx.x];
    }
  }

  const Rsrc rw = make_rsrc(a.w[0], (uint32_t)R * (K / 2));
  const Rsrc rsc = make_rsrc(a.s[0], (uint32_t)R * (K / 32));
  const int r = lane >> 4, sub = lane & 15;
  const uint32_t vw = (uint32_t)(r * (K / 2) + sub * 16);
  const int g0 = sub >> 1;  // group of chunk 0; chunk 1 is in group 8 + g0
  const uint32_t vs = (uint32_t)(r * (K / 32) + 4 * ((lane & 1) ? 4 + (g0 >> 1) : (g0 >> 1)));
  const int sshift = (g0 & 1) * 16;
  const bool even = (lane & 1) == 0;

  auto load4 = [&](int t) {
    t = t < NT4 ? t : NT4 - 1;
    const int row0 = min(4 * t, R - 4);
    Tile4 d;
    d.w0 = __builtin_amdgcn_raw_buffer_load_b128(rw, vw, (uint32_t)row0 * (K / 2), kLoadNT);
    d.w1 = __builtin_amdgcn_raw_buffer_load_b128(rw, vw + 256, (uint32_t)row0 * (K / 2), kLoadNT);
    d.s = __builtin_amdgcn_raw_buffer_load_b32(rsc, vs, (uint32_t)row0 * (K / 32), kLoadNT);
    return d;
  };

  // waves are numbered wave-major (wave w of every block, then wave w + 1), so the waves
  // that take one tile more than the others are spread about one per SIMD
  const int base = wid * gridDim.x + blockIdx.x;
  const int step = gridDim.x * NWB;
  Tile4 A[U], B[U];
#pragma unroll
  for (int u = 0; u < U; ++u) A[u] = load4(base + u * step);
  if constexpr (PARTS) {
    if (threadIdx.x < K / 4) {
      f32x4 v = ar.x[0];
#pragma unroll
      for (int g = 0; g < kXcdGroups; ++g) v = v + pp[g];
      ar.x[0] = v;
      if (blockIdx.x == 0 && a.x_out) reinterpret_cast<f32x4*>(a.x_out)[threadIdx.x] = v;
    }
  }
  // stage 1 goes out after the activation prologue: issued with stage 0 the
  // grid's 15 MB of weight requests queue the activation loads behind them
  // (measured ~1 µs later prologue).  It is unconditional (clamped): a
  // conditional issue makes the wait-count pass assume at every later merge
  // that it may be missing.
  act_prepare(a.eps, ar, s_act);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < U; ++u) B[u] = load4(base + (U + u) * step);

  XChunk xh0, xl0, xh1, xl1;
  act_chunk(s_act, sub, xh0, xl0);
  act_chunk(s_act, 16 + sub, xh1, xl1);
  const float s80 = (xh0.sum8 + (XP == 2 ? xl0.sum8 : 0.f)) * (1.0f / 16384.0f);
  const float s81 = (xh1.sum8 + (XP == 2 ? xl1.sum8 : 0.f)) * (1.0f / 16384.0f);
  __builtin_amdgcn_sched_barrier(0);

  float best = -INFINITY;
  int besti = 0x7fffffff;
  auto consume = [&](const Tile4 (&D)[U], int first) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = first + u * step;
      // the even lane of a pair loaded chunk 0's scale word, the odd lane chunk 1's
      const uint32_t other = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)D[u].s, kDppQuadSwap1, 0xF, 0xF, false);
      const uint32_t w0s = even ? D[u].s : other, w1s = even ? other : D[u].s;
      const float c0 = (float)((w0s >> sshift) & 0xFFFFu);
      const float c1 = (float)((w1s >> sshift) & 0xFFFFu);
      float p = chunk_scaled<XP>(D[u].w0, xh0, xl0, s80, c0) + chunk_scaled<XP>(D[u].w1, xh1, xl1, s81, c1);
      p = row16_sum(p);
      if (t < NT4 && sub == 15) {
        const int row = min(4 * t, R - 4) + r;
        if (a.logits) a.logits[row] = p;
        // rows rise along a lane's sequence: strict > keeps the lowest index
        // among equal scores
        if (p > best) {
          best = p;
          besti = row;
        }
      }
    }
  };
  // S stages of U tiles for this wave (the host sizes the grid so that S >= 2
  // wherever the matrix allows; tiles past the matrix are masked).  Steady state:
  // both reloads are unconditional, so each consume waits only for its own stage.
  const int S = base < NT4 ? (NT4 - base + U * step - 1) / (U * step) : 0;
  auto reload = [&](Tile4 (&D)[U], int st) {
#pragma unroll
    for (int u = 0; u < U; ++u) D[u] = load4(base + (st * U + u) * step);
  };
  // Issue priority falls as a wave progresses, from 3 to 0 over its S stages, with
  // the older waves of a SIMD (wid / 4: 0 oldest) given a head start: among equal
  // priorities the SIMD issues the oldest wave first, which left the youngest slot
  // 30 % slower per tile and finishing ~3 us after the oldest.
  const int lead = 2 * (3 - (wid >> 2));
  auto prio = [&](int k) { set_prio(3 - min(3, (4 * k + lead) / max(S, 1))); };
  int st = 0;
  for (; st + 3 < S; st += 2) {
    prio(st);
    consume(A, base + st * U * step);
    reload(A, st + 2);
    prio(st + 1);
    consume(B, base + (st + 1) * U * step);
    reload(B, st + 3);
  }
  prio(st);
  consume(A, base + st * U * step);
  if (st + 2 < S) {
    reload(A, st + 2);
    prio(st + 1);
    consume(B, base + (st + 1) * U * step);
    prio(st + 2);
    consume(A, base + (st + 2) * U * step);
  } else {
    prio(st + 1);
    consume(B, base + (st + 1) * U * step);  // may lie wholly past the matrix
  }
  set_prio(0);

  unsigned long long key = argmax_key(best, besti);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const unsigned long long o = __shfl_xor(key, m, kWave);
    key = o > key ? o : key;
  }
  if (lane == 0) s_key[wid] = key;
  __syncthreads();
  if (wid == 0) {
    unsigned long long bk = s_key[0];
#pragma unroll
    for (int w = 1; w < NWB; ++w) bk = s_key[w] > bk ? s_key[w] : bk;
    // two levels (see kLmHandBytes): fold into group key g and wait for the atomic to
    // be performed, count in on group counter g; the last block of a group counts in
    // on the top counter, and the last of those reads the group keys (8 lanes, one
    // load).  With one key and one counter for all 256 blocks, arrivals queued ~1.3 us
    // at the single address.
    char* const hb = a.lm_hand;
    const int G = gridDim.x, ng = G < kLmGroups ? G : kLmGroups, g = blockIdx.x % kLmGroups;
    int tdone = -1;
    if (lane == 0) {
      const unsigned long long old = __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(hb + 128 * g), bk,
                                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("" ::"v"((uint32_t)old), "v"((uint32_t)(old >> 32)) : "memory");
      const int done = __hip_atomic_fetch_add(reinterpret_cast<int*>(hb + 1024 + 128 * g), 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
      if (done == (G - g + kLmGroups - 1) / kLmGroups - 1)
        tdone = __hip_atomic_fetch_add(reinterpret_cast<int*>(hb + 2048), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    tdone = __builtin_amdgcn_readfirstlane(tdone);
    if (tdone == ng - 1) {
      const int li = lane < ng ? lane : 0;
      unsigned long long fin = __hip_atomic_load(reinterpret_cast<unsigned long long*>(hb + 128 * li),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int m = kLmGroups / 2; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(fin, m, kWave);
        fin = o > fin ? o : fin;
      }
      // ready for the next launch (stream order makes these visible to it)
      if (lane < ng) {
        __hip_atomic_store(reinterpret_cast<unsigned long long*>(hb + 128 * lane), 0ull, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(reinterpret_cast<int*>(hb + 1024 + 128 * lane), 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      if (lane == 0) {
        float sc;
        int ix;
        argmax_unkey(fin, &sc, &ix);
        a.out_token[0] = ix;
        a.out_score[0] = sc;
        if (a.adv_tokens) {  // greedy feedback, as advance_kernel
          a.adv_tokens[0] = ix;
          a.adv_positions[0] += 1;
          if (a.hist_tokens) {
            const int32_t c = a.hist_count[0];
            if (c < a.hist_cap) {
              a.hist_tokens[c] = ix;
              if (a.hist_scores) a.hist_scores[c] = sc;
              a.hist_count[0] = c + 1;
            }
          }
        }
        __hip_atomic_store(reinterpret_cast<int*>(hb + 2048), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// ---------------------------------------------------------------------------
template <class F>
int resident_blocks(F kernel, int threads) {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu < 1)
      return 256;  // conservative fallback, recomputed next call
    cached = cus * (per_cu < kLmBlocksPerCU ? per_cu : kLmBlocksPerCU);
  }
  return cached;
}

template <int XP>
int launch_lm(const GemvArgs& a, hipStream_t stream) {
  constexpr int U = kLmStage, NWB = kLmWaves;
  if (a.rows < 4) return Q4D_ERR_SHAPE;
  const int NT4 = (a.rows + 3) / 4;
  // the resident grid, or fewer blocks where that leaves every wave two stages
  const int res = resident_blocks(lm_kernel<XP, U, NWB, false>, NWB * 64);
  int blocks = (int)((long)NT4 / ((long)NWB * U * 2));
  if (blocks > res) blocks = res;
  if (blocks < 1) blocks = 1;
  if (a.x_parts)
    hipLaunchKernelGGL((lm_kernel<XP, U, NWB, true>), dim3(blocks), dim3(NWB * 64), 0, stream, a);
  else
    hipLaunchKernelGGL((lm_kernel<XP, U, NWB, false>), dim3(blocks), dim3(NWB * 64), 0, stream, a);
  return check_launch();
}

template <int KS, int NWB, int XM, int XP, int EP, bool PAIR, int U>
int launch_inst(const GemvArgs& a, hipStream_t stream) {
  constexpr int TEAMS = NWB / KS;
  const int NP = a.rows / 2;
  int blocks = (NP + TEAMS * U - 1) / (TEAMS * U);
  if (blocks < 1) blocks = 1;
  dim3 grid(blocks, a.batch);
  hipLaunchKernelGGL((gemv_kernel<KS, NWB, XM, XP, EP, PAIR, U>), grid, dim3(NWB * 64), 0, stream, a);
  return check_launch();
}

// Block shapes: K = 1024 -> 4 one-slice waves (fp16 activations: 8, which stage the
// vector once for twice the rows; the 3072 x 1024 GEMV from HBM in a chain of launches:
// 2.38 -> 2.29 us, with 2, 6, 12 or 16 waves or two row pairs per wave slower);
// K = 2048 -> 2 teams of 2; K = 3072 -> 2 teams of 3 (384 threads).
template <int KS, int XM>
constexpr int nwb_of() {
  return KS == 3 ? 6 : (KS == 1 && XM == X_F16) ? 8 : 4;
}

template <int KS, int XM, int XP, int EP, bool PAIR>
int launch_sel(const GemvArgs& a, hipStream_t st) {
  if constexpr (EP == EP_ARGMAX) {
    static_assert(KS == 1 && XM == X_RMS, "LM head: K = 1024 with the final RMSNorm");
    return launch_lm<XP>(a, st);
  } else if constexpr (XM == X_ATTN) {
    // every block merges the whole attention output: fewer, fatter blocks
    // (same waves in total) cut that re-read
    return launch_inst<KS, KS * (kAttnMergeWaves / KS), XM, XP, EP, PAIR, 1>(a, st);
  } else {
    return launch_inst<KS, nwb_of<KS, XM>(), XM, XP, EP, PAIR, 1>(a, st);
  }
}

template <int KS, int XM, int XP, int EP>
int launch_group_inst(const GemvGroupArgs& G, int count, hipStream_t stream) {
  constexpr int NWB = KS == 1 ? kGroupWaves : nwb_of<KS, XM>(), TEAMS = NWB / KS;
  const int NP = G.a.rows / 2;
  const int blocks = (NP + TEAMS * kGroupU - 1) / (TEAMS * kGroupU);
  hipLaunchKernelGGL((gemv_group_kernel<KS, NWB, XM, XP, EP>), dim3(blocks, G.a.batch, count), dim3(NWB * 64), 0,
                     stream, G);
  return check_launch();
}

template <int KS>
int dispatch_group_k(const GemvGroupArgs& G, int count, int xm, int xp, int ep, hipStream_t st) {
  if (xm == X_F16) return ep == EP_F16 ? launch_group_inst<KS, X_F16, 1, EP_F16>(G, count, st)
                                       : launch_group_inst<KS, X_F16, 1, EP_F32>(G, count, st);
  if (xm == X_F32 && xp == 1) return ep == EP_F16 ? launch_group_inst<KS, X_F32, 1, EP_F16>(G, count, st)
                                                  : launch_group_inst<KS, X_F32, 1, EP_F32>(G, count, st);
  if (xm == X_F32 && xp == 2) return ep == EP_F16 ? launch_group_inst<KS, X_F32, 2, EP_F16>(G, count, st)
                                                  : launch_group_inst<KS, X_F32, 2, EP_F32>(G, count, st);
  return Q4D_ERR_SHAPE;
}

template <int KS>
int dispatch_k(const GemvArgs& a, int xm, int xp, int ep, bool pair, hipStream_t st) {
  // primitive linear: fp16 / fp32 in, fp16 / fp32 out
  if (!pair && (ep == EP_F16 || ep == EP_F32)) {
    if (xm == X_F16) return ep == EP_F16 ? launch_sel<KS, X_F16, 1, EP_F16, false>(a, st)
                                         : launch_sel<KS, X_F16, 1, EP_F32, false>(a, st);
    if (xm == X_F32 && xp == 1) return ep == EP_F16 ? launch_sel<KS, X_F32, 1, EP_F16, false>(a, st)
                                                    : launch_sel<KS, X_F32, 1, EP_F32, false>(a, st);
    if (xm == X_F32 && xp == 2) return ep == EP_F16 ? launch_sel<KS, X_F32, 2, EP_F16, false>(a, st)
                                                    : launch_sel<KS, X_F32, 2, EP_F32, false>(a, st);
  }
  if constexpr (KS == 1) {
    if (xm == X_RMS && ep == EP_F32 && !pair)
      return xp == 2 ? launch_sel<1, X_RMS, 2, EP_F32, false>(a, st) : launch_sel<1, X_RMS, 1, EP_F32, false>(a, st);
    if (xm == X_EMB && ep == EP_F32 && !pair)
      return xp == 2 ? launch_sel<1, X_EMB, 2, EP_F32, false>(a, st) : launch_sel<1, X_EMB, 1, EP_F32, false>(a, st);
    if (xm == X_RMS && ep == EP_SWIGLU && pair)
      return xp == 2 ? launch_sel<1, X_RMS, 2, EP_SWIGLU, true>(a, st)
                     : launch_sel<1, X_RMS, 1, EP_SWIGLU, true>(a, st);
    if (xm == X_RMS && ep == EP_ARGMAX && !pair)
      return xp == 2 ? launch_sel<1, X_RMS, 2, EP_ARGMAX, false>(a, st)
                     : launch_sel<1, X_RMS, 1, EP_ARGMAX, false>(a, st);
  } else {
    if (xm == X_F32 && ep == EP_RESID && !pair)
      return xp == 2 ? launch_sel<KS, X_F32, 2, EP_RESID, false>(a, st)
                     : launch_sel<KS, X_F32, 1, EP_RESID, false>(a, st);
    if (xm == X_ATTN && ep == EP_RESID && !pair)
      return xp == 2 ? launch_sel<KS, X_ATTN, 2, EP_RESID, false>(a, st)
                     : launch_sel<KS, X_ATTN, 1, EP_RESID, false>(a, st);
  }
  return Q4D_ERR_SHAPE;
}

}  // namespace

// Validates geometry and launches.  fp32 activations enter the GEMV as fp16
// hi + lo pairs when xp == 2, rounded to fp16 when xp == 1.
int launch_gemv_xp(const GemvArgs& a, int xm, int xp, int ep, bool pair, hipStream_t st) {
  if (a.cols != 1024 && a.cols != 2048 && a.cols != 3072) return Q4D_ERR_SHAPE;
  if (a.nseg < 1 || a.nseg > 3 || a.rows <= 0 || (a.rows % 2) || a.batch <= 0 || a.batch > 65535)
    return Q4D_ERR_SHAPE;
  // buffer resources hold 32-bit byte counts
  if ((long long)a.rows * (a.cols / 2) >= (1ll << 31)) return Q4D_ERR_SHAPE;
  if (pair) {
    if (a.cols != 1024 || a.nseg != 2) return Q4D_ERR_SHAPE;
  } else {
    for (int i = 0; i < a.nseg; ++i)
      if (a.seg_end[i] % 2 || (i > 0 && a.seg_end[i] < a.seg_end[i - 1])) return Q4D_ERR_SHAPE;
    if (a.seg_end[a.nseg - 1] != a.rows) return Q4D_ERR_SHAPE;
  }
  for (int i = 0; i < a.nseg; ++i) {
    if (!a.w[i] || !a.s[i]) return Q4D_ERR_NULL;
    if (!aligned(a.w[i], 16) || !aligned(a.s[i], 4)) return Q4D_ERR_BAD_ADDR;
  }
  if (xm == X_ATTN) {
    if (!a.part_ml || !a.part_acc || !a.positions || a.nsplit_max <= 0 || a.attn_chunk <= 0) return Q4D_ERR_NULL;
    if (a.cols % 128 || !aligned(a.part_acc, 16) || !aligned(a.part_ml, 8)) return Q4D_ERR_SHAPE;
  } else if (xm == X_EMB) {
    if (!a.emb_token || !a.emb_w || !a.emb_s || !a.emb_out || a.emb_vocab <= 0 || a.cols != 1024) return Q4D_ERR_NULL;
    if (!aligned(a.emb_w, 2) || !aligned(a.emb_s, 2) || !aligned(a.emb_out, 16)) return Q4D_ERR_BAD_ADDR;
  } else if (!a.x) {
    return Q4D_ERR_NULL;
  }
  if (!a.y && ep != EP_ARGMAX) return Q4D_ERR_NULL;
  if (xm != X_ATTN && xm != X_EMB && !aligned(a.x, 16)) return Q4D_ERR_BAD_ADDR;
  if ((xm == X_RMS || xm == X_EMB) && (!a.gamma || !aligned(a.gamma, 16))) return Q4D_ERR_NULL;
  if (a.adv_tokens && (ep != EP_ARGMAX || !a.adv_positions || (a.hist_tokens && !a.hist_count))) return Q4D_ERR_NULL;
  if (ep == EP_RESID && !a.resid) return Q4D_ERR_NULL;
  if (ep == EP_ARGMAX && (!a.lm_hand || !a.out_token || !a.out_score || a.batch != 1))
    return Q4D_ERR_NULL;
  if (ep == EP_ARGMAX && (!aligned(a.lm_hand, 256) || a.nseg != 1)) return Q4D_ERR_BAD_ADDR;
  if ((a.x_parts || a.x_out) && (ep != EP_ARGMAX || xm != X_RMS || a.cols != 1024 || !a.x_parts)) return Q4D_ERR_SHAPE;
  if ((a.x_parts && !aligned(a.x_parts, 16)) || (a.x_out && !aligned(a.x_out, 16))) return Q4D_ERR_BAD_ADDR;
  if (xm == X_F16 && xp != 1) return Q4D_ERR_DTYPE;
  // unused segments: empty ranges on segment 0's memory, never selected
  GemvArgs b = a;
  if (pair) {
    b.seg_end[0] = b.rows;
    b.seg_end[1] = b.rows;
  }
  for (int i = b.nseg; i < 3; ++i) {
    b.w[i] = b.w[0];
    b.s[i] = b.s[0];
    b.seg_end[i] = b.seg_end[i - 1];
  }
  switch (a.cols) {
    case 1024: return dispatch_k<1>(b, xm, xp, ep, pair, st);
    case 2048: return dispatch_k<2>(b, xm, xp, ep, pair, st);
    default: return dispatch_k<3>(b, xm, xp, ep, pair, st);
  }
}

int launch_gemv_group(int rows, int cols, int batch, const uint8_t* const* w, const uint16_t* const* s,
                      const void* const* x, void* const* y, int count, int xm, int xp, int ep, hipStream_t st) {
  if (cols != 1024 && cols != 2048 && cols != 3072) return Q4D_ERR_SHAPE;
  if (rows <= 0 || (rows % 2) || batch <= 0 || batch > 65535 || count <= 0) return Q4D_ERR_SHAPE;
  if ((long long)rows * (cols / 2) >= (1ll << 31)) return Q4D_ERR_SHAPE;  // 32-bit buffer sizes
  if (!(xm == X_F16 && xp == 1) && !(xm == X_F32 && (xp == 1 || xp == 2))) return Q4D_ERR_DTYPE;
  if (ep != EP_F16 && ep != EP_F32) return Q4D_ERR_DTYPE;
  for (int i = 0; i < count; ++i) {
    if (!w[i] || !s[i] || !x[i] || !y[i]) return Q4D_ERR_NULL;
    if (!aligned(w[i], 16) || !aligned(s[i], 4) || !aligned(x[i], 16)) return Q4D_ERR_BAD_ADDR;
  }
  GemvGroupArgs G;
  memset(&G, 0, sizeof(G));
  G.a.rows = rows;
  G.a.cols = cols;
  G.a.batch = batch;
  G.a.nseg = 1;
  G.a.seg_end[0] = G.a.seg_end[1] = G.a.seg_end[2] = rows;  // segments 1, 2 empty
  for (int i0 = 0; i0 < count; i0 += kGemvGroupMax) {
    const int n = count - i0 < kGemvGroupMax ? count - i0 : kGemvGroupMax;
    for (int k = 0; k < kGemvGroupMax; ++k) {
      const int i = i0 + (k < n ? k : 0);  // unused slots repeat the first matrix, never read
      G.w[k] = w[i];
      G.s[k] = s[i];
      G.x[k] = x[i];
      G.y[k] = y[i];
    }
    int rc;
    switch (cols) {
      case 1024: rc = dispatch_group_k<1>(G, n, xm, xp, ep, st); break;
      case 2048: rc = dispatch_group_k<2>(G, n, xm, xp, ep, st); break;
      default: rc = dispatch_group_k<3>(G, n, xm, xp, ep, st); break;
    }
    if (rc) return rc;
  }
  return Q4D_OK;
}

int launch_gemv(const GemvArgs& a, int xmode, int epmode, bool pair, hipStream_t stream) {
  return launch_gemv_xp(a, xmode, xmode == X_F16 ? 1 : 2, epmode, pair, stream);
}

}  // namespace q4d
