// Fixed-point (RTL-exact) decode layer on gfx950: the integer arithmetic of the
// reference's FPGA datapath, bit for bit
// (Qwen3-0.6B-Base/python_each_module/56_export_persistent_multitoken_layer_golden.py:468-561
// and the stage exporters it loads).
//
// Exactness: every sum is an integer sum, so it is exact in any order once each
// partial fits its register: a Q4 GEMV lane partial (16 products of |x| <= 2^23
// and |q| <= 8) fits int32; a scaled partial, a norm product x * inv * gamma
// (< 2^62), a score q . k (< 2^53) and a value sum (sum_p p <= 2^16, so < 2^39)
// fit int64; the Q0.31 score scale is applied as hi * s + ((lo * s) >> 31) with
// raw = hi * 2^31 + lo, which equals (raw * s) >> 31 exactly.  Integer square
// roots start from the double-precision root and are corrected until
// r^2 <= v < (r + 1)^2; divisions are 64-bit integer divisions.
//
// Kernels of one layer (batch 1, five launches like the float path):
//   fx_gemv<NORM, Q12>     input RMSNorm in every block's prologue, q|k|v   -> qkv
//   fx_attn<FULL>          q/k RMSNorm, RoPE, K/V append, scores, LUT softmax,
//                          value sums; one 1024-thread block per query head -> attn
//   fx_gemv<LOAD, RESID>   o_proj, post = sat24(hidden + (o >> 2))         -> post
//   fx_gemv<NORM, SILU>    post RMSNorm, gate and up rows of the same index,
//                          sigmoid-LUT SiLU times up                         -> mlp
//   fx_gemv<LOAD, RESID>   down_proj, out = sat24(post + (down >> 2))      -> hidden_out
// and for a token: fx_embed, the layers, fx_gemv<NORM, LOGITS> over the tied
// table (one (score, row) per block) and fx_argmax over the block results.
#include <limits.h>
#include <math.h>
#include <string.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

namespace {

constexpr int kFxMaxCtx = 4096;  // positions one attention block keeps in LDS
constexpr int kFxExpLut = 257;
constexpr int kFxSigLut = 1025;
constexpr int kFxRowsLm = 8;     // rows per wave of the LM-head scan (32 per block)
constexpr int kFxLmRowsPerBlock = 4 * kFxRowsLm;

typedef int i32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- host tables
void fx_tables_host(int32_t* e, int32_t* s) {
  for (int i = 0; i < kFxExpLut; ++i) e[i] = (int32_t)nearbyint(exp(-(double)i / 16.0) * 1048576.0);
  for (int i = 0; i < kFxSigLut; ++i) {
    const double x = -8.0 + (double)i / 64.0;
    double r = nearbyint(1.0 / (1.0 + exp(-x)) * 65536.0);
    r = r < 0.0 ? 0.0 : (r > 65535.0 ? 65535.0 : r);
    s[i] = (int32_t)r;
  }
}

struct FxTables {
  int32_t e[kFxExpLut], s[kFxSigLut];
  FxTables() { fx_tables_host(e, s); }
};

const FxTables& fx_tables() {
  static const FxTables t;  // built once, thread-safe
  return t;
}

// ---------------------------------------------------------------- device helpers
__device__ __forceinline__ long long shfl_xor_ll(long long v, int m) {
  const int lo = __shfl_xor((int)(unsigned long long)v, m, kWave);
  const int hi = __shfl_xor((int)((unsigned long long)v >> 32), m, kWave);
  return (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

__device__ __forceinline__ long long wave_sum_ll(long long v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_ll(v, m);
  return v;
}

__device__ __forceinline__ long long wave_max_ll(long long v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const long long o = shfl_xor_ll(v, m);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ int sat24(long long v, int& nsat) {
  const long long lo = -(1LL << 23), hi = (1LL << 23) - 1;
  nsat += (v < lo) | (v > hi);
  return (int)(v < lo ? lo : (v > hi ? hi : v));
}

__device__ __forceinline__ unsigned long long isqrt_u64(unsigned long long v) {
  unsigned long long r = (unsigned long long)sqrt((double)v);
  while (r * r > v) --r;
  while ((r + 1) * (r + 1) <= v) ++r;
  return r;
}

// RMSNorm kinds: 0 = hidden (Q14.10 in; 17_...:31-47), 1 = head (Q12.12 in; 22_...:41-57).
struct NormParams {
  long long sum, mean, rad, rms, inv;
};

__device__ __forceinline__ NormParams norm_params(long long sum_sq, int kind) {
  NormParams p;
  p.sum = sum_sq;
  p.mean = sum_sq >> (kind ? 7 : 10);
  p.rad = p.mean + (kind ? 17 : 1);
  const unsigned long long r = isqrt_u64((unsigned long long)p.rad);
  p.rms = (long long)r;
  const unsigned long long num = 1ull << (kind ? 28 : 26);
  const unsigned long long q = r ? num / r : 0xFFFFFFull;
  p.inv = (long long)(q > 0xFFFFFFull ? 0xFFFFFFull : q);
  return p;
}

__device__ __forceinline__ int norm_apply(int x, int gamma, long long inv, int kind, int& nsat) {
  return sat24(((long long)x * inv * (long long)gamma) >> (kind ? 23 : 21), nsat);
}

// floor(a / b) for a < 2^53, 0 < b < 2^53: double quotient, corrected to exact.
__device__ __forceinline__ unsigned long long udiv_small(unsigned long long a, unsigned long long b) {
  unsigned long long q = (unsigned long long)((double)a / (double)b);
  while (q * b > a) --q;
  while ((q + 1) * b <= a) ++q;
  return q;
}

// Saturation counters: kFxStripes copies of the Q4D_FX_COUNTS words, 256 bytes apart, so
// that the waves of a saturating launch spread their atomics over many L2 channels
// instead of queueing on one word (the host sums the stripes).
constexpr int kFxStripes = 64;
constexpr int kFxStripeWords = 64;

// Adds the wave's saturation count to its stripe of counter `slot`: one atomic per wave,
// none when no lane saturated.  Called by every lane of a wave (wave-uniform control flow).
__device__ __forceinline__ void count(int32_t* counts, int slot, int n) {
  if (!counts || __ballot(n != 0) == 0) return;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) n += __shfl_xor(n, m, kWave);
  const int stripe = (int)((blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) & (kFxStripes - 1));
  if ((threadIdx.x & 63) == 0) atomicAdd(counts + stripe * kFxStripeWords + slot, n);
}

// sum_{i<16} x_i * q_i for the 16 columns of an 8-byte weight word pair (column i in
// bits 4i..4i+3, signed).  |x| <= 2^23: the sum fits int32.
// x is a saturated 24-bit value and q a 4-bit code, so the 24-bit multiply is exact.
__device__ __forceinline__ int dot16(uint32_t w0, uint32_t w1, const int (&x)[16]) {
  int s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += __mul24(x[i], ((int)(w0 << (28 - 4 * i))) >> 28);
#pragma unroll
  for (int i = 0; i < 8; ++i) s += __mul24(x[8 + i], ((int)(w1 << (28 - 4 * i))) >> 28);
  return s;
}

// ---------------------------------------------------------------- Q4 GEMV with prologue / epilogue
enum { FX_PRO_LOAD = 0, FX_PRO_NORM = 1 };
enum { FX_EPI_Q12 = 0, FX_EPI_RESID = 1, FX_EPI_SILU = 2, FX_EPI_LOGITS = 3 };

struct FxGemv {
  const uint8_t* w0;
  const uint8_t* w1;
  const uint8_t* w2;
  const uint16_t* s0;
  const uint16_t* s1;
  const uint16_t* s2;
  int e0, e1;  // rows [0, e0) from matrix 0, [e0, e1) from 1, the rest from 2
  int rows;    // output rows (index pairs for FX_EPI_SILU: gate = matrix 0, up = matrix 1)
  int K;
  const int32_t* x;       // Q14.10 hidden (NORM) or Q12.12 activations (LOAD), [K]
  const int16_t* gamma;   // NORM
  int32_t* y;             // Q12 / RESID / SILU output
  const int32_t* resid;   // RESID
  const int32_t* lut;     // SILU: sigmoid LUT [1025]
  int64_t* logits;        // LOGITS (may be null)
  int64_t* part_score;    // LOGITS: per-block best
  int32_t* part_idx;
  int32_t* counts;        // [Q4D_FX_COUNTS] or null
  int slot_norm, slot_a, slot_b, slot_c, slot_d;
};

template <int KC, int R, int PRO, int EPI>
__global__ __launch_bounds__(256) void fx_gemv_kernel(const FxGemv a) {
  // activations, 16 per 20-word LDS line: lane l's 16 columns sit at 20 l + 1280 j, so one
  // ds_read_b128 per lane covers all 64 banks once per 16 lanes
  __shared__ __align__(16) int xs[KC * 1280];
  __shared__ long long red[4];
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  // 1. activation loads first, then every weight / scale load of this wave: the weights
  //    stream in while the prologue runs (its barriers wait on LDS only)
  constexpr int NX = PRO == FX_PRO_NORM ? 4 : KC * 4;
  int xv[NX];
#pragma unroll
  for (int i = 0; i < NX; ++i) xv[i] = a.x[t + 256 * i];
  __builtin_amdgcn_sched_barrier(0);

  constexpr int ND = EPI == FX_EPI_SILU ? 2 * R : R;
  const int row0 = (blockIdx.x * 4 + wid) * R;
  const size_t wpitch = (size_t)a.K / 2, spitch = (size_t)a.K / 64;
  uint32_t wlo[ND][KC], whi[ND][KC], sv[ND][KC];
#pragma unroll
  for (int r = 0; r < ND; ++r) {
    int row = EPI == FX_EPI_SILU ? row0 + (r >> 1) : row0 + r;
    row = row < a.rows ? row : a.rows - 1;  // clamped: loads stay in bounds, stores are skipped
    const uint8_t* wb;
    const uint16_t* sb;
    int local;
    if (EPI == FX_EPI_SILU) {
      wb = (r & 1) ? a.w1 : a.w0;
      sb = (r & 1) ? a.s1 : a.s0;
      local = row;
    } else {
      const bool m0 = row < a.e0, m1 = row < a.e1;
      wb = m0 ? a.w0 : (m1 ? a.w1 : a.w2);
      sb = m0 ? a.s0 : (m1 ? a.s1 : a.s2);
      local = m0 ? row : (m1 ? row - a.e0 : row - a.e1);
    }
    const uint8_t* wr = wb + (size_t)local * wpitch + 8 * lane;
    const uint16_t* sr = sb + (size_t)local * spitch + (lane >> 2);
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const u32x2 v = *reinterpret_cast<const u32x2*>(wr + 512 * j);
      wlo[r][j] = v.x;
      whi[r][j] = v.y;
      sv[r][j] = sr[16 * j];
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. prologue: the activations (normalised for NORM) into LDS
  if constexpr (PRO == FX_PRO_NORM) {
    static_assert(KC == 1, "the norm prologue covers the 1024-wide hidden state");
    long long ss = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += (long long)xv[i] * xv[i];
    ss = wave_sum_ll(ss);
    if (lane == 0) red[wid] = ss;
    block_sync_lds();
    const NormParams p = norm_params(red[0] + red[1] + red[2] + red[3], 0);
    int nsat = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = t + 256 * i;
      xs[c + (c >> 4) * 4] = norm_apply(xv[i], a.gamma[c], p.inv, 0, nsat);
    }
    if (blockIdx.x == 0) count(a.counts, a.slot_norm, nsat);
  } else {
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int c = t + 256 * i;
      xs[c + (c >> 4) * 4] = xv[i];
    }
  }
  block_sync_lds();

  long long acc[ND];
#pragma unroll
  for (int r = 0; r < ND; ++r) acc[r] = 0;
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    int xr[16];
    const i32x4* xp = reinterpret_cast<const i32x4*>(xs + 20 * lane + 1280 * j);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const i32x4 q = xp[v];
      xr[4 * v + 0] = q.x;
      xr[4 * v + 1] = q.y;
      xr[4 * v + 2] = q.z;
      xr[4 * v + 3] = q.w;
    }
#pragma unroll
    for (int r = 0; r < ND; ++r)
      acc[r] += (long long)dot16(wlo[r][j], whi[r][j], xr) * (long long)sv[r][j];
  }
#pragma unroll
  for (int r = 0; r < ND; ++r) acc[r] = wave_sum_ll(acc[r]);

  // epilogue: every lane holds every row sum; lane r finishes row r
  if constexpr (EPI == FX_EPI_LOGITS) {
    __shared__ long long bs[4];
    __shared__ int bi[4];
    long long best = LLONG_MIN;
    int besti = INT_MAX;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row < a.rows) {
        if (a.logits && lane == r) a.logits[row] = acc[r];
        if (acc[r] > best || besti == INT_MAX) {  // ascending rows: strict > keeps the first
          best = acc[r];
          besti = row;
        }
      }
    }
    if (lane == 0) {
      bs[wid] = best;
      bi[wid] = besti;
    }
    __syncthreads();
    if (t == 0) {
#pragma unroll
      for (int k = 1; k < 4; ++k)
        if (bi[k] != INT_MAX && (bs[k] > best || besti == INT_MAX)) {
          best = bs[k];
          besti = bi[k];
        }
      a.part_score[blockIdx.x] = best;
      a.part_idx[blockIdx.x] = besti;
    }
  } else {
    int n0 = 0, n1 = 0, n2 = 0, n3 = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (lane == r && row < a.rows) {
        if constexpr (EPI == FX_EPI_Q12) {
          a.y[row] = sat24(acc[r] >> 14, n0);
        } else if constexpr (EPI == FX_EPI_RESID) {
          const int v = sat24(acc[r] >> 14, n0);
          a.y[row] = sat24((long long)a.resid[row] + (v >> 2), n1);
        } else {  // SILU: gate row, up row
          const int g = sat24(acc[2 * r] >> 14, n0);
          const int u = sat24(acc[2 * r + 1] >> 14, n1);
          const int gc = g < -32768 ? -32768 : (g > 32768 ? 32768 : g);
          int idx = (gc + 32768 + 32) >> 6;
          idx = idx < 0 ? 0 : (idx > kFxSigLut - 1 ? kFxSigLut - 1 : idx);
          const int silu = sat24(((long long)g * a.lut[idx]) >> 16, n2);
          a.y[row] = sat24(((long long)silu * u) >> 12, n3);
        }
      }
    }
    count(a.counts, a.slot_a, n0);
    count(a.counts, a.slot_b, n1);
    count(a.counts, a.slot_c, n2);
    count(a.counts, a.slot_d, n3);
  }
}

// ---------------------------------------------------------------- attention
// Two launches per layer:
//   fx_attn_scores, (chunk, head) blocks of 256 threads, CH positions per chunk: q/k norm +
//     RoPE (the chunk holding the new position of the first q head of a kv group appends the
//     K/V row), the chunk's scaled scores and their maximum to the workspace.
//   fx_attn_value, (32 dims, head) blocks of 256 threads: the head's integer softmax over
//     all T positions (global maximum of the chunk maxima, LUT exp values, their sum,
//     floor((e << 16) / sum)) into LDS, then sum_p prob_p * v_p for the block's 32 dims,
//     exact in int64, and sat24(sum >> 16).  Every block of a head recomputes the same
//     softmax (T scores and at most 16 maxima), which costs less than handing it over.
// The kernel boundary orders the workspace traffic; no counters or device-scope atomics.
constexpr int kFxMaxChunks = 16;

struct FxAttn {
  const int32_t* qkv;       // FULL: q|k|v projections of this token
  const int32_t* q_in;      // !FULL: q after norm and RoPE [qh, 128]
  const int16_t* q_gamma;
  const int16_t* k_gamma;
  const int16_t* cos;       // [max_ctx, 128] Q1.15
  const int16_t* sin;
  const int32_t* position;  // FULL
  int cache_length;         // !FULL
  int32_t* kc;              // K plane of the layer [kvh][max_ctx][128]
  int32_t* vc;              // V plane
  int max_ctx, qh, kvh, ch;
  int score_scale;
  const int32_t* exp_lut;
  int32_t* out;             // [qh, 128]
  int64_t* sc;              // workspace: scaled scores [qh][max_ctx]
  int64_t* cmax;            // workspace: chunk maxima [qh][kFxMaxChunks]
  int64_t* raw;             // debug outputs [qh, T] (may be null)
  int64_t* scaled;
  int32_t* lut_index;
  int32_t* prob;
  int32_t* counts;
  int32_t* status;
};

// Position of this step; false (nothing to do) for an out-of-range device position.
template <bool FULL>
__device__ __forceinline__ bool fx_attn_pos(const FxAttn& a, int& pos) {
  if constexpr (FULL) {
    pos = *a.position;
    if (pos < 0 || pos >= a.max_ctx) {  // uniform over the grid: nothing is written
      if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0 && a.status)
        atomicOr(a.status, Q4D_STATUS_BAD_POSITION);
      return false;
    }
  } else {
    pos = a.cache_length - 1;
  }
  return true;
}

template <bool FULL>
__global__ __launch_bounds__(256) void fx_attn_scores_kernel(const FxAttn a) {
  __shared__ int qn[128], kn[128], qr[128], kr[128];
  __shared__ long long wred[4];
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int c = blockIdx.x, h = blockIdx.y, rep = a.qh / a.kvh, g = h / rep;
  int pos;
  if (!fx_attn_pos<FULL>(a, pos)) return;
  const int T = pos + 1, p_begin = c * a.ch;
  if (p_begin >= T) return;  // chunk past the context
  const int p_end = min(T, p_begin + a.ch);

  // loads in the order they are consumed (completion is counted in issue order): this
  // token's q / k / v rows and RoPE row, then the chunk's first two passes of K rows
  const int qd = a.qh * 128, kd = a.kvh * 128, d = t & 127;
  const bool app = FULL && c == pos / a.ch && h % rep == 0;  // one block per kv head appends
  int v = 0, vrow = 0, cs = 0, sn = 0;
  if constexpr (FULL) {
    cs = a.cos[(size_t)pos * 128 + d];
    sn = a.sin[(size_t)pos * 128 + d];
    v = t < 128 ? a.qkv[h * 128 + d] : a.qkv[qd + g * 128 + d];
    vrow = app && t < 128 ? a.qkv[qd + kd + g * 128 + d] : 0;
  } else {
    v = t < 128 ? a.q_in[h * 128 + t] : 0;
  }
  const int sub = lane & 7, grp = (wid << 3) | (lane >> 3);
  const int32_t* kbase = a.kc + (size_t)g * a.max_ctx * 128 + 16 * sub;
  i32x4 k4[2][4];
  auto load_k = [&](int pp) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = pp + 32 * u + grp;
      const int pc = p < p_end ? p : p_end - 1;  // clamped: in bounds, result unused
      const i32x4* kp = reinterpret_cast<const i32x4*>(kbase + (size_t)pc * 128);
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) k4[u][v4] = kp[v4];
    }
  };
  __builtin_amdgcn_sched_barrier(0);
  load_k(p_begin);
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (FULL) {
    // q/k RMSNorm per head (22_...:127-182), RoPE (22_...:185-212), K/V append
    long long ss = wave_sum_ll((long long)v * v);
    if (lane == 0) wred[wid] = ss;
    block_sync_lds();
    const NormParams p = norm_params(t < 128 ? wred[0] + wred[1] : wred[2] + wred[3], 1);
    int nsat = 0;
    const int y = norm_apply(v, (t < 128 ? a.q_gamma : a.k_gamma)[d], p.inv, 1, nsat);
    if (t < 128) qn[d] = y;
    else kn[d] = y;
    const bool counter_block = c == 0 && (t < 128 || h % rep == 0);  // each head counted once
    if (counter_block) count(a.counts, Q4D_FX_SAT_QK_NORM, nsat);
    block_sync_lds();
    nsat = 0;
    const int* src = t < 128 ? qn : kn;
    const int rot = d < 64 ? -src[d + 64] : src[d - 64];
    const int r = sat24(((long long)src[d] * cs + (long long)rot * sn) >> 15, nsat);
    if (t < 128) {
      qr[d] = r;
      if (app) a.vc[((size_t)g * a.max_ctx + pos) * 128 + d] = vrow;
    } else {
      kr[d] = r;
      if (app) a.kc[((size_t)g * a.max_ctx + pos) * 128 + d] = r;
    }
    if (counter_block) count(a.counts, Q4D_FX_SAT_ROPE, nsat);
  } else {
    if (t < 128) qr[t] = v;
  }
  block_sync_lds();

  // scores of this chunk: 8 lanes per position (16 dims each), 32 positions per pass
  int qreg[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) qreg[i] = qr[16 * sub + i];
  long long cm = LLONG_MIN;
  auto score_round = [&](int pp) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = pp + 32 * u + grp;
      long long dot = 0;
      if (FULL && p == pos) {  // this token's K from LDS: the cache row may not be written yet
#pragma unroll
        for (int i = 0; i < 16; ++i) dot += (long long)qreg[i] * kr[16 * sub + i];
      } else {
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          const i32x4 kk = k4[u][v4];
          dot += (long long)qreg[4 * v4 + 0] * kk.x + (long long)qreg[4 * v4 + 1] * kk.y +
                 (long long)qreg[4 * v4 + 2] * kk.z + (long long)qreg[4 * v4 + 3] * kk.w;
        }
      }
      dot += shfl_xor_ll(dot, 1);
      dot += shfl_xor_ll(dot, 2);
      dot += shfl_xor_ll(dot, 4);
      if (p < p_end && sub == 0) {
        const long long hi = dot >> 31, lo = dot & 0x7FFFFFFFLL;
        const long long sv = hi * (long long)a.score_scale + ((lo * (long long)a.score_scale) >> 31);
        a.sc[(size_t)h * a.max_ctx + p] = sv;
        cm = sv > cm ? sv : cm;
        if (a.raw) a.raw[(size_t)h * T + p] = dot;
        if (a.scaled) a.scaled[(size_t)h * T + p] = sv;
      }
    }
  };
  score_round(p_begin);
  for (int pp = p_begin + 64; pp < p_end; pp += 64) {
    load_k(pp);
    score_round(pp);
  }
  cm = wave_max_ll(cm);
  if (lane == 0) wred[wid] = cm;
  block_sync_lds();
  if (t == 0) {
    long long m = wred[0];
#pragma unroll
    for (int k = 1; k < 4; ++k) m = wred[k] > m ? wred[k] : m;
    a.cmax[h * kFxMaxChunks + c] = m;
  }
}

template <bool FULL>
__global__ __launch_bounds__(256) void fx_attn_value_kernel(const FxAttn a) {
  __shared__ int prs[kFxMaxCtx];  // probabilities of the head
  __shared__ int lut[kFxExpLut];
  __shared__ long long wred[4];
  __shared__ long long vred[4][32];
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int db = blockIdx.x, h = blockIdx.y, rep = a.qh / a.kvh, g = h / rep;
  int pos;
  if (!fx_attn_pos<FULL>(a, pos)) return;
  const int T = pos + 1, nct = (T + a.ch - 1) / a.ch;

  // loads in the order they are consumed: chunk maxima, scores, LUT, then the first round
  // of V rows (thread = 4 dims x position residue mod 32)
  long long cmv[kFxMaxChunks];
#pragma unroll
  for (int i = 0; i < kFxMaxChunks; ++i) cmv[i] = a.cmax[h * kFxMaxChunks + (i < nct ? i : nct - 1)];
  constexpr int NP = kFxMaxCtx / 256;  // score positions per thread
  long long sv[NP];
#pragma unroll
  for (int k = 0; k < NP; ++k) {  // clamped: slots past the context re-read the last score
    const int p = t + 256 * k;
    sv[k] = a.sc[(size_t)h * a.max_ctx + (p < T ? p : T - 1)];
  }
  for (int i = t; i < kFxExpLut; i += 256) lut[i] = a.exp_lut[i];
  const int dq = t & 7, j = t >> 3;
  const int32_t* vbase = a.vc + (size_t)g * a.max_ctx * 128 + 32 * db + 4 * dq;
  i32x4 v4[8];
  auto load_v = [&](int p0) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = p0 + 32 * u;
      v4[u] = *reinterpret_cast<const i32x4*>(vbase + (size_t)(p < T ? p : T - 1) * 128);
    }
  };
  __builtin_amdgcn_sched_barrier(0);
  load_v(j);
  __builtin_amdgcn_sched_barrier(0);

  // softmax (46_...:96-121)
  long long m = cmv[0];
#pragma unroll
  for (int i = 1; i < kFxMaxChunks; ++i) m = cmv[i] > m ? cmv[i] : m;
  block_sync_lds();  // LUT in LDS
  int e[NP];
  long long se = 0;
  const bool dbg = db == 0;
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    e[k] = 0;
    if (256 * k >= T) continue;  // block-uniform: slots past the context are skipped whole
    const int p = t + 256 * k;
    const long long neg = m - sv[k];
    int idx = 0;
    if (neg > 0) {
      const long long r = (neg + (1LL << 19)) >> 20;
      idx = r > kFxExpLut - 1 ? kFxExpLut - 1 : (int)r;
    }
    e[k] = p < T ? lut[idx] : 0;
    se += e[k];
    if (dbg && a.lut_index && p < T) a.lut_index[(size_t)h * T + p] = idx;
  }
  se = wave_sum_ll(se);
  if (lane == 0) wred[wid] = se;
  block_sync_lds();
  se = wred[0] + wred[1] + wred[2] + wred[3];
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    if (256 * k >= T) break;
    const int p = t + 256 * k;
    if (p < T) {
      const int pv = (int)udiv_small((unsigned long long)e[k] << 16, (unsigned long long)se);
      prs[p] = pv;
      if (dbg && a.prob) a.prob[(size_t)h * T + p] = pv;
    }
  }
  block_sync_lds();

  // value sums (46_...:124-137) for dims 32 db + 4 dq .. + 3
  long long acc0 = 0, acc1 = 0, acc2 = 0, acc3 = 0;
  auto value_round = [&](int p0) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int p = p0 + 32 * u;
      const long long pr = p < T ? prs[p] : 0;
      acc0 += pr * v4[u].x;
      acc1 += pr * v4[u].y;
      acc2 += pr * v4[u].z;
      acc3 += pr * v4[u].w;
    }
  };
  value_round(j);
  for (int p0 = j + 256; p0 < T; p0 += 256) {
    load_v(p0);
    value_round(p0);
  }
  // the 8 residues of a wave sit in lanes dq + 8 r: reduce over r, then over the 4 waves
#pragma unroll
  for (int m2 = 8; m2 <= 32; m2 <<= 1) {
    acc0 += shfl_xor_ll(acc0, m2);
    acc1 += shfl_xor_ll(acc1, m2);
    acc2 += shfl_xor_ll(acc2, m2);
    acc3 += shfl_xor_ll(acc3, m2);
  }
  if (lane < 8) {
    vred[wid][4 * dq + 0] = acc0;
    vred[wid][4 * dq + 1] = acc1;
    vred[wid][4 * dq + 2] = acc2;
    vred[wid][4 * dq + 3] = acc3;
  }
  block_sync_lds();
  if (t < 64) {  // one full wave: the saturation count below is wave-uniform
    int nsat = 0;
    if (t < 32) {
      const long long sum = vred[0][t] + vred[1][t] + vred[2][t] + vred[3][t];
      a.out[h * 128 + 32 * db + t] = sat24(sum >> 16, nsat);
    }
    count(a.counts, Q4D_FX_SAT_ATTENTION, nsat);
  }
}

struct FxAttnLayout {
  size_t sc, cmax, total;
  int ch, nch;
};

// Chunk length: 64 positions, longer (by 32) until at most kFxMaxChunks chunks cover max_ctx.
FxAttnLayout fx_attn_layout(int qh, int max_ctx) {
  FxAttnLayout L{};
  L.ch = 64;
  while ((max_ctx + L.ch - 1) / L.ch > kFxMaxChunks) L.ch += 32;
  L.nch = (max_ctx + L.ch - 1) / L.ch;
  const size_t A = 256;
  size_t o = 0;
  L.sc = o;   o = align_up(o + (size_t)qh * max_ctx * 8, A);
  L.cmax = o; o = align_up(o + (size_t)qh * kFxMaxChunks * 8, A);
  L.total = o;
  return L;
}

void fx_attn_bind(FxAttn& a, void* ws, const FxAttnLayout& L) {
  a.sc = ws_ptr<int64_t>(ws, L.sc);
  a.cmax = ws_ptr<int64_t>(ws, L.cmax);
  a.ch = L.ch;
}

template <bool FULL>
int fx_launch_attention(const FxAttn& a, int nch, hipStream_t st) {
  hipLaunchKernelGGL(fx_attn_scores_kernel<FULL>, dim3(nch, a.qh), dim3(256), 0, st, a);
  int rc = check_launch();
  if (rc) return rc;
  hipLaunchKernelGGL(fx_attn_value_kernel<FULL>, dim3(4, a.qh), dim3(256), 0, st, a);
  return check_launch();
}

// ---------------------------------------------------------------- small stage kernels
__global__ __launch_bounds__(256) void fx_rmsnorm_kernel(const int32_t* x, const int16_t* gamma, int dim, int kind,
                                                         int32_t* y, int64_t* stats) {
  __shared__ long long red[4];
  __shared__ int sred[4];
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int32_t* xr = x + (size_t)blockIdx.x * dim;
  long long ss = 0;
  for (int c = t; c < dim; c += 256) ss += (long long)xr[c] * xr[c];
  ss = wave_sum_ll(ss);
  if (lane == 0) red[wid] = ss;
  __syncthreads();
  const NormParams p = norm_params(red[0] + red[1] + red[2] + red[3], kind);
  int nsat = 0;
  for (int c = t; c < dim; c += 256) y[(size_t)blockIdx.x * dim + c] = norm_apply(xr[c], gamma[c], p.inv, kind, nsat);
  nsat = (int)wave_sum_ll(nsat);
  if (lane == 0) sred[wid] = nsat;
  __syncthreads();
  if (t == 0 && stats) {
    int64_t* st = stats + (size_t)blockIdx.x * 6;
    st[0] = p.sum;
    st[1] = p.mean;
    st[2] = p.rad;
    st[3] = p.rms;
    st[4] = p.inv;
    st[5] = sred[0] + sred[1] + sred[2] + sred[3];
  }
}

__global__ __launch_bounds__(128) void fx_qknorm_rope_kernel(const int32_t* q, const int32_t* k, int qh,
                                                             const int16_t* qg, const int16_t* kg,
                                                             const int16_t* cosr, const int16_t* sinr,
                                                             int32_t* q_rope, int32_t* k_rope, int32_t* q_norm,
                                                             int32_t* k_norm) {
  __shared__ long long red[2];
  __shared__ int xn[128];
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const bool isq = (int)blockIdx.x < qh;
  const int head = isq ? blockIdx.x : blockIdx.x - qh;
  const int v = (isq ? q : k)[head * 128 + t];
  const int16_t* gam = isq ? qg : kg;
  long long ss = wave_sum_ll((long long)v * v);
  if (lane == 0) red[wid] = ss;
  __syncthreads();
  const NormParams p = norm_params(red[0] + red[1], 1);
  int nsat = 0;
  const int y = gam ? norm_apply(v, gam[t], p.inv, 1, nsat) : v;  // no gamma: RoPE of the input
  xn[t] = y;
  int32_t* nout = isq ? q_norm : k_norm;
  if (nout) nout[head * 128 + t] = y;
  __syncthreads();
  const int rot = t < 64 ? -xn[t + 64] : xn[t - 64];
  const long long s = (long long)y * cosr[t] + (long long)rot * sinr[t];
  (isq ? q_rope : k_rope)[head * 128 + t] = sat24(s >> 15, nsat);
}

__global__ __launch_bounds__(256) void fx_kv_append_kernel(int32_t* kc, int32_t* vc, int kvh, int max_ctx,
                                                           const int32_t* positions, const int32_t* k,
                                                           const int32_t* v) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int pos = *positions;
  if (i >= kvh * 128 || pos < 0 || pos >= max_ctx) return;
  const int g = i >> 7, d = i & 127;
  kc[((size_t)g * max_ctx + pos) * 128 + d] = k[i];
  vc[((size_t)g * max_ctx + pos) * 128 + d] = v[i];
}

__global__ __launch_bounds__(256) void fx_silu_kernel(const int32_t* gate, const int32_t* up, int n,
                                                      const int32_t* lutg, int32_t* hidden, int32_t* lut_index,
                                                      int32_t* sigmoid, int32_t* silu_gate) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int g = gate[i];
  const int gc = g < -32768 ? -32768 : (g > 32768 ? 32768 : g);
  int idx = (gc + 32768 + 32) >> 6;
  idx = idx < 0 ? 0 : (idx > kFxSigLut - 1 ? kFxSigLut - 1 : idx);
  const int sg = lutg[idx];
  int nsat = 0;
  const int silu = sat24(((long long)g * sg) >> 16, nsat);
  hidden[i] = sat24(((long long)silu * up[i]) >> 12, nsat);
  if (lut_index) lut_index[i] = idx;
  if (sigmoid) sigmoid[i] = sg;
  if (silu_gate) silu_gate[i] = silu;
}

__global__ __launch_bounds__(256) void fx_resid_kernel(const int32_t* h, const int32_t* x, int n, int32_t* out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  int nsat = 0;
  out[i] = sat24((long long)h[i] + (x[i] >> 2), nsat);
}

// Q14.10 embedding rows (q * scale) >> 4 of the tied Q4 table (56_...:214-221).
__global__ __launch_bounds__(256) void fx_embed_kernel(const uint8_t* w, const uint16_t* s, int vocab, int cols,
                                                       const int32_t* tokens, int32_t* hidden, int32_t* status) {
  const int tok = tokens[blockIdx.x];
  if (tok < 0 || tok >= vocab) {
    if (threadIdx.x == 0 && status) atomicOr(status, Q4D_STATUS_BAD_TOKEN);
    return;
  }
  for (int c = threadIdx.x; c < cols; c += 256) {
    const int byte = w[(size_t)tok * (cols / 2) + c / 2];
    const int q = (((c & 1) ? byte >> 4 : byte) << 28) >> 28;
    hidden[(size_t)blockIdx.x * cols + c] = (q * (int)s[(size_t)tok * (cols / 64) + c / 64]) >> 4;
  }
}

// Best (score, row) over the LM-head blocks: highest score, lowest row on ties.
__global__ __launch_bounds__(1024) void fx_argmax_kernel(const int64_t* ps, const int32_t* pi, int n, int32_t* tok,
                                                         int64_t* score) {
  __shared__ long long sb[16];
  __shared__ int si[16];
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  long long bs = LLONG_MIN;
  int bi = INT_MAX;
  for (int base = 0; base < n; base += 8 * 1024) {  // eight loads in flight per thread
    long long v[8];
    int ix[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = base + t + 1024 * k;
      const int ic = i < n ? i : n - 1;
      v[k] = ps[ic];
      ix[k] = i < n ? pi[ic] : INT_MAX;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (ix[k] != INT_MAX && (v[k] > bs || (v[k] == bs && ix[k] < bi) || bi == INT_MAX)) {
        bs = v[k];
        bi = ix[k];
      }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const long long os = shfl_xor_ll(bs, m);
    const int oi = __shfl_xor(bi, m, kWave);
    if (oi != INT_MAX && (os > bs || (os == bs && oi < bi) || bi == INT_MAX)) {
      bs = os;
      bi = oi;
    }
  }
  if (lane == 0) {
    sb[wid] = bs;
    si[wid] = bi;
  }
  __syncthreads();
  if (t == 0) {
    for (int k = 1; k < 16; ++k)
      if (si[k] != INT_MAX && (sb[k] > bs || (sb[k] == bs && si[k] < bi) || bi == INT_MAX)) {
        bs = sb[k];
        bi = si[k];
      }
    *tok = bi;
    *score = bs;
  }
}

// ---------------------------------------------------------------- host side
struct FxLayout {
  size_t counts, exp_lut, sig_lut, hidden, qkv, attn, post, mlp, part_score, part_idx, attn_ws, total;
  int nparts;
  FxAttnLayout al;  // attention scratch, at attn_ws
};

FxLayout fx_layout(const q4d_model_t* m) {
  FxLayout L{};
  const size_t A = 256;
  const int qd = m->num_q_heads * m->head_dim, kd = m->num_kv_heads * m->head_dim;
  L.nparts = (m->vocab_size + kFxLmRowsPerBlock - 1) / kFxLmRowsPerBlock;
  size_t o = 0;
  L.counts = o;     o = align_up(o + kFxStripes * kFxStripeWords * 4, A);
  L.exp_lut = o;    o = align_up(o + kFxExpLut * 4, A);
  L.sig_lut = o;    o = align_up(o + kFxSigLut * 4, A);
  L.hidden = o;     o = align_up(o + (size_t)m->hidden_size * 4, A);
  L.qkv = o;        o = align_up(o + (size_t)(qd + 2 * kd) * 4, A);
  L.attn = o;       o = align_up(o + (size_t)qd * 4, A);
  L.post = o;       o = align_up(o + (size_t)m->hidden_size * 4, A);
  L.mlp = o;        o = align_up(o + (size_t)m->intermediate_size * 4, A);
  L.part_score = o; o = align_up(o + (size_t)L.nparts * 8, A);
  L.part_idx = o;   o = align_up(o + (size_t)L.nparts * 4, A);
  L.al = fx_attn_layout(m->num_q_heads, m->max_ctx);
  L.attn_ws = o;    o = align_up(o + L.al.total, A);
  L.total = o;
  return L;
}

inline hipStream_t fx_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

int fx_check_matrix(const q4d_matrix_t& w, int rows, int cols) {
  if (!w.w || !w.s) return Q4D_ERR_NULL;
  if (w.rows != rows || w.cols != cols) return Q4D_ERR_BAD_LAYER;
  if (!aligned(w.w, 16) || !aligned(w.s, 4)) return Q4D_ERR_BAD_ADDR;
  return Q4D_OK;
}

bool fx_k_ok(int k) { return k == 1024 || k == 2048 || k == 3072; }

int fx_check_model(const q4d_fixed_model_t* fm) {
  if (!fm || !fm->base || !fm->layers || !fm->final_gamma || !fm->rope_cos || !fm->rope_sin) return Q4D_ERR_NULL;
  const q4d_model_t* m = fm->base;
  if (!m->layers) return Q4D_ERR_NULL;
  if (m->hidden_size != 1024 || m->head_dim != 128 || m->num_kv_heads <= 0 || m->num_q_heads <= 0 ||
      m->num_q_heads % m->num_kv_heads)
    return Q4D_ERR_SHAPE;
  const int qd = m->num_q_heads * 128, kd = m->num_kv_heads * 128, I = m->intermediate_size;
  if (!fx_k_ok(qd) || !fx_k_ok(I) || m->num_layers <= 0 || m->vocab_size <= 0) return Q4D_ERR_SHAPE;
  if (m->max_ctx <= 0 || m->max_ctx > kFxMaxCtx) return Q4D_ERR_CONTEXT;
  if (fm->score_scale_q0_31 <= 0) return Q4D_ERR_SHAPE;
  int rc;
  if (!m->embed_tokens.w || !m->embed_tokens.s) return Q4D_ERR_NULL;
  if (m->embed_tokens.rows != m->vocab_size || m->embed_tokens.cols != 1024) return Q4D_ERR_BAD_TABLE;
  if (!aligned(m->embed_tokens.w, 16) || !aligned(m->embed_tokens.s, 4)) return Q4D_ERR_BAD_ADDR;
  for (int l = 0; l < m->num_layers; ++l) {
    const q4d_layer_t& L = m->layers[l];
    if ((rc = fx_check_matrix(L.q_proj, qd, 1024)) || (rc = fx_check_matrix(L.k_proj, kd, 1024)) ||
        (rc = fx_check_matrix(L.v_proj, kd, 1024)) || (rc = fx_check_matrix(L.o_proj, 1024, qd)) ||
        (rc = fx_check_matrix(L.gate_proj, I, 1024)) || (rc = fx_check_matrix(L.up_proj, I, 1024)) ||
        (rc = fx_check_matrix(L.down_proj, 1024, I)))
      return rc;
    const q4d_fixed_layer_t& F = fm->layers[l];
    if (!F.input_gamma || !F.post_gamma || !F.q_gamma || !F.k_gamma) return Q4D_ERR_NULL;
  }
  return Q4D_OK;
}

int fx_check_kv(const q4d_fixed_kv_t* kv, int layers, int kvh, int max_ctx) {
  if (!kv || !kv->data) return Q4D_ERR_NULL;
  if (kv->head_dim != 128 || kv->num_kv_heads != kvh || kv->num_layers != layers || kv->max_ctx != max_ctx)
    return Q4D_ERR_SHAPE;
  if (!aligned(kv->data, 16)) return Q4D_ERR_BAD_ADDR;
  return Q4D_OK;
}

void fx_planes(const q4d_fixed_kv_t* kv, int layer, int32_t** kp, int32_t** vp) {
  const size_t plane = (size_t)kv->num_kv_heads * kv->max_ctx * kv->head_dim;
  *kp = kv->data + (size_t)layer * 2 * plane;
  *vp = *kp + plane;
}

template <int KC, int R, int PRO, int EPI>
int fx_launch_gemv_t(const FxGemv& g, hipStream_t st) {
  const int rows_per_block = 4 * R;
  hipLaunchKernelGGL((fx_gemv_kernel<KC, R, PRO, EPI>), dim3((g.rows + rows_per_block - 1) / rows_per_block),
                     dim3(256), 0, st, g);
  return check_launch();
}

// Row sums of one GEMV per output row (R rows per wave); K = 1024 KC.
template <int PRO, int EPI>
int fx_launch_gemv(const FxGemv& g, hipStream_t st) {
  constexpr int R = EPI == FX_EPI_LOGITS ? kFxRowsLm : (EPI == FX_EPI_Q12 ? 2 : 1);
  switch (g.K) {
    case 1024: return fx_launch_gemv_t<1, R, PRO, EPI>(g, st);
    case 2048:
      if constexpr (PRO == FX_PRO_LOAD) return fx_launch_gemv_t<2, R, PRO, EPI>(g, st);
      break;
    case 3072:
      if constexpr (PRO == FX_PRO_LOAD) return fx_launch_gemv_t<3, R, PRO, EPI>(g, st);
      break;
  }
  return Q4D_ERR_SHAPE;
}

FxGemv fx_gemv_base() {
  FxGemv g;
  memset(&g, 0, sizeof(g));
  return g;
}

int fx_run_layer(const q4d_fixed_model_t* fm, int l, const int32_t* hin, int32_t* hout, const q4d_fixed_kv_t* kv,
                 const int32_t* positions, void* ws, const FxLayout& W, hipStream_t st) {
  const q4d_model_t* m = fm->base;
  const q4d_layer_t& L = m->layers[l];
  const q4d_fixed_layer_t& F = fm->layers[l];
  const int qd = m->num_q_heads * 128, kd = m->num_kv_heads * 128;
  int32_t* counts = ws_ptr<int32_t>(ws, W.counts);
  int32_t* qkv = ws_ptr<int32_t>(ws, W.qkv);
  int32_t* attn = ws_ptr<int32_t>(ws, W.attn);
  int32_t* post = ws_ptr<int32_t>(ws, W.post);
  int32_t* mlp = ws_ptr<int32_t>(ws, W.mlp);
  int rc;

  FxGemv g = fx_gemv_base();  // 1. input RMSNorm + q|k|v
  g.w0 = L.q_proj.w; g.s0 = L.q_proj.s;
  g.w1 = L.k_proj.w; g.s1 = L.k_proj.s;
  g.w2 = L.v_proj.w; g.s2 = L.v_proj.s;
  g.e0 = qd; g.e1 = qd + kd; g.rows = qd + 2 * kd; g.K = 1024;
  g.x = hin; g.gamma = F.input_gamma; g.y = qkv; g.counts = counts;
  g.slot_norm = Q4D_FX_SAT_INPUT_NORM; g.slot_a = Q4D_FX_SAT_QKV;
  if ((rc = fx_launch_gemv<FX_PRO_NORM, FX_EPI_Q12>(g, st))) return rc;

  FxAttn a;  // 2. q/k norm, RoPE, K/V append, attention
  memset(&a, 0, sizeof(a));
  a.qkv = qkv; a.q_gamma = F.q_gamma; a.k_gamma = F.k_gamma;
  a.cos = fm->rope_cos; a.sin = fm->rope_sin; a.position = positions;
  fx_planes(kv, l, &a.kc, &a.vc);
  a.max_ctx = kv->max_ctx; a.qh = m->num_q_heads; a.kvh = m->num_kv_heads;
  a.score_scale = fm->score_scale_q0_31;
  a.exp_lut = ws_ptr<int32_t>(ws, W.exp_lut);
  a.out = attn; a.counts = counts; a.status = counts + Q4D_FX_STATUS;
  fx_attn_bind(a, ws_ptr<char>(ws, W.attn_ws), W.al);
  if ((rc = fx_launch_attention<true>(a, W.al.nch, st))) return rc;

  g = fx_gemv_base();  // 3. o_proj + residual
  g.w0 = L.o_proj.w; g.s0 = L.o_proj.s; g.e0 = g.e1 = g.rows = 1024; g.K = qd;
  g.x = attn; g.resid = hin; g.y = post; g.counts = counts;
  g.slot_a = Q4D_FX_SAT_O_PROJ; g.slot_b = Q4D_FX_SAT_POST_RESIDUAL;
  if ((rc = fx_launch_gemv<FX_PRO_LOAD, FX_EPI_RESID>(g, st))) return rc;

  g = fx_gemv_base();  // 4. post RMSNorm + gate/up + SiLU * up
  g.w0 = L.gate_proj.w; g.s0 = L.gate_proj.s; g.w1 = L.up_proj.w; g.s1 = L.up_proj.s;
  g.rows = m->intermediate_size; g.K = 1024;
  g.x = post; g.gamma = F.post_gamma; g.y = mlp; g.lut = ws_ptr<int32_t>(ws, W.sig_lut); g.counts = counts;
  g.slot_norm = Q4D_FX_SAT_POST_NORM; g.slot_a = Q4D_FX_SAT_GATE; g.slot_b = Q4D_FX_SAT_UP;
  g.slot_c = Q4D_FX_SAT_SILU; g.slot_d = Q4D_FX_SAT_MLP_HIDDEN;
  if ((rc = fx_launch_gemv<FX_PRO_NORM, FX_EPI_SILU>(g, st))) return rc;

  g = fx_gemv_base();  // 5. down + residual
  g.w0 = L.down_proj.w; g.s0 = L.down_proj.s; g.e0 = g.e1 = g.rows = 1024; g.K = m->intermediate_size;
  g.x = mlp; g.resid = post; g.y = hout; g.counts = counts;
  g.slot_a = Q4D_FX_SAT_DOWN; g.slot_b = Q4D_FX_SAT_LAYER_RESIDUAL;
  return fx_launch_gemv<FX_PRO_LOAD, FX_EPI_RESID>(g, st);
}

int fx_check_ws(const void* ws, size_t bytes, const q4d_model_t* m) {
  if (!ws) return Q4D_ERR_NULL;
  if (!aligned(ws, 256)) return Q4D_ERR_BAD_ADDR;
  if (bytes < fx_layout(m).total) return Q4D_ERR_CAPACITY;
  return Q4D_OK;
}

}  // namespace
}  // namespace q4d

using namespace q4d;

extern "C" {

int q4d_fixed_tables(int32_t* exp_lut, int32_t n_exp, int32_t* sigmoid_lut, int32_t n_sigmoid) {
  if (!exp_lut || !sigmoid_lut) return Q4D_ERR_NULL;
  if (n_exp != kFxExpLut || n_sigmoid != kFxSigLut) return Q4D_ERR_SHAPE;
  fx_tables_host(exp_lut, sigmoid_lut);
  return Q4D_OK;
}

size_t q4d_fixed_workspace_bytes(const q4d_fixed_model_t* model) {
  if (fx_check_model(model)) return 0;
  return fx_layout(model->base).total;
}

int q4d_fixed_workspace_init(void* ws, size_t ws_bytes, const q4d_fixed_model_t* model, void* stream) {
  int rc = fx_check_model(model);
  if (rc) return rc;
  if ((rc = fx_check_ws(ws, ws_bytes, model->base))) return rc;
  const FxTables& tab = fx_tables();
  const FxLayout W = fx_layout(model->base);
  hipStream_t st = fx_stream(stream);
  if (hipMemsetAsync(ws, 0, W.total, st) != hipSuccess) return Q4D_ERR_LAUNCH;
  if (hipMemcpyAsync(ws_ptr<int32_t>(ws, W.exp_lut), tab.e, sizeof(tab.e), hipMemcpyHostToDevice, st) != hipSuccess)
    return Q4D_ERR_LAUNCH;
  if (hipMemcpyAsync(ws_ptr<int32_t>(ws, W.sig_lut), tab.s, sizeof(tab.s), hipMemcpyHostToDevice, st) != hipSuccess)
    return Q4D_ERR_LAUNCH;
  return Q4D_OK;
}

int q4d_fixed_read_counts(const void* ws, size_t ws_bytes, int32_t* counts, int32_t n, void* stream) {
  if (!ws || !counts) return Q4D_ERR_NULL;
  if (n <= 0 || n > Q4D_FX_COUNTS) return Q4D_ERR_SHAPE;
  static_assert(Q4D_FX_COUNTS <= kFxStripeWords, "counter stripe too small");
  const size_t bytes = (size_t)kFxStripes * kFxStripeWords * 4;
  if (ws_bytes < bytes) return Q4D_ERR_CAPACITY;
  int32_t stripes[kFxStripes * kFxStripeWords];
  hipStream_t st = fx_stream(stream);
  if (hipMemcpyAsync(stripes, ws, bytes, hipMemcpyDeviceToHost, st) != hipSuccess) return Q4D_ERR_LAUNCH;
  if (hipStreamSynchronize(st) != hipSuccess) return Q4D_ERR_LAUNCH;
  for (int i = 0; i < n; ++i) {
    int64_t v = 0;
    for (int k = 0; k < kFxStripes; ++k) v += stripes[k * kFxStripeWords + i];
    counts[i] = i == Q4D_FX_STATUS ? stripes[i] : (int32_t)(v > INT32_MAX ? INT32_MAX : v);
  }
  return Q4D_OK;
}

int q4d_fixed_rms_norm(const int32_t* x, const int16_t* gamma, int32_t rows, int32_t dim, int32_t kind, int32_t* y,
                       int64_t* stats, void* stream) {
  if (!x || !gamma || !y) return Q4D_ERR_NULL;
  if (kind != 0 && kind != 1) return Q4D_ERR_SHAPE;
  if (rows <= 0 || (kind == 0 && dim != 1024) || (kind == 1 && dim != 128)) return Q4D_ERR_SHAPE;
  if (stats && !aligned(stats, 8)) return Q4D_ERR_BAD_ADDR;
  hipLaunchKernelGGL(fx_rmsnorm_kernel, dim3(rows), dim3(256), 0, fx_stream(stream), x, gamma, dim, kind, y, stats);
  return check_launch();
}

int q4d_fixed_qk_norm_rope(const int32_t* q, const int32_t* k, int32_t q_heads, int32_t kv_heads,
                           const int16_t* q_gamma, const int16_t* k_gamma, const int16_t* cos_row,
                           const int16_t* sin_row, int32_t* q_rope, int32_t* k_rope, int32_t* q_norm,
                           int32_t* k_norm, void* stream) {
  if (!q || !k || !cos_row || !sin_row || !q_rope || !k_rope) return Q4D_ERR_NULL;
  if (!q_gamma != !k_gamma) return Q4D_ERR_NULL;
  if (q_heads <= 0 || kv_heads <= 0 || q_heads > 64 || kv_heads > 64) return Q4D_ERR_SHAPE;
  hipLaunchKernelGGL(fx_qknorm_rope_kernel, dim3(q_heads + kv_heads), dim3(128), 0, fx_stream(stream), q, k,
                     q_heads, q_gamma, k_gamma, cos_row, sin_row, q_rope, k_rope, q_norm, k_norm);
  return check_launch();
}

size_t q4d_fixed_attention_workspace_bytes(int32_t q_heads, int32_t max_ctx) {
  if (q_heads <= 0 || q_heads > 64 || max_ctx <= 0 || max_ctx > kFxMaxCtx) return 0;
  return fx_attn_layout(q_heads, max_ctx).total;
}

int q4d_fixed_attention(const q4d_fixed_kv_t* kv, int32_t layer, int32_t q_heads, int32_t cache_length,
                        const int32_t* q_rope, int32_t score_scale_q0_31, const int32_t* exp_lut, int32_t* out,
                        int64_t* raw, int64_t* scaled, int32_t* lut_index, int32_t* prob, void* ws,
                        size_t ws_bytes, void* stream) {
  if (!kv || !kv->data || !q_rope || !exp_lut || !out || !ws) return Q4D_ERR_NULL;
  if (kv->head_dim != 128 || kv->num_kv_heads <= 0 || kv->max_ctx <= 0 || kv->max_ctx > kFxMaxCtx) return Q4D_ERR_SHAPE;
  if (layer < 0 || layer >= kv->num_layers) return Q4D_ERR_BAD_LAYER;
  if (q_heads <= 0 || q_heads % kv->num_kv_heads) return Q4D_ERR_SHAPE;
  if (cache_length <= 0 || cache_length > kv->max_ctx) return Q4D_ERR_CONTEXT;
  if (score_scale_q0_31 <= 0) return Q4D_ERR_SHAPE;
  if (!aligned(kv->data, 16) || (raw && !aligned(raw, 8)) || (scaled && !aligned(scaled, 8)) || !aligned(ws, 256))
    return Q4D_ERR_BAD_ADDR;
  const FxAttnLayout AL = fx_attn_layout(q_heads, kv->max_ctx);
  if (q_heads > 64) return Q4D_ERR_SHAPE;
  if (ws_bytes < AL.total) return Q4D_ERR_CAPACITY;
  FxAttn a;
  memset(&a, 0, sizeof(a));
  a.q_in = q_rope;
  a.cache_length = cache_length;
  fx_planes(kv, layer, &a.kc, &a.vc);
  a.max_ctx = kv->max_ctx;
  a.qh = q_heads;
  a.kvh = kv->num_kv_heads;
  a.score_scale = score_scale_q0_31;
  a.exp_lut = exp_lut;
  a.out = out;
  a.raw = raw;
  a.scaled = scaled;
  a.lut_index = lut_index;
  a.prob = prob;
  fx_attn_bind(a, ws, AL);
  return fx_launch_attention<false>(a, AL.nch, fx_stream(stream));
}

int q4d_fixed_kv_append(const q4d_fixed_kv_t* kv, int32_t layer, const int32_t* positions, const int32_t* k,
                        const int32_t* v, void* stream) {
  if (!kv || !kv->data || !positions || !k || !v) return Q4D_ERR_NULL;
  if (kv->head_dim != 128 || kv->num_kv_heads <= 0 || kv->max_ctx <= 0) return Q4D_ERR_SHAPE;
  if (layer < 0 || layer >= kv->num_layers) return Q4D_ERR_BAD_LAYER;
  int32_t *kp, *vp;
  fx_planes(kv, layer, &kp, &vp);
  const int n = kv->num_kv_heads * 128;
  hipLaunchKernelGGL(fx_kv_append_kernel, dim3((n + 255) / 256), dim3(256), 0, fx_stream(stream), kp, vp,
                     kv->num_kv_heads, kv->max_ctx, positions, k, v);
  return check_launch();
}

int q4d_fixed_silu_mul(const int32_t* gate, const int32_t* up, int32_t n, const int32_t* sigmoid_lut, int32_t* hidden,
                       int32_t* lut_index, int32_t* sigmoid, int32_t* silu_gate, void* stream) {
  if (!gate || !up || !sigmoid_lut || !hidden) return Q4D_ERR_NULL;
  if (n <= 0) return Q4D_ERR_SHAPE;
  hipLaunchKernelGGL(fx_silu_kernel, dim3((n + 255) / 256), dim3(256), 0, fx_stream(stream), gate, up, n, sigmoid_lut,
                     hidden, lut_index, sigmoid, silu_gate);
  return check_launch();
}

int q4d_fixed_residual_add(const int32_t* hidden, const int32_t* x, int32_t n, int32_t* out, void* stream) {
  if (!hidden || !x || !out) return Q4D_ERR_NULL;
  if (n <= 0) return Q4D_ERR_SHAPE;
  hipLaunchKernelGGL(fx_resid_kernel, dim3((n + 255) / 256), dim3(256), 0, fx_stream(stream), hidden, x, n, out);
  return check_launch();
}

int q4d_fixed_embedding(const q4d_matrix_t* table, const int32_t* tokens, int32_t n, int32_t* hidden, void* stream) {
  if (!table || !table->w || !table->s || !tokens || !hidden) return Q4D_ERR_NULL;
  if (n <= 0 || table->rows <= 0 || table->cols <= 0 || table->cols % 64) return Q4D_ERR_SHAPE;
  hipLaunchKernelGGL(fx_embed_kernel, dim3(n), dim3(256), 0, fx_stream(stream), table->w, table->s, table->rows,
                     table->cols, tokens, hidden, (int32_t*)nullptr);
  return check_launch();
}

int q4d_fixed_q4_gemv(const q4d_matrix_t* w, const int32_t* x, const int16_t* input_gamma, int32_t* y,
                      void* stream) {
  if (!w || !w->w || !w->s || !x || !y) return Q4D_ERR_NULL;
  if (w->rows <= 0 || !fx_k_ok(w->cols) || (input_gamma && w->cols != 1024)) return Q4D_ERR_SHAPE;
  if (!aligned(w->w, 16) || !aligned(w->s, 4) || !aligned(x, 16)) return Q4D_ERR_BAD_ADDR;
  FxGemv g = fx_gemv_base();
  g.w0 = g.w1 = g.w2 = w->w;
  g.s0 = g.s1 = g.s2 = w->s;
  g.e0 = g.e1 = g.rows = w->rows;
  g.K = w->cols;
  g.x = x;
  g.gamma = input_gamma;
  g.y = y;
  hipStream_t st = fx_stream(stream);
  return input_gamma ? fx_launch_gemv<FX_PRO_NORM, FX_EPI_Q12>(g, st) : fx_launch_gemv<FX_PRO_LOAD, FX_EPI_Q12>(g, st);
}

int q4d_fixed_decoder_layer(const q4d_fixed_model_t* model, int32_t layer, const int32_t* hidden_in,
                            int32_t* hidden_out, const q4d_fixed_kv_t* kv, const int32_t* positions, void* ws,
                            size_t ws_bytes, void* stream) {
  if (!hidden_in || !hidden_out || !positions) return Q4D_ERR_NULL;
  int rc = fx_check_model(model);
  if (rc) return rc;
  const q4d_model_t* m = model->base;
  if (layer < 0 || layer >= m->num_layers) return Q4D_ERR_BAD_LAYER;
  if ((rc = fx_check_kv(kv, m->num_layers, m->num_kv_heads, m->max_ctx))) return rc;
  if ((rc = fx_check_ws(ws, ws_bytes, m))) return rc;
  if (!aligned(hidden_in, 16)) return Q4D_ERR_BAD_ADDR;
  return fx_run_layer(model, layer, hidden_in, hidden_out, kv, positions, ws, fx_layout(m), fx_stream(stream));
}

int q4d_fixed_run_one_token(const q4d_fixed_model_t* model, const int32_t* tokens, const int32_t* positions,
                            const q4d_fixed_kv_t* kv, int32_t* next_token, int64_t* score, int64_t* logits,
                            int32_t* hidden_out, void* ws, size_t ws_bytes, void* stream) {
  if (!tokens || !positions || !next_token || !score) return Q4D_ERR_NULL;
  int rc = fx_check_model(model);
  if (rc) return rc;
  const q4d_model_t* m = model->base;
  if ((rc = fx_check_kv(kv, m->num_layers, m->num_kv_heads, m->max_ctx))) return rc;
  if ((rc = fx_check_ws(ws, ws_bytes, m))) return rc;
  if (!aligned(score, 8) || (logits && !aligned(logits, 8))) return Q4D_ERR_BAD_ADDR;
  const FxLayout W = fx_layout(m);
  hipStream_t st = fx_stream(stream);
  int32_t* counts = ws_ptr<int32_t>(ws, W.counts);
  int32_t* hidden = ws_ptr<int32_t>(ws, W.hidden);
  hipLaunchKernelGGL(fx_embed_kernel, dim3(1), dim3(256), 0, st, m->embed_tokens.w, m->embed_tokens.s,
                     m->vocab_size, 1024, tokens, hidden, counts + Q4D_FX_STATUS);
  if ((rc = check_launch())) return rc;
  for (int l = 0; l < m->num_layers; ++l)
    if ((rc = fx_run_layer(model, l, hidden, hidden, kv, positions, ws, W, st))) return rc;
  if (hidden_out &&
      hipMemcpyAsync(hidden_out, hidden, (size_t)m->hidden_size * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
    return Q4D_ERR_LAUNCH;
  FxGemv g = fx_gemv_base();  // final RMSNorm + full-vocabulary scan
  g.w0 = m->embed_tokens.w; g.s0 = m->embed_tokens.s;
  g.e0 = g.e1 = g.rows = m->vocab_size; g.K = 1024;
  g.x = hidden; g.gamma = model->final_gamma; g.logits = logits;
  g.part_score = ws_ptr<int64_t>(ws, W.part_score); g.part_idx = ws_ptr<int32_t>(ws, W.part_idx);
  g.counts = counts; g.slot_norm = Q4D_FX_SAT_FINAL_NORM;
  if ((rc = fx_launch_gemv<FX_PRO_NORM, FX_EPI_LOGITS>(g, st))) return rc;
  hipLaunchKernelGGL(fx_argmax_kernel, dim3(1), dim3(1024), 0, st, g.part_score, g.part_idx, W.nparts, next_token,
                     score);
  return check_launch();
}

}  // extern "C"
