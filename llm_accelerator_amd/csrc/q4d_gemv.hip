// Fused Q4 dequant-GEMV for gfx950 (wave64).
//
// One wave owns a "row group": the smallest set of whole rows whose 16-byte
// chunks tile an exact multiple of 64 lanes (K=1024: 2 rows, one 16 B load
// per lane; K=2048: 1 row; K=3072: 2 rows, three loads per lane).  Because a
// lane always sees the same column chunks, its activations are unpacked into
// registers once (XChunk) and reused for every row group the wave visits.
// Waves stride over row groups, issuing U groups of 128-bit loads before
// consuming any, so each lane keeps U*LG loads in flight.
//
// Prologues: fp16 x, fp32 x (rounded to fp16, or split hi+lo into two fp16
// halves for ~22-bit activations), or RMSNorm of an fp32 hidden vector
// (reference common.py:129-134) computed by every block.
// Epilogues: fp16/fp32 store, residual add (common.py:284,297), SwiGLU over a
// gate/up row pair (common.py:293-295), and LM-head argmax with the
// lowest-index tie rule (56_export_persistent_multitoken_layer_golden.py:860).
#include <math.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }

template <int K>
struct Geo {
  static constexpr int C = K / 32;                       // 16-byte chunks per row
  static constexpr int G = K / 64;                       // scale groups per row
  static constexpr int L = C / gcd_c(C, 64) * 64;        // lcm(C, 64)
  static constexpr int RG = L / C;                       // rows per row group
  static constexpr int LG = L / 64;                      // loads per lane per group
};

// Build hi (and optionally lo) XChunks from 32 fp32 activations.
template <int XP>
__device__ __forceinline__ void xchunks_from_f32(const float (&v)[32], XChunk& hi, XChunk& lo) {
  float sh = 0.f, sl = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = v[8 * m + i], b = v[8 * m + i + 4];
      const _Float16 ah = (_Float16)a, bh = (_Float16)b;
      hi.p[4 * m + i] = make_h2(ah, bh);
      sh += (float)ah + (float)bh;
      if constexpr (XP == 2) {
        const _Float16 al = (_Float16)(a - (float)ah), bl = (_Float16)(b - (float)bh);
        lo.p[4 * m + i] = make_h2(al, bl);
        sl += (float)al + (float)bl;
      }
    }
  }
  hi.sum8 = 8.f * sh;
  if constexpr (XP == 2) lo.sum8 = 8.f * sl;
}

// hi/lo variant of chunk_dot sharing the dequant masks.
__device__ __forceinline__ float chunk_dot_hl(const u32x4 w, const XChunk& h, const XChunk& l) {
  float a = 0.f, b = 0.f, c = 0.f, d = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t v = w[m] ^ 0x88888888u;
    const uint32_t t = v >> 8;
    const uint32_t m0 = v & 0x000F000Fu, m1 = v & 0x00F000F0u;
    const uint32_t m2 = t & 0x000F000Fu, m3 = t & 0x00F000F0u;
    a = dot2(m0, h.p[4 * m + 0], a);
    b = dot2(m1, h.p[4 * m + 1], b);
    a = dot2(m2, h.p[4 * m + 2], a);
    b = dot2(m3, h.p[4 * m + 3], b);
    c = dot2(m0, l.p[4 * m + 0], c);
    d = dot2(m1, l.p[4 * m + 1], d);
    c = dot2(m2, l.p[4 * m + 2], c);
    d = dot2(m3, l.p[4 * m + 3], d);
  }
  return fmaf(a, 16777216.f, fmaf(b, 1048576.f, -h.sum8)) +
         fmaf(c, 16777216.f, fmaf(d, 1048576.f, -l.sum8));
}

// Issue the loads of U row groups starting at gbase (wave-uniform guards).
template <int K, int U, bool PAIR>
__device__ __forceinline__ void load_batch(int gbase, int nw, int NG, int lane, const uint8_t* w0,
                                           const uint8_t* w1, const uint8_t* w2, const uint16_t* s0,
                                           const uint16_t* s1, const uint16_t* s2, int e0, int e1,
                                           u32x4 (&wv)[U][Geo<K>::LG], uint32_t (&sv)[U][Geo<K>::LG]) {
  constexpr int C = Geo<K>::C, RG = Geo<K>::RG, LG = Geo<K>::LG, G = Geo<K>::G;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int g = gbase + u * nw;
    if (g < NG) {
      int seg = 0, local0 = g;
      if constexpr (!PAIR) {
        const int row0 = g * RG;
        seg = (row0 < e0) ? 0 : ((row0 < e1) ? 1 : 2);
        local0 = row0 - (seg == 0 ? 0 : (seg == 1 ? e0 : e1));
      }
#pragma unroll
      for (int j = 0; j < LG; ++j) {
        const int f = j * 64 + lane;
        const int r = f / C, c = f % C;
        const int sg = PAIR ? r : seg;
        const int row = PAIR ? g : local0 + r;
        const uint8_t* wb = sg == 0 ? w0 : (sg == 1 ? w1 : w2);
        const uint16_t* sb = sg == 0 ? s0 : (sg == 1 ? s1 : s2);
        wv[u][j] = *reinterpret_cast<const u32x4*>(wb + (size_t)row * (K / 2) + c * 16);
        sv[u][j] = sb[(size_t)row * G + (c >> 1)];
      }
    }
  }
}

template <int K, int U, int XM, int XP, int EP, bool PAIR>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvArgs a) {
  using Gm = Geo<K>;
  constexpr int C = Gm::C, RG = Gm::RG, LG = Gm::LG;
  static_assert(!PAIR || RG == 2, "row-pair epilogue needs two rows per group");
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int bat = blockIdx.y;

  __shared__ float s_red[4];
  __shared__ int s_idx[4];
  __shared__ int s_last;
  __shared__ f32x4 s_x[XM == X_RMS ? K / 4 : 1];

  // Segment pointers are read with constant indices (scalar kernel-argument
  // loads) and selected in registers: indexing a.w[] with a runtime value
  // turns every weight load into a dependent load from the argument block.
  const uint8_t* const w0 = a.w[0];
  const uint8_t* const w1 = a.w[1];
  const uint8_t* const w2 = a.w[2];
  const uint16_t* const s0 = a.s[0];
  const uint16_t* const s1 = a.s[1];
  const uint16_t* const s2 = a.s[2];
  const int e0 = a.seg_end[0], e1 = a.seg_end[1];
  const int NG = PAIR ? a.rows : a.rows / RG;
  const int gw = blockIdx.x * 4 + wid;
  const int nw = gridDim.x * 4;

  // ---- activation loads go out first --------------------------------------
  // vmcnt drains in issue order, so anything issued after the weight prefetch
  // could only be waited for together with the weights.
  f32x4 hreg = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 gam[XM == X_RMS ? LG : 1][8];
  u32x4 xr16[XM == X_F16 ? LG : 1][4];
  f32x4 xr32[XM == X_F32 ? LG : 1][8];
  if constexpr (XM == X_RMS) {
    static_assert(K / 4 <= 256, "RMS prologue stages one 16-byte vector per thread");
    if (threadIdx.x < K / 4)
      hreg = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.x) + (size_t)bat * K)[threadIdx.x];
#pragma unroll
    for (int j = 0; j < LG; ++j) {
      const int c = (j * 64 + lane) % C;
#pragma unroll
      for (int q = 0; q < 8; ++q) gam[j][q] = reinterpret_cast<const f32x4*>(a.gamma + c * 32)[q];
    }
  } else if constexpr (XM == X_F16) {
#pragma unroll
    for (int j = 0; j < LG; ++j) {
      const int c = (j * 64 + lane) % C;
      const u32x4* xp = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.x) + (size_t)bat * K + c * 32);
#pragma unroll
      for (int q = 0; q < 4; ++q) xr16[j][q] = xp[q];
    }
  } else {
#pragma unroll
    for (int j = 0; j < LG; ++j) {
      const int c = (j * 64 + lane) % C;
      const f32x4* xp = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.x) + (size_t)bat * K + c * 32);
#pragma unroll
      for (int q = 0; q < 8; ++q) xr32[j][q] = xp[q];
    }
  }

  // ---- first batch of weights in flight while the activations are prepared ---
  u32x4 wv[U][LG];
  uint32_t sv[U][LG];
  load_batch<K, U, PAIR>(gw, nw, NG, lane, w0, w1, w2, s0, s1, s2, e0, e1, wv, sv);

  XChunk xh[LG];
  XChunk xl[XP == 2 ? LG : 1];
  if constexpr (XM == X_RMS) {
    // stage the fp32 hidden vector in LDS and reduce sum(x^2) in a fixed order
    // (identical in every block); LDS-only barriers keep the weights in flight
    float ss = 0.f;
    if (threadIdx.x < K / 4) {
      s_x[threadIdx.x] = hreg;
      ss = fmaf(hreg[0], hreg[0], ss);
      ss = fmaf(hreg[1], hreg[1], ss);
      ss = fmaf(hreg[2], hreg[2], ss);
      ss = fmaf(hreg[3], hreg[3], ss);
    }
    ss = wave_sum_dpp(ss);
    if (lane == 63) s_red[wid] = ss;
    block_sync_lds();
    const float inv_rms = 1.0f / sqrtf(((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) / (float)K + a.eps);
#pragma unroll
    for (int j = 0; j < LG; ++j) {
      const int c = (j * 64 + lane) % C;
      float v[32];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const f32x4 t = s_x[c * 8 + q];
        const f32x4 g = gam[j][q];
        v[4 * q + 0] = (t[0] * inv_rms) * g[0];
        v[4 * q + 1] = (t[1] * inv_rms) * g[1];
        v[4 * q + 2] = (t[2] * inv_rms) * g[2];
        v[4 * q + 3] = (t[3] * inv_rms) * g[3];
      }
      xchunks_from_f32<XP>(v, xh[j], xl[XP == 2 ? j : 0]);
    }
  } else if constexpr (XM == X_F16) {
#pragma unroll
    for (int j = 0; j < LG; ++j) {
      uint32_t xw[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 t = xr16[j][q];
        xw[4 * q + 0] = t[0];
        xw[4 * q + 1] = t[1];
        xw[4 * q + 2] = t[2];
        xw[4 * q + 3] = t[3];
      }
      xchunk_from_words(xw, xh[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < LG; ++j) {
      float v[32];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const f32x4 t = xr32[j][q];
        v[4 * q + 0] = t[0];
        v[4 * q + 1] = t[1];
        v[4 * q + 2] = t[2];
        v[4 * q + 3] = t[3];
      }
      xchunks_from_f32<XP>(v, xh[j], xl[XP == 2 ? j : 0]);
    }
  }

  // ---- stream row groups (software-pipelined: next batch in flight) -----------
  float best = -INFINITY;
  int besti = 0x7fffffff;

  for (int g0 = gw; g0 < NG; g0 += nw * U) {
    u32x4 cw[U][LG];
    uint32_t cs[U][LG];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < LG; ++j) {
        cw[u][j] = wv[u][j];
        cs[u][j] = sv[u][j];
      }
    if (g0 + nw * U < NG)
      load_batch<K, U, PAIR>(g0 + nw * U, nw, NG, lane, w0, w1, w2, s0, s1, s2, e0, e1, wv, sv);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = g0 + u * nw;
      if (g < NG) {
      float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
      for (int j = 0; j < LG; ++j) {
        const int r = (j * 64 + lane) / C;
        float p;
        if constexpr (XP == 2)
          p = chunk_dot_hl(cw[u][j], xh[j], xl[j]);
        else
          p = chunk_dot(cw[u][j], xh[j]);
        p *= scale_q2_14(cs[u][j]);
        if (RG == 1 || r == 0)
          acc0 += p;
        else
          acc1 += p;
      }
      // DPP reductions: lane 63 ends up with row g*RG (RG == 1) or, for
      // RG == 2, lane 31 with row 2g and lane 63 with row 2g+1
      float v;
      if constexpr (RG == 1) {
        v = wave_sum_dpp(acc0);
      } else if constexpr (K == 1024) {
        // lanes 0-31 only hold row 0, lanes 32-63 only row 1
        v = half_wave_sum_dpp(lane < 32 ? acc0 : acc1);
      } else {
        // both rows spread over all lanes: full-wave sums, then lane 31
        // takes row 0 from lane 63's neighbourhood via a row broadcast
        const float r0 = wave_sum_dpp(acc0);
        const float r1 = wave_sum_dpp(acc1);
        // the permute must run with every lane active: an inactive source
        // lane reads as zero
        const float r0_all = __shfl(r0, 63, kWave);
        v = lane < 32 ? r0_all : r1;
      }
      const bool owner = (RG == 1) ? (lane == 63) : ((lane & 31) == 31);
      const int row = (RG == 1) ? g : (g * 2 + (lane >> 5));
      if constexpr (EP == EP_SWIGLU) {
        // lane 63 holds up; row_bcast31 brings the gate from lane 31
        const float gate = dpp_f<kDppRowBcast31, 0xC>(v);
        if (lane == 63) {
          const float act = (gate / (1.0f + expf(-gate))) * v;
          static_cast<float*>(a.y)[(size_t)bat * a.rows + g] = act;
        }
      } else if (owner) {
        const size_t o = (size_t)bat * a.rows + row;
        if constexpr (EP == EP_F16) {
          static_cast<_Float16*>(a.y)[o] = (_Float16)v;
        } else if constexpr (EP == EP_F32) {
          static_cast<float*>(a.y)[o] = v;
        } else if constexpr (EP == EP_RESID) {
          static_cast<float*>(a.y)[o] = a.resid[o] + v;
        } else if constexpr (EP == EP_ARGMAX) {
          if (a.logits) a.logits[row] = v;
          if (arg_better(v, row, best, besti)) {
            best = v;
            besti = row;
          }
        }
      }
      }  // g < NG
    }
  }

  if constexpr (EP == EP_ARGMAX) {
    // wave -> block -> grid (last block to finish reduces all block results)
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float ob = shfl_xor_f(best, m);
      const int oi = __shfl_xor(besti, m, kWave);
      if (arg_better(ob, oi, best, besti)) {
        best = ob;
        besti = oi;
      }
    }
    __syncthreads();  // s_red may still be read by the RMS prologue
    if (lane == 0) {
      s_red[wid] = best;
      s_idx[wid] = besti;
    }
    __syncthreads();
    float* part = static_cast<float*>(a.lm_part);
    if (threadIdx.x == 0) {
      float bb = s_red[0];
      int bi = s_idx[0];
      for (int w = 1; w < 4; ++w)
        if (arg_better(s_red[w], s_idx[w], bb, bi)) {
          bb = s_red[w];
          bi = s_idx[w];
        }
      part[2 * blockIdx.x] = bb;
      reinterpret_cast<int*>(part)[2 * blockIdx.x + 1] = bi;
      // release this thread's partial before counting in (agent scope)
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      const int done = atomicAdd(a.counter, 1);
      s_last = (done == (int)gridDim.x - 1);
    }
    __syncthreads();
    if (s_last) {
      // acquire the partials released by every other block
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      float bb = -INFINITY;
      int bi = 0x7fffffff;
      for (int i = threadIdx.x; i < (int)gridDim.x; i += 256) {
        const float sc = part[2 * i];
        const int ix = reinterpret_cast<int*>(part)[2 * i + 1];
        if (arg_better(sc, ix, bb, bi)) {
          bb = sc;
          bi = ix;
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        const float ob = shfl_xor_f(bb, m);
        const int oi = __shfl_xor(bi, m, kWave);
        if (arg_better(ob, oi, bb, bi)) {
          bb = ob;
          bi = oi;
        }
      }
      __syncthreads();
      if (lane == 0) {
        s_red[wid] = bb;
        s_idx[wid] = bi;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w)
          if (arg_better(s_red[w], s_idx[w], s_red[0], s_idx[0])) {
            s_red[0] = s_red[w];
            s_idx[0] = s_idx[w];
          }
        a.out_token[0] = s_idx[0];
        a.out_score[0] = s_red[0];
        *a.counter = 0;  // ready for the next launch
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Blocks of one kernel instance that fit on the device at once (queried once
// per instance); large GEMVs launch one resident wave set that loops, so the
// per-block activation prologue is paid once per resident block.
template <class F>
static int resident_blocks(F kernel) {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess || per_cu < 1)
      return 1024;  // conservative fallback, recomputed next call
    cached = cus * per_cu;
  }
  return cached;
}

template <int K, int U, int XM, int XP, int EP, bool PAIR>
static int launch_inst(const GemvArgs& a, int max_blocks, hipStream_t stream) {
  using Gm = Geo<K>;
  const int NG = PAIR ? a.rows : a.rows / Gm::RG;
  int waves = (NG + U - 1) / U;
  int blocks = (waves + 3) / 4;
  const int res = resident_blocks(gemv_kernel<K, U, XM, XP, EP, PAIR>);
  if (blocks > res) blocks = res;
  if (blocks > max_blocks) blocks = max_blocks;
  if (blocks < 1) blocks = 1;
  dim3 grid(blocks, a.batch);
  hipLaunchKernelGGL((gemv_kernel<K, U, XM, XP, EP, PAIR>), grid, dim3(256), 0, stream, a);
  return check_launch();
}

template <int K, int XM, int XP, int EP, bool PAIR>
static int launch_u(const GemvArgs& a, hipStream_t stream) {
  if constexpr (EP == EP_ARGMAX) return launch_inst<K, 4, XM, XP, EP, PAIR>(a, kLmMaxBlocks, stream);
  const int rg = Geo<K>::RG;
  const int NG = PAIR ? a.rows : a.rows / rg;
  // three chunks per lane: one row group per batch keeps VGPRs below 256
  if constexpr (K == 3072) return launch_inst<K, 1, XM, XP, EP, PAIR>(a, 4096, stream);
  if (NG <= 16384) return launch_inst<K, 2, XM, XP, EP, PAIR>(a, 4096, stream);
  return launch_inst<K, 4, XM, XP, EP, PAIR>(a, 4096, stream);
}

template <int K>
static int dispatch_k(const GemvArgs& a, int xm, int xp, int ep, bool pair, hipStream_t st) {
  // primitive linear: fp16 / fp32 in, fp16 / fp32 out
  if (!pair && (ep == EP_F16 || ep == EP_F32)) {
    if (xm == X_F16) return ep == EP_F16 ? launch_u<K, X_F16, 1, EP_F16, false>(a, st)
                                         : launch_u<K, X_F16, 1, EP_F32, false>(a, st);
    if (xm == X_F32 && xp == 1) return ep == EP_F16 ? launch_u<K, X_F32, 1, EP_F16, false>(a, st)
                                                    : launch_u<K, X_F32, 1, EP_F32, false>(a, st);
    if (xm == X_F32 && xp == 2) return ep == EP_F16 ? launch_u<K, X_F32, 2, EP_F16, false>(a, st)
                                                    : launch_u<K, X_F32, 2, EP_F32, false>(a, st);
  }
  if constexpr (K == 1024) {
    if (xm == X_RMS && ep == EP_F32 && !pair)
      return xp == 2 ? launch_u<K, X_RMS, 2, EP_F32, false>(a, st) : launch_u<K, X_RMS, 1, EP_F32, false>(a, st);
    if (xm == X_RMS && ep == EP_SWIGLU && pair)
      return xp == 2 ? launch_u<K, X_RMS, 2, EP_SWIGLU, true>(a, st) : launch_u<K, X_RMS, 1, EP_SWIGLU, true>(a, st);
    if (xm == X_RMS && ep == EP_ARGMAX && !pair)
      return xp == 2 ? launch_u<K, X_RMS, 2, EP_ARGMAX, false>(a, st) : launch_u<K, X_RMS, 1, EP_ARGMAX, false>(a, st);
  }
  if constexpr (K == 2048 || K == 3072) {
    if (xm == X_F32 && ep == EP_RESID && !pair)
      return xp == 2 ? launch_u<K, X_F32, 2, EP_RESID, false>(a, st) : launch_u<K, X_F32, 1, EP_RESID, false>(a, st);
  }
  return Q4D_ERR_SHAPE;
}

// Environment-free default: fp32 activations enter the GEMV as hi+lo fp16 pairs.
int launch_gemv_xp(const GemvArgs& a, int xm, int xp, int ep, bool pair, hipStream_t st) {
  if (a.cols != 1024 && a.cols != 2048 && a.cols != 3072) return Q4D_ERR_SHAPE;
  if (a.nseg < 1 || a.nseg > 3 || a.rows <= 0 || a.batch <= 0) return Q4D_ERR_SHAPE;
  const int rg = (a.cols == 2048) ? 1 : 2;
  if (pair) {
    if (a.cols != 1024 || a.nseg != 2) return Q4D_ERR_SHAPE;
  } else {
    if (a.rows % rg) return Q4D_ERR_SHAPE;
    for (int i = 0; i < a.nseg; ++i)
      if (a.seg_end[i] % rg) return Q4D_ERR_SHAPE;
    if (a.seg_end[a.nseg - 1] != a.rows) return Q4D_ERR_SHAPE;
  }
  for (int i = 0; i < a.nseg; ++i) {
    if (!a.w[i] || !a.s[i]) return Q4D_ERR_NULL;
    if (!aligned(a.w[i], 16) || !aligned(a.s[i], 2)) return Q4D_ERR_BAD_ADDR;
  }
  if (!a.x || (!a.y && ep != EP_ARGMAX)) return Q4D_ERR_NULL;
  if (!aligned(a.x, 16)) return Q4D_ERR_BAD_ADDR;
  if (xm == X_RMS && (!a.gamma || !aligned(a.gamma, 16))) return Q4D_ERR_NULL;
  if (ep == EP_RESID && !a.resid) return Q4D_ERR_NULL;
  if (ep == EP_ARGMAX && (!a.lm_part || !a.counter || !a.out_token || !a.out_score || a.batch != 1))
    return Q4D_ERR_NULL;
  if (xm == X_F16 && xp != 1) return Q4D_ERR_DTYPE;
  switch (a.cols) {
    case 1024: return dispatch_k<1024>(a, xm, xp, ep, pair, st);
    case 2048: return dispatch_k<2048>(a, xm, xp, ep, pair, st);
    default: return dispatch_k<3072>(a, xm, xp, ep, pair, st);
  }
}

int launch_gemv(const GemvArgs& a, int xmode, int epmode, bool pair, hipStream_t stream) {
  return launch_gemv_xp(a, xmode, xmode == X_F16 ? 1 : 2, epmode, pair, stream);
}

}  // namespace q4d
