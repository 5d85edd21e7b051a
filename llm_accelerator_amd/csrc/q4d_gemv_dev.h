// Device building blocks of the Q4 GEMVs (the one-shot decode kernels and the
// streaming LM head of q4d_gemv.hip): buffer-resource weight tiles (2 rows x 1024 columns per wave, lane l reads
// the 16-byte chunk l % 32 of row l / 32 and the word holding its Q2.14
// scale), the hi/lo dequant dot products, and the block-cooperative
// activation staging in LDS (stage x and gamma, RMSNorm, conversion into the
// fp16 pair order the dequant trick consumes, per-chunk sums).
#pragma once

#include <math.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

namespace {

constexpr int kRsrcFlags = 0x00020000;

typedef __amdgpu_buffer_rsrc_t Rsrc;

__device__ __forceinline__ Rsrc make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcFlags);
}

// One tile's weight chunk and the 32-bit word holding this lane's scale code
// (two consecutive Q2.14 codes; the lane's half is chosen by the shift).
struct TileData {
  u32x4 w;
  uint32_t s;
};

// Per-lane constant parts of a one-shot tile load.
struct LaneOff {
  uint32_t w;  // byte offset of the lane's chunk inside the tile's row pair
  uint32_t s;  // byte offset of the lane's scale word
  int sshift;  // bit offset of the lane's scale code inside that word
};

template <int K>
__device__ __forceinline__ LaneOff lane_off(int ks, int lane) {
  const int r = lane >> 5;
  const int c = ks * 32 + (lane & 31);  // 16-byte chunk within the row
  LaneOff o;
  o.w = (uint32_t)(r * (K / 2) + c * 16);
  o.s = (uint32_t)(r * (K / 32) + (c >> 2) * 4);
  o.sshift = ((c >> 1) & 1) * 16;
  return o;
}

// Cache-policy bits of a buffer load: non-temporal.  Weights and their scales are
// read once per step; as non-temporal loads the 3072 x 1024 GEMV takes 2.38 instead
// of 2.85 us from HBM (no change when the matrix is cache-resident).
constexpr int kLoadNT = 2;

// Load tile rows (lrow0, lrow0 + 1) of one matrix (lrow0 uniform).
template <int K>
__device__ __forceinline__ TileData load_rows(Rsrc rw, Rsrc rs, int lrow0, const LaneOff& o) {
  TileData d;
  d.w = __builtin_amdgcn_raw_buffer_load_b128(rw, o.w, (uint32_t)lrow0 * (K / 2), kLoadNT);
  d.s = __builtin_amdgcn_raw_buffer_load_b32(rs, o.s, (uint32_t)lrow0 * (K / 32), kLoadNT);
  return d;
}

// Segment resources are separate scalars selected with uniform conditions:
// held in an array, the select becomes a dynamic index into a private copy.
#define SEG_RS rw0, rw1, rw2, rs0, rs1, rs2, e0, e1
template <int K>
__device__ __forceinline__ TileData load_tile(int t, const LaneOff& o, Rsrc rw0, Rsrc rw1, Rsrc rw2, Rsrc rs0,
                                              Rsrc rs1, Rsrc rs2, int e0, int e1) {
  const int row0 = 2 * t;
  const bool in0 = row0 < e0, in1 = row0 < e1;
  const Rsrc rw = in0 ? rw0 : (in1 ? rw1 : rw2);
  const Rsrc rs = in0 ? rs0 : (in1 ? rs1 : rs2);
  return load_rows<K>(rw, rs, row0 - (in0 ? 0 : (in1 ? e0 : e1)), o);
}

// hi/lo variant of chunk_dot sharing the dequant masks.
__device__ __forceinline__ float chunk_dot_hl(const u32x4 w, const XChunk& h, const XChunk& l) {
  float a = 0.f, b = 0.f, c = 0.f, d = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t v = w[m], t = v >> 8;
    const uint32_t m0 = (v ^ 0x88888888u) & 0x000F000Fu, m1 = (v ^ 0x88888888u) & 0x00F000F0u;
    const uint32_t m2 = (t ^ 0x00888888u) & 0x000F000Fu, m3 = (t ^ 0x00888888u) & 0x00F000F0u;
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

// Row sums of one tile: lanes 16-31 hold row 0, lanes 48-63 row 1.
template <int XP>
__device__ __forceinline__ float tile_rows(const TileData& d, int sshift, const XChunk& xh, const XChunk& xl) {
  float p;
  if constexpr (XP == 2)
    p = chunk_dot_hl(d.w, xh, xl);
  else
    p = chunk_dot(d.w, xh);
  p *= scale_q2_14((d.s >> sshift) & 0xFFFFu);
  return half_wave_sum_dpp(p);
}

// Order-preserving 64-bit argmax key: higher score first, then lower index.
// NaN never wins (as with the reference's strict greater-than scan) and
// -0 compares equal to +0.
__device__ __forceinline__ unsigned long long argmax_key(float s, int idx) {
  if (!(s == s)) s = -INFINITY;
  s = s + 0.0f;
  const uint32_t b = __float_as_uint(s);
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)o << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ void argmax_unkey(unsigned long long k, float* s, int* idx) {
  const uint32_t o = (uint32_t)(k >> 32);
  const uint32_t b = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
  *s = __uint_as_float(b);
  *idx = (int)(0xFFFFFFFFu - (uint32_t)k);
}

__device__ __forceinline__ uint32_t pack_h2(_Float16 lo, _Float16 hi) {
  return __builtin_bit_cast(uint32_t, make_h2(lo, hi));
}

// ---- activation prologue ------------------------------------------------------
// Prologues that apply an RMSNorm (with gamma) to the activations.
constexpr bool rms_mode(int xm) { return xm == X_RMS || xm == X_EMB; }

// LDS a block needs for K columns of activations.
template <int K, int NWB, int XM, int XP>
struct ActLds {
  static constexpr int XV = (XM == X_F16) ? K / 8 : K / 4;  // 16-byte vectors of x
  static constexpr int CH = K / 32;                         // 32-column chunks
  f32x4 x[XV];
  f32x4 g[rms_mode(XM) ? XV : 1];
  alignas(16) uint32_t ph[CH * 16];                // hi pairs, dequant order
  alignas(16) uint32_t pl[XP == 2 ? CH * 16 : 4];  // lo pairs
  float2 sm[CH];                                   // 8 * chunk sums (hi, lo)
  float red[NWB];
};

template <int K, int NWB, int XM, int XP>
struct ActRegs {
  static constexpr int XV = ActLds<K, NWB, XM, XP>::XV;
  static constexpr int XPT = (XV + NWB * 64 - 1) / (NWB * 64);  // vectors per thread
  f32x4 x[XPT];
  f32x4 g[rms_mode(XM) ? XPT : 1];
  // X_EMB: the raw embedding codes (4 nibbles) and scale code of each vector
  uint32_t ec[XM == X_EMB ? XPT : 1];
  uint32_t es[XM == X_EMB ? XPT : 1];
};

// Stage x (and gamma) in LDS, reduce sum(x^2) for the RMSNorm, and convert
// the vector into the dequant pair order.  Chunk c holds columns
// 32c..32c+31; pair p = 4m + i of the chunk is (x[32c + 8m + i],
// x[32c + 8m + i + 4]).  Thread q handles pairs 4m + i0 and 4m + i0 + 1 of
// chunk q / 8 (m = (q % 8) / 2, i0 = 2 (q % 2)), so the 8 threads of a chunk
// are 8 consecutive lanes.  Both barriers are LDS-only: the weight loads
// issued before this stay in flight.
template <int K, int NWB, int XM, int XP>
__device__ __forceinline__ void act_prepare(float eps, const ActRegs<K, NWB, XM, XP>& r,
                                            ActLds<K, NWB, XM, XP>& s) {
  using R = ActRegs<K, NWB, XM, XP>;
  constexpr int NT = NWB * 64, CH = K / 32;
  const int lane = threadIdx.x & 63;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < R::XPT; ++i) {
    const int v = threadIdx.x + i * NT;
    if (v < R::XV) {
      s.x[v] = r.x[i];
      if constexpr (rms_mode(XM)) {
        s.g[v] = r.g[i];
        ss = fmaf(r.x[i][0], r.x[i][0], ss);
        ss = fmaf(r.x[i][1], r.x[i][1], ss);
        ss = fmaf(r.x[i][2], r.x[i][2], ss);
        ss = fmaf(r.x[i][3], r.x[i][3], ss);
      }
    }
  }
  if constexpr (rms_mode(XM)) {
    ss = wave_sum_dpp(ss);
    if (lane == 63) s.red[threadIdx.x >> 6] = ss;
  }
  block_sync_lds();

  float inv_rms = 1.f;
  if constexpr (rms_mode(XM)) {
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < NWB; ++w) tot += s.red[w];
    inv_rms = 1.0f / sqrtf(tot / (float)K + eps);
  }
  const float* sxf = reinterpret_cast<const float*>(s.x);
  const float* sgf = reinterpret_cast<const float*>(s.g);
  const _Float16* sxh = reinterpret_cast<const _Float16*>(s.x);
  for (int q = threadIdx.x; q < CH * 8; q += NT) {
    const int c = q >> 3, m = (q & 7) >> 1, i0 = (q & 1) * 2;
    const int ea = c * 32 + m * 8 + i0, eb = ea + 4;
    _Float16 h[4];  // pairs (h[0], h[1]) and (h[2], h[3])
    _Float16 l[4];
    if constexpr (XM == X_F16) {
      h[0] = sxh[ea];
      h[1] = sxh[eb];
      h[2] = sxh[ea + 1];
      h[3] = sxh[eb + 1];
    } else {
      float v[4] = {sxf[ea], sxf[eb], sxf[ea + 1], sxf[eb + 1]};
      if constexpr (rms_mode(XM)) {
        v[0] = (v[0] * inv_rms) * sgf[ea];
        v[1] = (v[1] * inv_rms) * sgf[eb];
        v[2] = (v[2] * inv_rms) * sgf[ea + 1];
        v[3] = (v[3] * inv_rms) * sgf[eb + 1];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // The hi / lo split needs every use of v to see one fp32 number.  Left
        // visible, the product above goes into hi's fp16 conversion as one fused
        // rounding (v_fma_mix) while the stored pair takes the fp32 product, so at
        // fp16 rounding ties hi, lo and the chunk sums disagree by one fp16 ulp of
        // hi (found as a 1e-3 relative error of a gate/up row); the empty asm makes
        // the rounded fp32 value the only one.
        asm("" : "+v"(v[j]));
        h[j] = (_Float16)v[j];
        if constexpr (XP == 2) l[j] = (_Float16)(v[j] - (float)h[j]);
      }
    }
    float sh = ((float)h[0] + (float)h[1]) + ((float)h[2] + (float)h[3]);
    float sl = 0.f;
    *reinterpret_cast<u32x2*>(&s.ph[c * 16 + m * 4 + i0]) = u32x2{pack_h2(h[0], h[1]), pack_h2(h[2], h[3])};
    if constexpr (XP == 2) {
      sl = ((float)l[0] + (float)l[1]) + ((float)l[2] + (float)l[3]);
      *reinterpret_cast<u32x2*>(&s.pl[c * 16 + m * 4 + i0]) = u32x2{pack_h2(l[0], l[1]), pack_h2(l[2], l[3])};
    }
    // chunk sums over its 8 consecutive lanes
    sh += dpp_f<kDppQuadSwap1>(sh);
    sh += dpp_f<kDppQuadSwap2>(sh);
    sh += dpp_f<kDppRowHalfMirror>(sh);
    if constexpr (XP == 2) {
      sl += dpp_f<kDppQuadSwap1>(sl);
      sl += dpp_f<kDppQuadSwap2>(sl);
      sl += dpp_f<kDppRowHalfMirror>(sl);
    }
    if ((q & 7) == 0) s.sm[c] = make_float2(8.f * sh, 8.f * sl);
  }
  block_sync_lds();
}

// The prepared hi (and lo) chunk c.
template <int K, int NWB, int XM, int XP>
__device__ __forceinline__ void act_chunk(const ActLds<K, NWB, XM, XP>& s, int c, XChunk& xh, XChunk& xl) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4 t = reinterpret_cast<const u32x4*>(&s.ph[c * 16])[j];
#pragma unroll
    for (int e = 0; e < 4; ++e) xh.p[4 * j + e] = __builtin_bit_cast(h2, (uint32_t)t[e]);
    if constexpr (XP == 2) {
      const u32x4 t2 = reinterpret_cast<const u32x4*>(&s.pl[c * 16])[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) xl.p[4 * j + e] = __builtin_bit_cast(h2, (uint32_t)t2[e]);
    }
  }
  const float2 sm = s.sm[c];
  xh.sum8 = sm.x;
  xl.sum8 = sm.y;
}

}  // namespace

}  // namespace q4d
