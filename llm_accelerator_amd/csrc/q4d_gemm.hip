// Q4 weight GEMM on MFMA for prefill and batched decode (gfx950).
//
//   Y[M, N] = X[M, K] . W[N, K]^T,   X fp16, W Q4 (reference Source/Q4_FORMAT.md)
//
// When many activation rows share each weight (prefill, batched decode), the
// work becomes a dense contraction: each 128(N) x 64(K) Q4 tile (one scale
// group per row) is dequantised once per block into LDS as fp16 and read by
// every MFMA of the block.  Dequantisation uses packed fp16: after
// v = w ^ 0x88888888 the nibble u = q + 8 placed in the low byte of an fp16
// with exponent bits 0x6400 reads 1024 + u, so (0x6400|u) - 1032 = q exactly,
// and q * scale is one correctly rounded fp16 multiply (the scale code is an
// exact fp16 below 2048, i.e. scale < 0.125).
//
// Block tile 128 (M, BM = 128) or 64 (BM = 64) x 128 (N) x 64 (K), 256 threads
// = 2 x 2 waves; each wave owns (BM/2) x 64 of the output as 16x16 tiles of
// v_mfma_f32_16x16x32_f16 with fp32 accumulation.  LDS is double-buffered:
// the global loads of the next K step are issued before the MFMAs of the
// current one.
//
// Epilogues: fp32 / fp16 store, residual add (common.py:284,297), SwiGLU of a
// gate/up row pair (common.py:293-295; the B tile then holds 64 gate rows and
// the matching 64 up rows), per-row argmax partials over the block's columns
// for the batched LM head (lowest index wins ties), and prefill's q|k|v heads:
// q/k RMSNorm + RoPE + K/V append straight from the accumulators (EP_ROPE).
//
// Split-K: when the output tiles alone cannot fill the device (batched
// decode: M = 64 rows, N = 1024 gives 8 tiles), blockIdx.z takes a
// contiguous range of the K steps and stores its raw fp32 tile; a second
// kernel adds the splits in order (deterministic) and applies the epilogue.
#include <math.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kGemmBN = 128;
// waves per block for 128- and 64-row tiles
constexpr int kGemmWaves128 = 8;
constexpr int kGemmWaves64 = 8;
constexpr int kGemmBK = 64;
// fp16 elements of padding per LDS row (row stride 80 = 160 B): of 8 / 16 / 24 / 40 the
// fastest on the prefill projections (fewer store bank conflicts than 72)
constexpr int kGemmPad = 16;
constexpr int kGemmLds = kGemmBK + kGemmPad;

// Dequantise 8 consecutive int4 (one 32-bit word, low nibble first) times `scale` to
// fp16, in column order: word p of the result holds columns 2p, 2p + 1.
__device__ __forceinline__ u32x4 dequant8(uint32_t w, h2 scale2) {
  const h2 bias = make_h2((_Float16)1032.0f, (_Float16)1032.0f);
  const uint32_t v = w ^ 0x88888888u;
  const uint32_t lo = v & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6 in bytes 0..3
  const uint32_t hi = (v >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
  u32x4 out;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    // fp16 pair (nibble 2p, nibble 2p+1): low byte of each half from lo / hi byte p
    const uint32_t sel = (uint32_t)(p) | (0x0Cu << 8) | ((uint32_t)(4 + p) << 16) | (0x0Cu << 24);
    const uint32_t pr = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
    const h2 q = __builtin_bit_cast(h2, pr) - bias;
    out[p] = __builtin_bit_cast(uint32_t, q * scale2);
  }
  return out;
}

// Dequantise 32 consecutive int4 (one 16-byte chunk) times `scale` to fp16,
// in column order.
__device__ __forceinline__ void dequant32(const u32x4 w, h2 scale2, uint32_t (&out)[16]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const u32x4 o = dequant8(w[m], scale2);
#pragma unroll
    for (int p = 0; p < 4; ++p) out[4 * m + p] = o[p];
  }
}

struct GemmTileLoad {
  u32x4 x[4];  // up to 4 x 16 B of X per thread
  u32x4 w;     // 16 B of Q4 codes
  uint32_t s;  // the row's scale code for this K step
};

// Segment pointers read with constant indices and selected in registers;
// indexing a.w[] with a runtime segment number copies the argument block to
// scratch memory.
struct SegPtrs {
  const uint8_t* w0;
  const uint8_t* w1;
  const uint8_t* w2;
  const uint16_t* s0;
  const uint16_t* s1;
  const uint16_t* s2;
  int e0, e1;
};

__device__ __forceinline__ SegPtrs seg_ptrs(const GemmArgs& a) {
  return SegPtrs{a.w[0], a.w[1], a.w[2], a.s[0], a.s[1], a.s[2], a.seg_end[0], a.seg_end[1]};
}

template <int BM, bool PAIR, int NT>
__device__ __forceinline__ void gemm_load(const GemmArgs& a, const SegPtrs& P, int m0, int nblk, int k0, int t,
                                          GemmTileLoad& L) {
  // X: BM x 64 fp16 = BM * 8 chunks of 16 B, spread over the NT threads
#pragma unroll
  for (int i = 0; i < BM * 8 / NT; ++i) {
    const int c = t + NT * i;
    const int row = c >> 3, seg = c & 7;
    const int m = m0 + row;
    if (m < a.M)
      L.x[i] = *reinterpret_cast<const u32x4*>(a.x + (size_t)m * a.K + k0 + seg * 8);
    else
      L.x[i] = u32x4{0u, 0u, 0u, 0u};
  }
  // W: 128 rows x 32 B; thread t < 256 -> row t/2, half t%2 (the first four waves)
  if (t >= 256) return;
  const int r = t >> 1, half = t & 1;
  const uint8_t* wb;
  const uint16_t* sb;
  int grow;
  if (PAIR) {
    const int n0 = nblk * 64;
    const int sg = r >> 6;
    grow = n0 + (r & 63);
    wb = sg == 0 ? P.w0 : P.w1;
    sb = sg == 0 ? P.s0 : P.s1;
  } else {
    const int row = nblk * kGemmBN + r;
    if (row < P.e0) {
      grow = row;
      wb = P.w0;
      sb = P.s0;
    } else if (row < P.e1) {
      grow = row - P.e0;
      wb = P.w1;
      sb = P.s1;
    } else {
      grow = row - P.e1;
      wb = P.w2;
      sb = P.s2;
    }
  }
  L.w = *reinterpret_cast<const u32x4*>(wb + (size_t)grow * (a.K / 2) + k0 / 2 + half * 16);
  L.s = sb[(size_t)grow * (a.K / 64) + k0 / 64];
}

template <int BM, int NT>
__device__ __forceinline__ void gemm_store_lds(_Float16 (*As)[kGemmLds], _Float16 (*Bs)[kGemmLds], int t,
                                               const GemmTileLoad& L) {
#pragma unroll
  for (int i = 0; i < BM * 8 / NT; ++i) {
    const int c = t + NT * i;
    *reinterpret_cast<u32x4*>(&As[c >> 3][(c & 7) * 8]) = L.x[i];
  }
  if (t >= 256) return;
  const int r = t >> 1, half = t & 1;
  const _Float16 sc = (_Float16)((float)L.s * (1.0f / 16384.0f));
  uint32_t out[16];
  dequant32(L.w, make_h2(sc, sc), out);
  u32x4* dst = reinterpret_cast<u32x4*>(&Bs[r][half * 32]);
#pragma unroll
  for (int q = 0; q < 4; ++q) dst[q] = u32x4{out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]};
}

// ---- q|k|v epilogue of prefill (EP_ROPE) -------------------------------------------
// An output tile's 128 columns are one head (head_dim = the N tile): head h = nblk,
// q heads [0, qh), k heads [qh, qh + kvh), v heads after.  Per token row, q and k get
// the per-head RMSNorm (common.py:258-262) and RoPE (common.py:264-268); q, scaled by
// attention scaling * log2(e), goes to q16[h][token] as fp16; k and v go to the fp16
// cache at position p0 + token (append_cache, common.py:186-189).  The tile's columns
// are dealt to the waves as for a gate/up pair: wave wn holds dims d = 32 wn + 16 j + cl
// (j = 0, 1) in acc[.][j] and their rotate-half partners d + 64 in acc[.][j + 2], so
// the rotation is lane-local; the sum of squares of a row is a 16-lane reduction per
// wave plus one exchange through LDS between the two waves of the row.
template <int BM, int MI>
__device__ __forceinline__ void rope_epilogue(const GemmArgs& a, const f32x4 (&acc)[MI][4], float* ssx, int m0,
                                              int nblk, int wm, int wn, int lane) {
  const PrefillArgs& R = a.rope;
  const int h = nblk, cl = lane & 15, rq = (lane >> 4) * 4;
  if (h >= R.qh + R.kvh) {  // v head: fp16 into the cache
    uint16_t* vb = R.vcache + (size_t)(h - R.qh - R.kvh) * R.max_ctx * kGemmBN;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = m0 + wm + 16 * i + rq + r;
        if (tok >= a.M) continue;
        uint16_t* dst = vb + (size_t)(R.p0 + tok) * kGemmBN;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int d = 32 * wn + 16 * j + cl;
          dst[d] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][j][r]);
          dst[d + 64] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][j + 2][r]);
        }
      }
    return;
  }
  const bool isq = h < R.qh;
  const float* gam = isq ? R.q_gamma : R.k_gamma;
  float g0[2], g1[2], cs[MI][4][2], sn[MI][4][2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    g0[j] = gam[32 * wn + 16 * j + cl];
    g1[j] = gam[64 + 32 * wn + 16 * j + cl];
  }
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int tok = m0 + wm + 16 * i + rq + r;
      tok = tok < a.M ? tok : a.M - 1;
      const size_t tb = (size_t)(R.p0 + tok) * (kGemmBN / 2) + 32 * wn + cl;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        cs[i][r][j] = R.rope_cos[tb + 16 * j];
        sn[i][r][j] = R.rope_sin[tb + 16 * j];
      }
    }
  // sum of squares of each row over this wave's 64 columns, then over both waves
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = acc[i][0][r] * acc[i][0][r];
      v = fmaf(acc[i][1][r], acc[i][1][r], v);
      v = fmaf(acc[i][2][r], acc[i][2][r], v);
      v = fmaf(acc[i][3][r], acc[i][3][r], v);
      v = row16_sum(v);
      if (cl == 0) ssx[wn * BM + wm + 16 * i + rq + r] = v;
    }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = wm + 16 * i + rq + r, tok = m0 + row;
      if (tok >= a.M) continue;
      const float ss = ssx[row] + ssx[BM + row];
      const float inv = 1.0f / sqrtf(ss / (float)kGemmBN + R.eps);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int d = 32 * wn + 16 * j + cl;
        const float n0 = (acc[i][j][r] * inv) * g0[j], n1 = (acc[i][j + 2][r] * inv) * g1[j];
        // rotate_half: dim d < 64 takes -x[d + 64], dim d + 64 takes x[d]
        const float r0 = n0 * cs[i][r][j] - n1 * sn[i][r][j];
        const float r1 = n1 * cs[i][r][j] + n0 * sn[i][r][j];
        if (isq) {
          _Float16* dst = R.q16 + ((size_t)h * R.n + tok) * kGemmBN;
          dst[d] = (_Float16)(r0 * R.qscale);
          dst[d + 64] = (_Float16)(r1 * R.qscale);
        } else {
          uint16_t* dst = R.kcache + ((size_t)(h - R.qh) * R.max_ctx + R.p0 + tok) * kGemmBN;
          dst[d] = __builtin_bit_cast(uint16_t, (_Float16)r0);
          dst[d + 64] = __builtin_bit_cast(uint16_t, (_Float16)r1);
        }
      }
    }
}

// NW waves per block: NW / 2 along M x 2 along N; each wave owns
// (BM / (NW / 2)) x 64 of the output.
template <int BM, int EP, bool PAIR, int NW>
__global__ __launch_bounds__(NW * 64) void q4_gemm_kernel(const GemmArgs a) {
  constexpr int NT = NW * 64;
  constexpr int WM = BM / (NW / 2);  // rows per wave
  constexpr int MI = WM / 16;        // 16-row MFMA tiles per wave
  constexpr int NI = 4;              // 16-col MFMA tiles per wave (64 columns)
  static_assert(MI >= 1 && BM * 8 % NT == 0, "tile / wave split");
  __shared__ _Float16 As[2][BM][kGemmLds];
  __shared__ _Float16 Bs[2][kGemmBN][kGemmLds];
  __shared__ float s_best[2][BM];
  __shared__ int s_bidx[2][BM];

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int wm = (w >> 1) * WM, wn = (w & 1);
  // XCD-aware tile order: linear block b runs on XCD b % 8, and each XCD has its
  // own L2.  Tiles are numbered n fastest, then m, then the K split, and XCD x
  // takes the x-th contiguous eighth of them, so its blocks share a few rows of
  // X (and a K range) instead of each XCD reading all of X.
  int nblk = blockIdx.x, mblk = blockIdx.y, z = blockIdx.z;
  {
    const int gx = gridDim.x, gy = gridDim.y, total = gx * gy * (int)gridDim.z;
    if ((total & 7) == 0) {
      const int lin = (int)blockIdx.x + gx * ((int)blockIdx.y + gy * (int)blockIdx.z);
      const int v = (lin & 7) * (total >> 3) + (lin >> 3);
      nblk = v % gx;
      mblk = (v / gx) % gy;
      z = v / (gx * gy);
    }
  }
  const int m0 = mblk * BM;
  // K steps [k_begin, k_end) of this split
  const int nk_all = a.K / kGemmBK, ksplit = gridDim.z;
  const int k_begin = z * nk_all / ksplit;
  const int nk = (z + 1) * nk_all / ksplit - k_begin;

  f32x4 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // B-tile rows read by this wave's four 16-col tiles (a gate/up pair and EP_ROPE:
  // 32 columns from each half of the tile)
  int brow[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j)
    brow[j] = PAIR || EP == EP_ROPE ? ((j < 2) ? (32 * wn + 16 * j) : (64 + 32 * wn + 16 * (j - 2)))
                                    : (64 * wn + 16 * j);

  const SegPtrs P = seg_ptrs(a);
  GemmTileLoad L;
  gemm_load<BM, PAIR, NT>(a, P, m0, nblk, k_begin * kGemmBK, t, L);
  gemm_store_lds<BM, NT>(As[0], Bs[0], t, L);
  __syncthreads();

  for (int ks = 0; ks < nk; ++ks) {
    const int buf = ks & 1;
    if (ks + 1 < nk) gemm_load<BM, PAIR, NT>(a, P, m0, nblk, (k_begin + ks + 1) * kGemmBK, t, L);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int kc = kk * 32 + (lane >> 4) * 8;
      h8 bf[NI];
#pragma unroll
      for (int j = 0; j < NI; ++j) bf[j] = *reinterpret_cast<const h8*>(&Bs[buf][brow[j] + (lane & 15)][kc]);
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const h8 af = *reinterpret_cast<const h8*>(&As[buf][wm + 16 * i + (lane & 15)][kc]);
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
    if (ks + 1 < nk) gemm_store_lds<BM, NT>(As[buf ^ 1], Bs[buf ^ 1], t, L);
    __syncthreads();
  }

  // ---- epilogue: lane holds rows (lane/16)*4 + r of each 16x16 tile, column lane%16
  if constexpr (EP == EP_ROPE) {  // no split (the launcher checks)
    rope_epilogue<BM, MI>(a, acc, reinterpret_cast<float*>(&Bs[0][0][0]), m0, nblk, wm, wn, lane);
    return;
  }
  const int cl = lane & 15, rq = (lane >> 4) * 4;
  if (EP != EP_ARGMAX && ksplit > 1) {
    // raw split tile: [z][m][n], PAIR: gate columns n, up columns N + n
    const int wp = PAIR ? 2 * a.N : a.N;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int n = PAIR ? (j < 2 ? 0 : a.N) + nblk * 64 + 32 * wn + 16 * (j & 1) + cl
                           : nblk * kGemmBN + 64 * wn + 16 * j + cl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + rq + r;
          if (m < a.M) a.part[((size_t)z * a.M + m) * wp + n] = acc[i][j][r];
        }
      }
    return;
  }
  if constexpr (EP == EP_SWIGLU) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = nblk * 64 + 32 * wn + 16 * j + cl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + rq + r;
          if (m < a.M) {
            const float g = acc[i][j][r], u = acc[i][j + 2][r];
            const float act = (g / (1.0f + expf(-g))) * u;
            static_cast<_Float16*>(a.y)[(size_t)m * a.ldy + n] = (_Float16)act;
          }
        }
      }
  } else if constexpr (EP == EP_ARGMAX) {
    // per row: best (score, column) over this wave's 64 columns, then over the block's two N-waves
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int lrow = wm + 16 * i + rq + r;
        float bs = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int n = nblk * kGemmBN + 64 * wn + 16 * j + cl;
          const float v = acc[i][j][r];
          if (a.logits && m0 + lrow < a.M) a.logits[(size_t)(m0 + lrow) * a.N + n] = v;
          if (arg_better(v, n, bs, bi)) {
            bs = v;
            bi = n;
          }
        }
        // the 16 lanes sharing this row differ in lane & 15
#pragma unroll
        for (int msk = 8; msk >= 1; msk >>= 1) {
          const float os = shfl_xor_f(bs, msk);
          const int oi = __shfl_xor(bi, msk, kWave);
          if (arg_better(os, oi, bs, bi)) {
            bs = os;
            bi = oi;
          }
        }
        if (cl == 0) {
          s_best[wn][lrow] = bs;
          s_bidx[wn][lrow] = bi;
        }
      }
    __syncthreads();
    for (int lr = t; lr < BM; lr += NT) {
      const int m = m0 + lr;
      if (m < a.M) {
        float bs = s_best[0][lr];
        int bi = s_bidx[0][lr];
        if (arg_better(s_best[1][lr], s_bidx[1][lr], bs, bi)) {
          bs = s_best[1][lr];
          bi = s_bidx[1][lr];
        }
        a.part_score[(size_t)m * gridDim.x + nblk] = bs;
        a.part_idx[(size_t)m * gridDim.x + nblk] = bi;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int n = nblk * kGemmBN + 64 * wn + 16 * j + cl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + rq + r;
          if (m < a.M) {
            const size_t o = (size_t)m * a.ldy + n;
            const float v = acc[i][j][r];
            if constexpr (EP == EP_F16)
              static_cast<_Float16*>(a.y)[o] = (_Float16)v;
            else if constexpr (EP == EP_RESID)
              static_cast<float*>(a.y)[o] = a.resid[o] + v;
            else
              static_cast<float*>(a.y)[o] = v;
          }
        }
      }
  }
}

// ---- pipelined kernel for large M (prefill) --------------------------------------
// Block tile 128 (M) x 128 (N) x 64 (K), 8 waves as in q4_gemm_kernel<128> (same
// MFMA sequence, so the same sums bit for bit), one block per CU.  The raw tiles
// of a K step -- 128 rows of fp16 X and 128 rows of Q4 codes -- go global -> LDS
// with global_load_lds_dwordx4, three K steps ahead, into a ring of four stages:
// no registers hold data in flight and the loads of three steps overlap the
// MFMAs.  One step ahead the codes of a stage are dequantised into an fp16 B
// tile (two buffers); step k's MFMAs read X from its raw stage and B from its
// fp16 tile.  One barrier per K step orders the stages:
//   wait for this wave's loads of step k+1, barrier,
//   issue the loads of step k+3 (into the stage of step k-1, read by then),
//   dequantise step k+1 (into the B tile step k-1 used), MFMAs of step k.
// A DMA wave writes 64 consecutive 16-byte slots, so an X row is 8 slots of
// 128 B with no padding; slot g of row r holds column group g ^ (r & 7), which
// spreads the 16 rows a fragment read touches over the banks.  Steps past the
// last reload the last one (the stage is not read again), so every wave issues
// the same number of loads per step and the waits are constants.
constexpr int kPipeMaxGroups = 48;  // K <= 3072: Q2.14 scales of the block's rows, all K steps

// 16 consecutive int4 (two words) times `scale` to fp16, in column order.
__device__ __forceinline__ void dequant16(uint32_t w0, uint32_t w1, h2 scale2, uint32_t (&out)[8]) {
  const h2 bias = make_h2((_Float16)1032.0f, (_Float16)1032.0f);
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const uint32_t v = (m ? w1 : w0) ^ 0x88888888u;
    const uint32_t lo = v & 0x0F0F0F0Fu;
    const uint32_t hi = (v >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t sel = (uint32_t)(p) | (0x0Cu << 8) | ((uint32_t)(4 + p) << 16) | (0x0Cu << 24);
      const uint32_t pr = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
      const h2 q = __builtin_bit_cast(h2, pr) - bias;
      out[4 * m + p] = __builtin_bit_cast(uint32_t, q * scale2);
    }
  }
}

// Row r (< 128) of the block's B tile: its segment's code / scale pointers and row.
template <bool PAIR>
__device__ __forceinline__ void pipe_brow(const SegPtrs& P, int nblk, int r, const uint8_t*& wb, const uint16_t*& sb,
                                          int& grow) {
  if (PAIR) {
    const bool up = r >= 64;
    grow = nblk * 64 + (r & 63);
    wb = up ? P.w1 : P.w0;
    sb = up ? P.s1 : P.s0;
  } else {
    const int row = nblk * kGemmBN + r;
    if (row < P.e0) {
      grow = row; wb = P.w0; sb = P.s0;
    } else if (row < P.e1) {
      grow = row - P.e0; wb = P.w1; sb = P.s1;
    } else {
      grow = row - P.e1; wb = P.w2; sb = P.s2;
    }
  }
}

// Wait until at most N of this wave's vector-memory loads are outstanding and
// its LDS operations are done, then barrier; the compiler sees a memory fence.
template <int N>
__device__ __forceinline__ void pipe_sync() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0070 | N);  // vmcnt(N) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS of the pipelined kernel.  Each stage is an object of its own: the
// compiler then knows that a load into one stage does not alias reads of
// another, and does not drain every load in flight before each LDS read.
struct PipeStage {
  _Float16 x[128][kGemmBK];         // X rows, 16-byte column groups swizzled by row
  uint8_t w[kGemmBN][kGemmBK / 2];  // Q4 codes
};
__shared__ __attribute__((aligned(16))) PipeStage g_ps0, g_ps1, g_ps2, g_ps3;
__shared__ __attribute__((aligned(16))) _Float16 g_pb0[kGemmBN][kGemmLds], g_pb1[kGemmBN][kGemmLds];
__shared__ uint16_t g_psc[kGemmBN][kPipeMaxGroups];

template <int S>
__device__ __forceinline__ PipeStage& pipe_stage() {
  if constexpr (S == 0) return g_ps0;
  else if constexpr (S == 1) return g_ps1;
  else if constexpr (S == 2) return g_ps2;
  else return g_ps3;
}
template <int S>
__device__ __forceinline__ _Float16 (&pipe_x())[128][kGemmBK] {
  return pipe_stage<S>().x;
}
template <int S>
__device__ __forceinline__ uint8_t (&pipe_w())[kGemmBN][kGemmBK / 2] {
  return pipe_stage<S>().w;
}
template <int B>
__device__ __forceinline__ _Float16 (&pipe_b())[kGemmBN][kGemmLds] {
  if constexpr (B == 0) return g_pb0;
  else return g_pb1;
}

// Per-thread state of the pipelined kernel.
struct PipeCtx {
  const _Float16* xsrc[2];  // this lane's X rows (clamped into M), column group applied
  const uint8_t* wsrc;      // waves 0-3: this lane's code row and half
  int w, t, lane, k_begin, nk;
};

// global_load_lds_dwordx4: lane i of the wave writes 16 bytes from `src` at LDS
// address lds + 16 i (lds wave-uniform, through M0).  Issued by inline asm so the
// compiler does not treat the LDS it writes as pending: it cannot tell the
// ring's stages apart and would drain every load in flight before LDS reads.
// The kernel orders these loads itself with explicit waits and barriers.
__device__ __forceinline__ void dma16(const void* src, void* lds) {
  const uint32_t off = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(off), "v"(src) : "memory");
}

// Raw tiles of local K step j (clamped to the last) into stage S.
template <int S>
__device__ __forceinline__ void pipe_issue(const PipeCtx& c, int j) {
  const int kstep = c.k_begin + (j < c.nk ? j : c.nk - 1);
#pragma unroll
  for (int i = 0; i < 2; ++i)
    dma16(c.xsrc[i] + kstep * kGemmBK, &pipe_x<S>()[16 * c.w + 8 * i][0]);
  if (c.w < 4) dma16(c.wsrc + kstep * (kGemmBK / 2), &pipe_w<S>()[32 * c.w][0]);
}

// Codes of local K step j (in stage S) -> fp16 B tile B.
template <int S, int B>
__device__ __forceinline__ void pipe_dequant(const PipeCtx& c, int j) {
  const int r = c.t >> 2, q = c.t & 3;
  const u32x2 raw = *reinterpret_cast<const u32x2*>(&pipe_w<S>()[r][8 * q]);
  const _Float16 sc = (_Float16)((float)g_psc[r][c.k_begin + j] * (1.0f / 16384.0f));
  uint32_t out[8];
  dequant16(raw[0], raw[1], make_h2(sc, sc), out);
  u32x4* dst = reinterpret_cast<u32x4*>(&pipe_b<B>()[r][16 * q]);
  dst[0] = u32x4{out[0], out[1], out[2], out[3]};
  dst[1] = u32x4{out[4], out[5], out[6], out[7]};
}

// MFMAs of one K step: X from stage S, B from tile B.
template <int S, int B, int MI, int NI>
__device__ __forceinline__ void pipe_mma(const PipeCtx& c, int wm, const int (&brow)[NI], f32x4 (&acc)[MI][NI]) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int kc = kk * 32 + (c.lane >> 4) * 8;
    h8 bf[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) bf[j] = *reinterpret_cast<const h8*>(&pipe_b<B>()[brow[j] + (c.lane & 15)][kc]);
    const int G = kk * 4 + (c.lane >> 4);
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int ar = wm + 16 * i + (c.lane & 15);
      const h8 af = *reinterpret_cast<const h8*>(&pipe_x<S>()[ar][(G ^ (ar & 7)) * 8]);
#pragma unroll
      for (int j = 0; j < NI; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
    }
  }
}

// One K step (local index k, its stage S = k % 4): this wave's loads of step k+1
// have landed and every wave wrote B tile k; the loads of step k+3 go out into
// the stage step k-1 used; step k+1 is dequantised; step k's MFMAs run.
template <int S, int MI, int NI>
__device__ __forceinline__ void pipe_step(const PipeCtx& c, int k, int wm, const int (&brow)[NI],
                                          f32x4 (&acc)[MI][NI]) {
  if (c.w < 4) pipe_sync<3>(); else pipe_sync<2>();
  pipe_issue<(S + 3) % 4>(c, k + 3);
  if (k + 1 < c.nk) pipe_dequant<(S + 1) % 4, (S + 1) & 1>(c, k + 1);
  pipe_mma<S, S & 1, MI, NI>(c, wm, brow, acc);
}

template <int EP, bool PAIR, int NK>
__global__ __launch_bounds__(512) void q4_gemm_pipe_kernel(const GemmArgs a) {
  constexpr int BM = 128, NW = 8, NT = NW * 64;
  constexpr int WM = BM / (NW / 2);  // 32 rows per wave
  constexpr int MI = WM / 16, NI = 4;
  static_assert(EP != EP_ARGMAX, "argmax tiles use q4_gemm_kernel");

  PipeCtx c;
  c.t = threadIdx.x;
  c.lane = c.t & 63;
  c.w = __builtin_amdgcn_readfirstlane(c.t >> 6);
  const int lane = c.lane, w = c.w, t = c.t;
  const int wm = (w >> 1) * WM, wn = w & 1;
  // XCD-aware tile order (as in q4_gemm_kernel)
  int nblk = blockIdx.x, mblk = blockIdx.y, z = blockIdx.z;
  {
    const int gx = gridDim.x, gy = gridDim.y, total = gx * gy * (int)gridDim.z;
    if ((total & 7) == 0) {
      const int lin = (int)blockIdx.x + gx * ((int)blockIdx.y + gy * (int)blockIdx.z);
      const int v = (lin & 7) * (total >> 3) + (lin >> 3);
      nblk = v % gx;
      mblk = (v / gx) % gy;
      z = v / (gx * gy);
    }
  }
  const int m0 = mblk * BM;
  const int nk_all = a.K / kGemmBK, ksplit = gridDim.z;
  c.k_begin = z * nk_all / ksplit;
  c.nk = NK;  // K steps of this split (the launcher picks the instance)
  const int ng = a.K / 64;
  const SegPtrs P = seg_ptrs(a);

  // Q2.14 scale codes of the block's B rows, every K step
  for (int idx = t; idx < kGemmBN * ng; idx += NT) {
    const int r = idx / ng, gi = idx - r * ng;
    const uint8_t* wb;
    const uint16_t* sb;
    int grow;
    pipe_brow<PAIR>(P, nblk, r, wb, sb, grow);
    g_psc[r][gi] = sb[(size_t)grow * ng + gi];
  }
  // this lane's DMA sources: X rows 16w + lane/8 and + 8, slot lane % 8 holding
  // column group (lane % 8) ^ (row & 7); waves 0-3: code row 32w + lane/2, half lane % 2
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 16 * w + (lane >> 3) + 8 * i;
    int m = m0 + r;
    m = m < a.M ? m : a.M - 1;
    c.xsrc[i] = reinterpret_cast<const _Float16*>(a.x) + (size_t)m * a.K + ((lane & 7) ^ (r & 7)) * 8;
  }
  c.wsrc = nullptr;
  if (w < 4) {
    const uint8_t* wb;
    const uint16_t* sb;
    int grow;
    pipe_brow<PAIR>(P, nblk, 32 * w + (lane >> 1), wb, sb, grow);
    c.wsrc = wb + (size_t)grow * (a.K / 2) + (lane & 1) * 16;
  }

  f32x4 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  int brow[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j)
    brow[j] = PAIR || EP == EP_ROPE ? ((j < 2) ? (32 * wn + 16 * j) : (64 + 32 * wn + 16 * (j - 2)))
                                    : (64 * wn + 16 * j);

  // scale codes stored; steps 0, 1, 2 go out; step 0 is dequantised once landed
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  pipe_issue<0>(c, 0);
  pipe_issue<1>(c, 1);
  pipe_issue<2>(c, 2);
  if (w < 4) pipe_sync<6>(); else pipe_sync<4>();
  pipe_dequant<0, 0>(c, 0);
  // fully unrolled: with a loop, the wait-count pass loses track at the loop
  // head of which stage each load in flight writes and drains them all
#pragma unroll
  for (int k = 0; k < NK; k += 4) {
    pipe_step<0>(c, k, wm, brow, acc);
    pipe_step<1>(c, k + 1, wm, brow, acc);
    pipe_step<2>(c, k + 2, wm, brow, acc);
    pipe_step<3>(c, k + 3, wm, brow, acc);
  }
  // every load of the ring has landed before the block's LDS is released
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) expcnt(7) lgkmcnt(0)

  // ---- epilogue (as in q4_gemm_kernel)
  if constexpr (EP == EP_ROPE) {  // no split (the launcher checks)
    __syncthreads();  // every wave's MFMAs are done with the B tiles
    rope_epilogue<BM, MI>(a, acc, reinterpret_cast<float*>(&g_pb0[0][0]), m0, nblk, wm, wn, lane);
    return;
  }
  const int cl = lane & 15, rq = (lane >> 4) * 4;
  if (ksplit > 1) {
    const int wp = PAIR ? 2 * a.N : a.N;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int n = PAIR ? (j < 2 ? 0 : a.N) + nblk * 64 + 32 * wn + 16 * (j & 1) + cl
                           : nblk * kGemmBN + 64 * wn + 16 * j + cl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + rq + r;
          if (m < a.M) a.part[((size_t)z * a.M + m) * wp + n] = acc[i][j][r];
        }
      }
    return;
  }
  if constexpr (EP == EP_SWIGLU) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = nblk * 64 + 32 * wn + 16 * j + cl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + rq + r;
          if (m < a.M) {
            const float g = acc[i][j][r], u = acc[i][j + 2][r];
            const float act = (g / (1.0f + expf(-g))) * u;
            static_cast<_Float16*>(a.y)[(size_t)m * a.ldy + n] = (_Float16)act;
          }
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int n = nblk * kGemmBN + 64 * wn + 16 * j + cl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + rq + r;
          if (m < a.M) {
            const size_t o = (size_t)m * a.ldy + n;
            const float v = acc[i][j][r];
            if constexpr (EP == EP_F16)
              static_cast<_Float16*>(a.y)[o] = (_Float16)v;
            else if constexpr (EP == EP_RESID)
              static_cast<float*>(a.y)[o] = a.resid[o] + v;
            else
              static_cast<float*>(a.y)[o] = v;
          }
        }
      }
  }
}

// ---- skinny GEMM: at most 64 activation rows (batched decode) -------------------------
// Y^T[n, m] = sum_k W[n, k] X[m, k] with the weights as the MFMA A operand (16 rows per
// block; a gate/up pair: 8 gate rows and the matching 8 up rows) and the activation rows
// as B (4 tiles of 16).  Each wave takes 128 consecutive columns of K and issues every
// load of its work at entry: one 16-byte chunk of codes per lane straight into registers
// (no LDS for the weights), the two scale codes of its row, and 16 x 16 bytes of X; a
// block of NW waves covers 128 NW columns (a K split takes the rest), and its waves' 16 x 64
// partial tiles are summed through LDS in wave order, so the result is deterministic.
//
// MFMA k order: in step s the lanes of row group G (lanes 16G..16G+15) supply columns
// 32s + 8G .. +7 of the wave's 128, so that one load instruction reads 64 contiguous bytes
// of each of 16 X rows.  A lane's 16 bytes of codes hold columns 32G .. 32G+31 instead;
// a 4 x 4 transpose of 32-bit words across the four row groups (two v_permlane32_swap,
// two v_permlane16_swap) brings the codes into that order before dequantisation.
constexpr int kSkRows = 16;        // weight rows per block
constexpr int kSkKW = 128;         // K columns per wave
constexpr int kSkMaxWaves = 8;     // waves per block at most (K columns per block <= 1024)
constexpr int kSkRedStride = 68;   // LDS row stride of the partial tiles (floats; conflict-free)

// Word s of lane row group G becomes word G of row group s (lane l % 16 kept).
// v_permlane32_swap(A, B) returns (A.lo | B.lo, A.hi | B.hi) over lanes 0-31 | 32-63;
// v_permlane16_swap(A, B) returns (A.r0 | B.r0 | A.r2 | B.r2, A.r1 | B.r1 | A.r3 | B.r3)
// over the 16-lane rows r0..r3.
__device__ __forceinline__ void rows_transpose4(uint32_t (&d)[4]) {
  // the off-diagonal 2 x 2 blocks: rows 0-1 words 2-3 <-> rows 2-3 words 0-1
  const auto a = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
  const uint32_t e0 = a[0], e2 = a[1], e1 = b[0], e3 = b[1];
  // inside each 2 x 2 block: the even rows' odd words <-> the odd rows' even words
  const auto c = __builtin_amdgcn_permlane16_swap(e0, e1, false, false);
  const auto f = __builtin_amdgcn_permlane16_swap(e2, e3, false, false);
  d[0] = c[0];
  d[1] = c[1];
  d[2] = f[0];
  d[3] = f[1];
}

template <int EP, bool PAIR>
__global__ __launch_bounds__(kSkMaxWaves * 64) void q4_skinny_kernel(const GemmArgs a) {
  __shared__ float red[kSkMaxWaves][kSkRows][kSkRedStride];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, nw = (int)blockDim.x >> 6;
  const int nl = lane & 15, G = lane >> 4;
  const int nb = blockIdx.x, z = blockIdx.z;
  const int k0 = (z * nw + w) * kSkKW;

  // the lane's weight row (a block's 16 rows lie in one segment: seg_end % 16 == 0)
  const uint8_t* wb;
  const uint16_t* sb;
  int grow;
  if (PAIR) {
    const bool up = nl >= 8;
    grow = nb * 8 + (nl & 7);
    wb = up ? a.w[1] : a.w[0];
    sb = up ? a.s[1] : a.s[0];
  } else {
    const int r0 = nb * kSkRows;
    if (r0 < a.seg_end[0]) {
      grow = r0 + nl; wb = a.w[0]; sb = a.s[0];
    } else if (r0 < a.seg_end[1]) {
      grow = r0 + nl - a.seg_end[0]; wb = a.w[1]; sb = a.s[1];
    } else {
      grow = r0 + nl - a.seg_end[1]; wb = a.w[2]; sb = a.s[2];
    }
  }
  // codes: columns k0 + 32G .. +31 of the row (read once: non-temporal); the scale codes
  // of the two 64-column groups k0 / 64, k0 / 64 + 1 (one aligned 32-bit word)
  const u32x4 wc = __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(wb + (size_t)grow * (a.K / 2) + k0 / 2 + 16 * G));
  const uint32_t sc2 = *reinterpret_cast<const uint32_t*>(sb + (size_t)grow * (a.K / 64) + k0 / 64);
  // X: rows m = 16 ct + l % 16 (rows past M read row M - 1; their columns are not
  // stored), columns k0 + 32 s + 8 G .. +7.  Row-major X gives each load instruction 16
  // pieces of 64 bytes; the tiled layout makes it 1 KB of contiguous memory (a 3072 x 1024
  // pair GEMM at M = 64: 11.1 -> ~7 us)
  u32x4 xf[4][4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    const int m = min(16 * ct + nl, a.M - 1);
    if (a.x_tiled) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
        xf[ct][s] = *reinterpret_cast<const u32x4*>(a.x + xt_index(m, k0 + 32 * s) + 8 * G);
    } else {
      const uint16_t* xr = a.x + (size_t)m * a.K + k0 + 8 * G;
#pragma unroll
      for (int s = 0; s < 4; ++s) xf[ct][s] = *reinterpret_cast<const u32x4*>(xr + 32 * s);
    }
  }
  // every load above goes out before the first use (left alone, the scheduler sinks most
  // of the X loads between the MFMAs, one memory round trip per step)
  __builtin_amdgcn_sched_barrier(0);

  uint32_t d[4] = {wc[0], wc[1], wc[2], wc[3]};
  rows_transpose4(d);
  const _Float16 slo = (_Float16)((float)(sc2 & 0xFFFFu) * (1.0f / 16384.0f));
  const _Float16 shi = (_Float16)((float)(sc2 >> 16) * (1.0f / 16384.0f));
  f32x4 acc[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const _Float16 sc = s < 2 ? slo : shi;
    const h8 af = __builtin_bit_cast(h8, dequant8(d[s], make_h2(sc, sc)));
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
      acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(h8, xf[ct][s]), acc[ct], 0, 0, 0);
  }
  // lane holds rows 4G + r (weight rows) of column 16 ct + l % 16 (activation rows)
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[w][4 * G + r][16 * ct + nl] = acc[ct][r];
  __syncthreads();

  if constexpr (PAIR) {
    // SwiGLU of gate row i (tile row i) and up row i (tile row 8 + i)
    for (int o = t; o < 8 * 64; o += (int)blockDim.x) {
      const int i = o & 7, mm = o >> 3;
      if (mm >= a.M) continue;
      float g = red[0][i][mm], u = red[0][8 + i][mm];
      for (int v = 1; v < nw; ++v) {
        g += red[v][i][mm];
        u += red[v][8 + i][mm];
      }
      const size_t yo = a.y_tiled ? xt_index(mm, nb * 8 + i) : (size_t)mm * a.ldy + nb * 8 + i;
      static_cast<_Float16*>(a.y)[yo] = (_Float16)((g / (1.0f + expf(-g))) * u);
    }
  } else {
    const bool split = gridDim.z > 1;
    for (int o = t; o < kSkRows * 64; o += (int)blockDim.x) {
      const int row = o & 15, mm = o >> 4;
      if (mm >= a.M) continue;
      float v = red[0][row][mm];
      for (int q = 1; q < nw; ++q) v += red[q][row][mm];
      const int n = nb * kSkRows + row;
      if (split) {
        a.part[((size_t)z * a.M + mm) * a.N + n] = v;  // raw split tile [z][m][n]
        continue;
      }
      const size_t oo = (size_t)mm * a.ldy + n;
      if constexpr (EP == EP_F16)
        static_cast<_Float16*>(a.y)[oo] = (_Float16)v;
      else if constexpr (EP == EP_RESID)
        static_cast<float*>(a.y)[oo] = a.resid[oo] + v;
      else
        static_cast<float*>(a.y)[oo] = v;
    }
  }
}

// Sum of the split-K tiles in split order, then the epilogue; one thread per
// four consecutive outputs of the [M, N] result (N % 4 == 0).
template <int EP, bool PAIR>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const GemmArgs a, int ksplit) {
  const int q = blockIdx.x * 256 + threadIdx.x;
  const int per_row = a.N / 4;
  if (q >= a.M * per_row) return;
  const int m = q / per_row, n = (q % per_row) * 4;
  const int wp = PAIR ? 2 * a.N : a.N;
  f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f}, u = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int z = 0; z < ksplit; ++z) {
    const float* row = a.part + ((size_t)z * a.M + m) * wp;
    v += *reinterpret_cast<const f32x4*>(row + n);
    if constexpr (PAIR) u += *reinterpret_cast<const f32x4*>(row + a.N + n);
  }
  const size_t o = (size_t)m * a.ldy + n;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (EP == EP_SWIGLU) {
      const float g = v[e];
      static_cast<_Float16*>(a.y)[o + e] = (_Float16)((g / (1.0f + expf(-g))) * u[e]);
    } else if constexpr (EP == EP_F16) {
      static_cast<_Float16*>(a.y)[o + e] = (_Float16)v[e];
    } else if constexpr (EP == EP_RESID) {
      static_cast<float*>(a.y)[o + e] = a.resid[o + e] + v[e];
    } else {
      static_cast<float*>(a.y)[o + e] = v[e];
    }
  }
}

// Split-K sum + residual fused with the next RMSNorm: one 256-thread block per row, up to
// four f32x4 of the row per thread.
__global__ __launch_bounds__(256) void splitk_resid_norm_kernel(const GemmArgs a, int ksplit, const float* gamma,
                                                                float eps, _Float16* xn) {
  __shared__ float sred[4];
  const int m = blockIdx.x, t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int nv = a.N / 4;  // f32x4 of the row
  f32x4 y[4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = 4 * (t + 256 * i);
    y[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (t + 256 * i < nv) {
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int z = 0; z < ksplit; ++z) v += *reinterpret_cast<const f32x4*>(a.part + ((size_t)z * a.M + m) * a.N + n);
      const size_t o = (size_t)m * a.ldy + n;
#pragma unroll
      for (int e = 0; e < 4; ++e) y[i][e] = a.resid[o + e] + v[e];
      *reinterpret_cast<f32x4*>(static_cast<float*>(a.y) + o) = y[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) ss = fmaf(y[i][e], y[i][e], ss);
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) sred[wid] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf(((sred[0] + sred[1]) + (sred[2] + sred[3])) / (float)a.N + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = 4 * (t + 256 * i);
    if (t + 256 * i < nv) {
      h2 lo = make_h2((_Float16)((y[i][0] * inv) * gamma[n]), (_Float16)((y[i][1] * inv) * gamma[n + 1]));
      h2 hi = make_h2((_Float16)((y[i][2] * inv) * gamma[n + 2]), (_Float16)((y[i][3] * inv) * gamma[n + 3]));
      const size_t xo = a.y_tiled ? xt_index(m, n) : (size_t)m * a.N + n;  // 4 columns of one chunk
      *reinterpret_cast<u32x2*>(xn + xo) = u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
    }
  }
}

int launch_splitk_resid_norm(const GemmArgs& a, int ksplit, const float* gamma, float eps, uint16_t* xn,
                             hipStream_t st) {
  if (!a.part || !a.resid || !a.y || !gamma || !xn) return Q4D_ERR_NULL;
  if (a.N % 4 || a.N > 4096 || a.M <= 0 || ksplit < 1 || (size_t)ksplit * a.M * a.N > a.part_cap) return Q4D_ERR_SHAPE;
  if (a.y_tiled && (a.M > kXtRows || a.N % 32)) return Q4D_ERR_SHAPE;
  if (a.ldy % 4 || !aligned(a.y, 16) || !aligned(a.resid, 16) || !aligned(xn, 8) || !aligned(a.part, 16))
    return Q4D_ERR_BAD_ADDR;
  hipLaunchKernelGGL(splitk_resid_norm_kernel, dim3(a.M), dim3(256), 0, st, a, ksplit, gamma, eps,
                     reinterpret_cast<_Float16*>(xn));
  return check_launch();
}

// Row-wise reduction of the argmax partials: one wave per activation row.
__global__ __launch_bounds__(64) void argmax_rows_kernel(const float* part_score, const int* part_idx, int nparts,
                                                         int M, int32_t* out_token, float* out_score) {
  const int m = blockIdx.x, lane = threadIdx.x;
  if (m >= M) return;
  float bs = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = lane; i < nparts; i += 64) {
    const float s = part_score[(size_t)m * nparts + i];
    const int ix = part_idx[(size_t)m * nparts + i];
    if (arg_better(s, ix, bs, bi)) {
      bs = s;
      bi = ix;
    }
  }
#pragma unroll
  for (int msk = 32; msk >= 1; msk >>= 1) {
    const float os = shfl_xor_f(bs, msk);
    const int oi = __shfl_xor(bi, msk, kWave);
    if (arg_better(os, oi, bs, bi)) {
      bs = os;
      bi = oi;
    }
  }
  if (lane == 0) {
    out_token[m] = bi;
    out_score[m] = bs;
  }
}

// Splits of K for a grid of `tiles` output tiles: enough to reach ~256
// blocks, each split keeping at least two K steps, within the partial buffer.
static int choose_ksplit(const GemmArgs& a, int tiles, bool pair) {
  if (a.ksplit > 0) return a.ksplit;
  if (!a.part || tiles >= 128) return 1;
  const int nk = a.K / kGemmBK;
  int ks = (256 + tiles - 1) / tiles;
  if (ks > nk / 2) ks = nk / 2;
  if (ks > kGemmMaxSplit) ks = kGemmMaxSplit;
  const size_t per_split = (size_t)a.M * (pair ? 2 * a.N : a.N);
  while (ks > 1 && (size_t)ks * per_split > a.part_cap) --ks;
  return ks < 1 ? 1 : ks;
}

template <int BM, int EP, bool PAIR>
static int launch_gemm_inst(const GemmArgs& a, hipStream_t st) {
  const int nblk = PAIR ? a.N / 64 : a.N / kGemmBN;
  const int mblk = (a.M + BM - 1) / BM;
  const int ks = EP == EP_ARGMAX ? 1 : choose_ksplit(a, nblk * mblk, PAIR);
  if (ks > 1 && (!a.part || (size_t)ks * a.M * (PAIR ? 2 * a.N : a.N) > a.part_cap || a.N % 4 ||
                 ks > a.K / kGemmBK))
    return Q4D_ERR_CAPACITY;
  constexpr int NW = BM == 128 ? kGemmWaves128 : kGemmWaves64;
  if (a.ksplit_used) *a.ksplit_used = ks;
  hipLaunchKernelGGL((q4_gemm_kernel<BM, EP, PAIR, NW>), dim3(nblk, mblk, ks), dim3(NW * 64), 0, st, a);
  int rc = check_launch();
  if (rc || ks == 1 || a.defer_reduce) return rc;
  if constexpr (EP != EP_ARGMAX && EP != EP_ROPE) {
    const int n4 = a.M * (a.N / 4);
    hipLaunchKernelGGL((splitk_reduce_kernel<EP, PAIR>), dim3((n4 + 255) / 256), dim3(256), 0, st, a, ks);
  }
  return check_launch();
}

int device_cus() {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                hipSuccess || cus < 1)
      return 256;
    cached = cus;
  }
  return cached;
}

// K steps per split for the pipelined kernel (it unrolls them fully), or 0 where
// the old kernel runs.  The pipelined kernel holds one block per CU, so it is
// used where its grid fits the device in one round (prefill's N = 1024
// projections with a 2-way K split: 256 blocks; o_proj 20.3 against 26.4 µs);
// grids of several rounds (q|k|v, gate/up) run faster as two blocks per CU of
// q4_gemm_kernel<128> (33.9 / 48.4 against 28.1 / 44.0 µs).
static int pipe_steps(const GemmArgs& a, bool pair) {
  const int nblk = pair ? a.N / 64 : a.N / kGemmBN;
  const int tiles = nblk * ((a.M + 127) / 128);
  const int ks = choose_ksplit(a, tiles, pair);
  const int nk_all = a.K / kGemmBK;
  if (a.K / 64 > kPipeMaxGroups || nk_all % ks || (size_t)tiles * ks > (size_t)device_cus()) return 0;
  const int nk = nk_all / ks;
  return (nk == 16 || nk == 24 || nk == 32 || nk == 48) ? nk : 0;
}

template <int EP, bool PAIR>
static int launch_gemm_pipe(const GemmArgs& a, hipStream_t st) {
  const int nblk = PAIR ? a.N / 64 : a.N / kGemmBN;
  const int mblk = (a.M + 127) / 128;
  const int ks = choose_ksplit(a, nblk * mblk, PAIR);
  if (ks > 1 && (!a.part || (size_t)ks * a.M * (PAIR ? 2 * a.N : a.N) > a.part_cap || a.N % 4 ||
                 ks > a.K / kGemmBK))
    return Q4D_ERR_CAPACITY;
  const dim3 grid(nblk, mblk, ks);
  if (a.ksplit_used) *a.ksplit_used = ks;
  switch (a.K / kGemmBK / ks) {
    case 16: hipLaunchKernelGGL((q4_gemm_pipe_kernel<EP, PAIR, 16>), grid, dim3(512), 0, st, a); break;
    case 24: hipLaunchKernelGGL((q4_gemm_pipe_kernel<EP, PAIR, 24>), grid, dim3(512), 0, st, a); break;
    case 32: hipLaunchKernelGGL((q4_gemm_pipe_kernel<EP, PAIR, 32>), grid, dim3(512), 0, st, a); break;
    case 48: hipLaunchKernelGGL((q4_gemm_pipe_kernel<EP, PAIR, 48>), grid, dim3(512), 0, st, a); break;
    default: return Q4D_ERR_SHAPE;
  }
  int rc = check_launch();
  if (rc || ks == 1 || a.defer_reduce) return rc;
  if constexpr (EP != EP_ROPE) {
    const int n4 = a.M * (a.N / 4);
    hipLaunchKernelGGL((splitk_reduce_kernel<EP, PAIR>), dim3((n4 + 255) / 256), dim3(256), 0, st, a, ks);
  }
  return check_launch();
}

// Split of the skinny kernel (K columns per block = 128 x waves), or 0 where it does not
// apply: asked for (GemmArgs::skinny), at most 64 activation rows, no split asked for,
// K % 128 == 0, 16-row tiles
// (a gate/up pair: 8 + 8 rows) and at most 8 waves per block without a split.  With a
// partial buffer the split grows (over divisors of K / 128, at least 2 waves per block)
// until the grid has 256 blocks.
static int skinny_split(const GemmArgs& a, int ep, bool pair) {
  if (!a.skinny || a.M > 64 || a.ksplit != 0 || a.K % kSkKW) return 0;
  if (pair ? ep != EP_SWIGLU : (ep != EP_F32 && ep != EP_F16 && ep != EP_RESID)) return 0;
  if (pair ? a.N % 8 : (a.N % kSkRows || a.seg_end[0] % kSkRows || a.seg_end[1] % kSkRows)) return 0;
  const int nk = a.K / kSkKW, tiles = pair ? a.N / 8 : a.N / kSkRows;
  int ks = 1;
  while (ks <= nk && (nk % ks || nk / ks > kSkMaxWaves)) ++ks;
  if (ks > nk) return 0;
  const bool can_split = !pair && a.part && a.N % 4 == 0;
  if (ks > 1 && !can_split) return 0;
  if (can_split) {
    for (int k2 = ks + 1; tiles * ks < 256 && k2 <= kGemmMaxSplit && nk / k2 >= 2; ++k2)
      if (nk % k2 == 0) ks = k2;
  }
  if (ks > 1 && (size_t)ks * a.M * a.N > a.part_cap) return 0;
  return ks;
}

template <int EP, bool PAIR>
static int launch_skinny(const GemmArgs& a, int ks, hipStream_t st) {
  const int tiles = PAIR ? a.N / 8 : a.N / kSkRows, nw = a.K / kSkKW / ks;
  if (a.ksplit_used) *a.ksplit_used = ks;
  hipLaunchKernelGGL((q4_skinny_kernel<EP, PAIR>), dim3(tiles, 1, ks), dim3(64 * nw), 0, st, a);
  int rc = check_launch();
  if (rc || ks == 1 || a.defer_reduce) return rc;
  const int n4 = a.M * (a.N / 4);
  hipLaunchKernelGGL((splitk_reduce_kernel<EP, PAIR>), dim3((n4 + 255) / 256), dim3(256), 0, st, a, ks);
  return check_launch();
}

template <int BM>
static int launch_gemm_bm(const GemmArgs& a, int ep, bool pair, hipStream_t st) {
  if (pair) return ep == EP_SWIGLU ? launch_gemm_inst<BM, EP_SWIGLU, true>(a, st) : Q4D_ERR_SHAPE;
  switch (ep) {
    case EP_F32: return launch_gemm_inst<BM, EP_F32, false>(a, st);
    case EP_F16: return launch_gemm_inst<BM, EP_F16, false>(a, st);
    case EP_RESID: return launch_gemm_inst<BM, EP_RESID, false>(a, st);
    case EP_ARGMAX: return launch_gemm_inst<BM, EP_ARGMAX, false>(a, st);
    case EP_ROPE: return launch_gemm_inst<BM, EP_ROPE, false>(a, st);
    default: return Q4D_ERR_SHAPE;
  }
}

int launch_gemm(const GemmArgs& a, int ep, bool pair, hipStream_t st) {
  if (a.M <= 0 || a.K <= 0 || a.K % kGemmBK || a.N <= 0) return Q4D_ERR_SHAPE;
  if (a.nseg < 1 || a.nseg > 3) return Q4D_ERR_SHAPE;
  if (pair) {
    if (a.nseg != 2 || a.N % 64) return Q4D_ERR_SHAPE;
  } else {
    if (a.N % kGemmBN || a.seg_end[a.nseg - 1] != a.N) return Q4D_ERR_SHAPE;
    for (int i = 0; i < a.nseg; ++i)
      if (a.seg_end[i] % kGemmBN) return Q4D_ERR_SHAPE;
  }
  for (int i = 0; i < a.nseg; ++i) {
    if (!a.w[i] || !a.s[i]) return Q4D_ERR_NULL;
    if (!aligned(a.w[i], 16) || !aligned(a.s[i], 2)) return Q4D_ERR_BAD_ADDR;
  }
  if (!a.x || !aligned(a.x, 16)) return a.x ? Q4D_ERR_BAD_ADDR : Q4D_ERR_NULL;
  if (ep == EP_ARGMAX) {
    if (!a.part_score || !a.part_idx) return Q4D_ERR_NULL;
  } else if (ep == EP_ROPE) {
    const PrefillArgs& R = a.rope;
    if (pair || a.part || a.ksplit > 1) return Q4D_ERR_SHAPE;  // the epilogue needs whole tiles
    if (R.qh <= 0 || R.kvh <= 0 || a.N != (R.qh + 2 * R.kvh) * kGemmBN || R.n != a.M) return Q4D_ERR_SHAPE;
    if (!R.q_gamma || !R.k_gamma || !R.rope_cos || !R.rope_sin || !R.kcache || !R.vcache || !R.q16)
      return Q4D_ERR_NULL;
  } else if (!a.y) {
    return Q4D_ERR_NULL;
  }
  if (ep == EP_RESID && !a.resid) return Q4D_ERR_NULL;
  // large M (prefill): the pipelined kernel, 128-row tiles
  if (a.M > 64 && ep != EP_ARGMAX && pipe_steps(a, pair)) {
    if (pair) return ep == EP_SWIGLU ? launch_gemm_pipe<EP_SWIGLU, true>(a, st) : Q4D_ERR_SHAPE;
    switch (ep) {
      case EP_F32: return launch_gemm_pipe<EP_F32, false>(a, st);
      case EP_F16: return launch_gemm_pipe<EP_F16, false>(a, st);
      case EP_RESID: return launch_gemm_pipe<EP_RESID, false>(a, st);
      case EP_ROPE: return launch_gemm_pipe<EP_ROPE, false>(a, st);
      default: return Q4D_ERR_SHAPE;
    }
  }
  // at most 64 activation rows (batched decode): the skinny kernel where it applies (the
  // only kernel that reads or writes the tiled layout)
  const int sks = skinny_split(a, ep, pair);
  if ((a.x_tiled || a.y_tiled) && (!sks || a.M > kXtRows || a.K % 32 || (a.y_tiled && a.N % 32)))
    return Q4D_ERR_SHAPE;
  if (const int ks = sks) {
    if (pair) return launch_skinny<EP_SWIGLU, true>(a, ks, st);
    switch (ep) {
      case EP_F32: return launch_skinny<EP_F32, false>(a, ks, st);
      case EP_F16: return launch_skinny<EP_F16, false>(a, ks, st);
      default: return launch_skinny<EP_RESID, false>(a, ks, st);
    }
  }
  // small M (batched decode) uses 64-row tiles, and so does a large M whose
  // 128-row tiles would leave CUs idle
  const int nblk = pair ? a.N / 64 : a.N / kGemmBN;
  const bool bm64 = a.M <= 64 || (size_t)nblk * ((a.M + 127) / 128) < 256;
  return bm64 ? launch_gemm_bm<64>(a, ep, pair, st) : launch_gemm_bm<128>(a, ep, pair, st);
}

int launch_argmax_rows(const float* part_score, const int* part_idx, int nparts, int M, int32_t* out_token,
                       float* out_score, hipStream_t st) {
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(M), dim3(64), 0, st, part_score, part_idx, nparts, M, out_token,
                     out_score);
  return check_launch();
}

}  // namespace q4d
