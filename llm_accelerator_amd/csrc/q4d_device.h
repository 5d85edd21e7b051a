// Device-side building blocks for the Q4 decode kernels (gfx950, wave64).
//
// Q4 weight layout (reference Source/Q4_FORMAT.md:75-140): row-major
// [N, K/2] bytes, two signed two's-complement int4 per byte with the even
// column in the low nibble, so a little-endian u32 holds columns 8m..8m+7
// with column 8m in bits 3:0.  Scales are uint16 Q2.14, one per 64-column
// group, in a separate [N, K/64] array.
//
// Dequantisation trick used by every GEMV here: after v = w ^ 0x88888888
// each nibble holds u = q + 8 in [0, 15].  Masking v with 0x000F000F gives
// two fp16 *denormals* u0 * 2^-24 and u4 * 2^-24 in one register (no
// exponent bits set, so the value is exactly linear in u); masking with
// 0x00F000F0 gives u1 * 2^-20 and u5 * 2^-20.  v_dot2_f32_f16 multiplies
// such a pair by a pair of fp16 activations and accumulates in fp32, with
// exact products.  The int4 sum is then
//     sum q*x = 2^24*A + 2^20*B - 8*sum x
// where A/B are the two accumulators.  Per 8 weights this costs one xor,
// one shift, four ands and four dot2 instructions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q4d {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float dot2(uint32_t pair_bits, h2 x, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pair_bits), x, acc, false);
}

__device__ __forceinline__ h2 make_h2(_Float16 lo, _Float16 hi) {
  h2 r;
  r.x = lo;
  r.y = hi;
  return r;
}

// Activations for one 16-byte weight chunk (32 consecutive columns), laid
// out in the pair order the dequant trick produces: for word m (columns
// 8m..8m+7 of the chunk) p[4m+i] = (x[8m+i], x[8m+i+4]), i = 0..3.
struct XChunk {
  h2 p[16];
  float sum8;  // 8 * sum of the 32 (fp16) activations, accumulated in fp32
};

// Build an XChunk from 32 fp16 activations given as 16 u32 words
// (word t holds columns 2t and 2t+1).
__device__ __forceinline__ void xchunk_from_words(const uint32_t (&xw)[16], XChunk& xc) {
  float s = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    // columns 8m..8m+7 live in words 4m..4m+3
    h2 c01 = __builtin_bit_cast(h2, xw[4 * m + 0]);
    h2 c23 = __builtin_bit_cast(h2, xw[4 * m + 1]);
    h2 c45 = __builtin_bit_cast(h2, xw[4 * m + 2]);
    h2 c67 = __builtin_bit_cast(h2, xw[4 * m + 3]);
    xc.p[4 * m + 0] = make_h2(c01.x, c45.x);
    xc.p[4 * m + 1] = make_h2(c01.y, c45.y);
    xc.p[4 * m + 2] = make_h2(c23.x, c67.x);
    xc.p[4 * m + 3] = make_h2(c23.y, c67.y);
    s += (float)c01.x + (float)c01.y + (float)c23.x + (float)c23.y +
         (float)c45.x + (float)c45.y + (float)c67.x + (float)c67.y;
  }
  xc.sum8 = 8.f * s;
}

// sum_{j<32} q_j * x_j for one 16-byte chunk, exact products, fp32 sums.
__device__ __forceinline__ float chunk_dot(const u32x4 w, const XChunk& xc) {
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t v = w[m] ^ 0x88888888u;
    const uint32_t t = v >> 8;
    a = dot2(v & 0x000F000Fu, xc.p[4 * m + 0], a);
    b = dot2(v & 0x00F000F0u, xc.p[4 * m + 1], b);
    a = dot2(t & 0x000F000Fu, xc.p[4 * m + 2], a);
    b = dot2(t & 0x00F000F0u, xc.p[4 * m + 3], b);
  }
  return fmaf(a, 16777216.f, fmaf(b, 1048576.f, -xc.sum8));
}

// Q2.14 scale code -> float (exact).
__device__ __forceinline__ float scale_q2_14(uint32_t code) {
  return (float)code * (1.0f / 16384.0f);
}

// ---------------------------------------------------------------- reductions
// DPP lane movement (gfx9 DPP: quad_perm, row mirrors, row broadcasts).
// Lanes whose DPP source is disabled by the row mask read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                0xF, false));
}
constexpr int kDppQuadSwap1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowBcast15 = 0x142;   // lane 15 of each row -> next row
constexpr int kDppRowBcast31 = 0x143;   // lane 31 -> rows 2 and 3

// Sum over each 16-lane row; every lane of the row receives the row sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<kDppQuadSwap1>(v);
  v += dpp_f<kDppQuadSwap2>(v);
  v += dpp_f<kDppRowHalfMirror>(v);
  v += dpp_f<kDppRowMirror>(v);
  return v;
}

// Sums of lanes 0-31 and 32-63: valid in lanes 16-31 and 48-63 respectively.
__device__ __forceinline__ float half_wave_sum_dpp(float v) {
  v = row16_sum(v);
  return v + dpp_f<kDppRowBcast15, 0xA>(v);
}

// Sum of all 64 lanes, valid in lanes 48-63.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = half_wave_sum_dpp(v);
  return v + dpp_f<kDppRowBcast31, 0xC>(v);
}

// Sum of all 64 lanes, in every lane.
__device__ __forceinline__ float wave_sum_bcast(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_dpp(v)), 63));
}

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// Sum over the 32 lanes of each wave half (lanes 0-31 and 32-63 separately).
__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) v += shfl_xor_f(v, m);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v += shfl_xor_f(v, 32);
  return half_wave_sum(v);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor_f(v, m));
  return v;
}

// Workgroup barrier for LDS exchange only: waits for this wave's LDS
// operations, not for its outstanding global loads (which __syncthreads()
// would drain), so prefetched weights stay in flight across it.
__device__ __forceinline__ void block_sync_lds() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt/expcnt untouched
  __builtin_amdgcn_s_barrier();
}

// Argmax order: higher score wins; equal scores -> lower index wins
// (reference tie rule: strict greater-than in ascending row order).
__device__ __forceinline__ bool arg_better(float s, int i, float bs, int bi) {
  return s > bs || (s == bs && i < bi);
}

}  // namespace q4d
