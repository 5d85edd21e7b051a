// Integer Q4 GEMV of the reference's fixed-point path (gfx950).
//
//   partial[n, g] = sum_{j < 64} x[64g + j] * q[n, 64g + j]
//   y_q26[n]      = sum_g partial[n, g] * scale[n, g]            (int64, exact)
//   y_q12_12[n]   = sat24(y_q26[n] >> 14)                        (arithmetic shift)
//
// Follows compute_q4_gemv_q26 / q26_to_q12_12
// (Qwen3-0.6B-Base/python_each_module/28_export_mlp_gate_up_vectors.py:124-138,
// saturate_signed_array :93-96) and q4_gemv_from_ints
// (13_export_q4_gemv_vectors.py:138-154): x is Q12.12 (or Q4.12) in 24-bit
// signed range, q the signed int4 codes, scale the Q2.14 codes.
//
// One wave per row; lane l takes columns 16 l .. 16 l + 15 of each 1024-column
// pass.  Exactness: |x| <= 2^23 and |q| <= 8, so a lane's 16-term partial is at
// most 2^30 in magnitude and fits int32; multiplying it by the scale of its
// 64-column group (4 lanes share a group) and summing the lanes in int64 gives
// sum_g scale * partial by distributivity, at most 2^52 for K <= 3072.
//
// argmax_q26_kernel: the streamed scan's result (56_export_persistent_
// multitoken_layer_golden.py:766-798,860): the highest score, and among equal
// scores the lowest row.
#include <limits.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ long long shfl_xor_ll(long long v, int m) {
  const int lo = __shfl_xor((int)(unsigned long long)v, m, kWave);
  const int hi = __shfl_xor((int)((unsigned long long)v >> 32), m, kWave);
  return (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

__global__ __launch_bounds__(256) void gemv_q26_kernel(const uint8_t* __restrict__ w, const uint16_t* __restrict__ s,
                                                       int N, int K, const int32_t* __restrict__ x,
                                                       int64_t* y_q26, int32_t* y_q12, int32_t* saturated) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;  // whole waves
  const uint8_t* wr = w + (size_t)row * (K / 2);
  const uint16_t* sr = s + (size_t)row * (K / 64);
  long long acc = 0;
  for (int c0 = 16 * lane; c0 < K; c0 += 1024) {
    const unsigned long long wv = *reinterpret_cast<const unsigned long long*>(wr + c0 / 2);
    const i32x4* xv = reinterpret_cast<const i32x4*>(x + c0);
    int part = 0;
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const i32x4 xx = xv[v4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * v4 + e;  // column c0 + i: byte i / 2, low nibble for even i
        const int q = ((int)((wv >> (4 * i)) & 0xFu) ^ 8) - 8;
        part += xx[e] * q;
      }
    }
    acc += (long long)part * (long long)sr[c0 / 64];
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc += shfl_xor_ll(acc, m);
  if (lane == 0) {
    if (y_q26) y_q26[row] = acc;
    long long sh = acc >> 14;
    const long long lo = -(1LL << 23), hi = (1LL << 23) - 1;
    const bool sat = sh < lo || sh > hi;
    sh = sh < lo ? lo : (sh > hi ? hi : sh);
    if (y_q12) y_q12[row] = (int32_t)sh;
    if (sat && saturated) atomicAdd(saturated, 1);
  }
}

__device__ __forceinline__ bool better_ll(long long s, int i, long long bs, int bi) {
  return s > bs || (s == bs && i < bi);
}

__global__ __launch_bounds__(1024) void argmax_q26_kernel(const int64_t* __restrict__ sc, int n, int32_t* tok,
                                                          int64_t* score) {
  __shared__ long long s_best[16];
  __shared__ int s_idx[16];
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  long long bs = LLONG_MIN;
  int bi = INT_MAX;
  for (int i = t; i < n; i += 1024) {  // ascending per thread: strict > keeps the first
    const long long v = sc[i];
    if (v > bs || bi == INT_MAX) {
      bs = v;
      bi = i;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const long long os = shfl_xor_ll(bs, m);
    const int oi = __shfl_xor(bi, m, kWave);
    if (better_ll(os, oi, bs, bi)) {
      bs = os;
      bi = oi;
    }
  }
  if (lane == 0) {
    s_best[wid] = bs;
    s_idx[wid] = bi;
  }
  __syncthreads();
  if (t == 0) {
    for (int k = 1; k < 16; ++k)
      if (better_ll(s_best[k], s_idx[k], bs, bi)) {
        bs = s_best[k];
        bi = s_idx[k];
      }
    *tok = bi;
    *score = bs;
  }
}

}  // namespace

int launch_gemv_q26(const q4d_matrix_t* w, const int32_t* x, int64_t* y_q26, int32_t* y_q12, int32_t* saturated,
                    hipStream_t st) {
  hipLaunchKernelGGL(gemv_q26_kernel, dim3((w->rows + 3) / 4), dim3(256), 0, st, w->w, w->s, w->rows, w->cols, x,
                     y_q26, y_q12, saturated);
  return check_launch();
}

int launch_argmax_q26(const int64_t* scores, int n, int32_t* tok, int64_t* score, hipStream_t st) {
  hipLaunchKernelGGL(argmax_q26_kernel, dim3(1), dim3(1024), 0, st, scores, n, tok, score);
  return check_launch();
}

}  // namespace q4d
