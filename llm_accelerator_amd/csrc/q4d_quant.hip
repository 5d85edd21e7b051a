// Float -> Q4 weight quantizer (gfx950), the reference's conversion rule
// (Qwen3-0.6B-Base/python_each_module/13_export_q4_gemv_vectors.py:101-135, restated
// identically in 26_...:126-145, 28_...:103-121, 30_...:103-121, 33_...:95-113):
//
//   absmax  = max_{j<64} |w[64g + j]|                               (fp32)
//   code    = rint(fp32(absmax / 7) * 2^14)        round-half-even, the fp32 quotient
//   code    = 1 if absmax > 0 and code == 0                         (nonzero rule)
//   s       = code / 2^14,  safe = s if s > 0 else 1                (fp32, exact)
//   q[j]    = clip(rint(fp32(w[j] / safe)), -8, 7)                  (correctly rounded /)
//   packed  = q[2i] & 15 | (q[2i+1] & 15) << 4                      (even column low)
//
// A code above 65535 (absmax above ~28) does not fit Q2.14 and a non-finite weight has
// no code: the reference raises for both; here they are counted per group into
// status[0] / status[1] (the caller zeroes status and checks it) and the code clamps.
//
// Layout of the work: a lane owns E consecutive elements of one group (E = 8 for fp32,
// 16 for bf16: two 16-byte loads), so L = 64 / E lanes share a group and a 64-lane chunk
// covers E groups.  Waves stride over batches of 2 chunks, loading the next batch before
// quantising the current one; the group absmax is an L-lane DPP reduction (bf16
// magnitudes compared two at a time as 16-bit halves).
//
// The per-element quotient: w / safe equals w * 2^14 / code exactly, so t = w * inv with
// inv = 2^14 * rcp(code) (v_rcp_f32, within 1 ulp) is within 10.5 * 3 * 2^-24 < 2^-19 of
// the true quotient Q (|Q| <= 10.5 for any finite group: code >= rint(absmax * 2^14 / 7)
// or the nonzero rule's 1), and numpy's fl(Q) within 2^-20 of Q.  Exact ties are found
// exactly (see quantize_chunk); away from half-integers rint(t) = rint(fl(Q)).  So the
// codes equal numpy's bit for bit with one multiply instead of one division per element
// (no fast-math in this build).
#include <math.h>
#include <string.h>

#include <algorithm>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

namespace {

struct QuantArgs {
  const void* w;
  long long ld;         // row pitch in elements
  int rows, cols, groups_per_row;
  uint32_t groups;      // rows * groups_per_row (< 2^32)
  uint32_t magic;       // g / groups_per_row = (t + ((g - t) >> sh1)) >> sh2, t = umulhi(g, magic)
  int sh1, sh2;
  uint8_t* packed;      // [rows, cols/2]
  uint16_t* scale;      // [rows, cols/64]
  int32_t* status;      // [2]: scale overflow groups, non-finite groups
};

constexpr int kQuantChunks = 2;  // chunks per batch (each: two 16-byte loads per lane)

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }

// Division by the invariant groups_per_row (Granlund & Montgomery, round-up multiplier).
__device__ __forceinline__ uint32_t row_of(const QuantArgs& a, uint32_t g) {
  const uint32_t t = __umulhi(g, a.magic);
  return (t + ((g - t) >> a.sh1)) >> a.sh2;
}

// Maximum over the L lanes of a group (L = 4, 8 or 16, aligned): quad swaps, then the
// mirror within 8 (and 16) lanes, as DPP moves.
template <int L>
__device__ __forceinline__ uint32_t group_max(uint32_t x) {
  static_assert(L == 4 || L == 8 || L == 16, "groups of 4, 8 or 16 lanes");
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  if constexpr (L >= 8)
    x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false));  // row_half_mirror
  if constexpr (L == 16)
    x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xF, 0xF, false));  // row_mirror
  return x;
}

__device__ __forceinline__ void add_status(int32_t* status, int slot, int n) {
  if (__ballot(n != 0) == 0) return;
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) n += __shfl_xor(n, k, kWave);
  if ((threadIdx.x & 63) == 0) atomicAdd(status + slot, n);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// max of the |bf16| magnitudes held in the halves of the words (v_pk_max_u16)
__device__ __forceinline__ uint32_t bf16_absmax_bits(const u32x4 (&w)[2]) {
  u16x2 m = __builtin_bit_cast(u16x2, w[0].x & 0x7FFF7FFFu);
  m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[0].y & 0x7FFF7FFFu));
  m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[0].z & 0x7FFF7FFFu));
  m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[0].w & 0x7FFF7FFFu));
  m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[1].x & 0x7FFF7FFFu));
  m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[1].y & 0x7FFF7FFFu));
  m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[1].z & 0x7FFF7FFFu));
  m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[1].w & 0x7FFF7FFFu));
  return (uint32_t)(m.x > m.y ? m.x : m.y) << 16;
}

template <bool BF16>
struct QuantTile {
  static constexpr int E = BF16 ? 16 : 8;  // elements per lane per chunk: two 16-byte loads
  static constexpr int L = 64 / E;         // lanes per group
  static constexpr int PER_LOAD = E / 2;   // elements per 16-byte load
};

// The raw words of chunk `chunk` for this lane (clamped to the last group past the end)
// and the byte offset of its packed codes (-1 past the end).
template <bool BF16>
__device__ __forceinline__ void load_chunk(const QuantArgs& a, uint32_t chunk, int lane, u32x4 (&raw)[2],
                                           long long& dst_off) {
  using T = QuantTile<BF16>;
  const uint32_t g = chunk * T::E + lane / T::L;
  const int j = T::E * (lane % T::L);
  const uint32_t gl = g < a.groups ? g : a.groups - 1;
  const uint32_t row = row_of(a, gl), grp = gl - row * (uint32_t)a.groups_per_row;
  const long long e = (long long)row * a.ld + grp * 64 + j;
  dst_off = g < a.groups ? (long long)row * (a.cols / 2) + grp * 32 + j / 2 : -1;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if constexpr (BF16)
      raw[h] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.w) + e + h * T::PER_LOAD);
    else
      raw[h] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(a.w) + e + h * T::PER_LOAD);
  }
}

// Codes and scale of one chunk from its raw words; stores them.  Called by every lane.
template <bool BF16>
__device__ __forceinline__ void quantize_chunk(const QuantArgs& a, uint32_t chunk, int lane, const u32x4 (&raw)[2],
                                               long long dst_off, int& ovf_total, int& nf_total) {
  using T = QuantTile<BF16>;
  constexpr int E = T::E, L = T::L;
  const bool active = dst_off >= 0;
  float v[E];
  uint32_t mb;
  if constexpr (BF16) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t wd[4] = {raw[h].x, raw[h].y, raw[h].z, raw[h].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[8 * h + 2 * k] = bf16_lo(wd[k]);
        v[8 * h + 2 * k + 1] = bf16_hi(wd[k]);
      }
    }
    mb = bf16_absmax_bits(raw);
  } else {
    mb = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t wd[4] = {raw[h].x, raw[h].y, raw[h].z, raw[h].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[4 * h + k] = __uint_as_float(wd[k]);
        mb = max(mb, wd[k] & 0x7FFFFFFFu);
      }
    }
  }
  // absmax on the magnitude bits: non-negative IEEE floats order like their bit
  // patterns, and a non-finite value has every exponent bit set
  mb = group_max<L>(mb);
  const bool bad = mb >= 0x7F800000u;
  const float m = bad ? 0.0f : __uint_as_float(mb);
  const float cf = rintf((m / 7.0f) * 16384.0f);
  int code = cf > 65535.0f ? 65535 : (int)cf;
  if (active && lane % L == 0) {
    ovf_total += (cf > 65535.0f) && !bad;
    nf_total += bad;
  }
  if (m > 0.0f && code == 0) code = 1;
  const float safe = code > 0 ? (float)code * (1.0f / 16384.0f) : 1.0f;
  const float inv = code > 0 ? __builtin_amdgcn_rcpf((float)code) * 16384.0f : 1.0f;
  // clamp, then round and convert in one add: x + 1.5 * 2^23 leaves rint(x) in the low
  // mantissa bits (round-half-even, two's complement), so its low nibble is the code
  // Exact ties: w / safe = h (a half-integer) exactly iff w == h * safe, a product that is
  // exact in fp32 (h has at most 5 significant bits, safe 16); then rint(h) is numpy's
  // rint(fl(w / safe)).  A bf16 weight (8 significant bits) that is not a tie has its
  // quotient at least 2^-17 from every half-integer (the numerator of Q - h is a nonzero
  // multiple of 2^min(0, e + 15) over 2 code), farther than t's error: rint(t) is exact.
  // An fp32 weight can fall closer, so fp32 also takes the IEEE division for any non-tie
  // within 2^-16 of a half-integer.
  uint64_t bits = 0;
  bool near = false;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float t = v[i] * inv;
    const float h = floorf(t) + 0.5f;
    const bool tie = v[i] == h * safe;
    if constexpr (!BF16) near |= !tie && fabsf(t - h) < 0x1p-16f;
    const float r = fminf(fmaxf(tie ? h : t, -8.0f), 7.0f) + 12582912.0f;
    bits |= (uint64_t)(__float_as_uint(r) & 0xFu) << (4 * i);
  }
  if (near) {  // an fp32 non-tie within 2^-16 of a half-integer: the IEEE quotient decides
    bits = 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float q = fminf(fmaxf(rintf(v[i] / safe), -8.0f), 7.0f);
      bits |= (uint64_t)((uint32_t)(int)q & 0xFu) << (4 * i);
    }
  }
  if (active) {
    uint8_t* dst = a.packed + dst_off;
    if constexpr (BF16) {
      u32x2 o;
      o.x = (uint32_t)bits;
      o.y = (uint32_t)(bits >> 32);
      *reinterpret_cast<u32x2*>(dst) = o;
    } else {
      *reinterpret_cast<uint32_t*>(dst) = (uint32_t)bits;
    }
    if (lane % L == 0) a.scale[chunk * E + lane / L] = (uint16_t)code;
  }
}

// Grid-stride over batches of kQuantChunks chunks: the loads of the wave's next batch are
// issued before the current batch is quantised, so memory and arithmetic overlap.
template <bool BF16>
__global__ __launch_bounds__(256) void quantize_q4_kernel(const QuantArgs a, uint32_t batches) {
  const int lane = threadIdx.x & 63;
  const uint32_t first = blockIdx.x * 4 + (threadIdx.x >> 6), stride = gridDim.x * 4;
  int ovf_total = 0, nf_total = 0;
  u32x4 cur[kQuantChunks][2], nxt[kQuantChunks][2];
  long long cur_off[kQuantChunks], nxt_off[kQuantChunks];
  if (first < batches) {
#pragma unroll
    for (int c = 0; c < kQuantChunks; ++c) load_chunk<BF16>(a, first * kQuantChunks + c, lane, cur[c], cur_off[c]);
  }
  for (uint32_t b = first; b < batches; b += stride) {
    const uint32_t nb = b + stride;
    if (nb < batches) {
#pragma unroll
      for (int c = 0; c < kQuantChunks; ++c) load_chunk<BF16>(a, nb * kQuantChunks + c, lane, nxt[c], nxt_off[c]);
    }
#pragma unroll
    for (int c = 0; c < kQuantChunks; ++c)
      quantize_chunk<BF16>(a, b * kQuantChunks + c, lane, cur[c], cur_off[c], ovf_total, nf_total);
#pragma unroll
    for (int c = 0; c < kQuantChunks; ++c) {
      cur[c][0] = nxt[c][0];
      cur[c][1] = nxt[c][1];
      cur_off[c] = nxt_off[c];
    }
  }
  add_status(a.status, 0, ovf_total);
  add_status(a.status, 1, nf_total);
}

// Several matrices of one shape per launch: blockIdx.y picks the matrix, whose pointers
// come from the kernel-argument block (read through the kernarg segment pointer, so the
// runtime index does not copy the block to scratch); within a matrix the work is that of
// quantize_q4_kernel, so the codes are the same bit for bit.
constexpr int kQuantBatchMax = 64;

struct QuantBatchArgs {
  QuantArgs g;  // the shared geometry (its w / packed / scale unused)
  const void* w[kQuantBatchMax];
  uint8_t* packed[kQuantBatchMax];
  uint16_t* scale[kQuantBatchMax];
};

template <bool BF16>
__global__ __launch_bounds__(256) void quantize_q4_batch_kernel(const QuantBatchArgs args, uint32_t batches) {
  typedef __attribute__((address_space(4))) const QuantBatchArgs* KernargPtr;
  const KernargPtr P = (KernargPtr)__builtin_amdgcn_kernarg_segment_ptr();
  const int m = blockIdx.y;
  QuantArgs a = args.g;  // fixed offsets: read as kernel arguments
  a.w = P->w[m];
  a.packed = P->packed[m];
  a.scale = P->scale[m];
  const int lane = threadIdx.x & 63;
  const uint32_t first = blockIdx.x * 4 + (threadIdx.x >> 6), stride = gridDim.x * 4;
  int ovf_total = 0, nf_total = 0;
  u32x4 cur[kQuantChunks][2], nxt[kQuantChunks][2];
  long long cur_off[kQuantChunks], nxt_off[kQuantChunks];
  if (first < batches) {
#pragma unroll
    for (int c = 0; c < kQuantChunks; ++c) load_chunk<BF16>(a, first * kQuantChunks + c, lane, cur[c], cur_off[c]);
  }
  for (uint32_t b = first; b < batches; b += stride) {
    const uint32_t nb = b + stride;
    if (nb < batches) {
#pragma unroll
      for (int c = 0; c < kQuantChunks; ++c) load_chunk<BF16>(a, nb * kQuantChunks + c, lane, nxt[c], nxt_off[c]);
    }
#pragma unroll
    for (int c = 0; c < kQuantChunks; ++c)
      quantize_chunk<BF16>(a, b * kQuantChunks + c, lane, cur[c], cur_off[c], ovf_total, nf_total);
#pragma unroll
    for (int c = 0; c < kQuantChunks; ++c) {
      cur[c][0] = nxt[c][0];
      cur[c][1] = nxt[c][1];
      cur_off[c] = nxt_off[c];
    }
  }
  add_status(a.status, 0, ovf_total);
  add_status(a.status, 1, nf_total);
}

// Checks shared by both entry points; fills the geometry of a (not its pointers).
int quant_geometry(int32_t dtype, int64_t ld, int32_t rows, int32_t cols, QuantArgs& a, long long& batches) {
  if (dtype != Q4D_F32 && dtype != Q4D_BF16) return Q4D_ERR_DTYPE;
  if (rows <= 0 || cols <= 0 || cols % 64 || ld < cols) return Q4D_ERR_SHAPE;
  const size_t esz = dtype == Q4D_F32 ? 4 : 2;
  if ((ld * (int64_t)esz) % 16) return Q4D_ERR_BAD_ADDR;  // 16-byte aligned rows
  memset(&a, 0, sizeof(a));
  a.ld = ld;
  a.rows = rows;
  a.cols = cols;
  a.groups_per_row = cols / 64;
  const unsigned long long groups = (unsigned long long)rows * a.groups_per_row;
  if (groups > 0xFFFFFF00ull) return Q4D_ERR_SHAPE;  // group indices stay 32-bit
  a.groups = (uint32_t)groups;
  {  // round-up multiplier for the invariant divisor groups_per_row
    const unsigned long long d = (unsigned long long)a.groups_per_row;
    int l = 0;
    while ((1ull << l) < d) ++l;  // ceil(log2 d)
    a.magic = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    a.sh1 = l < 1 ? l : 1;
    a.sh2 = l > 1 ? l - 1 : 0;
  }
  const int per_chunk = dtype == Q4D_F32 ? 8 : 16;  // groups per 64-lane chunk
  const long long chunks = ((long long)a.groups + per_chunk - 1) / per_chunk;
  batches = (chunks + kQuantChunks - 1) / kQuantChunks;
  return Q4D_OK;
}

// 16-byte loads; 8-byte (bf16) / 4-byte (fp32) packed stores
bool quant_ptrs_ok(const void* w, int32_t dtype, const uint8_t* packed, const uint16_t* scale) {
  return aligned(w, 16) && aligned(packed, dtype == Q4D_BF16 ? 8 : 4) && aligned(scale, 2);
}

}  // namespace
}  // namespace q4d

using namespace q4d;

extern "C" int q4d_quantize_q4(const void* weight, int32_t dtype, int64_t ld, int32_t rows, int32_t cols,
                               uint8_t* packed, uint16_t* scale, int32_t* status, void* stream) {
  if (!weight || !packed || !scale || !status) return Q4D_ERR_NULL;
  QuantArgs a;
  long long batches = 0;
  int rc = quant_geometry(dtype, ld, rows, cols, a, batches);
  if (rc) return rc;
  if (!quant_ptrs_ok(weight, dtype, packed, scale) || !aligned(status, 4)) return Q4D_ERR_BAD_ADDR;
  a.w = weight;
  a.packed = packed;
  a.scale = scale;
  a.status = status;
  // enough waves to fill every SIMD several times over; each loops over its batches
  const long long blocks = std::min<long long>((batches + 3) / 4, 4096);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == Q4D_F32)
    hipLaunchKernelGGL(quantize_q4_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, st, a, (uint32_t)batches);
  else
    hipLaunchKernelGGL(quantize_q4_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, st, a, (uint32_t)batches);
  return check_launch();
}

extern "C" int q4d_quantize_q4_batch(const void* const* weights, int32_t dtype, int64_t ld, int32_t rows,
                                     int32_t cols, int32_t count, uint8_t* const* packed, uint16_t* const* scales,
                                     int32_t* status, void* stream) {
  if (!weights || !packed || !scales || !status) return Q4D_ERR_NULL;
  if (count <= 0) return Q4D_ERR_SHAPE;
  QuantBatchArgs A;
  long long batches = 0;
  int rc = quant_geometry(dtype, ld, rows, cols, A.g, batches);
  if (rc) return rc;
  if (!aligned(status, 4)) return Q4D_ERR_BAD_ADDR;
  for (int i = 0; i < count; ++i) {
    if (!weights[i] || !packed[i] || !scales[i]) return Q4D_ERR_NULL;
    if (!quant_ptrs_ok(weights[i], dtype, packed[i], scales[i])) return Q4D_ERR_BAD_ADDR;
  }
  A.g.status = status;
  // the grid-stride share of one matrix: up to 4096 blocks spread over the matrices of a launch
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  for (int i0 = 0; i0 < count; i0 += kQuantBatchMax) {
    const int n = std::min(kQuantBatchMax, count - i0);
    for (int k = 0; k < kQuantBatchMax; ++k) {
      const int i = i0 + (k < n ? k : 0);  // unused slots repeat the first matrix, never read
      A.w[k] = weights[i];
      A.packed[k] = packed[i];
      A.scale[k] = scales[i];
    }
    const long long bx = std::max<long long>(1, std::min<long long>((batches + 3) / 4, 4096 / n));
    const dim3 grid((unsigned)bx, (unsigned)n);
    if (dtype == Q4D_F32)
      hipLaunchKernelGGL(quantize_q4_batch_kernel<false>, grid, dim3(256), 0, st, A, (uint32_t)batches);
    else
      hipLaunchKernelGGL(quantize_q4_batch_kernel<true>, grid, dim3(256), 0, st, A, (uint32_t)batches);
    if ((rc = check_launch())) return rc;
  }
  return Q4D_OK;
}
