// Causal GQA attention of a prefill on MFMA (gfx950).
//
// The reference's prefill is serial: run_manual_one_token once per prompt
// token (10_validate_full_run_one_token.py:81-135), each call appending one
// K/V row and attending over the cache (common.py:231-298).  Here the n new
// tokens at positions p0 .. p0 + n - 1 go through each layer together; the
// projections are Q4 GEMMs (q4d_gemm.hip), whose q|k|v epilogue also applies
// the per-head q/k RMSNorm and RoPE, appends K/V to the cache and leaves q as
// fp16 [q_head][token][128] with the softmax scale and log2(e) folded in.
//
// prefill_attn_kernel: flash attention forward, causal, one block per
// (64-query tile, q head), 4 waves of 16 queries.  Per 64-key tile:
//   S^T = K . Q^T (16x16x32 f16 MFMA; K rows straight from the cache tile
//   in LDS, Q^T from registers); online softmax per query (exp2);
//   O^T += V^T . P^T, where the S^T accumulator layout is already the B
//   operand layout of P^T (each lane holds 4 keys of two 16-key tiles for one
//   query), so P never leaves registers.  V is transposed into LDS as it is
//   staged: each thread loads a 4-key x 8-dim block, transposes it in
//   registers and writes 8-byte rows of V^T.
// Row strides of the LDS tiles: 136 and 68 fp16 (measured best of the 16-byte /
// 8-byte aligned choices; SQ_LDS_BANK_CONFLICT fell with the row-contiguous K stores).
#include <math.h>
#include <string.h>

#include "q4d_device.h"
#include "q4d_internal.h"

namespace q4d {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kBQ = 64;   // queries per block
constexpr int kBK = 64;   // keys per tile
constexpr int kLdk = kD + 8;   // fp16 row stride of the K tile
constexpr int kLdv = kBK + 4;  // fp16 row stride of the V^T tile (+4 beat +8, +12 and +16 when measured)
constexpr float kRescale = 8.0f;  // log2 headroom of the lazily moved running max

// Global loads of one K/V tile.  K: thread (kr = t >> 4, kc = t & 15) holds dims
// 8kc .. 8kc+7 of keys kr + 16b, so 16 lanes store one whole 256-byte K row and the
// LDS stores meet every bank once.  V: thread (kq = t & 15, dc = t >> 4) holds keys
// 4kq .. 4kq+3, dims 8dc .. 8dc+7, the 4 x 8 block it transposes into V^T.
struct KVRegs {
  u32x4 k[4], v[4];
};

__device__ __forceinline__ void load_kv(const uint16_t* kb, const uint16_t* vb, int key0, int kend, int t,
                                        KVRegs& R) {
  const int kq = t & 15, dc = t >> 4;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    int kk = key0 + dc + 16 * b;        // K row of piece b (dc doubles as the row index kr)
    kk = kk < kend ? kk : kend - 1;     // rows past the end are masked out of the softmax
    R.k[b] = *reinterpret_cast<const u32x4*>(kb + (size_t)kk * kD + kq * 8);
    int key = key0 + 4 * kq + b;
    key = key < kend ? key : kend - 1;
    R.v[b] = *reinterpret_cast<const u32x4*>(vb + (size_t)key * kD + dc * 8);
  }
}

__device__ __forceinline__ void store_kv(const KVRegs& R, int t, _Float16 (*Ks)[kLdk], _Float16 (*Vt)[kLdv]) {
  const int kq = t & 15, dc = t >> 4;
#pragma unroll
  for (int b = 0; b < 4; ++b) *reinterpret_cast<u32x4*>(&Ks[dc + 16 * b][kq * 8]) = R.k[b];
  // transpose the 4-key x 8-dim block: dim e of keys 4kq..4kq+3 -> one 8-byte row piece
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int wrd = e >> 1, hi = e & 1;
    const uint32_t sel = hi ? 0x07060302u : 0x05040100u;  // high or low halves of (src0, src1)
    const uint32_t k01 = __builtin_amdgcn_perm(R.v[1][wrd], R.v[0][wrd], sel);
    const uint32_t k23 = __builtin_amdgcn_perm(R.v[3][wrd], R.v[2][wrd], sel);
    *reinterpret_cast<u32x2*>(&Vt[dc * 8 + e][4 * kq]) = u32x2{k01, k23};
  }
}

// Max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (one query's 4 quarters), the
// same value in each of them, by cross-row lane swaps (VALU, no LDS traffic):
// v_permlane32_swap(x, x) returns (x of lanes 0-31 in both halves, x of lanes 32-63 in
// both halves), v_permlane16_swap the same for rows 0, 2 and rows 1, 3 of 16 lanes.  The
// result elements are copied to scalars before the bit casts (a bit cast of an
// ext-vector element expression reads element 0 with this compiler).
template <bool SUM>
__device__ __forceinline__ float quarters_reduce(float v) {
  const uint32_t a = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(a, a, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  const float x0 = __builtin_bit_cast(float, r0), x1 = __builtin_bit_cast(float, r1);
  const float u = SUM ? x0 + x1 : fmaxf(x0, x1);
  const uint32_t b = __builtin_bit_cast(uint32_t, u);
  const auto q = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  const uint32_t q0 = q[0], q1 = q[1];
  const float y0 = __builtin_bit_cast(float, q0), y1 = __builtin_bit_cast(float, q1);
  return SUM ? y0 + y1 : fmaxf(y0, y1);
}

// Register budget of two waves per SIMD: the grid gives each CU two blocks of four waves,
// and with the default budget (three) the compiler issues the LDS operand reads later,
// which measured ~20 % slower.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void prefill_attn_kernel(
    const PrefillArgs a) {
  __shared__ _Float16 Ks[kBK][kLdk];
  __shared__ _Float16 Vt[kD][kLdv];

  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  // Block order.  Linear block b runs on XCD b % 8 (each XCD has its own L2), and an
  // XCD's blocks go round robin over its 32 CUs, so its blocks i and i + 32 share a
  // CU.  With 16 heads each XCD takes two consecutive q heads (one kv head: its
  // K/V stay in that L2), the first heaviest query tile first and the second
  // lightest first, so every CU gets a complementary pair of causal loads.
  // Other head counts: linear order, heaviest query tile first.
  const int gx = gridDim.x, gy = gridDim.y;
  const int lin = (int)blockIdx.x + gx * (int)blockIdx.y;
  int qt, h;
  if (gy % 16 == 0) {
    const int per = gx * gy / 8, i = lin >> 3, u = i % gx;
    h = (gy / 8) * (lin & 7) + i / gx;
    qt = i >= per / 2 ? u : gx - 1 - u;
  } else {
    h = blockIdx.y;
    qt = gx - 1 - (int)blockIdx.x;
  }
  const int j = h / (a.qh / a.kvh);
  const int i0 = qt * kBQ;                 // first query (token index) of the block
  const int q_lo = i0 + 16 * w;            // first query of this wave
  const int kend = a.p0 + min(a.n, i0 + kBQ);  // keys [0, kend) can be attended by the block
  const int ntiles = (kend + kBK - 1) / kBK;
  const uint16_t* kb = a.kcache + (size_t)j * a.max_ctx * kD;
  const uint16_t* vb = a.vcache + (size_t)j * a.max_ctx * kD;

  // Q^T operand: lane (n = query q_lo + (l & 15), quarter l >> 4) holds dims 32s + 8q .. +7
  const int qn = lane & 15, qq = lane >> 4;
  const int my_q = q_lo + qn;            // token index of this lane's query column
  const int my_pos = a.p0 + my_q;        // its position
  h8 qop[4];
  {
    const int qrow = my_q < a.n ? my_q : a.n - 1;
    const _Float16* qp = a.q16 + ((size_t)h * a.n + qrow) * kD;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[s] = *reinterpret_cast<const h8*>(qp + 32 * s + 8 * qq);
  }

  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;  // per query column (replicated over the 4 quarters)

  KVRegs R;
  load_kv(kb, vb, 0, kend, t, R);
  for (int kt = 0; kt < ntiles; ++kt) {
    __syncthreads();  // the previous tile's LDS reads are done
    store_kv(R, t, Ks, Vt);
    __syncthreads();
    if (kt + 1 < ntiles) load_kv(kb, vb, (kt + 1) * kBK, kend, t, R);

    // S^T tile: 64 keys x 16 queries, 4 D tiles of 16 keys
    f32x4 st[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      st[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const h8 kop = *reinterpret_cast<const h8*>(&Ks[16 * mt + qn][32 * s + 8 * qq]);
        st[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[s], st[mt], 0, 0, 0);
      }
    }
    // causal / range mask: lane holds keys kt*64 + 16mt + 4qq + i for query my_pos.  Only
    // a tile that reaches past the wave's first query or past kend needs it.
    const int kbase = kt * kBK + 4 * qq;
    if (kt * kBK + kBK - 1 > a.p0 + q_lo || kt * kBK + kBK > kend) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kbase + 16 * mt + i;
          if (key > my_pos || key >= kend) st[mt][i] = -INFINITY;
        }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) tmax = fmaxf(tmax, fmaxf(fmaxf(st[mt][0], st[mt][1]), fmaxf(st[mt][2], st[mt][3])));
    tmax = quarters_reduce<false>(tmax);
    // Lazy rescaling: the running max moves only when a score exceeds it by more than
    // kRescale (log2 units), so P = 2^(s - m_run) stays below 2^kRescale (far inside fp16's
    // range) and the O / l rescale is skipped for the wave unless some query needs it.
    // The first tile always moves it (m_run = -inf; key 0 is visible to every query).
    const bool move = tmax > m_run + kRescale;
    if (__builtin_amdgcn_ballot_w64(move)) {
      const float m_new = move ? tmax : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
    }
    float psum = 0.f;
    h4 p[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(st[mt][i] - m_run);
        psum += e;
        p[mt][i] = (_Float16)e;
      }
    l_run += psum;
    // O^T += V^T . P^T over two 32-key steps
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const h8 pop = __builtin_shufflevector(p[2 * s2], p[2 * s2 + 1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const h4 va = *reinterpret_cast<const h4*>(&Vt[16 * dt + qn][32 * s2 + 4 * qq]);
        const h4 vb2 = *reinterpret_cast<const h4*>(&Vt[16 * dt + qn][32 * s2 + 16 + 4 * qq]);
        const h8 vop = __builtin_shufflevector(va, vb2, 0, 1, 2, 3, 4, 5, 6, 7);
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop, o[dt], 0, 0, 0);
      }
    }
  }

  // ---- normalise and store: lane holds O^T[d = 16dt + 4qq + i][query my_q] ---------
  float l_tot = l_run;
  l_tot = quarters_reduce<true>(l_tot);
  if (my_q < a.n) {
    const float inv = 1.0f / l_tot;
    _Float16* out = a.out + (size_t)my_q * a.qh * kD + (size_t)h * kD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      h4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (_Float16)(o[dt][i] * inv);
      *reinterpret_cast<h4*>(out + 16 * dt + 4 * qq) = v;
    }
  }
}

}  // namespace

int launch_prefill_attention(const PrefillArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(prefill_attn_kernel, dim3((a.n + kBQ - 1) / kBQ, a.qh), dim3(256), 0, st, a);
  return check_launch();
}

// ---- the causal-attention primitive (manual_causal_attention, common.py:201-216) -----
// The fp32 operands are rounded to the fp16 layouts prefill_attn_kernel reads (q with
// the softmax scale and log2(e) folded in, as the prefill's q|k|v epilogue leaves it;
// k / v as a cache plane of max_ctx = seq positions), and its fp16 output
// [seq][qh][128] is widened back to fp32 [qh][seq][128].
namespace {

__global__ __launch_bounds__(256) void to_f16_kernel(const float* x, _Float16* y, long long n4, float mul) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (long long)gridDim.x * blockDim.x) {
    const f32x4 v = reinterpret_cast<const f32x4*>(x)[i];
    h4 h;
    h[0] = (_Float16)(v[0] * mul);
    h[1] = (_Float16)(v[1] * mul);
    h[2] = (_Float16)(v[2] * mul);
    h[3] = (_Float16)(v[3] * mul);
    reinterpret_cast<h4*>(y)[i] = h;
  }
}

// out[h][s][d] = o16[s][h][d] for one sequence
__global__ __launch_bounds__(256) void attn_out_kernel(const _Float16* o16, float* out, int seq, int qh) {
  const long long n4 = (long long)qh * seq * (kD / 4);
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (long long)gridDim.x * blockDim.x) {
    const int d4 = (int)(i % (kD / 4));
    const long long hs = i / (kD / 4);
    const int sp = (int)(hs % seq), h = (int)(hs / seq);
    const h4 v = *reinterpret_cast<const h4*>(o16 + ((size_t)sp * qh + h) * kD + 4 * d4);
    reinterpret_cast<f32x4*>(out)[i] = f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  }
}

inline unsigned grid_for(long long n4) {
  const long long b = (n4 + 255) / 256;
  return (unsigned)(b < 16384 ? b : 16384);
}

}  // namespace

size_t causal_attention_ws_bytes(int batch, int qh, int kvh, int seq) {
  const size_t A = 256;
  const size_t q = align_up((size_t)batch * qh * seq * kD * 2, A);
  const size_t kv = align_up((size_t)batch * kvh * seq * kD * 2, A);
  const size_t o = align_up((size_t)seq * qh * kD * 2, A);
  return q + 2 * kv + o;
}

int launch_causal_attention(const float* q, const float* k, const float* v, float* out, int batch, int qh,
                            int kvh, int seq, float scaling, void* ws, hipStream_t st) {
  const size_t A = 256;
  const size_t qn = (size_t)batch * qh * seq * kD, kvn = (size_t)batch * kvh * seq * kD;
  char* base = static_cast<char*>(ws);
  _Float16* q16 = reinterpret_cast<_Float16*>(base);
  _Float16* k16 = reinterpret_cast<_Float16*>(base + align_up(qn * 2, A));
  _Float16* v16 = reinterpret_cast<_Float16*>(reinterpret_cast<char*>(k16) + align_up(kvn * 2, A));
  _Float16* o16 = reinterpret_cast<_Float16*>(reinterpret_cast<char*>(v16) + align_up(kvn * 2, A));
  hipLaunchKernelGGL(to_f16_kernel, dim3(grid_for(qn / 4)), dim3(256), 0, st, q, q16, (long long)(qn / 4),
                     scaling * 1.4426950408889634f);
  hipLaunchKernelGGL(to_f16_kernel, dim3(grid_for(kvn / 4)), dim3(256), 0, st, k, k16, (long long)(kvn / 4), 1.0f);
  hipLaunchKernelGGL(to_f16_kernel, dim3(grid_for(kvn / 4)), dim3(256), 0, st, v, v16, (long long)(kvn / 4), 1.0f);
  int rc = check_launch();
  if (rc) return rc;
  for (int b = 0; b < batch; ++b) {
    PrefillArgs a;
    memset(&a, 0, sizeof(a));
    a.q16 = q16 + (size_t)b * qh * seq * kD;
    a.kcache = reinterpret_cast<uint16_t*>(k16 + (size_t)b * kvh * seq * kD);
    a.vcache = reinterpret_cast<uint16_t*>(v16 + (size_t)b * kvh * seq * kD);
    a.out = o16;
    a.n = seq;
    a.p0 = 0;
    a.qh = qh;
    a.kvh = kvh;
    a.max_ctx = seq;
    if ((rc = launch_prefill_attention(a, st))) return rc;
    const long long n4 = (long long)qh * seq * (kD / 4);
    hipLaunchKernelGGL(attn_out_kernel, dim3(grid_for(n4)), dim3(256), 0, st, o16, out + (size_t)b * qh * seq * kD,
                       seq, qh);
    if ((rc = check_launch())) return rc;
  }
  return Q4D_OK;
}

}  // namespace q4d
