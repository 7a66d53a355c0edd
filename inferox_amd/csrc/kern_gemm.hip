// kern_gemm.hip — dequant-to-LDS GEMM on the fp16 matrix cores (gfx950), the
// batched prefill form of ops::matmul_t (src/ops.rs:33-44,104-134) over the
// quantized weights of Weights::tensor_f32_by_index (src/gguf/weights.rs:66-74):
// C[t][n] = sum_k A[t][k] W[n][k], for t < M tokens and the n < rows of a
// weight matrix in the device layout (ifx_common.h).
//
// Arithmetic.  One fp16 rounding of either operand moves the logits of the
// synthetic models by up to 4% (their activations amplify rounding ~100x, and
// reach 4e7, past the fp16 range), so both operands are carried as fp16 pairs:
//   * W: every element is dequantized exactly as the reference does it (the
//     same f32 operations in the same order), then split w = w_hi + w_lo with
//     w_hi = fp16(w), w_lo = fp16(w - w_hi).  |w| is bounded by the block
//     scales (checked at model upload) and stays inside the fp16 range.
//   * A: row t is scaled by s_t = 2^(14 - e_t), e_t the exponent of the row's
//     largest magnitude (given as float bits in rowmax[t]), so that
//     |A s_t| < 2^15, then split the same way.
//   * Each 16x16x32 step runs three MFMAs, A_hi W_hi + A_hi W_lo + A_lo W_hi,
//     accumulating in f32; the A_lo W_lo term is below 2^-22 relative.  The
//     result is multiplied back by 2^(e_t - 14) (exact).
// Per product that is about 2^-21 relative, the level of the f32 reference's
// own roundings (float64 model of this scheme: 1e-5 relative L2 on the tiny
// model's logits, 5e-8 on the 8B shape).
//
// Tiling: a workgroup of 4 waves computes a 128 (tokens) x 128 (weight rows)
// tile; wave (wm, wn) owns 64 x 64 as 4 x 4 MFMA tiles.  Per 32-wide K step the
// workgroup converts one 128 x 32 slab of A and dequantizes one 128 x 32 slab
// of W into LDS (hi and lo planes, double-buffered: one barrier per step; 64 KB,
// two workgroups per CU), and
// the raw loads of the next step are in flight while the MFMAs run.  MFMA
// v_mfma_f32_16x16x32_f16: lane i + 16g holds A[i][8g..8g+7] and
// B[8g..8g+7][i]; C[4g + r][i] arrives in lane i + 16g, register r.
// Compiled with -ffp-contract=off: the dequant keeps the reference's roundings.
#include <algorithm>

#include "kernels.h"

namespace ifx {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kLdk = 32;  // halves per LDS row (64 B), 16-byte chunks XOR-swizzled by swz()
constexpr int kThreads = 256;
constexpr int kPlane = kBM * kLdk;  // halves in one 128 x 32 plane

struct GemmArgs {
  const float* a;         // [m x lda] f32
  const uint32_t* rowmax; // [m] float bits of max |A[t][:]|
  uint32_t m, lda, k;     // k = cols of the weight matrix, a multiple of 32
  GemmW w0, w1;           // w1: the second matrix of a paired launch (gate/up)
  uint32_t n;             // output columns: rows of w0 (paired: of each)
  uint32_t ksplit;        // K ranges over grid.z; > 1: partial tiles to `part`
  uint32_t kps;           // 32-wide K steps per range
  float* part;            // [ksplit][m][ncols], ncols = n (paired: 2n, up after gate)
};

// ---------------------------------------------------------------------------
// Weight slab loaders: thread (row n of the tile, half h) holds the raw bytes
// of elements [k0 + 16h, k0 + 16h + 16) of weight row `row`, then writes their
// dequantized fp16 pairs to LDS.  Element arithmetic as in dev_quant.h.
// ---------------------------------------------------------------------------
template <int T>
struct WRaw;

template <>
struct WRaw<T_Q4K> {  // tiled Q4_K (src/gguf/dequant.rs:133-161)
  uint4 hdr;
  uint2 qs;
  uint32_t sb;
  __device__ void load(const GemmW& w, uint32_t row, uint32_t k0, int h, bool ok) {
    sb = (k0 & 255u) >> 5;
    if (!ok) { hdr = make_uint4(0, 0, 0, 0); qs = make_uint2(0, 0); return; }
    const uint8_t* u = w.body + ((uint64_t)(row >> 4) * (w.cols >> 8) + (k0 >> 8)) * kUnitQ4K;
    const uint32_t nt = row & 15u;
    hdr = *(const uint4*)(u + 16u * nt);
    qs = *(const uint2*)(u + 256u + (sb >> 2) * 1024u + (nt + 16u * (sb & 3u)) * 16u + 8u * (uint32_t)h);
  }
  __device__ void dequant(float* y) const {
    // get_scale_min_k4 on the 12 scale bytes held in hdr.y/z/w (bytes 0-3, 4-7, 8-11)
    const uint32_t g = sb & 3u, y8 = hdr.y >> (8 * g), z8 = hdr.z >> (8 * g), w8 = hdr.w >> (8 * g);
    const uint32_t sc = sb < 4 ? (y8 & 63u) : ((w8 & 15u) | (((y8 >> 6) & 3u) << 4));
    const uint32_t mn = sb < 4 ? (z8 & 63u) : (((w8 >> 4) & 15u) | (((z8 >> 6) & 3u) << 4));
    const float d = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
    const float dall = d * (float)sc, dm = dmin * (float)mn;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t b = ((i < 4 ? qs.x : qs.y) >> (8 * (i & 3))) & 255u;
      y[2 * i] = dall * (float)(b & 15u) - dm;
      y[2 * i + 1] = dall * (float)(b >> 4) - dm;
    }
  }
};

template <>
struct WRaw<T_Q6K> {  // tiled Q6_K (src/gguf/dequant.rs:182-197)
  uint2 ql;
  uint32_t hw, sc, d;
  __device__ void load(const GemmW& w, uint32_t row, uint32_t k0, int h, bool ok) {
    if (!ok) { ql = make_uint2(0, 0); hw = sc = d = 0; return; }
    const uint32_t sb = (k0 & 255u) >> 5, nt = row & 15u;
    const uint8_t* u = w.body + ((uint64_t)(row >> 4) * (w.cols >> 8) + (k0 >> 8)) * kUnitQ6K;
    const uint32_t lane = nt + 16u * (sb & 3u), c = 2u * (sb >> 2) + (uint32_t)h;
    ql = *(const uint2*)(u + (sb >> 2) * 1024u + lane * 16u + 8u * (uint32_t)h);
    hw = *(const uint32_t*)(u + 2048u + lane * 16u + 4u * c);
    sc = u[3072u + 4u * lane + c];
    d = *(const uint16_t*)(u + 3328u + 2u * nt);
  }
  __device__ void dequant(float* y) const {
    const float ds = h2f(d) * (float)sc;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t b = ((k < 8 ? ql.x : ql.y) >> (8 * ((k >> 1) & 3))) & 255u;
      const uint32_t lo = (k & 1) ? (b >> 4) : (b & 15u);
      const uint32_t hi = (hw >> (8 * ((k & 7) >> 1) + 2 * (k & 1) + 4 * (k >> 3))) & 3u;
      y[k] = ds * (float)((int)(lo | (hi << 4)) - 32);
    }
  }
};

template <>
struct WRaw<T_Q8_0> {  // Q8_0: qs[nb][32] | d[nb] (src/gguf/dequant.rs:101-109)
  uint4 q;
  uint32_t d;
  __device__ void load(const GemmW& w, uint32_t row, uint32_t k0, int h, bool ok) {
    if (!ok) { q = make_uint4(0, 0, 0, 0); d = 0; return; }
    const uint64_t b = (uint64_t)row * (w.cols >> 5) + (k0 >> 5);
    q = *(const uint4*)(w.body + b * 32u + 16u * (uint32_t)h);
    d = ((const uint16_t*)w.scal)[b];
  }
  __device__ void dequant(float* y) const {
    const float delta = h2f(d);
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 16; k++) y[k] = (float)(int8_t)((v[k >> 2] >> (8 * (k & 3))) & 255u) * delta;
  }
};

template <>
struct WRaw<T_Q4_0> {  // Q4_0: qs[nb][16] | d[nb]; low nibbles -> j, high -> j + 16 (dequant.rs:70-82)
  uint4 q;
  uint32_t d;
  int half;
  __device__ void load(const GemmW& w, uint32_t row, uint32_t k0, int h, bool ok) {
    half = h;
    if (!ok) { q = make_uint4(0, 0, 0, 0); d = 0; return; }
    const uint64_t b = (uint64_t)row * (w.cols >> 5) + (k0 >> 5);
    q = *(const uint4*)(w.body + b * 16u);
    d = ((const uint16_t*)w.scal)[b];
  }
  __device__ void dequant(float* y) const {
    const float delta = h2f(d);
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t b = (v[k >> 2] >> (8 * (k & 3))) & 255u;
      y[k] = (float)((int)(half ? (b >> 4) : (b & 15u)) - 8) * delta;
    }
  }
};

// Physical 16-byte chunk of logical chunk c (0..3) in LDS row r: rows 4a + b
// keep chunk c at c ^ a, so the 16 rows of a fragment read land on 16
// distinct 4-bank groups (64-byte rows: rows b, b + 4, ... share banks).
__device__ __forceinline__ int swz(int r, int c) { return r * kLdk + 8 * (c ^ ((r >> 2) & 3)); }

// y[0..16) -> hi/lo halves of logical chunks 2h, 2h + 1 of LDS row r
__device__ __forceinline__ void split_store(const float* y, _Float16* hi_plane, _Float16* lo_plane, int r, int h) {
  _Float16* hi0 = hi_plane + swz(r, 2 * h);
  _Float16* hi1 = hi_plane + swz(r, 2 * h + 1);
  _Float16* lo0 = lo_plane + swz(r, 2 * h);
  _Float16* lo1 = lo_plane + swz(r, 2 * h + 1);
  h8 a0, a1, b0, b1;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const _Float16 x0 = (_Float16)y[k], x1 = (_Float16)y[k + 8];
    a0[k] = x0;
    a1[k] = x1;
    b0[k] = (_Float16)(y[k] - (float)x0);
    b1[k] = (_Float16)(y[k + 8] - (float)x1);
  }
  *(h8*)hi0 = a0;
  *(h8*)hi1 = a1;
  *(h8*)lo0 = b0;
  *(h8*)lo1 = b1;
}

// row t's scale exponent: |A[t][:] * 2^(14 - e)| < 2^15
__device__ __forceinline__ int row_exp(uint32_t bits) {
  const int e = (int)((bits >> 23) & 255u) - 127;
  return e < -100 ? -100 : e;
}

// ---------------------------------------------------------------------------
// Epilogues: v(t, n) for token t < m and output column n < a.n.
// ---------------------------------------------------------------------------
struct EpStore {  // y[t * ld + n] = v
  float* y;
  uint32_t ld;
  __device__ void operator()(uint32_t t, uint32_t n, float v, float) const { y[(uint64_t)t * ld + n] = v; }
};

struct EpResid {  // x[t * ld + n] += v (src/ops.rs:212-217)
  float* x;
  uint32_t ld;
  __device__ void operator()(uint32_t t, uint32_t n, float v, float) const {
    float* p = x + (uint64_t)t * ld + n;
    *p = *p + v;
  }
};

// Output (t, n) of a q/k/v projection at y[(row0 + t) ld + (n / head_dim)
// hstride + n % head_dim]: a row-major [t][heads * head_dim] buffer, or the
// head-major KV cache.
__device__ __forceinline__ uint64_t head_addr(uint32_t t, uint32_t n, uint32_t row0, uint32_t ld, uint64_t hstride,
                                              uint32_t head_dim) {
  return (uint64_t)(row0 + t) * ld + (uint64_t)(n / head_dim) * hstride + n % head_dim;
}

// RoPE on adjacent pairs (src/ops.rs:273-284) at position pos0 + t; `partner`
// is column n ^ 1 of the same token.
struct EpRope {
  float* y;
  uint64_t hstride;
  uint32_t ld, row0, pos0, head_dim, rope_dim, half;
  const float2* cs;  // [pos][rope_dim / 2]
  __device__ void operator()(uint32_t t, uint32_t n, float v, float partner) const {
    const uint32_t c = n % head_dim;
    float out = v;
    if (c < rope_dim) {
      const float2 r = cs[(uint64_t)(pos0 + t) * half + (c >> 1)];
      out = (c & 1u) ? (partner * r.y) + (v * r.x) : (v * r.x) - (partner * r.y);
    }
    y[head_addr(t, n, row0, ld, hstride, head_dim)] = out;
  }
};

struct EpRows {  // the V cache append
  float* y;
  uint64_t hstride;
  uint32_t ld, row0, head_dim;
  __device__ void operator()(uint32_t t, uint32_t n, float v, float) const {
    y[head_addr(t, n, row0, ld, hstride, head_dim)] = v;
  }
};

// swiglu (src/ops.rs:190-209): mid[t][n] = (g * (1 / (1 + expf(-clamp(g, -80, 80))))) * u
struct EpSwiglu {
  float* mid;
  uint32_t ld;
  __device__ void operator()(uint32_t t, uint32_t n, float g, float u) const {
    const float c = fminf(fmaxf(g, -80.f), 80.f);
    mid[(uint64_t)t * ld + n] = (g * (1.0f / (1.0f + expf(-c)))) * u;
  }
};

template <class Ep>
struct EpTraits {
  static constexpr bool kPaired = false, kNeighbor = false;
};
template <>
struct EpTraits<EpSwiglu> {
  static constexpr bool kPaired = true, kNeighbor = false;
};
template <>
struct EpTraits<EpRope> {
  static constexpr bool kPaired = false, kNeighbor = true;
};

__device__ __forceinline__ f4 mfma3(h8 ah, h8 al, h8 bh, h8 bl, f4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, c, 0, 0, 0);
}

template <int T, class Ep>
__global__ void __launch_bounds__(kThreads, 2) k_gemm(GemmArgs a, Ep ep) {
  constexpr bool kPaired = EpTraits<Ep>::kPaired;
  // [buffer][A hi, A lo, W hi, W lo][128][kLdk]
  __shared__ __attribute__((aligned(16))) _Float16 lds[2][4][kPlane];
  __shared__ int rexp[kBM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t m0 = blockIdx.y * kBM;
  // output columns of the tile (paired: gate rows n0.. in W rows 0..63, up in 64..127)
  const uint32_t n0 = blockIdx.x * (kPaired ? kBN / 2 : kBN);

  // staging roles: A row ar, W row wr, 16-element half h
  const int h = tid & 1, ar = tid >> 1, wr = tid >> 1;
  const uint32_t at = m0 + (uint32_t)ar;
  const bool a_ok = at < a.m;
  const GemmW& ws = (kPaired && wr >= 64) ? a.w1 : a.w0;
  const uint32_t wrow = kPaired ? n0 + (uint32_t)(wr & 63) : n0 + (uint32_t)wr;
  const uint32_t w_rows_avail = (T == T_Q4K || T == T_Q6K) ? (ws.rows + 15u) & ~15u : ws.rows;
  const bool w_ok = wrow < w_rows_avail && (!kPaired || n0 + (uint32_t)(wr & 63) < a.n);
  if (tid < kBM) rexp[tid] = m0 + (uint32_t)tid < a.m ? row_exp(a.rowmax[m0 + tid]) : 0;
  __syncthreads();
  const float ascale = ldexpf(1.0f, 14 - rexp[ar]);

  const float* arow = a.a + (uint64_t)(a_ok ? at : 0u) * a.lda + 16 * h;
  float4 ra[4];
  WRaw<T> rw;
  auto load_step = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < 4; i++) ra[i] = a_ok ? *(const float4*)(arow + k0 + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
    rw.load(ws, wrow, k0, h, w_ok);
  };
  auto stage = [&](int buf) {
    float y[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      y[4 * i] = ra[i].x * ascale;
      y[4 * i + 1] = ra[i].y * ascale;
      y[4 * i + 2] = ra[i].z * ascale;
      y[4 * i + 3] = ra[i].w * ascale;
    }
    split_store(y, lds[buf][0], lds[buf][1], ar, h);
    rw.dequant(y);
    split_store(y, lds[buf][2], lds[buf][3], wr, h);
  };

  f4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int fi = lane & 15, fg = lane >> 4;
  // W rows of this wave's four 16-column fragments
  int wcol[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    wcol[j] = kPaired ? (j < 2 ? wn * 32 + 16 * j : 64 + wn * 32 + 16 * (j - 2)) : wn * 64 + 16 * j;

  // this workgroup's K steps [ks0, ks1)
  const uint32_t ks0 = blockIdx.z * a.kps, ks1 = min(a.k / kBK, ks0 + a.kps);
  load_step(ks0 * kBK);
  for (uint32_t ks = ks0; ks < ks1; ks++) {
    const int buf = ks & 1;
    stage(buf);
    __syncthreads();
    if (ks + 1 < ks1) load_step((ks + 1) * kBK);
    h8 bh[4], bl[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      bh[j] = *(const h8*)&lds[buf][2][swz(wcol[j] + fi, fg)];
      bl[j] = *(const h8*)&lds[buf][3][swz(wcol[j] + fi, fg)];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = wm * 64 + 16 * i + fi;
      const h8 ah = *(const h8*)&lds[buf][0][swz(r, fg)];
      const h8 al = *(const h8*)&lds[buf][1][swz(r, fg)];
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = mfma3(ah, al, bh[j], bl[j], acc[i][j]);
    }
  }

  // epilogue: C[4 fg + r][fi] of fragment (i, j)
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int tl = wm * 64 + 16 * i + 4 * fg + r;
      const uint32_t t = m0 + (uint32_t)tl;
      const float inv = ldexpf(1.0f, rexp[tl] - 14);
      if (a.ksplit > 1) {  // partial tile of this K range; the reduce applies the epilogue
        const uint32_t ncols = kPaired ? 2 * a.n : a.n;
        float* pr = a.part + ((uint64_t)blockIdx.z * a.m + t) * ncols;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          uint32_t n, col;
          if (kPaired) {
            n = n0 + (uint32_t)(wn * 32 + 16 * (j & 1) + fi);
            col = n + (j >= 2 ? a.n : 0u);
          } else {
            n = n0 + (uint32_t)(wcol[j] + fi);
            col = n;
          }
          if (t < a.m && n < a.n) pr[col] = acc[i][j][r] * inv;
        }
        continue;
      }
      if (kPaired) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const uint32_t n = n0 + (uint32_t)(wn * 32 + 16 * j + fi);
          if (t < a.m && n < a.n) ep(t, n, acc[i][j][r] * inv, acc[i][j + 2][r] * inv);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint32_t n = n0 + (uint32_t)(wcol[j] + fi);
          const float v = acc[i][j][r] * inv;
          float partner = 0.f;
          if (EpTraits<Ep>::kNeighbor) partner = __shfl_xor(v, 1, 64);
          if (t < a.m && n < a.n) ep(t, n, v, partner);
        }
      }
    }
  }
}

// Sum of the K-range partials of output (t, n) in range order, then the
// epilogue: partner = column n ^ 1 (RoPE) or the up value of n (paired).
template <class Ep>
__global__ void k_gemm_reduce(GemmArgs a, Ep ep) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (uint64_t)a.m * a.n) return;
  const uint32_t t = (uint32_t)(idx / a.n), n = (uint32_t)(idx % a.n);
  const uint32_t ncols = EpTraits<Ep>::kPaired ? 2 * a.n : a.n;
  float v = 0.f, partner = 0.f;
  for (uint32_t z = 0; z < a.ksplit; z++) {
    const float* pr = a.part + ((uint64_t)z * a.m + t) * ncols;
    v += pr[n];
    if (EpTraits<Ep>::kPaired) partner += pr[n + a.n];
    else if (EpTraits<Ep>::kNeighbor && (n ^ 1u) < a.n) partner += pr[n ^ 1u];
  }
  ep(t, n, v, partner);
}

template <int T, class Ep>
hipError_t go(const GemmArgs& a, const Ep& ep, hipStream_t st) {
  const uint32_t bn = EpTraits<Ep>::kPaired ? kBN / 2 : kBN;
  dim3 grid((a.n + bn - 1) / bn, (a.m + kBM - 1) / kBM, a.ksplit);
  hipLaunchKernelGGL((k_gemm<T, Ep>), grid, dim3(kThreads), 0, st, a, ep);
  if (a.ksplit > 1) {
    const uint64_t total = (uint64_t)a.m * a.n;
    hipLaunchKernelGGL((k_gemm_reduce<Ep>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a, ep);
  }
  return hipGetLastError();
}

template <class Ep>
hipError_t dispatch(const GemmArgs& a, const Ep& ep, hipStream_t st) {
  if (a.m == 0 || a.n == 0) return hipSuccess;
  if (a.k == 0 || a.k % kBK || a.lda < a.k || a.lda % 4) return hipErrorInvalidValue;
  if (EpTraits<Ep>::kPaired && (a.w1.type != a.w0.type || a.w1.rows != a.w0.rows || a.w1.cols != a.w0.cols))
    return hipErrorInvalidValue;
  if (a.w0.cols != a.k) return hipErrorInvalidValue;
  if (a.ksplit == 0 || a.kps == 0) return hipErrorInvalidValue;
  switch (a.w0.type) {
    case T_Q4K: return go<T_Q4K, Ep>(a, ep, st);
    case T_Q6K: return go<T_Q6K, Ep>(a, ep, st);
    case T_Q8_0: return go<T_Q8_0, Ep>(a, ep, st);
    case T_Q4_0: return go<T_Q4_0, Ep>(a, ep, st);
    default: return hipErrorInvalidValue;
  }
}

// Tiles of fewer than two workgroups per CU split K over grid.z (at least 8
// steps per range), as far as the partial buffer holds them.
constexpr uint32_t kTargetWgs = 512, kMinStepsPerSplit = 8;

GemmArgs args_of(const GemmIn& in, const GemmW& w, bool paired) {
  GemmArgs a{};
  a.a = in.a;
  a.rowmax = in.rowmax;
  a.m = in.m;
  a.lda = in.lda;
  a.k = (uint32_t)w.cols;
  a.w0 = w;
  a.w1 = w;
  a.n = w.rows;
  const uint32_t nk = a.k / kBK, bn = paired ? kBN / 2 : kBN;
  const uint64_t tiles = (uint64_t)((a.n + bn - 1) / bn) * ((a.m + kBM - 1) / kBM);
  uint32_t split = 1;
  if (in.part && tiles < kTargetWgs) {
    split = (uint32_t)std::min<uint64_t>((kTargetWgs + tiles - 1) / tiles, std::max<uint32_t>(1, nk / kMinStepsPerSplit));
    const uint64_t per = (uint64_t)a.m * a.n * (paired ? 2 : 1) * 4;
    split = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>({split, in.part_bytes / per, 64}));
  }
  a.kps = (nk + split - 1) / split;
  a.ksplit = (nk + a.kps - 1) / a.kps;
  a.part = a.ksplit > 1 ? in.part : nullptr;
  return a;
}

// ---- row statistics and RMSNorm for the A operands ----

// rowmax[t] = float bits of max_k |x[t][k]| (positive floats order as integers)
__global__ void k_rowmax(const float* x, uint32_t ld, uint32_t cols, uint32_t* out) {
  const float* r = x + (uint64_t)blockIdx.x * ld;
  float m = 0.f;
  for (uint32_t k = threadIdx.x; k < cols; k += blockDim.x) m = fmaxf(m, fabsf(r[k]));
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  __shared__ float red[16];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (unsigned w = 1; w < blockDim.x / 64; w++) m = fmaxf(m, red[w]);
    m = fmaxf(m, red[0]);
    out[blockIdx.x] = __float_as_uint(m);
  }
}

// rms_norm (src/ops.rs:155-168) of each row into y, with the row's max |y|:
// scale = 1 / sqrt(sum(x^2) / n + eps), y = (x * scale) * w.
__global__ void k_rmsnorm_rows(const float* x, const float* w, uint32_t n, float eps, float* y, uint32_t* rowmax) {
  const float* r = x + (uint64_t)blockIdx.x * n;
  float* o = y + (uint64_t)blockIdx.x * n;
  float ss = 0.f;
  for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) ss = fmaf(r[k], r[k], ss);
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  __shared__ float red[16];
  __shared__ float scale_s;
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (unsigned v = 0; v < blockDim.x / 64; v++) t += red[v];
    scale_s = 1.0f / sqrtf(t / (float)n + eps);
  }
  __syncthreads();
  const float scale = scale_s;
  float m = 0.f;
  for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
    const float v = (r[k] * scale) * w[k];
    o[k] = v;
    m = fmaxf(m, fabsf(v));
  }
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (unsigned v = 1; v < blockDim.x / 64; v++) m = fmaxf(m, red[v]);
    m = fmaxf(m, red[0]);
    rowmax[blockIdx.x] = __float_as_uint(m);
  }
}

}  // namespace

bool gemm_type(uint32_t t) { return t == T_Q4K || t == T_Q6K || t == T_Q8_0 || t == T_Q4_0; }

hipError_t gemm_store(const GemmIn& in, const GemmW& w, float* y, uint32_t ldy, hipStream_t st) {
  return dispatch(args_of(in, w, false), EpStore{y, ldy}, st);
}

hipError_t gemm_residual(const GemmIn& in, const GemmW& w, float* x, uint32_t ldx, hipStream_t st) {
  return dispatch(args_of(in, w, false), EpResid{x, ldx}, st);
}

hipError_t gemm_rope(const GemmIn& in, const GemmW& w, float* y, uint32_t ldy, uint64_t hstride, uint32_t row0,
                     uint32_t pos0, uint32_t head_dim, uint32_t rope_dim, const float2* cs, hipStream_t st) {
  if (head_dim == 0 || head_dim % 2 || rope_dim % 2 || rope_dim > head_dim) return hipErrorInvalidValue;
  return dispatch(args_of(in, w, false), EpRope{y, hstride, ldy, row0, pos0, head_dim, rope_dim, rope_dim / 2, cs},
                  st);
}

hipError_t gemm_rows(const GemmIn& in, const GemmW& w, float* y, uint32_t ldy, uint64_t hstride, uint32_t row0,
                     uint32_t head_dim, hipStream_t st) {
  if (head_dim == 0) return hipErrorInvalidValue;
  return dispatch(args_of(in, w, false), EpRows{y, hstride, ldy, row0, head_dim}, st);
}

hipError_t gemm_swiglu(const GemmIn& in, const GemmW& gate, const GemmW& up, float* mid, uint32_t ld,
                       hipStream_t st) {
  GemmArgs a = args_of(in, gate, true);
  a.w1 = up;
  return dispatch(a, EpSwiglu{mid, ld}, st);
}

hipError_t launch_rowmax(const float* x, uint32_t rows, uint32_t ld, uint32_t cols, uint32_t* out, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rowmax, dim3(rows), dim3(256), 0, st, x, ld, cols, out);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows_to(const float* x, const float* w, uint32_t rows, uint32_t n, float eps, float* y,
                                  uint32_t* rowmax, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rmsnorm_rows, dim3(rows), dim3(256), 0, st, x, w, n, eps, y, rowmax);
  return hipGetLastError();
}

}  // namespace ifx
