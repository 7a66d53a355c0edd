// kern_gemm.hip — dequant-to-LDS GEMM on the fp16 matrix cores (gfx950), the
// batched prefill form of ops::matmul_t (src/ops.rs:33-44,104-134) over the
// quantized weights of Weights::tensor_f32_by_index (src/gguf/weights.rs:66-74):
// C[t][n] = sum_k A[t][k] W[n][k], for t < M tokens and the n < rows of a
// weight matrix in the device layout (ifx_common.h).
//
// Arithmetic (scale-factored).  Each quantized element is w = s * p - c with
// an integer p and scales shared by a block (src/gguf/dequant.rs):
//   Q4_K: p = sc q in 0..945, s = d per 256-element super-block, c = dmin mn
//         per 32-element group (dequant.rs:133-161);
//   Q6_K: p = sc (q - 32) with the u8 scale reaches 8160, past fp16's
//         integers: the weight (d sc)(q - 32) itself is carried instead, as
//         an fp16 pair w_hi + w_lo (dequant.rs:165-199);
//   Q8_0: p = q, s = delta per 32-block (dequant.rs:93-111);
//   Q4_0: p = q - 8, s = delta (dequant.rs:62-84).
// p is an exact fp16 integer, so the MFMAs run on the integers and the block
// scale is applied in f32 once per block: C = sum_b s[n][b] (sum_{k in b} p[n][k] A[t][k]) - sum_g c[n][g] S[t][g],
// S[t][g] the group sums of A.  The Q4_K min term is itself one K = 32 MFMA
// per super-block and tile (8 groups x the hi/lo parts of S against dmin mn,
// an exact fp16 pair).
// The activations are carried as fp16 pairs: k_prep_rows scales row t by
// 2^(14 - e_t) (e_t the exponent of its largest magnitude, |A s| < 2^15) and
// splits a = a_hi + a_lo; each 16x16x32 step runs a_hi p + a_lo p (Q6_K:
// a_hi w_hi + a_lo w_hi + a_hi w_lo), accumulating in f32.  Only the lo x lo
// term (below 2^-22 relative) is dropped: per product about 2^-21 relative, the level of the f32
// reference's own roundings.  One fp16 rounding of either operand would move
// the synthetic models' logits by up to 4%: their activations amplify
// rounding ~100x and reach 4e7, past the fp16 range.
//
// Element order: within every 8-element chunk of K both operands hold
// elements 0 4 1 5 2 6 3 7, the order in which a 32-bit word of nibbles
// unpacks into fp16 pairs ((w >> 4j) & 0x000F000F holds elements j, j + 4);
// k_prep_rows writes A in that order.
//
// Tiling: a workgroup of 8 waves (one per CU) computes a 128 (tokens) x 256
// (weight rows) tile; wave (wm, wn) owns 64 x 64 as 4 x 4 MFMA tiles.  The
// wide tile halves the A bytes (two fp16 planes, 7x the weight bytes) per
// MFMA against a 128 x 128 one.  Per 32-wide K step the workgroup copies one
// 128 x 32 slab of A (hi and lo planes) and unpacks one 256 x 32 slab of p
// into LDS (double-buffered: one barrier per step), and the raw loads of the
// next step are in flight while the MFMAs run.
// Block scales and the Q4_K min operands go to a per-block side area.
// MFMA v_mfma_f32_16x16x32_f16: lane i + 16g holds A[i][8g..8g+7] and
// B[8g..8g+7][i]; C[4g + r][i] arrives in lane i + 16g, register r
#include <algorithm>
#include <type_traits>

#include "kernels.h"

namespace ifx {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 256, kBK = 32;
constexpr int kLdk = 32;  // halves per LDS row (64 B), 16-byte chunks XOR-swizzled by swz()
constexpr int kThreads = 512;
constexpr int kAPlane = kBM * kLdk, kWPlane = kBN * kLdk;  // halves in one 128 (256) x 32 plane
constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024 in both halves: 0x6400 | u is 1024 + u (u < 1024)

struct GemmArgs {
  const uint16_t* ahi;   // [m][k] fp16, chunk order 0 4 1 5 2 6 3 7
  const uint16_t* alo;
  const uint16_t* gsum;  // [m][k / 256][16]: S_hi[8], S_lo[8] of each super-block (Q4_K)
  const int* rexp;       // [m] row scale exponents
  uint32_t m, k;         // k = cols of the weight matrix, a multiple of 32
  GemmW w0, w1;          // w1: the second matrix of a paired launch (gate/up)
  uint32_t n;            // output columns: rows of w0 (paired: of each)
  uint32_t ksplit;       // K ranges over grid.z; > 1: partial tiles to `part`
  uint32_t kps;          // 32-wide K steps per range (a multiple of the block's steps)
  float* part;           // [ksplit][m][ncols], ncols = n (paired: 2n, up after gate)
};

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 splat(float v) { return h2{(_Float16)v, (_Float16)v}; }

// Physical 16-byte chunk of logical chunk c (0..3) in LDS row r (64-byte
// rows): c ^ ((r >> 1) ^ (r >> 2)) & 3.  A fragment read (16 rows, one chunk)
// and a staging write (8 rows x 2 chunks per 16 lanes) then touch distinct
// banks both 8 lanes per cycle over 32 banks and 16 lanes over 64 (an
// r >> 2 swizzle left 2-way conflicts on every fragment read, measured).
__device__ __forceinline__ int swz(int r, int c) { return r * kLdk + 8 * (c ^ (((r >> 1) ^ (r >> 2)) & 3)); }

// Per-block side data: block scale of each weight row (f32) and, for Q4_K,
// the min-term operands: bm[n] = {hi[8], lo[8]} of -32 dmin mn per group,
// sa[t] = {hi[8], lo[8]} of S / 32 per group; rows padded to 40 bytes so the
// 8-byte reads of 16 rows fall on distinct banks.
constexpr int kSideRow = 20;
struct SideD {
  float d[kBN];
};
struct SideMin {
  float d[kBN];
  _Float16 bm[kBN][kSideRow];
  _Float16 sa[kBM][kSideRow];
};

// ---------------------------------------------------------------------------
// Weight staging: thread (row n of the tile, half h) loads the raw bytes of
// elements [16h, 16h + 16) of the step's 32 for weight row `row`, then writes
// their integers p as chunks 2h, 2h + 1 of LDS row n.
// ---------------------------------------------------------------------------
template <int T>
struct WQ;

template <>
struct WQ<T_Q4K> {  // tiled Q4_K (src/gguf/dequant.rs:133-161)
  static constexpr int kSb = 8;  // steps per super-block
  static constexpr bool kMins = true, kPLo = false, kScaled = true;
  typedef SideMin Side;
  uint4 hdr;  // d, dmin, 12 scale bytes: kept through the super-block
  uint2 qs;
  // g: the step's group within its super-block (a constant of the unrolled loop)
  __device__ void load(const GemmW& w, uint32_t row, uint32_t ks, uint32_t g, int h, bool sb0) {
    const uint8_t* u = w.body + (uint64_t)(row >> 4) * w.tstride + (uint64_t)(ks >> 3) * w.bstride;
    const uint32_t nt = row & 15u;
    if (sb0) hdr = *(const uint4*)(u + 16u * nt);
    qs = *(const uint2*)(u + 256u + (g >> 2) * 1024u + (nt + 16u * (g & 3u)) * 16u + 8u * (uint32_t)h);
  }
  // get_scale_min_k4 (dequant.rs:141-149) on the scale bytes in hdr.y/z/w
  __device__ void scale_min(uint32_t grp, uint32_t& sc, uint32_t& mn) const {
    const uint32_t s8 = 8 * (grp & 3u), y8 = hdr.y >> s8, z8 = hdr.z >> s8, w8 = hdr.w >> s8;
    sc = grp < 4 ? (y8 & 63u) : ((w8 & 15u) | (((y8 >> 6) & 3u) << 4));
    mn = grp < 4 ? (z8 & 63u) : (((w8 >> 4) & 15u) | (((z8 >> 6) & 3u) << 4));
  }
  __device__ void stage(_Float16* bp, _Float16*, Side& sd, uint32_t g, int wr, int h, bool sb0) const {
    uint32_t sc, mn;
    scale_min(g, sc, mn);
    // (1024 + q) sc - 1024 sc = q sc, one rounding of an exact integer <= 945
    const h2 s2 = splat((float)sc), o2 = splat(-1024.f * (float)sc);
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[j] = as_u32(__builtin_elementwise_fma(as_h2(((qs.x >> (4 * j)) & 0x000F000Fu) | kMagic), s2, o2));
      v[4 + j] = as_u32(__builtin_elementwise_fma(as_h2(((qs.y >> (4 * j)) & 0x000F000Fu) | kMagic), s2, o2));
    }
    *(uint4*)(bp + swz(wr, 2 * h)) = make_uint4(v[0], v[1], v[2], v[3]);
    *(uint4*)(bp + swz(wr, 2 * h + 1)) = make_uint4(v[4], v[5], v[6], v[7]);
    if (sb0) {
      const float d = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
      sd.d[wr] = d;  // both halves store the same value
      h4 bh, bl;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint32_t s_, m_;
        scale_min(4u * (uint32_t)h + (uint32_t)i, s_, m_);
        const float c = -(dmin * (float)m_) * 32.f;  // exact in f32; |c| < 2^16 (checked at upload)
        bh[i] = (_Float16)c;
        bl[i] = (_Float16)(c - (float)bh[i]);
      }
      *(h4*)&sd.bm[wr][4 * h] = bh;
      *(h4*)&sd.bm[wr][8 + 4 * h] = bl;
    }
  }
};

template <>
struct WQ<T_Q6K> {  // tiled Q6_K (src/gguf/dequant.rs:182-197)
  // The u8 scale makes p = sc (q - 32) up to 8160, past fp16's integers, so the
  // weight itself is carried: w = (d sc)(q - 32) as the reference rounds it
  // (d sc is exact, one rounding of the product), split w = w_hi + w_lo (22
  // bits of its 24).  No block scale is left to apply; |w| <= 8160 |d| stays
  // inside the fp16 range (checked at upload).
  static constexpr int kSb = 8;
  static constexpr bool kMins = false, kPLo = true, kScaled = false;
  typedef SideD Side;
  uint2 ql;
  uint32_t hw, d;
  int32_t sc;  // u8, or int8 for a tensor read in ggml's layout
  __device__ void load(const GemmW& w, uint32_t row, uint32_t ks, uint32_t g, int h, bool sb0) {
    const uint32_t nt = row & 15u;
    const uint8_t* u = w.body + (uint64_t)(row >> 4) * w.tstride + (uint64_t)(ks >> 3) * w.bstride;
    const uint32_t lane = nt + 16u * (g & 3u), c = 2u * (g >> 2) + (uint32_t)h;
    ql = *(const uint2*)(u + (g >> 2) * 1024u + lane * 16u + 8u * (uint32_t)h);
    hw = *(const uint32_t*)(u + 2048u + lane * 16u + 4u * c);
    const uint32_t sb = u[3072u + 4u * lane + c];
    sc = w.q6_signed ? (int32_t)(int8_t)sb : (int32_t)sb;
    if (sb0) d = *(const uint16_t*)(u + 3328u + 2u * nt);
  }
  // q of elements (j, j + 4) of chunk cc: low nibbles from ql, high parts at
  // bits 8 (j / 2) + 2 (j & 1) + 4 cc of hw (16 bits apart), as 1024 + q
  template <int CC, int J>
  __device__ __forceinline__ uint32_t q_pair() const {
    constexpr int s = 8 * (J >> 1) + 2 * (J & 1) + 4 * CC;
    const uint32_t lo = ((CC ? ql.y : ql.x) >> (4 * J)) & 0x000F000Fu;
    const uint32_t hi = (s >= 4 ? (hw >> (s - 4)) : (hw << (4 - s))) & 0x00300030u;
    return lo | hi | kMagic;
  }
  // The pair in packed fp16, three instructions per two elements (the f32
  // product and its split took ten): d sc (19 bits) = dh + dl exactly;
  // wh = fl(dh t); r = dh t - wh, exact (dh t has 17 bits, so r fits in 6)
  // from one fma; wl = fl(dl t + r).  Over every scale, quant and d from 1e-6
  // to 1, wh + wl is within 3.3e-7 relative of the reference's f32 weight
  // (the f32 split: 1.2e-7).
  __device__ void stage(_Float16* bp, _Float16* bpl, Side&, uint32_t, int wr, int h, bool) const {
    const float ds = h2f(d) * (float)sc;  // exact: 11 x 8 bits
    const _Float16 dh = (_Float16)ds;
    const _Float16 dl = (_Float16)(ds - (float)dh);  // exact: the low 8 of the 19 bits
    const h2 m2 = splat(-1056.f), dh2 = h2{dh, dh}, dl2 = h2{dl, dl};
    uint32_t vh[8], vl[8];
    auto pair = [&](uint32_t qv, int o) {
      const h2 t = as_h2(qv) + m2;  // q - 32, exact
      const h2 wh = dh2 * t;
      const h2 r = __builtin_elementwise_fma(dh2, t, -wh);
      const h2 wl = __builtin_elementwise_fma(dl2, t, r);
      vh[o] = as_u32(wh);
      vl[o] = as_u32(wl);
    };
    pair(q_pair<0, 0>(), 0);
    pair(q_pair<0, 1>(), 1);
    pair(q_pair<0, 2>(), 2);
    pair(q_pair<0, 3>(), 3);
    pair(q_pair<1, 0>(), 4);
    pair(q_pair<1, 1>(), 5);
    pair(q_pair<1, 2>(), 6);
    pair(q_pair<1, 3>(), 7);
    *(uint4*)(bp + swz(wr, 2 * h)) = make_uint4(vh[0], vh[1], vh[2], vh[3]);
    *(uint4*)(bp + swz(wr, 2 * h + 1)) = make_uint4(vh[4], vh[5], vh[6], vh[7]);
    *(uint4*)(bpl + swz(wr, 2 * h)) = make_uint4(vl[0], vl[1], vl[2], vl[3]);
    *(uint4*)(bpl + swz(wr, 2 * h + 1)) = make_uint4(vl[4], vl[5], vl[6], vl[7]);
  }
};

// bytes j of x and y as the fp16-pair word (x_j, 0, y_j, 0)
__device__ __forceinline__ uint32_t byte_pair(uint32_t x, uint32_t y, int j) {
  return __builtin_amdgcn_perm(y, x, (uint32_t)j | (0x0cu << 8) | ((uint32_t)(4 + j) << 16) | (0x0cu << 24));
}

template <>
struct WQ<T_Q8_0> {  // Q8_0: qs[nb][32] | d[nb] (src/gguf/dequant.rs:101-109)
  static constexpr int kSb = 1;
  static constexpr bool kMins = false, kPLo = false, kScaled = true;
  typedef SideD Side;
  uint4 q;
  uint32_t d;
  __device__ void load(const GemmW& w, uint32_t row, uint32_t ks, uint32_t, int h, bool) {
    const uint64_t b = (uint64_t)row * (w.cols >> 5) + ks;
    q = *(const uint4*)(w.body + b * 32u + 16u * (uint32_t)h);
    d = ((const uint16_t*)w.scal)[b];
  }
  __device__ void stage(_Float16* bp, _Float16*, Side& sd, uint32_t, int wr, int h, bool) const {
    // int8 -> 1024 + (q + 128) by flipping the sign bit under the fp16 1024 pattern
    const h2 m2 = splat(-1152.f);
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[j] = as_u32(as_h2(byte_pair(q.x, q.y, j) ^ 0x64806480u) + m2);
      v[4 + j] = as_u32(as_h2(byte_pair(q.z, q.w, j) ^ 0x64806480u) + m2);
    }
    *(uint4*)(bp + swz(wr, 2 * h)) = make_uint4(v[0], v[1], v[2], v[3]);
    *(uint4*)(bp + swz(wr, 2 * h + 1)) = make_uint4(v[4], v[5], v[6], v[7]);
    sd.d[wr] = h2f(d);
  }
};

template <>
struct WQ<T_Q4_0> {  // Q4_0: qs[nb][16] | d[nb]; low nibbles -> j, high -> j + 16 (dequant.rs:70-82)
  static constexpr int kSb = 1;
  static constexpr bool kMins = false, kPLo = false, kScaled = true;
  typedef SideD Side;
  uint4 q;
  uint32_t d;
  __device__ void load(const GemmW& w, uint32_t row, uint32_t ks, uint32_t, int, bool) {
    const uint64_t b = (uint64_t)row * (w.cols >> 5) + ks;
    q = *(const uint4*)(w.body + b * 16u);
    d = ((const uint16_t*)w.scal)[b];
  }
  __device__ void stage(_Float16* bp, _Float16*, Side& sd, uint32_t, int wr, int h, bool) const {
    const h2 m2 = splat(-1032.f);  // 1024 + q - 1032 = q - 8
    const int sh = 4 * h;          // half h: the high nibbles (elements 16..31)
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[j] = as_u32(as_h2(((byte_pair(q.x, q.y, j) >> sh) & 0x000F000Fu) | kMagic) + m2);
      v[4 + j] = as_u32(as_h2(((byte_pair(q.z, q.w, j) >> sh) & 0x000F000Fu) | kMagic) + m2);
    }
    *(uint4*)(bp + swz(wr, 2 * h)) = make_uint4(v[0], v[1], v[2], v[3]);
    *(uint4*)(bp + swz(wr, 2 * h + 1)) = make_uint4(v[4], v[5], v[6], v[7]);
    sd.d[wr] = h2f(d);
  }
};

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
// y_f16: y holds binary16 (the f16 KV cache), rounded to nearest even.
__device__ __forceinline__ void store_y(void* y, bool f16, uint64_t i, float v) {
  if (f16) ((_Float16*)y)[i] = (_Float16)v;
  else ((float*)y)[i] = v;
}

struct EpRope {
  void* y;
  uint64_t hstride;
  uint32_t ld, row0, pos0, head_dim, rope_dim, half;
  const float2* cs;  // [pos][rope_dim / 2]
  bool y_f16;
  __device__ void operator()(uint32_t t, uint32_t n, float v, float partner) const {
    const uint32_t c = n % head_dim;
    float out = v;
    if (c < rope_dim) {
      const float2 r = cs[(uint64_t)(pos0 + t) * half + (c >> 1)];
      out = (c & 1u) ? (partner * r.y) + (v * r.x) : (v * r.x) - (partner * r.y);
    }
    store_y(y, y_f16, head_addr(t, n, row0, ld, hstride, head_dim), out);
  }
};

struct EpRows {  // the V cache append
  void* y;
  uint64_t hstride;
  uint32_t ld, row0, head_dim;
  bool y_f16;
  __device__ void operator()(uint32_t t, uint32_t n, float v, float) const {
    store_y(y, y_f16, head_addr(t, n, row0, ld, hstride, head_dim), v);
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

template <int T, class Ep>
__global__ void __launch_bounds__(kThreads, 1) k_gemm(GemmArgs a, Ep ep) {
  using Q = WQ<T>;
  constexpr bool kPaired = EpTraits<Ep>::kPaired;
  constexpr int kNw = Q::kPLo ? 2 : 1;  // weight planes: p (hi), [p lo]
  __shared__ __attribute__((aligned(16))) _Float16 la[2][2][kAPlane];    // [buffer][A hi, A lo]
  __shared__ __attribute__((aligned(16))) _Float16 lw[2][kNw][kWPlane];  // [buffer][p hi, p lo]
  __shared__ __attribute__((aligned(16))) typename Q::Side side[2];
  __shared__ int rexp[kBM];
  // the wave index as a scalar: the wave's fragment rows and columns are
  // uniform over it and stay out of the vector registers
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const uint32_t m0 = blockIdx.y * kBM;
  // output columns of the tile (paired: gate rows n0.. in W rows 0..127, up in 128..255)
  const uint32_t n0 = blockIdx.x * (kPaired ? kBN / 2 : kBN);

  // staging roles: A row ar chunk ac (both planes), W row wr half h.
  // Rows past the operands read a clamped row: their outputs are never stored.
  const int h = tid & 1, wr = tid >> 1, ar = tid >> 2, ac = tid & 3;
  const uint32_t at = min(m0 + (uint32_t)ar, a.m - 1);
  const GemmW& ws = (kPaired && wr >= kBN / 2) ? a.w1 : a.w0;
  const uint32_t w_rows_avail = (T == T_Q4K || T == T_Q6K) ? (ws.rows + 15u) & ~15u : ws.rows;
  const uint32_t wrow =
      min(kPaired ? n0 + (uint32_t)(wr & (kBN / 2 - 1)) : n0 + (uint32_t)wr, w_rows_avail - 1);
  if (tid < kBM) rexp[tid] = m0 + (uint32_t)tid < a.m ? a.rexp[m0 + tid] : 0;

  const uint64_t arow = (uint64_t)at * a.k + 8u * (uint32_t)ac;
  const uint16_t* ahi = a.ahi + arow;
  const uint16_t* alo = a.alo + arow;
  // group sums: thread (row ar, ac < 2) fetches S_hi (ac 0) or S_lo (ac 1)
  const uint16_t* gs = Q::kMins ? a.gsum + (uint64_t)at * (a.k >> 8) * 16u + 8u * (uint32_t)(ac & 1) : nullptr;
  uint4 ra0, ra1;  // chunk ac of the hi and lo planes
  uint4 rs = make_uint4(0, 0, 0, 0);  // S_hi or S_lo of the row's super-block (Q4_K)
  Q rw;
  // raw loads of step ks, group g of its block (sb0: g == 0)
  auto load_step = [&](uint32_t ks, uint32_t g, bool sb0) __attribute__((always_inline)) {
    const uint32_t k0 = ks * kBK;
    ra0 = *(const uint4*)(ahi + k0);
    ra1 = *(const uint4*)(alo + k0);
    if (Q::kMins && sb0) rs = *(const uint4*)(gs + (ks >> 3) * 16u);  // ac >= 2: a duplicate, unused
    rw.load(ws, wrow, ks, g, h, sb0);
  };
  auto stage = [&](int buf, int sbi, uint32_t g, bool sb0) __attribute__((always_inline)) {
    *(uint4*)(la[buf][0] + swz(ar, ac)) = ra0;
    *(uint4*)(la[buf][1] + swz(ar, ac)) = ra1;
    if constexpr (Q::kMins) {
      if (sb0 && ac < 2) {  // 8-byte aligned rows: two 8-byte stores
        *(uint2*)&side[sbi].sa[ar][8 * ac] = make_uint2(rs.x, rs.y);
        *(uint2*)&side[sbi].sa[ar][8 * ac + 4] = make_uint2(rs.z, rs.w);
      }
    }
    rw.stage(lw[buf][0], Q::kPLo ? lw[buf][kNw - 1] : nullptr, side[sbi], g, wr, h, sb0);
  };

  f4 acc[4][4], cs[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
      cs[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    }

  const int fi = lane & 15, fg = lane >> 4;
  // W rows of this wave's four 16-column fragments
  int wcol[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    wcol[j] = kPaired ? (j < 2 ? wn * 32 + 16 * j : kBN / 2 + wn * 32 + 16 * (j - 2)) : wn * 64 + 16 * j;

  // the block's integer dot products: cs = (first step of a block ? 0 : cs) + a p
  auto mma = [&](int buf, auto first) __attribute__((always_inline)) {
    constexpr bool kFirst = decltype(first)::value;
    h8 bh[4], bl[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      bh[j] = *(const h8*)&lw[buf][0][swz(wcol[j] + fi, fg)];
      if (Q::kPLo) bl[j] = *(const h8*)&lw[buf][kNw - 1][swz(wcol[j] + fi, fg)];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = wm * 64 + 16 * i + fi;
      const h8 ah = *(const h8*)&la[buf][0][swz(r, fg)];
      const h8 al = *(const h8*)&la[buf][1][swz(r, fg)];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if constexpr (Q::kScaled) {
          f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[j], kFirst ? f4{0.f, 0.f, 0.f, 0.f} : cs[i][j], 0, 0, 0);
          cs[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[j], c, 0, 0, 0);
        } else {  // the weight itself: straight into acc
          f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[j], acc[i][j], 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[j], c, 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[j], c, 0, 0, 0);
        }
      }
    }
  };
  // end of a block: acc += s cs (and the Q4_K min term)
  auto flush = [&](int sbi) __attribute__((always_inline)) {
    if constexpr (!Q::kScaled) return;
    const typename Q::Side& sd = side[sbi];
    float dj[4];
#pragma unroll
    for (int j = 0; j < 4; j++) dj[j] = sd.d[wcol[j] + fi];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[i][j][r] = fmaf(dj[j], cs[i][j][r], acc[i][j][r]);
    if constexpr (Q::kMins) {
      // Two K = 16 products: lanes of group g take S_hi (g < 2) or S_lo
      // (g >= 2) of groups 4 (g & 1) .. + 3 against the hi parts; the second
      // adds S_hi against the lo parts.  They run as one K = 32 MFMA (a1 a2
      // against b1 b2 in each lane's 8 k slots: the same sum of products), at
      // the cost of one K = 16 one on gfx950.
      const h4 z = {0, 0, 0, 0};
      h4 a1[4], a2[4], b1[4], b2[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        a1[i] = *(const h4*)&sd.sa[wm * 64 + 16 * i + fi][4 * fg];
        a2[i] = fg < 2 ? a1[i] : z;
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        b1[j] = *(const h4*)&sd.bm[wcol[j] + fi][4 * (fg & 1)];
        const h4 lo = *(const h4*)&sd.bm[wcol[j] + fi][8 + 4 * (fg & 1)];
        b2[j] = fg < 2 ? lo : z;
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const h8 a = __builtin_shufflevector(a1[i], a2[i], 0, 1, 2, 3, 4, 5, 6, 7);
          const h8 b = __builtin_shufflevector(b1[j], b2[j], 0, 1, 2, 3, 4, 5, 6, 7);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[i][j], 0, 0, 0);
        }
    }
  };

  // this workgroup's K steps [ks0, ks1): whole blocks.  Step ks runs the
  // MFMAs of buffer ks & 1 while unpacking step ks + 1 into the other buffer
  // (its last readers finished before the previous barrier), then issues the
  // raw loads of step ks + 2: one barrier per step, and a whole block of
  // steps unrolled so that the MFMAs and the unpacking interleave.
  const uint32_t ks0 = blockIdx.z * a.kps, ks1 = min(a.k / kBK, ks0 + a.kps);
  const uint32_t klast = ks1 - 1;  // loads past the range re-read its last step (unused)
  __syncthreads();  // rexp
  load_step(ks0, 0, true);
  stage(ks0 & 1, (ks0 / Q::kSb) & 1, 0, true);
  load_step(min(ks0 + 1, klast), 1 % Q::kSb, Q::kSb == 1);
  __syncthreads();
  auto step = [&](uint32_t kb, int i) __attribute__((always_inline)) {
    const int sbi = (kb / Q::kSb) & 1;
    const uint32_t ks = kb + (uint32_t)i;
    const int buf = Q::kSb % 2 == 0 ? (i & 1) ^ (int)(kb & 1) : (int)(ks & 1);
    if (i == 0) mma(buf, std::true_type{});
    else mma(buf, std::false_type{});
    // step ks + 1 starts a block when i is the block's last step
    stage(buf ^ 1, i == Q::kSb - 1 ? sbi ^ 1 : sbi, (uint32_t)((i + 1) % Q::kSb), i == Q::kSb - 1);
    if (i == Q::kSb - 1) flush(sbi);
    // the next raw loads reuse the registers just unpacked: no second set
    __builtin_amdgcn_sched_barrier(0);
    // group and block start by position (a clamped load past the range is unused)
    load_step(min(ks + 2, klast), (uint32_t)((i + 2) % Q::kSb), (i + 2) % Q::kSb == 0);
    __syncthreads();
  };
  for (uint32_t kb = ks0; kb < ks1; kb += Q::kSb) {
#pragma unroll
    for (int i = 0; i < Q::kSb; i++) step(kb, i);
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

// The same sums four outputs (t, 4i .. 4i + 3) per thread, as 16-byte loads
// (n % 4 == 0): each output's partials are added in the same order, so the
// bits are those of k_gemm_reduce.  The RoPE partner n ^ 1 is in the same four.
template <class Ep>
__global__ void k_gemm_reduce4(GemmArgs a, Ep ep) {
  const uint32_t n4 = a.n / 4;
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (uint64_t)a.m * n4) return;
  const uint32_t t = (uint32_t)(idx / n4), n = 4 * (uint32_t)(idx % n4);
  const uint32_t ncols = EpTraits<Ep>::kPaired ? 2 * a.n : a.n;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f), u = v;
  for (uint32_t z = 0; z < a.ksplit; z++) {
    const float* pr = a.part + ((uint64_t)z * a.m + t) * ncols;
    const float4 x = *(const float4*)(pr + n);
    v.x += x.x; v.y += x.y; v.z += x.z; v.w += x.w;
    if (EpTraits<Ep>::kPaired) {
      const float4 y = *(const float4*)(pr + n + a.n);
      u.x += y.x; u.y += y.y; u.z += y.z; u.w += y.w;
    }
  }
  if (!EpTraits<Ep>::kPaired && EpTraits<Ep>::kNeighbor) u = make_float4(v.y, v.x, v.w, v.z);
  ep(t, n, v.x, u.x);
  ep(t, n + 1, v.y, u.y);
  ep(t, n + 2, v.z, u.z);
  ep(t, n + 3, v.w, u.w);
}

template <int T, class Ep>
hipError_t go(const GemmArgs& a, const Ep& ep, hipStream_t st) {
  const uint32_t bn = EpTraits<Ep>::kPaired ? kBN / 2 : kBN;
  dim3 grid((a.n + bn - 1) / bn, (a.m + kBM - 1) / kBM, a.ksplit);
  hipLaunchKernelGGL((k_gemm<T, Ep>), grid, dim3(kThreads), 0, st, a, ep);
  if (a.ksplit > 1) {
    if (a.n % 4 == 0) {
      const uint64_t total = (uint64_t)a.m * (a.n / 4);
      hipLaunchKernelGGL((k_gemm_reduce4<Ep>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a, ep);
    } else {
      const uint64_t total = (uint64_t)a.m * a.n;
      hipLaunchKernelGGL((k_gemm_reduce<Ep>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a, ep);
    }
  }
  return hipGetLastError();
}

template <class Ep>
hipError_t dispatch(const GemmArgs& a, const Ep& ep, hipStream_t st) {
  if (a.m == 0 || a.n == 0) return hipSuccess;
  if (a.k == 0 || a.k % kBK || !a.ahi || !a.alo || !a.rexp) return hipErrorInvalidValue;
  if (EpTraits<Ep>::kPaired && (a.w1.type != a.w0.type || a.w1.rows != a.w0.rows || a.w1.cols != a.w0.cols))
    return hipErrorInvalidValue;
  if (a.w0.cols != a.k) return hipErrorInvalidValue;
  if (a.ksplit == 0 || a.kps == 0) return hipErrorInvalidValue;
  switch (a.w0.type) {
    case T_Q4K:
      if (a.k % 256 || !a.gsum || a.kps % WQ<T_Q4K>::kSb) return hipErrorInvalidValue;
      return go<T_Q4K, Ep>(a, ep, st);
    case T_Q6K:
      if (a.k % 256 || a.kps % WQ<T_Q6K>::kSb) return hipErrorInvalidValue;
      return go<T_Q6K, Ep>(a, ep, st);
    case T_Q8_0: return go<T_Q8_0, Ep>(a, ep, st);
    case T_Q4_0: return go<T_Q4_0, Ep>(a, ep, st);
    default: return hipErrorInvalidValue;
  }
}

// Tiles of fewer than one workgroup per CU split K over grid.z (at least 8
// steps per range), as far as the partial buffer holds them.
constexpr uint32_t kTargetWgs = 256, kMinStepsPerSplit = 8;

GemmArgs args_of(const GemmIn& in, const GemmW& w, bool paired) {
  GemmArgs a{};
  a.ahi = in.hi;
  a.alo = in.lo;
  a.gsum = in.gsum;
  a.rexp = in.rexp;
  a.m = in.m;
  a.k = (uint32_t)w.cols;
  a.w0 = w;
  a.w1 = w;
  a.n = w.rows;
  const uint32_t nk = a.k / kBK, bn = paired ? kBN / 2 : kBN;
  const uint32_t sb = (w.type == T_Q4K || w.type == T_Q6K) ? 8u : 1u;  // steps per scale block
  const uint64_t tiles = (uint64_t)((a.n + bn - 1) / bn) * ((a.m + kBM - 1) / kBM);
  uint32_t split = 1;
  if (in.part && tiles < kTargetWgs) {
    split = (uint32_t)std::min<uint64_t>((kTargetWgs + tiles - 1) / tiles, std::max<uint32_t>(1, nk / kMinStepsPerSplit));
    const uint64_t per = (uint64_t)a.m * a.n * (paired ? 2 : 1) * 4;
    split = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>({split, in.part_bytes / per, 64}));
  }
  a.kps = (nk + split - 1) / split;
  a.kps = (a.kps + sb - 1) / sb * sb;  // ranges of whole scale blocks
  a.ksplit = (nk + a.kps - 1) / a.kps;
  a.part = a.ksplit > 1 ? in.part : nullptr;
  return a;
}

// ---- the A operand: fp16 pairs, group sums and row exponents ----

// Row t of x (optionally rms_norm'ed, src/ops.rs:155-168: y = (x * scale) * w,
// scale = 1 / sqrt(sum(x^2) / n + eps)), scaled by 2^(14 - e) with e the
// exponent of its largest magnitude, split into fp16 hi + lo in the chunk
// order 0 4 1 5 2 6 3 7; the 32-element group sums of the scaled row / 32 as
// fp16 pairs when cols % 256 == 0.  One workgroup per row; thread i takes the
// 8-element chunks i, i + 256, ... (a group is four consecutive threads).
__global__ void __launch_bounds__(256) k_prep_rows(const float* x, uint32_t ld, uint32_t cols, const float* nw,
                                                   float eps, uint16_t* hi, uint16_t* lo, uint16_t* gsum,
                                                   int* rexp) {
  const uint32_t t = blockIdx.x, nch = cols / 8;
  const float4* r4 = (const float4*)(x + (uint64_t)t * ld);
  const float4* w4 = (const float4*)nw;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ float red[4];
  __shared__ float bcast;
  auto row8 = [&](uint32_t c, float* v, float scale) {
    const float4 u0 = r4[2 * c], u1 = r4[2 * c + 1];
    v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
    v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
    if (nw) {
      const float4 g0 = w4[2 * c], g1 = w4[2 * c + 1];
      const float w[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int k = 0; k < 8; k++) v[k] = (v[k] * scale) * w[k];
    }
  };
  float scale = 1.f;
  if (nw) {
    float ss = 0.f;
    for (uint32_t c = tid; c < nch; c += 256) {
      const float4 u0 = r4[2 * c], u1 = r4[2 * c + 1];
      ss = fmaf(u0.x, u0.x, ss); ss = fmaf(u0.y, u0.y, ss); ss = fmaf(u0.z, u0.z, ss); ss = fmaf(u0.w, u0.w, ss);
      ss = fmaf(u1.x, u1.x, ss); ss = fmaf(u1.y, u1.y, ss); ss = fmaf(u1.z, u1.z, ss); ss = fmaf(u1.w, u1.w, ss);
    }
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    if (tid == 0) bcast = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)cols + eps);
    __syncthreads();
    scale = bcast;
  }
  float m = 0.f;
  for (uint32_t c = tid; c < nch; c += 256) {
    float v[8];
    row8(c, v, scale);
#pragma unroll
    for (int k = 0; k < 8; k++) m = fmaxf(m, fabsf(v[k]));
  }
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  __syncthreads();
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = (int)((__float_as_uint(m) >> 23) & 255u) - 127;
  e = e < -100 ? -100 : e;
  if (tid == 0) rexp[t] = e;
  const float s = ldexpf(1.0f, 14 - e);
  const bool sums = gsum && cols % 256 == 0;
  uint16_t* ho = hi + (uint64_t)t * cols;
  uint16_t* lw = lo + (uint64_t)t * cols;
  for (uint32_t c0 = 0; c0 < nch; c0 += 256) {
    const uint32_t c = c0 + tid;
    const bool ok = c < nch;  // nch is a multiple of 4: a group's threads agree
    float v[8];
    if (ok) row8(c, v, scale);
    else
      for (int k = 0; k < 8; k++) v[k] = 0.f;
    h8 vh, vl;
    float s8 = 0.f;
#pragma unroll
    for (int p = 0; p < 8; p++) {
      const float y = v[(p >> 1) + 4 * (p & 1)] * s;
      vh[p] = (_Float16)y;
      vl[p] = (_Float16)(y - (float)vh[p]);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) s8 += v[k] * s;
    if (ok) {
      *(h8*)(ho + 8u * c) = vh;
      *(h8*)(lw + 8u * c) = vl;
    }
    if (sums) {
      s8 += __shfl_xor(s8, 1, 64);
      s8 += __shfl_xor(s8, 2, 64);
      if (ok && (c & 3u) == 0) {
        const uint32_t g = c >> 2;
        const float sg = s8 * 0.03125f;
        const _Float16 sh = (_Float16)sg, sl = (_Float16)(sg - (float)sh);
        _Float16* dst = (_Float16*)gsum + ((uint64_t)t * (cols >> 8) + (g >> 3)) * 16u + (g & 7u);
        dst[0] = sh;
        dst[8] = sl;
      }
    }
  }
}

// The same with the thread's chunks of the row held in registers from one
// load (up to NCT of them: rows of up to 2048 NCT columns), instead of
// reading the row again for the maximum and the split.  Same arithmetic in
// the same order: the same bits.
template <int NCT>
__global__ void __launch_bounds__(256) k_prep_rows_reg(const float* x, uint32_t ld, uint32_t cols, const float* nw,
                                                       float eps, uint16_t* hi, uint16_t* lo, uint16_t* gsum,
                                                       int* rexp) {
  const uint32_t t = blockIdx.x, nch = cols / 8;
  const float4* r4 = (const float4*)(x + (uint64_t)t * ld);
  const float4* w4 = (const float4*)nw;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ float red[4];
  __shared__ float bcast;
  // the thread's chunks tid + 256 j, loaded once (zeros past the row)
  float4 ru[NCT][2];
#pragma unroll
  for (int j = 0; j < NCT; j++) {
    const uint32_t c = tid + 256u * j;
    ru[j][0] = c < nch ? r4[2 * c] : make_float4(0.f, 0.f, 0.f, 0.f);
    ru[j][1] = c < nch ? r4[2 * c + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  auto row8 = [&](int j, uint32_t c, float* v, float scale) {
    const float4 u0 = ru[j][0], u1 = ru[j][1];
    v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
    v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
    if (nw) {
      const float4 g0 = w4[2 * c], g1 = w4[2 * c + 1];
      const float w[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int k = 0; k < 8; k++) v[k] = (v[k] * scale) * w[k];
    }
  };
  float scale = 1.f;
  if (nw) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NCT; j++) {
      if (tid + 256u * j >= nch) break;
      const float4 u0 = ru[j][0], u1 = ru[j][1];
      ss = fmaf(u0.x, u0.x, ss); ss = fmaf(u0.y, u0.y, ss); ss = fmaf(u0.z, u0.z, ss); ss = fmaf(u0.w, u0.w, ss);
      ss = fmaf(u1.x, u1.x, ss); ss = fmaf(u1.y, u1.y, ss); ss = fmaf(u1.z, u1.z, ss); ss = fmaf(u1.w, u1.w, ss);
    }
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    if (tid == 0) bcast = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)cols + eps);
    __syncthreads();
    scale = bcast;
  }
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < NCT; j++) {
    const uint32_t c = tid + 256u * j;
    if (c >= nch) break;
    float v[8];
    row8(j, c, v, scale);
#pragma unroll
    for (int k = 0; k < 8; k++) m = fmaxf(m, fabsf(v[k]));
  }
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  __syncthreads();
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = (int)((__float_as_uint(m) >> 23) & 255u) - 127;
  e = e < -100 ? -100 : e;
  if (tid == 0) rexp[t] = e;
  const float s = ldexpf(1.0f, 14 - e);
  const bool sums = gsum && cols % 256 == 0;
  uint16_t* ho = hi + (uint64_t)t * cols;
  uint16_t* lw = lo + (uint64_t)t * cols;
#pragma unroll
  for (int j = 0; j < NCT; j++) {
    if (256u * j >= nch) break;
    const uint32_t c = 256u * j + tid;
    const bool ok = c < nch;  // nch is a multiple of 4: a group's threads agree
    float v[8];
    if (ok) row8(j, c, v, scale);
    else
      for (int k = 0; k < 8; k++) v[k] = 0.f;
    h8 vh, vl;
    float s8 = 0.f;
#pragma unroll
    for (int p = 0; p < 8; p++) {
      const float y = v[(p >> 1) + 4 * (p & 1)] * s;
      vh[p] = (_Float16)y;
      vl[p] = (_Float16)(y - (float)vh[p]);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) s8 += v[k] * s;
    if (ok) {
      *(h8*)(ho + 8u * c) = vh;
      *(h8*)(lw + 8u * c) = vl;
    }
    if (sums) {
      s8 += __shfl_xor(s8, 1, 64);
      s8 += __shfl_xor(s8, 2, 64);
      if (ok && (c & 3u) == 0) {
        const uint32_t g = c >> 2;
        const float sg = s8 * 0.03125f;
        const _Float16 sh = (_Float16)sg, sl = (_Float16)(sg - (float)sh);
        _Float16* dst = (_Float16*)gsum + ((uint64_t)t * (cols >> 8) + (g >> 3)) * 16u + (g & 7u);
        dst[0] = sh;
        dst[8] = sl;
      }
    }
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

hipError_t gemm_rope(const GemmIn& in, const GemmW& w, void* y, uint32_t ldy, uint64_t hstride, uint32_t row0,
                     uint32_t pos0, uint32_t head_dim, uint32_t rope_dim, const float2* cs, hipStream_t st,
                     bool y_f16) {
  if (head_dim == 0 || head_dim % 2 || rope_dim % 2 || rope_dim > head_dim) return hipErrorInvalidValue;
  return dispatch(args_of(in, w, false),
                  EpRope{y, hstride, ldy, row0, pos0, head_dim, rope_dim, rope_dim / 2, cs, y_f16}, st);
}

hipError_t gemm_rows(const GemmIn& in, const GemmW& w, void* y, uint32_t ldy, uint64_t hstride, uint32_t row0,
                     uint32_t head_dim, hipStream_t st, bool y_f16) {
  if (head_dim == 0) return hipErrorInvalidValue;
  return dispatch(args_of(in, w, false), EpRows{y, hstride, ldy, row0, head_dim, y_f16}, st);
}

hipError_t gemm_swiglu(const GemmIn& in, const GemmW& gate, const GemmW& up, float* mid, uint32_t ld,
                       hipStream_t st) {
  GemmArgs a = args_of(in, gate, true);
  a.w1 = up;
  return dispatch(a, EpSwiglu{mid, ld}, st);
}

hipError_t launch_prep_rows(const float* x, uint32_t rows, uint32_t ld, uint32_t cols, const float* norm_w,
                            float eps, const GemmIn& out, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  if (cols == 0 || cols % 32 || ld % 4 || ld < cols || !out.hi || !out.lo || !out.rexp || out.k != cols ||
      rows > out.m)
    return hipErrorInvalidValue;
  const uint32_t nct = (cols / 8 + 255) / 256;  // chunks of 8 per thread
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(rows), dim3(256), 0, st, x, ld, cols, norm_w, eps, (uint16_t*)out.hi,
                       (uint16_t*)out.lo, (uint16_t*)out.gsum, (int*)out.rexp);
  };
  if (nct <= 2) go(k_prep_rows_reg<2>);
  else if (nct <= 4) go(k_prep_rows_reg<4>);
  else if (nct <= 8) go(k_prep_rows_reg<8>);
  else if (nct <= 16) go(k_prep_rows_reg<16>);
  else go(k_prep_rows);
  return hipGetLastError();
}

}  // namespace ifx
