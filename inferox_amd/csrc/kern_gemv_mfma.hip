// kern_gemv_mfma.hip — int8-MFMA dequant-GEMV for Q4_K / Q6_K on gfx950.
//
// Replaces, for the K-quant matrices of a Q4_K_M model, the decode use of
// ops::matmul_t (src/ops.rs:33-44,104-134) fed by the f32 dequant of
// Weights::tensor_f32_by_index (src/gguf/weights.rs:66-74): y = W x with W
// streamed once in its quantized form.
//
// Arithmetic.  The K-quant element is w = a * q - m (Q4_K: a = d * sc,
// m = dmin * mn, q in 0..15, per 32-element sub-block; Q6_K: a = d * sc,
// m = 32 a, q in 0..63, per 16-element part), so a row's dot with x is
// sum over groups of a * (q . x) - m * sum(x).  The integer dot q . x runs on
// v_mfma_i32_16x16x64_i8 with x in fixed point: each 32-element group of x is
// scaled by 2^(22 - E) (E: the exponent of its largest magnitude), rounded to
// an integer X with |X| <= 2^22, and split into three signed base-256 digits
// (X = d0 + 256 d1 + 65536 d2).  The digit sums are exact in int32 and are
// recombined in f32, so q . x carries one rounding of the 22-bit x and one of
// the f32 recombination: within a few ulp of an f32 dot product.  sum(x) is
// taken in f32 from the unrounded x.
//
// MFMA mapping (16x16x64, A-lane i + 16g byte b meets B-lane j + 16g byte b;
// result C[i][j] in lane j + 16 (i / 4), register i % 4):
//   * B = weights.  Tiles are 16 rows; B-lane n + 16g holds 16 quants of row n
//     from group g's part (tiled device layout, ifx_common.h), unpacked from
//     nibbles (and Q6_K high bits) into bytes in the order
//     0 2 4 6 1 3 5 7 8 10 12 14 9 11 13 15 that two mask/shift steps give.
//   * A = x digits, staged in LDS by the workgroup prologue in the same order.
//     A-row 4g + d (d < 3) holds digit d of the x part that B-group g uses and
//     zero elsewhere, so lane n + 16g of C receives, in registers 0..2, the
//     three digit sums of row n over its own part: the epilogue needs no
//     cross-lane traffic until the row reduction.
//   * Per 256-element block a lane runs 4 MFMAs (Q4_K: two accumulate per
//     sub-block), so the decode costs about one VALU instruction per weight
//     per lane instead of four for the f32 dot.
//
// Work decomposition: persistent workgroups of 8 waves (1 or 2 per CU).  An item is
// one 16-row tile (two for paired gate/up launches, sharing the A reads); its
// blocks are split over `split` waves and reduced through LDS.  Each wave
// keeps the loads of D blocks in flight in a ring: block i is computed, then
// its registers are refilled with the loads of block i + D (which may belong
// to the next item), so HBM stays busy through reductions and epilogues.
// Compiled with -ffp-contract=off: only the explicit fmaf below are fused.
#include <algorithm>
#include <type_traits>

#include "gemv_epi.h"

namespace ifx {

bool mfma_type(uint32_t t) { return t == T_Q4K || t == T_Q6K; }

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
// Up to two workgroups per CU (at most 128 VGPRs).  Launches use one per CU
// except the mixed-type QKV launch: with 16 waves per CU the loads in flight
// (~55 MB GPU-wide for the output matrix) exceed what HBM serves efficiently
// (8 waves stream the 431 MB output matrix in 86 us instead of 95 us), while
// the QKV launch, two short segments per wave, gains from the second one.
constexpr int kMaxBlocksPerCu = 2;
constexpr int kWavesPerSimd = kMaxBlocksPerCu * kWaves / 4;  // 4
constexpr uint32_t kPartBytes = 48;   // 3 digit planes x 16 bytes per 16-element part
constexpr uint32_t kBlockA = 16 * kPartBytes;  // A bytes of one 256-element block
constexpr uint32_t kZeroBytes = 512;  // read by the lanes that feed zero A rows
constexpr uint32_t kM4 = 0x0F0F0F0Fu, kM2 = 0x30303030u;
// dynamic LDS limit: the CU's 160 KiB less the kernel's static arrays (< 4 KiB)
constexpr size_t kMaxDynLds = 156 * 1024;

struct MArgs {
  GemvSeg seg[3];      // paired: seg[0] gate, seg[1] up
  uint32_t ntiles[3];  // 16-row tiles per logical segment
  // Items per segment: items below half0 are whole tiles; item half0 + 2i + h
  // is half h (8 rows) of tile half0 + i, up to nitems (= ntiles: no halves)
  uint32_t half0[3], nitems[3];
  uint32_t rot[3];     // first-group rotation per segment (balances small segments)
  uint32_t use_b;      // bit s: segment s has the kernel's second type
  uint32_t split;      // waves per item: 1, 2, 4 or 8
  uint32_t steps;      // blocks per wave per item, padded to a multiple of D
  int nseg;
  uint32_t cols, nbr;  // nbr = cols / 256
  const float* x;
  const float* norm_w;
  float eps;
  uint32_t xs_off, zero_off;  // LDS byte offsets (the digit planes start at 0)
};

// ---- lane exchanges without LDS round trips (whole wave active) ----
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_xor1(float v) { return dpp_mov<0xb1>(v); }  // quad_perm [1,0,3,2]
__device__ __forceinline__ float lane_xor2(float v) { return dpp_mov<0x4e>(v); }  // quad_perm [2,3,0,1]
// One butterfly step: v op (v of lane ^ OFF) in every lane.  OFF 32 / 16: the
// gfx950 swaps of the two halves / of rows 0<->1, 2<->3 return {own, partner}
// in some order (the pair's op either way); 8: row_ror:8; 4: row_half_mirror
// then quad_perm [3,2,1,0]; 2, 1: quad_perm.  The operands are those of a
// __shfl_xor butterfly, so sums come out bit for bit the same.
template <int OFF, bool MAX>
__device__ __forceinline__ float bfly(float v) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "lane offset");
  float a = v, b;
  if constexpr (OFF == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else if constexpr (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else if constexpr (OFF == 8) {
    b = dpp_mov<0x128>(v);
  } else if constexpr (OFF == 4) {
    b = dpp_mov<0x1b>(dpp_mov<0x141>(v));
  } else if constexpr (OFF == 2) {
    b = lane_xor2(v);
  } else {
    b = lane_xor1(v);
  }
  return MAX ? fmaxf(a, b) : a + b;
}
// sum / max over the 64 lanes, in every lane (the xor butterfly 32, 16, ..., 1)
template <bool MAX>
__device__ __forceinline__ float wave_reduce(float v) {
  v = bfly<32, MAX>(v);
  v = bfly<16, MAX>(v);
  v = bfly<8, MAX>(v);
  v = bfly<4, MAX>(v);
  v = bfly<2, MAX>(v);
  return bfly<1, MAX>(v);
}
__device__ __forceinline__ float wave_sum(float v) { return wave_reduce<false>(v); }

__device__ __forceinline__ v4i mfma(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// q . X from the three digit sums: c0 + 256 c1 is exact in int32 (|c| < 2^17
// per digit) and rounds once on conversion, as the fma it replaces did
__device__ __forceinline__ float digits(v4i c) {
  return fmaf(65536.f, (float)c[2], (float)(c[0] + c[1] * 256));
}

// 16 Q4_K nibbles (8 bytes) -> 16 bytes in the A/B element order
__device__ __forceinline__ v4i nib(uint32_t w0, uint32_t w1) {
  return v4i{(int)(w0 & kM4), (int)((w0 >> 4) & kM4), (int)(w1 & kM4), (int)((w1 >> 4) & kM4)};
}

// 16 Q6_K quants: low nibbles (8 bytes) and the part's word of high parts
__device__ __forceinline__ v4i six(uint32_t l0, uint32_t l1, uint32_t h) {
  return v4i{(int)((l0 & kM4) | ((h << 4) & kM2)), (int)(((l0 >> 4) & kM4) | ((h << 2) & kM2)),
             (int)((l1 & kM4) | (h & kM2)), (int)(((l1 >> 4) & kM4) | ((h >> 2) & kM2))};
}

__device__ __forceinline__ float cvtb(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xffu); }

// One (tile, block) unit of a segment in registers.  dot() returns this lane's
// share of row (lane & 15)'s dot product over the block: sub-blocks g and
// g + 4 (g = lane >> 4).  xa / xb: {scale, sum32, -32 sum16 (part 0),
// -32 sum16 (part 1)} of x over those sub-blocks.
template <int T>
struct KBuf;

// Weight loads: nontemporal (NTL; the weights are read once per token) or
// plain.  Over the block-major layout the GPU streams one region at a time
// and nontemporal loads beat plain ones (gate/up 15.3 -> 14.8 us, the output
// matrix 83.6 -> 80.4 us); the q/k/v launch runs faster on plain loads
// (8.6 against 9.3 us).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <bool NTL>
__device__ __forceinline__ uint4 ld16(const uint8_t* p) {
  if (!NTL) return *(const uint4*)p;
  const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
template <bool NTL>
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) {
  if (!NTL) return *(const uint32_t*)p;
  return __builtin_nontemporal_load((const uint32_t*)p);
}

// Q4_K (src/gguf/dequant.rs:133-161): scales/mins of sub-blocks s < 4 are the
// low 6 bits of bytes s / s + 4; of s >= 4, the nibbles of byte s + 4 with the
// top bits of bytes s - 4 / s (dequant.rs:141-149).
template <>
struct KBuf<T_Q4K> {
  uint4 h, q0, q1;
  // u: wave-uniform unit base; 32-bit unsigned lane offsets keep the
  // scalar-base addressing form (no 64-bit address per lane)
  template <bool NTL = true>
  __device__ __forceinline__ void load(const uint8_t* u, uint32_t lane, uint32_t) {
    h = ld16<NTL>(u + 16u * (lane & 15u));
    q0 = ld16<NTL>(u + (256u + 16u * lane));
    q1 = ld16<NTL>(u + (1280u + 16u * lane));
  }
  __device__ __forceinline__ float dot(const v4i* A, float4 xa, float4 xb, int g) const {
    const v4i z = {0, 0, 0, 0};
    v4i ca = mfma(A[0], nib(q0.x, q0.y), z);
    ca = mfma(A[1], nib(q0.z, q0.w), ca);
    v4i cb = mfma(A[2], nib(q1.x, q1.y), z);
    cb = mfma(A[3], nib(q1.z, q1.w), cb);
    const uint32_t sh = 8 * g, y = h.y >> sh, zz = h.z >> sh, w = h.w >> sh;
    const uint32_t sca = y & 63u, mna = zz & 63u;
    const uint32_t scb = (w & 15u) | ((y >> 2) & 48u), mnb = ((w >> 4) & 15u) | ((zz >> 2) & 48u);
    const float d = h2f(h.x), dmin = h2f(h.x >> 16);
    float v = ((d * (float)sca) * xa.x) * digits(ca);
    v = fmaf(-(dmin * (float)mna), xa.y, v);
    v = fmaf((d * (float)scb) * xb.x, digits(cb), v);
    return fmaf(-(dmin * (float)mnb), xb.y, v);
  }
};

// Q6_K (reference layout, src/gguf/dequant.rs:165-199): w = (d * sc) * (q - 32),
// sc u8, or int8 for a tensor read in ggml's layout (sgn).
template <>
struct KBuf<T_Q6K> {
  uint4 l0, l1, hq;
  uint32_t sc, d, xm;
  float off;  // int8 scales: each byte's top bit flipped (xm) and 128 taken off at use
  template <bool NTL = true>
  __device__ __forceinline__ void load(const uint8_t* u, uint32_t lane, uint32_t q6_signed) {
    xm = q6_signed ? 0x80808080u : 0u;
    off = q6_signed ? 128.f : 0.f;
    l0 = ld16<NTL>(u + 16u * lane);
    l1 = ld16<NTL>(u + (1024u + 16u * lane));
    hq = ld16<NTL>(u + (2048u + 16u * lane));
    sc = ld4<NTL>(u + (3072u + 4u * lane));
    // the dword holding rows 2k, 2k+1's d: a 16-bit load would be
    // zero-extended where the ring slot is carried, waiting for the slot
    d = ld4<NTL>(u + (3328u + 4u * ((lane & 15u) >> 1)));
  }
  __device__ __forceinline__ float dot(const v4i* A, float4 xa, float4 xb, int) const {
    const v4i z = {0, 0, 0, 0};
    const float df = h2f(d >> (16u * (__lane_id() & 1u)));
    const v4i c0 = mfma(A[0], six(l0.x, l0.y, hq.x), z);
    const v4i c1 = mfma(A[1], six(l0.z, l0.w, hq.y), z);
    const v4i c2 = mfma(A[2], six(l1.x, l1.y, hq.z), z);
    const v4i c3 = mfma(A[3], six(l1.z, l1.w, hq.w), z);
    const uint32_t s4 = sc ^ xm;
    float v = (df * (cvtb(s4, 0) - off)) * fmaf(xa.x, digits(c0), xa.z);
    v = fmaf(df * (cvtb(s4, 1) - off), fmaf(xa.x, digits(c1), xa.w), v);
    v = fmaf(df * (cvtb(s4, 2) - off), fmaf(xb.x, digits(c2), xb.z), v);
    return fmaf(df * (cvtb(s4, 3) - off), fmaf(xb.x, digits(c3), xb.w), v);
  }
};

template <int T>
__device__ __forceinline__ const uint8_t* unit_ptr(const GemvSeg& sg, uint32_t nbr, uint32_t tile, uint32_t b) {
  (void)nbr;
  return sg.body + (uint64_t)tile * sg.tstride + (uint64_t)b * sg.bstride;
}

// ---------------------------------------------------------------------------
// Prologue: x (optionally RMS-normalised) -> digit planes + group sums in LDS.
// ---------------------------------------------------------------------------

// Chunk c = 8 consecutive elements (half of part c / 2); the 4 threads of a
// 32-element group are consecutive lanes.  Every lane takes part in the
// shuffles; only `ok` lanes write.
__device__ __forceinline__ void quantize_chunk(const float* v, uint32_t c, bool ok, uint8_t* lds, float4* xsum) {
  float m = 0.f;
#pragma unroll
  for (int k = 0; k < 8; k++) m = fmaxf(m, fabsf(v[k]));
  m = bfly<1, true>(m);
  m = bfly<2, true>(m);
  int e;
  (void)frexpf(m, &e);  // m < 2^e
  e = e < -100 ? -100 : e;
  const float inv = ldexpf(1.f, 22 - e), xs = ldexpf(1.f, e - 22);
  uint32_t p0[2] = {0u, 0u}, p1[2] = {0u, 0u}, p2[2] = {0u, 0u};
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int X = (int)rintf(v[k] * inv);  // |X| <= 2^22
    const int X1 = (X + 128) >> 8, X2 = (X1 + 128) >> 8;
    const int sh = 8 * (k >> 1), w = k & 1;  // even elements: word 0, odd: word 1
    p0[w] |= (uint32_t)(X & 255) << sh;
    p1[w] |= (uint32_t)(X1 & 255) << sh;
    p2[w] |= (uint32_t)(X2 & 255) << sh;
  }
  const float s8 = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  const float s16 = bfly<1, false>(s8);
  const float s16o = lane_xor2(s16);
  if (ok) {
    uint8_t* dst = lds + (c >> 1) * kPartBytes + 8 * (c & 1);
    *(uint2*)dst = make_uint2(p0[0], p0[1]);
    *(uint2*)(dst + 16) = make_uint2(p1[0], p1[1]);
    *(uint2*)(dst + 32) = make_uint2(p2[0], p2[1]);
    if ((c & 3) == 0) xsum[c >> 2] = make_float4(xs, s16 + s16o, -32.f * s16, -32.f * s16o);
  }
}

// The prologue in two halves, so that a workgroup issues its x (and norm
// weight) loads before the weight prefetch: loads return in issue order, and
// staging must not wait for the prefetched weights.
// KB: chunks of 8 elements per thread per batch (the launch takes 1 up to
// 4096 columns: with more, the clamped surplus loads queued ahead of the
// weight ring and delayed its issue)
template <bool NORM, int KB>
struct XStage {
  static constexpr int kB = KB;
  float4 xv[kB][2], wv[kB][2];

  __device__ __forceinline__ void load(const MArgs& a, uint32_t base, int tid) {
    const uint32_t nch = a.cols / 8;
    const float4* x4 = (const float4*)a.x;
    const float4* w4 = (const float4*)a.norm_w;
#pragma unroll
    for (int i = 0; i < kB; i++) {
      const uint32_t c = min(base + tid + i * kThreads, nch - 1);  // clamped: loads stay unconditional
      xv[i][0] = x4[2 * c];
      xv[i][1] = x4[2 * c + 1];
      if (NORM) {
        wv[i][0] = w4[2 * c];
        wv[i][1] = w4[2 * c + 1];
      }
    }
  }

  __device__ __forceinline__ void quantize(const MArgs& a, uint32_t base, float scale, uint8_t* lds, int tid) {
    const uint32_t nch = a.cols / 8;
    float4* xsum = (float4*)(lds + a.xs_off);
#pragma unroll
    for (int i = 0; i < kB; i++) {
      const uint32_t c = base + tid + i * kThreads;
      float v[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w, xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
      if (NORM) {
        const float w[8] = {wv[i][0].x, wv[i][0].y, wv[i][0].z, wv[i][0].w,
                            wv[i][1].x, wv[i][1].y, wv[i][1].z, wv[i][1].w};
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = (v[k] * scale) * w[k];
      }
      quantize_chunk(v, c, c < nch, lds, xsum);
    }
  }

  // after load(a, 0, tid): digit planes and group sums of all of x (with the
  // norm: of x * w), and the norm scale, returned (1 without the norm).
  // rms_norm's scale (src/ops.rs:162-167) is one scalar per vector, so the
  // kernel applies it to each row's dot product instead of to x: the
  // quantization does not wait for the workgroup reduction of x . x.
  __device__ __forceinline__ float finish(const MArgs& a, uint8_t* lds, float* red, int tid, int lane, int wave) {
    const uint32_t nch = a.cols / 8, step = kB * kThreads;
    if (NORM) {
      float ss = 0.f;
      if (nch <= step) {  // x is in registers
#pragma unroll
        for (int i = 0; i < kB; i++) {
          if (tid + i * kThreads < nch) {
#pragma unroll
            for (int hlf = 0; hlf < 2; hlf++) {
              const float4 u = xv[i][hlf];
              ss = fmaf(u.x, u.x, ss); ss = fmaf(u.y, u.y, ss); ss = fmaf(u.z, u.z, ss); ss = fmaf(u.w, u.w, ss);
            }
          }
        }
      } else {
        const float4* x4 = (const float4*)a.x;
        for (uint32_t c = tid; c < nch; c += kThreads) {
          const float4 u = x4[2 * c], v = x4[2 * c + 1];
          ss = fmaf(u.x, u.x, ss); ss = fmaf(u.y, u.y, ss); ss = fmaf(u.z, u.z, ss); ss = fmaf(u.w, u.w, ss);
          ss = fmaf(v.x, v.x, ss); ss = fmaf(v.y, v.y, ss); ss = fmaf(v.z, v.z, ss); ss = fmaf(v.w, v.w, ss);
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) red[wave] = ss;
    }
    quantize(a, 0, 1.f, lds, tid);
    for (uint32_t base = step; base < nch; base += step) {
      load(a, base, tid);
      quantize(a, base, 1.f, lds, tid);
    }
    if (tid < (int)(kZeroBytes / 16)) *(uint4*)(lds + a.zero_off + 16 * tid) = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    if (!NORM) return 1.f;
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) tot += red[w];
    return 1.0f / sqrtf(tot / (float)a.cols + a.eps);
  }
};

// ---------------------------------------------------------------------------
// Main loop
// ---------------------------------------------------------------------------

// nontemporal weight loads (ld16), except in the q/k/v launch
template <class Epi>
struct NtLoads {
  static constexpr bool value = true;
};
template <>
struct NtLoads<EpiQkv> {
  static constexpr bool value = false;
};

// Item v of segment s: its tile, and hl = 0 (the whole tile) or 1 + h (rows
// 8h..8h+7 of it).  A half item runs the whole tile's code with lane n + 16g
// reading row 8h + (n & 7): lanes n and n + 8 load the same bytes and compute
// the same sum, lanes 0..7 emit it.  Half items split the last round of a
// launch whose items do not fill it, so that every workgroup streams in it.
struct Item {
  uint32_t tile, hl;
  __device__ __forceinline__ Item(const MArgs& a, int s, uint32_t v) {
    const uint32_t h0 = a.half0[s];
    tile = v < h0 ? v : h0 + ((v - h0) >> 1);
    hl = v < h0 ? 0u : 1u + ((v - h0) & 1u);
  }
  // the lane index the unit loads use
  __device__ __forceinline__ uint32_t lane_of(uint32_t lane) const {
    return hl ? (lane & 0x37u) + 8u * (hl - 1u) : lane;
  }
  // the row lane (< 16) emits, and whether it emits
  __device__ __forceinline__ uint32_t row(uint32_t lane) const {
    return tile * (uint32_t)kTileRows + lane_of(lane & 15u);
  }
  __device__ __forceinline__ bool emits(uint32_t lane) const { return lane < (hl ? 8u : 16u); }
};

template <class Epi, int NT>
__device__ __forceinline__ void emit(const Epi& epi, typename Epi::Wave& ws, const MArgs& a, int s, const Item& it,
                                     const float* acc, const typename Epi::Pre& pre, int lane) {
  const float v = acc[0];
  float partner = 0.f;
  if (Epi::kPaired) partner = acc[NT - 1];
  else if (Epi::kNeighbor) partner = lane_xor1(v);
  const uint32_t r = it.row((uint32_t)lane);
  if (it.emits((uint32_t)lane) && r < a.seg[s].rows) epi.row(ws, Epi::kPaired ? 0 : s, r, v, partner, pre);
}

// The items of segment s owned by this wave's group (a.split waves of one
// workgroup): tiles first, first + TG, ..., `iters` of them (the same count for
// every wave of the workgroup, so that split reductions can use workgroup
// barriers).  Wave j of the group takes blocks j, j + split, ... of each item.
// `buf` arrives holding the loads of the wave's first D blocks.
template <int T, int NT, int D, class Epi>
__device__ __forceinline__ void run_seg(const MArgs& a, const Epi& epi, typename Epi::Wave& ws, int s,
                                        KBuf<T> (&buf)[D][NT], uint32_t first, uint32_t TG, uint32_t iters,
                                        uint32_t j, const uint8_t* lds, uint32_t a_base, uint32_t a_step,
                                        float* part, float nscale, int lane, int wave) {
  const uint32_t S = a.split, NB = a.steps, nbr = a.nbr, nt = a.nitems[s];
  const int g = lane >> 4;
  const float4* xsum = (const float4*)(lds + a.xs_off) + g;
  for (uint32_t k = 0; k < iters; k++) {
    const uint32_t item = first + k * TG;
    const bool live = item < nt;  // uniform over the wave
    const Item it(a, s, item);
    // the epilogue's global reads, in flight while the item is decoded
    typename Epi::Pre pre{};
    {
      const uint32_t r = it.row((uint32_t)lane);
      if (live && it.emits((uint32_t)lane) && r < a.seg[s].rows) pre = epi.pre(ws, Epi::kPaired ? 0 : s, r);
    }
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.f;
    for (uint32_t r = 0; r < NB; r += D) {
#pragma unroll
      for (int i = 0; i < D; i++) {
        const uint32_t m = r + i, b = j + S * m;
        const bool valid = live && b < nbr;
        const uint32_t bc = min(b, nbr - 1);
        const uint8_t* ap = lds + a_base + a_step * bc;
        const v4i A[4] = {*(const v4i*)ap, *(const v4i*)(ap + kPartBytes), *(const v4i*)(ap + 8 * kPartBytes),
                          *(const v4i*)(ap + 9 * kPartBytes)};
        const float4 xa = xsum[8 * bc], xb = xsum[8 * bc + 4];
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const float v = buf[i][t].dot(A, xa, xb, g);
          acc[t] += valid ? v : 0.f;
        }
        // refill with block m + D of this item, or block i of the next one.
        // Past the wave's last item the (unused) refill reads the segment's
        // first unit, which every such refill on the XCD shares: an L2 hit,
        // so the wave does not wait an HBM round trip for it before it ends.
        uint32_t nm = m + D, nit = item;
        if (nm >= NB) {
          nm -= NB;
          nit += TG;
        }
        const bool past = nit >= nt;
        const uint32_t nb = past ? 0u : min(j + S * nm, nbr - 1);
        const Item nx(a, s, past ? 0u : nit);
#pragma unroll
        for (int t = 0; t < NT; t++)
          buf[i][t].template load<NtLoads<Epi>::value>(unit_ptr<T>(a.seg[NT == 2 ? t : s], nbr, nx.tile, nb),
                                                       nx.lane_of((uint32_t)lane), a.seg[NT == 2 ? t : s].q6_signed);
        // keep the ring order: the next block's decode may not be hoisted above
        // these loads (it would wait for every buffer at once)
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      acc[t] = bfly<16, false>(acc[t]);
      acc[t] = bfly<32, false>(acc[t]);
    }
    if (S > 1) {
      // partial sums of the group's waves through LDS (double-buffered: one barrier per item)
      float* pb = part + (k & 1) * (kWaves * 16 * NT);
      if (lane < 16) {
#pragma unroll
        for (int t = 0; t < NT; t++) pb[(wave * NT + t) * 16 + lane] = acc[t];
      }
      __syncthreads();
      if (j == 0 && live) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
          float v = 0.f;
          for (uint32_t q = 0; q < S; q++) v += pb[((wave + q) * NT + t) * 16 + (lane & 15)];
          acc[t] = v * nscale;
        }
        emit<Epi, NT>(epi, ws, a, s, it, acc, pre, lane);
      }
    } else if (live) {
#pragma unroll
      for (int t = 0; t < NT; t++) acc[t] *= nscale;
      emit<Epi, NT>(epi, ws, a, s, it, acc, pre, lane);
    }
  }
}

// Loads of the wave's blocks i0..i1-1 (ring slots) of the first item.
template <int T, int NT, int D, bool NTL>
__device__ __forceinline__ void prefetch(const MArgs& a, int s, KBuf<T> (&buf)[D][NT], uint32_t first, uint32_t j,
                                         int lane, int i0 = 0, int i1 = D) {
  const Item it(a, s, min(first, a.nitems[s] - 1));
#pragma unroll
  for (int i = 0; i < D; i++) {
    if (i < i0 || i >= i1) continue;
    const uint32_t b = min(j + a.split * i, a.nbr - 1);
#pragma unroll
    for (int t = 0; t < NT; t++)
      buf[i][t].template load<NTL>(unit_ptr<T>(a.seg[NT == 2 ? t : s], a.nbr, it.tile, b), it.lane_of((uint32_t)lane),
                                   a.seg[NT == 2 ? t : s].q6_signed);
    // issue the slots in ring order: the loop's waits assume slot i is older
    // than slot i + 1 on every path into it (reordered prefetches made each
    // step wait for the whole ring)
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Segment s0 (the workgroup's first segment with work): x loads, the loads of
// the wave's first D blocks (issued after x, so x is not queued behind them),
// staging, then the segment.  With the whole ring in flight during staging the
// 9.4 MB attn_output launch takes 5.4 us instead of 5.8 us.
template <bool NORM, int KB, int T, int NT, int D, class Epi>
__device__ __forceinline__ float lead(const MArgs& a, const Epi& epi, typename Epi::Wave& ws, int s0, uint32_t first,
                                     uint32_t TG, uint32_t iters, uint32_t j, uint8_t* lds, float* red,
                                     uint32_t a_base, uint32_t a_step, float* part, int tid, int lane, int wave) {
  XStage<NORM, KB> xs;
  xs.load(a, 0, tid);
  // every wave's x loads enter the CU's memory queues before any weight load
  // (a bare barrier: nothing waits for the loads here)
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  KBuf<T> buf[D][NT];
  prefetch<T, NT, D, NtLoads<Epi>::value>(a, s0, buf, first, j, lane, 0, D);
  const float nscale = xs.finish(a, lds, red, tid, lane, wave);
  run_seg<T, NT, D, Epi>(a, epi, ws, s0, buf, first, TG, iters, j, lds, a_base, a_step, part, nscale, lane, wave);
  return nscale;
}

template <class Epi, int TA, int TB, int D, bool NORM, int KB>
__global__ void __launch_bounds__(kThreads, kWavesPerSimd) k_gemv_mfma(MArgs a, Epi epi) {
  constexpr int NT = Epi::kPaired ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ float red[kWaves];
  __shared__ float part[2 * kWaves * 16 * NT];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t S = a.split, GPB = kWaves / S, TG = gridDim.x * GPB;
  const uint32_t tg = blockIdx.x * GPB + wave / S, j = wave % S;
  // A operand: lane i + 16g feeds row i of the 16x64 A tile within k-range g;
  // rows 4g..4g+2 carry the digits of group g's part, the rest read zeros
  const int ai = lane & 15, ag = lane >> 4;
  const bool active = (ai >> 2) == ag && (ai & 3) < 3;
  const uint32_t a_base = active ? (uint32_t)(2 * kPartBytes * ag + 16 * (ai & 3)) : a.zero_off;
  const uint32_t a_step = active ? kBlockA : 0u;
  typename Epi::Wave ws;
  epi.begin(ws);
  // items per group of this workgroup for segment s: the count of its busiest group
  auto block_iters = [&](int s) -> uint32_t {
    uint32_t n = 0;
    for (uint32_t q = 0; q < GPB; q++) {
      const uint32_t f0 = (blockIdx.x * GPB + q + TG - a.rot[s]) % TG;
      if (f0 < a.nitems[s]) n = max(n, (a.nitems[s] - 1 - f0) / TG + 1);
    }
    return n;
  };
  int s0 = 0;  // uniform over the workgroup
  while (s0 < a.nseg && block_iters(s0) == 0) s0++;
  float nscale = 1.f;
  if (s0 < a.nseg) {
    const uint32_t first = (tg + TG - a.rot[s0]) % TG, iters = block_iters(s0);
    if (TA != TB && ((a.use_b >> s0) & 1u))
      nscale = lead<NORM, KB, TB, NT, D>(a, epi, ws, s0, first, TG, iters, j, lds, red, a_base, a_step, part, tid, lane, wave);
    else
      nscale = lead<NORM, KB, TA, NT, D>(a, epi, ws, s0, first, TG, iters, j, lds, red, a_base, a_step, part, tid, lane, wave);
  }
  // paired launches have one logical segment: no later segments to run
  for (int s = s0 + 1; !Epi::kPaired && s < a.nseg; s++) {
    const uint32_t first = (tg + TG - a.rot[s]) % TG;
    const uint32_t iters = block_iters(s);
    if (iters == 0) continue;
    if (TA != TB && ((a.use_b >> s) & 1u)) {
      KBuf<TB> buf[D][NT];
      prefetch<TB, NT, D, NtLoads<Epi>::value>(a, s, buf, first, j, lane);
      run_seg<TB, NT, D, Epi>(a, epi, ws, s, buf, first, TG, iters, j, lds, a_base, a_step, part, nscale, lane, wave);
    } else {
      KBuf<TA> buf[D][NT];
      prefetch<TA, NT, D, NtLoads<Epi>::value>(a, s, buf, first, j, lane);
      run_seg<TA, NT, D, Epi>(a, epi, ws, s, buf, first, TG, iters, j, lds, a_base, a_step, part, nscale, lane, wave);
    }
  }
  epi.finish(ws, lane);
}

// ---------------------------------------------------------------------------
// K-split residual GEMV: h += W x for the O and down projections.  The
// kernel above gives each 16-row tile to the waves of one workgroup, so every
// workgroup stages all of x, the previous kernel's output; staging it (the
// loads queue behind the weight stream, then the quantization) is the longest
// part of those launches (~3.4 us of the O projection's ~5.5 at 4096
// columns).  Here K is cut into kKs slices: workgroup g takes slice g mod kKs
// and each of its waves one tile per pass, so a workgroup stages 1 / kKs of
// x (and workgroup g runs on XCD g mod 8, so each XCD's L2 serves one
// slice).  The kKs partial dot products of a row meet in h through float
// atomic adds at agent scope, which are coherent across the XCDs; their order,
// and so the last bits of h, may differ from run to run.
//
// With 8 kv heads the O projection's slices are the kv heads' query-head
// groups, so k_gemv_ks_merge can take the attention's chunk records in place
// of x: its prologue merges the records of kv head g mod 8 (what k_attn_merge
// does for every head) and quantizes the result as its slice of x.
// ---------------------------------------------------------------------------
constexpr uint32_t kKs = 8;
// one x chunk of 8 elements per thread: slices of up to 16 blocks (4096
// columns), K up to 32768.  (A loop of clamped loads would leave dead
// destinations the compiler waits on, and a conditional prefetch makes its
// waits assume the shorter path.)
constexpr uint32_t kKsMaxBlocks = kThreads * 8 / 256;
// Units in flight per wave.  Two: the ring is issued in well under a
// microsecond, so the prologue and the first units' arithmetic overlap the
// stream.  With all of a wave's units in flight (8 for the 8B down
// projection) issuing them stalled until the data drained (per-wave
// timestamps: loads issued at a median 5.2 us, the arithmetic of every unit
// after 7 us): 13.5 us per launch against 10.7 with 2, 11.6 with 4.
constexpr int kKsRing = 2;

struct KsArgs {
  GemvSeg seg;
  uint32_t ntiles, nbr, nbs;  // 16-row tiles, 256-column blocks, blocks per slice
  const float* x;
  float* h;
  uint32_t xs_off, zero_off;  // LDS byte offsets (the slice's digit planes start at 0)
  // k_gemv_ks_merge: the chunk records of the decode attention and the state
  // that gives the attended rows
  const float* partial;
  const DevState* state;
  uint32_t max_chunks, chunk;
  uint32_t first;  // the prologue loads chunks [0, first) (a bound the host keeps above the step's count)
};

// The wave's units: tiles t0, t0 + tstride, ... x the slice's nbs blocks.
struct KsWave {
  uint32_t t0, tstride, b0, W;
  __device__ __forceinline__ KsWave(uint32_t t0_, uint32_t tstride_, uint32_t b0_, uint32_t ntiles, uint32_t nbs)
      : t0(t0_), tstride(tstride_), b0(b0_), W(t0_ < ntiles ? ((ntiles - 1 - t0_) / tstride_ + 1) * nbs : 0u) {}
  __device__ __forceinline__ KsWave(const KsArgs& a, uint32_t wave) {
    b0 = (blockIdx.x % kKs) * a.nbs;
    t0 = (blockIdx.x / kKs) * kWaves + wave;
    tstride = (gridDim.x / kKs) * kWaves;
    W = t0 < a.ntiles ? ((a.ntiles - 1 - t0) / tstride + 1) * a.nbs : 0u;
  }
};

// Where a K-split wave's tiles live and where their row sums go.
// One segment, the sums added into h (the O and down projections).
template <int T>
struct KsToH {
  const KsArgs& a;
  __device__ __forceinline__ const uint8_t* unit(uint32_t tile, uint32_t b) const {
    return unit_ptr<T>(a.seg, a.nbr, tile, b);
  }
  __device__ __forceinline__ uint32_t q6(uint32_t) const { return a.seg.q6_signed; }
  struct Pre {};
  __device__ __forceinline__ Pre pre(uint32_t, int) const { return Pre{}; }
  __device__ __forceinline__ void emit(uint32_t tile, float r, int lane, Pre) const {
    const uint32_t row = tile * (uint32_t)kTileRows + (uint32_t)(lane & 15);
    if (lane < 16 && row < a.seg.rows) atomicAdd(a.h + row, r);
  }
};

// Ring: slot i holds unit u = i (mod D); unit u is block b0 + u mod nbs of
// tile t0 + (u / nbs) tstride.  Loads past the wave's last unit (and all of a
// wave without tiles) read the slice's first unit (tile 0): in bounds, unused,
// shared (an L2 hit), and unconditional, so that the compiler's waits count
// one path.
template <int T, int D, class M>
__device__ __forceinline__ void ks_prefetch(uint32_t nbs, const KsWave& w, const M& m, KBuf<T> (&buf)[D],
                                            int lane) {
#pragma unroll
  for (int i = 0; i < D; i++) {
    const bool past = (uint32_t)i >= w.W;
    const uint32_t u = past ? 0u : (uint32_t)i, tl = past ? 0u : w.t0 + (u / nbs) * w.tstride;
    buf[i].load(m.unit(tl, w.b0 + u % nbs), (uint32_t)lane, m.q6(tl));
    __builtin_amdgcn_sched_barrier(0);  // slots in ring order
  }
}

// The wave's units against the slice of x staged in LDS (digit planes at 0,
// group sums at xs_off); each finished tile's 16 row sums go to m.emit.
// LOCK: every wave of the workgroup runs Wu units (the workgroup's largest
// count; units past its own W are the ring's unused loads) and the waves meet
// at a barrier after each round of D units.
template <int T, int D, class M, bool LOCK = false>
__device__ __forceinline__ void ks_run(uint32_t nbs, uint32_t xs_off, uint32_t zero_off, const KsWave& w, const M& m,
                                       KBuf<T> (&buf)[D], const uint8_t* lds, int lane, uint32_t Wu = 0) {
  if ((LOCK ? Wu : w.W) == 0) return;
  const int ai = lane & 15, ag = lane >> 4;
  const bool active = (ai >> 2) == ag && (ai & 3) < 3;
  const uint32_t a_base = active ? (uint32_t)(2 * kPartBytes * ag + 16 * (ai & 3)) : zero_off;
  const uint32_t a_step = active ? kBlockA : 0u;
  const float4* xs4 = (const float4*)(lds + xs_off) + ag;
  const uint32_t Wp = ((LOCK ? Wu : w.W) + D - 1) / D * D;
  float acc = 0.f;
  uint32_t bl = 0, tile = w.t0;                                            // unit u: local block, tile
  uint32_t rb = (uint32_t)D % nbs, rt = w.t0 + ((uint32_t)D / nbs) * w.tstride;  // unit u + D
  typename M::Pre pre = m.pre(tile, lane);  // the epilogue's reads, in flight during the tile
  for (uint32_t u0 = 0; u0 < Wp; u0 += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      const uint32_t u = u0 + (uint32_t)i;
      const uint8_t* ap = lds + a_base + a_step * bl;
      const v4i A[4] = {*(const v4i*)ap, *(const v4i*)(ap + kPartBytes), *(const v4i*)(ap + 8 * kPartBytes),
                        *(const v4i*)(ap + 9 * kPartBytes)};
      const float4 xa = xs4[8 * bl], xb = xs4[8 * bl + 4];
      const float v = buf[i].dot(A, xa, xb, ag);
      acc += u < w.W ? v : 0.f;
      // past the wave's last unit: the slice's first unit, which every such
      // refill shares (an L2 hit; the wave's own first unit is gone from L2
      // under the stream)
      const bool past = u + D >= w.W;
      buf[i].load(m.unit(past ? 0u : rt, w.b0 + (past ? 0u : rb)), (uint32_t)lane, m.q6(past ? 0u : rt));
      // keep the ring order (see run_seg)
      __builtin_amdgcn_sched_barrier(0);
      if (++rb == nbs) {
        rb = 0;
        rt += w.tstride;
      }
      if (++bl == nbs) {  // the tile's slice is done (uniform over the wave)
        if (u < w.W) {
          float r = acc;
          r = bfly<16, false>(r);
          r = bfly<32, false>(r);
          m.emit(tile, r, lane, pre);
        }
        acc = 0.f;
        bl = 0;
        tile += w.tstride;
        pre = m.pre(tile, lane);
      }
    }
    if constexpr (LOCK) __builtin_amdgcn_s_barrier();
  }
}

__device__ __forceinline__ void ks_zero(const KsArgs& a, uint8_t* lds, int tid) {
  if (tid < (int)(kZeroBytes / 16)) *(uint4*)(lds + a.zero_off + 16 * tid) = make_uint4(0u, 0u, 0u, 0u);
}

// every wave's prologue loads enter the CU's memory queues before any weight load
__device__ __forceinline__ void loads_first() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

template <int T, int D, bool LOCK>
__global__ void __launch_bounds__(kThreads, 1) k_gemv_ks(KsArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const KsWave w(a, (uint32_t)__builtin_amdgcn_readfirstlane(tid >> 6));
  // the slice of x: elements [256 b0, 256 (b0 + nbs)), chunk tid of 8
  const uint32_t nch = a.nbs * 32, c = (uint32_t)tid;
  const float4* x4 = (const float4*)(a.x + (uint64_t)w.b0 * 256u) + 2 * min(c, nch - 1);  // clamped: unconditional
  const float4 xv0 = x4[0], xv1 = x4[1];
  loads_first();
  KBuf<T> buf[D];
  const KsToH<T> m{a};
  ks_prefetch<T, D>(a.nbs, w, m, buf, lane);
  {  // whole 32-element groups are in or out of the slice (nch % 32 == 0)
    float v[8] = {xv0.x, xv0.y, xv0.z, xv0.w, xv1.x, xv1.y, xv1.z, xv1.w};
    quantize_chunk(v, c, c < nch, lds, (float4*)(lds + a.xs_off));
  }
  ks_zero(a, lds, tid);
  __syncthreads();
  // wave 0 has the workgroup's first tile, so the most units
  ks_run<T, D, KsToH<T>, LOCK>(a.nbs, a.xs_off, a.zero_off, w, m, buf, lds, lane, KsWave(a, 0u).W);
}

// ---------------------------------------------------------------------------
// K-split q/k/v: the three projections of rms_norm(h) in one K-split launch
// (what k_gemv_mfma<EpiQkv> computes with whole rows per workgroup).  The
// tiled launch takes 384 workgroups for the 8B shape (384 tiles), two on half
// of the CUs, and those CUs take twice the units: per-wave timestamps showed
// the second workgroups ending at 8.3-9.2 us against 5.9-6.5 us.  Here every
// CU takes the same share.  Each workgroup stages its slice of x * w (w: the
// norm weight; the norm's scale, one scalar, is applied to the row sums as in
// the tiled launch), reading all of h for the sum of squares.
// RoPE rotates each (even, odd) pair of a q or k row, a linear map, so each
// slice rotates its own partial sums (the pair's partner row sits in the
// neighbouring lane) and adds them, as the O and down launches add into h,
// straight into q and into the f32 cache's new row (cache row state->len):
// the attention reads both as the tiled launch leaves them.  Those rows are
// cleared beforehand, every layer's at once by the step's embedding gather
// (QkvClear; each layer has its own q buffer).
// The waves of a slice are shared out over q, k and v in proportion to their
// tiles, and each wave runs tiles of one segment (one buffer type, and its
// segment's fields at fixed kernel-argument offsets: a segment looked up per
// unit went through scratch).  Wave slot (wave, workgroup r of the slice) =
// wave * R + r spreads the waves with two tiles and those with one over the
// workgroups.
// ---------------------------------------------------------------------------
struct KsQkvArgs {
  GemvSeg seg[3];      // q, k, v
  uint32_t ntiles[3];
  uint32_t nbr, nbs, cols;
  uint32_t wq, wk;     // waves per slice on q and on k tiles (v takes the rest)
  const float* x;      // h
  const float* norm_w;
  float eps;
  QkvDst dst;          // where q, k and v go
  uint32_t xs_off, zero_off;
};

// One segment's tiles (KIND 0: q, 1: k, 2: v); each row sum, times the norm
// scale, with RoPE for q and k (src/ops.rs:281-296, as EpiQkv applies it), is
// added into q or into its cache row.
template <int T, int KIND>
struct KsToQkv {
  const GemvSeg& seg;
  const QkvDst& d;
  float scale;
  uint32_t len, pos;  // cache row of the new key/value, RoPE position
  __device__ __forceinline__ const uint8_t* unit(uint32_t tile, uint32_t b) const {
    return unit_ptr<T>(seg, 0u, tile, b);
  }
  __device__ __forceinline__ uint32_t q6(uint32_t) const { return seg.q6_signed; }
  struct Pre {
    float2 cs;
  };
  // the (cos, sin) of the row's RoPE pair (clamped rows past the segment's end
  // read an in-bounds pair and are not stored)
  __device__ __forceinline__ Pre pre(uint32_t tile, int lane) const {
    Pre p{make_float2(1.f, 0.f)};
    if (KIND < 2 && d.rope_dim) {
      const uint32_t row = min(tile * (uint32_t)kTileRows + (uint32_t)(lane & 15), seg.rows - 1);
      const uint32_t i = min(row % d.head_dim, d.rope_dim - 1);
      p.cs = d.rope_cs[(uint64_t)pos * (d.rope_dim / 2) + i / 2];
    }
    return p;
  }
  __device__ __forceinline__ void emit(uint32_t tile, float r, int lane, const Pre& p) const {
    const uint32_t row = tile * (uint32_t)kTileRows + (uint32_t)(lane & 15);
    float v = r * scale;
    if (KIND < 2) {
      const float other = lane_xor1(v);
      const uint32_t i = row % d.head_dim;
      if (i < d.rope_dim) v = (i & 1) ? (other * p.cs.y + v * p.cs.x) : (v * p.cs.x - other * p.cs.y);
    }
    if (lane < 16 && row < seg.rows) {
      if (KIND == 0) {
        atomicAdd(d.q + row, v);
      } else {
        float* c = KIND == 1 ? d.k_cache : d.v_cache;
        atomicAdd(c + ((uint64_t)(row / d.head_dim) * d.max_seq + len) * d.head_dim + row % d.head_dim, v);
      }
    }
  }
};

// KX: chunks of 8 elements of h per thread for the sum of squares (1 up to
// 4096 columns, 2 up to 8192).
template <int TA, int TB, int D, int KX>
__global__ void __launch_bounds__(kThreads, 1) k_gemv_ks_qkv(KsQkvArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ float red[kWaves];
  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t sl = blockIdx.x % kKs, R = gridDim.x / kKs, slot = wave * R + blockIdx.x / kKs;
  const uint32_t b0 = sl * a.nbs, ws = R * kWaves;
  // the wave's segment (uniform) and its place among that segment's waves
  const uint32_t sg = slot < a.wq ? 0u : slot < a.wq + a.wk ? 1u : 2u;
  const uint32_t w0 = sg == 0 ? 0u : sg == 1 ? a.wq : a.wq + a.wk;
  const uint32_t nw = sg == 0 ? a.wq : sg == 1 ? a.wk : ws - a.wq - a.wk;
  const KsWave w(slot - w0, max(nw, 1u), b0, a.ntiles[sg], a.nbs);
  // all of h (the sum of squares), then the slice's chunk tid of h and of w
  const uint32_t nchx = a.cols / 8, nch = a.nbs * 32;
  const float4* x4 = (const float4*)a.x;
  const float4* w4 = (const float4*)a.norm_w;
  float4 hv[KX][2];
#pragma unroll
  for (int i = 0; i < KX; i++) {
    const uint32_t c = min((uint32_t)tid + kThreads * i, nchx - 1);  // clamped: unconditional
    hv[i][0] = x4[2 * c];
    hv[i][1] = x4[2 * c + 1];
  }
  const uint32_t cs = b0 * 32 + min((uint32_t)tid, nch - 1);
  const float4 xv0 = x4[2 * cs], xv1 = x4[2 * cs + 1], wv0 = w4[2 * cs], wv1 = w4[2 * cs + 1];
  loads_first();
  KBuf<TA> bufa[D];
  KBuf<TB> bufb[D];
  const uint32_t len = a.dst.state->len, pos = a.dst.state->rope_pos;
  if (sg == 0) ks_prefetch<TA, D>(a.nbs, w, KsToQkv<TA, 0>{a.seg[0], a.dst, 0.f, len, pos}, bufa, lane);
  else if (sg == 1) ks_prefetch<TA, D>(a.nbs, w, KsToQkv<TA, 1>{a.seg[1], a.dst, 0.f, len, pos}, bufa, lane);
  else ks_prefetch<TB, D>(a.nbs, w, KsToQkv<TB, 2>{a.seg[2], a.dst, 0.f, len, pos}, bufb, lane);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < KX; i++) {
    if ((uint32_t)tid + kThreads * i < nchx) {
#pragma unroll
      for (int hlf = 0; hlf < 2; hlf++) {
        const float4 u = hv[i][hlf];
        ss = fmaf(u.x, u.x, ss); ss = fmaf(u.y, u.y, ss); ss = fmaf(u.z, u.z, ss); ss = fmaf(u.w, u.w, ss);
      }
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  {  // whole 32-element groups are in or out of the slice (nch % 32 == 0)
    float v[8] = {xv0.x * wv0.x, xv0.y * wv0.y, xv0.z * wv0.z, xv0.w * wv0.w,
                  xv1.x * wv1.x, xv1.y * wv1.y, xv1.z * wv1.z, xv1.w * wv1.w};
    quantize_chunk(v, (uint32_t)tid, (uint32_t)tid < nch, lds, (float4*)(lds + a.xs_off));
  }
  if (tid < (int)(kZeroBytes / 16)) *(uint4*)(lds + a.zero_off + 16 * tid) = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int q = 0; q < kWaves; q++) tot += red[q];
  const float nscale = 1.0f / sqrtf(tot / (float)a.cols + a.eps);
  if (sg == 0)
    ks_run<TA, D>(a.nbs, a.xs_off, a.zero_off, w, KsToQkv<TA, 0>{a.seg[0], a.dst, nscale, len, pos}, bufa, lds, lane);
  else if (sg == 1)
    ks_run<TA, D>(a.nbs, a.xs_off, a.zero_off, w, KsToQkv<TA, 1>{a.seg[1], a.dst, nscale, len, pos}, bufa, lds, lane);
  else
    ks_run<TB, D>(a.nbs, a.xs_off, a.zero_off, w, KsToQkv<TB, 2>{a.seg[2], a.dst, nscale, len, pos}, bufb, lds, lane);
}

__device__ __forceinline__ float wave_max(float v) { return wave_reduce<true>(v); }
__device__ __forceinline__ float4 fma4(float w, float4 v, float4 acc) {
  acc.x = fmaf(w, v.x, acc.x);
  acc.y = fmaf(w, v.y, acc.y);
  acc.z = fmaf(w, v.z, acc.z);
  acc.w = fmaf(w, v.w, acc.w);
  return acc;
}

// The O projection fed by the attention's chunk records (head dim 128, G
// query heads per kv head; the slice of workgroup g is kv head g mod 8).
// Per query head h of the slice, over the chunk records c (k_attn_decode:
// unnormalised o_c, max m_c, sum l_c), as k_attn_merge forms them:
//   M = max_c m_c,  x_h = sum_c exp(m_c - M) o_c / sum_c exp(m_c - M) l_c
// (softmax over all attended rows, src/model/forward.rs:398-409).  Wave g < G
// reduces M and the denominator of head g; thread (split sp, float4 column)
// sums chunks sp, sp + NS, ...; the first kMergeFirst chunks' loads are
// issued with the prologue, later chunks (long contexts) are read in a loop.
constexpr uint32_t kMergeFirst = 48;
constexpr uint32_t kMergeBoundStep = 8;  // the host's bounds are multiples of this

// FB: the host's bound on the step's chunk count (a multiple of
// kMergeBoundStep up to kMergeFirst), the chunks whose records the prologue
// loads: each of those loads costs the CU's address path 1 KB per wave, hit
// or miss, so the launch loads no more of them than the bound.
template <int T, int D, int G, int FB>
__global__ void __launch_bounds__(kThreads, 1) k_gemv_ks_merge(KsArgs a) {
  constexpr int HD = 128, SD = G * HD, NC4 = SD / 4, NS = kThreads / NC4, KB = FB / NS;
  static_assert(kThreads % NC4 == 0 && SD / 8 <= kThreads && FB % NS == 0, "slice shape");
  static_assert(FB <= (int)kMergeFirst && kMergeFirst <= 64, "the first loads' weights come from one lane each");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ float4 red[kThreads];
  __shared__ __attribute__((aligned(16))) float xsl[SD];
  __shared__ float sm[G], sd[G];
  __shared__ float wts[G][64];  // exp(m_c - M) of head g for chunks c < 64 (weights of the first loads)
  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(tid >> 6);
  const KsWave w(a, wave);
  // attended rows (as k_attn_decode reads them) and their chunk records
  const uint32_t len = a.state->len, attn_lo = a.state->attn_lo, attn_end = a.state->attn_end;
  const uint32_t hi = attn_end ? attn_end : len + 1, nrows = hi > attn_lo ? hi - attn_lo : 0u;
  const uint32_t nch = min((nrows + a.chunk - 1) / a.chunk, a.max_chunks);
  const uint32_t rec = attn_partial_floats(G, HD);
  const float* base = a.partial + (uint64_t)(blockIdx.x % kKs) * a.max_chunks * rec;
  const float* ml = base + SD;  // chunk c: max at ml[c rec + g], sum at ml[c rec + G + g]
  const uint32_t sp = (uint32_t)tid / NC4, col = (uint32_t)tid % NC4, g = col / (HD / 4);
  // The first loads do not wait for the state: the max and sum of chunks
  // lane < 64 are clamped to the buffer, the records' o of chunks < fe (the
  // host's bound, a multiple of NS, or the buffer) to fe - 1 (repeats: cache
  // hits); what lies past nch (records of earlier steps, or never written)
  // is masked out by selects.
  const uint32_t fe = min(min(a.first, (uint32_t)FB), a.max_chunks), cl = fe - 1;
  // wave g < G: the max and sum of head g over chunks lane, lane + 64, ... (issued first)
  float m0 = -INFINITY, l0 = 0.f;
  if (wave < (uint32_t)G) {
    const uint64_t at = (uint64_t)min((uint32_t)lane, a.max_chunks - 1) * rec;
    m0 = ml[at + wave];
    l0 = ml[at + G + wave];
  }
  float4 ov[KB];
#pragma unroll
  for (int k = 0; k < KB; k++) {
    const uint64_t at = (uint64_t)min(sp + (uint32_t)(NS * k), cl) * rec;  // clamped: unconditional
    ov[k] = ((const float4*)(base + at))[col];
  }
  loads_first();
  KBuf<T> buf[D];
  const KsToH<T> m{a};
  ks_prefetch<T, D>(a.nbs, w, m, buf, lane);

  if (wave < (uint32_t)G) {
    float M = (uint32_t)lane < nch ? m0 : -INFINITY;
    for (uint32_t c = lane + 64; c < nch; c += 64) M = fmaxf(M, ml[(uint64_t)c * rec + wave]);
    M = wave_max(M);
    // each weight once, for every thread that sums chunk `lane` of head g
    const float w0 = (uint32_t)lane < nch ? expf(m0 - M) : 0.f;
    wts[wave][lane] = w0;
    float den = (uint32_t)lane < nch ? l0 * w0 : 0.f;
    for (uint32_t c = lane + 64; c < nch; c += 64)
      den = fmaf(ml[(uint64_t)c * rec + G + wave], expf(ml[(uint64_t)c * rec + wave] - M), den);
    den = wave_sum(den);
    if (lane == 0) {
      sm[wave] = M;
      sd[wave] = den;
    }
  }
  __syncthreads();
  const float M = sm[g];
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const uint32_t nb = min(nch, fe);
#pragma unroll
  for (int k = 0; k < KB; k++)
    if (sp + (uint32_t)(NS * k) < nb) acc = fma4(wts[g][sp + NS * k], ov[k], acc);
  for (uint32_t c = sp + fe; c < nch; c += NS) {
    const uint64_t at = (uint64_t)c * rec;
    acc = fma4(expf(ml[at + g] - M), ((const float4*)(base + at))[col], acc);
  }
  red[tid] = acc;
  __syncthreads();
  if ((uint32_t)tid < NC4) {
    float4 o = red[tid];
#pragma unroll
    for (int q = 1; q < NS; q++) {
      const float4 r = red[q * NC4 + tid];
      o = make_float4(o.x + r.x, o.y + r.y, o.z + r.z, o.w + r.w);
    }
    const float den = sd[g];
    *(float4*)&xsl[4 * tid] = nch > 0 ? make_float4(o.x / den, o.y / den, o.z / den, o.w / den)
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __syncthreads();
  if (wave < (uint32_t)(SD / 8 / 64)) {  // whole waves: chunk tid of 8 elements
    const float4 u = *(const float4*)&xsl[8 * tid], v4 = *(const float4*)&xsl[8 * tid + 4];
    float v[8] = {u.x, u.y, u.z, u.w, v4.x, v4.y, v4.z, v4.w};
    quantize_chunk(v, (uint32_t)tid, true, lds, (float4*)(lds + a.xs_off));
  }
  ks_zero(a, lds, tid);
  __syncthreads();
  ks_run<T, D>(a.nbs, a.xs_off, a.zero_off, w, m, buf, lds, lane);
}

int cu_count() {
  // initialised once, thread-safe (sessions may run on several threads)
  static const int n = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      return v;
    return 256;
  }();
  return n;
}

template <class Epi, int TA, int TB, int D, bool NORM, int KB>
hipError_t go_one(const MArgs& a, const Epi& epi, uint32_t blocks, size_t lds, hipStream_t st) {
  if (lds > 64 * 1024) {  // rows of more than ~18K columns (the 70B down projection: 28672)
    // the instance opts in once; a block-scope static is initialised the first
    // time a launch gets here, once even when sessions run on several threads
    static const hipError_t opted = hipFuncSetAttribute((const void*)k_gemv_mfma<Epi, TA, TB, D, NORM, KB>,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxDynLds);
    if (opted != hipSuccess) return opted;
  }
  hipLaunchKernelGGL((k_gemv_mfma<Epi, TA, TB, D, NORM, KB>), dim3(blocks), dim3(kThreads), lds, st, a, epi);
  return hipGetLastError();
}

template <class Epi, int TA, int TB, int D>
hipError_t go(const MArgs& a, const Epi& epi, uint32_t blocks, size_t lds, hipStream_t st) {
  const bool one = a.cols <= 8u * kThreads;  // one chunk of 8 per thread stages all of x
  if (a.norm_w) return one ? go_one<Epi, TA, TB, D, true, 1>(a, epi, blocks, lds, st)
                           : go_one<Epi, TA, TB, D, true, 2>(a, epi, blocks, lds, st);
  return one ? go_one<Epi, TA, TB, D, false, 1>(a, epi, blocks, lds, st)
             : go_one<Epi, TA, TB, D, false, 4>(a, epi, blocks, lds, st);
}

template <class Epi, int D>
hipError_t go_types(const MArgs& a, uint32_t ta, uint32_t tb, const Epi& epi, uint32_t blocks, size_t lds,
                    hipStream_t st) {
  if (ta == T_Q4K && tb == T_Q4K) return go<Epi, T_Q4K, T_Q4K, D>(a, epi, blocks, lds, st);
  if (ta == T_Q6K && tb == T_Q6K) return go<Epi, T_Q6K, T_Q6K, D>(a, epi, blocks, lds, st);
  // mixed launches (a Q4_K_M layer's QKV: Q4_K q/k, Q6_K v) run the 2-deep
  // ring: two buffer types in one kernel leave no registers for a deeper one
  if constexpr (!Epi::kPaired && D == 2) {
    if (ta == T_Q4K && tb == T_Q6K) return go<Epi, T_Q4K, T_Q6K, D>(a, epi, blocks, lds, st);
    if (ta == T_Q6K && tb == T_Q4K) return go<Epi, T_Q6K, T_Q4K, D>(a, epi, blocks, lds, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace

template <class Epi>
hipError_t launch_mfma(const GemvLaunch& L, const Epi& epi, hipStream_t st) {
  constexpr int NT = Epi::kPaired ? 2 : 1;
  if (L.nseg < 1 || L.nseg > 3 || L.cols == 0 || L.cols % 256) return hipErrorInvalidValue;
  MArgs a{};
  a.cols = L.cols;
  a.nbr = L.cols / 256;
  a.x = L.x;
  a.norm_w = L.norm_w;
  a.eps = L.eps;
  for (int s = 0; s < L.nseg; s++) {
    if (!mfma_type(L.seg[s].type) || L.seg[s].rows == 0) return hipErrorInvalidValue;
    a.seg[s] = L.seg[s];
  }
  if (Epi::kPaired) {
    if (L.nseg != 2 || L.seg[0].rows != L.seg[1].rows || L.seg[0].type != L.seg[1].type) return hipErrorInvalidValue;
    a.nseg = 1;
  } else {
    a.nseg = L.nseg;
  }
  uint32_t total = 0;
  for (int s = 0; s < a.nseg; s++) {
    a.ntiles[s] = (uint32_t)((L.seg[s].rows + kTileRows - 1) / kTileRows);
    total += a.ntiles[s];
  }
  a.xs_off = 3 * a.cols;                    // digit planes: 48 bytes per 16 elements
  a.zero_off = a.xs_off + a.cols / 2;       // group sums: 16 bytes per 32 elements
  const size_t lds = a.zero_off + kZeroBytes;
  if (lds > kMaxDynLds) return hipErrorInvalidValue;
  bool mixed = false;
  for (int s = 1; s < a.nseg; s++) mixed |= L.seg[s].type != L.seg[0].type;
  const size_t want = mixed ? kMaxBlocksPerCu : 1;
  const uint32_t per_cu = (uint32_t)std::max<size_t>(1, std::min<size_t>(want, (160 * 1024) / lds));
  const uint32_t resident = per_cu * cu_count() * kWaves;
  uint32_t split = 1;
  while (split < (uint32_t)kWaves && split < a.nbr && total * split < resident) split *= 2;
  if (a.nseg == 1) {
    // One segment (gate and up paired, the output head, ...): of the splits
    // from that one up to kWaves, the one whose busiest wave streams the
    // fewest blocks, the larger on a tie.  The waves that share an item meet
    // at its reduction, so a larger split keeps a CU's waves in step and
    // fewer of them idle at the end:
    //   8B gate/up (896 tile pairs, 16 blocks): split 4 gives 128 of 512
    //   wave groups one item against two, split 8 gives 128 of 256
    //   workgroups three against four, 8 blocks on the busiest wave either
    //   way: 14.30 -> 14.07 us.  70B (1792 pairs, 32 blocks): 32 blocks at
    //   split 2, 28 at split 8.
    //   8B head (8016 tiles): 64 blocks on the busiest wave at every split;
    //   one wave per tile ended anywhere from 36 to 77 us (the waves of a CU
    //   stream at unequal rates), 80 us per launch against 69 at split 8.
    auto busiest = [&](uint32_t sp) {
      const uint32_t nb = std::min<uint32_t>((total * sp + kWaves - 1) / kWaves, per_cu * cu_count());
      const uint32_t tg = nb * ((uint32_t)kWaves / sp);
      return ((total + tg - 1) / tg) * ((a.nbr + sp - 1) / sp);
    };
    for (uint32_t sp = split * 2; sp <= (uint32_t)kWaves && sp <= a.nbr; sp *= 2)
      if (busiest(sp) <= busiest(split)) split = sp;
  }
  a.split = split;
  const uint32_t nbm = (a.nbr + split - 1) / split;
  const uint32_t blocks = std::min<uint32_t>((total * split + kWaves - 1) / kWaves, per_cu * cu_count());
  // ring depth (a deeper ring at lower occupancy measured slower)
  const int D = (NT == 2 || mixed || nbm <= 2) ? 2 : 4;
  a.steps = (nbm + D - 1) / D * D;
  const uint32_t TG = blocks * (kWaves / split);
  uint32_t acc = 0;
  for (int s = 0; s < a.nseg; s++) {
    a.rot[s] = acc % TG;
    acc += a.ntiles[s];
  }
  // Half items in the last round of a one-segment launch whose tiles leave
  // it at most half full (8B gate/up: 896 tile pairs on 256 groups, so that
  // 128 workgroups streamed a fourth pair while the other CUs idled; now
  // every workgroup takes three pairs and a half.  The head: 8016 tiles,
  // 31 rounds and 160 halves).  IFX_GEMV_HALVES=0 keeps whole tiles.
  for (int s = 0; s < 3; s++) a.half0[s] = a.nitems[s] = a.ntiles[s];
  const char* hv = getenv("IFX_GEMV_HALVES");
  if (!(hv && hv[0] == '0' && hv[1] == 0) && a.nseg == 1) {
    const uint32_t nt = a.ntiles[0], rounds = nt / TG, rest = nt % TG;
    if (rounds >= 1 && rest > 0 && 2 * rest <= TG) {
      a.half0[0] = rounds * TG;
      a.nitems[0] = rounds * TG + 2 * rest;
    }
  }
  // One tile per workgroup on more workgroups than CUs (the mixed QKV launch:
  // 384 on 256): workgroup i shares a CU with workgroup i + CUs, and those
  // pairs end last (per-workgroup stamps: the second ones at 8.3-9.2 us,
  // against 5.9-6.5 us for workgroups that run alone).  The Q6_K tiles
  // (3360-byte units against Q4_K's 2304) go to the workgroups that run
  // alone, [blocks - CUs, CUs), so that no pair carries one: the busiest CU
  // streams 73.7 KB instead of 90.6 (8B), and the launch takes 8.41-8.44 us
  // against 8.49-8.63 (graph-order traces).  IFX_QKV_PLACE=0 keeps the plain
  // rotation.
  const uint32_t cus = (uint32_t)cu_count();
  const char* pf = getenv("IFX_QKV_PLACE");
  const bool place = !(pf && pf[0] == '0' && pf[1] == 0);
  if (place && mixed && split == (uint32_t)kWaves && acc == TG && blocks > cus && blocks <= 2 * cus) {
    uint32_t pos = blocks - cus;  // the first workgroup that runs alone
    for (int heavy = 1; heavy >= 0; heavy--)
      for (int s = 0; s < a.nseg; s++)
        if ((L.seg[s].type == T_Q6K) == (heavy == 1)) {
          a.rot[s] = pos % TG;
          pos += a.ntiles[s];
        }
  }
  const uint32_t ta = L.seg[0].type;
  uint32_t tb = ta;
  for (int s = 1; s < a.nseg; s++)
    if (L.seg[s].type != ta) {
      tb = L.seg[s].type;
      a.use_b |= 1u << s;
    }
  if constexpr (Epi::kPaired) {
    return go_types<Epi, 2>(a, ta, tb, epi, blocks, lds, st);
  } else {
    if (D == 2) return go_types<Epi, 2>(a, ta, tb, epi, blocks, lds, st);
    return go_types<Epi, 4>(a, ta, tb, epi, blocks, lds, st);
  }
}

// The K-split residual launches where they apply: one Q4_K / Q6_K segment
// without a norm, K in whole slices of at most 16 blocks, and at least one
// tile per wave of the grid; hipErrorNotSupported otherwise (the caller takes
// launch_mfma).
namespace {
hipError_t ks_plan(const GemvLaunch& L, float* h, KsArgs& a, uint32_t& blocks, size_t& lds) {
  if (L.nseg != 1 || L.norm_w || L.paired || !mfma_type(L.seg[0].type) || L.cols == 0 || L.cols % 256)
    return hipErrorNotSupported;
  const uint32_t nbr = L.cols / 256;
  blocks = (uint32_t)cu_count();
  const uint32_t ntiles = (uint32_t)((L.seg[0].rows + kTileRows - 1) / kTileRows);
  if (nbr % kKs || nbr / kKs > kKsMaxBlocks || blocks % kKs || ntiles < blocks / kKs * kWaves)
    return hipErrorNotSupported;
  a = KsArgs{};
  a.seg = L.seg[0];
  a.ntiles = ntiles;
  a.nbr = nbr;
  a.nbs = nbr / kKs;
  a.x = L.x;
  a.h = h;
  a.xs_off = 768u * a.nbs;              // digit planes: 48 bytes per 16 elements
  a.zero_off = a.xs_off + 128u * a.nbs;  // group sums: 16 bytes per 32 elements
  lds = a.zero_off + kZeroBytes;
  return hipSuccess;
}
}  // namespace

hipError_t launch_mfma_residual_ks(const GemvLaunch& L, float* h, hipStream_t st) {
  KsArgs a;
  uint32_t blocks;
  size_t lds;
  const hipError_t e = ks_plan(L, h, a, blocks, lds);
  if (e != hipSuccess) return e;
  // The waves of a workgroup in lockstep (a barrier per ring round): 70B
  // down 30.45 -> 29.55 us (28 units per wave), O 7.91 -> 7.80; no change at
  // 8B (7 units per wave).  IFX_KS_LOCK=0 runs each wave on its own.
  const char* lk = getenv("IFX_KS_LOCK");
  const bool lock = !(lk && lk[0] == '0' && lk[1] == 0);
  if (L.seg[0].type == T_Q6K) {
    if (lock) hipLaunchKernelGGL((k_gemv_ks<T_Q6K, kKsRing, true>), dim3(blocks), dim3(kThreads), lds, st, a);
    else hipLaunchKernelGGL((k_gemv_ks<T_Q6K, kKsRing, false>), dim3(blocks), dim3(kThreads), lds, st, a);
  } else {
    if (lock) hipLaunchKernelGGL((k_gemv_ks<T_Q4K, kKsRing, true>), dim3(blocks), dim3(kThreads), lds, st, a);
    else hipLaunchKernelGGL((k_gemv_ks<T_Q4K, kKsRing, false>), dim3(blocks), dim3(kThreads), lds, st, a);
  }
  return hipGetLastError();
}

// The K-split q/k/v launch where it applies: three Q4_K / Q6_K segments with
// the norm, q and k of one type, K in whole slices of at most 16 blocks and
// at most 8192 columns.
namespace {
bool qkv_ks_plan(const GemvLaunch& L, const QkvDst& d, KsQkvArgs& a, uint32_t& blocks, size_t& lds) {
  // whole heads per segment, RoPE pairs inside a head
  if (d.head_dim == 0 || d.head_dim % 2 || d.rope_dim > d.head_dim || d.rope_dim % 2 || d.max_seq == 0) return false;
  if (L.nseg != 3 || !L.norm_w || L.paired || L.cols == 0 || L.cols % 256 || L.cols > 2 * 8 * kThreads) return false;
  for (int s = 0; s < 3; s++)
    if (!mfma_type(L.seg[s].type) || L.seg[s].rows == 0) return false;
  if (L.seg[0].type != L.seg[1].type) return false;
  const uint32_t nbr = L.cols / 256;
  blocks = (uint32_t)cu_count();
  if (nbr % kKs || nbr / kKs > kKsMaxBlocks || blocks % kKs) return false;
  a = KsQkvArgs{};
  for (int s = 0; s < 3; s++) {
    if (L.seg[s].rows % d.head_dim) return false;
    a.seg[s] = L.seg[s];
    a.ntiles[s] = (uint32_t)((L.seg[s].rows + kTileRows - 1) / kTileRows);
  }
  a.nbr = nbr;
  a.nbs = nbr / kKs;
  a.cols = L.cols;
  a.x = L.x;
  a.norm_w = L.norm_w;
  a.eps = L.eps;
  a.dst = d;
  // waves per slice for each segment, in proportion to its tiles (at least one each)
  const uint32_t ws = blocks / kKs * kWaves, nt = a.ntiles[0] + a.ntiles[1] + a.ntiles[2];
  if (ws < 3) return false;
  auto share = [&](uint32_t n) { return std::max(1u, (uint32_t)(((uint64_t)ws * n + nt / 2) / nt)); };
  a.wk = std::min(share(a.ntiles[1]), ws - 2);
  const uint32_t wv = std::min(share(a.ntiles[2]), ws - a.wk - 1);
  a.wq = ws - a.wk - wv;
  a.xs_off = 768u * a.nbs;               // digit planes: 48 bytes per 16 elements
  a.zero_off = a.xs_off + 128u * a.nbs;  // group sums: 16 bytes per 32 elements
  lds = a.zero_off + kZeroBytes;
  return true;
}

template <int TA, int TB>
hipError_t go_qkv(const KsQkvArgs& a, uint32_t blocks, size_t lds, hipStream_t st) {
  if (a.cols <= 8u * kThreads)
    hipLaunchKernelGGL((k_gemv_ks_qkv<TA, TB, kKsRing, 1>), dim3(blocks), dim3(kThreads), lds, st, a);
  else
    hipLaunchKernelGGL((k_gemv_ks_qkv<TA, TB, kKsRing, 2>), dim3(blocks), dim3(kThreads), lds, st, a);
  return hipGetLastError();
}
}  // namespace

bool qkv_ks_supported(const GemvLaunch& L, const QkvDst& d) {
  KsQkvArgs a;
  uint32_t blocks;
  size_t lds;
  return qkv_ks_plan(L, d, a, blocks, lds);
}

hipError_t launch_qkv_ks(const GemvLaunch& L, const QkvDst& d, hipStream_t st) {
  KsQkvArgs a;
  uint32_t blocks;
  size_t lds;
  if (!d.q || !d.k_cache || !d.v_cache || !d.state || !qkv_ks_plan(L, d, a, blocks, lds)) return hipErrorInvalidValue;
  const uint32_t ta = a.seg[0].type, tb = a.seg[2].type;
  if (ta == T_Q4K) return tb == T_Q4K ? go_qkv<T_Q4K, T_Q4K>(a, blocks, lds, st) : go_qkv<T_Q4K, T_Q6K>(a, blocks, lds, st);
  return tb == T_Q6K ? go_qkv<T_Q6K, T_Q6K>(a, blocks, lds, st) : go_qkv<T_Q6K, T_Q4K>(a, blocks, lds, st);
}

uint32_t merge_o_first_chunks() { return kMergeFirst; }
uint32_t merge_o_bound_step() { return kMergeBoundStep; }

bool merge_o_supported(const GemvLaunch& L, const AttnArgs& at) {
  KsArgs a;
  uint32_t blocks;
  size_t lds;
  if (ks_plan(L, nullptr, a, blocks, lds) != hipSuccess) return false;
  const uint32_t G = at.n_kv_heads ? at.n_heads / at.n_kv_heads : 0;
  return at.n_kv_heads == kKs && at.n_heads == G * kKs && at.head_dim == 128 && (G == 4 || G == 8) &&
         a.nbs * 256 == G * 128 && at.max_chunks > 0 && at.chunk > 0;
}

hipError_t launch_mfma_residual_merge(const GemvLaunch& L, const AttnArgs& at, float* h, hipStream_t st,
                                      uint32_t first) {
  if (!merge_o_supported(L, at) || first == 0) return hipErrorInvalidValue;
  KsArgs a;
  uint32_t blocks;
  size_t lds;
  (void)ks_plan(L, h, a, blocks, lds);
  a.x = nullptr;
  a.partial = at.partial;
  a.state = at.state;
  a.max_chunks = at.max_chunks;
  a.chunk = at.chunk;
  // a multiple of the splits of a workgroup's chunks (2 or 4): the batch and
  // the loop after it then cover each chunk once
  a.first = std::min((first + kMergeBoundStep - 1) / kMergeBoundStep * kMergeBoundStep, kMergeFirst);
  const bool g8 = at.n_heads / at.n_kv_heads == 8, q6 = L.seg[0].type == T_Q6K;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), lds, st, a);
    return hipGetLastError();
  };
  auto types = [&](auto fb) {
    constexpr int FB = decltype(fb)::value;
    if (g8) return q6 ? go(k_gemv_ks_merge<T_Q6K, kKsRing, 8, FB>) : go(k_gemv_ks_merge<T_Q4K, kKsRing, 8, FB>);
    return q6 ? go(k_gemv_ks_merge<T_Q6K, kKsRing, 4, FB>) : go(k_gemv_ks_merge<T_Q4K, kKsRing, 4, FB>);
  };
  static_assert(kMergeFirst == 48 && kMergeBoundStep == 8, "one kernel per bound below");
  switch (a.first) {
    case 8: return types(std::integral_constant<int, 8>{});
    case 16: return types(std::integral_constant<int, 16>{});
    case 24: return types(std::integral_constant<int, 24>{});
    case 32: return types(std::integral_constant<int, 32>{});
    case 40: return types(std::integral_constant<int, 40>{});
    default: return types(std::integral_constant<int, 48>{});
  }
}

template hipError_t launch_mfma<EpiStore>(const GemvLaunch&, const EpiStore&, hipStream_t);
template hipError_t launch_mfma<EpiResidual>(const GemvLaunch&, const EpiResidual&, hipStream_t);
template hipError_t launch_mfma<EpiQkv>(const GemvLaunch&, const EpiQkv&, hipStream_t);
template hipError_t launch_mfma<EpiSwiglu>(const GemvLaunch&, const EpiSwiglu&, hipStream_t);
template hipError_t launch_mfma<EpiLogits>(const GemvLaunch&, const EpiLogits&, hipStream_t);

}  // namespace ifx
