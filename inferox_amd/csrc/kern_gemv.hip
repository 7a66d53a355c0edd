// kern_gemv.hip — fused dequant-GEMV for batch-1 decode on gfx950.
//
// Replaces the decode use of ops::matmul_t (src/ops.rs:33-44,104-134) fed by
// the per-call f32 dequant of Weights::tensor_f32_by_index
// (src/gguf/weights.rs:66-74): y = W x with W read once from HBM in its
// quantized form and decoded in registers.
//
// Work decomposition
//   * Persistent workgroups of 8 wave64, two per CU (16 waves per CU, at most
//     128 VGPRs each).  Each wave issues the loads of its first unit, then the
//     workgroup stages x in LDS, optionally applying RMSNorm (ops::rms_norm,
//     src/ops.rs:155-168) so the norm costs no launch, and precomputes
//     16-element partial sums of x (the min/offset terms of the K-quants factor
//     out as scale * sum(x)).
//   * A wave owns tiles of R = 4 rows.  A "unit" is one 32-element group of
//     each of the R rows per lane (lane l takes group l + 64 i), so each lane
//     reads contiguous 16-byte pieces of the packed blocks and one x group read
//     from LDS serves R rows.  The loads of the next unit are issued as soon as
//     the current one is decoded; the other waves of the CU cover the latency.
//     Tile and row bookkeeping is wave-uniform (scalar registers).
//   * Row sums are reduced across the wave; the epilogue fuses RoPE + KV
//     append (QKV), SwiGLU (gate/up), the residual add (O, down) or the logits
//     store + greedy argmax (output head).
// Compiled with -ffp-contract=off: only the explicit fmaf below are fused.
#include <algorithm>
#include <type_traits>

#include "kernels.h"

namespace ifx {

namespace {

constexpr int kWaves = 8;
constexpr int kBlocksPerCu = 2;  // 16 waves per CU
constexpr int kWavesPerSimd = kBlocksPerCu * kWaves / 4;  // 4: at most 128 VGPRs per lane
constexpr int kThreads = kWaves * 64;
constexpr int kR = 4;

struct KArgs {
  GemvSeg seg[3];
  uint32_t ntiles[3];  // tiles per logical segment (paired: one logical segment)
  uint32_t rot[3];     // first-wave rotation per segment (balances small segments)
  uint32_t use_b;      // bit s: segment s decodes with the kernel's second type
  uint32_t split;      // waves per row tile (1, 2, 4 or 8): they share its units
  int nseg;            // logical segments
  uint32_t cols, groups;
  const float* x;
  const float* norm_w;
  float eps;
};

__device__ __forceinline__ float cvtb(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xffu); }
// Hides a masked word from the combiner so that cvtb(w, k) selects
// v_cvt_f32_ubyte<k> (one instruction) instead of a bit-field extract of the
// unmasked word followed by a convert.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}
// byte b of v as a signed int8, to f32 (v_bfe_i32 + v_cvt_f32_i32)
__device__ __forceinline__ float sbyte(int v, int b) { return (float)((v << (24 - 8 * b)) >> 24); }

// x lives in LDS with each 32-element group padded to 36 floats, so lanes
// reading consecutive groups (a 144-byte stride) spread over the banks.
constexpr int kGroupStride = 36;
__device__ __forceinline__ uint32_t xpad(uint32_t i) { return (i >> 5) * kGroupStride + (i & 31); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <class T>
__device__ __forceinline__ T ldg(const void* p) { return *(const T*)p; }

// Selects acc[r] for lane r (r < kR) with a chain of selects; the asm
// barriers keep the compiler from folding it back into a dynamic index of a
// register array (which it would place in scratch memory).
__device__ __forceinline__ float lane_acc(const float* acc, int lane) {
  float v = acc[0];
#pragma unroll
  for (int r = 1; r < kR; r++) {
    v = lane == r ? acc[r] : v;
    asm("" : "+v"(v));
  }
  return v;
}

// Row r of tile `tile` of logical segment s, wave-uniform.  Paired launches
// (gate/up) put rows 2t, 2t+1 of segment 0 in r = 0, 1 and the same rows of
// segment 1 in r = 2, 3.
struct RowRef {
  const uint8_t* body;
  const uint8_t* scal;
  uint64_t row;
  bool ok;  // false for padding rows past the end of the segment
};

template <bool PAIRED>
__device__ __forceinline__ RowRef row_of(const KArgs& a, int s, uint32_t tile, int r) {
  // padding rows read the last real row (loads stay unconditional) and are
  // skipped by the decode and the epilogue
  if (PAIRED) {
    const GemvSeg& sg = a.seg[r < kR / 2 ? 0 : 1];
    const uint32_t row = tile * (kR / 2) + (r % (kR / 2));
    return RowRef{sg.body, sg.scal, row < sg.rows ? row : sg.rows - 1, row < sg.rows};
  }
  const GemvSeg& sg = a.seg[s];
  const uint32_t row = tile * kR + r;
  return RowRef{sg.body, sg.scal, row < sg.rows ? row : sg.rows - 1, row < sg.rows};
}

// ---------------------------------------------------------------------------
// Per-type fragments: the raw bytes of one unit (group g of the kR rows of a
// tile) held in registers, and the decode + dot of that group with x.
//   load_row(a, s, tile, g, r): issue the loads of row r, group g (always a
//     real group of a real row: padding rows and lanes are clamped).
//   dot_row(a, s, tile, g, valid, xv, xsa, xsb, acc, r): acc[r] += row r . x
//     over group g; xv holds the group's 32 x values, xsa/xsb its two
//     16-element sums.  Lanes with !valid and padding rows add nothing.
// The main loop is free of branches so that the compiler can wait for exactly
// the loads a row needs (a join in the control flow makes it wait for all).
// ---------------------------------------------------------------------------

// Q4_K (src/gguf/dequant.rs:133-161): element 32g+l is nibble (l&1) of
// qs[16g + l/2];  sum_l ((d*sc)*q_l - dmin*mn) x_l = (d*sc)*S - (dmin*mn)*sum(x).
struct FragQ4K {
  uint4 h[kR], q[kR];
  template <bool P>
  __device__ void load_row(const KArgs& a, int s, uint32_t tile, uint32_t g, int r) {
    const RowRef rr = row_of<P>(a, s, tile, r);
    // wave-uniform row base + 32-bit lane offset (scalar-base loads)
    const uint8_t* row = rr.body + rr.row * ((a.groups / 8) * 144);
    const uint32_t off = (g / 8) * 144;
    h[r] = ldg<uint4>(row + off);
    q[r] = ldg<uint4>(row + off + 16 + 16 * (g & 7));
  }
  template <bool P>
  __device__ void dot_row(const KArgs& a, int s, uint32_t tile, uint32_t g, bool valid, const float4* xv, float xsa,
                          float xsb, float* acc, int r) const {
    const uint32_t sub = g & 7, j = sub & 3;
    const uint4 hv = h[r];
    // 6-bit scale / min of sub-block `sub` (get_scale_min_k4), selected without a branch
    const uint32_t sc_lo = (hv.y >> (8 * j)) & 63u, mn_lo = (hv.z >> (8 * j)) & 63u;
    const uint32_t sc_hi = ((hv.w >> (8 * j)) & 15u) | (((hv.y >> (8 * j + 6)) & 3u) << 4);
    const uint32_t mn_hi = ((hv.w >> (8 * j + 4)) & 15u) | (((hv.z >> (8 * j + 6)) & 3u) << 4);
    const uint32_t sc = sub < 4 ? sc_lo : sc_hi, mn = sub < 4 ? mn_lo : mn_hi;
    const float d = h2f(hv.x), dmin = h2f(hv.x >> 16);
    float s0 = 0.f, s1 = 0.f;
    const uint32_t qw[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
#pragma unroll
    for (int w = 0; w < 4; w++) {
      // high nibbles stay in place (16 q): s1 is scaled by 1/16 below, exactly
      const uint32_t lo = opaque(qw[w] & 0x0F0F0F0Fu), hi = opaque(qw[w] & 0xF0F0F0F0u);
      const float4 xa = xv[2 * w], xb = xv[2 * w + 1];
      s0 = fmaf(cvtb(lo, 0), xa.x, s0);
      s1 = fmaf(cvtb(hi, 0), xa.y, s1);
      s0 = fmaf(cvtb(lo, 1), xa.z, s0);
      s1 = fmaf(cvtb(hi, 1), xa.w, s1);
      s0 = fmaf(cvtb(lo, 2), xb.x, s0);
      s1 = fmaf(cvtb(hi, 2), xb.y, s1);
      s0 = fmaf(cvtb(lo, 3), xb.z, s0);
      s1 = fmaf(cvtb(hi, 3), xb.w, s1);
    }
    const float A = d * (float)sc, M = dmin * (float)mn;
    const float v = fmaf(A, fmaf(s1, 0.0625f, s0), -M * (xsa + xsb));
    acc[r] += (valid && row_of<P>(a, s, tile, r).ok) ? v : 0.f;
  }
};

// Q6_K in the device layout (ql | re-ordered qh | u8 sc; d separate):
// q = lo | hi<<4, y = (d*sc)*(q-32)  (src/gguf/dequant.rs:182-197).
struct FragQ6K {
  uint4 ql[kR];
  uint2 qh[kR];
  uint32_t sd[kR];  // the group's two scale bytes (low 16 bits) | d bits (high 16)
  template <bool P>
  __device__ void load_row(const KArgs& a, int s, uint32_t tile, uint32_t g, int r) {
    const RowRef rr = row_of<P>(a, s, tile, r);
    const uint32_t nb = a.groups / 8;
    const uint8_t* row = rr.body + rr.row * (nb * 208);
    const uint8_t* rowd = rr.scal + rr.row * (nb * 2);
    const uint32_t off = (g / 8) * 208, h = g & 7;
    ql[r] = ldg<uint4>(row + off + 16 * h);
    qh[r] = ldg<uint2>(row + off + 128 + 8 * h);
    sd[r] = (uint32_t)ldg<uint16_t>(row + off + 192 + 2 * h) | ((uint32_t)ldg<uint16_t>(rowd + (g / 8) * 2) << 16);
  }
  template <bool P>
  __device__ void dot_row(const KArgs& a, int s, uint32_t tile, uint32_t, bool valid, const float4* xv, float xsa,
                          float xsb, float* acc, int r) const {
    const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
    const uint4 L = ql[r];
    const uint2 H = qh[r];
    // half a: elements 0..15 (L.x: 0-7, L.y: 8-15; high bits in H.x); half b: 16..31
    const uint32_t ev[4] = {opaque((L.x & m4) | (H.x & m2)), opaque((L.y & m4) | ((H.x << 4) & m2)),
                            opaque((L.z & m4) | (H.y & m2)), opaque((L.w & m4) | ((H.y << 4) & m2))};
    const uint32_t ov[4] = {opaque(((L.x >> 4) & m4) | ((H.x >> 2) & m2)),
                            opaque(((L.y >> 4) & m4) | ((H.x << 2) & m2)),
                            opaque(((L.z >> 4) & m4) | ((H.y >> 2) & m2)),
                            opaque(((L.w >> 4) & m4) | ((H.y << 2) & m2))};
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
    for (int w = 0; w < 2; w++) {
      const float4 xa = xv[2 * w], xb = xv[2 * w + 1];
      a0 = fmaf(cvtb(ev[w], 0), xa.x, a0);
      a1 = fmaf(cvtb(ov[w], 0), xa.y, a1);
      a0 = fmaf(cvtb(ev[w], 1), xa.z, a0);
      a1 = fmaf(cvtb(ov[w], 1), xa.w, a1);
      a0 = fmaf(cvtb(ev[w], 2), xb.x, a0);
      a1 = fmaf(cvtb(ov[w], 2), xb.y, a1);
      a0 = fmaf(cvtb(ev[w], 3), xb.z, a0);
      a1 = fmaf(cvtb(ov[w], 3), xb.w, a1);
    }
#pragma unroll
    for (int w = 2; w < 4; w++) {
      const float4 xa = xv[2 * w], xb = xv[2 * w + 1];
      b0 = fmaf(cvtb(ev[w], 0), xa.x, b0);
      b1 = fmaf(cvtb(ov[w], 0), xa.y, b1);
      b0 = fmaf(cvtb(ev[w], 1), xa.z, b0);
      b1 = fmaf(cvtb(ov[w], 1), xa.w, b1);
      b0 = fmaf(cvtb(ev[w], 2), xb.x, b0);
      b1 = fmaf(cvtb(ov[w], 2), xb.y, b1);
      b0 = fmaf(cvtb(ev[w], 3), xb.z, b0);
      b1 = fmaf(cvtb(ov[w], 3), xb.w, b1);
    }
    const float d = h2f(sd[r] >> 16);
    const float sa = (float)(sd[r] & 0xffu), sb = (float)((sd[r] >> 8) & 0xffu);
    const float ta = fmaf(-32.f, xsa, a0 + a1), tb = fmaf(-32.f, xsb, b0 + b1);
    const float v = d * fmaf(sa, ta, sb * tb);
    acc[r] += (valid && row_of<P>(a, s, tile, r).ok) ? v : 0.f;
  }
};

// Q8_0 (device layout qs[32] | d): y = f32(i8 q) * delta (src/gguf/dequant.rs:101-109).
struct FragQ80 {
  uint4 qa[kR], qb[kR];
  uint32_t d[kR];
  template <bool P>
  __device__ void load_row(const KArgs& a, int s, uint32_t tile, uint32_t g, int r) {
    const RowRef rr = row_of<P>(a, s, tile, r);
    const uint8_t* row = rr.body + rr.row * (a.groups * 32);
    qa[r] = ldg<uint4>(row + g * 32);
    qb[r] = ldg<uint4>(row + g * 32 + 16);
    d[r] = ldg<uint16_t>(rr.scal + rr.row * (a.groups * 2) + g * 2);
  }
  // q x = (u - 128) x with u = q ^ 0x80 unsigned: one convert per byte, the
  // -128 sum(x) term from the staged group sums
  template <bool P>
  __device__ void dot_row(const KArgs& a, int s, uint32_t tile, uint32_t, bool valid, const float4* xv, float xsa,
                          float xsb, float* acc, int r) const {
    const uint32_t qw[8] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w, qb[r].x, qb[r].y, qb[r].z, qb[r].w};
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int w = 0; w < 8; w++) {
      const float4 xa = xv[w];
      const uint32_t u = opaque(qw[w] ^ 0x80808080u);
      s0 = fmaf(cvtb(u, 0), xa.x, s0);
      s1 = fmaf(cvtb(u, 1), xa.y, s1);
      s0 = fmaf(cvtb(u, 2), xa.z, s0);
      s1 = fmaf(cvtb(u, 3), xa.w, s1);
    }
    const float v = h2f(d[r]) * fmaf(-128.f, xsa + xsb, s0 + s1);
    acc[r] += (valid && row_of<P>(a, s, tile, r).ok) ? v : 0.f;
  }
};

// Q4_0 (device layout qs[16] | d): low nibble -> element j, high -> j+16, value q-8.
struct FragQ40 {
  uint4 q[kR];
  uint32_t d[kR];
  template <bool P>
  __device__ void load_row(const KArgs& a, int s, uint32_t tile, uint32_t g, int r) {
    const RowRef rr = row_of<P>(a, s, tile, r);
    q[r] = ldg<uint4>(rr.body + rr.row * (a.groups * 16) + g * 16);
    d[r] = ldg<uint16_t>(rr.scal + rr.row * (a.groups * 2) + g * 2);
  }
  template <bool P>
  __device__ void dot_row(const KArgs& a, int s, uint32_t tile, uint32_t, bool valid, const float4* xv, float xsa,
                          float xsb, float* acc, int r) const {
    const uint32_t qw[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const uint32_t lo = opaque(qw[w] & 0x0F0F0F0Fu), hi = opaque(qw[w] & 0xF0F0F0F0u);  // hi: 16 q
      const float4 xa = xv[w], xb = xv[4 + w];
      s0 = fmaf(cvtb(lo, 0), xa.x, s0);
      s0 = fmaf(cvtb(lo, 1), xa.y, s0);
      s0 = fmaf(cvtb(lo, 2), xa.z, s0);
      s0 = fmaf(cvtb(lo, 3), xa.w, s0);
      s1 = fmaf(cvtb(hi, 0), xb.x, s1);
      s1 = fmaf(cvtb(hi, 1), xb.y, s1);
      s1 = fmaf(cvtb(hi, 2), xb.z, s1);
      s1 = fmaf(cvtb(hi, 3), xb.w, s1);
    }
    const float v = h2f(d[r]) * fmaf(-8.f, xsa + xsb, fmaf(s1, 0.0625f, s0));
    acc[r] += (valid && row_of<P>(a, s, tile, r).ok) ? v : 0.f;
  }
};

// Q8_K (device layout sc[32] | qs[256]; {d, dmin}): y = ((d*sc)*q) - dmin.
struct FragQ8K {
  uint4 qa[kR], qb[kR];
  uint32_t sc[kR], dd[kR];
  template <bool P>
  __device__ void load_row(const KArgs& a, int s, uint32_t tile, uint32_t g, int r) {
    const RowRef rr = row_of<P>(a, s, tile, r);
    const uint32_t nb = a.groups / 8, sub = g & 7;
    const uint8_t* blk = rr.body + rr.row * (nb * 288) + (g / 8) * 288;
    sc[r] = ldg<uint32_t>(blk + 4 * sub);
    qa[r] = ldg<uint4>(blk + 32 + 32 * sub);
    qb[r] = ldg<uint4>(blk + 48 + 32 * sub);
    dd[r] = ldg<uint32_t>(rr.scal + rr.row * (nb * 4) + (g / 8) * 4);
  }
  template <bool P>
  __device__ void dot_row(const KArgs& a, int s, uint32_t tile, uint32_t, bool valid, const float4* xv, float xsa,
                          float xsb, float* acc, int r) const {
    const uint32_t qw[8] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w, qb[r].x, qb[r].y, qb[r].z, qb[r].w};
    const float d = h2f(dd[r]), dmin = h2f(dd[r] >> 16);
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {  // sub-blocks of 8 elements share one scale byte
      float acc8 = 0.f;
#pragma unroll
      for (int w = 0; w < 2; w++) {
        const int v = (int)qw[2 * k + w];
        const float4 x4 = xv[2 * k + w];
        acc8 = fmaf(sbyte(v, 0), x4.x, acc8);
        acc8 = fmaf(sbyte(v, 1), x4.y, acc8);
        acc8 = fmaf(sbyte(v, 2), x4.z, acc8);
        acc8 = fmaf(sbyte(v, 3), x4.w, acc8);
      }
      tot = fmaf(d * cvtb(sc[r], k), acc8, tot);
    }
    const float v = fmaf(-dmin, xsa + xsb, tot);
    acc[r] += (valid && row_of<P>(a, s, tile, r).ok) ? v : 0.f;
  }
};

// F32 / F16 rows of whole groups: read at use, no prefetch (toy models, tests).
struct FragF32 {
  template <bool P>
  __device__ void load_row(const KArgs&, int, uint32_t, uint32_t, int) {}
  template <bool P>
  __device__ void dot_row(const KArgs& a, int s, uint32_t tile, uint32_t g, bool valid, const float4* xv, float,
                          float, float* acc, int r) const {
    const RowRef rr = row_of<P>(a, s, tile, r);
    const float4* w4 = (const float4*)rr.body + (rr.row * (uint64_t)a.groups + g) * 8;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 w = w4[i], x = xv[i];
      s0 = fmaf(w.x, x.x, s0);
      s1 = fmaf(w.y, x.y, s1);
      s0 = fmaf(w.z, x.z, s0);
      s1 = fmaf(w.w, x.w, s1);
    }
    acc[r] += (valid && rr.ok) ? s0 + s1 : 0.f;
  }
};

struct FragF16 {
  template <bool P>
  __device__ void load_row(const KArgs&, int, uint32_t, uint32_t, int) {}
  template <bool P>
  __device__ void dot_row(const KArgs& a, int s, uint32_t tile, uint32_t g, bool valid, const float4* xv, float,
                          float, float* acc, int r) const {
    const RowRef rr = row_of<P>(a, s, tile, r);
    const uint4* w4 = (const uint4*)rr.body + (rr.row * (uint64_t)a.groups + g) * 4;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint4 w = w4[i];
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const float4 x = xv[2 * i + k];
        s0 = fmaf(h2f(ww[2 * k]), x.x, s0);
        s1 = fmaf(h2f(ww[2 * k] >> 16), x.y, s1);
        s0 = fmaf(h2f(ww[2 * k + 1]), x.z, s0);
        s1 = fmaf(h2f(ww[2 * k + 1] >> 16), x.w, s1);
      }
    }
    acc[r] += (valid && rr.ok) ? s0 + s1 : 0.f;
  }
};

// ---- epilogues: apply(segment, tile, reduced sums); lane r < kR owns row r ----
struct EpiStore {
  static constexpr bool kPaired = false;
  float* y;
  uint32_t seg_out[3];  // output offset of each segment
  struct Wave {};
  __device__ void apply(Wave&, const KArgs& a, int s, uint32_t tile, const float* acc, int lane) const {
    if (lane < kR) {
      const RowRef rr = row_of<false>(a, s, tile, lane);
      if (rr.ok) y[seg_out[s] + rr.row] = lane_acc(acc, lane);
    }
  }
  __device__ void finish(Wave&, int) const {}
};

struct EpiResidual {
  static constexpr bool kPaired = false;
  float* h;
  struct Wave {};
  __device__ void apply(Wave&, const KArgs& a, int s, uint32_t tile, const float* acc, int lane) const {
    if (lane < kR) {
      const RowRef rr = row_of<false>(a, s, tile, lane);
      if (rr.ok) h[rr.row] = lane_acc(acc, lane) + h[rr.row];
    }
  }
  __device__ void finish(Wave&, int) const {}
};

struct EpiQkv {
  static constexpr bool kPaired = false;
  QkvEpi e;
  struct Wave {};
  // rope (src/ops.rs:273-284): x[2i] = a*cos - b*sin, x[2i+1] = a*sin + b*cos
  __device__ void apply(Wave&, const KArgs& a, int s, uint32_t tile, const float* acc, int lane) const {
    if (lane >= kR) return;
    const RowRef rr = row_of<false>(a, s, tile, lane);
    if (!rr.ok) return;
    const uint32_t r = (uint32_t)rr.row;
    float v = lane_acc(acc, lane);
    if (s < 2) {
      const uint32_t i = r % e.head_dim;
      if (i < e.rope_dim) {
        const float2 cs = e.rope_cs[(uint64_t)e.state->rope_pos * (e.rope_dim / 2) + i / 2];
        const float other = lane_acc(acc, lane ^ 1);
        v = (i & 1) ? (other * cs.y + v * cs.x) : (v * cs.x - other * cs.y);
      }
    }
    if (s == 0) {
      e.q_out[r] = v;
    } else {
      const uint64_t off = (uint64_t)e.state->len * e.kv_dim + r;
      if (s == 1) e.k_cache[off] = v;
      else e.v_cache[off] = v;
    }
  }
  __device__ void finish(Wave&, int) const {}
};

struct EpiSwiglu {
  static constexpr bool kPaired = true;
  float* mid;
  struct Wave {};
  // swiglu (src/ops.rs:190-209): silu(g) * u, sigmoid clamped to +-80
  __device__ void apply(Wave&, const KArgs& a, int, uint32_t tile, const float* acc, int lane) const {
    constexpr int H = kR / 2;
    if (lane >= H) return;
    const RowRef rr = row_of<true>(a, 0, tile, lane);
    if (!rr.ok) return;
    const float g = lane_acc(acc, lane), u = lane_acc(acc, lane + H);
    float c = fminf(fmaxf(g, -80.f), 80.f);
    if (g != g) c = g;
    const float sig = 1.0f / (1.0f + expf(-c));
    mid[rr.row] = (g * sig) * u;
  }
  __device__ void finish(Wave&, int) const {}
};

__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | idx;
}

struct EpiLogits {
  static constexpr bool kPaired = false;
  float* logits;
  DevState* state;
  struct Wave {
    unsigned long long best = 0;
    bool nan = false;
  };
  __device__ void apply(Wave& w, const KArgs& a, int s, uint32_t tile, const float* acc, int lane) const {
#pragma unroll
    for (int r = 0; r < kR; r++) {
      const RowRef rr = row_of<false>(a, s, tile, r);
      if (!rr.ok) continue;
      if (lane == r) logits[rr.row] = acc[r];
      if (acc[r] != acc[r]) w.nan = true;
      const unsigned long long k = argmax_key(acc[r], (uint32_t)rr.row);
      w.best = k > w.best ? k : w.best;
    }
  }
  __device__ void finish(Wave& w, int lane) const {
    if (lane == 0) {
      if (w.best) atomicMax(&state->argmax_key, w.best);
      if (w.nan) atomicExch(&state->status, (int)IFX_E_NAN_LOGIT);
    }
  }
};

// The row tiles of one logical segment owned by this wave's tile group
// (a.split waves of one workgroup): tiles first, first+TG, ..., `iters` of them
// (the same count for every wave of the workgroup, so that the LDS reduction
// of a split tile can use workgroup barriers).  Wave j of the group takes the
// units j, j+split, ... of each tile.  `f` arrives holding the loads of the
// first unit.  As soon as row r of the current unit is decoded, the loads of
// row r of the next unit are issued into the same registers, so the wave keeps
// loads in flight while it computes (a second register buffer would cost
// occupancy).  Past the wave's last unit the loads repeat a real unit.
template <class Frag, class Epi>
__device__ __forceinline__ void run_segment(const KArgs& a, const Epi& epi, typename Epi::Wave& ws, int s,
                                            uint32_t first, uint32_t TG, uint32_t iters, uint32_t j, Frag& f,
                                            const float* xl, const float* xs, float* part, int lane, int wave) {
  constexpr bool P = Epi::kPaired;
  const uint32_t NG = (a.groups + 63) / 64, S = a.split;
  for (uint32_t k = 0; k < iters; k++) {
    const uint32_t tile = first + k * TG;
    const bool live = tile < a.ntiles[s];  // uniform over the wave
    float acc[kR];
#pragma unroll
    for (int r = 0; r < kR; r++) acc[r] = 0.f;
    if (live) {
      for (uint32_t it = j; it < NG; it += S) {
        const uint32_t g = lane + 64 * it, gc = min(g, a.groups - 1);
        uint32_t nt = tile, ni = it + S;
        if (ni >= NG) {
          ni = j;
          nt += TG;
        }
        if (nt >= a.ntiles[s]) nt = tile;  // uniform select: no branch around the loads
        const uint32_t ng = min(lane + 64 * ni, a.groups - 1);
        const float4* xv4 = (const float4*)(xl + kGroupStride * gc);
        float4 xv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = xv4[i];
        const float xsa = xs[2 * gc], xsb = xs[2 * gc + 1];
#pragma unroll
        for (int r = 0; r < kR; r++) {
          f.template dot_row<P>(a, s, tile, gc, g < a.groups, xv, xsa, xsb, acc, r);
          f.template load_row<P>(a, s, nt, ng, r);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kR; r++) acc[r] = wave_sum(acc[r]);
    if (S > 1) {
      // partial sums of the group's waves through LDS (double-buffered: one barrier per tile)
      float* pb = part + (k & 1) * kWaves * kR;
      if (lane < kR) pb[wave * kR + lane] = lane_acc(acc, lane);
      __syncthreads();
      if (j == 0 && live) {
#pragma unroll
        for (int r = 0; r < kR; r++) {
          float v = 0.f;
          for (uint32_t i = 0; i < S; i++) v += pb[(wave + i) * kR + r];
          acc[r] = v;
        }
        epi.apply(ws, a, s, tile, acc, lane);
      }
    } else if (live) {
      epi.apply(ws, a, s, tile, acc, lane);
    }
  }
}

// rms_norm (src/ops.rs:162-167): scale = 1/sqrt(mean(x^2) + eps); x = (x*scale)*w.
// Reduces the per-thread sums of squares over the workgroup.
__device__ __forceinline__ float norm_scale(const KArgs& a, float ss, float* red, int lane, int wave) {
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; w++) tot += red[w];
  return 1.0f / sqrtf(tot / (float)a.cols + a.eps);
}

// Workgroup prologue (cols % 32 == 0): x, optionally RMS-normalised, into LDS
// and the 16-element sums of x.  Every thread issues all its float4 loads of
// x (and of the norm weights, staged in wl) before the first wait, so the
// prologue costs one memory round trip.
constexpr int kStage = 8;  // float4 loads per thread per batch
template <bool NORM>
__device__ __forceinline__ float stage_load(const KArgs& a, float* xl, float* wl, int tid) {
  const uint32_t n4 = a.cols / 4;
  const float4* x4 = (const float4*)a.x;
  const float4* w4 = (const float4*)a.norm_w;
  float ss = 0.f;
  for (uint32_t b = tid; b < n4; b += kThreads * kStage) {
    float4 v[kStage], w[kStage];
#pragma unroll
    for (int k = 0; k < kStage; k++) {
      const uint32_t i = min(b + k * kThreads, n4 - 1);  // clamped: loads stay unconditional
      v[k] = x4[i];
      if (NORM) w[k] = w4[i];
    }
#pragma unroll
    for (int k = 0; k < kStage; k++) {
      const uint32_t i = b + k * kThreads;
      if (i < n4) {
        *(float4*)(xl + xpad(4 * i)) = v[k];  // 4 | 32: a float4 never straddles a group
        if (NORM) {
          *(float4*)(wl + 4 * i) = w[k];
          ss = fmaf(v[k].x, v[k].x, ss);
          ss = fmaf(v[k].y, v[k].y, ss);
          ss = fmaf(v[k].z, v[k].z, ss);
          ss = fmaf(v[k].w, v[k].w, ss);
        }
      }
    }
  }
  return ss;
}

__device__ __forceinline__ void stage_x(const KArgs& a, float* xl, float* xs, float* wl, float* red, int tid,
                                        int lane, int wave) {
  const uint32_t n4 = a.cols / 4;
  if (a.norm_w) {
    const float ss = stage_load<true>(a, xl, wl, tid);
    const float scale = norm_scale(a, ss, red, lane, wave);
    for (uint32_t i = tid; i < n4; i += kThreads) {
      float4 v = *(float4*)(xl + xpad(4 * i));
      const float4 w = *(const float4*)(wl + 4 * i);
      v.x = (v.x * scale) * w.x;
      v.y = (v.y * scale) * w.y;
      v.z = (v.z * scale) * w.z;
      v.w = (v.w * scale) * w.w;
      *(float4*)(xl + xpad(4 * i)) = v;
    }
  } else {
    stage_load<false>(a, xl, wl, tid);
  }
  __syncthreads();
  for (uint32_t j = tid; j < a.cols / 16; j += kThreads) {
    const float4* p = (const float4*)(xl + (j >> 1) * kGroupStride + 16 * (j & 1));
    const float4 u0 = p[0], u1 = p[1], u2 = p[2], u3 = p[3];
    xs[j] = ((u0.x + u0.y) + (u0.z + u0.w)) + ((u1.x + u1.y) + (u1.z + u1.w)) +
            (((u2.x + u2.y) + (u2.z + u2.w)) + ((u3.x + u3.y) + (u3.z + u3.w)));
  }
  __syncthreads();
}

// Prologue of the generic kernel (any cols): x, optionally RMS-normalised, into LDS.
__device__ __forceinline__ void stage_x_generic(const KArgs& a, float* xl, float* red, int tid, int lane,
                                                int wave) {
  float ss = 0.f;
  for (uint32_t i = tid; i < a.cols; i += kThreads) {
    const float v = a.x[i];
    xl[xpad(i)] = v;
    ss = fmaf(v, v, ss);
  }
  if (a.norm_w) {
    const float scale = norm_scale(a, ss, red, lane, wave);
    for (uint32_t i = tid; i < a.cols; i += kThreads) xl[xpad(i)] = (xl[xpad(i)] * scale) * a.norm_w[i];
  }
  __syncthreads();
}

// Main kernel: segments decode with FragA, or with FragB where use_b is set
// (a Q4_K_M layer's QKV has Q4_K q/k and Q6_K v).
template <class Epi, class FragA, class FragB>
__global__ void __launch_bounds__(kThreads, kWavesPerSimd) k_gemv(KArgs a, Epi epi) {
  extern __shared__ float lds[];
  float* xl = lds;                                    // [groups][36]
  float* xs = lds + (size_t)a.groups * kGroupStride;  // [cols/16]
  float* wl = xs + ((a.cols / 16 + 3) & ~3u);         // [cols] norm weights (norm launches), 16-B aligned
  __shared__ float red[kWaves];
  __shared__ float part[2 * kWaves * kR];
  // the wave index is uniform: tile and row bookkeeping stays in scalar registers
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // tile groups of a.split waves; TG groups in the grid
  const uint32_t S = a.split, GPB = kWaves / S, TG = gridDim.x * GPB;
  const uint32_t tg = blockIdx.x * GPB + wave / S, j = wave % S;
  typename Epi::Wave ws;
  // tiles per group of this workgroup for segment s: the count of its busiest group
  auto block_iters = [&](int s) -> uint32_t {
    uint32_t n = 0;
    for (uint32_t q = 0; q < GPB; q++) {
      const uint32_t f0 = (blockIdx.x * GPB + q + TG - a.rot[s]) % TG;
      if (f0 < a.ntiles[s]) n = max(n, (a.ntiles[s] - 1 - f0) / TG + 1);
    }
    return n;
  };
  const uint32_t NG = (a.groups + 63) / 64;
  const uint32_t g0 = min(lane + 64 * min(j, NG - 1), a.groups - 1);

  // first unit of segment 0 (always FragA) in flight while x is staged
  constexpr bool P = Epi::kPaired;
  constexpr bool kMixed = !std::is_same<FragA, FragB>::value;
  {
    const uint32_t first = (tg + TG - a.rot[0]) % TG;
    FragA f;
    // lanes past the last group load a real group (unconditional loads keep
    // the fragments' live ranges short); their values are never used
    if (first < a.ntiles[0]) {
#pragma unroll
      for (int r = 0; r < kR; r++) f.template load_row<P>(a, 0, first, g0, r);
    }
    stage_x(a, xl, xs, wl, red, tid, lane, wave);
    run_segment<FragA, Epi>(a, epi, ws, 0, first, TG, block_iters(0), j, f, xl, xs, part, lane, wave);
  }
  for (int s = 1; s < a.nseg; s++) {
    const uint32_t first = (tg + TG - a.rot[s]) % TG;
    const uint32_t iters = block_iters(s);
    if (iters == 0) continue;
    const uint32_t t0 = first < a.ntiles[s] ? first : 0;
    if (kMixed && ((a.use_b >> s) & 1u)) {
      FragB f;
#pragma unroll
      for (int r = 0; r < kR; r++) f.template load_row<P>(a, s, t0, g0, r);
      run_segment<FragB, Epi>(a, epi, ws, s, first, TG, iters, j, f, xl, xs, part, lane, wave);
    } else {
      FragA f;
#pragma unroll
      for (int r = 0; r < kR; r++) f.template load_row<P>(a, s, t0, g0, r);
      run_segment<FragA, Epi>(a, epi, ws, s, first, TG, iters, j, f, xl, xs, part, lane, wave);
    }
  }
  epi.finish(ws, lane);
}

// Rows that are not whole 32-element groups (F32/F16 only): lanes stride over
// the elements of each row.
template <class Epi>
__global__ void __launch_bounds__(kThreads) k_gemv_generic(KArgs a, Epi epi) {
  extern __shared__ float lds[];
  __shared__ float red[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  stage_x_generic(a, lds, red, tid, lane, wave);
  const uint32_t W = gridDim.x * kWaves, wid = blockIdx.x * kWaves + wave;
  typename Epi::Wave ws;
  for (int s = 0; s < a.nseg; s++) {
    for (uint32_t t = (wid + W - a.rot[s]) % W; t < a.ntiles[s]; t += W) {
      float acc[kR] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < kR; r++) {
        const RowRef rr = row_of<Epi::kPaired>(a, s, t, r);
        if (!rr.ok) continue;
        const bool f32 = a.seg[Epi::kPaired ? (r < kR / 2 ? 0 : 1) : s].type == T_F32;
        const uint64_t base = rr.row * a.cols;
        float v = 0.f;
        for (uint32_t l = lane; l < a.cols; l += 64) {
          const float w = f32 ? ((const float*)rr.body)[base + l] : h2f(((const uint16_t*)rr.body)[base + l]);
          v = fmaf(w, lds[xpad(l)], v);
        }
        acc[r] = v;
      }
#pragma unroll
      for (int r = 0; r < kR; r++) acc[r] = wave_sum(acc[r]);
      epi.apply(ws, a, s, t, acc, lane);
    }
  }
  epi.finish(ws, lane);
}

int device_cu_count() {
  static int n = 0;
  if (n == 0) {
    int dev = 0;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess) n = p.multiProcessorCount;
    if (n <= 0) n = 256;
  }
  return n;
}

template <class K>
hipError_t lds_opt_in(K kernel, size_t lds, bool& done) {
  if (lds > 64 * 1024 && !done) {  // rows of >16K columns need more than 64 KiB of LDS
    hipError_t e = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
    if (e != hipSuccess) return e;
    done = true;
  }
  return hipSuccess;
}

template <class Epi, class FA, class FB>
hipError_t dispatch(const KArgs& a, const Epi& epi, uint32_t blocks, size_t lds, hipStream_t st) {
  static bool done = false;
  hipError_t e = lds_opt_in(k_gemv<Epi, FA, FB>, lds, done);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_gemv<Epi, FA, FB>), dim3(blocks), dim3(kThreads), lds, st, a, epi);
  return hipGetLastError();
}

template <class Epi, class FA>
hipError_t dispatch_b(const KArgs& a, uint32_t tb, const Epi& epi, uint32_t blocks, size_t lds, hipStream_t st) {
  switch (tb) {
    case T_Q4K: return dispatch<Epi, FA, FragQ4K>(a, epi, blocks, lds, st);
    case T_Q6K: return dispatch<Epi, FA, FragQ6K>(a, epi, blocks, lds, st);
    default: return hipErrorInvalidValue;
  }
}

template <class Epi>
hipError_t launch(const GemvLaunch& L, const Epi& epi, hipStream_t st) {
  if (L.nseg < 1 || L.nseg > 3 || L.cols == 0) return hipErrorInvalidValue;
  KArgs a{};
  a.cols = L.cols;
  a.groups = (L.cols + 31) / 32;
  a.x = L.x;
  a.norm_w = L.norm_w;
  a.eps = L.eps;
  const bool generic = L.cols % 32 != 0;
  for (int s = 0; s < L.nseg; s++) {
    a.seg[s] = L.seg[s];
    const uint32_t t = L.seg[s].type;
    if ((t == T_Q4K || t == T_Q6K || t == T_Q8K) && L.cols % 256) return hipErrorInvalidValue;
    if (generic && t != T_F32 && t != T_F16) return hipErrorInvalidValue;
  }
  if (Epi::kPaired) {
    if (L.nseg != 2 || L.seg[0].rows != L.seg[1].rows || L.seg[0].type != L.seg[1].type) return hipErrorInvalidValue;
    a.nseg = 1;
    a.ntiles[0] = (L.seg[0].rows + kR / 2 - 1) / (kR / 2);
  } else {
    a.nseg = L.nseg;
    for (int s = 0; s < L.nseg; s++) a.ntiles[s] = (L.seg[s].rows + kR - 1) / kR;
  }
  const size_t lds = (size_t)a.groups * kGroupStride * 4 + (size_t)((a.cols / 16 + 3) & ~3u) * 4 +
                     (L.norm_w && !generic ? (size_t)a.cols * 4 : 0);
  if (lds > 150 * 1024) return hipErrorInvalidValue;
  uint32_t total = 0;
  for (int s = 0; s < a.nseg; s++) total += a.ntiles[s];
  if (total == 0) return hipSuccess;
  // persistent grid: as many workgroups as fit per CU (LDS-bound for long
  // rows).  Long rows (at least 4 units) with fewer row tiles than resident
  // waves share each tile's units among `split` waves (the 8B down projection:
  // 1024 tiles of 7 units).
  const uint32_t per_cu = (uint32_t)std::max<size_t>(1, std::min<size_t>(kBlocksPerCu, (160 * 1024) / lds));
  const uint32_t resident = per_cu * device_cu_count() * kWaves;
  const uint32_t NG = (a.groups + 63) / 64;
  uint32_t split = 1;
  if (!generic && NG >= 4)
    while (split < (uint32_t)kWaves && split < NG && total * split < resident) split *= 2;
  a.split = split;
  const uint32_t blocks = std::min<uint32_t>((total * split + kWaves - 1) / kWaves, per_cu * device_cu_count());
  const uint32_t TG = blocks * (kWaves / split);
  uint32_t acc = 0;
  for (int s = 0; s < a.nseg; s++) {
    a.rot[s] = acc % TG;
    acc += a.ntiles[s];
  }
  if (generic) {
    static bool done = false;
    hipError_t e = lds_opt_in(k_gemv_generic<Epi>, lds, done);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_gemv_generic<Epi>, dim3(blocks), dim3(kThreads), lds, st, a, epi);
    return hipGetLastError();
  }
  // segments of the first type decode with FragA, the others with FragB
  const uint32_t ta = L.seg[0].type;
  uint32_t tb = ta;
  for (int s = 0; s < a.nseg; s++)
    if (L.seg[s].type != ta) {
      if (tb != ta && L.seg[s].type != tb) return hipErrorInvalidValue;  // at most two types
      tb = L.seg[s].type;
      a.use_b |= 1u << s;
    }
  if (tb == ta) {
    switch (ta) {
      case T_Q4K: return dispatch<Epi, FragQ4K, FragQ4K>(a, epi, blocks, lds, st);
      case T_Q6K: return dispatch<Epi, FragQ6K, FragQ6K>(a, epi, blocks, lds, st);
      case T_Q8_0: return dispatch<Epi, FragQ80, FragQ80>(a, epi, blocks, lds, st);
      case T_Q4_0: return dispatch<Epi, FragQ40, FragQ40>(a, epi, blocks, lds, st);
      case T_Q8K: return dispatch<Epi, FragQ8K, FragQ8K>(a, epi, blocks, lds, st);
      case T_F32: return dispatch<Epi, FragF32, FragF32>(a, epi, blocks, lds, st);
      case T_F16: return dispatch<Epi, FragF16, FragF16>(a, epi, blocks, lds, st);
      default: return hipErrorInvalidValue;
    }
  }
  switch (ta) {  // mixed Q4_K / Q6_K (Q4_K_M layers)
    case T_Q4K: return dispatch_b<Epi, FragQ4K>(a, tb, epi, blocks, lds, st);
    case T_Q6K: return dispatch_b<Epi, FragQ6K>(a, tb, epi, blocks, lds, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int gemv_supported(uint32_t t) {
  return t == T_F32 || t == T_F16 || t == T_Q4_0 || t == T_Q8_0 || t == T_Q4K || t == T_Q6K ||
         t == T_Q8K;
}

hipError_t gemv_store(const GemvLaunch& L, float* y, hipStream_t st) {
  EpiStore e{};
  e.y = y;
  uint32_t off = 0;
  for (int s = 0; s < L.nseg; s++) { e.seg_out[s] = off; off += L.seg[s].rows; }
  return launch(L, e, st);
}

hipError_t gemv_residual(const GemvLaunch& L, float* hidden, hipStream_t st) {
  if (L.nseg != 1) return hipErrorInvalidValue;
  return launch(L, EpiResidual{hidden}, st);
}

hipError_t gemv_qkv(const GemvLaunch& L, const QkvEpi& e, hipStream_t st) {
  if (L.nseg != 3 || (e.head_dim & 1) || (e.rope_dim & 1)) return hipErrorInvalidValue;
  return launch(L, EpiQkv{e}, st);
}

hipError_t gemv_swiglu(const GemvLaunch& L, float* mid, hipStream_t st) {
  if (!L.paired) return hipErrorInvalidValue;
  return launch(L, EpiSwiglu{mid}, st);
}

hipError_t gemv_logits(const GemvLaunch& L, float* logits, DevState* state, hipStream_t st) {
  if (L.nseg != 1) return hipErrorInvalidValue;
  return launch(L, EpiLogits{logits, state}, st);
}

}  // namespace ifx
