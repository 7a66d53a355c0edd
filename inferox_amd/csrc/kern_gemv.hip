// kern_gemv.hip — fused dequant-GEMV for batch-1 decode on gfx950.
//
// Replaces the decode use of ops::matmul_t (src/ops.rs:33-44,104-134) fed by
// the per-call f32 dequant of Weights::tensor_f32_by_index
// (src/gguf/weights.rs:66-74): y = W x with W read once from HBM in its
// quantized form and decoded in registers.  This file holds the f32-dot path
// (Q8_0, Q4_0, Q8_K, F32, F16) and the launcher of every GEMV; Q4_K and Q6_K
// matrices go to the int8-MFMA kernel of kern_gemv_mfma.hip.
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

#include "gemv_epi.h"

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

// Hands the reduced sums of a finished tile to the row epilogue (gemv_epi.h):
// lane r < kR owns row r (paired: lanes 0, 1 own the gate rows, whose up rows
// sit at r + 2).
template <class Epi>
__device__ __forceinline__ void emit(const Epi& epi, typename Epi::Wave& ws, const KArgs& a, int s, uint32_t tile,
                                     const float* acc, int lane) {
  constexpr bool P = Epi::kPaired;
  if (lane < (P ? kR / 2 : kR)) {
    const RowRef rr = row_of<P>(a, s, tile, lane);
    if (rr.ok) {
      const float v = lane_acc(acc, lane);
      const float partner = P ? lane_acc(acc, lane + kR / 2) : (Epi::kNeighbor ? lane_acc(acc, lane ^ 1) : 0.f);
      const int es = P ? 0 : s;
      epi.row(ws, es, (uint32_t)rr.row, v, partner, epi.pre(ws, es, (uint32_t)rr.row));
    }
  }
}

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
        emit(epi, ws, a, s, tile, acc, lane);
      }
    } else if (live) {
      emit(epi, ws, a, s, tile, acc, lane);
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

// Main kernel: every segment decodes with Frag.
template <class Epi, class Frag>
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
  epi.begin(ws);
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

  // first unit of segment 0 in flight while x is staged
  constexpr bool P = Epi::kPaired;
  {
    const uint32_t first = (tg + TG - a.rot[0]) % TG;
    Frag f;
    // lanes past the last group load a real group (unconditional loads keep
    // the fragments' live ranges short); their values are never used
    if (first < a.ntiles[0]) {
#pragma unroll
      for (int r = 0; r < kR; r++) f.template load_row<P>(a, 0, first, g0, r);
    }
    stage_x(a, xl, xs, wl, red, tid, lane, wave);
    run_segment<Frag, Epi>(a, epi, ws, 0, first, TG, block_iters(0), j, f, xl, xs, part, lane, wave);
  }
  for (int s = 1; s < a.nseg; s++) {
    const uint32_t first = (tg + TG - a.rot[s]) % TG;
    const uint32_t iters = block_iters(s);
    if (iters == 0) continue;
    const uint32_t t0 = first < a.ntiles[s] ? first : 0;
    Frag f;
#pragma unroll
    for (int r = 0; r < kR; r++) f.template load_row<P>(a, s, t0, g0, r);
    run_segment<Frag, Epi>(a, epi, ws, s, first, TG, iters, j, f, xl, xs, part, lane, wave);
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
  epi.begin(ws);
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
      emit(epi, ws, a, s, t, acc, lane);
    }
  }
  epi.finish(ws, lane);
}

int device_cu_count() {
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

// Rows of >16K columns need more than 64 KiB of LDS: each kernel instance
// opts in once, through a block-scope static of a function instantiated per
// kernel (initialised the first time a launch gets there, once even when
// sessions run on several threads).
template <class K>
hipError_t allow_lds(K kernel) {
  return hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
}

template <class Epi, class F>
hipError_t dispatch(const KArgs& a, const Epi& epi, uint32_t blocks, size_t lds, hipStream_t st) {
  if (lds > 64 * 1024) {
    static const hipError_t opted = allow_lds(k_gemv<Epi, F>);
    if (opted != hipSuccess) return opted;
  }
  hipLaunchKernelGGL((k_gemv<Epi, F>), dim3(blocks), dim3(kThreads), lds, st, a, epi);
  return hipGetLastError();
}

template <class Epi>
hipError_t launch(const GemvLaunch& L, const Epi& epi, hipStream_t st) {
  if (L.nseg < 1 || L.nseg > 3 || L.cols == 0) return hipErrorInvalidValue;
  // Q4_K / Q6_K (tiled layout): the int8-MFMA kernel; a launch does not mix the two families
  int n_mfma = 0;
  for (int s = 0; s < L.nseg; s++) n_mfma += mfma_type(L.seg[s].type) ? 1 : 0;
  if (n_mfma == L.nseg) return launch_mfma(L, epi, st);
  if (n_mfma != 0) return hipErrorInvalidValue;
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
    if (t == T_Q8K && L.cols % 256) return hipErrorInvalidValue;
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
    if (lds > 64 * 1024) {
      static const hipError_t opted = allow_lds(k_gemv_generic<Epi>);
      if (opted != hipSuccess) return opted;
    }
    hipLaunchKernelGGL(k_gemv_generic<Epi>, dim3(blocks), dim3(kThreads), lds, st, a, epi);
    return hipGetLastError();
  }
  // one type per launch on this path (the mixed Q4_K / Q6_K layers take the MFMA kernel)
  const uint32_t ta = L.seg[0].type;
  for (int s = 1; s < a.nseg; s++)
    if (L.seg[s].type != ta) return hipErrorInvalidValue;
  switch (ta) {
    case T_Q8_0: return dispatch<Epi, FragQ80>(a, epi, blocks, lds, st);
    case T_Q4_0: return dispatch<Epi, FragQ40>(a, epi, blocks, lds, st);
    case T_Q8K: return dispatch<Epi, FragQ8K>(a, epi, blocks, lds, st);
    case T_F32: return dispatch<Epi, FragF32>(a, epi, blocks, lds, st);
    case T_F16: return dispatch<Epi, FragF16>(a, epi, blocks, lds, st);
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
  const hipError_t e = launch_mfma_residual_ks(L, hidden, st);
  if (e != hipErrorNotSupported) return e;
  return launch(L, EpiResidual{hidden}, st);
}

hipError_t gemv_residual_fixed(const GemvLaunch& L, float* hidden, hipStream_t st) {
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
