// kern_gemv.hip — fused dequant-GEMV for batch-1 decode on gfx950.
//
// Replaces the decode use of ops::matmul_t (src/ops.rs:33-44,104-134) fed by
// the per-call f32 dequant of Weights::tensor_f32_by_index
// (src/gguf/weights.rs:66-74): y = W x with W read once from HBM in its
// quantized form and decoded in registers.
//
// Work decomposition
//   * A workgroup (4 wave64) first stages x in LDS, optionally applying
//     RMSNorm (ops::rms_norm, src/ops.rs:155-168) so the norm costs no launch,
//     and precomputes 16-element partial sums of x (the min/offset terms of the
//     K-quants factor out as scale * sum(x)).
//   * A wave owns a tile of R = 4 rows and sweeps K with each lane on one
//     32-element group per step (lane = group within a 64-group step), so each
//     lane reads contiguous 16-byte pieces of the packed blocks and the x group
//     read from LDS is reused for all R rows.
//   * The R row sums are reduced across the wave; the epilogue fuses RoPE + KV
//     append (QKV), SwiGLU (gate/up), the residual add (O, down) or the logits
//     store + greedy argmax (output head).
// Compiled with -ffp-contract=off: only the explicit fmaf below are fused.
#include "kernels.h"

namespace ifx {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kR = 4;

struct KArgs {
  GemvSeg seg[3];
  uint32_t vbegin[4];  // first virtual row of each segment (padded to kR)
  int nseg;
  int paired;
  int generic;  // rows are not whole 32-element groups (F32/F16 only)
  uint32_t cols, groups, ntiles;
  const float* x;
  const float* norm_w;
  float eps;
};

__device__ __forceinline__ float cvtb(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xffu); }
// byte b of v as a signed int8, to f32 (v_bfe_i32 + v_cvt_f32_i32)
__device__ __forceinline__ float sbyte(int v, int b) { return (float)((v << (24 - 8 * b)) >> 24); }

// x lives in LDS with each 32-element group padded to 36 floats, so lanes
// reading consecutive groups (a 144-byte stride) hit distinct banks.
constexpr int kGroupStride = 36;
__device__ __forceinline__ uint32_t xpad(uint32_t i) { return (i >> 5) * kGroupStride + (i & 31); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---- per-type dot of one 32-element group of one row with x (xv: 8 float4) ----

// Q4_K (src/gguf/dequant.rs:133-161): element 32g+l is nibble (l&1) of
// qs[16g + l/2];  sum_l ((d*sc)*q_l - dmin*mn) x_l = (d*sc)*S - (dmin*mn)*sum(x).
__device__ __forceinline__ float dot_q4k(const uint8_t* blk, int sub, const float4* xv, float xsum) {
  const uint4 h = *(const uint4*)blk;
  const uint4 q = *(const uint4*)(blk + 16 + 16 * sub);
  const int j = sub & 3;
  uint32_t sc, mn;
  if (sub < 4) {
    sc = (h.y >> (8 * j)) & 63u;
    mn = (h.z >> (8 * j)) & 63u;
  } else {
    sc = ((h.w >> (8 * j)) & 15u) | (((h.y >> (8 * j + 6)) & 3u) << 4);
    mn = ((h.w >> (8 * j + 4)) & 15u) | (((h.z >> (8 * j + 6)) & 3u) << 4);
  }
  const float d = h2f(h.x), dmin = h2f(h.x >> 16);
  float s0 = 0.f, s1 = 0.f;
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int w = 0; w < 4; w++) {
    const uint32_t lo = qw[w] & 0x0F0F0F0Fu, hi = (qw[w] >> 4) & 0x0F0F0F0Fu;
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
  return fmaf(A, s0 + s1, -(M * xsum));
}

// Q6_K in the device layout (ql | re-ordered qh | u8 sc; d separate):
// q = lo | hi<<4, y = (d*sc)*(q-32)  (src/gguf/dequant.rs:182-197).
__device__ __forceinline__ float dot_q6k(const uint8_t* blk, uint32_t dbits, int h, const float4* xv,
                                         float xs_a, float xs_b) {
  const uint4 ql = *(const uint4*)(blk + 16 * h);
  const uint2 qh = *(const uint2*)(blk + 128 + 8 * h);
  const uint32_t scw = *(const uint16_t*)(blk + 192 + 2 * h);
  const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
  // half a: elements 0..15 (ql.x: 0-7, ql.y: 8-15; high bits in qh.x)
  const uint32_t e0 = (ql.x & m4) | (qh.x & m2), o0 = ((ql.x >> 4) & m4) | ((qh.x >> 2) & m2);
  const uint32_t e1 = (ql.y & m4) | ((qh.x << 4) & m2), o1 = ((ql.y >> 4) & m4) | ((qh.x << 2) & m2);
  // half b: elements 16..31 (ql.z, ql.w; qh.y)
  const uint32_t e2 = (ql.z & m4) | (qh.y & m2), o2 = ((ql.z >> 4) & m4) | ((qh.y >> 2) & m2);
  const uint32_t e3 = (ql.w & m4) | ((qh.y << 4) & m2), o3 = ((ql.w >> 4) & m4) | ((qh.y << 2) & m2);
  float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
  const uint32_t ev[4] = {e0, e1, e2, e3}, ov[4] = {o0, o1, o2, o3};
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
  const float d = h2f(dbits);
  const float sa = (float)(scw & 0xffu), sb = (float)(scw >> 8);
  const float ta = fmaf(-32.f, xs_a, a0 + a1), tb = fmaf(-32.f, xs_b, b0 + b1);
  return d * fmaf(sa, ta, sb * tb);
}

// Q8_0 (device layout qs[32] | d): y = f32(i8 q) * delta (src/gguf/dequant.rs:101-109).
__device__ __forceinline__ float dot_q80(const uint8_t* qs, uint32_t dbits, const float4* xv) {
  const uint4 qa = *(const uint4*)qs, qb = *(const uint4*)(qs + 16);
  const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int w = 0; w < 8; w++) {
    const float4 xa = xv[w];
    const int v = (int)qw[w];
    s0 = fmaf(sbyte(v, 0), xa.x, s0);
    s1 = fmaf(sbyte(v, 1), xa.y, s1);
    s0 = fmaf(sbyte(v, 2), xa.z, s0);
    s1 = fmaf(sbyte(v, 3), xa.w, s1);
  }
  return h2f(dbits) * (s0 + s1);
}

// Q4_0 (device layout qs[16] | d): low nibble -> element j, high -> j+16, value q-8.
__device__ __forceinline__ float dot_q40(const uint8_t* qs, uint32_t dbits, const float4* xv, float xsum) {
  const uint4 q = *(const uint4*)qs;
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int w = 0; w < 4; w++) {
    const uint32_t lo = qw[w] & 0x0F0F0F0Fu, hi = (qw[w] >> 4) & 0x0F0F0F0Fu;
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
  return h2f(dbits) * fmaf(-8.f, xsum, s0 + s1);
}

// Q8_K (device layout sc[32] | qs[256]; {d, dmin}): y = ((d*sc)*q) - dmin.
__device__ __forceinline__ float dot_q8k(const uint8_t* blk, uint32_t dd, int sub, const float4* xv,
                                         float xsum) {
  const uint32_t scw = *(const uint32_t*)(blk + 4 * sub);
  const uint4 qa = *(const uint4*)(blk + 32 + 32 * sub), qb = *(const uint4*)(blk + 48 + 32 * sub);
  const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  const float d = h2f(dd), dmin = h2f(dd >> 16);
  float tot = 0.f;
#pragma unroll
  for (int s = 0; s < 4; s++) {  // sub-blocks of 8 elements share one scale byte
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < 2; w++) {
      const int v = (int)qw[2 * s + w];
      const float4 x4 = xv[2 * s + w];
      a = fmaf(sbyte(v, 0), x4.x, a);
      a = fmaf(sbyte(v, 1), x4.y, a);
      a = fmaf(sbyte(v, 2), x4.z, a);
      a = fmaf(sbyte(v, 3), x4.w, a);
    }
    tot = fmaf(d * cvtb(scw, s), a, tot);
  }
  return fmaf(-dmin, xsum, tot);
}

__device__ __forceinline__ float dot_f32(const float* w, const float4* xv) {
  const float4* w4 = (const float4*)w;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float4 a = w4[i], x = xv[i];
    s0 = fmaf(a.x, x.x, s0);
    s1 = fmaf(a.y, x.y, s1);
    s0 = fmaf(a.z, x.z, s0);
    s1 = fmaf(a.w, x.w, s1);
  }
  return s0 + s1;
}

__device__ __forceinline__ float dot_f16(const uint16_t* w, const float4* xv) {
  const uint4* w4 = (const uint4*)w;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint4 a = w4[i];
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const float4 x = xv[2 * i + k];
      s0 = fmaf(h2f(aw[2 * k]), x.x, s0);
      s1 = fmaf(h2f(aw[2 * k] >> 16), x.y, s1);
      s0 = fmaf(h2f(aw[2 * k + 1]), x.z, s0);
      s1 = fmaf(h2f(aw[2 * k + 1] >> 16), x.w, s1);
    }
  }
  return s0 + s1;
}

// Sweep all groups of a tile of kR rows (one segment type) for this lane.
template <int TYPE>
__device__ __forceinline__ void tile_dot(const GemvSeg* segs, const int* segof, const int* rows,
                                         const float* xl, const float* xs, uint32_t groups,
                                         uint32_t cols, int lane, float* acc) {
  for (uint32_t g = lane; g < groups; g += 64) {
    const float4* xv4 = (const float4*)(xl + kGroupStride * g);
    float4 xv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) xv[i] = xv4[i];
    const float xsa = xs[2 * g], xsb = xs[2 * g + 1];
#pragma unroll
    for (int r = 0; r < kR; r++) {
      if (rows[r] < 0) continue;
      const GemvSeg& s = segs[segof[r]];
      const uint64_t row = (uint64_t)rows[r];
      float v;
      if (TYPE == T_Q4K) {
        const uint64_t blk = row * (groups / 8) + g / 8;
        v = dot_q4k(s.body + blk * 144, g & 7, xv, xsa + xsb);
      } else if (TYPE == T_Q6K) {
        const uint64_t blk = row * (groups / 8) + g / 8;
        v = dot_q6k(s.body + blk * 208, ((const uint16_t*)s.scal)[blk], g & 7, xv, xsa, xsb);
      } else if (TYPE == T_Q8_0) {
        const uint64_t blk = row * groups + g;
        v = dot_q80(s.body + blk * 32, ((const uint16_t*)s.scal)[blk], xv);
      } else if (TYPE == T_Q4_0) {
        const uint64_t blk = row * groups + g;
        v = dot_q40(s.body + blk * 16, ((const uint16_t*)s.scal)[blk], xv, xsa + xsb);
      } else if (TYPE == T_Q8K) {
        const uint64_t blk = row * (groups / 8) + g / 8;
        v = dot_q8k(s.body + blk * 288, ((const uint32_t*)s.scal)[blk], g & 7, xv, xsa + xsb);
      } else if (TYPE == T_F32) {
        v = dot_f32((const float*)s.body + row * cols + 32 * g, xv);
      } else {
        v = dot_f16((const uint16_t*)s.body + row * cols + 32 * g, xv);
      }
      acc[r] += v;
    }
  }
}

// Any row length (F32/F16 rows that are not whole 32-element groups): lanes
// stride over the elements of each row.
__device__ __forceinline__ void tile_dot_generic(const GemvSeg* segs, const int* segof, const int* rows,
                                                 const float* xl, uint32_t cols, int lane, float* acc) {
#pragma unroll
  for (int r = 0; r < kR; r++) {
    if (rows[r] < 0) continue;
    const GemvSeg& s = segs[segof[r]];
    const uint64_t base = (uint64_t)rows[r] * cols;
    float a = 0.f;
    for (uint32_t l = lane; l < cols; l += 64) {
      const float w = s.type == T_F32 ? ((const float*)s.body)[base + l] : h2f(((const uint16_t*)s.body)[base + l]);
      a = fmaf(w, xl[xpad(l)], a);
    }
    acc[r] += a;
  }
}

// ---- epilogues ----
struct EpiStore {
  float* y;
  uint32_t seg_out[3];  // output offset of each segment
  struct Wave {};
  __device__ void apply(Wave&, int segi, const int* rows, const int* segof, const float* acc, int lane) const {
    if (lane < kR && rows[lane] >= 0) y[seg_out[segof[lane]] + rows[lane]] = acc[lane];
  }
  __device__ void finish(Wave&, int) const {}
};

struct EpiResidual {
  float* h;
  struct Wave {};
  __device__ void apply(Wave&, int, const int* rows, const int*, const float* acc, int lane) const {
    if (lane < kR && rows[lane] >= 0) h[rows[lane]] = acc[lane] + h[rows[lane]];
  }
  __device__ void finish(Wave&, int) const {}
};

struct EpiQkv {
  QkvEpi e;
  struct Wave {};
  // rope (src/ops.rs:273-284): x[2i] = a*cos - b*sin, x[2i+1] = a*sin + b*cos
  __device__ void apply(Wave&, int segi, const int* rows, const int*, const float* acc, int lane) const {
    if (lane >= kR || rows[lane] < 0) return;
    const int r = rows[lane];
    float v = acc[lane];
    if (segi < 2) {
      const uint32_t i = (uint32_t)r % e.head_dim;
      if (i < e.rope_dim) {
        const float2 cs = e.rope_cs[(uint64_t)e.state->rope_pos * (e.rope_dim / 2) + i / 2];
        const float other = acc[lane ^ 1];
        v = (i & 1) ? (other * cs.y + v * cs.x) : (v * cs.x - other * cs.y);
      }
    }
    if (segi == 0) {
      e.q_out[r] = v;
    } else {
      const uint64_t off = (uint64_t)e.state->len * e.kv_dim + (uint64_t)r;
      if (segi == 1) e.k_cache[off] = v;
      else e.v_cache[off] = v;
    }
  }
  __device__ void finish(Wave&, int) const {}
};

struct EpiSwiglu {
  float* mid;
  struct Wave {};
  // swiglu (src/ops.rs:190-209): silu(g) * u, sigmoid clamped to +-80
  __device__ void apply(Wave&, int, const int* rows, const int*, const float* acc, int lane) const {
    constexpr int H = kR / 2;
    if (lane >= H || rows[lane] < 0) return;
    float g = acc[lane];
    const float u = acc[lane + H];
    float c = fminf(fmaxf(g, -80.f), 80.f);
    if (g != g) c = g;
    const float sig = 1.0f / (1.0f + expf(-c));
    mid[rows[lane]] = (g * sig) * u;
  }
  __device__ void finish(Wave&, int) const {}
};

__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | idx;
}

struct EpiLogits {
  float* logits;
  DevState* state;
  struct Wave {
    unsigned long long best = 0;
    bool nan = false;
  };
  __device__ void apply(Wave& w, int, const int* rows, const int*, const float* acc, int lane) const {
    if (lane < kR && rows[lane] >= 0) logits[rows[lane]] = acc[lane];
#pragma unroll
    for (int r = 0; r < kR; r++) {
      if (rows[r] < 0) continue;
      if (acc[r] != acc[r]) w.nan = true;
      const unsigned long long k = argmax_key(acc[r], (uint32_t)rows[r]);
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

template <class Epi>
__global__ void __launch_bounds__(kThreads) k_gemv(KArgs a, Epi epi) {
  extern __shared__ float lds[];
  float* xl = lds;                                        // [groups][36]
  float* xs = lds + (size_t)a.groups * kGroupStride;      // [cols/16]
  __shared__ float red[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // ---- prologue: x (optionally RMS-normalised) into LDS ----
  float ss = 0.f;
  for (uint32_t i = tid; i < a.cols; i += kThreads) {
    const float v = a.x[i];
    xl[xpad(i)] = v;
    ss = fmaf(v, v, ss);
  }
  if (a.norm_w) {
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) tot += red[w];
    // rms_norm (src/ops.rs:162-167): scale = 1/sqrt(mean + eps); x = (x*scale)*w
    const float scale = 1.0f / sqrtf(tot / (float)a.cols + a.eps);
    for (uint32_t i = tid; i < a.cols; i += kThreads) xl[xpad(i)] = (xl[xpad(i)] * scale) * a.norm_w[i];
  }
  __syncthreads();
  if (!a.generic) {
    for (uint32_t j = tid; j < a.cols / 16; j += kThreads) {
      const float4* p = (const float4*)(xl + (j >> 1) * kGroupStride + 16 * (j & 1));
      const float4 u0 = p[0], u1 = p[1], u2 = p[2], u3 = p[3];
      xs[j] = ((u0.x + u0.y) + (u0.z + u0.w)) + ((u1.x + u1.y) + (u1.z + u1.w)) +
              (((u2.x + u2.y) + (u2.z + u2.w)) + ((u3.x + u3.y) + (u3.z + u3.w)));
    }
    __syncthreads();
  }

  // ---- row tiles ----
  typename Epi::Wave ws;
  for (uint32_t tile = blockIdx.x * kWaves + wave; tile < a.ntiles; tile += gridDim.x * kWaves) {
    int rows[kR], segof[kR], segi = 0;
    if (a.paired) {
      constexpr int H = kR / 2;
#pragma unroll
      for (int r = 0; r < kR; r++) {
        const int s = r < H ? 0 : 1;
        const uint32_t row = tile * H + (r % H);
        segof[r] = s;
        rows[r] = row < a.seg[s].rows ? (int)row : -1;
      }
    } else {
      const uint32_t v0 = tile * kR;
      while (segi + 1 < a.nseg && v0 >= a.vbegin[segi + 1]) segi++;
#pragma unroll
      for (int r = 0; r < kR; r++) {
        const uint32_t row = v0 + r - a.vbegin[segi];
        segof[r] = segi;
        rows[r] = row < a.seg[segi].rows ? (int)row : -1;
      }
    }
    float acc[kR];
#pragma unroll
    for (int r = 0; r < kR; r++) acc[r] = 0.f;
    if (a.generic) tile_dot_generic(a.seg, segof, rows, xl, a.cols, lane, acc);
    else switch (a.seg[segi].type) {
      case T_Q4K: tile_dot<T_Q4K>(a.seg, segof, rows, xl, xs, a.groups, a.cols, lane, acc); break;
      case T_Q6K: tile_dot<T_Q6K>(a.seg, segof, rows, xl, xs, a.groups, a.cols, lane, acc); break;
      case T_Q8_0: tile_dot<T_Q8_0>(a.seg, segof, rows, xl, xs, a.groups, a.cols, lane, acc); break;
      case T_Q4_0: tile_dot<T_Q4_0>(a.seg, segof, rows, xl, xs, a.groups, a.cols, lane, acc); break;
      case T_Q8K: tile_dot<T_Q8K>(a.seg, segof, rows, xl, xs, a.groups, a.cols, lane, acc); break;
      case T_F32: tile_dot<T_F32>(a.seg, segof, rows, xl, xs, a.groups, a.cols, lane, acc); break;
      default: tile_dot<T_F16>(a.seg, segof, rows, xl, xs, a.groups, a.cols, lane, acc); break;
    }
#pragma unroll
    for (int r = 0; r < kR; r++) acc[r] = wave_sum(acc[r]);
    epi.apply(ws, segi, rows, segof, acc, lane);
  }
  epi.finish(ws, lane);
}

bool build_args(const GemvLaunch& L, KArgs* a) {
  if (L.nseg < 1 || L.nseg > 3 || L.cols == 0) return false;
  *a = KArgs{};
  a->nseg = L.nseg;
  a->paired = L.paired ? 1 : 0;
  a->cols = L.cols;
  a->generic = L.cols % 32 ? 1 : 0;
  a->groups = (L.cols + 31) / 32;
  a->x = L.x;
  a->norm_w = L.norm_w;
  a->eps = L.eps;
  uint32_t v = 0;
  for (int s = 0; s < L.nseg; s++) {
    a->seg[s] = L.seg[s];
    a->vbegin[s] = v;
    v += (L.seg[s].rows + kR - 1) / kR * kR;
    if ((L.seg[s].type == T_Q4K || L.seg[s].type == T_Q6K || L.seg[s].type == T_Q8K) && L.cols % 256)
      return false;
    if (a->generic && L.seg[s].type != T_F32 && L.seg[s].type != T_F16) return false;
  }
  a->vbegin[L.nseg] = v;
  if (L.paired) {
    if (L.nseg != 2 || L.seg[0].rows != L.seg[1].rows || L.seg[0].type != L.seg[1].type) return false;
    a->ntiles = (L.seg[0].rows + kR / 2 - 1) / (kR / 2);
  } else {
    a->ntiles = v / kR;
  }
  return true;
}

template <class Epi>
hipError_t launch(const GemvLaunch& L, const Epi& epi, hipStream_t st) {
  KArgs a;
  if (!build_args(L, &a)) return hipErrorInvalidValue;
  const size_t lds = (size_t)a.groups * kGroupStride * 4 + (size_t)(a.cols / 16) * 4;
  if (lds > 150 * 1024) return hipErrorInvalidValue;
  uint32_t blocks = (a.ntiles + kWaves - 1) / kWaves;
  if (blocks > 1024) blocks = 1024;
  if (blocks == 0) return hipSuccess;
  static bool lds_attr_set = false;  // rows of >16K columns need more than 64 KiB of LDS
  if (lds > 64 * 1024 && !lds_attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k_gemv<Epi>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       150 * 1024);
    if (e != hipSuccess) return e;
    lds_attr_set = true;
  }
  hipLaunchKernelGGL(k_gemv<Epi>, dim3(blocks), dim3(kThreads), lds, st, a, epi);
  return hipGetLastError();
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
