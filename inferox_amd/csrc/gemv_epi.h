// gemv_epi.h — row epilogues shared by the GEMV kernels (kern_gemv.hip,
// kern_gemv_mfma.hip).
//
// Per wave, a kernel calls begin(ws) once at its start (uniform state reads
// issued early), pre(ws, s, r) when it starts an item, on the lane that will
// own row r (global reads the epilogue needs, in flight while the item's
// weights are decoded), and row(ws, s, r, v, partner, pre) once per real row
// r of segment s of the finished item, on the lane that holds the row's sum v.
// `partner` is the sum of row r ^ 1 (kNeighbor: the RoPE pair) or, for paired
// launches, the second segment's sum of row r (gate/up).  finish(ws, lane)
// runs once per wave at the end of the kernel, on every lane.
// Compiled with -ffp-contract=off.
#pragma once

#include "kernels.h"

namespace ifx {

struct EpiStore {
  static constexpr bool kPaired = false, kNeighbor = false;
  float* y;
  uint32_t seg_out[3];  // output offset of each segment
  struct Wave {};
  struct Pre {};
  __device__ void begin(Wave&) const {}
  __device__ Pre pre(const Wave&, int, uint32_t) const { return Pre{}; }
  __device__ void row(Wave&, int s, uint32_t r, float v, float, const Pre&) const { y[seg_out[s] + r] = v; }
  __device__ void finish(Wave&, int) const {}
};

// Layer::decode_step residual adds (src/model/forward.rs:418,437).
struct EpiResidual {
  static constexpr bool kPaired = false, kNeighbor = false;
  float* h;
  struct Wave {};
  struct Pre {
    float h;
  };
  __device__ void begin(Wave&) const {}
  __device__ Pre pre(const Wave&, int, uint32_t r) const { return Pre{h[r]}; }
  __device__ void row(Wave&, int, uint32_t r, float v, float, const Pre& p) const { h[r] = v + p.h; }
  __device__ void finish(Wave&, int) const {}
};

// q / k with RoPE (src/ops.rs:273-284: x[2i] = a*cos - b*sin,
// x[2i+1] = a*sin + b*cos) and the K/V append at row state->len.
struct EpiQkv {
  static constexpr bool kPaired = false, kNeighbor = true;
  QkvEpi e;
  struct Wave {
    uint32_t len, pos;  // cache row of the new key/value, RoPE position
  };
  struct Pre {
    float2 cs;  // (cos, sin) of the row's RoPE pair, q and k rows inside rope_dim
  };
  __device__ void begin(Wave& w) const {
    w.len = e.state->len;
    w.pos = e.state->rope_pos;
  }
  __device__ Pre pre(const Wave& w, int s, uint32_t r) const {
    Pre p{make_float2(1.f, 0.f)};
    const uint32_t i = r % e.head_dim;
    if (s < 2 && i < e.rope_dim) p.cs = e.rope_cs[(uint64_t)w.pos * (e.rope_dim / 2) + i / 2];
    return p;
  }
  __device__ void row(Wave& w, int s, uint32_t r, float v, float other, const Pre& p) const {
    if (s < 2) {
      const uint32_t i = r % e.head_dim;
      if (i < e.rope_dim) {
        const float2 cs = p.cs;
        v = (i & 1) ? (other * cs.y + v * cs.x) : (v * cs.x - other * cs.y);
      }
    }
    if (s == 0) {
      e.q_out[r] = v;
    } else {
      const uint64_t off = ((uint64_t)(r / e.head_dim) * e.max_seq + w.len) * e.head_dim + r % e.head_dim;
      void* c = s == 1 ? e.k_cache : e.v_cache;
      if (e.kv_f16) ((_Float16*)c)[off] = (_Float16)v;  // round to nearest even
      else ((float*)c)[off] = v;
    }
  }
  __device__ void finish(Wave&, int) const {}
};

// swiglu (src/ops.rs:190-209): silu(g) * u with the sigmoid argument clamped to +-80.
struct EpiSwiglu {
  static constexpr bool kPaired = true, kNeighbor = false;
  float* mid;
  struct Wave {};
  struct Pre {};
  __device__ void begin(Wave&) const {}
  __device__ Pre pre(const Wave&, int, uint32_t) const { return Pre{}; }
  __device__ void row(Wave&, int, uint32_t r, float g, float u, const Pre&) const {
    float c = fminf(fmaxf(g, -80.f), 80.f);
    if (g != g) c = g;
    const float sig = 1.0f / (1.0f + expf(-c));
    mid[r] = (g * sig) * u;
  }
  __device__ void finish(Wave&, int) const {}
};

// Orders floats as unsigned keys; the low word carries the row, so the max
// key is the largest logit and, among equal logits, the last index
// (argmax, src/model/forward.rs:615-622).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | idx;
}

// Logits store + greedy argmax: each lane keeps the best key of its rows, the
// wave reduces once at the end and publishes with one atomicMax.
struct EpiLogits {
  static constexpr bool kPaired = false, kNeighbor = false;
  float* logits;
  DevState* state;
  struct Wave {
    unsigned long long best = 0;
    bool nan = false;
  };
  struct Pre {};
  __device__ void begin(Wave&) const {}
  __device__ Pre pre(const Wave&, int, uint32_t) const { return Pre{}; }
  __device__ void row(Wave& w, int, uint32_t r, float v, float, const Pre&) const {
    logits[r] = v;
    if (v != v) w.nan = true;
    const unsigned long long k = argmax_key(v, r);
    w.best = k > w.best ? k : w.best;
  }
  // Every wave of the workgroup calls finish once, at the kernel's end: the
  // waves' keys meet in LDS and the workgroup publishes one atomicMax.  With
  // one per wave, the thousands of waves of a short head launch (32000 rows of
  // 288 columns) queued their atomics on one address at once: the tiny
  // model's 128 greedy steps took 35.95 ms on the device, 34.94 ms now.
  __device__ void finish(Wave& w, int lane) const {
    unsigned long long b = w.best;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint32_t lo = __shfl_xor((uint32_t)b, off, 64), hi = __shfl_xor((uint32_t)(b >> 32), off, 64);
      const unsigned long long o = ((unsigned long long)hi << 32) | lo;
      b = o > b ? o : b;
    }
    const bool nan = __any(w.nan);
    constexpr int kMaxWaves = 16;
    __shared__ unsigned long long wbest[kMaxWaves];
    __shared__ int wnan[kMaxWaves];
    const int wave = (int)(threadIdx.x >> 6), nw = (int)((blockDim.x + 63) >> 6);
    if (lane == 0 && wave < kMaxWaves) {
      wbest[wave] = b;
      wnan[wave] = nan ? 1 : 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned long long m = 0;
      int any = 0;
      for (int i = 0; i < nw && i < kMaxWaves; i++) {
        m = wbest[i] > m ? wbest[i] : m;
        any |= wnan[i];
      }
      if (m) atomicMax(&state->argmax_key, m);
      if (any) atomicExch(&state->status, (int)IFX_E_NAN_LOGIT);
    }
  }
};

// The launcher of the int8-MFMA kernel for Q4_K / Q6_K segments
// (kern_gemv_mfma.hip), instantiated for the epilogues above.
template <class Epi>
hipError_t launch_mfma(const GemvLaunch& L, const Epi& epi, hipStream_t st);

bool mfma_type(uint32_t t);  // Q4_K and Q6_K: tiled device layout, MFMA GEMV



}  // namespace ifx
