// kern_sample.hip — temperature / top-k / top-p sampling of the next token on
// the device, for generate loops that do not take the greedy pick.
//
// Follows Sampler::sample (src/sampler.rs:28-76): p_i = exp(z_i / T)
// normalised over the vocabulary; top-k keeps the k most likely (ties in index
// order, the reference's stable sort); top-p then keeps the smallest prefix of
// that list, in decreasing probability, whose cumulative probability reaches
// top_p (the probabilities still normalised over the whole vocabulary); the
// draw is proportional to the kept probabilities.  It diverges from the
// reference on purpose in two places: the logits are shifted by their maximum
// before the exponential (the reference's exp(z / T) overflows for z / T > 88),
// and the uniform number comes from a counter-based generator (splitmix64 of
// seed and step) instead of the reference's thread_rng, so a run is
// reproducible from its seed.  Temperature 0 is the greedy argmax and does not
// run this kernel.
//
// One workgroup of 1024 threads; thread t owns the contiguous index range
// [t per, (t + 1) per) so that index order is thread order.  The k-th largest
// probability and the top-p threshold are found by a 4-pass radix select on
// the float bits (non-negative floats order as integers): counts for top-k,
// probability mass for top-p.
#include "kernels.h"

namespace ifx {

namespace {

constexpr int kT = 1024, kWaves = kT / 64;

struct Blk {
  float f[kWaves];
  uint32_t u[kWaves];
  uint32_t hc[256];
  float hm[256];
  uint32_t bc[4];
  float bf[4];
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ float block_sum(float v, Blk& b) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) b.f[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; w++) t += b.f[w];
  return t;
}
__device__ float block_max(float v, Blk& b) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) b.f[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; w++) t = fmaxf(t, b.f[w]);
  return t;
}
// exclusive prefix over thread order
__device__ uint32_t block_scan_u(uint32_t v, Blk& b) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) b.u[w] = x;
  __syncthreads();
  uint32_t base = 0;
  for (int i = 0; i < w; i++) base += b.u[i];
  return base + x - v;
}
__device__ float block_scan_f(float v, Blk& b) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) b.f[w] = x;
  __syncthreads();
  float base = 0.f;
  for (int i = 0; i < w; i++) base += b.f[i];
  return base + x - v;
}

// splitmix64 of (seed, counter) -> uniform [0, 1) with 24 bits
__device__ __forceinline__ float uniform01(uint64_t seed, uint64_t ctr) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (ctr + 1);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (float)(uint32_t)(z >> 40) * (1.0f / 16777216.0f);
}

// Radix select from the top over p[i0, i1) of this thread (keys: float bits).
// by_mass == false: the key of the rank-`target` largest element (1-based) and
// how many elements equal to it complete the rank; by_mass == true: the key at
// which the mass from the top first reaches `mass`, and the mass still missing
// at that key.
__device__ void radix_top(const float* p, uint32_t i0, uint32_t i1, bool by_mass, uint32_t target, float mass,
                          Blk& b, uint32_t& key, uint32_t& rem_count, float& rem_mass) {
  uint32_t prefix = 0, mask = 0, rc = target;
  float rm = mass;
  for (int sh = 24; sh >= 0; sh -= 8) {
    for (int i = threadIdx.x; i < 256; i += kT) {
      b.hc[i] = 0;
      b.hm[i] = 0.f;
    }
    __syncthreads();
    for (uint32_t i = i0; i < i1; i++) {
      const float v = p[i];
      const uint32_t k = __float_as_uint(v);
      if (v > 0.f && (k & mask) == prefix) {
        const uint32_t d = (k >> sh) & 255u;
        if (by_mass) atomicAdd(&b.hm[d], v);
        else atomicAdd(&b.hc[d], 1u);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t sel = 0, cum = 0;
      float cm = 0.f;
      for (int d = 255; d >= 0; d--) {
        if (by_mass) {
          if (cm + b.hm[d] >= rm || d == 0) {
            sel = (uint32_t)d;
            break;
          }
          cm += b.hm[d];
        } else {
          if (cum + b.hc[d] >= rc || d == 0) {
            sel = (uint32_t)d;
            break;
          }
          cum += b.hc[d];
        }
      }
      b.bc[0] = sel;
      b.bc[1] = rc - cum;
      b.bf[0] = rm - cm;
    }
    __syncthreads();
    prefix |= b.bc[0] << sh;
    mask |= 255u << sh;
    rc = b.bc[1];
    rm = b.bf[0];
    __syncthreads();
  }
  key = prefix;
  rem_count = rc;
  rem_mass = rm;
}

// keep p > key and the first `ties` elements equal to key (index order); zero the rest
__device__ void keep_top(float* p, uint32_t i0, uint32_t i1, uint32_t key, uint32_t ties, Blk& b) {
  uint32_t mine = 0;
  for (uint32_t i = i0; i < i1; i++) mine += (p[i] > 0.f && __float_as_uint(p[i]) == key) ? 1u : 0u;
  uint32_t rank = block_scan_u(mine, b);
  for (uint32_t i = i0; i < i1; i++) {
    const float v = p[i];
    if (!(v > 0.f)) continue;
    const uint32_t k = __float_as_uint(v);
    bool keep = k > key;
    if (k == key) keep = rank++ < ties;
    if (!keep) p[i] = 0.f;
  }
  __syncthreads();
}

__global__ void __launch_bounds__(kT) k_sample(const float* logits, float* p, uint32_t V, DevState* s) {
  __shared__ Blk b;
  __shared__ uint32_t pick;
  const float T = s->temperature;
  if (!(T > 0.f) || s->status != IFX_OK) return;  // greedy pick stands; a NaN is flagged by finalize
  const uint32_t per = (V + kT - 1) / kT;
  const uint32_t i0 = min(V, threadIdx.x * per), i1 = min(V, i0 + per);
  // temperature softmax with the maximum shifted out
  float m = -INFINITY;
  for (uint32_t i = i0; i < i1; i++) m = fmaxf(m, logits[i]);
  m = block_max(m, b);
  const float invT = 1.0f / T;
  float part = 0.f;
  for (uint32_t i = i0; i < i1; i++) {
    const float v = expf((logits[i] - m) * invT);
    p[i] = v;
    part += v;
  }
  const float S = block_sum(part, b);  // the reference's normaliser (up to the shift)
  __syncthreads();
  // top-k (src/sampler.rs:46-49)
  const uint32_t top_k = s->top_k;
  if (top_k > 0 && top_k < V) {
    uint32_t key, ties;
    float unused;
    radix_top(p, i0, i1, false, top_k, 0.f, b, key, ties, unused);
    keep_top(p, i0, i1, key, ties, b);
  }
  // top-p (src/sampler.rs:52-64): the prefix reaching top_p of the whole-vocabulary mass
  const float top_p = s->top_p;
  if (top_p < 1.0f) {
    part = 0.f;
    for (uint32_t i = i0; i < i1; i++) part += p[i];
    const float kept = block_sum(part, b);
    const float R = top_p * S;
    if (kept > R) {
      uint32_t key, unused;
      float rem;
      radix_top(p, i0, i1, true, 0u, fmaxf(R, 0.f), b, key, unused, rem);
      const float tau = __uint_as_float(key);
      uint32_t ties = tau > 0.f ? (uint32_t)ceilf(rem / tau) : 1u;
      ties = ties < 1u ? 1u : ties;
      keep_top(p, i0, i1, key, ties, b);
    }
  }
  // draw (src/sampler.rs:67-73), over the kept weights in index order
  part = 0.f;
  uint32_t last = 0;
  for (uint32_t i = i0; i < i1; i++) {
    part += p[i];
    if (p[i] > 0.f) last = i + 1;
  }
  const float W = block_sum(part, b);
  const float base = block_scan_f(part, b);
  const uint32_t last_all = (uint32_t)block_max((float)last, b);  // exact below 2^24
  if (threadIdx.x == 0) pick = last_all > 0 ? last_all - 1 : 0u;
  __syncthreads();
  const float target = uniform01(s->seed, s->step) * W;
  if (part > 0.f && base <= target && target < base + part) {
    float acc = base;
    for (uint32_t i = i0; i < i1; i++) {
      acc += p[i];
      if (p[i] > 0.f && target < acc) {
        pick = i;
        break;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) s->argmax_key = (unsigned long long)pick;
}

}  // namespace

hipError_t launch_sample(const float* logits, float* probs, uint32_t vocab, DevState* state, hipStream_t st) {
  if (vocab == 0 || vocab >= (1u << 24)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sample, dim3(1), dim3(kT), 0, st, logits, probs, vocab, state);
  return hipGetLastError();
}

}  // namespace ifx
