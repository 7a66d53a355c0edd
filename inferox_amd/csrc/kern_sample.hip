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
// Three launches per draw:
//   k_sample_weights (64 workgroups of 1024 threads, each a contiguous index
//     range): p_i = exp((z_i - m) / T), m the maximum logit the head's argmax
//     left in state->argmax_key; each workgroup's sum of p (the normaliser S
//     is their sum in one fixed order); a histogram of p by exponent and four
//     significand bits, counts and mass lower bounds, merged with integer
//     atomics (the same in any order).
//   k_sample_gather (256 workgroups): each computes the same plan from the
//     histogram.  With neither top-k nor top-p, the workgroup holding the
//     draw walks its range: the draw over the whole vocabulary in index
//     order, the reference's order for an unsorted list.  Otherwise every
//     element in the bins that can hold a kept one (the bin where the count
//     from the top reaches k, the bin where the mass reaches top_p S) goes to
//     a candidate list.
//   k_sample_select (one workgroup): the candidates sorted by decreasing p,
//     ties in index order, in LDS; top-k, top-p, and the draw walking the kept
//     list in that order, as the reference walks its sorted list.  With more
//     candidates than the sort holds (draw_many), only the bins that can hold
//     the last kept entry are gathered and sorted, and the draw walks the kept
//     set in index order (the same distribution in another order).  When
//     those bins alone exceed the sort (equal logits), the single-workgroup
//     draw below (sample_one_wg) runs from the logits: thread t owns the index
//     range [t per, (t + 1) per) so that index order is thread order, and the
//     k-th largest probability and the top-p threshold come from a 4-pass
//     radix select on the float bits (non-negative floats order as integers).
// One workgroup swept the vocabulary by itself for every draw before: 1.14 ms
// of a sampled 8B step at 128256 entries.
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

// The whole draw in one workgroup of kT threads, from the logits: the
// last resort of k_sample_select, when the bins that can hold the last kept
// entry alone hold more than kCap entries.
__device__ void sample_one_wg(const float* logits, float* p, uint32_t V, DevState* s) {
  __shared__ Blk b;
  __shared__ uint32_t pick;
  const float T = s->temperature;
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

// ---- the multi-workgroup draw ----

// k_sample_weights: kWG workgroups of kWT threads, workgroup w the index range
// [w per, (w + 1) per), per = ceil(V / kWG); part[w] its sum.  Fewer, larger
// workgroups merge fewer partial histograms with global atomics: at 128256
// entries of logits ~ N(0, 16), T 0.8, the launch takes 11 us with 256
// workgroups of 256 threads, 5 us with 64 of 1024.
constexpr int kWG = 64, kWT = 1024;
// k_sample_gather (and k_logits_max): kG workgroups of kST threads.
constexpr int kG = 256, kST = 256;
static_assert(kWG <= kST && kWG <= kG, "the plan scans the sums one per thread; a gather workgroup walks each range");
constexpr int kSW = kST / 64;
// Probability bins: bin 0 holds 0 < p < 2^-32; bin 1 + 16 (e - 95) + (the top
// four significand bits) holds 2^-32 <= p <= 1 of biased exponent e, so the
// bins order as the values do and equal values share one.
constexpr uint32_t kBins = 1u + 16u * 32u + 1u;   // p = 1 is bin 513
constexpr uint32_t kBinBase = (127u - 32u) << 4;  // the float bits >> 19 of 2^-32
// A bin's count (bits 63:40) and mass (bits 39:0: its elements' significands
// truncated to 16 bits, in units of 2^(e - 142)) in one 64-bit word: fewer
// than 2^24 elements of less than 2^16 each fit in the 40 bits.
constexpr int kCountShift = 40;
constexpr unsigned long long kMassMask = (1ull << kCountShift) - 1;
constexpr uint32_t kCap = 4096;  // candidates k_sample_select sorts in LDS
constexpr uint32_t kNone = 0xffffffffu;
enum : uint32_t { kModeAll = 1, kModeCand = 2, kModeMany = 3 };

constexpr size_t kOffHist = 0;
constexpr size_t kOffPart = (kOffHist + kBins * 8 + 255) & ~size_t(255);
constexpr size_t kOffCand = (kOffPart + kWG * 4 + 255) & ~size_t(255);
constexpr size_t kOffCtl = (kOffCand + kCap * 8 + 255) & ~size_t(255);
constexpr size_t kWsBytes = kOffCtl + 256;

__device__ __forceinline__ uint32_t bin_of(uint32_t bits) {
  const uint32_t b = bits >> 19;
  return b < kBinBase ? 0u : min(b - kBinBase + 1u, kBins - 1u);
}
__device__ __forceinline__ unsigned long long bin_entry(uint32_t bits) {
  return (1ull << kCountShift) | (((bits & 0x7fffffu) | 0x800000u) >> 8);
}
// A lower bound of bin b's probability mass (bin 0: none).
__device__ __forceinline__ double bin_mass(uint32_t b, unsigned long long h) {
  if (b == 0) return 0.0;
  return ldexp((double)(h & kMassMask), 95 + (int)((b - 1) >> 4) - 142);
}

// Exclusive prefix of v over the threads of a workgroup of NW waves, in thread
// order; total: the sum over all threads (the same bits in every thread).  wt:
// NW slots of LDS.
template <int NW, class T>
__device__ T wg_scan(T v, T* wt, T& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  T x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  T ex = __shfl_up(x, 1, 64);
  if (lane == 0) ex = T(0);
  __syncthreads();
  if (lane == 63) wt[w] = x;
  __syncthreads();
  T base = T(0), all = T(0);
#pragma unroll
  for (int i = 0; i < NW; i++) {
    if (i < w) base += wt[i];
    all += wt[i];
  }
  total = all;
  return base + ex;
}

// The normaliser S: the kWG workgroup sums added in one fixed order.  Called
// by the first wave of a workgroup; every caller gets the same bits.
__device__ float part_total(const float* part) {
  float v = 0.f;
  for (int i = (int)(threadIdx.x & 63); i < kWG; i += 64) v += part[i];
  return wave_sum(v);
}

// The wave's lowest / highest lane with pred set (false in every other lane).
// Where values ascend with the lane, the one lane that publishes the wave's
// minimum / maximum: one LDS atomic per wave instead of one per lane (same-
// address LDS atomics serialise; one per lane cost the gather 18 us).
__device__ __forceinline__ bool lowest_lane(bool pred) {
  const unsigned long long b = __ballot(pred);
  return b && (threadIdx.x & 63) == (unsigned)(__ffsll((long long)b) - 1);
}
__device__ __forceinline__ bool highest_lane(bool pred) {
  const unsigned long long b = __ballot(pred);
  return b && (threadIdx.x & 63) == (unsigned)(63 - __clzll((long long)b));
}

__device__ __forceinline__ unsigned long long order_key(float v, uint32_t idx) {
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | idx;
}

// The weights p_i = exp((z_i - m) / T) of workgroup w's index range, with m
// the maximum logit (state->argmax_key), their sum, and the histogram.
__global__ void __launch_bounds__(kWT) k_sample_weights(const float* __restrict__ logits, float* __restrict__ p,
                                                        SampleWs ws, uint32_t V, const DevState* __restrict__ s) {
  constexpr int kW = kWT / 64;
  __shared__ unsigned long long lh[kBins];
  __shared__ float wsum[kW];
  __shared__ uint32_t wlow[kW];
  const float T = s->temperature;
  if (!(T > 0.f) || s->status != IFX_OK) return;  // the greedy pick stands; finalize flags a NaN
  const uint32_t hi = (uint32_t)(s->argmax_key >> 32);
  const float m = __uint_as_float((hi & 0x80000000u) ? (hi & 0x7fffffffu) : ~hi);
  const float invT = 1.0f / T;
  for (uint32_t b = threadIdx.x; b < kBins; b += kWT) lh[b] = 0ull;
  __syncthreads();
  const uint32_t per = (V + kWG - 1) / kWG, i0 = min(V, blockIdx.x * per), i1 = min(V, i0 + per);
  float part = 0.f;
  uint32_t low = 0;
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += kWT) {
    const float v = expf((logits[i] - m) * invT);
    p[i] = v;
    part += v;
    if (v > 0.f) {
      const uint32_t bits = __float_as_uint(v), b = bin_of(bits);
      if (b == 0) low++;  // counted, not binned: most of a vocabulary lands here
      else atomicAdd(&lh[b], bin_entry(bits));
    }
  }
  part = wave_sum(part);
  low = wave_sum_u(low);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    wsum[w] = part;
    wlow[w] = low;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    uint32_t n = 0;
    for (int i = 0; i < kW; i++) {
      t += wsum[i];
      n += wlow[i];
    }
    ws.part[blockIdx.x] = t;
    if (n) atomicAdd(&ws.hist[0], (unsigned long long)n << kCountShift);
  }
  for (uint32_t b = 1 + threadIdx.x; b < kBins; b += kWT) {
    const unsigned long long h = lh[b];
    if (h) atomicAdd(&ws.hist[b], h);
  }
}

struct Plan {
  uint32_t mode, lo_bin, n;
  float S;
};

// The draw's plan, alike in every workgroup of kST threads (a function of the
// histogram, the workgroup sums and the sampler settings).  With top-k and/or
// top-p: the lowest bin that can hold a kept element and the count of
// elements at or above it.  Top-k needs the bin where the count from the top
// reaches k; top-p the bin where the mass from the top reaches top_p S, with
// the masses' lower bounds and a margin of 2^-9 over the rounding of the
// select's float running sum, so that its cut falls among the candidates.
__device__ Plan make_plan(const SampleWs& ws, uint32_t V, const DevState* s) {
  __shared__ uint32_t wt_u[kSW];
  __shared__ double wt_d[kSW];
  __shared__ uint32_t first[3];
  __shared__ uint32_t n_at;
  __shared__ float S_sh;
  const uint32_t top_k = s->top_k;
  const float top_p = s->top_p;
  bool kon = top_k > 0 && top_k < V;
  const bool pon = top_p < 1.0f;
  if (threadIdx.x < 64) {
    const float S = part_total(ws.part);
    if (threadIdx.x == 0) S_sh = S;
  }
  if (threadIdx.x < 3) first[threadIdx.x] = kNone;
  __syncthreads();
  Plan pl{kModeAll, 0u, 0u, S_sh};
  if (!kon && !pon) return pl;
  // thread t: the bins at descending positions j = 3t .. 3t + 2 (bin kBins - 1 - j)
  constexpr uint32_t kPer = (kBins + kST - 1) / kST;
  uint32_t cnt[kPer];
  double mass[kPer];
  uint32_t ct = 0;
  double mt = 0.0;
#pragma unroll
  for (uint32_t q = 0; q < kPer; q++) {
    const uint32_t j = threadIdx.x * kPer + q;
    cnt[q] = 0;
    mass[q] = 0.0;
    if (j < kBins) {
      const uint32_t b = kBins - 1 - j;
      const unsigned long long h = ws.hist[b];
      cnt[q] = (uint32_t)(h >> kCountShift);
      mass[q] = bin_mass(b, h);
    }
    ct += cnt[q];
    mt += mass[q];
  }
  uint32_t ctot;
  double mtot;
  const uint32_t c0 = wg_scan<kSW>(ct, wt_u, ctot);
  const double m0 = wg_scan<kSW>(mt, wt_d, mtot);
  // a top-k of at least every positive weight keeps them all (zero weights
  // are never drawn): no filter
  if (kon && top_k >= ctot) kon = false;
  if (!kon && !pon) return pl;
  const double R = (double)top_p * (double)pl.S * (1.0 + 1.0 / 512);
  // each predicate's first position in this thread (they hold from there on);
  // positions ascend with the lane, so a wave's first is its lowest such lane
  uint32_t c = c0;
  double mm = m0;
  uint32_t fj[3] = {kNone, kNone, kNone};
#pragma unroll
  for (uint32_t q = 0; q < kPer; q++) {
    const uint32_t j = threadIdx.x * kPer + q;
    if (j < kBins) {
      c += cnt[q];
      mm += mass[q];
      if (kon && c >= top_k) fj[0] = min(fj[0], j);
      if (c >= 1) fj[1] = min(fj[1], j);
      if (mm >= R) fj[2] = min(fj[2], j);
    }
  }
#pragma unroll
  for (int f = 0; f < 3; f++)
    if (lowest_lane(fj[f] != kNone)) atomicMin(&first[f], fj[f]);
  __syncthreads();
  // the kept list is the shorter of the two prefixes: its last element lies
  // at or above the higher of the two bins (the smaller position)
  const uint32_t last = kBins - 1;
  const uint32_t jk = kon ? min(first[0], last) : last;
  const uint32_t jp = pon ? max(min(first[2], last), min(first[1], last)) : last;
  const uint32_t lo = min(jk, jp);
  if (threadIdx.x == lo / kPer) {
    uint32_t x = c0;
#pragma unroll
    for (uint32_t q = 0; q < kPer; q++)
      if (q <= lo % kPer) x += cnt[q];
    n_at = x;
  }
  __syncthreads();
  pl.lo_bin = last - lo;
  pl.n = n_at;
  pl.mode = pl.n <= kCap ? kModeCand : kModeMany;
  return pl;
}

// Neither top-k nor top-p: the draw over the whole vocabulary in index order.
// The sums of the weights kernel's ranges locate the range holding target =
// u S; gather workgroup w walks range w (threads own consecutive sub-ranges,
// so index order is thread order).  Rounding that leaves the target past
// every sum takes the last positive weight.
__device__ void draw_all(const float* p, const SampleWs& ws, uint32_t V, DevState* s, float S) {
  __shared__ float wt_f[kSW];
  __shared__ uint32_t sel[2];
  __shared__ float base_w;
  __shared__ uint32_t found, lastpos;
  const float target = uniform01(s->seed, s->step) * S;
  const float mine = threadIdx.x < kWG ? ws.part[threadIdx.x] : 0.f;
  float tot;
  const float ex = wg_scan<kSW>(mine, wt_f, tot);
  if (threadIdx.x == 0) {
    sel[0] = kNone;
    sel[1] = 0u;
    found = kNone;
    lastpos = 0;
  }
  __syncthreads();
  if (lowest_lane(mine > 0.f && target < ex + mine)) atomicMin(&sel[0], threadIdx.x);
  if (highest_lane(mine > 0.f)) atomicMax(&sel[1], threadIdx.x + 1);
  __syncthreads();
  const uint32_t w = sel[0] != kNone ? sel[0] : (sel[1] ? sel[1] - 1 : kNone);
  if (w != blockIdx.x) return;
  if (threadIdx.x == w) base_w = ex;
  __syncthreads();
  const float tl = target - base_w;
  const uint32_t per = (V + kWG - 1) / kWG, i0 = min(V, w * per), i1 = min(V, i0 + per);
  const uint32_t q = (i1 - i0 + kST - 1) / kST;
  const uint32_t a0 = min(i1, i0 + threadIdx.x * q), a1 = min(i1, a0 + q);
  float sum = 0.f;
  uint32_t lp = 0;
  for (uint32_t i = a0; i < a1; i++) {
    const float v = p[i];
    sum += v;
    if (v > 0.f) lp = i + 1;
  }
  float unused;
  const float b = wg_scan<kSW>(sum, wt_f, unused);
  if (highest_lane(lp != 0)) atomicMax(&lastpos, lp);
  uint32_t hit = kNone;
  if (sum > 0.f && b <= tl && tl < b + sum) {
    float acc = b;
    for (uint32_t i = a0; i < a1; i++) {
      const float v = p[i];
      acc += v;
      if (v > 0.f && tl < acc) {
        hit = i;
        break;
      }
    }
  }
  if (lowest_lane(hit != kNone)) atomicMin(&found, hit);
  __syncthreads();
  if (threadIdx.x == 0 && (found != kNone || lastpos)) s->argmax_key = found != kNone ? found : lastpos - 1;
}

// The candidates (p > 0 in bins at or above lo_bin) of this workgroup's range
// appended to ws.cand; one atomic per workgroup.
__device__ void gather(const float* p, const SampleWs& ws, uint32_t V, uint32_t lo_bin) {
  __shared__ uint32_t wt_u[kSW];
  __shared__ uint32_t at0;
  const uint32_t per = (V + kG - 1) / kG, i0 = min(V, blockIdx.x * per), i1 = min(V, i0 + per);
  uint32_t n = 0;
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += kST) {
    const float v = p[i];
    n += (v > 0.f && bin_of(__float_as_uint(v)) >= lo_bin) ? 1u : 0u;
  }
  uint32_t tot;
  uint32_t at = wg_scan<kSW>(n, wt_u, tot);
  if (tot == 0) return;
  if (threadIdx.x == 0) at0 = atomicAdd(&ws.ctl->count, tot);
  __syncthreads();
  at += at0;
  if (n == 0) return;
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += kST) {
    const float v = p[i];
    const uint32_t bits = __float_as_uint(v);
    if (v > 0.f && bin_of(bits) >= lo_bin) {
      if (at < kCap) ws.cand[at] = make_uint2(i, bits);
      at++;
    }
  }
}

__global__ void __launch_bounds__(kST) k_sample_gather(const float* __restrict__ p, SampleWs ws, uint32_t V,
                                                       DevState* s) {
  const float T = s->temperature;
  if (!(T > 0.f) || s->status != IFX_OK) return;
  const Plan pl = make_plan(ws, V, s);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    ws.ctl->mode = pl.mode;
    ws.ctl->lo_bin = pl.lo_bin;
    ws.ctl->n_cand = pl.n;
  }
  if (pl.mode == kModeAll) draw_all(p, ws, V, s, pl.S);
  else if (pl.mode == kModeCand) gather(p, ws, V, pl.lo_bin);
}

// Ascending bitonic sort of a[0, n) in LDS, n a power of two.
__device__ void bitonic(unsigned long long* a, uint32_t n) {
  for (uint32_t k = 2; k <= n; k <<= 1)
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      for (uint32_t t = threadIdx.x; t < n / 2; t += kT) {
        const uint32_t i = 2 * t - (t & (j - 1)), l = i + j;
        const unsigned long long x = a[i], y = a[l];
        if ((x > y) == ((i & k) == 0)) {
          a[i] = y;
          a[l] = x;
        }
      }
      __syncthreads();
    }
}

// Ascending sort of the distinct keys a[0, n), n <= kCap.  Up to kT keys by
// rank: each thread counts the keys below its own and stores it there, with
// one barrier where the bitonic network has log2(n) (log2(n) + 1) / 2 (13.5 us
// for 92 candidates that way, the barriers of 16 waves).  A wave takes the
// keys 64 at a time into registers and broadcasts them lane by lane
// (readlane), so the count runs without LDS round trips.  More keys: the
// bitonic network over the next power of two, padded with ~0.
__device__ void sort_keys(unsigned long long* a, uint32_t n) {
  if (n <= (uint32_t)kT) {
    const uint32_t lane = threadIdx.x & 63, wave0 = threadIdx.x & ~63u;
    unsigned long long mine = 0;
    uint32_t r = 0;
    if (wave0 < n) {
      mine = threadIdx.x < n ? a[threadIdx.x] : ~0ull;
      for (uint32_t c0 = 0; c0 < n; c0 += 64) {
        const unsigned long long kv = c0 + lane < n ? a[c0 + lane] : ~0ull;
        const int klo = (int)(uint32_t)kv, khi = (int)(uint32_t)(kv >> 32);
#pragma unroll 16
        for (int l = 0; l < 64; l++) {
          const unsigned long long o = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane(khi, l) << 32) |
                                       (uint32_t)__builtin_amdgcn_readlane(klo, l);
          r += o < mine ? 1u : 0u;
        }
      }
    }
    __syncthreads();
    if (threadIdx.x < n) a[r] = mine;
    __syncthreads();
    return;
  }
  uint32_t np2 = 1;
  while (np2 < n) np2 <<= 1;
  for (uint32_t j = n + threadIdx.x; j < np2; j += kT) a[j] = ~0ull;
  __syncthreads();
  bitonic(a, np2);
}

// The thread's consecutive share [a0, a1) of n positions.
__device__ __forceinline__ void share(uint32_t n, uint32_t& a0, uint32_t& a1) {
  const uint32_t q = (n + kT - 1) / kT;
  a0 = min(n, threadIdx.x * q);
  a1 = min(n, a0 + q);
}

// The draw from a sorted candidate list key[0, n) (keys (~p bits) << 32 |
// index, ascending: p descending, ties by index, the reference's stable
// sort): top-k, then top-p, the first position whose running sum reaches
// top_p S; the draw over the kept prefix in that order, as the reference's
// WeightedIndex walks its sorted, truncated list.
__device__ void draw_sorted(const unsigned long long* key, uint32_t n, float S, DevState* s) {
  __shared__ float wt_f[kWaves];
  __shared__ uint32_t cut, found;
  if (threadIdx.x == 0) {
    cut = kNone;
    found = kNone;
  }
  __syncthreads();
  uint32_t kept = n;
  const uint32_t top_k = s->top_k;
  if (top_k > 0 && top_k < kept) kept = top_k;
  const float top_p = s->top_p;
  if (top_p < 1.0f) {
    const float R = top_p * S;
    uint32_t a0, a1;
    share(kept, a0, a1);
    float sum = 0.f;
    for (uint32_t j = a0; j < a1; j++) sum += __uint_as_float(~(uint32_t)(key[j] >> 32));
    float unused;
    float acc = wg_scan<kWaves>(sum, wt_f, unused);
    uint32_t hit = kNone;
    for (uint32_t j = a0; j < a1; j++) {
      acc += __uint_as_float(~(uint32_t)(key[j] >> 32));
      if (acc >= R) {
        hit = j;
        break;
      }
    }
    if (lowest_lane(hit != kNone)) atomicMin(&cut, hit);
    __syncthreads();
    if (cut != kNone) kept = cut + 1;
  }
  uint32_t a0, a1;
  share(kept, a0, a1);
  float sum = 0.f;
  for (uint32_t j = a0; j < a1; j++) sum += __uint_as_float(~(uint32_t)(key[j] >> 32));
  float W;
  const float base = wg_scan<kWaves>(sum, wt_f, W);
  const float target = uniform01(s->seed, s->step) * W;
  uint32_t hit = kNone;
  if (sum > 0.f && base <= target && target < base + sum) {
    float acc = base;
    for (uint32_t j = a0; j < a1; j++) {
      const float v = __uint_as_float(~(uint32_t)(key[j] >> 32));
      acc += v;
      if (v > 0.f && target < acc) {
        hit = j;
        break;
      }
    }
  }
  if (lowest_lane(hit != kNone)) atomicMin(&found, hit);
  __syncthreads();
  if (threadIdx.x == 0) s->argmax_key = key[found != kNone ? found : kept - 1] & 0xffffffffull;
}

constexpr uint32_t kRow = 4096;  // entries of one row of the index-order draw (16 float4 per lane of a wave)
static_assert(((1u << 24) / kRow) * 4 <= kCap * 8, "the row sums fit where the candidate keys were");

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ unsigned long long sample_key(uint32_t bits, uint32_t i) {
  return ((unsigned long long)(~bits) << 32) | i;
}
// the weight of entry i in the draw over the kept set {key <= kstar}
__device__ __forceinline__ float kept_w(float v, uint32_t i, unsigned long long kstar) {
  return (v > 0.f && sample_key(__float_as_uint(v), i) <= kstar) ? v : 0.f;
}

// More candidates than the sort holds (a flat distribution with top-p near 1,
// a large top-k): the kept set is every entry whose key is at most the last
// kept one's, K*, and only the entries of the bins that can hold that one are
// sorted.  From the histogram: the top-k bin (exact counts) and the bins
// between which the top-p boundary lies (the mass lower bounds, and those plus
// one significand unit per entry).  One sweep over p gathers those bins'
// entries and sums in double the mass of every entry above them; the gathered
// ones are sorted and cut (top-k by count, top-p by the running sum from that
// mass).  The draw walks the kept set in index order: each wave sums whole
// 4096-entry rows, the workgroup finds the row holding u W, and one wave walks
// that row.  The reference walks its sorted list instead: the same
// distribution.  Returns false when the boundary bins alone hold more than
// kCap entries.
__device__ bool draw_many(const float* p, const SampleWs& ws, uint32_t V, float S, DevState* s,
                          unsigned long long* key) {
  __shared__ uint32_t wt_u[kWaves];
  __shared__ double wt_d[kWaves];
  __shared__ float wt_f[kWaves];
  __shared__ uint32_t fj[4];
  __shared__ uint32_t c_above, c_incl, n_g;
  __shared__ double m_above;
  __shared__ uint32_t cut;
  __shared__ unsigned long long kstar, rowpick;
  __shared__ uint32_t found, lastpos;
  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t top_k = s->top_k;
  const float top_p = s->top_p;
  const bool kon = top_k > 0 && top_k < V, pon = top_p < 1.0f;
  const double R = (double)(top_p * S);
  // bins in descending positions j = tid (bin kBins - 1 - j)
  const uint32_t j = (uint32_t)tid;
  const bool in = j < kBins;
  uint32_t c = 0;
  double lm = 0.0, um = 0.0;
  if (in) {
    const uint32_t b = kBins - 1 - j;
    const unsigned long long h = ws.hist[b];
    c = (uint32_t)(h >> kCountShift);
    lm = bin_mass(b, h);
    um = lm + (double)c * (b == 0 ? ldexp(1.0, -32) : ldexp(1.0, 95 + (int)((b - 1) >> 4) - 142));
  }
  uint32_t ctot;
  double ltot, utot;
  const uint32_t cex = wg_scan<kWaves>(c, wt_u, ctot);
  const double lex = wg_scan<kWaves>(lm, wt_d, ltot);
  const double uex = wg_scan<kWaves>(um, wt_d, utot);
  if (tid < 4) fj[tid] = kNone;
  if (tid == 0) {
    n_g = 0;
    cut = kNone;
    found = kNone;
    lastpos = 0;
    rowpick = ~0ull;
  }
  __syncthreads();
  if (lowest_lane(in && kon && cex + c >= top_k)) atomicMin(&fj[0], j);
  if (lowest_lane(in && pon && lex + lm >= R * (1.0 + 1e-9))) atomicMin(&fj[1], j);
  if (lowest_lane(in && pon && uex + um >= R * (1.0 - 1e-9))) atomicMin(&fj[2], j);
  if (lowest_lane(in && cex + c >= 1)) atomicMin(&fj[3], j);
  __syncthreads();
  const uint32_t last = kBins - 1, j1 = min(fj[3], last);
  const uint32_t jk = kon ? min(fj[0], last) : last;
  const uint32_t jl = pon ? max(min(fj[1], last), j1) : last;  // the top-p boundary lies at or above it
  const uint32_t ju = pon ? max(min(fj[2], last), j1) : last;  // ... and at or below this one
  const uint32_t ja = min(jk, ju), jb = min(jk, jl);
  if (in && j == ja) c_above = cex;
  if (in && j == jb) c_incl = cex + c;
  __syncthreads();
  const uint32_t n = c_incl - c_above;
  if (n == 0 || n > kCap) return false;
  const uint32_t blo = last - jb, bhi = last - ja;

  // gather bins [blo, bhi]; the mass above them.  A wave covers 256
  // consecutive entries per load, kBatch loads in flight per lane.
  constexpr uint32_t kBatch = 8;
  double above = 0.0;
  for (uint32_t w0 = 4u * (uint32_t)(tid & ~63); w0 < V; w0 += 4u * kT * kBatch) {  // uniform in the wave
    float4 q[kBatch];
#pragma unroll
    for (uint32_t u = 0; u < kBatch; u++) {
      const uint32_t i0 = w0 + 4u * kT * u + 4u * (uint32_t)lane;
      if (i0 + 3 < V) {
        q[u] = *(const float4*)(p + i0);
      } else {
        q[u].x = i0 < V ? p[i0] : 0.f;
        q[u].y = i0 + 1 < V ? p[i0 + 1] : 0.f;
        q[u].z = i0 + 2 < V ? p[i0 + 2] : 0.f;
        q[u].w = 0.f;
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < kBatch; u++) {
      const uint32_t i0 = w0 + 4u * kT * u + 4u * (uint32_t)lane;
      const float v[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
      uint32_t mine = 0;
      bool take[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t b = bin_of(__float_as_uint(v[e]));
        take[e] = v[e] > 0.f && b >= blo && b <= bhi;
        if (v[e] > 0.f && b > bhi) above += (double)v[e];
        mine += take[e] ? 1u : 0u;
      }
      if (!__any(mine != 0)) continue;
      uint32_t x = mine;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
      }
      uint32_t base = 0;
      if (lane == 63) base = atomicAdd(&n_g, x);
      base = __shfl(base, 63, 64);
      uint32_t at = base + x - mine;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        if (take[e]) {
          if (at < kCap) key[at] = sample_key(__float_as_uint(v[e]), i0 + (uint32_t)e);
          at++;
        }
      }
    }
  }
  above = wave_sum_d(above);
  if (lane == 0) wt_d[wave] = above;
  __syncthreads();
  if (tid == 0) {
    double t = 0.0;
    for (int w = 0; w < kWaves; w++) t += wt_d[w];
    m_above = t;
  }
  const uint32_t ng = min(n_g, kCap);
  if (ng == 0) return false;
  sort_keys(key, ng);  // ends with a barrier
  // top-k by count, then top-p by the running sum from the mass above
  uint32_t kept = ng;
  if (kon) kept = c_above < top_k ? min(kept, top_k - c_above) : 1u;
  if (pon) {
    uint32_t a0, a1;
    share(kept, a0, a1);
    double sum = 0.0;
    for (uint32_t q = a0; q < a1; q++) sum += (double)__uint_as_float(~(uint32_t)(key[q] >> 32));
    double unused;
    double acc = m_above + wg_scan<kWaves>(sum, wt_d, unused);
    uint32_t hit = kNone;
    for (uint32_t q = a0; q < a1; q++) {
      acc += (double)__uint_as_float(~(uint32_t)(key[q] >> 32));
      if (acc >= R) {
        hit = q;
        break;
      }
    }
    if (lowest_lane(hit != kNone)) atomicMin(&cut, hit);
    __syncthreads();
    if (cut != kNone) kept = min(kept, cut + 1);
  }
  if (tid == 0) kstar = key[kept - 1];
  __syncthreads();
  const unsigned long long ks = kstar;

  // row sums of the kept weights (rows of kRow entries, one wave per row)
  float* rowsum = (float*)key;
  const uint32_t rows = (V + kRow - 1) / kRow;
  for (uint32_t r = (uint32_t)wave; r < rows; r += kWaves) {
    float sum = 0.f;
#pragma unroll
    for (uint32_t q = 0; q < kRow / 256; q++) {
      const uint32_t i0 = r * kRow + 256 * q + 4 * (uint32_t)lane;
      if (i0 + 3 < V) {
        const float4 v = *(const float4*)(p + i0);
        sum += kept_w(v.x, i0, ks) + kept_w(v.y, i0 + 1, ks) + kept_w(v.z, i0 + 2, ks) + kept_w(v.w, i0 + 3, ks);
      } else {
        for (uint32_t e = 0; e < 4; e++)
          if (i0 + e < V) sum += kept_w(p[i0 + e], i0 + e, ks);
      }
    }
    sum = wave_sum(sum);
    if (lane == 0) rowsum[r] = sum;
  }
  __syncthreads();
  // the row holding target = u W (thread t: rows [t q, (t + 1) q))
  uint32_t r0, r1;
  share(rows, r0, r1);
  float rs = 0.f;
  uint32_t lastrow = 0;
  for (uint32_t r = r0; r < r1; r++) {
    rs += rowsum[r];
    if (rowsum[r] > 0.f) lastrow = r + 1;
  }
  float W;
  const float rb = wg_scan<kWaves>(rs, wt_f, W);
  const float target = uniform01(s->seed, s->step) * W;
  unsigned long long pickrow = ~0ull;
  if (rs > 0.f && rb <= target && target < rb + rs) {
    float acc = rb;
    for (uint32_t r = r0; r < r1; r++) {
      if (rowsum[r] > 0.f && target < acc + rowsum[r]) {
        pickrow = ((unsigned long long)r << 32) | __float_as_uint(target - acc);
        break;
      }
      acc += rowsum[r];
    }
  }
  if (lowest_lane(pickrow != ~0ull)) atomicMin(&rowpick, pickrow);
  if (highest_lane(lastrow != 0)) atomicMax(&lastpos, lastrow);
  __syncthreads();
  if (rowpick == ~0ull && lastpos == 0) return true;  // no kept weight (not reached: K* is kept)
  // the walk: wave 0 over the row, lane l its entries [64 l, 64 l + 64)
  const bool fallback = rowpick == ~0ull;
  const uint32_t prow = fallback ? lastpos - 1 : (uint32_t)(rowpick >> 32);
  const float tl = fallback ? INFINITY : __uint_as_float((uint32_t)rowpick);
  if (wave == 0) {
    const uint32_t a0 = min(V, prow * kRow + 64 * (uint32_t)lane), a1 = min(V, a0 + 64);
    float ls = 0.f;
    uint32_t lp = 0;
    if (a1 - a0 == 64) {
      float4 q[16];
#pragma unroll
      for (int u = 0; u < 16; u++) q[u] = *(const float4*)(p + a0 + 4 * u);
#pragma unroll
      for (int u = 0; u < 16; u++) {
        const float v[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t i = a0 + 4 * u + e;
          const float w = kept_w(v[e], i, ks);
          ls += w;
          if (w > 0.f) lp = i + 1;
        }
      }
    } else {
      for (uint32_t i = a0; i < a1; i++) {
        const float w = kept_w(p[i], i, ks);
        ls += w;
        if (w > 0.f) lp = i + 1;
      }
    }
    float x = ls;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    const float ex = x - ls;
    uint32_t hit = kNone;
    if (ls > 0.f && ex <= tl && tl < ex + ls) {
      float acc = ex;
      for (uint32_t i = a0; i < a1; i++) {
        const float w = kept_w(p[i], i, ks);
        acc += w;
        if (w > 0.f && tl < acc) {
          hit = i;
          break;
        }
      }
    }
    const unsigned long long hb = __ballot(hit != kNone), lb = __ballot(lp != 0);
    const uint32_t pick_lane = hb ? (uint32_t)(__ffsll((long long)hb) - 1) : (lb ? (uint32_t)(63 - __clzll((long long)lb)) : 64u);
    const uint32_t pick = hb ? __shfl(hit, (int)pick_lane, 64) : (lb ? __shfl(lp, (int)pick_lane, 64) - 1 : kNone);
    if (lane == 0 && pick != kNone) s->argmax_key = pick;
  }
  return true;
}

// The draw: from the sorted candidates (at most kCap), from the boundary bins
// (draw_many) when there are more, and from the logits by one workgroup
// (sample_one_wg) when the boundary bins alone hold more than kCap.  Leaves
// the histogram and the candidate count zero for the next draw.
__global__ void __launch_bounds__(kT) k_sample_select(const float* __restrict__ logits, float* __restrict__ p,
                                                      SampleWs ws, uint32_t V, DevState* s) {
  __shared__ unsigned long long key[kCap];
  __shared__ uint32_t sh_mode, sh_n;
  __shared__ float sh_S;
  const float T = s->temperature;
  if (!(T > 0.f) || s->status != IFX_OK) return;
  if (threadIdx.x == 0) {
    sh_mode = ws.ctl->mode;
    sh_n = min(ws.ctl->count, kCap);
  }
  if (threadIdx.x < 64) {
    const float S = part_total(ws.part);
    if (threadIdx.x == 0) sh_S = S;
  }
  __syncthreads();
  const uint32_t mode = sh_mode, n = sh_n;
  const float S = sh_S;
  if (mode == kModeCand && n > 0) {
    for (uint32_t j = threadIdx.x; j < n; j += kT) {
      const uint2 c = ws.cand[j];
      key[j] = sample_key(c.y, c.x);
    }
    __syncthreads();
    sort_keys(key, n);
    draw_sorted(key, n, S, s);
  } else if (mode == kModeMany) {
    if (!draw_many(p, ws, V, S, s, key)) sample_one_wg(logits, p, V, s);
  }
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < kBins; i += kT) ws.hist[i] = 0ull;
  if (threadIdx.x == 0) ws.ctl->count = 0;
}

// The maximum logit's key and the NaN flag, as the head's argmax leaves them.
__global__ void __launch_bounds__(kST) k_logits_max(const float* __restrict__ logits, uint32_t V, DevState* s) {
  __shared__ unsigned long long wb[kSW];
  __shared__ int wn[kSW];
  const uint32_t per = (V + kG - 1) / kG, i0 = min(V, blockIdx.x * per), i1 = min(V, i0 + per);
  unsigned long long best = 0;
  bool nan = false;
  for (uint32_t i = i0 + threadIdx.x; i < i1; i += kST) {
    const float v = logits[i];
    nan |= v != v;
    const unsigned long long k = order_key(v, i);
    best = k > best ? k : best;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long x = __shfl_xor(best, o, 64);
    best = x > best ? x : best;
  }
  const bool any = __any(nan);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    wb[w] = best;
    wn[w] = any ? 1 : 0;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long m = 0;
    int a = 0;
    for (int i = 0; i < kSW; i++) {
      m = wb[i] > m ? wb[i] : m;
      a |= wn[i];
    }
    if (m) atomicMax(&s->argmax_key, m);
    if (a) atomicExch(&s->status, (int)IFX_E_NAN_LOGIT);
  }
}

}  // namespace

size_t sample_ws_bytes() { return kWsBytes; }

SampleWs sample_ws(void* base) {
  uint8_t* b = (uint8_t*)base;
  SampleWs w;
  w.hist = (unsigned long long*)(b + kOffHist);
  w.part = (float*)(b + kOffPart);
  w.cand = (uint2*)(b + kOffCand);
  w.ctl = (SampleCtl*)(b + kOffCtl);
  return w;
}

hipError_t launch_sample(const float* logits, float* probs, const SampleWs& ws, uint32_t vocab, DevState* state,
                         hipStream_t st) {
  if (vocab == 0 || vocab >= (1u << 24)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sample_weights, dim3(kWG), dim3(kWT), 0, st, logits, probs, ws, vocab, state);
  hipLaunchKernelGGL(k_sample_gather, dim3(kG), dim3(kST), 0, st, probs, ws, vocab, state);
  hipLaunchKernelGGL(k_sample_select, dim3(1), dim3(kT), 0, st, logits, probs, ws, vocab, state);
  return hipGetLastError();
}

hipError_t launch_logits_max(const float* logits, uint32_t vocab, DevState* state, hipStream_t st) {
  if (vocab == 0 || vocab >= (1u << 24)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_logits_max, dim3(kG), dim3(kST), 0, st, logits, vocab, state);
  return hipGetLastError();
}

}  // namespace ifx
