// kern_attn.hip — split-K flash-decode attention over the device KV cache (GQA).
//
// Replaces the decode attention loops of Layer::decode_step
// (src/model/forward.rs:383-414): per query head h with kv head h / (n_heads /
// n_kv_heads), s_t = (q . k_t) / sqrt(head_dim), p = softmax(s), o = sum_t p_t v_t.
//
// Grid = (chunk index, kv head).  A workgroup handles one kv head and kChunk
// cache rows for all `group` query heads that share it, so each K/V row is read
// from HBM once per token.  All K and V loads of the chunk are issued before the
// first wait, so a workgroup costs one memory round trip.  It writes a partial
// record (unnormalised o, running max, sum) for its chunk; the last workgroup to
// finish a kv head (agent-scope counter) merges the records with the usual
// max-rescaling and resets the counter for the next launch.
// The cache rows attended are [attn_lo, len] (or [attn_lo, attn_end)), read
// from the session state, so the launch is identical for every token.
#include "kernels.h"

namespace ifx {

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 64;       // cache rows per workgroup (4 threads per row for the scores)
constexpr int kMaxGroup = 8;
constexpr int kMaxHd = 256;
constexpr int kMaxMerge = 256;   // chunks per kv head (max_seq <= kMaxMerge * kChunk)
constexpr int kMergeBatch = 16;  // partial rows loaded together per merging thread

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float4 fma4(float w, float4 v, float4 acc) {
  acc.x = fmaf(w, v.x, acc.x);
  acc.y = fmaf(w, v.y, acc.y);
  acc.z = fmaf(w, v.z, acc.z);
  acc.w = fmaf(w, v.w, acc.w);
  return acc;
}
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// HDT: the head dim when > 0 (register arrays sized exactly), 0 for any
// multiple of 4 up to kMaxHd.
template <int HDT>
__global__ void __launch_bounds__(kThreads) k_attn_decode(AttnArgs a) {
  constexpr int NC4M = (HDT > 0 ? HDT : kMaxHd) / 4;                    // float4 per head row
  constexpr int KPT = (NC4M + 3) / 4;                                    // K float4 per thread
  constexpr int VPT = HDT > 0 ? (kChunk * NC4M + kThreads - 1) / kThreads : 16;  // V float4 per thread
  __shared__ float4 qs[kMaxGroup * NC4M];
  __shared__ float sc[kMaxGroup * kChunk];
  __shared__ float4 red[kThreads * kMaxGroup];  // [position group][g][float4 column], npg * nc4 <= kThreads
  __shared__ float mstat[kMaxGroup], lstat[kMaxGroup];
  __shared__ float cw[kMaxGroup * kMaxMerge];
  __shared__ int is_last;

  const uint32_t c = blockIdx.x, hk = blockIdx.y;
  const uint32_t G = a.n_heads / a.n_kv_heads;
  const uint32_t HD = HDT > 0 ? (uint32_t)HDT : a.head_dim, nc4 = HD / 4, kvd = a.n_kv_heads * HD;
  const uint32_t lo = a.state->attn_lo;
  const uint32_t hi = a.state->attn_end ? a.state->attn_end : a.state->len + 1;
  const uint32_t nrows = hi > lo ? hi - lo : 0;
  const uint32_t nch = (nrows + kChunk - 1) / kChunk;
  if (c >= nch) return;
  const uint32_t t0 = lo + c * kChunk;
  const uint32_t n = (t0 + kChunk <= hi) ? kChunk : hi - t0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // ---- K rows (4 threads per row, every 4th float4) and V rows (thread =
  // float4 column x position group), all loads in flight together ----
  const uint32_t kp = tid >> 2, kq = tid & 3;
  float4 kr[KPT];
  {
    const float4* k4 = (const float4*)(a.k_cache + (uint64_t)(t0 + kp) * kvd + hk * HD);
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const uint32_t ch = kq + 4 * i;
      if (kp < n && ch < nc4) kr[i] = k4[ch];
    }
  }
  const uint32_t npg = kThreads / nc4, vch = tid % nc4, pg = tid / nc4;
  float4 vr[VPT];
#pragma unroll
  for (int i = 0; i < VPT; i++) {
    const uint32_t p = pg + npg * i;
    if (pg < npg && p < n) vr[i] = ((const float4*)(a.v_cache + (uint64_t)(t0 + p) * kvd + hk * HD))[vch];
  }
  for (uint32_t i = tid; i < G * nc4; i += kThreads) qs[i] = ((const float4*)(a.q + (uint64_t)hk * G * HD))[i];
  __syncthreads();

  // ---- scores (src/model/forward.rs:388-397) ----
  {
    float s[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; g++) s[g] = 0.f;
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const uint32_t ch = kq + 4 * i;
      if (kp < n && ch < nc4) {
#pragma unroll
        for (int g = 0; g < kMaxGroup; g++) {
          if (g < (int)G) {
            const float4 qv = qs[g * nc4 + ch];
            s[g] = fmaf(qv.x, kr[i].x, s[g]);
            s[g] = fmaf(qv.y, kr[i].y, s[g]);
            s[g] = fmaf(qv.z, kr[i].z, s[g]);
            s[g] = fmaf(qv.w, kr[i].w, s[g]);
          }
        }
      }
    }
    const float rs = sqrtf((float)HD);
#pragma unroll
    for (int g = 0; g < kMaxGroup; g++) {
      s[g] += __shfl_xor(s[g], 1, 64);
      s[g] += __shfl_xor(s[g], 2, 64);
      if (g < (int)G && kq == 0 && kp < n) sc[g * kChunk + kp] = s[g] / rs;
    }
  }
  __syncthreads();

  // ---- chunk-local softmax statistics (softmax_rows, src/ops.rs:223-239) ----
  for (uint32_t g = wave; g < G; g += kThreads / 64) {
    const float v = lane < (int)n ? sc[g * kChunk + lane] : -INFINITY;
    const float m = wave_max(v);
    const float e = lane < (int)n ? expf(v - m) : 0.f;
    const float l = wave_sum(e);
    if (lane < (int)n) sc[g * kChunk + lane] = e;
    if (lane == 0) {
      mstat[g] = m;
      lstat[g] = l;
    }
  }
  __syncthreads();

  // ---- o = sum_t e_t v_t (src/model/forward.rs:401-409), position groups
  // summed through LDS ----
  if (pg < npg) {
    float4 o[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; g++) o[g] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < VPT; i++) {
      const uint32_t p = pg + npg * i;
      if (p < n) {
#pragma unroll
        for (int g = 0; g < kMaxGroup; g++)
          if (g < (int)G) o[g] = fma4(sc[g * kChunk + p], vr[i], o[g]);
      }
    }
#pragma unroll
    for (int g = 0; g < kMaxGroup; g++)
      if (g < (int)G) red[(pg * G + g) * nc4 + vch] = o[g];
  }
  __syncthreads();
  const uint32_t rec = attn_partial_floats(G, HD);
  float* part = a.partial + ((uint64_t)hk * a.max_chunks + c) * rec;
  for (uint32_t item = tid; item < G * nc4; item += kThreads) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t q = 0; q < npg; q++) acc = add4(acc, red[q * G * nc4 + item]);
    ((float4*)part)[item] = acc;
  }
  if (tid < (int)G) {
    part[G * HD + tid] = mstat[tid];
    part[G * HD + G + tid] = lstat[tid];
  }

  // ---- the last workgroup of this kv head merges all chunks ----
  // Every wave waits until its partial stores have reached L2; after the
  // barrier one agent-scope release (an L2 write-back) by wave 0 publishes the
  // whole record before the counter increment.  One write-back per workgroup
  // instead of one per wave: these serialise per L2 and dominate otherwise.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (wave == 0) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(&a.counters[hk], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (old == nch - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!is_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

  const float* base = a.partial + (uint64_t)hk * a.max_chunks * rec;
  const uint32_t items = G * nc4;
  const uint32_t nsplit = items >= (uint32_t)kThreads ? 1u : kThreads / items;
  const uint32_t sp = tid / items, item0 = tid % items;
  // first batch of partial o rows in flight while the chunk weights are formed
  float4 ov[kMergeBatch];
  if (sp < nsplit) {
#pragma unroll
    for (int k = 0; k < kMergeBatch; k++) {
      const uint32_t cc = min(sp + nsplit * k, nch - 1);
      ov[k] = ((const float4*)(base + (uint64_t)cc * rec))[item0];
    }
  }
  // weights w_c = exp(m_c - M) and den = sum_c l_c w_c, one wave per query head
  for (uint32_t g = wave; g < G; g += kThreads / 64) {
    float m[kMaxMerge / 64], l[kMaxMerge / 64];
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMaxMerge / 64; j++) {
      const uint32_t cc = lane + 64 * j;
      m[j] = cc < nch ? base[(uint64_t)cc * rec + G * HD + g] : -INFINITY;
      l[j] = cc < nch ? base[(uint64_t)cc * rec + G * HD + G + g] : 0.f;
      M = fmaxf(M, m[j]);
    }
    M = wave_max(M);
    float den = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxMerge / 64; j++) {
      const uint32_t cc = lane + 64 * j;
      if (cc < nch) {
        const float w = expf(m[j] - M);
        cw[g * kMaxMerge + cc] = w;
        den = fmaf(l[j], w, den);
      }
    }
    den = wave_sum(den);
    if (lane == 0) lstat[g] = den;
  }
  __syncthreads();
  // o_g = sum_c w_c o_c / den: thread (split sp, float4 item), splits summed in LDS
  for (uint32_t item = item0; item < items; item += kThreads) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (sp < nsplit) {
      const uint32_t g = item / nc4;
      for (uint32_t c0 = sp;; c0 += nsplit * kMergeBatch) {
        if (item != item0 || c0 != sp) {
#pragma unroll
          for (int k = 0; k < kMergeBatch; k++) {
            const uint32_t cc = min(c0 + nsplit * k, nch - 1);
            ov[k] = ((const float4*)(base + (uint64_t)cc * rec))[item];
          }
        }
#pragma unroll
        for (int k = 0; k < kMergeBatch; k++) {
          const uint32_t cc = c0 + nsplit * k;
          if (cc < nch) acc = fma4(cw[g * kMaxMerge + cc], ov[k], acc);
        }
        if (c0 + nsplit * kMergeBatch >= nch) break;
      }
    }
    if (nsplit > 1) {
      if (sp < nsplit) red[sp * items + item] = acc;
    } else {
      const float den = lstat[item / nc4];
      ((float4*)(a.out + (uint64_t)hk * G * HD))[item] =
          make_float4(acc.x / den, acc.y / den, acc.z / den, acc.w / den);
    }
  }
  if (nsplit > 1) {
    __syncthreads();
    if ((uint32_t)tid < items) {
      float4 acc = red[tid];
      for (uint32_t q = 1; q < nsplit; q++) acc = add4(acc, red[q * items + tid]);
      const float den = lstat[tid / nc4];
      ((float4*)(a.out + (uint64_t)hk * G * HD))[tid] =
          make_float4(acc.x / den, acc.y / den, acc.z / den, acc.w / den);
    }
  }
  if (tid == 0) __hip_atomic_store(&a.counters[hk], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t st) {
  if (a.n_kv_heads == 0 || a.n_heads % a.n_kv_heads || a.n_heads / a.n_kv_heads > kMaxGroup ||
      a.head_dim == 0 || a.head_dim > kMaxHd || a.head_dim % 4 || a.chunk != kChunk || a.max_chunks > kMaxMerge ||
      a.max_chunks == 0)
    return hipErrorInvalidValue;
  const dim3 grid(a.max_chunks, a.n_kv_heads);
  switch (a.head_dim) {
    case 64: hipLaunchKernelGGL(k_attn_decode<64>, grid, dim3(kThreads), 0, st, a); break;
    case 128: hipLaunchKernelGGL(k_attn_decode<128>, grid, dim3(kThreads), 0, st, a); break;
    default: hipLaunchKernelGGL(k_attn_decode<0>, grid, dim3(kThreads), 0, st, a); break;
  }
  return hipGetLastError();
}

}  // namespace ifx
