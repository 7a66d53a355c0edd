// kern_attn.hip — split-K flash-decode attention over the device KV cache (GQA).
//
// Replaces the decode attention loops of Layer::decode_step
// (src/model/forward.rs:383-414): per query head h with kv head h / (n_heads /
// n_kv_heads), s_t = (q . k_t) / sqrt(head_dim), p = softmax(s), o = sum_t p_t v_t.
//
// Grid = (chunk index, kv head).  A workgroup handles one kv head and `chunk`
// cache rows for all `group` query heads that share it, so each K/V row is read
// from HBM once per token.  It writes (o_partial, max, sum) for its chunk; the
// last workgroup to finish a head (agent-scope counter) merges the chunks with
// the usual max-rescaling and resets the counter for the next launch.
// The cache rows attended are [attn_lo, len] (or [attn_lo, attn_end)), read
// from the session state, so the launch is identical for every token.
#include "kernels.h"

namespace ifx {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxGroup = 8;
constexpr int kMaxHd = 256;
constexpr int kMaxChunk = 64;

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

__global__ void __launch_bounds__(kThreads) k_attn_decode(AttnArgs a) {
  __shared__ float qs[kMaxGroup * kMaxHd];
  __shared__ float sc[kMaxGroup * kMaxChunk];
  __shared__ float red[kThreads * 4 * kMaxGroup];  // phase-3 partials [pos group][g][HD]: npg*HD <= 1024
  __shared__ float mstat[kMaxGroup], lstat[kMaxGroup];
  __shared__ int is_last;

  const uint32_t c = blockIdx.x, hk = blockIdx.y;
  const uint32_t G = a.n_heads / a.n_kv_heads, HD = a.head_dim, kvd = a.n_kv_heads * HD;
  const uint32_t nc4 = HD / 4;  // float4 chunks per head row
  const uint32_t lo = a.state->attn_lo;
  const uint32_t hi = a.state->attn_end ? a.state->attn_end : a.state->len + 1;
  const uint32_t nrows = hi > lo ? hi - lo : 0;
  const uint32_t nch = (nrows + a.chunk - 1) / a.chunk;
  if (c >= nch) return;
  const uint32_t t0 = lo + c * a.chunk;
  const uint32_t n = (t0 + a.chunk <= hi) ? a.chunk : hi - t0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  for (uint32_t i = tid; i < G * HD; i += kThreads) qs[i] = a.q[(hk * G) * HD + i];
  __syncthreads();

  // ---- scores (src/model/forward.rs:388-397): 4 threads per cache row, each on
  // every 4th float4 of the row; all K loads of a thread issued together.
  {
    const uint32_t p = tid >> 2, part = tid & 3;
    float4 kr[16];
    const float4* k4 = (const float4*)(a.k_cache + (uint64_t)(t0 + p) * kvd + hk * HD);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t ch = part + 4 * i;
      if (p < n && ch < nc4) kr[i] = k4[ch];
    }
    float s[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; g++) s[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t ch = part + 4 * i;
      if (p < n && ch < nc4) {
#pragma unroll
        for (int g = 0; g < kMaxGroup; g++) {
          if (g < (int)G) {
            const float4 qv = *(const float4*)(qs + g * HD + 4 * ch);
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
      if (g < (int)G && part == 0 && p < n) sc[g * kMaxChunk + p] = s[g] / rs;
    }
  }
  __syncthreads();

  // ---- chunk-local softmax statistics (softmax_rows, src/ops.rs:223-239) ----
  for (uint32_t g = wave; g < G; g += kThreads / 64) {
    const float v = lane < (int)n ? sc[g * kMaxChunk + lane] : -INFINITY;
    const float m = wave_max(v);
    const float e = lane < (int)n ? expf(v - m) : 0.f;
    const float l = wave_sum(e);
    if (lane < (int)n) sc[g * kMaxChunk + lane] = e;
    if (lane == 0) { mstat[g] = m; lstat[g] = l; }
  }
  __syncthreads();

  // ---- o = sum_t e_t v_t (src/model/forward.rs:401-409): thread = (float4
  // column chunk, position group); its V loads are issued together, then the
  // position groups are summed through LDS.
  const uint32_t npg = kThreads / nc4;
  {
    const uint32_t ch = tid % nc4, pg = tid / nc4;
    float4 vr[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t p = pg + npg * i;
      if (pg < npg && p < n) vr[i] = *((const float4*)(a.v_cache + (uint64_t)(t0 + p) * kvd + hk * HD) + ch);
    }
    float4 o[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; g++) o[g] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t p = pg + npg * i;
      if (pg < npg && p < n) {
#pragma unroll
        for (int g = 0; g < kMaxGroup; g++) {
          if (g < (int)G) {
            const float e = sc[g * kMaxChunk + p];
            o[g].x = fmaf(e, vr[i].x, o[g].x);
            o[g].y = fmaf(e, vr[i].y, o[g].y);
            o[g].z = fmaf(e, vr[i].z, o[g].z);
            o[g].w = fmaf(e, vr[i].w, o[g].w);
          }
        }
      }
    }
    if (pg < npg) {
#pragma unroll
      for (int g = 0; g < kMaxGroup; g++)
        if (g < (int)G) *(float4*)(red + ((size_t)pg * G + g) * HD + 4 * ch) = o[g];
    }
  }
  __syncthreads();
  const uint32_t pstride = HD + 2;
  float* part = a.partial + ((uint64_t)hk * a.max_chunks + c) * G * pstride;
  for (uint32_t item = tid; item < G * HD; item += kThreads) {
    const uint32_t g = item / HD, d = item % HD;
    float acc = 0.f;
    for (uint32_t pg = 0; pg < npg; pg++) acc += red[((size_t)pg * G + g) * HD + d];
    part[g * pstride + d] = acc;
  }
  if (tid < (int)G) {
    part[tid * pstride + HD] = mstat[tid];
    part[tid * pstride + HD + 1] = lstat[tid];
  }

  // ---- merge: the last workgroup of this kv head combines all chunks ----
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(&a.counters[hk], 1u, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_AGENT);
    is_last = (old == nch - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const float* base = a.partial + (uint64_t)hk * a.max_chunks * G * pstride;
  if (tid < (int)G) {
    float M = -INFINITY;
    for (uint32_t cc = 0; cc < nch; cc++) M = fmaxf(M, base[(cc * G + tid) * pstride + HD]);
    float den = 0.f;
    for (uint32_t cc = 0; cc < nch; cc++) {
      const float* p = base + (cc * G + tid) * pstride;
      den = fmaf(p[HD + 1], expf(p[HD] - M), den);
    }
    mstat[tid] = M;
    lstat[tid] = den;
  }
  __syncthreads();
  for (uint32_t item = tid; item < G * HD; item += kThreads) {
    const uint32_t g = item / HD, d = item % HD;
    const float M = mstat[g];
    float num = 0.f;
    for (uint32_t cc = 0; cc < nch; cc++) {
      const float* p = base + (cc * G + g) * pstride;
      num = fmaf(p[d], expf(p[HD] - M), num);
    }
    a.out[(hk * G + g) * HD + d] = num / lstat[g];
  }
  if (tid == 0) __hip_atomic_store(&a.counters[hk], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t st) {
  if (a.n_kv_heads == 0 || a.n_heads % a.n_kv_heads || a.n_heads / a.n_kv_heads > kMaxGroup ||
      a.head_dim > kMaxHd || a.head_dim % 4 || a.chunk == 0 || a.chunk > kMaxChunk ||
      kThreads / (a.head_dim / 4) * 16 < a.chunk)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_decode, dim3(a.max_chunks, a.n_kv_heads), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace ifx
