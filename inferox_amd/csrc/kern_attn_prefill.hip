// kern_attn_prefill.hip — attention of a prefill chunk (src/model/forward.rs:
// 215-337, the batched Layer::prefill; non-causal for Layer::forward,
// src/model/forward.rs:62-207).  Query row t of head h attends to the K/V
// cache rows row0 .. row0 + t (causal) or row0 .. row0 + n - 1 of kv head
// h / (n_heads / n_kv_heads): s = (q . k) / sqrt(head_dim), softmax, o = p V,
// all in f32 (src/model/forward.rs:383-414 per row, src/ops.rs:223-239).
//
// A workgroup owns 64 query rows of one head and walks the key blocks of 64
// rows with the running-max softmax: per block, Q K^T from LDS with 4 x 4
// register tiles, the block's row max / sum by 16-lane shuffles, the weights
// through LDS, then O += P V.  Thread (ty, tx) holds queries ty + 16 i and keys
// tx + 16 j (rows one apart across a 16-lane group: conflict-free LDS reads),
// and output dims tx + 16 j.  The softmax and the order of the sums differ from
// the reference's sequential loops only by f32 rounding.
#include "kernels.h"

namespace ifx {

namespace {

constexpr int kQ = 64, kKB = 64, kThreads = 256;

template <int HD>
__global__ void __launch_bounds__(kThreads) k_attn_prefill(AttnPrefillArgs a) {
  constexpr int KS = HD + 4;      // K/Q row stride (floats): 16 consecutive rows start on distinct bank groups
  constexpr int ND = HD / 16;     // output dims per thread
  constexpr int PS = kKB + 4;
  extern __shared__ __attribute__((aligned(16))) float sm[];
  float* Qs = sm;                 // [kQ][KS]
  float* Ks = Qs + kQ * KS;       // [kKB][KS]
  float* Vs = Ks + kKB * KS;      // [kKB][HD]
  float* Ps = Vs + kKB * HD;      // [kQ][PS]

  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  // heavier (later) query blocks first
  const uint32_t qb = gridDim.x - 1 - blockIdx.x, h = blockIdx.y;
  const uint32_t q0 = qb * kQ, group = a.n_heads / a.n_kv_heads, hk = h / group;
  const uint32_t qd = a.n_heads * HD, kvd = a.n_kv_heads * HD;
  const float sqrt_hd = sqrtf((float)HD);

  // Q block (rows beyond n read as zero)
  for (int i = tid; i < kQ * (HD / 4); i += kThreads) {
    const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
    const uint32_t t = q0 + r;
    const float4 v = t < a.n ? *(const float4*)(a.q + (uint64_t)t * qd + h * HD + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    *(float4*)(Qs + r * KS + c) = v;
  }

  float o[4][ND], m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    m[i] = -INFINITY;
    l[i] = 0.f;
#pragma unroll
    for (int j = 0; j < ND; j++) o[i][j] = 0.f;
  }

  const uint32_t last_q = min(q0 + kQ, a.n) - 1;
  const uint32_t kend = a.causal ? last_q + 1 : a.n;  // keys [0, kend)
  const uint32_t nkb = (kend + kKB - 1) / kKB;
  for (uint32_t kb = 0; kb < nkb; kb++) {
    const uint32_t k0 = kb * kKB;
    __syncthreads();  // previous block's Ks/Vs/Ps reads are done
    for (int i = tid; i < kKB * (HD / 4); i += kThreads) {
      const int r = i / (HD / 4), c = 4 * (i % (HD / 4));
      const uint32_t key = k0 + r;
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      if (key < kend) {
        const uint64_t off = (uint64_t)(a.row0 + key) * kvd + hk * HD + c;
        kv = *(const float4*)(a.k_cache + off);
        vv = *(const float4*)(a.v_cache + off);
      }
      *(float4*)(Ks + r * KS + c) = kv;
      *(float4*)(Vs + r * HD + c) = vv;
    }
    __syncthreads();

    // scores s[i][j] = q(ty + 16 i) . k(tx + 16 j)
    float s[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) s[i][j] = 0.f;
#pragma unroll 4
    for (int d = 0; d < HD; d += 4) {
      float4 qv[4], kv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) qv[i] = *(const float4*)(Qs + (ty + 16 * i) * KS + d);
#pragma unroll
      for (int j = 0; j < 4; j++) kv[j] = *(const float4*)(Ks + (tx + 16 * j) * KS + d);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          s[i][j] = fmaf(qv[i].x, kv[j].x, s[i][j]);
          s[i][j] = fmaf(qv[i].y, kv[j].y, s[i][j]);
          s[i][j] = fmaf(qv[i].z, kv[j].z, s[i][j]);
          s[i][j] = fmaf(qv[i].w, kv[j].w, s[i][j]);
        }
    }
    // mask, running max, weights
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t qt = q0 + ty + 16 * i;
      float bm = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t key = k0 + tx + 16 * j;
        const bool ok = key < kend && (!a.causal || key <= qt);
        s[i][j] = ok ? s[i][j] / sqrt_hd : -INFINITY;
        bm = fmaxf(bm, s[i][j]);
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) bm = fmaxf(bm, __shfl_xor(bm, off, 64));
      const float mn = fmaxf(m[i], bm);
      // rows with no key yet (mn = -inf) keep zero weights
      const float alpha = mn == -INFINITY ? 1.f : expf(m[i] - mn);
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float p = mn == -INFINITY ? 0.f : expf(s[i][j] - mn);
        Ps[(ty + 16 * i) * PS + tx + 16 * j] = p;
        ps += p;
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) ps += __shfl_xor(ps, off, 64);
      l[i] = l[i] * alpha + ps;
      m[i] = mn;
#pragma unroll
      for (int j = 0; j < ND; j++) o[i][j] *= alpha;
    }
    __syncthreads();
    // O += P V
    const int kn = (int)min((uint32_t)kKB, kend - k0);
    for (int c = 0; c < kn; c++) {
      float p[4], v[ND];
#pragma unroll
      for (int i = 0; i < 4; i++) p[i] = Ps[(ty + 16 * i) * PS + c];
#pragma unroll
      for (int j = 0; j < ND; j++) v[j] = Vs[c * HD + tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < ND; j++) o[i][j] = fmaf(p[i], v[j], o[i][j]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t t = q0 + ty + 16 * i;
    if (t >= a.n) continue;
    const float inv = 1.0f / l[i];
#pragma unroll
    for (int j = 0; j < ND; j++) a.out[(uint64_t)t * qd + h * HD + tx + 16 * j] = o[i][j] * inv;
  }
}

template <int HD>
hipError_t go(const AttnPrefillArgs& a, hipStream_t st) {
  const size_t lds = ((size_t)kQ * (HD + 4) + (size_t)kKB * (HD + 4) + (size_t)kKB * HD + (size_t)kQ * (kKB + 4)) * 4;
  static bool opted = false;
  if (!opted) {
    hipError_t e = hipFuncSetAttribute((const void*)k_attn_prefill<HD>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    opted = true;
  }
  dim3 grid((a.n + kQ - 1) / kQ, a.n_heads);
  hipLaunchKernelGGL(k_attn_prefill<HD>, grid, dim3(kThreads), lds, st, a);
  return hipGetLastError();
}

}  // namespace

bool attn_prefill_head_dim(uint32_t hd) { return hd == 48 || hd == 64 || hd == 96 || hd == 128; }

hipError_t launch_attn_prefill(const AttnPrefillArgs& a, hipStream_t st) {
  if (a.n == 0) return hipSuccess;
  if (a.n_kv_heads == 0 || a.n_heads % a.n_kv_heads) return hipErrorInvalidValue;
  switch (a.head_dim) {
    case 48: return go<48>(a, st);
    case 64: return go<64>(a, st);
    case 96: return go<96>(a, st);
    case 128: return go<128>(a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ifx
