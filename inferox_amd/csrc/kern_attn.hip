// kern_attn.hip — split-K flash-decode attention over the device KV cache (GQA).
//
// Replaces the decode attention loops of Layer::decode_step
// (src/model/forward.rs:383-414): per query head h with kv head h / (n_heads /
// n_kv_heads), s_t = (q . k_t) / sqrt(head_dim), p = softmax(s), o = sum_t p_t v_t.
//
// Grid = (chunk index, kv head), or (kv head, chunk index) for small grids
// (AttnArgs::hk_fast, see launch_typed).  A workgroup handles one kv head and kChunk
// cache rows for all `group` query heads that share it, so each K/V row is read
// from HBM once per token.  The q, K and V loads of the chunk are all issued
// before the first wait (q, then K, then V: the scores start while V is still
// arriving), so a workgroup costs one memory round trip.  It writes a partial
// record (unnormalised o, running max, sum) for its chunk.  A second launch,
// one workgroup per query head, merges the records with the usual
// max-rescaling (a kernel boundary publishes them: no counters or fences,
// which cost more than the launch on this part).
// The cache rows attended are [attn_lo, len] (or [attn_lo, attn_end)), read
// from the session state, so the launch is identical for every token.  The
// cache holds f32 (the reference's KvCache) or, in an f16-KV session,
// binary16 elements (E = _Float16), widened to f32 as they are loaded; all
// arithmetic is f32 either way.
#include <type_traits>

#include "kernels.h"

namespace ifx {

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 64;       // cache rows per workgroup (4 threads per row for the scores)
constexpr int kMaxGroup = 8;
constexpr int kMaxHd = 256;
constexpr int kMergeBatch = 8;   // partial o loads in flight per merging thread

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

typedef uint32_t u4 __attribute__((ext_vector_type(4)));  // 16 raw bytes, kept in registers
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

// two adjacent V elements as loaded (f32 pair, or an f16 pair in one dword)
template <typename E>
using VPair = typename std::conditional<sizeof(E) == 4, float2, uint32_t>::type;
__device__ __forceinline__ float2 widen(float2 v) { return v; }
__device__ __forceinline__ float2 widen(uint32_t u) {
  const h2 h = __builtin_bit_cast(h2, u);
  return make_float2((float)h[0], (float)h[1]);
}
// elements 4j .. 4j + 3 of a 16-byte K chunk
template <typename E>
__device__ __forceinline__ float4 chunk4(u4 raw, int j) {
  if constexpr (sizeof(E) == 4) {
    const f4v f = __builtin_bit_cast(f4v, raw);
    return make_float4(f[0], f[1], f[2], f[3]);
  } else {
    const h8 h = __builtin_bit_cast(h8, raw);
    return make_float4((float)h[4 * j], (float)h[4 * j + 1], (float)h[4 * j + 2], (float)h[4 * j + 3]);
  }
}

// ---- wave reductions on the DPP network (no LDS round trips) ----
// gfx9 DPP controls: row_shr:n = 0x110 + n, row_bcast:15 = 0x142, row_bcast:31 = 0x143.
// Prefix doubling inside each 16-lane row (shr 1, 2, then 4 and 8 on the upper
// banks) leaves the row total in its lane 15; the row broadcasts carry rows
// 0..2 into lane 63.  Lanes whose source is outside the row take the identity.
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK,
                                                    BANK_MASK, false));
}
// max / sum over the 64 lanes, returned uniform (lane 63 holds the full result)
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f<0x111, 0xf, 0xf>(-INFINITY, v));
  v = fmaxf(v, dpp_f<0x112, 0xf, 0xf>(-INFINITY, v));
  v = fmaxf(v, dpp_f<0x114, 0xf, 0xe>(-INFINITY, v));
  v = fmaxf(v, dpp_f<0x118, 0xf, 0xc>(-INFINITY, v));
  v = fmaxf(v, dpp_f<0x142, 0xa, 0xf>(-INFINITY, v));
  v = fmaxf(v, dpp_f<0x143, 0xc, 0xf>(-INFINITY, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<0x111, 0xf, 0xf>(0.f, v);
  v += dpp_f<0x112, 0xf, 0xf>(0.f, v);
  v += dpp_f<0x114, 0xf, 0xe>(0.f, v);
  v += dpp_f<0x118, 0xf, 0xc>(0.f, v);
  v += dpp_f<0x142, 0xa, 0xf>(0.f, v);
  v += dpp_f<0x143, 0xc, 0xf>(0.f, v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// sum over the four lanes of each quad, result in all four (quad_perm [1,0,3,2], [2,3,0,1])
__device__ __forceinline__ float quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));
  return v;
}
// Quad reduce-scatter: lane q of each quad holds partial sums v[0..N); on
// return v[j] (j < N / 4) holds the quad's total of element q + 4j.  Round 1
// (lane ^ 1) keeps the elements h with h % 2 == q % 2 and sends the others,
// round 2 (lane ^ 2) likewise on h / 2.  Lane q adds (v_q + v_q^1) + (v_q^2 +
// v_q^3) exactly as quad_sum does, so the totals are bit-identical to it.
template <int N>
__device__ __forceinline__ void quad_reduce_scatter(float (&v)[N], uint32_t q) {
  static_assert(N % 4 == 0, "whole quads");
  float t[N / 2];  // t[p]: element 2p + q % 2 over lanes q, q ^ 1
  const bool b0 = q & 1, b1 = q & 2;
#pragma unroll
  for (int p = 0; p < N / 2; p++) {
    const float keep = b0 ? v[2 * p + 1] : v[2 * p], send = b0 ? v[2 * p] : v[2 * p + 1];
    t[p] = keep + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), 0xb1, 0xf, 0xf, false));
  }
#pragma unroll
  for (int j = 0; j < N / 4; j++) {
    const float keep = b1 ? t[2 * j + 1] : t[2 * j], send = b1 ? t[2 * j] : t[2 * j + 1];
    v[j] = keep + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), 0x4e, 0xf, 0xf, false));
  }
}
// max / sum over the 16 lanes of a wave that share lane % 4, in every lane:
// row_ror:4 and row_ror:8 (0x124, 0x128) inside each 16-lane row, then the
// gfx950 swaps of rows 0<->1, 2<->3 and of the two halves (each returns the
// pair as {own, partner} in some order: the pair's max / sum either way).
__device__ __forceinline__ float pair16(float a, float b, bool mx) { return mx ? fmaxf(a, b) : a + b; }
template <bool MAX>
__device__ __forceinline__ float class4_reduce(float v) {
  v = pair16(v, dpp_f<0x124, 0xf, 0xf>(v, v), MAX);
  v = pair16(v, dpp_f<0x128, 0xf, 0xf>(v, v), MAX);
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = pair16(__uint_as_float(r16[0]), __uint_as_float(r16[1]), MAX);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return pair16(__uint_as_float(r32[0]), __uint_as_float(r32[1]), MAX);
}

// v + (v of lane ^ OFF), OFF a power of two from 4 to 32, whole wave active:
// row_half_mirror then quad_perm [3,2,1,0] (4), row_ror:8 (8), the gfx950
// swaps of rows 0<->1, 2<->3 (16) and of the two halves (32).
template <int OFF>
__device__ __forceinline__ float xor_add(float v) {
  static_assert(OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "lane offset");
  if constexpr (OFF == 32 || OFF == 16) {
    const uint32_t u = __float_as_uint(v);
    const auto r = OFF == 32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                             : __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (OFF == 8) {
    return v + dpp_f<0x128, 0xf, 0xf>(v, v);
  } else {
    return v + dpp_f<0x1b, 0xf, 0xf>(0.f, dpp_f<0x141, 0xf, 0xf>(v, v));
  }
}
// the sum over the lanes l, l ^ OFF, l ^ 2 OFF, ... (l < OFF), in each of them
template <int OFF>
__device__ __forceinline__ float4 lanes_sum4(float4 v) {
  if constexpr (OFF < 64) {
    v = make_float4(xor_add<OFF>(v.x), xor_add<OFF>(v.y), xor_add<OFF>(v.z), xor_add<OFF>(v.w));
    return lanes_sum4<2 * OFF>(v);
  } else {
    return v;
  }
}

constexpr int kRowsPerWave = kChunk / (kThreads / 64);  // 16

// Cache rows [lo, hi) the current token attends to.  The three fields are read
// unconditionally, so that they come in one memory round trip (a conditional
// read of len would be a second one).
__device__ __forceinline__ void attended_rows(const DevState* st, uint32_t& lo, uint32_t& hi) {
  const uint32_t len = st->len, attn_lo = st->attn_lo, attn_end = st->attn_end;
  lo = attn_lo;
  hi = attn_end ? attn_end : len + 1;
}

// HDT: the head dim when > 0 (register arrays sized exactly), 0 for any
// multiple of 16 / sizeof(E) up to kMaxHd.  GT: the query heads per kv head
// when > 0, 0 for any up to kMaxGroup.  With both fixed the unrolled loops
// carry no branches.
//
// Each wave owns 16 cache rows of the chunk end to end:
//   scores  lane = (row l/4, quarter l%4): the quarter's 16-byte K chunks
//           ch = l%4 + 4i, q from LDS, a quad reduction on the DPP network;
//   softmax the wave's max on the DPP network, the chunk's max M over the
//           four waves through LDS, then exp(s - M) and the wave's sums;
//   p . V   lane = columns 2l, 2l+1 (+128 j) of all 16 rows, the row weights
//           broadcast from LDS: no cross-lane reduction.
// The four waves' o and sums (all relative to M) add up through LDS into the
// chunk's record.
// At least 3 waves per SIMD: the 70B shape (group 8) otherwise takes 172
// registers, 2 waves per SIMD, and its ~1040 workgroups at ctx 8192 run in 3
// rounds instead of 2.
template <int HDT, int GT, typename E>
__global__ void __launch_bounds__(kThreads, GT == 8 ? 3 : 1) k_attn_decode(AttnArgs a) {
  constexpr int EPC = 16 / (int)sizeof(E);     // cache elements per 16-byte K chunk
  constexpr int GM = GT > 0 ? GT : kMaxGroup;  // loop bound over query heads
  constexpr int NC4M = (HDT > 0 ? HDT : kMaxHd) / 4;      // float4 of q per head row
  constexpr int KPT = (NC4M * 4 / EPC + 3) / 4;            // K chunks per lane
  constexpr int VJ = ((HDT > 0 ? HDT : kMaxHd) + 127) / 128;  // column pairs per lane
  constexpr int QPT = (GM * NC4M + kThreads - 1) / kThreads;  // q float4 per thread
  __shared__ float4 qs[GM * NC4M];
  __shared__ float wst[kThreads / 64][2][GM];                      // per wave: max, sum
  __shared__ float2 wo[kThreads / 64][GM][NC4M * 2];               // per wave: unnormalised o
  __shared__ __attribute__((aligned(16))) float es[kThreads / 64][kRowsPerWave][GM];  // per wave: row weights

  const uint32_t c = a.hk_fast ? blockIdx.y : blockIdx.x, hk = a.hk_fast ? blockIdx.x : blockIdx.y;
  const uint32_t G = GT > 0 ? (uint32_t)GT : a.n_heads / a.n_kv_heads;
  const uint32_t HD = HDT > 0 ? (uint32_t)HDT : a.head_dim, nc4 = HD / 4, nck = HD / EPC;
  uint32_t lo, hi;
  attended_rows(a.state, lo, hi);
  const uint32_t nrows = hi > lo ? hi - lo : 0;
  const uint32_t nch = (nrows + kChunk - 1) / kChunk;
  if (c >= nch) return;
  const uint32_t t0 = lo + c * kChunk;
  const uint32_t n = (t0 + kChunk <= hi) ? kChunk : hi - t0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t r0 = wave * kRowsPerWave;  // first chunk row of this wave
  // rows past the chunk's end read the last real row (weight 0)
  auto cache_row = [&](uint32_t r) -> uint64_t { return ((uint64_t)hk * a.max_seq + t0 + min(r, n - 1)) * HD; };

  // ---- q, K and V loads, all in flight together (in this order: the loads
  // complete in issue order, so the q copy to LDS waits for q alone and the
  // scores for q and K) ----
  float4 qr[QPT];
  {
    const float4* q4 = (const float4*)(a.q + (uint64_t)hk * G * HD);
#pragma unroll
    for (int i = 0; i < QPT; i++) {
      const uint32_t at = tid + kThreads * i;
      qr[i] = at < G * nc4 ? q4[at] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const uint32_t kr_row = r0 + lane / 4, kq = lane & 3;
  u4 kr[KPT];
  {
    const E* krow = (const E*)a.k_cache + cache_row(kr_row);
#pragma unroll
    for (int i = 0; i < KPT; i++) {
      const uint32_t ch = kq + 4 * i;
      kr[i] = ch < nck ? *(const u4*)(krow + EPC * ch) : u4{0u, 0u, 0u, 0u};
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every K load issues before the first V load
  VPair<E> vr[kRowsPerWave][VJ];
#pragma unroll
  for (int r = 0; r < kRowsPerWave; r++) {
    const E* vrow = (const E*)a.v_cache + cache_row(r0 + r);
#pragma unroll
    for (int jj = 0; jj < VJ; jj++) {
      const uint32_t col = 2 * lane + 128 * jj;
      vr[r][jj] = col < HD ? *(const VPair<E>*)(vrow + col) : VPair<E>{};
    }
  }
#pragma unroll
  for (int i = 0; i < QPT; i++) {
    const uint32_t at = tid + kThreads * i;
    if (at < G * nc4) qs[at] = qr[i];
  }
  __syncthreads();

  // ---- scores (src/model/forward.rs:388-397) and the wave's softmax statistics
  // (softmax_rows, src/ops.rs:223-239) ----
  const bool row_ok = kr_row < n;
  const float rs = sqrtf((float)HD);
  // the query heads' dot products advance together: each LDS round trip for q
  // feeds GM independent FMA chains (one chain per head would wait for every read)
  float sg[GM];
#pragma unroll
  for (int g = 0; g < GM; g++) sg[g] = 0.f;
#pragma unroll
  for (int i = 0; i < KPT; i++) {
    const uint32_t ch = kq + 4 * i;
    if (ch < nck) {
#pragma unroll
      for (int j = 0; j < EPC / 4; j++) {
        const float4 kv = chunk4<E>(kr[i], j);
        float4 qv[GM];
#pragma unroll
        for (int g = 0; g < GM; g++)
          if (g < (int)G) qv[g] = qs[g * nc4 + (EPC / 4) * ch + j];
#pragma unroll
        for (int g = 0; g < GM; g++) {
          if (g < (int)G) {
            sg[g] = fmaf(qv[g].x, kv.x, sg[g]);
            sg[g] = fmaf(qv[g].y, kv.y, sg[g]);
            sg[g] = fmaf(qv[g].z, kv.z, sg[g]);
            sg[g] = fmaf(qv[g].w, kv.w, sg[g]);
          }
        }
      }
    }
  }
  // The softmax runs against the chunk's max M over all four waves (one
  // barrier after the scores), so the waves' o and sums add up in the
  // combine without rescaling.  The row weights e go to LDS (es, read back as
  // broadcasts by the whole wave in p . V: LDS keeps a wave's accesses in
  // order), the wave's max and sum per head to wst.
  constexpr bool kSpread = GT > 0 && GT % 4 == 0;
  float sv[GM];
  if constexpr (kSpread) {
    // Whole quads of heads: the quad's reduce-scatter leaves lane (row l / 4,
    // q = l % 4) the row's scores of heads q + 4j, so each lane takes one
    // division, exp and pair of class reductions per four heads.
    quad_reduce_scatter(sg, (uint32_t)kq);
#pragma unroll
    for (int j = 0; j < GM / 4; j++) {
      sv[j] = sg[j] / rs;
      const float m = class4_reduce<true>(row_ok ? sv[j] : -INFINITY);
      if (lane < 4) wst[wave][0][kq + 4 * j] = m;
    }
  } else {
#pragma unroll
    for (int g = 0; g < GM; g++) {
      if (g < (int)G) {
        sv[g] = quad_sum(sg[g]) / rs;
        const float m = wave_max_dpp(row_ok ? sv[g] : -INFINITY);
        if (lane == 0) wst[wave][0][g] = m;
      }
    }
  }
  __syncthreads();
  auto chunk_max = [&](uint32_t g) {
    float M = wst[0][0][g];
#pragma unroll
    for (int w = 1; w < kThreads / 64; w++) M = fmaxf(M, wst[w][0][g]);
    return M;
  };
  if constexpr (kSpread) {
#pragma unroll
    for (int j = 0; j < GM / 4; j++) {
      const uint32_t g = (uint32_t)kq + 4 * j;
      const float e = row_ok ? expf(sv[j] - chunk_max(g)) : 0.f;
      const float l = class4_reduce<false>(e);
      es[wave][lane >> 2][g] = e;
      if (lane < 4) wst[wave][1][g] = l;
    }
  } else {
#pragma unroll
    for (int g = 0; g < GM; g++) {
      if (g < (int)G) {
        const float e = row_ok ? expf(sv[g] - chunk_max(g)) : 0.f;
        const float l = wave_sum_dpp(kq == 0 ? e : 0.f);
        if (kq == 0) es[wave][lane >> 2][g] = e;
        if (lane == 0) wst[wave][1][g] = l;
      }
    }
  }

  // ---- o = sum_t e_t v_t over the wave's rows (src/model/forward.rs:401-409) ----
  float2 o[GM][VJ];
#pragma unroll
  for (int g = 0; g < GM; g++)
#pragma unroll
    for (int jj = 0; jj < VJ; jj++) o[g][jj] = make_float2(0.f, 0.f);
#pragma unroll
  for (int r = 0; r < kRowsPerWave; r++) {
    float e[GM];
#pragma unroll
    for (int g = 0; g < GM; g++) e[g] = es[wave][r][g];
    float2 v[VJ];
#pragma unroll
    for (int jj = 0; jj < VJ; jj++) v[jj] = widen(vr[r][jj]);
#pragma unroll
    for (int g = 0; g < GM; g++) {
      if (g < (int)G) {
#pragma unroll
        for (int jj = 0; jj < VJ; jj++) {
          o[g][jj].x = fmaf(e[g], v[jj].x, o[g][jj].x);
          o[g][jj].y = fmaf(e[g], v[jj].y, o[g][jj].y);
        }
      }
    }
  }

  // ---- combine the four waves into the chunk's record ----
#pragma unroll
  for (int g = 0; g < GM; g++)
#pragma unroll
    for (int jj = 0; jj < VJ; jj++)
      if (g < (int)G && 2 * lane + 128 * jj < HD) wo[wave][g][lane + 64 * jj] = o[g][jj];
  __syncthreads();
  const uint32_t rec = attn_partial_floats(G, HD);
  float* part = a.partial + ((uint64_t)hk * a.max_chunks + c) * rec;
  for (uint32_t item = tid; item < G * HD / 2; item += kThreads) {
    const uint32_t g = item / (HD / 2), cp = item % (HD / 2);
    float2 acc = wo[0][g][cp];
#pragma unroll
    for (int w = 1; w < kThreads / 64; w++) {
      // waves whose rows are all past the chunk end hold zeros
      acc.x += wo[w][g][cp].x;
      acc.y += wo[w][g][cp].y;
    }
    *(float2*)(part + g * HD + 2 * cp) = acc;
  }
  if (tid < (int)G) {
    float L = wst[0][1][tid];
#pragma unroll
    for (int w = 1; w < kThreads / 64; w++) L += wst[w][1][tid];
    part[G * HD + tid] = chunk_max((uint32_t)tid);
    part[G * HD + G + tid] = L;
  }

}

// Combines the chunk records of query head h = blockIdx.x (kv head h / G):
// o_h = sum_c w_c o_c / sum_c w_c l_c, w_c = exp(m_c - M), M = max_c m_c
// (softmax over all cached rows, src/model/forward.rs:398-409, taken chunk by
// chunk).  Any number of chunks: M and the denominator are reduced over the
// workgroup (thread t reads chunks t, t + 256, ...), then the weights are
// staged in LDS 256 chunks at a time.  Thread (split sp, float4 column) sums
// the batch's chunks sp, sp + nsplit, ...; the first loads of o are in flight
// while M is formed.
// CS workgroups per query head, each producing HD / CS of its columns (every
// one forms the same weights from all records' max and sum).
template <int HDT, int GT, int CS>
__global__ void __launch_bounds__(kThreads) k_attn_merge(AttnArgs a) {
  __shared__ float cw[kThreads];
  __shared__ float wred[2][kThreads / 64];
  __shared__ float4 red[kThreads];
  const uint32_t G = GT > 0 ? (uint32_t)GT : a.n_heads / a.n_kv_heads;
  const uint32_t HD = HDT > 0 ? (uint32_t)HDT : a.head_dim, nc4 = HD / 4 / CS;  // float4 columns of the slice
  const uint32_t h = blockIdx.x / CS, hk = h / G, g = h % G, cb = (blockIdx.x % CS) * nc4;
  uint32_t lo, hi;
  attended_rows(a.state, lo, hi);
  const uint32_t nrows = hi > lo ? hi - lo : 0;
  const uint32_t nch = (nrows + kChunk - 1) / kChunk;
  if (nch == 0) return;
  const uint32_t rec = attn_partial_floats(G, HD);
  const float* base = a.partial + (uint64_t)hk * a.max_chunks * rec;
  const float* ml = base + G * HD;  // chunk c: max at ml[c rec + g], sum at ml[c rec + G + g]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t nsplit = kThreads / nc4, sp = tid / nc4, col = tid % nc4;
  const bool worker = sp < nsplit;  // nc4 need not divide the workgroup
  float4 ov[kMergeBatch];
#pragma unroll
  for (int k = 0; k < kMergeBatch; k++) {
    const uint32_t c = min(min(sp, nsplit - 1) + nsplit * k, nch - 1);  // clamped: loads stay unconditional
    ov[k] = ((const float4*)(base + (uint64_t)c * rec + g * HD))[cb + col];
  }
  // M over every chunk (chunk tid's max and sum are kept for the first batch)
  float m0, l0;
  {
    const uint64_t at = (uint64_t)min((uint32_t)tid, nch - 1) * rec;
    const float mv = ml[at + g], lv = ml[at + G + g];
    m0 = (uint32_t)tid < nch ? mv : -INFINITY;
    l0 = (uint32_t)tid < nch ? lv : 0.f;
  }
  float M = m0;
  for (uint32_t c = tid + kThreads; c < nch; c += kThreads) M = fmaxf(M, ml[(uint64_t)c * rec + g]);
  M = wave_max_dpp(M);
  if (lane == 0) wred[0][wave] = M;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kThreads / 64; w++) M = fmaxf(M, wred[0][w]);
  const float w0 = (uint32_t)tid < nch ? expf(m0 - M) : 0.f;
  float den = l0 * w0;
  for (uint32_t c = tid + kThreads; c < nch; c += kThreads)
    den = fmaf(ml[(uint64_t)c * rec + G + g], expf(ml[(uint64_t)c * rec + g] - M), den);
  den = wave_sum_dpp(den);
  if (lane == 0) wred[1][wave] = den;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t b = 0; b < nch; b += kThreads) {
    if (b) __syncthreads();  // the previous batch's weights are no longer read
    cw[tid] = b == 0 ? w0 : (b + tid < nch ? expf(ml[(uint64_t)(b + tid) * rec + g] - M) : 0.f);
    __syncthreads();
    if (worker) {
      const uint32_t end = min(nch, b + (uint32_t)kThreads);
      for (uint32_t c0 = b + sp;; c0 += nsplit * kMergeBatch) {
        if (c0 != sp) {
#pragma unroll
          for (int k = 0; k < kMergeBatch; k++) {
            const uint32_t c = min(c0 + nsplit * k, nch - 1);
            ov[k] = ((const float4*)(base + (uint64_t)c * rec + g * HD))[cb + col];
          }
        }
#pragma unroll
        for (int k = 0; k < kMergeBatch; k++) {
          const uint32_t c = c0 + nsplit * k;
          if (c < end) acc = fma4(cw[c - b], ov[k], acc);
        }
        if (c0 + nsplit * kMergeBatch >= end) break;
      }
    }
  }
  // the splits' partial sums: with a power-of-two column count up to 32 the
  // wave's splits (lane = nc4 (sp mod 64 / nc4) + col) meet through xor
  // butterflies and the waves' sums through LDS; otherwise one thread per
  // column adds them up through LDS
  constexpr int NC4 = HDT > 0 ? HDT / 4 / CS : 0;
  constexpr bool kTree = NC4 >= 4 && NC4 <= 32 && (NC4 & (NC4 - 1)) == 0;
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (kTree) {
    acc = lanes_sum4<NC4>(acc);
    if (lane < NC4) red[wave * NC4 + lane] = acc;
    __syncthreads();
    if (tid < NC4) {
      o = red[tid];
#pragma unroll
      for (int w = 1; w < kThreads / 64; w++) o = add4(o, red[w * NC4 + tid]);
    }
  } else {
    red[tid] = acc;
    __syncthreads();
    if ((uint32_t)tid < nc4) {
      o = red[tid];
      for (uint32_t q = 1; q < nsplit; q++) o = add4(o, red[q * nc4 + tid]);
    }
  }
  if ((uint32_t)tid < nc4) {
    float dsum = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; w++) dsum += wred[1][w];
    ((float4*)(a.out + (uint64_t)h * HD))[cb + tid] = make_float4(o.x / dsum, o.y / dsum, o.z / dsum, o.w / dsum);
  }
}

// compute units of the current device (looked up once)
int attn_cu_count() {
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

template <typename E>
void launch_typed(const AttnArgs& a0, hipStream_t st, bool merge) {
  // Chunk grid order: kv head fastest while the grid holds at most two
  // workgroups per CU, so that every chunk of kv head hk runs on XCD hk
  // (workgroup g runs on XCD g mod 8) with that head's contiguous K/V rows,
  // and its records stay in the L2 the merged O launch's slice hk reads (8B
  // at ctx 2048, 296 workgroups: decode 679.5 -> 684.8 tok/s on one box; an
  // order that only put the light last chunks last gained nothing).  Chunk
  // fastest for larger grids (70B at ctx 8192, 1048 workgroups: attention
  // 20.17 against 20.74 us kv head fastest).  IFX_ATTN_HKF=0 / 1 forces either.
  AttnArgs a = a0;
  const char* hf = getenv("IFX_ATTN_HKF");
  const bool forced = hf && (hf[0] == '0' || hf[0] == '1') && hf[1] == 0;
  a.hk_fast = forced ? hf[0] == '1' : (uint64_t)a.max_chunks * a.n_kv_heads <= 2ull * (uint64_t)attn_cu_count();
  const dim3 grid = a.hk_fast ? dim3(a.n_kv_heads, a.max_chunks) : dim3(a.max_chunks, a.n_kv_heads);
  const uint32_t G = a.n_heads / a.n_kv_heads;
#define IFX_ATTN(HD_, G_)                                                                          \
  do {                                                                                             \
    hipLaunchKernelGGL((k_attn_decode<HD_, G_, E>), grid, dim3(kThreads), 0, st, a);              \
    constexpr int CS_ = (HD_ > 0 && (HD_ / 4) % 4 == 0) ? 4 : 1;                                  \
    if (merge)                                                                                     \
      hipLaunchKernelGGL((k_attn_merge<HD_, G_, CS_>), dim3(a.n_heads * CS_), dim3(kThreads), 0, st, a); \
  } while (0)
  if (a.head_dim == 128 && G == 4) IFX_ATTN(128, 4);        // Llama-3 8B
  else if (a.head_dim == 128 && G == 8) IFX_ATTN(128, 8);   // Llama-3 70B
  else if (a.head_dim == 128 && G == 1) IFX_ATTN(128, 1);
  else if (a.head_dim == 64 && G == 4) IFX_ATTN(64, 4);
  else if (a.head_dim == 64 && G == 1) IFX_ATTN(64, 1);
  else if (a.head_dim == 48 && G == 1) IFX_ATTN(48, 1);  // the tiny Llama shape (dim 288, 6 heads)
  else IFX_ATTN(0, 0);
#undef IFX_ATTN
}

}  // namespace

bool attn_decode_head_dim(uint32_t head_dim, bool kv_f16) {
  return head_dim > 0 && head_dim <= kMaxHd && head_dim % (kv_f16 ? 8 : 4) == 0;
}

namespace {
hipError_t launch_attn(const AttnArgs& a, hipStream_t st, bool merge) {
  if (a.n_kv_heads == 0 || a.n_heads % a.n_kv_heads || a.n_heads / a.n_kv_heads > kMaxGroup ||
      !attn_decode_head_dim(a.head_dim, a.kv_f16) || a.chunk != kChunk ||
      a.max_chunks == 0)
    return hipErrorInvalidValue;
  if (a.kv_f16) launch_typed<_Float16>(a, st, merge);
  else launch_typed<float>(a, st, merge);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t st) { return launch_attn(a, st, true); }
hipError_t launch_attn_partials(const AttnArgs& a, hipStream_t st) { return launch_attn(a, st, false); }

}  // namespace ifx
