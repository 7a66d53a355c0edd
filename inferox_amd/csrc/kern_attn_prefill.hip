// kern_attn_prefill.hip — attention of a prefill chunk on the fp16 matrix
// cores (src/model/forward.rs:215-337, the batched Layer::prefill; non-causal
// for Layer::forward, src/model/forward.rs:62-207).  Query row t of head h
// attends to the K/V cache rows row0 .. row0 + t (causal) or row0 .. row0 + n - 1
// of kv head h / (n_heads / n_kv_heads): s = (q . k) / sqrt(head_dim), softmax,
// o = p V (src/model/forward.rs:383-414 per row, src/ops.rs:223-239).
//
// Arithmetic as in kern_gemm.hip: both products run on the fp16 matrix cores
// with each operand an fp16 hi/lo pair (three MFMAs per step, f32
// accumulation), within the rounding of the f32 reference.  The fp16 range is
// kept by power-of-2 scales: per query row and per key row for q . k (undone
// per score), and one per 64-key V block.  The V block scales are folded into
// the softmax weights against a running reference exponent (the weights of a
// block with a smaller scale shrink; a block with a larger one rescales the
// accumulated output as a new running maximum does), so the output
// accumulates in place.
//
// Two launches per layer:
//   * k_kv_prep: one workgroup per (64-key block, kv head) splits the chunk's
//     K rows (row scale) and its V block, transposed (block scale), into fp16
//     hi/lo planes in the workspace, once for all the query heads and query
//     blocks that read them.
//   * k_attn_prefill: a workgroup of 8 waves owns 128 query rows of one head,
//     wave w rows 16w .. 16w + 15 with their q scale and fp16 pairs in
//     registers.  Per 64-key block it copies K and V^T into LDS (the next
//     block's copies wait in registers meanwhile) and computes the scores
//     transposed, S^T = K Q^T (16x16x32 MFMAs): lane i + 16g then holds the
//     scores of query i against keys 16j + 4g + r.  O^T = V^T P^T runs on
//     the same 16x16x32 MFMA with each 32-key step's k slots 8g..8g+7 taken
//     as keys 32c + 4g + r and 32c + 16 + 4g + r, the weights lane i + 16g
//     already holds (V^T's columns read in that order), so the softmax
//     weights never leave registers, and the row max and sum take two
//     shuffles.  64 KB of LDS and one workgroup per CU (two waves per SIMD):
//     each staged block serves 128 queries.
// MFMA lane layout (16x16x32): lane i + 16g holds A[i][8g..8g+7] and
// B[8g..8g+7][i], and receives C[4g + r][i] in register r.
#include "kernels.h"

namespace ifx {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));  // a native vector: stays in registers

constexpr int kQ = 128, kKB = 64, kThreads = 512, kPrepThreads = 256;

__device__ __forceinline__ int exp_of(uint32_t bits) {
  const int e = (int)((bits >> 23) & 255u) - 127;
  return e < -100 ? -100 : e;
}

template <int HD>
struct Dims {
  static constexpr int HP = (HD + 31) / 32 * 32;  // padded head dim
  static constexpr int NCH = HP / 8;              // 16-byte chunks per K row
  static constexpr int NKS = HP / 32;             // 16x16x32 steps over the head dim
  static constexpr int NT = HP / 16;              // O^T tiles (16 dims each)
};

// Workspace of a chunk of n keys: K hi/lo [kvh][npad][HP], V^T hi/lo
// [kvh][nkb][HP][64] (fp16 bits), key exponents [kvh][npad], V block
// exponents [kvh][nkb].
struct PrepWs {
  uint16_t *kh, *kl, *vh, *vl;
  int *kexp, *vexp;
};

constexpr uint64_t al256(uint64_t b) { return (b + 255) & ~255ull; }

PrepWs prep_ws(void* base, uint32_t n, uint32_t n_kv, uint32_t hp) {
  const uint64_t nkb = (n + kKB - 1) / kKB, npad = nkb * kKB, plane = (uint64_t)n_kv * npad * hp;
  uint8_t* p = (uint8_t*)base;
  PrepWs w;
  w.kh = (uint16_t*)p;
  p += al256(plane * 2);
  w.kl = (uint16_t*)p;
  p += al256(plane * 2);
  w.vh = (uint16_t*)p;
  p += al256(plane * 2);
  w.vl = (uint16_t*)p;
  p += al256(plane * 2);
  w.kexp = (int*)p;
  p += al256((uint64_t)n_kv * npad * 4);
  w.vexp = (int*)p;
  return w;
}

uint64_t prep_ws_bytes(uint32_t n, uint32_t n_kv, uint32_t hp) {
  const uint64_t nkb = (n + kKB - 1) / kKB, npad = nkb * kKB, plane = (uint64_t)n_kv * npad * hp;
  return 4 * al256(plane * 2) + al256((uint64_t)n_kv * npad * 4) + al256((uint64_t)n_kv * nkb * 4);
}

// LDS K rows (HP halves): 16-byte chunk c of row r at c ^ (r & 15) for
// 256-byte rows, c ^ ((r >> 1) & 7) for 128, c ^ ((r >> 2) & 3) for 64 and
// 192: the 16 rows of a fragment read at one chunk land on distinct banks.
template <int W>
__device__ __forceinline__ int swz(int r, int c) {
  constexpr int RB = 2 * W;
  const int x = (RB % 256 == 0) ? (r & 15) : (RB % 128 == 0) ? ((r >> 1) & 7) : ((r >> 2) & 3);
  return r * W + 8 * (c ^ x);
}
// LDS V^T rows (64 keys, 128 bytes): chunk c of row r at c ^ ((r ^ r >> 3) & 7),
// so that the 8-byte reads of 16 consecutive rows at one offset land on
// distinct banks (16 lanes over 64 banks; 8-lane groups see 8 distinct chunks)
__device__ __forceinline__ int swzv(int r, int c) { return r * kKB + 8 * (c ^ ((r ^ (r >> 3)) & 7)); }

// Cache elements (E = float, or _Float16 for the f16 KV cache) as floats.
template <typename E>
__device__ __forceinline__ void load8(const E* p, float* v) {
  if constexpr (sizeof(E) == 4) {
    const float4 x0 = *(const float4*)p, x1 = *(const float4*)(p + 4);
    v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
    v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
  } else {
    const h8 x = *(const h8*)p;
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = (float)x[k];
  }
}
template <typename E>
__device__ __forceinline__ float4 load4(const E* p) {
  if constexpr (sizeof(E) == 4) {
    return *(const float4*)p;
  } else {
    const h4 x = *(const h4*)p;
    return make_float4((float)x[0], (float)x[1], (float)x[2], (float)x[3]);
  }
}

// ---------------------------------------------------------------------------
// K/V preparation: grid (key block, kv head).
// ---------------------------------------------------------------------------
template <int HD, typename E>
__global__ void __launch_bounds__(kPrepThreads) k_kv_prep(AttnPrefillArgs a, PrepWs w) {
  using D = Dims<HD>;
  constexpr int HP = D::HP, CPT = D::NCH / 4;  // K: four threads per key row
  __shared__ float vblk[kKB][HD + 1];
  __shared__ float red[kPrepThreads / 64];
  const uint32_t b = blockIdx.x, hk = blockIdx.y, k0 = b * kKB;
  const uint32_t nkb = gridDim.x, npad = nkb * kKB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const E* kbase = (const E*)a.k_cache + ((uint64_t)hk * a.max_seq + a.row0) * HD;
  const E* vbase = (const E*)a.v_cache + ((uint64_t)hk * a.max_seq + a.row0) * HD;

  // K: row kr, chunks qq * CPT .. + CPT - 1; the row scale from the four threads' maxima
  {
    const int kr = tid >> 2, qq = tid & 3;
    const uint32_t key = k0 + (uint32_t)kr;
    float v[CPT][8];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      const int col = 8 * (qq * CPT + i);
#pragma unroll
      for (int k = 0; k < 8; k++) v[i][k] = 0.f;
      if (key < a.n && col < HD) load8(kbase + (uint64_t)key * HD + col, v[i]);
#pragma unroll
      for (int k = 0; k < 8; k++) mx = fmaxf(mx, fabsf(v[i][k]));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    const int e = exp_of(__float_as_uint(mx));
    if (qq == 0) w.kexp[(uint64_t)hk * npad + key] = e;
    const float sc = ldexpf(1.f, 14 - e);
    const uint64_t row = ((uint64_t)hk * npad + key) * HP;
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      h8 hi, lo;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float y = v[i][k] * sc;
        hi[k] = (_Float16)y;
        lo[k] = (_Float16)(y - (float)hi[k]);
      }
      const int ch = qq * CPT + i;
      *(h8*)(w.kh + row + 8 * ch) = hi;
      *(h8*)(w.kl + row + 8 * ch) = lo;
    }
  }

  // V block: into LDS, block maximum, then transposed rows d (64 keys each)
  float mx = 0.f;
  for (int c = tid; c < kKB * (HD / 4); c += kPrepThreads) {
    const int r = c / (HD / 4), col = 4 * (c % (HD / 4));
    const uint32_t key = k0 + (uint32_t)r;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (key < a.n) x = load4(vbase + (uint64_t)key * HD + col);
    vblk[r][col] = x.x;
    vblk[r][col + 1] = x.y;
    vblk[r][col + 2] = x.z;
    vblk[r][col + 3] = x.w;
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const int ev = exp_of(__float_as_uint(mx));
  if (tid == 0) w.vexp[(uint64_t)hk * nkb + b] = ev;
  const float sc = ldexpf(1.f, 14 - ev);
  // thread: V^T row d (< HP), 16-byte chunk c of its 64 keys
  for (int u = tid; u < HP * 8; u += kPrepThreads) {
    const int d = u >> 3, c = u & 7;
    h8 hi, lo;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float y = d < HD ? vblk[8 * c + k][d] * sc : 0.f;
      hi[k] = (_Float16)y;
      lo[k] = (_Float16)(y - (float)hi[k]);
    }
    const uint64_t off = (((uint64_t)hk * nkb + b) * HP + d) * kKB + 8 * c;
    *(h8*)(w.vh + off) = hi;
    *(h8*)(w.vl + off) = lo;
  }
}

// ---------------------------------------------------------------------------
// Attention: grid 1-D over (query block, head), heaviest query blocks first.
// ---------------------------------------------------------------------------
template <int HD>
__global__ void __launch_bounds__(kThreads, 1) k_attn_prefill(AttnPrefillArgs a, PrepWs w) {
  using D = Dims<HD>;
  constexpr int HP = D::HP, NCH = D::NCH, NKS = D::NKS, NT = D::NT;
  constexpr int UK = kKB * NCH * 2 / kThreads;  // K chunks per thread (both planes)
  constexpr int UV = HP * 8 * 2 / kThreads;     // V^T chunks per thread
  __shared__ __attribute__((aligned(16))) _Float16 Kh[kKB * HP], Kl[kKB * HP];
  __shared__ __attribute__((aligned(16))) _Float16 Vh[HP * kKB], Vl[HP * kKB];
  __shared__ __attribute__((aligned(16))) float kfac_s[kKB];  // per key of the block: 2^(e_k - 14) log2(e) / sqrt(hd)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fi = lane & 15, fg = lane >> 4;
  const uint32_t nqb = (a.n + kQ - 1) / kQ;
  const uint32_t qb = nqb - 1 - blockIdx.x / a.n_heads, h = blockIdx.x % a.n_heads;
  const uint32_t q0 = qb * kQ, group = a.n_heads / a.n_kv_heads, hk = h / group;
  const uint32_t qd = a.n_heads * HD;
  const uint32_t nkb_all = (a.n + kKB - 1) / kKB, npad = nkb_all * kKB;
  const float kc = 1.44269504088896341f / sqrtf((float)HD);  // log2(e) / sqrt(hd)

  // ---- this lane's query (fi) as the B operand of S^T = K Q^T, in registers ----
  const uint32_t qt = q0 + 16 * wave + fi;
  h8 qh[NKS], ql[NKS];
  float qinv;
  {
    float v[NKS][8];
    float mx = 0.f;
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) {
      const int col = 32 * ks + 8 * fg;
#pragma unroll
      for (int k = 0; k < 8; k++) v[ks][k] = 0.f;
      if (qt < a.n && col < HD) {
        const float* src = a.q + (uint64_t)qt * qd + h * HD + col;
        const float4 x0 = *(const float4*)src, x1 = *(const float4*)(src + 4);
        v[ks][0] = x0.x; v[ks][1] = x0.y; v[ks][2] = x0.z; v[ks][3] = x0.w;
        v[ks][4] = x1.x; v[ks][5] = x1.y; v[ks][6] = x1.z; v[ks][7] = x1.w;
      }
#pragma unroll
      for (int k = 0; k < 8; k++) mx = fmaxf(mx, fabsf(v[ks][k]));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const int e = exp_of(__float_as_uint(mx));
    qinv = ldexpf(1.f, e - 14);
    const float sc = ldexpf(1.f, 14 - e);
#pragma unroll
    for (int ks = 0; ks < NKS; ks++)
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float y = v[ks][k] * sc;
        qh[ks][k] = (_Float16)y;
        ql[ks][k] = (_Float16)(y - (float)qh[ks][k]);
      }
  }

  const uint32_t last_q = min(q0 + kQ, a.n) - 1;
  const uint32_t kend = a.causal ? last_q + 1 : a.n;  // keys [0, kend)
  const uint32_t nkb = (kend + kKB - 1) / kKB;

  // ---- K / V^T block copies: the next block's chunks wait in registers ----
  u4 rk[UK], rv[UV];
  int rke = 0, rve = 0;
  auto load_k = [&](uint32_t kb) __attribute__((always_inline)) {
    const uint64_t kbase = ((uint64_t)hk * npad + kb * kKB) * HP;
#pragma unroll
    for (int u = 0; u < UK; u++) {
      const int c = tid + kThreads * u, pl = c / (kKB * NCH), rem = c % (kKB * NCH);
      rk[u] = *(const u4*)((pl ? w.kl : w.kh) + kbase + (uint64_t)rem * 8);
    }
    if (tid < kKB) rke = w.kexp[(uint64_t)hk * npad + kb * kKB + tid];
  };
  auto load_v = [&](uint32_t kb) __attribute__((always_inline)) {
    const uint64_t vbase = ((uint64_t)hk * nkb_all + kb) * HP * kKB;
#pragma unroll
    for (int u = 0; u < UV; u++) {
      const int c = tid + kThreads * u, pl = c / (HP * 8), rem = c % (HP * 8);
      rv[u] = *(const u4*)((pl ? w.vl : w.vh) + vbase + (uint64_t)rem * 8);
    }
    rve = w.vexp[(uint64_t)hk * nkb_all + kb];
  };
  auto store_block = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < UK; u++) {
      const int c = tid + kThreads * u, pl = c / (kKB * NCH), rem = c % (kKB * NCH);
      *(u4*)((pl ? Kl : Kh) + swz<HP>(rem / NCH, rem % NCH)) = rk[u];
    }
#pragma unroll
    for (int u = 0; u < UV; u++) {
      const int c = tid + kThreads * u, pl = c / (HP * 8), rem = c % (HP * 8);
      *(u4*)((pl ? Vl : Vh) + swzv(rem >> 3, rem & 7)) = rv[u];
    }
    if (tid < kKB) kfac_s[tid] = ldexpf(kc, rke - 14);
  };

  f4 o[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) o[t] = f4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  int vref = -1000;  // reference V exponent of the accumulated output

  load_k(0);
  load_v(0);
  for (uint32_t kb = 0; kb < nkb; kb++) {
    const uint32_t k0 = kb * kKB;
    __syncthreads();  // every wave is past the previous block's reads
    store_block();
    const int ve = rve;
    __syncthreads();
    // the next block's K now, its V after the scores (fewer registers held)
    const bool more = kb + 1 < nkb;
    if (more) load_k(kb + 1);

    // ---- S^T: keys 16j + 4fg + r (rows) x this lane's query fi (column) ----
    // (one head-dim step at a time: four independent accumulator chains, and
    // the fragments of one step live at once)
    f4 s[4];
#pragma unroll
    for (int j = 0; j < 4; j++) s[j] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const h8 kh8 = *(const h8*)&Kh[swz<HP>(16 * j + fi, 4 * ks + fg)];
        const h8 kl8 = *(const h8*)&Kl[swz<HP>(16 * j + fi, 4 * ks + fg)];
        s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh8, qh[ks], s[j], 0, 0, 0);
        s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh8, ql[ks], s[j], 0, 0, 0);
        s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl8, qh[ks], s[j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // Scores in the log2 domain (src/ops.rs:223-239 takes exp(s - max); here
    // 2^(log2(e) (s - max))): t = S^T * kf, kf = 2^(e_k - 14) log2(e) /
    // sqrt(hd) per key, staged with the block, so that qinv t (qinv = 2^(e_q - 14),
    // exact) is the score times log2(e).  The weights are 2^(qinv (t - m)),
    // from one fma and v_exp_f32.  Masks only where the block crosses the
    // wave's diagonal or the chunk's end (a uniform branch).
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float4 kf = *(const float4*)&kfac_s[16 * j + 4 * fg];
      s[j][0] *= kf.x;
      s[j][1] *= kf.y;
      s[j][2] *= kf.z;
      s[j][3] *= kf.w;
    }
    const bool full = k0 + kKB <= kend && (!a.causal || k0 + kKB - 1 <= q0 + 16 * (uint32_t)wave);
    if (!full) {
      // key k0 + 4 fg + 16 j + r is attended iff 16 j + r <= lim
      const int lim = (int)(a.causal ? min(qt, kend - 1) : kend - 1) - (int)(k0 + 4 * (uint32_t)fg);
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) s[j][r] = 16 * j + r <= lim ? s[j][r] : -INFINITY;
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) bm = fmaxf(bm, s[j][r]);
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(m, bm);
    const bool none = mn == -INFINITY;  // no attended key yet (m and every t are -inf)
    const float alpha = none ? 1.f : __builtin_amdgcn_exp2f(qinv * (m - mn));
    const int vnew = ve > vref ? ve : vref;
    const float oscale = alpha * ldexpf(1.f, vref - vnew);  // the output's rescale
    const float pscale = ldexpf(1.f, ve - vnew);            // this block's weights, <= 1
    const float c = none ? 0.f : -(qinv * mn);              // exact: qinv is a power of 2
    float ps = 0.f;
    h4 ph[4], pl[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float p = __builtin_amdgcn_exp2f(fmaf(qinv, s[j][r], c));
        ps += p;
        const float pw = p * pscale;
        ph[j][r] = (_Float16)pw;
        pl[j][r] = (_Float16)(pw - (float)ph[j][r]);
      }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = mn;
    vref = vnew;
    if (more) load_v(kb + 1);
    // ---- O^T = V^T P^T: dims 16t + 4fg + r x query fi, 32 keys per MFMA ----
    // The K = 32 step over keys 32c..32c+31 takes, in lane group fg, the keys
    // this lane's weights already hold: 32c + 4fg + r (tile 2c) and
    // 32c + 16 + 4fg + r (tile 2c + 1).  V^T's columns are read in the same
    // order, so the sum over k is the sum over the 32 keys.
    if (__any(oscale != 1.f)) {  // a new running max or V scale on some lane
#pragma unroll
      for (int t = 0; t < NT; t++) o[t] *= oscale;
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const h8 p8h = __builtin_shufflevector(ph[2 * c], ph[2 * c + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      const h8 p8l = __builtin_shufflevector(pl[2 * c], pl[2 * c + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      const int va = 32 * c + 4 * fg, vb = va + 16;
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const int vr = 16 * t + fi;
        const h4 vha = *(const h4*)&Vh[swzv(vr, va >> 3) + (va & 7)];
        const h4 vhb = *(const h4*)&Vh[swzv(vr, vb >> 3) + (vb & 7)];
        const h4 vla = *(const h4*)&Vl[swzv(vr, va >> 3) + (va & 7)];
        const h4 vlb = *(const h4*)&Vl[swzv(vr, vb >> 3) + (vb & 7)];
        const h8 vh8 = __builtin_shufflevector(vha, vhb, 0, 1, 2, 3, 4, 5, 6, 7);
        const h8 vl8 = __builtin_shufflevector(vla, vlb, 0, 1, 2, 3, 4, 5, 6, 7);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh8, p8h, o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh8, p8l, o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl8, p8h, o[t], 0, 0, 0);
        if (t % 4 == 3) __builtin_amdgcn_sched_barrier(0);  // V fragments of four tiles live at once
      }
    }
  }
  if (qt < a.n) {
    const float inv = ldexpf(1.f, vref - 14) / l;
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const int d = 16 * t + 4 * fg;
      if (d < HD)
        *(float4*)(a.out + (uint64_t)qt * qd + h * HD + d) =
            make_float4(o[t][0] * inv, o[t][1] * inv, o[t][2] * inv, o[t][3] * inv);
    }
  }
}

template <int HD>
hipError_t go(const AttnPrefillArgs& a, hipStream_t st) {
  using D = Dims<HD>;
  const PrepWs w = prep_ws(a.ws, a.n, a.n_kv_heads, D::HP);
  const uint32_t nkb = (a.n + kKB - 1) / kKB;
  if (a.kv_f16) hipLaunchKernelGGL((k_kv_prep<HD, _Float16>), dim3(nkb, a.n_kv_heads), dim3(kPrepThreads), 0, st, a, w);
  else hipLaunchKernelGGL((k_kv_prep<HD, float>), dim3(nkb, a.n_kv_heads), dim3(kPrepThreads), 0, st, a, w);
  const dim3 grid(((a.n + kQ - 1) / kQ) * a.n_heads);
  hipLaunchKernelGGL(k_attn_prefill<HD>, grid, dim3(kThreads), 0, st, a, w);
  return hipGetLastError();
}

}  // namespace

bool attn_prefill_head_dim(uint32_t hd) { return hd == 48 || hd == 64 || hd == 96 || hd == 128; }

uint64_t attn_prefill_ws_bytes(uint32_t n, uint32_t n_kv_heads, uint32_t head_dim) {
  return prep_ws_bytes(n, n_kv_heads, (head_dim + 31) / 32 * 32);
}

hipError_t launch_attn_prefill(const AttnPrefillArgs& a, hipStream_t st) {
  if (a.n == 0) return hipSuccess;
  if (a.n_kv_heads == 0 || a.n_heads % a.n_kv_heads || !a.ws) return hipErrorInvalidValue;
  switch (a.head_dim) {
    case 48: return go<48>(a, st);
    case 64: return go<64>(a, st);
    case 96: return go<96>(a, st);
    case 128: return go<128>(a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ifx
