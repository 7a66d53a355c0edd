// kern_attn_prefill.hip — attention of a prefill chunk on the fp16 matrix
// cores (src/model/forward.rs:215-337, the batched Layer::prefill; non-causal
// for Layer::forward, src/model/forward.rs:62-207).  Query row t of head h
// attends to the K/V cache rows row0 .. row0 + t (causal) or row0 .. row0 + n - 1
// of kv head h / (n_heads / n_kv_heads): s = (q . k) / sqrt(head_dim), softmax,
// o = p V (src/model/forward.rs:383-414 per row, src/ops.rs:223-239).
//
// Arithmetic as in kern_gemm.hip: both products run on
// v_mfma_f32_16x16x32_f16 with each operand an fp16 hi/lo pair (three MFMAs
// per step, f32 accumulation), within the rounding of the f32 reference.  The
// fp16 range is kept by power-of-2 scales: per query row and per key row for
// q . k (undone per score: the key scale is per lane, each lane holding one
// key column of the score tile), and one per 64-row V block (P V of a block
// lands in a temporary and is added as tmp / s).  Softmax weights lie in
// [0, 1].
//
// A workgroup of 4 waves owns 64 query rows of one head and walks the key
// blocks of 64 rows with the running-max softmax; wave w owns queries
// 16w .. 16w + 15: scores as a 16 x 64 tile (4 MFMA tiles), the weights through
// the wave's LDS slab into A-operand order, O as head_dim / 16 tiles.  V is
// staged transposed so that B fragments are contiguous.  The head dim is padded
// to a multiple of 32 with zeros.
#include "kernels.h"

namespace ifx {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kQ = 64, kKB = 64, kThreads = 256;

__device__ __forceinline__ f4 mfma3(h8 ah, h8 al, h8 bh, h8 bl, f4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, c, 0, 0, 0);
}

__device__ __forceinline__ int exp_of(uint32_t bits) {
  const int e = (int)((bits >> 23) & 255u) - 127;
  return e < -100 ? -100 : e;
}

// LDS row of W halves in 16-byte chunks; logical chunk c of row r sits at
// c ^ x(r), x chosen so that the 16 consecutive rows of a fragment read at one
// logical chunk land on 16 distinct 4-bank groups: rows of 256 bytes start on
// the same bank (x = r mod 16), rows of 128 bytes on two (x = r / 2 mod 8),
// rows of 64 or 192 bytes on four (x = r / 4 mod 4).
template <int W>
__device__ __forceinline__ int swz(int r, int c) {
  constexpr int RB = 2 * W;
  const int x = (RB % 256 == 0) ? (r & 15) : (RB % 128 == 0) ? ((r >> 1) & 7) : ((r >> 2) & 3);
  return r * W + 8 * (c ^ x);
}

__device__ __forceinline__ void split8(const float* y, float scale, h8& hi, h8& lo) {
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const float v = y[k] * scale;
    const _Float16 x = (_Float16)v;
    hi[k] = x;
    lo[k] = (_Float16)(v - (float)x);
  }
}

template <int HD>
__global__ void __launch_bounds__(kThreads) k_attn_prefill(AttnPrefillArgs a) {
  constexpr int HP = (HD + 31) / 32 * 32;  // padded head dim (halves per Q/K row)
  constexpr int NCH = HP / 8;              // 16-byte chunks per Q/K row
  constexpr int NT = HD / 16;              // output tiles per wave
  constexpr int NKS = HP / 32;             // MFMA steps over the head dim
  constexpr int KCH = NCH / 2;             // K staging: two threads per key row
  constexpr int QCH = NCH / 4;             // Q staging: four threads per query row
  extern __shared__ __attribute__((aligned(16))) _Float16 sm[];
  _Float16* Qh = sm;                  // [kQ][HP]
  _Float16* Ql = Qh + kQ * HP;
  _Float16* Kh = Ql + kQ * HP;        // [kKB][HP]
  _Float16* Kl = Kh + kKB * HP;
  _Float16* Vh = Kl + kKB * HP;       // [HP][kKB] (transposed)
  _Float16* Vl = Vh + HP * kKB;
  _Float16* Pb = Vl + HP * kKB;       // per wave [2][16][kKB]
  __shared__ int qexp[kQ], kexp[kKB];
  __shared__ float vwmax[2];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fi = lane & 15, fg = lane >> 4;
  // heaviest query blocks of every head first
  const uint32_t nqb = (a.n + kQ - 1) / kQ;
  const uint32_t qb = nqb - 1 - blockIdx.x / a.n_heads, h = blockIdx.x % a.n_heads;
  const uint32_t q0 = qb * kQ, group = a.n_heads / a.n_kv_heads, hk = h / group;
  const uint32_t qd = a.n_heads * HD;
  const float sqrt_hd = sqrtf((float)HD);

  // ---- Q block: four threads per row, row scale by shuffles ----
  {
    const int r = tid >> 2, qq = tid & 3;
    const uint32_t t = q0 + (uint32_t)r;
    float v[QCH][8];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < QCH; i++) {
      const int col = 8 * (qq * QCH + i);
      float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
      if (t < a.n && col < HD) {
        const float* src = a.q + (uint64_t)t * qd + h * HD + col;
        x0 = *(const float4*)src;
        x1 = *(const float4*)(src + 4);
      }
      v[i][0] = x0.x; v[i][1] = x0.y; v[i][2] = x0.z; v[i][3] = x0.w;
      v[i][4] = x1.x; v[i][5] = x1.y; v[i][6] = x1.z; v[i][7] = x1.w;
#pragma unroll
      for (int k = 0; k < 8; k++) mx = fmaxf(mx, fabsf(v[i][k]));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    const int e = exp_of(__float_as_uint(mx));
    if (qq == 0) qexp[r] = e;
    const float sc = ldexpf(1.f, 14 - e);
#pragma unroll
    for (int i = 0; i < QCH; i++) {
      h8 hi, lo;
      split8(v[i], sc, hi, lo);
      *(h8*)&Qh[swz<HP>(r, qq * QCH + i)] = hi;
      *(h8*)&Ql[swz<HP>(r, qq * QCH + i)] = lo;
    }
  }

  f4 o[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) o[t] = f4{0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    m[r] = -INFINITY;
    l[r] = 0.f;
  }

  const uint32_t last_q = min(q0 + kQ, a.n) - 1;
  const uint32_t kend = a.causal ? last_q + 1 : a.n;  // keys [0, kend)
  const uint32_t nkb = (kend + kKB - 1) / kKB;
  _Float16* Ph = Pb + wave * 2 * 16 * kKB;
  _Float16* Pl = Ph + 16 * kKB;

  // K/V staging roles: waves 0-1 stage K rows (two threads per row, KCH chunks
  // each), waves 2-3 stage V as 8 x 8 tiles (8 keys x 8 dims) for the transpose
  const bool krole = tid < 128;
  const int kr = tid >> 1, khalf = tid & 1;  // K role
  const int vt = tid - 128, vkc = vt / NCH, vdc = vt % NCH;  // V role (vt < 8 NCH)
  const bool vtile = !krole && vt < 8 * NCH;
  float st[64];  // the next block's K chunks or V tile, loaded one block ahead
  auto load_block = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
      if (krole) {
        const int col = 8 * (khalf * KCH + i);
        const uint32_t key = k0 + (uint32_t)kr;
        if (i < KCH && key < kend && col < HD) {
          const float* src = a.k_cache + ((uint64_t)hk * a.max_seq + a.row0 + key) * HD + col;
          x0 = *(const float4*)src;
          x1 = *(const float4*)(src + 4);
        }
      } else {
        const int col = 8 * vdc;
        const uint32_t key = k0 + (uint32_t)(8 * vkc + i);
        if (vtile && key < kend && col < HD) {
          const float* src = a.v_cache + ((uint64_t)hk * a.max_seq + a.row0 + key) * HD + col;
          x0 = *(const float4*)src;
          x1 = *(const float4*)(src + 4);
        }
      }
      st[8 * i] = x0.x; st[8 * i + 1] = x0.y; st[8 * i + 2] = x0.z; st[8 * i + 3] = x0.w;
      st[8 * i + 4] = x1.x; st[8 * i + 5] = x1.y; st[8 * i + 6] = x1.z; st[8 * i + 7] = x1.w;
    }
  };
  load_block(0);
  for (uint32_t kb = 0; kb < nkb; kb++) {
    const uint32_t k0 = kb * kKB;
    // phase A: maxima of the staged block
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < 64; k++) mx = fmaxf(mx, fabsf(st[k]));
    if (krole) {
      mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    } else {
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      if (lane == 0) vwmax[wave - 2] = mx;
    }
    // every wave is past the previous block's K/V/P reads
    __syncthreads();
    // phase B: hi/lo into LDS
    if (krole) {
      const int e = exp_of(__float_as_uint(mx));
      if (khalf == 0) kexp[kr] = e;
      const float sc = ldexpf(1.f, 14 - e);
#pragma unroll
      for (int i = 0; i < KCH; i++) {
        h8 hi, lo;
        split8(&st[8 * i], sc, hi, lo);
        *(h8*)&Kh[swz<HP>(kr, khalf * KCH + i)] = hi;
        *(h8*)&Kl[swz<HP>(kr, khalf * KCH + i)] = lo;
      }
    } else if (vtile) {
      const int e = exp_of(__float_as_uint(fmaxf(vwmax[0], vwmax[1])));
      const float sc = ldexpf(1.f, 14 - e);
#pragma unroll
      for (int d = 0; d < 8; d++) {  // V^T row 8 vdc + d: keys 8 vkc .. 8 vkc + 7
        float col[8];
#pragma unroll
        for (int k = 0; k < 8; k++) col[k] = st[8 * k + d];
        h8 hi, lo;
        split8(col, sc, hi, lo);
        *(h8*)&Vh[swz<kKB>(8 * vdc + d, vkc)] = hi;
        *(h8*)&Vl[swz<kKB>(8 * vdc + d, vkc)] = lo;
      }
    }
    __syncthreads();
    // the next block's loads fly during this block's products
    if (kb + 1 < nkb) load_block(k0 + kKB);
    const int ve = exp_of(__float_as_uint(fmaxf(vwmax[0], vwmax[1])));
    const float vinv = ldexpf(1.f, ve - 14);
    float qinv[4], kinv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) qinv[r] = ldexpf(1.f, qexp[16 * wave + 4 * fg + r] - 14);
#pragma unroll
    for (int j = 0; j < 4; j++) kinv[j] = ldexpf(1.f, kexp[16 * j + fi] - 14);

    // ---- scores: 16 queries of this wave x 64 keys ----
    f4 s[4];
#pragma unroll
    for (int j = 0; j < 4; j++) s[j] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) {
      const int qr = 16 * wave + fi;
      const h8 ah = *(const h8*)&Qh[swz<HP>(qr, 4 * ks + fg)];
      const h8 al = *(const h8*)&Ql[swz<HP>(qr, 4 * ks + fg)];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int krow = 16 * j + fi;
        const h8 bh = *(const h8*)&Kh[swz<HP>(krow, 4 * ks + fg)];
        const h8 bl = *(const h8*)&Kl[swz<HP>(krow, 4 * ks + fg)];
        s[j] = mfma3(ah, al, bh, bl, s[j]);
      }
    }
    // scale, mask, running max / sum; weights to LDS in A-operand order
    float alpha[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t qt = q0 + 16 * wave + 4 * fg + r;
      float bm = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t key = k0 + 16 * j + fi;
        const bool ok = key < kend && (!a.causal || key <= qt);
        s[j][r] = ok ? (s[j][r] * (qinv[r] * kinv[j])) / sqrt_hd : -INFINITY;
        bm = fmaxf(bm, s[j][r]);
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) bm = fmaxf(bm, __shfl_xor(bm, off, 64));
      const float mn = fmaxf(m[r], bm);
      alpha[r] = mn == -INFINITY ? 1.f : expf(m[r] - mn);
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float p = mn == -INFINITY ? 0.f : expf(s[j][r] - mn);
        ps += p;
        const _Float16 ph = (_Float16)p;
        const int row = 4 * fg + r, col = 16 * j + fi;
        Ph[swz<kKB>(row, col >> 3) + (col & 7)] = ph;
        Pl[swz<kKB>(row, col >> 3) + (col & 7)] = (_Float16)(p - (float)ph);
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) ps += __shfl_xor(ps, off, 64);
      l[r] = l[r] * alpha[r] + ps;
      m[r] = mn;
    }
    __syncthreads();  // the weights written by all lanes are visible
    // ---- O = alpha O + (P V_scaled) / s_v ----
    h8 pah[kKB / 32], pal[kKB / 32];
#pragma unroll
    for (int ks = 0; ks < kKB / 32; ks++) {
      pah[ks] = *(const h8*)&Ph[swz<kKB>(fi, 4 * ks + fg)];
      pal[ks] = *(const h8*)&Pl[swz<kKB>(fi, 4 * ks + fg)];
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      f4 tmp = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kKB / 32; ks++) {
        const h8 bh = *(const h8*)&Vh[swz<kKB>(16 * t + fi, 4 * ks + fg)];
        const h8 bl = *(const h8*)&Vl[swz<kKB>(16 * t + fi, 4 * ks + fg)];
        tmp = mfma3(pah[ks], pal[ks], bh, bl, tmp);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) o[t][r] = o[t][r] * alpha[r] + tmp[r] * vinv;
    }
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t t = q0 + 16 * wave + 4 * fg + r;
    if (t >= a.n) continue;
    const float inv = 1.0f / l[r];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) a.out[(uint64_t)t * qd + h * HD + 16 * tt + fi] = o[tt][r] * inv;
  }
}

template <int HD>
hipError_t go(const AttnPrefillArgs& a, hipStream_t st) {
  constexpr int HP = (HD + 31) / 32 * 32;
  const size_t lds = ((size_t)2 * kQ * HP + (size_t)2 * kKB * HP + (size_t)2 * HP * kKB + (size_t)4 * 2 * 16 * kKB) * 2;
  static bool opted = false;
  if (!opted) {
    hipError_t e = hipFuncSetAttribute((const void*)k_attn_prefill<HD>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    opted = true;
  }
  dim3 grid(((a.n + kQ - 1) / kQ) * a.n_heads);
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
