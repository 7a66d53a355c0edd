// kernels.h — host-side launchers of the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dev_quant.h"
#include "ifx_common.h"

namespace ifx {

// Per-session state that lives in device memory, so that one captured decode
// step replays correctly for every token (the kernels read positions from here,
// the finalize kernel advances them).
struct DevState {
  uint32_t len;          // cache rows holding keys/values before the current token
  uint32_t rope_pos;     // RoPE position of the current token
  uint32_t attn_lo;      // first cache row the current token attends to
  uint32_t cur_token;    // token fed to the next step's embedding gather
  uint32_t step;         // next slot of out_tokens
  uint32_t rope_mode;    // IFX_ROPE_REFERENCE / IFX_ROPE_ABSOLUTE
  uint32_t prefill;      // 1 while a prefill chunk is being fed
  uint32_t chunk_start;  // cache index of the first token of the prefill chunk
  uint32_t feed_n;       // tokens in feed_ids (prefill)
  int32_t status;        // IFX_OK, or IFX_E_NAN_LOGIT once a NaN logit was seen
  unsigned long long argmax_key;  // packed (ordered logit << 32 | index), max-reduced
  const uint32_t* feed_ids;       // prefill token ids (device)
  uint32_t* out_tokens;           // greedy picks (device)
  uint32_t out_cap;
  uint32_t attn_end;     // 0: attend rows [attn_lo, len]; else rows [attn_lo, attn_end)
  // sampler (kern_sample.hip; temperature 0: the greedy argmax)
  float temperature;
  uint32_t top_k;
  float top_p;
  unsigned long long seed;
};

// Where the K-split q/k/v launch adds its rows (launch_qkv_ks): q, and row
// state->len of the layer's f32 K and V caches ([n_kv][max_seq][head_dim]),
// all cleared beforehand (QkvClear); RoPE at state->rope_pos from rope_cs.
struct QkvDst {
  float* q;
  float* k_cache;
  float* v_cache;
  const float2* rope_cs;
  const DevState* state;
  uint32_t head_dim, rope_dim, max_seq;
};
// Rows a launch clears for K-split q/k/v launches, for each of n_layers
// layers: q[0, nq) (layer l's at q + l q_stride) and, for each of n_kv kv
// heads, row state->len (head_dim floats) of the K and V caches (layer l's at
// k_cache / v_cache + l kv_stride).  A null q clears nothing.
struct QkvClear {
  float* q = nullptr;
  float* k_cache = nullptr;
  float* v_cache = nullptr;
  const DevState* state = nullptr;
  uint32_t nq = 0, n_kv = 0, head_dim = 0, max_seq = 0;
  uint32_t n_layers = 1;
  uint64_t q_stride = 0, kv_stride = 0;  // floats
  __host__ __device__ uint64_t floats() const { return q ? (uint64_t)n_layers * (nq + 2ull * n_kv * head_dim) : 0; }
};
// workgroup wg of nwg clears its share, with threads tid of nthreads; len is
// c.state->len, read by the caller early (a read here would put its round trip
// where the clear is placed)
__device__ inline void qkv_clear(const QkvClear& c, uint32_t len, uint32_t wg, uint32_t nwg, uint32_t tid,
                                 uint32_t nthreads) {
  if (!c.q) return;
  const uint32_t nkv = c.n_kv * c.head_dim, layer_n = c.nq + 2 * nkv, total = (uint32_t)c.floats();
  const uint32_t per = (total + nwg - 1) / nwg, base = wg * per;
  for (uint32_t i = tid; i < per; i += nthreads) {
    const uint32_t e0 = base + i;
    if (e0 >= total) break;
    const uint32_t layer = e0 / layer_n, e = e0 % layer_n;
    // agent-scope stores, as the atomic adds that follow: they leave no dirty
    // line in this XCD's L2 (plain stores cost the launch ~0.5 us, the L2
    // write-back at its end)
    float* p;
    if (e < c.nq) {
      p = c.q + layer * c.q_stride + e;
    } else {
      const uint32_t f = e - c.nq, r = f % nkv;
      float* cache = (f >= nkv ? c.v_cache : c.k_cache) + layer * c.kv_stride;
      p = cache + ((uint64_t)(r / c.head_dim) * c.max_seq + len) * c.head_dim + r % c.head_dim;
    }
    __hip_atomic_store(p, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---- dequantization (kern_dequant.hip) ----
hipError_t launch_dequant_raw(uint32_t type, const uint8_t* bytes, uint64_t n, float* out,
                              hipStream_t st);
hipError_t launch_dequant_dev(const DevW& w, uint64_t n, float* out, hipStream_t st);
hipError_t launch_embed_rows(const DevW& w, const uint32_t* ids, uint64_t n_ids, float* out,
                             hipStream_t st);
// hidden[cols] = row state->cur_token of the table
// clr: rows cleared for the step's K-split q/k/v launches (extra workgroups
// take them, 1024 floats each)
hipError_t launch_embed_state(const DevW& w, const DevState* state, float* hidden, hipStream_t st,
                              const QkvClear& clr = QkvClear{});

// ---- fused GEMV (kern_gemv.hip) ----
struct GemvSeg {
  const uint8_t* body;
  const uint8_t* scal;
  uint32_t type;
  uint32_t rows;
  uint32_t q6_signed;  // Q6_K with int8 scale bytes (ggml's layout)
  uint64_t tstride, bstride;  // Q4_K / Q6_K: unit (t, b) at body + t tstride + b bstride (tile_strides)
};
inline GemvSeg gemv_seg(const DevLayout& L) {
  GemvSeg s{L.body, L.scal, L.type, (uint32_t)L.rows, L.q6_signed, 0, 0};
  if (L.type == T_Q4K || L.type == T_Q6K) tile_strides(L.type, L.rows, &s.tstride, &s.bstride);
  return s;
}

struct GemvLaunch {
  GemvSeg seg[3];
  int nseg = 0;
  uint32_t cols = 0;
  const float* x = nullptr;       // input vector [cols]
  const float* norm_w = nullptr;  // non-null: x := rms_norm(x, norm_w, eps) in the prologue
  float eps = 0.f;
  bool paired = false;            // seg[0]/seg[1] rows interleaved per tile (gate/up)
};

// The device KV cache is head-major: per layer [n_kv_heads][max_seq][head_dim]
// f32 (or binary16 in a session created with IFX_KV_F16), so a kv head's rows
// are contiguous for the attention kernels (the reference's [t][kv_dim] row
// order is what ifx_kv_import/export exchange).
struct QkvEpi {
  float* q_out;          // [q rows]
  void* k_cache;         // layer base, [n_kv_heads][max_seq][head_dim] f32, or f16 when kv_f16
  void* v_cache;
  const float2* rope_cs; // [max_pos][rope_dim/2] (cos, sin)
  const DevState* state;
  uint32_t head_dim, rope_dim, kv_dim, max_seq;
  uint32_t kv_f16;
};

hipError_t gemv_store(const GemvLaunch& L, float* y, hipStream_t st);
// h += W x: the K-split launch where it applies (its slices' partial sums are
// added with atomics, so the last bits may differ between runs), else the
// tiled launch
hipError_t gemv_residual(const GemvLaunch& L, float* hidden, hipStream_t st);
// h += W x by the tiled launch only: each row's sum formed in one fixed order
hipError_t gemv_residual_fixed(const GemvLaunch& L, float* hidden, hipStream_t st);
hipError_t gemv_qkv(const GemvLaunch& L, const QkvEpi& e, hipStream_t st);
hipError_t gemv_swiglu(const GemvLaunch& L, float* mid, hipStream_t st);
hipError_t gemv_logits(const GemvLaunch& L, float* logits, DevState* state, hipStream_t st);
int gemv_supported(uint32_t type);

// ---- batched prefill GEMM (kern_gemm.hip) ----
// A weight matrix as the GEMM reads it (the device layout of ifx_common.h).
struct GemmW {
  const uint8_t* body;
  const uint8_t* scal;
  uint32_t type;
  uint32_t rows;
  uint64_t cols;
  uint32_t q6_signed;  // Q6_K with int8 scale bytes (ggml's layout)
  uint64_t tstride, bstride;  // Q4_K / Q6_K: unit (t, b) at body + t tstride + b bstride (tile_strides)
};
inline GemmW gemm_w(const DevLayout& L) {
  GemmW w{L.body, L.scal, L.type, (uint32_t)L.rows, L.cols, L.q6_signed, 0, 0};
  if (L.type == T_Q4K || L.type == T_Q6K) tile_strides(L.type, L.rows, &w.tstride, &w.bstride);
  return w;
}
// The activation operand as k_prep_rows leaves it (launch_prep_rows): m rows
// of k columns scaled per row into the fp16 range and split into hi + lo fp16
// planes, the 32-element group sums, and each row's scale exponent.
struct GemmIn {
  const uint16_t* hi;    // [m][k] fp16 bits
  const uint16_t* lo;    // [m][k]
  const uint16_t* gsum;  // [m][k / 256][16] (needed by Q4_K weights; k % 256 == 0)
  const int* rexp;       // [m]
  uint32_t m, k;
  float* part = nullptr;     // optional workspace for split-K partial tiles
  uint64_t part_bytes = 0;
};
bool gemm_type(uint32_t type);
// y[t * ldy + n] = (A W^T)[t][n]
hipError_t gemm_store(const GemmIn& in, const GemmW& w, float* y, uint32_t ldy, hipStream_t st);
// x[t * ldx + n] += (A W^T)[t][n]
hipError_t gemm_residual(const GemmIn& in, const GemmW& w, float* x, uint32_t ldx, hipStream_t st);
// Output (t, n) of the q/k/v GEMMs goes to y[(row0 + t) ldy + (n / head_dim) hstride + n % head_dim]:
// row-major [t][heads * head_dim] with ldy = heads * head_dim, hstride = head_dim;
// the head-major KV cache with ldy = head_dim, hstride = max_seq * head_dim.
// y is f32, or binary16 (rounded to nearest even) when y_f16.
// RoPE at position pos0 + t
hipError_t gemm_rope(const GemmIn& in, const GemmW& w, void* y, uint32_t ldy, uint64_t hstride, uint32_t row0,
                     uint32_t pos0, uint32_t head_dim, uint32_t rope_dim, const float2* cs, hipStream_t st,
                     bool y_f16 = false);
// the V cache append
hipError_t gemm_rows(const GemmIn& in, const GemmW& w, void* y, uint32_t ldy, uint64_t hstride, uint32_t row0,
                     uint32_t head_dim, hipStream_t st, bool y_f16 = false);
// mid[t * ld + n] = swiglu(gate row n . A[t], up row n . A[t])
hipError_t gemm_swiglu(const GemmIn& in, const GemmW& gate, const GemmW& up, float* mid, uint32_t ld,
                       hipStream_t st);
// rows x cols of x (row stride ld), rms_norm'ed with norm_w when non-null
// (src/ops.rs:155-180), into the GEMM operand `out` (out.k == cols, rows <= out.m)
hipError_t launch_prep_rows(const float* x, uint32_t rows, uint32_t ld, uint32_t cols, const float* norm_w,
                            float eps, const GemmIn& out, hipStream_t st);

// ---- batched prefill attention (kern_attn_prefill.hip) ----
// Attention of n query rows over the chunk's keys (src/model/forward.rs:
// 215-337): query t (q row t) attends to cache rows row0 .. row0 + t
// (causal) or row0 .. row0 + n - 1; out[t] f32, the row's max |out| in rowmax.
struct AttnPrefillArgs {
  const float* q;        // [n][n_heads * head_dim]
  const void* k_cache;   // layer base [n_kv_heads][max_seq][head_dim], f32 or (kv_f16) f16
  const void* v_cache;
  float* out;            // [n][n_heads * head_dim]
  uint32_t n, row0, n_heads, n_kv_heads, head_dim, max_seq;
  bool causal;
  void* ws;              // attn_prefill_ws_bytes(n, n_kv_heads, head_dim): the split K/V
  bool kv_f16;
};
bool attn_prefill_head_dim(uint32_t head_dim);
uint64_t attn_prefill_ws_bytes(uint32_t n, uint32_t n_kv_heads, uint32_t head_dim);
hipError_t launch_attn_prefill(const AttnPrefillArgs& a, hipStream_t st);

// ---- small ops (kern_ops.hip) ----
hipError_t launch_matmul_t_f32(const float* a, const float* b, float* c, uint64_t m, uint64_t n,
                               uint64_t k, hipStream_t st);
hipError_t launch_rms_norm_rows(float* x, const float* w, uint64_t n, uint64_t rows, float eps,
                                hipStream_t st);
hipError_t launch_swiglu(const float* g, const float* u, float* o, uint64_t n, hipStream_t st);
hipError_t launch_add(float* o, const float* b, uint64_t n, hipStream_t st);
hipError_t launch_softmax_rows(float* x, uint64_t rows, uint64_t cols, hipStream_t st);
hipError_t launch_rope(float* x, uint64_t seq, uint64_t heads, uint64_t hd, uint64_t rope_dim,
                       float base, uint64_t pos0, hipStream_t st);
hipError_t launch_argmax(const float* x, uint64_t n, uint32_t* out, int* status, hipStream_t st);
hipError_t launch_finalize(DevState* state, hipStream_t st);
enum StateKind : uint32_t { STATE_RESET, STATE_MODE, STATE_DECODE, STATE_PREFILL, STATE_TOKEN_AT, STATE_BATCH,
                            STATE_SAMPLER };
// ---- sampling (kern_sample.hip) ----
// The sampler's device scratch: a histogram of the probabilities (counts and
// masses packed per bin), each sweeping workgroup's sum, the candidate list
// and the draw's plan.  Zeroed once when allocated; every draw leaves the
// histogram and the candidate count zero again for the next.
struct SampleCtl {
  uint32_t count;  // candidates appended by the gather
  uint32_t mode;   // the plan: 1 draw over all, 2 candidates, 3 more candidates than the select sorts
  uint32_t lo_bin, n_cand;
};
struct SampleWs {
  unsigned long long* hist;
  float* part;
  uint2* cand;  // (index, probability bits)
  SampleCtl* ctl;
};
size_t sample_ws_bytes();
SampleWs sample_ws(void* base);  // the scratch carved from sample_ws_bytes() zeroed bytes
// Overrides state->argmax_key with a temperature / top-k / top-p draw from
// logits[vocab] when state->temperature > 0 (probs: vocab floats of scratch).
// state->argmax_key must hold the maximum logit's key on entry (the head's
// greedy argmax, or launch_logits_max).
hipError_t launch_sample(const float* logits, float* probs, const SampleWs& ws, uint32_t vocab, DevState* state,
                         hipStream_t st);
// state->argmax_key and state->status from logits[vocab], as the head's
// argmax leaves them (for draws from logits the host supplies).
hipError_t launch_logits_max(const float* logits, uint32_t vocab, DevState* state, hipStream_t st);
struct StateOp {
  uint32_t kind;
  uint32_t value;
  uint32_t len;
  float f0 = 0.f, f1 = 0.f;  // STATE_SAMPLER: temperature, top_p (value: top_k)
  unsigned long long seed = 0;
};
hipError_t launch_state(DevState* state, const StateOp& op, hipStream_t st);
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, uint64_t n, hipStream_t st);

// ---- attention (kern_attn.hip) ----
struct AttnArgs {
  const float* q;        // [n_heads * head_dim]
  const void* k_cache;   // layer base [n_kv_heads][max_seq][head_dim], f32 or (kv_f16) f16
  const void* v_cache;
  float* out;            // [n_heads * head_dim]
  float* partial;        // [n_kv][max_chunks][attn_partial_floats(group, head_dim)]
  const DevState* state;
  uint32_t n_heads, n_kv_heads, head_dim, max_chunks, chunk, max_seq;
  uint32_t kv_f16;
  uint32_t hk_fast = 0;  // chunk grid ordered kv head fastest (set by the launcher)
};
hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t st);
// the chunk records only (their merge is left to launch_mfma_residual_merge)
hipError_t launch_attn_partials(const AttnArgs& a, hipStream_t st);
// The O projection h += W_o x with the attention's merge in its prologue
// (kern_gemv_mfma.hip): x is formed from a.partial, the chunk records that
// launch_attn_partials left, for the rows a.state attends.  Needs 8 kv heads,
// head dim 128, 4 or 8 query heads per kv head and a K-split launch of
// W_o (merge_o_supported).  Any chunk count: the first min(first,
// merge_o_first_chunks()) records are loaded with the prologue (without
// waiting for the state), the rest in a loop; `first` is best a bound a
// little above the steps' chunk count (a multiple of merge_o_bound_step()).
bool merge_o_supported(const GemvLaunch& L, const AttnArgs& a);
hipError_t launch_mfma_residual_merge(const GemvLaunch& L, const AttnArgs& a, float* h, hipStream_t st,
                                      uint32_t first);
// h += W x with K split over workgroups (kern_gemv_mfma.hip); returns
// hipErrorNotSupported for launches it does not take
hipError_t launch_mfma_residual_ks(const GemvLaunch& L, float* h, hipStream_t st);
// q/k/v of rms_norm(x) as one K-split launch (kern_gemv_mfma.hip): segments
// q, k, v of L (Q4_K / Q6_K, q and k of one type, with the norm, whole heads),
// added into d's targets.
bool qkv_ks_supported(const GemvLaunch& L, const QkvDst& d);
hipError_t launch_qkv_ks(const GemvLaunch& L, const QkvDst& d, hipStream_t st);
uint32_t merge_o_first_chunks();
uint32_t merge_o_bound_step();
// head dims the decode attention takes: multiples of 4 (f32 cache) or 8 (f16) up to 256
bool attn_decode_head_dim(uint32_t head_dim, bool kv_f16);
// floats of one partial record (per kv head and chunk): o[group][head_dim],
// max[group], sum[group], padded to a multiple of 4
__host__ __device__ inline uint32_t attn_partial_floats(uint32_t group, uint32_t head_dim) {
  return (group * head_dim + 2 * group + 3) & ~3u;
}

}  // namespace ifx
