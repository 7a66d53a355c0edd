// capi_attn.cpp — the decode step's attention, q/k/v and residual launches as
// operators of include/inferox.h (ifx_ops_attention_*, ifx_ops_qkv,
// ifx_ops_gemv_residual): the same launchers the captured step enqueues, on
// buffers the caller owns, so that each can be compared with the reference
// loops it replaces.  Each call allocates its small device state (the
// positions the kernels read, the chunk records or the split K/V), runs on the
// given stream and returns when the work is complete.
#include <math.h>

#include <algorithm>
#include <vector>

#include "ifx_common.h"
#include "kernels.h"

using namespace ifx;

namespace ifx {
int device_init();
hipStream_t ops_stream(void* s);
void rope_table_host(float base, uint64_t rope_dim, uint64_t n_pos, std::vector<float2>& out);
}  // namespace ifx

namespace {

// Device allocations of one call, freed after the stream has drained.
struct CallScratch {
  hipStream_t st = nullptr;
  std::vector<void*> ptrs;
  explicit CallScratch(hipStream_t s) : st(s) {}
  int alloc(void** p, size_t bytes) {
    if (hipMalloc(p, std::max<size_t>(bytes, 16)) != hipSuccess)
      return set_error(IFX_E_OOM, "hipMalloc(%zu) failed", bytes);
    ptrs.push_back(*p);
    return IFX_OK;
  }
  ~CallScratch() {
    if (!ptrs.empty()) (void)hipStreamSynchronize(st);
    for (void* p : ptrs) (void)hipFree(p);
  }
};

// The positions a step's kernels read: the token's cache row `len` (the
// attention covers rows [0, len]) and its RoPE position.
int put_state(CallScratch& cs, uint32_t len, uint32_t rope_pos, DevState** out) {
  IFX_TRY(cs.alloc((void**)out, sizeof(DevState)));
  DevState d{};
  d.len = len;
  d.rope_pos = rope_pos;
  d.top_p = 1.0f;
  IFX_HIP(hipMemcpy(*out, &d, sizeof d, hipMemcpyHostToDevice));
  return IFX_OK;
}

int check_kv_type(int kv_type) {
  if (kv_type != IFX_KV_F32 && kv_type != IFX_KV_F16) return set_error(IFX_E_INVALID_ARG, "kv_type %d", kv_type);
  return IFX_OK;
}

// Shape checks shared by the decode attention entry points; fills the launch
// arguments (a.partial and a.state are set by the caller).
int decode_args(const float* q, const void* k, const void* v, int kv_type, uint64_t max_seq, uint64_t n_rows,
                uint64_t n_heads, uint64_t n_kv, uint64_t hd, AttnArgs* a) {
  IFX_TRY(check_kv_type(kv_type));
  if (!q || !k || !v) return set_error(IFX_E_INVALID_ARG, "null buffer");
  if (max_seq == 0 || max_seq > 0x7fffffffull || n_rows == 0 || n_rows > max_seq)
    return set_error(IFX_E_INVALID_ARG, "attention over %llu rows of a %llu-row cache", (unsigned long long)n_rows,
                     (unsigned long long)max_seq);
  if (n_kv == 0 || n_heads % n_kv || n_heads / n_kv > 8 || n_heads > 4096 ||
      !attn_decode_head_dim((uint32_t)std::min<uint64_t>(hd, 1u << 20), kv_type == IFX_KV_F16))
    return set_error(IFX_E_INVALID_ARG, "attention shape (heads %llu/%llu, head_dim %llu) has no decode kernel",
                     (unsigned long long)n_heads, (unsigned long long)n_kv, (unsigned long long)hd);
  *a = AttnArgs{};
  a->q = q;
  a->k_cache = k;
  a->v_cache = v;
  a->n_heads = (uint32_t)n_heads;
  a->n_kv_heads = (uint32_t)n_kv;
  a->head_dim = (uint32_t)hd;
  a->chunk = 64;
  a->max_chunks = (uint32_t)((max_seq + 63) / 64);
  a->max_seq = (uint32_t)max_seq;
  a->kv_f16 = kv_type == IFX_KV_F16;
  return IFX_OK;
}

int alloc_records(CallScratch& cs, AttnArgs* a) {
  const uint64_t G = a->n_heads / a->n_kv_heads;
  return cs.alloc((void**)&a->partial,
                  (uint64_t)a->n_kv_heads * a->max_chunks * attn_partial_floats((uint32_t)G, a->head_dim) * 4);
}

GemvLaunch single(const ifx_tensor* w, const float* x) {
  GemvLaunch g;
  g.seg[0] = gemv_seg(w->L);
  g.nseg = 1;
  g.cols = (uint32_t)w->L.cols;
  g.x = x;
  return g;
}

}  // namespace

extern "C" {

int ifx_ops_attention_decode(const float* q, const void* k_cache, const void* v_cache, int kv_type, uint64_t max_seq,
                             uint64_t n_rows, uint64_t n_heads, uint64_t n_kv_heads, uint64_t head_dim, float* out,
                             void* stream) {
  clear_error();
  IFX_TRY(device_init());
  if (!out) return set_error(IFX_E_INVALID_ARG, "null output");
  AttnArgs a;
  IFX_TRY(decode_args(q, k_cache, v_cache, kv_type, max_seq, n_rows, n_heads, n_kv_heads, head_dim, &a));
  hipStream_t st = ops_stream(stream);
  CallScratch cs(st);
  DevState* state;
  IFX_TRY(put_state(cs, (uint32_t)(n_rows - 1), 0, &state));
  a.state = state;
  a.out = out;
  IFX_TRY(alloc_records(cs, &a));
  IFX_HIP(launch_attn_decode(a, st));
  IFX_HIP(hipStreamSynchronize(st));
  return IFX_OK;
}

int ifx_ops_attention_decode_o(const float* q, const void* k_cache, const void* v_cache, int kv_type,
                               uint64_t max_seq, uint64_t n_rows, uint64_t n_heads, uint64_t n_kv_heads,
                               uint64_t head_dim, const ifx_tensor* w_o, float* h, uint32_t merge_bound,
                               float* attn_out, void* stream) {
  clear_error();
  IFX_TRY(device_init());
  if (!w_o || !h) return set_error(IFX_E_INVALID_ARG, "null argument");
  AttnArgs a;
  IFX_TRY(decode_args(q, k_cache, v_cache, kv_type, max_seq, n_rows, n_heads, n_kv_heads, head_dim, &a));
  if (w_o->L.cols != n_heads * head_dim)
    return set_error(IFX_E_INVALID_ARG, "W_o has %llu columns, the attention output %llu",
                     (unsigned long long)w_o->L.cols, (unsigned long long)(n_heads * head_dim));
  hipStream_t st = ops_stream(stream);
  CallScratch cs(st);
  DevState* state;
  IFX_TRY(put_state(cs, (uint32_t)(n_rows - 1), 0, &state));
  a.state = state;
  IFX_TRY(alloc_records(cs, &a));
  float* attn = attn_out;
  if (!attn) IFX_TRY(cs.alloc((void**)&attn, n_heads * head_dim * 4));
  a.out = attn;
  const GemvLaunch go = single(w_o, attn);
  if (merge_bound) {
    if (!merge_o_supported(go, a))
      return set_error(IFX_E_INVALID_ARG, "the merge in the O projection needs 8 kv heads, head dim 128, 4 or 8 "
                                          "query heads per kv head and a K-split Q4_K/Q6_K W_o");
    IFX_HIP(launch_attn_partials(a, st));
    IFX_HIP(launch_mfma_residual_merge(go, a, h, st, merge_bound));
  } else {
    IFX_HIP(launch_attn_decode(a, st));
    IFX_HIP(gemv_residual(go, h, st));
  }
  IFX_HIP(hipStreamSynchronize(st));
  return IFX_OK;
}

int ifx_ops_attention_prefill(const float* q, const void* k_cache, const void* v_cache, int kv_type,
                              uint64_t max_seq, uint64_t row0, uint64_t n, uint64_t n_heads, uint64_t n_kv_heads,
                              uint64_t head_dim, int causal, float* out, void* stream) {
  clear_error();
  IFX_TRY(device_init());
  IFX_TRY(check_kv_type(kv_type));
  if (!q || !k_cache || !v_cache || !out) return set_error(IFX_E_INVALID_ARG, "null buffer");
  if (max_seq == 0 || max_seq > 0x7fffffffull || n == 0 || row0 > max_seq || n > max_seq - row0)
    return set_error(IFX_E_INVALID_ARG, "chunk of %llu rows at %llu in a %llu-row cache", (unsigned long long)n,
                     (unsigned long long)row0, (unsigned long long)max_seq);
  if (n_kv_heads == 0 || n_heads % n_kv_heads || n_heads > 4096 ||
      !attn_prefill_head_dim((uint32_t)std::min<uint64_t>(head_dim, 1u << 20)))
    return set_error(IFX_E_INVALID_ARG, "attention shape (heads %llu/%llu, head_dim %llu) has no prefill kernel",
                     (unsigned long long)n_heads, (unsigned long long)n_kv_heads, (unsigned long long)head_dim);
  hipStream_t st = ops_stream(stream);
  CallScratch cs(st);
  void* ws = nullptr;
  IFX_TRY(cs.alloc(&ws, attn_prefill_ws_bytes((uint32_t)n, (uint32_t)n_kv_heads, (uint32_t)head_dim)));
  const AttnPrefillArgs aa{q, k_cache, v_cache, out, (uint32_t)n, (uint32_t)row0, (uint32_t)n_heads,
                           (uint32_t)n_kv_heads, (uint32_t)head_dim, (uint32_t)max_seq, causal != 0, ws,
                           kv_type == IFX_KV_F16};
  IFX_HIP(launch_attn_prefill(aa, st));
  IFX_HIP(hipStreamSynchronize(st));
  return IFX_OK;
}

int ifx_ops_gemv_residual(const ifx_tensor* w, const float* x, float* h, int mode, int* path_out, void* stream) {
  clear_error();
  IFX_TRY(device_init());
  if (!w || !x || !h || (mode != 0 && mode != 1)) return set_error(IFX_E_INVALID_ARG, "bad argument");
  hipStream_t st = ops_stream(stream);
  const GemvLaunch g = single(w, x);
  int path = 0;
  if (mode == 0) {
    const hipError_t e = launch_mfma_residual_ks(g, h, st);
    if (e == hipSuccess) path = 1;
    else if (e != hipErrorNotSupported) IFX_HIP(e);
  }
  if (path == 0) IFX_HIP(gemv_residual_fixed(g, h, st));
  if (path_out) *path_out = path;
  IFX_HIP(hipStreamSynchronize(st));
  return IFX_OK;
}

int ifx_ops_qkv(const ifx_tensor* wq, const ifx_tensor* wk, const ifx_tensor* wv, const float* x, const float* norm_w,
                float eps, uint64_t head_dim, uint64_t rope_dim, float rope_base, uint64_t pos, float* q_out,
                void* k_cache, void* v_cache, int kv_type, uint64_t max_seq, uint64_t row, int mode, int* path_out,
                void* stream) {
  clear_error();
  IFX_TRY(device_init());
  IFX_TRY(check_kv_type(kv_type));
  if (!wq || !wk || !wv || !x || !norm_w || !q_out || !k_cache || !v_cache || (mode != 0 && mode != 1))
    return set_error(IFX_E_INVALID_ARG, "bad argument");
  const uint64_t D = wq->L.cols, kvd = wk->L.rows;
  if (wk->L.cols != D || wv->L.cols != D || wv->L.rows != kvd || head_dim == 0 || head_dim % 2 ||
      rope_dim > head_dim || rope_dim % 2 || wq->L.rows % head_dim || kvd % head_dim ||
      wq->L.type != wk->L.type || max_seq == 0 || max_seq > 0x7fffffffull || row >= max_seq ||
      pos >= (1ull << 17))
    return set_error(IFX_E_INVALID_ARG, "q/k/v shapes or cache row out of range");
  const bool kv16 = kv_type == IFX_KV_F16;
  hipStream_t st = ops_stream(stream);
  CallScratch cs(st);
  DevState* state;
  IFX_TRY(put_state(cs, (uint32_t)row, (uint32_t)pos, &state));
  std::vector<float2> tab;
  rope_table_host(rope_base, rope_dim, pos + 1, tab);
  float2* rope_cs = nullptr;
  IFX_TRY(cs.alloc((void**)&rope_cs, tab.size() * sizeof(float2)));
  IFX_HIP(hipMemcpy(rope_cs, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice));
  GemvLaunch g;
  g.seg[0] = gemv_seg(wq->L);
  g.seg[1] = gemv_seg(wk->L);
  g.seg[2] = gemv_seg(wv->L);
  g.nseg = 3;
  g.cols = (uint32_t)D;
  g.x = x;
  g.norm_w = norm_w;
  g.eps = eps;
  const QkvDst d{q_out, (float*)k_cache, (float*)v_cache, rope_cs, state, (uint32_t)head_dim, (uint32_t)rope_dim,
                 (uint32_t)max_seq};
  const bool split = mode == 0 && !kv16 && qkv_ks_supported(g, d);
  if (split) {
    // the K-split launch adds into q and the new cache rows: cleared first
    IFX_HIP(launch_fill_u32((uint32_t*)q_out, 0u, wq->L.rows, st));
    for (uint64_t hk = 0; hk < kvd / head_dim; hk++) {
      const uint64_t off = (hk * max_seq + row) * head_dim;
      IFX_HIP(launch_fill_u32((uint32_t*)k_cache + off, 0u, head_dim, st));
      IFX_HIP(launch_fill_u32((uint32_t*)v_cache + off, 0u, head_dim, st));
    }
    IFX_HIP(launch_qkv_ks(g, d, st));
  } else {
    const QkvEpi e{q_out, k_cache, v_cache, rope_cs, state, (uint32_t)head_dim, (uint32_t)rope_dim, (uint32_t)kvd,
                   (uint32_t)max_seq, kv16 ? 1u : 0u};
    IFX_HIP(gemv_qkv(g, e, st));
  }
  if (path_out) *path_out = split ? 1 : 0;
  IFX_HIP(hipStreamSynchronize(st));
  return IFX_OK;
}

}  // extern "C"
