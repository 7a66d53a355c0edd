// host_model.cpp — model upload, sessions and the token loop behind the model
// half of include/inferox.h.
//
// Model::open (src/model/mod.rs:64-92) + Config::from_gguf
// (src/model/config.rs:34-84), with every weight uploaded to HBM once in its
// quantized form.  A session owns the device KV cache (the reference's
// KvCache, src/model/cache.rs:8-24, same [t][kv_dim] f32 rows per layer), the
// scratch of DecodeBuffers, a HIP stream and one captured decode step that is
// replayed for every token (positions live in device memory).
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <thread>
#include <vector>

#include "host_config.h"
#include "host_gguf.h"
#include "ifx_common.h"
#include "kernels.h"

using namespace ifx;

namespace ifx {
int device_init();
int upload_matrix(uint32_t type, const uint8_t* src, uint64_t nbytes, uint64_t rows, uint64_t cols,
                  ifx_tensor** out, uint32_t flags);
DevW devw(const ifx_tensor* t);
}  // namespace ifx

struct LayerDev {
  ifx_tensor *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
  ifx_tensor *gate = nullptr, *up = nullptr, *down = nullptr;
  float *attn_norm = nullptr, *ffn_norm = nullptr;
};

struct ifx_model {
  uint32_t flags = 0;  // IFX_OPEN_* of ifx_model_open_ex
  MappedFile map;
  GgufFile gguf;
  ifx_config cfg{};
  std::vector<LayerDev> layers;
  ifx_tensor* embd = nullptr;
  ifx_tensor* output = nullptr;  // equals embd when output.weight is absent (forward.rs:573)
  float* out_norm = nullptr;
  std::vector<void*> norm_allocs;
  uint64_t dev_bytes = 0, gguf_bytes = 0;
  bool dims_ok = false;
  bool gemm_ok = false;  // every layer matrix and the output fit the batched prefill GEMM
};

struct ifx_session {
  ifx_model* m = nullptr;
  uint64_t max_seq = 0, len = 0, steps = 0;
  int rope_mode = IFX_ROPE_REFERENCE;
  hipStream_t stream = nullptr;
  uint8_t *kc = nullptr, *vc = nullptr;  // [layer][kv head][max_seq][head_dim] of kv_es-byte elements
  uint32_t kv_es = 4;                    // 4: f32 (IFX_KV_F32), 2: binary16 (IFX_KV_F16)
  float *hidden = nullptr, *q = nullptr, *attn = nullptr, *mid = nullptr, *logits = nullptr;
  float* partial = nullptr;
  int qkv_ks = -1;  // K-split q/k/v in every layer: 1 / 0, -1 not yet decided (qkv_split)
  float* qkv_q = nullptr;  // K-split q/k/v: each layer's q ([n_layers][hidden])
  float2* rope_cs = nullptr;
  DevState* state = nullptr;
  uint32_t *out_tokens = nullptr, *feed_ids = nullptr;
  uint32_t attn_chunk = 64, max_chunks = 0;
  // captured steps: [sampling][merge bound / 8] (the greedy step, the step
  // with the sampler before finalize; each with the attention merge in its own
  // launch (bound 0) or in the O projection's prologue, which loads the first
  // `merge_bound` chunk records up front)
  static constexpr int kMergeGraphs = 7;
  hipGraphExec_t exec[2][kMergeGraphs] = {};
  bool graph_tried[2][kMergeGraphs] = {};
  bool sampling = false;                 // set for the duration of ifx_generate_sampled
  // fixed summation order (ifx_session_set_deterministic): q/k/v, O and down
  // through the tiled launches, the attention merge in its own launch
  bool deterministic = false;
  uint32_t merge_bound = 0;              // of the step being enqueued: 0, or a multiple of 8 up to 48
  float* probs = nullptr;                // sampler weights [vocab]
  void* sample_ws = nullptr;             // sampler histogram, sums and candidates (sample_ws_bytes)
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  float last_ms = 0.f;
  std::vector<void*> allocs;
  // batched prefill: chunks of at least batch_min rows (0: never) run layer by
  // layer through the GEMMs; the workspace grows to the largest chunk seen
  uint64_t batch_min = 64;
  struct {
    uint64_t cap = 0, logit_rows = 0;
    void* alloc = nullptr;
    void* logits = nullptr;
    float *x = nullptr, *q = nullptr, *att = nullptr, *mid = nullptr;
    float* part = nullptr;  // split-K partial tiles of the GEMMs
    // the GEMM activation operand (launch_prep_rows), sized for the widest input
    uint16_t *ahi = nullptr, *alo = nullptr, *gsum = nullptr;
    int* rexp = nullptr;
    void* kv_split = nullptr;  // the attention's fp16 K/V pairs (attn_prefill_ws_bytes)
  } ws;
};

namespace ifx {
// RoPE table in the reference arithmetic (src/ops.rs:278-280), glibc
// powf/sinf/cosf: inv = 1/powf(base, i/rope_dim); angle = pos*inv; row pos of
// out holds (cos, sin) of pair i at [pos * rope_dim/2 + i], for pos < n_pos.
void rope_table_host(float base, uint64_t rope_dim, uint64_t n_pos, std::vector<float2>& out) {
  const uint64_t half = rope_dim / 2;
  out.assign(n_pos * std::max<uint64_t>(half, 1), make_float2(1.f, 0.f));
  std::vector<float> inv(half);
  for (uint64_t i = 0; i < half; i++) inv[i] = 1.0f / powf(base, (float)(2 * i) / (float)rope_dim);
  for (uint64_t p = 0; p < n_pos; p++)
    for (uint64_t i = 0; i < half; i++) {
      const float ang = (float)p * inv[i];
      out[p * half + i] = make_float2(cosf(ang), sinf(ang));
    }
}
}  // namespace ifx

namespace {


int dev_alloc(std::vector<void*>& owner, void** p, size_t bytes) {
  if (bytes == 0) bytes = 4;
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) return set_error(IFX_E_OOM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
  owner.push_back(*p);
  return IFX_OK;
}

// A norm vector: raw tensor bytes dequantized on the device to f32
// (Weights::tensor_f32_by_index of the norm weight, src/model/forward.rs:359).
int upload_norm(ifx_model* m, int64_t idx, uint64_t n, float** out) {
  const uint8_t* data;
  uint64_t sz;
  IFX_TRY(gguf_tensor_bytes(m->gguf, m->map, idx, &data, &sz));
  const GgufTensor& t = m->gguf.tensors[idx];
  if (!dequant_supported(t.type))
    return set_error(IFX_E_UNKNOWN_TENSOR_TYPE, "%s: type %u", t.name.c_str(), t.type);
  if (t.n_elements() != n)
    return set_error(IFX_E_INVALID_ARG, "%s has %llu elements, expected %llu", t.name.c_str(),
                     (unsigned long long)t.n_elements(), (unsigned long long)n);
  void* raw = nullptr;
  IFX_HIP(hipMalloc(&raw, sz));
  void* f = nullptr;
  IFX_TRY(dev_alloc(m->norm_allocs, &f, n * 4));
  IFX_HIP(hipMemcpy(raw, data, sz, hipMemcpyHostToDevice));
  IFX_HIP(launch_dequant_raw(t.type, (const uint8_t*)raw, n, (float*)f, nullptr));
  IFX_HIP(hipDeviceSynchronize());
  IFX_HIP(hipFree(raw));
  m->dev_bytes += n * 4;
  m->gguf_bytes += sz;
  *out = (float*)f;
  return IFX_OK;
}

int upload_weight(ifx_model* m, int64_t idx, uint64_t rows, uint64_t cols, ifx_tensor** out) {
  const uint8_t* data;
  uint64_t sz;
  IFX_TRY(gguf_tensor_bytes(m->gguf, m->map, idx, &data, &sz));
  const GgufTensor& t = m->gguf.tensors[idx];
  uint64_t n_el;
  if (!mul_u64(rows, cols, &n_el) || t.n_elements() != n_el)
    return set_error(IFX_E_INVALID_ARG, "%s has %llu elements, expected %llu x %llu", t.name.c_str(),
                     (unsigned long long)t.n_elements(), (unsigned long long)rows,
                     (unsigned long long)cols);
  int rc = upload_matrix(t.type, data, sz, rows, cols, out, m->flags);
  if (rc != IFX_OK) return rc;
  uint64_t db = (*out)->L.body_bytes + (*out)->L.scal_bytes;
  m->dev_bytes += db;
  m->gguf_bytes += sz;
  return IFX_OK;
}

void model_free(ifx_model* m) {
  if (!m) return;
  for (LayerDev& L : m->layers)
    for (ifx_tensor* t : {L.q, L.k, L.v, L.o, L.gate, L.up, L.down}) ifx_tensor_free(t);
  if (m->output && m->output != m->embd) ifx_tensor_free(m->output);
  ifx_tensor_free(m->embd);
  for (void* p : m->norm_allocs) (void)hipFree(p);
  delete m;
}

int check_dims(const ifx_model* m) {
  const ifx_config& c = m->cfg;
  uint64_t qd;
  if (c.n_kv_heads == 0 || c.n_heads % c.n_kv_heads || !mul_u64(c.n_heads, c.head_dim, &qd) || qd != c.hidden_size ||
      c.rope_dim > c.head_dim || (c.rope_dim & 1) || (c.head_dim & 1))
    return set_error(IFX_E_INVALID_ARG, "inconsistent attention shape (heads %llu/%llu, head_dim %llu, rope_dim %llu)",
                     (unsigned long long)c.n_heads, (unsigned long long)c.n_kv_heads,
                     (unsigned long long)c.head_dim, (unsigned long long)c.rope_dim);
  return IFX_OK;
}

GemvSeg seg_of(const ifx_tensor* t) {
  return gemv_seg(t->L);
}

// The batched prefill GEMM takes the quantized matrices whose operands it can
// carry exactly (gemm_layout_ok) and a head dim the prefill attention kernel
// is built for.
bool gemm_tensor_ok(const ifx_tensor* t) { return t && gemm_type(t->L.type) && gemm_layout_ok(t->L); }
bool gemm_eligible(const ifx_model* m) {
  const ifx_config& c = m->cfg;
  uint64_t qd;
  if (!attn_prefill_head_dim((uint32_t)c.head_dim) || !mul_u64(c.n_heads, c.head_dim, &qd) || c.hidden_size != qd ||
      c.n_kv_heads == 0 || c.n_heads % c.n_kv_heads || c.rope_dim > c.head_dim || c.rope_dim % 2)
    return false;
  if (!gemm_tensor_ok(m->output)) return false;
  for (const LayerDev& L : m->layers)
    for (const ifx_tensor* t : {L.q, L.k, L.v, L.o, L.gate, L.up, L.down})
      if (!gemm_tensor_ok(t)) return false;
  return true;
}
GemmW gw(const ifx_tensor* t) {
  return gemm_w(t->L);
}

// Kernel classes of one step (ifx_session_profile): 0 embed, 1 qkv + rope +
// kv-append, 2 attention (partials + merge), 3 attn_output + residual,
// 4 ffn gate/up + swiglu, 5 ffn_down + residual, 6 output head + argmax,
// 7 finalize.  Classes 1..5 run once per layer, the others once per step.
constexpr int kClasses = 8;
bool per_layer_class(int k) { return k >= 1 && k <= 5; }

// q/k/v + RoPE + KV append of a layer (rms-normed hidden in)
GemvLaunch qkv_launch(const ifx_session* s, const LayerDev& L) {
  GemvLaunch g;
  g.seg[0] = seg_of(L.q);
  g.seg[1] = seg_of(L.k);
  g.seg[2] = seg_of(L.v);
  g.nseg = 3;
  g.cols = (uint32_t)s->m->cfg.hidden_size;
  g.x = s->hidden;
  g.norm_w = L.attn_norm;
  g.eps = s->m->cfg.norm_eps;
  return g;
}

// ffn_down + residual of a layer (mid in)
GemvLaunch down_launch(const ifx_session* s, const LayerDev& L) {
  GemvLaunch gd;
  gd.seg[0] = seg_of(L.down);
  gd.nseg = 1;
  gd.cols = (uint32_t)s->m->cfg.intermediate_size;
  gd.x = s->mid;
  return gd;
}

// attn_output + residual of a layer (attention output in)
GemvLaunch o_launch(const ifx_session* s, const LayerDev& L) {
  GemvLaunch go;
  go.seg[0] = seg_of(L.o);
  go.nseg = 1;
  go.cols = (uint32_t)s->m->cfg.hidden_size;
  go.x = s->attn;
  return go;
}

float* layer_cache(const ifx_session* s, uint8_t* base, size_t l) {
  const uint64_t kvd = s->m->cfg.n_kv_heads * s->m->cfg.head_dim;
  return (float*)(base + l * s->max_seq * kvd * s->kv_es);
}

// layer l's q under the K-split q/k/v launch
float* layer_q(const ifx_session* s, size_t l) { return s->qkv_q + l * s->m->cfg.hidden_size; }

// the K-split q/k/v launch's targets for layer l
QkvDst qkv_dst(const ifx_session* s, size_t l) {
  const ifx_config& c = s->m->cfg;
  return QkvDst{layer_q(s, l), layer_cache(s, s->kc, l), layer_cache(s, s->vc, l), s->rope_cs, s->state,
                (uint32_t)c.head_dim, (uint32_t)c.rope_dim, (uint32_t)s->max_seq};
}

// the rows every layer's K-split q/k/v launch adds into (its q, and cache row
// len of its K and V), cleared by the step's embedding gather
QkvClear qkv_clear_rows(const ifx_session* s) {
  const ifx_config& c = s->m->cfg;
  QkvClear r;
  r.q = s->qkv_q;
  r.k_cache = layer_cache(s, s->kc, 0);
  r.v_cache = layer_cache(s, s->vc, 0);
  r.state = s->state;
  r.nq = (uint32_t)(c.n_heads * c.head_dim);
  r.n_kv = (uint32_t)c.n_kv_heads;
  r.head_dim = (uint32_t)c.head_dim;
  r.max_seq = (uint32_t)s->max_seq;
  r.n_layers = (uint32_t)s->m->layers.size();
  r.q_stride = c.hidden_size;
  r.kv_stride = (uint64_t)s->max_seq * c.n_kv_heads * c.head_dim;
  return r;
}

// q/k/v as one K-split launch in every layer (kern_gemv_mfma.hip) where each
// layer's launch applies and the cache is f32 (the atomic adds accumulate in
// the cache's own type).  Each layer adds into its own q buffer and its cache
// rows, all cleared at once by the step's embedding gather: a clear in each
// layer's O or down launch cost it 0.3-0.6 us.  The tiled
// launch with the q/k/v epilogue otherwise.  IFX_QKV_KS=0 keeps the tiled
// launch.  Decided once per session.
bool qkv_split(ifx_session* s) {
  if (s->deterministic) return false;
  if (s->qkv_ks >= 0) return s->qkv_ks == 1;
  const char* f = getenv("IFX_QKV_KS");
  bool ok = !(f && f[0] == '0' && f[1] == 0) && s->kv_es == 4 && !s->m->layers.empty();
  for (size_t l = 0; ok && l < s->m->layers.size(); l++) {
    const LayerDev& L = s->m->layers[l];
    ok = qkv_ks_supported(qkv_launch(s, L), qkv_dst(s, l));
  }
  s->qkv_ks = ok ? 1 : 0;
  return ok;
}

// Launches the kernel(s) of class k (for layer l where it applies).  Every
// kernel reads positions from s->state.
int enqueue_class(ifx_session* s, int k, size_t l) {
  ifx_model* m = s->m;
  const ifx_config& c = m->cfg;
  hipStream_t st = s->stream;
  const uint32_t D = (uint32_t)c.hidden_size;
  const uint32_t kvd = (uint32_t)(c.n_kv_heads * c.head_dim);
  switch (k) {
    case 0:
      IFX_HIP(launch_embed_state(devw(m->embd), s->state, s->hidden, st,
                                 qkv_split(s) ? qkv_clear_rows(s) : QkvClear{}));
      return IFX_OK;
    case 6: {
      GemvLaunch gh;
      gh.seg[0] = seg_of(m->output);
      gh.nseg = 1;
      gh.cols = D;
      gh.x = s->hidden;
      gh.norm_w = m->out_norm;
      gh.eps = c.norm_eps;
      IFX_HIP(gemv_logits(gh, s->logits, s->state, st));
      return IFX_OK;
    }
    case 7:
      if (s->sampling)
        IFX_HIP(launch_sample(s->logits, s->probs, sample_ws(s->sample_ws), (uint32_t)c.vocab_size, s->state, st));
      IFX_HIP(launch_finalize(s->state, st));
      return IFX_OK;
    default:
      break;
  }
  const LayerDev& L = m->layers[l];
  void* kc = s->kc + l * s->max_seq * kvd * s->kv_es;
  void* vc = s->vc + l * s->max_seq * kvd * s->kv_es;
  const uint32_t kv16 = s->kv_es == 2;
  switch (k) {
    case 1: {
      const GemvLaunch g = qkv_launch(s, L);
      if (qkv_split(s)) {
        IFX_HIP(launch_qkv_ks(g, qkv_dst(s, l), st));
        return IFX_OK;
      }
      QkvEpi e{s->q, kc, vc, s->rope_cs, s->state, (uint32_t)c.head_dim, (uint32_t)c.rope_dim, kvd,
               (uint32_t)s->max_seq, kv16};
      IFX_HIP(gemv_qkv(g, e, st));
      return IFX_OK;
    }
    case 2:
    case 3: {
      // q as the layer's q/k/v launch left it
      AttnArgs a{qkv_split(s) ? layer_q(s, l) : s->q, kc, vc, s->attn, s->partial, s->state, (uint32_t)c.n_heads,
                 (uint32_t)c.n_kv_heads, (uint32_t)c.head_dim, s->max_chunks, s->attn_chunk,
                 (uint32_t)s->max_seq, kv16};
      const GemvLaunch go = o_launch(s, L);
      // the merge of the chunk records moves into the O launch's prologue
      const bool fused = s->merge_bound && merge_o_supported(go, a);
      if (k == 2) IFX_HIP(fused ? launch_attn_partials(a, st) : launch_attn_decode(a, st));
      else if (fused) IFX_HIP(launch_mfma_residual_merge(go, a, s->hidden, st, s->merge_bound));
      else IFX_HIP(s->deterministic ? gemv_residual_fixed(go, s->hidden, st) : gemv_residual(go, s->hidden, st));
      return IFX_OK;
    }
    case 4: {
      GemvLaunch gf;
      gf.seg[0] = seg_of(L.gate);
      gf.seg[1] = seg_of(L.up);
      gf.nseg = 2;
      gf.paired = true;
      gf.cols = D;
      gf.x = s->hidden;
      gf.norm_w = L.ffn_norm;
      gf.eps = c.norm_eps;
      IFX_HIP(gemv_swiglu(gf, s->mid, st));
      return IFX_OK;
    }
    case 5:
      IFX_HIP(s->deterministic ? gemv_residual_fixed(down_launch(s, L), s->hidden, st)
                               : gemv_residual(down_launch(s, L), s->hidden, st));
      return IFX_OK;
    default:
      return set_error(IFX_E_INVALID_ARG, "kernel class %d", k);
  }
}

// One token through the whole model: embed -> layers -> final norm + head ->
// greedy bookkeeping.
int enqueue_step(ifx_session* s) {
  IFX_TRY(enqueue_class(s, 0, 0));
  for (size_t l = 0; l < s->m->layers.size(); l++)
    for (int k = 1; k <= 5; k++) IFX_TRY(enqueue_class(s, k, l));
  IFX_TRY(enqueue_class(s, 6, 0));
  IFX_TRY(enqueue_class(s, 7, 0));
  return IFX_OK;
}

uint64_t tensor_stream_bytes(const ifx_tensor* t) { return t->L.body_bytes + t->L.scal_bytes; }

// The attention merge goes into the O launch's prologue while the attended
// rows make at most merge_o_first_chunks() chunk records (every workgroup
// reads them all; past that the separate merge launch is faster), with the
// step's chunk count rounded up to a multiple of merge_o_bound_step() as the
// records its prologue loads.  `rows` bounds the rows the step attends (the
// cache rows before it + 1).  IFX_MERGE_O=0 / 1 takes the separate / the
// fused merge at any length.
void choose_merge(ifx_session* s, uint64_t rows) {
  if (s->deterministic) {
    s->merge_bound = 0;
    return;
  }
  const uint64_t nch = (rows + s->attn_chunk - 1) / s->attn_chunk, step = merge_o_bound_step();
  const uint32_t most = merge_o_first_chunks();
  const uint32_t bound = (uint32_t)std::max<uint64_t>(step, (nch + step - 1) / step * step);
  const char* f = getenv("IFX_MERGE_O");
  if (f && (f[0] == '0' || f[0] == '1') && f[1] == 0) s->merge_bound = f[0] == '1' ? std::min(bound, most) : 0;
  else s->merge_bound = nch <= most ? bound : 0;
}

// Replay the captured step (capturing it on first use); direct launches if the
// runtime refuses capture.
int run_step(ifx_session* s, uint64_t rows) {
  choose_merge(s, rows);
  const int gi = (int)(s->merge_bound / merge_o_bound_step());
  if (gi >= ifx_session::kMergeGraphs) return set_error(IFX_E_INVALID_ARG, "merge bound %u", s->merge_bound);
  hipGraphExec_t& exec = s->exec[s->sampling][gi];
  bool& tried = s->graph_tried[s->sampling][gi];
  if (!tried) {
    tried = true;
    // IFX_NO_GRAPH=1: launch the step's kernels directly (used under profilers
    // that do not follow captured graphs)
    const char* ng = getenv("IFX_NO_GRAPH");
    if (ng && ng[0] == '1') {
      s->steps++;
      return enqueue_step(s);
    }
    hipGraph_t g = nullptr;
    if (hipStreamBeginCapture(s->stream, hipStreamCaptureModeRelaxed) == hipSuccess) {
      int rc = enqueue_step(s);
      hipError_t e = hipStreamEndCapture(s->stream, &g);
      if (rc == IFX_OK && e == hipSuccess && g) {
        if (hipGraphInstantiate(&exec, g, nullptr, nullptr, 0) != hipSuccess) exec = nullptr;
      }
      if (g) (void)hipGraphDestroy(g);
      (void)hipGetLastError();
    }
  }
  s->steps++;
  if (exec) {
    IFX_HIP(hipGraphLaunch(exec, s->stream));
    return IFX_OK;
  }
  return enqueue_step(s);
}

int state_op(ifx_session* s, uint32_t kind, uint32_t value, uint32_t len) {
  StateOp op{kind, value, len};
  IFX_HIP(launch_state(s->state, op, s->stream));
  return IFX_OK;
}

// Prefill workspace for chunks of up to n rows (grows, never shrinks), plus a
// fixed buffer for the split-K partial tiles of short chunks.
constexpr uint64_t kSplitPartBytes = 64ull << 20;
int ensure_ws(ifx_session* s, uint64_t n) {
  if (n <= s->ws.cap) return IFX_OK;
  const ifx_config& c = s->m->cfg;
  const uint64_t D = c.hidden_size, F = c.intermediate_size;
  auto al = [](uint64_t b) { return (b + 255) & ~255ull; };
  const uint64_t W = std::max(D, F);  // widest GEMM input
  const uint64_t bx = al(n * D * 4), bm = al(n * F * 4), bh = al(n * W * 2), bg = al(n * (W / 256 + 1) * 32),
                 br = al(n * 4), bp = kSplitPartBytes;
  const uint64_t ba = al(attn_prefill_ws_bytes((uint32_t)n, (uint32_t)c.n_kv_heads, (uint32_t)c.head_dim));
  if (s->ws.alloc) {
    IFX_HIP(hipStreamSynchronize(s->stream));
    IFX_HIP(hipFree(s->ws.alloc));
    s->ws.alloc = nullptr;
    s->ws.cap = 0;
  }
  void* p = nullptr;
  if (hipMalloc(&p, 3 * bx + bm + 2 * bh + bg + br + bp + ba) != hipSuccess)
    return set_error(IFX_E_OOM, "prefill workspace of %llu rows", (unsigned long long)n);
  uint8_t* b = (uint8_t*)p;
  s->ws.x = (float*)b;
  s->ws.q = (float*)(b + bx);
  s->ws.att = (float*)(b + 2 * bx);
  b += 3 * bx;
  s->ws.mid = (float*)b;
  s->ws.ahi = (uint16_t*)(b + bm);
  s->ws.alo = (uint16_t*)(b + bm + bh);
  s->ws.gsum = (uint16_t*)(b + bm + 2 * bh);
  s->ws.rexp = (int*)(b + bm + 2 * bh + bg);
  s->ws.part = (float*)(b + bm + 2 * bh + bg + br);
  s->ws.kv_split = b + bm + 2 * bh + bg + br + bp;
  s->ws.alloc = p;
  s->ws.cap = n;
  return IFX_OK;
}

// Model::prefill (src/model/forward.rs:496-538) as whole-chunk GEMMs, layer by
// layer (Layer::prefill, src/model/forward.rs:215-337): the n ids at
// s->feed_ids (device) write K/V rows start .. start + n - 1; query t attends
// to rows start .. start + t (causal) or to all n rows (Layer::forward's
// non-causal attention, src/model/forward.rs:62-207).  RoPE positions are
// chunk-relative (0 .. n - 1) or, in ABSOLUTE mode, start + t.  The last row
// then takes the decode head (final RMSNorm, logits, argmax) and the state
// records its greedy pick as a step does; logits_out (host, n x vocab) gets
// every row's logits when non-null.
int batched_prefill(ifx_session* s, uint64_t n, uint64_t start, bool causal, float* logits_out) {
  ifx_model* m = s->m;
  const ifx_config& c = m->cfg;
  IFX_TRY(ensure_ws(s, n));
  hipStream_t st = s->stream;
  const uint32_t N = (uint32_t)n, D = (uint32_t)c.hidden_size, F = (uint32_t)c.intermediate_size;
  const uint32_t hd = (uint32_t)c.head_dim, rd = (uint32_t)c.rope_dim;
  const uint32_t kvd = (uint32_t)(c.n_kv_heads * c.head_dim), row0 = (uint32_t)start;
  const uint32_t pos0 = s->rope_mode == IFX_ROPE_ABSOLUTE ? row0 : 0u;
  auto& w = s->ws;
  // the GEMM operand of rows of k columns (prep writes it, the GEMMs read it)
  auto op = [&](uint32_t rows, uint32_t k) { return GemmIn{w.ahi, w.alo, w.gsum, w.rexp, rows, k, w.part, kSplitPartBytes}; };
  IFX_HIP(launch_embed_rows(devw(m->embd), s->feed_ids, n, w.x, st));
  for (size_t l = 0; l < m->layers.size(); l++) {
    const LayerDev& L = m->layers[l];
    void* kc = s->kc + l * s->max_seq * kvd * s->kv_es;
    void* vc = s->vc + l * s->max_seq * kvd * s->kv_es;
    const bool kv16 = s->kv_es == 2;
    const GemmIn in = op(N, D);
    IFX_HIP(launch_prep_rows(w.x, N, D, D, L.attn_norm, c.norm_eps, in, st));
    const uint64_t kv_hs = s->max_seq * hd;  // head stride of the head-major cache
    IFX_HIP(gemm_rope(in, gw(L.q), w.q, D, hd, 0, pos0, hd, rd, s->rope_cs, st));
    IFX_HIP(gemm_rope(in, gw(L.k), kc, hd, kv_hs, row0, pos0, hd, rd, s->rope_cs, st, kv16));
    IFX_HIP(gemm_rows(in, gw(L.v), vc, hd, kv_hs, row0, hd, st, kv16));
    const AttnPrefillArgs aa{w.q, kc, vc, w.att, N, row0, (uint32_t)c.n_heads, (uint32_t)c.n_kv_heads, hd,
                             (uint32_t)s->max_seq, causal, w.kv_split, kv16};
    IFX_HIP(launch_attn_prefill(aa, st));
    IFX_HIP(launch_prep_rows(w.att, N, D, D, nullptr, 0.f, in, st));
    IFX_HIP(gemm_residual(in, gw(L.o), w.x, D, st));
    IFX_HIP(launch_prep_rows(w.x, N, D, D, L.ffn_norm, c.norm_eps, in, st));
    IFX_HIP(gemm_swiglu(in, gw(L.gate), gw(L.up), w.mid, F, st));
    const GemmIn inf = op(N, F);
    IFX_HIP(launch_prep_rows(w.mid, N, F, F, nullptr, 0.f, inf, st));
    IFX_HIP(gemm_residual(inf, gw(L.down), w.x, D, st));
  }
  // the last row's greedy pick, recorded as a step records it (k_finalize)
  IFX_TRY(state_op(s, STATE_BATCH, 0, N));
  GemvLaunch gh;
  gh.seg[0] = seg_of(m->output);
  gh.nseg = 1;
  gh.cols = D;
  gh.x = w.x + (n - 1) * D;
  gh.norm_w = m->out_norm;
  gh.eps = c.norm_eps;
  IFX_HIP(gemv_logits(gh, s->logits, s->state, st));
  if (s->sampling)
    IFX_HIP(launch_sample(s->logits, s->probs, sample_ws(s->sample_ws), (uint32_t)c.vocab_size, s->state, st));
  IFX_HIP(launch_finalize(s->state, st));
  if (logits_out) {
    const uint64_t V = c.vocab_size, rows = std::min<uint64_t>(n, 512);
    if (w.logit_rows < rows) {
      if (w.logits) {
        IFX_HIP(hipStreamSynchronize(st));
        IFX_HIP(hipFree(w.logits));
        w.logits = nullptr;
        w.logit_rows = 0;
      }
      if (hipMalloc(&w.logits, rows * V * 4) != hipSuccess)
        return set_error(IFX_E_OOM, "prefill logits buffer of %llu rows", (unsigned long long)rows);
      w.logit_rows = rows;
    }
    for (uint64_t r0 = 0; r0 < n; r0 += rows) {
      const uint32_t nr = (uint32_t)std::min<uint64_t>(rows, n - r0);
      const GemmIn in = op(nr, D);
      IFX_HIP(launch_prep_rows(w.x + r0 * D, nr, D, D, m->out_norm, c.norm_eps, in, st));
      IFX_HIP(gemm_store(in, gw(m->output), (float*)w.logits, (uint32_t)V, st));
      IFX_HIP(hipMemcpyAsync(logits_out + r0 * V, w.logits, (size_t)nr * V * 4, hipMemcpyDeviceToHost, st));
    }
  }
  return IFX_OK;
}

int check_vocab(const ifx_model* m) {
  const ifx_config& c = m->cfg;
  if (m->embd->L.rows < c.vocab_size || m->output->L.rows != c.vocab_size)
    return set_error(IFX_E_INVALID_ARG, "vocab_size %u does not match the embedding/output rows",
                     c.vocab_size);
  return IFX_OK;
}


void session_free(ifx_session* s) {
  if (!s) return;
  if (s->stream) (void)hipStreamSynchronize(s->stream);
  if (s->ws.alloc) (void)hipFree(s->ws.alloc);
  if (s->ws.logits) (void)hipFree(s->ws.logits);
  for (auto& row : s->exec)
    for (hipGraphExec_t e : row)
      if (e) (void)hipGraphExecDestroy(e);
  if (s->ev0) (void)hipEventDestroy(s->ev0);
  if (s->ev1) (void)hipEventDestroy(s->ev1);
  for (void* p : s->allocs) (void)hipFree(p);
  if (s->stream) (void)hipStreamDestroy(s->stream);
  delete s;
}

int model_open(const char* path, uint32_t flags, ifx_model** out);

}  // namespace

extern "C" {

int ifx_model_open(const char* path, ifx_model** out) { return ifx_model_open_ex(path, 0, out); }

int ifx_model_open_ex(const char* path, uint32_t flags, ifx_model** out) {
  clear_error();
  if (!out) return set_error(IFX_E_INVALID_ARG, "null output");
  *out = nullptr;
  if (flags & ~(uint32_t)IFX_OPEN_GGML_KQUANTS) return set_error(IFX_E_INVALID_ARG, "unknown flags %#x", flags);
  // host allocations sized from the file (metadata, staging of a matrix) may
  // fail; that is a status here, never an exception across the C ABI
  try {
    return model_open(path, flags, out);
  } catch (const std::bad_alloc&) {
    return set_error(IFX_E_OOM, "out of host memory opening %s", path ? path : "(null)");
  }
}

}  // extern "C"

namespace {

int model_open(const char* path, uint32_t flags, ifx_model** out) {
  ifx_model* m = new ifx_model();
  m->flags = flags;
  int rc = m->map.open(path);
  if (rc == IFX_OK) rc = gguf_parse(m->map.data, m->map.size, &m->gguf);
  // Config::from_gguf and the name resolution (host_config.cpp): parse errors
  // are reported without touching a device
  ModelPlan plan;
  if (rc == IFX_OK) rc = plan_model(m->gguf, &plan);
  if (rc != IFX_OK) { model_free(m); return rc; }
  const GgufFile& f = m->gguf;
  ifx_config& c = m->cfg;
  c = plan.cfg;

  // upload once
  rc = device_init();
  if (rc != IFX_OK) { model_free(m); return rc; }
  uint64_t shapes[R_COUNT][2];
  rc = plan_shapes(f, &plan, shapes);
  if (rc != IFX_OK) { model_free(m); return rc; }
  const uint64_t D = c.hidden_size;
  m->dims_ok = check_dims(m) == IFX_OK;
  clear_error();
  const int64_t i_onorm = plan.out_norm;
  rc = upload_weight(m, plan.embd.idx, plan.embd.rows, D, &m->embd);
  if (rc == IFX_OK && plan.output.idx >= 0) rc = upload_weight(m, plan.output.idx, plan.output.rows, D, &m->output);
  else if (rc == IFX_OK) m->output = m->embd;
  if (rc == IFX_OK) rc = upload_norm(m, i_onorm, D, &m->out_norm);
  m->layers.resize(c.n_layers);
  for (uint64_t l = 0; l < c.n_layers && rc == IFX_OK; l++) {
    LayerDev& L = m->layers[l];
    const int64_t* x = &plan.layers[l * R_COUNT];
    auto mat = [&](int r, ifx_tensor** t) { return upload_weight(m, x[r], shapes[r][0], shapes[r][1], t); };
    if (rc == IFX_OK) rc = upload_norm(m, x[R_ATTN_NORM], D, &L.attn_norm);
    if (rc == IFX_OK) rc = mat(R_Q, &L.q);
    if (rc == IFX_OK) rc = mat(R_K, &L.k);
    if (rc == IFX_OK) rc = mat(R_V, &L.v);
    if (rc == IFX_OK) rc = mat(R_O, &L.o);
    if (rc == IFX_OK) rc = upload_norm(m, x[R_FFN_NORM], D, &L.ffn_norm);
    if (rc == IFX_OK) rc = mat(R_GATE, &L.gate);
    if (rc == IFX_OK) rc = mat(R_UP, &L.up);
    if (rc == IFX_OK) rc = mat(R_DOWN, &L.down);
    if (rc == IFX_OK && (L.q->L.type != L.k->L.type || L.gate->L.type != L.up->L.type))
      rc = set_error(IFX_E_INVALID_ARG, "layer %llu: attn_q/attn_k or ffn_gate/ffn_up types differ",
                     (unsigned long long)l);
  }
  if (rc != IFX_OK) { model_free(m); return rc; }
  m->gemm_ok = gemm_eligible(m);
  *out = m;
  return IFX_OK;
}

}  // namespace

extern "C" {

void ifx_model_close(ifx_model* m) { model_free(m); }

int ifx_model_config(const ifx_model* m, ifx_config* out) {
  if (!m || !out) return set_error(IFX_E_INVALID_ARG, "null argument");
  *out = m->cfg;
  return IFX_OK;
}

int ifx_model_weight_bytes(const ifx_model* m, uint64_t* dev, uint64_t* gguf) {
  if (!m) return set_error(IFX_E_INVALID_ARG, "null model");
  if (dev) *dev = m->dev_bytes;
  if (gguf) *gguf = m->gguf_bytes;
  return IFX_OK;
}

int ifx_session_create(ifx_model* m, uint64_t max_seq_len, ifx_session** out) {
  return ifx_session_create_kv(m, max_seq_len, IFX_KV_F32, out);
}

int ifx_session_create_kv(ifx_model* m, uint64_t max_seq_len, int kv_type, ifx_session** out) {
  clear_error();
  if (!m || !out || max_seq_len == 0 || max_seq_len > 0x7fffffffull || (kv_type != IFX_KV_F32 && kv_type != IFX_KV_F16))
    return set_error(IFX_E_INVALID_ARG, "bad session arguments");
  *out = nullptr;
  IFX_TRY(check_dims(m));
  const ifx_config& c = m->cfg;
  if (!attn_decode_head_dim((uint32_t)c.head_dim, kv_type == IFX_KV_F16))
    return set_error(IFX_E_INVALID_ARG, "head_dim %llu has no %s-cache attention", (unsigned long long)c.head_dim,
                     kv_type == IFX_KV_F16 ? "f16" : "f32");
  ifx_session* s = new ifx_session();
  s->m = m;
  s->max_seq = max_seq_len;
  s->kv_es = kv_type == IFX_KV_F16 ? 2 : 4;
  const uint64_t D = c.hidden_size, F = c.intermediate_size, kvd = c.n_kv_heads * c.head_dim;
  const uint64_t G = c.n_heads / c.n_kv_heads;
  s->max_chunks = (uint32_t)((max_seq_len + s->attn_chunk - 1) / s->attn_chunk);
  // bytes of the K (and of the V) cache, refused when they do not fit in 64 bits
  uint64_t kv_bytes = 0;
  if (!mul_u64(c.n_layers, max_seq_len, &kv_bytes) || !mul_u64(kv_bytes, kvd, &kv_bytes) ||
      !mul_u64(kv_bytes, s->kv_es, &kv_bytes)) {
    delete s;
    return set_error(IFX_E_OOM, "a KV cache of %llu rows does not fit in memory", (unsigned long long)max_seq_len);
  }
  int rc = IFX_OK;
  auto A = [&](void** p, size_t b) { if (rc == IFX_OK) rc = dev_alloc(s->allocs, p, b); };
  A((void**)&s->kc, kv_bytes);
  A((void**)&s->vc, kv_bytes);
  A((void**)&s->hidden, D * 4);
  A((void**)&s->q, D * 4);
  A((void**)&s->attn, D * 4);
  A((void**)&s->mid, F * 4);
  A((void**)&s->logits, (uint64_t)std::max<uint32_t>(c.vocab_size, 1) * 4);
  A((void**)&s->probs, (uint64_t)std::max<uint32_t>(c.vocab_size, 1) * 4);
  A(&s->sample_ws, sample_ws_bytes());
  A((void**)&s->partial, (uint64_t)c.n_kv_heads * s->max_chunks * attn_partial_floats(G, c.head_dim) * 4);
  A((void**)&s->qkv_q, (uint64_t)std::max<size_t>(m->layers.size(), 1) * D * 4);
  A((void**)&s->rope_cs, max_seq_len * std::max<uint64_t>(c.rope_dim / 2, 1) * 8);
  A((void**)&s->state, sizeof(DevState));
  A((void**)&s->out_tokens, max_seq_len * 4);
  A((void**)&s->feed_ids, max_seq_len * 4);
  if (rc != IFX_OK) { session_free(s); return rc; }
  if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreate(&s->ev0) != hipSuccess || hipEventCreate(&s->ev1) != hipSuccess) {
    session_free(s);
    return set_error(IFX_E_HIP, "stream/event creation failed");
  }
  std::vector<float2> cs;
  rope_table_host(c.rope_base, c.rope_dim, max_seq_len, cs);
  DevState init{};
  init.rope_mode = IFX_ROPE_REFERENCE;
  init.feed_ids = s->feed_ids;
  init.out_tokens = s->out_tokens;
  init.out_cap = (uint32_t)max_seq_len;
  init.top_p = 1.0f;
  if (hipMemcpy(s->rope_cs, cs.data(), cs.size() * 8, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(s->state, &init, sizeof init, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemset(s->kc, 0, kv_bytes) != hipSuccess || hipMemset(s->vc, 0, kv_bytes) != hipSuccess ||
      hipMemset(s->sample_ws, 0, sample_ws_bytes()) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
    session_free(s);
    return set_error(IFX_E_HIP, "session initialisation failed");
  }
  *out = s;
  return IFX_OK;
}

void ifx_session_destroy(ifx_session* s) { session_free(s); }

int ifx_session_clear(ifx_session* s) {
  if (!s) return set_error(IFX_E_INVALID_ARG, "null session");
  IFX_TRY(state_op(s, STATE_RESET, 0, 0));
  IFX_HIP(hipStreamSynchronize(s->stream));
  s->len = 0;
  s->steps = 0;
  return IFX_OK;
}

int ifx_session_len(const ifx_session* s, uint64_t* len) {
  if (!s || !len) return set_error(IFX_E_INVALID_ARG, "null argument");
  *len = s->len;
  return IFX_OK;
}

int ifx_session_set_prefill_batch(ifx_session* s, uint64_t min_rows) {
  if (!s) return set_error(IFX_E_INVALID_ARG, "null session");
  s->batch_min = min_rows;
  return IFX_OK;
}

int ifx_model_batched_prefill(const ifx_model* m, int* eligible) {
  if (!m || !eligible) return set_error(IFX_E_INVALID_ARG, "null argument");
  *eligible = m->gemm_ok ? 1 : 0;
  return IFX_OK;
}

int ifx_session_set_deterministic(ifx_session* s, int on) {
  if (!s || (on != 0 && on != 1)) return set_error(IFX_E_INVALID_ARG, "bad argument");
  if (s->deterministic == (on == 1)) return IFX_OK;
  // the captured steps hold the other launches: capture again on next use
  IFX_HIP(hipStreamSynchronize(s->stream));
  for (int i = 0; i < 2; i++)
    for (int j = 0; j < ifx_session::kMergeGraphs; j++) {
      if (s->exec[i][j]) IFX_HIP(hipGraphExecDestroy(s->exec[i][j]));
      s->exec[i][j] = nullptr;
      s->graph_tried[i][j] = false;
    }
  s->deterministic = on == 1;
  s->qkv_ks = -1;
  return IFX_OK;
}

int ifx_session_set_rope_mode(ifx_session* s, int mode) {
  if (!s || (mode != IFX_ROPE_REFERENCE && mode != IFX_ROPE_ABSOLUTE))
    return set_error(IFX_E_INVALID_ARG, "bad rope mode");
  s->rope_mode = mode;
  IFX_TRY(state_op(s, STATE_MODE, (uint32_t)mode, 0));
  IFX_HIP(hipStreamSynchronize(s->stream));
  return IFX_OK;
}

int ifx_decode_step(ifx_session* s, uint32_t token, float* logits_out) {
  clear_error();
  if (!s) return set_error(IFX_E_INVALID_ARG, "null session");
  ifx_model* m = s->m;
  if (token >= m->cfg.vocab_size)
    return set_error(IFX_E_INVALID_TENSOR_INDEX, "tensor index out of bounds: %u", token);
  IFX_TRY(check_vocab(m));
  if (s->len >= s->max_seq) return set_error(IFX_E_KV_FULL, "KV cache full (%llu rows)", (unsigned long long)s->max_seq);
  IFX_TRY(state_op(s, STATE_DECODE, token, 0));
  IFX_TRY(run_step(s, s->len + 1));
  if (logits_out)
    IFX_HIP(hipMemcpyAsync(logits_out, s->logits, (size_t)m->cfg.vocab_size * 4, hipMemcpyDeviceToHost, s->stream));
  IFX_HIP(hipStreamSynchronize(s->stream));
  s->len += 1;
  return IFX_OK;
}

int ifx_prefill(ifx_session* s, const uint32_t* ids, uint64_t n, float* logits_out) {
  clear_error();
  if (!s || (n && !ids)) return set_error(IFX_E_INVALID_ARG, "null argument");
  ifx_model* m = s->m;
  for (uint64_t i = 0; i < n; i++)
    if (ids[i] >= m->cfg.vocab_size) return set_error(IFX_E_INVALID_TENSOR_INDEX, "tensor index out of bounds: 0");
  if (n == 0) return IFX_OK;
  IFX_TRY(check_vocab(m));
  if (s->len + n > s->max_seq) return set_error(IFX_E_KV_FULL, "prefill of %llu rows overflows the KV cache", (unsigned long long)n);
  IFX_HIP(hipMemcpyAsync(s->feed_ids, ids, n * 4, hipMemcpyHostToDevice, s->stream));
  if (s->batch_min && n >= s->batch_min && m->gemm_ok) {
    IFX_HIP(hipEventRecord(s->ev0, s->stream));
    IFX_TRY(batched_prefill(s, n, s->len, true, logits_out));
    IFX_HIP(hipEventRecord(s->ev1, s->stream));
    IFX_HIP(hipStreamSynchronize(s->stream));
    (void)hipEventElapsedTime(&s->last_ms, s->ev0, s->ev1);
    s->len += n;
    s->steps += n;
    return IFX_OK;
  }
  IFX_TRY(state_op(s, STATE_PREFILL, 0, (uint32_t)n));
  IFX_HIP(hipEventRecord(s->ev0, s->stream));
  const size_t V = m->cfg.vocab_size;
  for (uint64_t t = 0; t < n; t++) {
    IFX_TRY(run_step(s, s->len + t + 1));
    if (logits_out)
      IFX_HIP(hipMemcpyAsync(logits_out + t * V, s->logits, V * 4, hipMemcpyDeviceToHost, s->stream));
  }
  IFX_HIP(hipEventRecord(s->ev1, s->stream));
  IFX_HIP(hipStreamSynchronize(s->stream));
  (void)hipEventElapsedTime(&s->last_ms, s->ev0, s->ev1);
  s->len += n;
  return IFX_OK;
}

int ifx_decode_greedy(ifx_session* s, uint32_t token, uint64_t n_steps, uint32_t* out_tokens) {
  clear_error();
  if (!s || (n_steps && !out_tokens)) return set_error(IFX_E_INVALID_ARG, "null argument");
  ifx_model* m = s->m;
  if (token >= m->cfg.vocab_size)
    return set_error(IFX_E_INVALID_TENSOR_INDEX, "tensor index out of bounds: %u", token);
  IFX_TRY(check_vocab(m));
  if (s->len + n_steps > s->max_seq) return set_error(IFX_E_KV_FULL, "%llu steps overflow the KV cache", (unsigned long long)n_steps);
  const uint64_t first = s->steps;
  IFX_TRY(state_op(s, STATE_DECODE, token, 0));
  IFX_HIP(hipEventRecord(s->ev0, s->stream));
  for (uint64_t i = 0; i < n_steps; i++) IFX_TRY(run_step(s, s->len + i + 1));
  IFX_HIP(hipEventRecord(s->ev1, s->stream));
  IFX_HIP(hipStreamSynchronize(s->stream));
  (void)hipEventElapsedTime(&s->last_ms, s->ev0, s->ev1);
  s->len += n_steps;
  if (n_steps == 0) return IFX_OK;
  IFX_HIP(hipMemcpy(out_tokens, s->out_tokens + first, n_steps * 4, hipMemcpyDeviceToHost));
  int rc = IFX_OK;
  for (uint64_t i = 0; i < n_steps; i++) {
    if (out_tokens[i] & 0x80000000u) rc = IFX_E_NAN_LOGIT;
    out_tokens[i] &= 0x7fffffffu;
  }
  return rc == IFX_OK ? IFX_OK : set_error(rc, "NaN logit met by argmax");
}

int ifx_generate(ifx_session* s, const uint32_t* prompt, uint64_t n, uint64_t max_tokens,
                 uint32_t* out_tokens) {
  clear_error();
  if (!s || !prompt || (max_tokens && !out_tokens)) return set_error(IFX_E_INVALID_ARG, "null argument");
  if (n == 0) return set_error(IFX_E_INVALID_ARG, "empty prompt");
  IFX_TRY(ifx_session_clear(s));
  if (n + max_tokens > s->max_seq) {
    // validate ids first so the reference's error order (InvalidTensorIndex) is kept
    for (uint64_t i = 0; i < n; i++)
      if (prompt[i] >= s->m->cfg.vocab_size) return set_error(IFX_E_INVALID_TENSOR_INDEX, "tensor index out of bounds: 0");
    return set_error(IFX_E_KV_FULL, "prompt + max_tokens exceeds the KV cache");
  }
  IFX_TRY(ifx_prefill(s, prompt, n, nullptr));
  // the greedy loop continues on the device: the last prefill step left its
  // argmax as the next input token (src/model/forward.rs:605-609)
  IFX_HIP(hipEventRecord(s->ev0, s->stream));
  for (uint64_t i = 0; i < max_tokens; i++) IFX_TRY(run_step(s, s->len + i + 1));
  IFX_HIP(hipEventRecord(s->ev1, s->stream));
  IFX_HIP(hipStreamSynchronize(s->stream));
  (void)hipEventElapsedTime(&s->last_ms, s->ev0, s->ev1);
  s->len += max_tokens;
  if (max_tokens == 0) return IFX_OK;
  IFX_HIP(hipMemcpy(out_tokens, s->out_tokens + (n - 1), max_tokens * 4, hipMemcpyDeviceToHost));
  int rc = IFX_OK;
  for (uint64_t i = 0; i < max_tokens; i++) {
    if (out_tokens[i] & 0x80000000u) rc = IFX_E_NAN_LOGIT;
    out_tokens[i] &= 0x7fffffffu;
  }
  return rc == IFX_OK ? IFX_OK : set_error(rc, "NaN logit met by argmax");
}

int ifx_session_set_sampler(ifx_session* s, float temperature, uint32_t top_k, float top_p, uint64_t seed) {
  clear_error();
  if (!s) return set_error(IFX_E_INVALID_ARG, "null session");
  if (!(temperature >= 0.f) || !isfinite(temperature) || !(top_p >= 0.f && top_p <= 1.f))
    return set_error(IFX_E_INVALID_ARG, "sampler needs temperature >= 0 and 0 <= top_p <= 1");
  StateOp op{STATE_SAMPLER, top_k, 0};
  op.f0 = temperature;
  op.f1 = top_p;
  op.seed = seed;
  IFX_HIP(launch_state(s->state, op, s->stream));
  IFX_HIP(hipStreamSynchronize(s->stream));
  return IFX_OK;
}

int ifx_generate_sampled(ifx_session* s, const uint32_t* prompt, uint64_t n, uint64_t max_tokens,
                         uint32_t* out_tokens) {
  if (!s) return set_error(IFX_E_INVALID_ARG, "null session");
  // the prompt's last step and every generated step draw with the session's sampler
  struct Guard {
    ifx_session* s;
    ~Guard() { s->sampling = false; }
  } guard{s};
  s->sampling = true;
  return ifx_generate(s, prompt, n, max_tokens, out_tokens);
}

int ifx_sample_logits(const float* logits, uint32_t vocab, float temperature, uint32_t top_k, float top_p,
                      uint64_t seed, uint32_t n_draws, uint32_t* out) {
  clear_error();
  if (!logits || (n_draws && !out) || vocab == 0 || vocab >= (1u << 24))
    return set_error(IFX_E_INVALID_ARG, "sample: bad arguments");
  IFX_TRY(device_init());
  if (!(temperature > 0.f) || !isfinite(temperature) || !(top_p >= 0.f && top_p <= 1.f))
    return set_error(IFX_E_INVALID_ARG, "sample needs temperature > 0 and 0 <= top_p <= 1");
  hipStream_t st = nullptr;
  float *dl = nullptr, *dp = nullptr;
  void* dw = nullptr;
  DevState* ds = nullptr;
  uint32_t* dt = nullptr;
  hipError_t e = hipMalloc(&dl, (size_t)vocab * 4);
  if (e == hipSuccess) e = hipMalloc(&dp, (size_t)vocab * 4);
  if (e == hipSuccess) e = hipMalloc(&dw, sample_ws_bytes());
  if (e == hipSuccess) e = hipMalloc(&ds, sizeof(DevState));
  if (e == hipSuccess) e = hipMalloc(&dt, (size_t)std::max<uint32_t>(n_draws, 1) * 4);
  if (e == hipSuccess) e = hipMemcpy(dl, logits, (size_t)vocab * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemset(dw, 0, sample_ws_bytes());
  DevState init{};
  init.out_tokens = dt;
  init.out_cap = n_draws;
  init.temperature = temperature;
  init.top_k = top_k;
  init.top_p = top_p;
  init.seed = seed;
  if (e == hipSuccess) e = hipMemcpy(ds, &init, sizeof init, hipMemcpyHostToDevice);
  // draw i uses step i, as generate step i would; the maximum first, as the
  // head leaves it; finalize stores the draw and advances
  const SampleWs ws = sample_ws(dw);
  for (uint32_t i = 0; i < n_draws && e == hipSuccess; i++) {
    e = launch_logits_max(dl, vocab, ds, st);
    if (e == hipSuccess) e = launch_sample(dl, dp, ws, vocab, ds, st);
    if (e == hipSuccess) e = launch_finalize(ds, st);
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess && n_draws) e = hipMemcpy(out, dt, (size_t)n_draws * 4, hipMemcpyDeviceToHost);
  for (void* p : {(void*)dl, (void*)dp, dw, (void*)ds, (void*)dt}) if (p) (void)hipFree(p);
  if (e != hipSuccess) return set_error(IFX_E_HIP, "sample: %s", hipGetErrorString(e));
  for (uint32_t i = 0; i < n_draws; i++)
    if (out[i] & 0x80000000u) return set_error(IFX_E_NAN_LOGIT, "sample: NaN among the logits");
  return IFX_OK;
}

// IEEE binary16 <-> binary32 for the f16 KV cache's import and export:
// round to nearest, ties to even; overflow to infinity; NaN stays NaN.
static uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // >= 65520 rounds past 65504
  if (ax < 0x38800000u) {                                     // below 2^-14: subnormal or zero
    if (ax <= 0x33000000u) return (uint16_t)sign;             // <= 2^-25 (the tie goes to 0)
    const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, r = 126 - e;  // units of 2^-24
    uint32_t q = m >> r;
    const uint32_t rem = m & ((1u << r) - 1), half = 1u << (r - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t h = (ax - 0x38000000u) >> 13;  // exponent rebiased 127 -> 15, 10 mantissa bits
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}
static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu;
  float f;
  if (e == 0) {
    f = ldexpf((float)m, -24);
    uint32_t x;
    memcpy(&x, &f, 4);
    x |= sign;
    memcpy(&f, &x, 4);
    return f;
  }
  const uint32_t x = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
  memcpy(&f, &x, 4);
  return f;
}

int ifx_kv_import(ifx_session* s, const float* k, const float* v, uint64_t len) {
  if (!s || (len && (!k || !v))) return set_error(IFX_E_INVALID_ARG, "null argument");
  if (len > s->max_seq) return set_error(IFX_E_KV_FULL, "import of %llu rows", (unsigned long long)len);
  const ifx_config& c = s->m->cfg;
  const uint64_t kvd = c.n_kv_heads * c.head_dim, hd = c.head_dim, es = s->kv_es;
  // reference rows [t][kv_dim] -> the head-major device cache, one strided copy per (layer, head)
  // (an f16 cache: one rounded head block at a time)
  std::vector<uint16_t> blk(s->kv_es == 2 ? len * hd : 0);
  if (es == 2) IFX_HIP(hipStreamSynchronize(s->stream));  // the blocking copies below bypass the stream
  for (uint64_t l = 0; l < c.n_layers && len; l++)
    for (uint64_t h = 0; h < c.n_kv_heads; h++) {
      const uint64_t dev = (l * c.n_kv_heads + h) * s->max_seq * hd * es, host = l * len * kvd + h * hd;
      if (es == 4) {
        IFX_HIP(hipMemcpy2DAsync(s->kc + dev, hd * 4, k + host, kvd * 4, hd * 4, len, hipMemcpyHostToDevice, s->stream));
        IFX_HIP(hipMemcpy2DAsync(s->vc + dev, hd * 4, v + host, kvd * 4, hd * 4, len, hipMemcpyHostToDevice, s->stream));
        continue;
      }
      for (int which = 0; which < 2; which++) {
        const float* src = (which ? v : k) + host;
        for (uint64_t t = 0; t < len; t++)
          for (uint64_t d = 0; d < hd; d++) blk[t * hd + d] = f32_to_f16(src[t * kvd + d]);
        IFX_HIP(hipMemcpy((which ? s->vc : s->kc) + dev, blk.data(), len * hd * 2, hipMemcpyHostToDevice));
      }
    }
  IFX_TRY(state_op(s, STATE_RESET, 0, (uint32_t)len));
  IFX_HIP(hipStreamSynchronize(s->stream));
  s->len = len;
  s->steps = 0;
  return IFX_OK;
}

int ifx_kv_export(ifx_session* s, float* k, float* v, uint64_t len) {
  if (!s || (len && (!k || !v))) return set_error(IFX_E_INVALID_ARG, "null argument");
  if (len > s->len) return set_error(IFX_E_INVALID_ARG, "export of %llu rows, %llu cached", (unsigned long long)len, (unsigned long long)s->len);
  const ifx_config& c = s->m->cfg;
  const uint64_t kvd = c.n_kv_heads * c.head_dim;
  const uint64_t hd = c.head_dim, es = s->kv_es;
  IFX_HIP(hipStreamSynchronize(s->stream));
  std::vector<uint16_t> blk(s->kv_es == 2 ? len * hd : 0);
  for (uint64_t l = 0; l < c.n_layers && len; l++)
    for (uint64_t h = 0; h < c.n_kv_heads; h++) {
      const uint64_t dev = (l * c.n_kv_heads + h) * s->max_seq * hd * es, host = l * len * kvd + h * hd;
      if (es == 4) {
        IFX_HIP(hipMemcpy2D(k + host, kvd * 4, s->kc + dev, hd * 4, hd * 4, len, hipMemcpyDeviceToHost));
        IFX_HIP(hipMemcpy2D(v + host, kvd * 4, s->vc + dev, hd * 4, hd * 4, len, hipMemcpyDeviceToHost));
        continue;
      }
      for (int which = 0; which < 2; which++) {
        IFX_HIP(hipMemcpy(blk.data(), (which ? s->vc : s->kc) + dev, len * hd * 2, hipMemcpyDeviceToHost));
        float* dst = (which ? v : k) + host;
        for (uint64_t t = 0; t < len; t++)
          for (uint64_t d = 0; d < hd; d++) dst[t * kvd + d] = f16_to_f32(blk[t * hd + d]);
      }
    }
  return IFX_OK;
}

// Measurement hook.  n_steps greedy decode steps run first (direct launches),
// so the state is a real decode state; then every kernel class is launched
// back to back, once per layer (or once), n_steps times over, between one HIP
// event pair on the session stream: avg_ms = mean time per launch (what a
// kernel trace reports as its duration, plus the gap between launches),
// launches = launches per step, bytes = stored weight bytes streamed per
// launch (attention: the f32 K and V rows it attends; 0 where no weights).
// The repeated launches leave scratch and the next token's KV slot written;
// the next decode step recomputes both.  Finalize (class 7) advances the
// device state and is not repeated: its avg_ms is 0.
int ifx_session_profile(ifx_session* s, uint32_t token, uint64_t n_steps, float* avg_ms,
                        uint64_t* launches, uint64_t* bytes) {
  clear_error();
  if (!s || !avg_ms || !launches || !bytes || n_steps == 0) return set_error(IFX_E_INVALID_ARG, "bad arguments");
  ifx_model* m = s->m;
  if (token >= m->cfg.vocab_size) return set_error(IFX_E_INVALID_TENSOR_INDEX, "token");
  IFX_TRY(check_vocab(m));
  // one spare row: the repeated qkv launches write the next token's slot
  if (s->len + n_steps + 1 > s->max_seq) return set_error(IFX_E_KV_FULL, "profile steps overflow the KV cache");
  const uint64_t len0 = s->len;
  IFX_TRY(state_op(s, STATE_DECODE, token, 0));
  choose_merge(s, len0 + n_steps);  // the repeated launches below attend the last step's rows
  for (uint64_t i = 0; i < n_steps; i++) {
    IFX_TRY(enqueue_step(s));
    s->steps++;
  }
  IFX_HIP(hipStreamSynchronize(s->stream));
  s->len += n_steps;
  const size_t NL = m->layers.size();
  for (int k = 0; k < kClasses; k++) {
    const uint64_t per_step = per_layer_class(k) ? NL : 1;
    launches[k] = per_step;
    avg_ms[k] = 0.f;
    // finalize advances the device state: not repeated (no weights, launch-bound)
    if (per_step == 0 || k == 7) continue;
    IFX_HIP(hipEventRecord(s->ev0, s->stream));
    for (uint64_t i = 0; i < n_steps; i++)
      for (size_t l = 0; l < per_step; l++) IFX_TRY(enqueue_class(s, k, l));
    IFX_HIP(hipEventRecord(s->ev1, s->stream));
    IFX_HIP(hipEventSynchronize(s->ev1));
    float ms = 0.f;
    IFX_HIP(hipEventElapsedTime(&ms, s->ev0, s->ev1));
    avg_ms[k] = ms / (float)(n_steps * per_step);
  }
  const LayerDev& L0 = m->layers.empty() ? LayerDev{} : m->layers[0];
  bytes[0] = 0;
  bytes[1] = m->layers.empty() ? 0 : tensor_stream_bytes(L0.q) + tensor_stream_bytes(L0.k) + tensor_stream_bytes(L0.v);
  // attention streams the K and V rows it attends (the state after the steps)
  const uint64_t kvd = m->cfg.n_kv_heads * m->cfg.head_dim;
  bytes[2] = 2 * (len0 + n_steps) * kvd * s->kv_es;
  bytes[3] = m->layers.empty() ? 0 : tensor_stream_bytes(L0.o);
  bytes[4] = m->layers.empty() ? 0 : tensor_stream_bytes(L0.gate) + tensor_stream_bytes(L0.up);
  bytes[5] = m->layers.empty() ? 0 : tensor_stream_bytes(L0.down);
  bytes[6] = tensor_stream_bytes(m->output);
  bytes[7] = 0;
  return IFX_OK;
}

int ifx_session_profile_ordered(ifx_session* s, uint32_t token, uint64_t n_steps, float* avg_ms) {
  clear_error();
  if (!s || !avg_ms || n_steps == 0) return set_error(IFX_E_INVALID_ARG, "bad arguments");
  ifx_model* m = s->m;
  if (token >= m->cfg.vocab_size) return set_error(IFX_E_INVALID_TENSOR_INDEX, "token");
  IFX_TRY(check_vocab(m));
  if (s->len + n_steps > s->max_seq) return set_error(IFX_E_KV_FULL, "profile steps overflow the KV cache");
  const size_t NL = m->layers.size();
  // the launches of one step, in step order: class 0, classes 1..5 per layer, 6, 7
  std::vector<std::pair<int, size_t>> seq;
  seq.emplace_back(0, 0);
  for (size_t l = 0; l < NL; l++)
    for (int k = 1; k <= 5; k++) seq.emplace_back(k, l);
  seq.emplace_back(6, 0);
  seq.emplace_back(7, 0);
  std::vector<hipEvent_t> ev(2 * seq.size(), nullptr);
  int rc = IFX_OK;
  for (hipEvent_t& e : ev)
    if (rc == IFX_OK && hipEventCreate(&e) != hipSuccess) rc = set_error(IFX_E_HIP, "hipEventCreate failed");
  double sum[kClasses] = {};
  uint64_t cnt[kClasses] = {};
  if (rc == IFX_OK) rc = state_op(s, STATE_DECODE, token, 0);
  for (uint64_t i = 0; i < n_steps && rc == IFX_OK; i++) {
    choose_merge(s, s->len + i + 1);  // the bound the step graph would take for this token
    for (size_t j = 0; j < seq.size() && rc == IFX_OK; j++) {
      if (hipEventRecord(ev[2 * j], s->stream) != hipSuccess) rc = set_error(IFX_E_HIP, "hipEventRecord failed");
      if (rc == IFX_OK) rc = enqueue_class(s, seq[j].first, seq[j].second);
      if (rc == IFX_OK && hipEventRecord(ev[2 * j + 1], s->stream) != hipSuccess)
        rc = set_error(IFX_E_HIP, "hipEventRecord failed");
    }
    if (rc == IFX_OK && hipStreamSynchronize(s->stream) != hipSuccess) rc = set_error(IFX_E_HIP, "sync failed");
    for (size_t j = 0; j < seq.size() && rc == IFX_OK; j++) {
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, ev[2 * j], ev[2 * j + 1]) != hipSuccess) rc = set_error(IFX_E_HIP, "event time");
      sum[seq[j].first] += ms;
      cnt[seq[j].first] += 1;
    }
    s->steps++;
  }
  if (rc == IFX_OK) s->len += n_steps;
  for (hipEvent_t e : ev)
    if (e) (void)hipEventDestroy(e);
  if (rc != IFX_OK) return rc;
  for (int k = 0; k < kClasses; k++) avg_ms[k] = cnt[k] ? (float)(sum[k] / (double)cnt[k]) : 0.f;
  return IFX_OK;
}

int ifx_session_last_token(ifx_session* s, uint32_t* token) {
  if (!s || !token) return set_error(IFX_E_INVALID_ARG, "null argument");
  IFX_HIP(hipStreamSynchronize(s->stream));
  IFX_HIP(hipMemcpy(token, &s->state->cur_token, 4, hipMemcpyDeviceToHost));
  return IFX_OK;
}

int ifx_session_last_elapsed_ms(const ifx_session* s, float* ms) {
  if (!s || !ms) return set_error(IFX_E_INVALID_ARG, "null argument");
  *ms = s->last_ms;
  return IFX_OK;
}

// Model::forward (src/model/forward.rs:448-482): non-causal attention over the
// chunk, no cache carried over.  Layer-major: each layer runs its GEMVs for all
// rows before the next layer, since every row attends to every other row.
// Model::forward: logits of every row into logits_out [n x vocab], or with
// last_only those of the last row alone [vocab] (the output head runs for
// that row only, on the decode head GEMV).
static int forward_rows(ifx_model* m, const uint32_t* ids, uint64_t n, float* logits_out, bool last_only) {
  if (!m || (n && (!ids || !logits_out))) return set_error(IFX_E_INVALID_ARG, "null argument");
  for (uint64_t i = 0; i < n; i++)
    if (ids[i] >= m->cfg.vocab_size) return set_error(IFX_E_INVALID_TENSOR_INDEX, "tensor index out of bounds: 0");
  if (n == 0) return IFX_OK;
  IFX_TRY(check_vocab(m));
  ifx_session* s = nullptr;
  IFX_TRY(ifx_session_create(m, n, &s));
  if (m->gemm_ok && n >= s->batch_min) {
    int rc = IFX_OK;
    if (hipMemcpyAsync(s->feed_ids, ids, n * 4, hipMemcpyHostToDevice, s->stream) != hipSuccess)
      rc = set_error(IFX_E_HIP, "forward: id upload failed");
    if (rc == IFX_OK) rc = batched_prefill(s, n, 0, false, last_only ? nullptr : logits_out);
    // the last row's logits, from the head GEMV the batched prefill runs on it
    if (rc == IFX_OK && last_only &&
        hipMemcpyAsync(logits_out, s->logits, (size_t)m->cfg.vocab_size * 4, hipMemcpyDeviceToHost, s->stream) !=
            hipSuccess)
      rc = set_error(IFX_E_HIP, "forward: logits copy failed");
    if (rc == IFX_OK && hipStreamSynchronize(s->stream) != hipSuccess) rc = set_error(IFX_E_HIP, "forward: sync failed");
    session_free(s);
    return rc;
  }
  const ifx_config& c = m->cfg;
  const uint64_t D = c.hidden_size, F = c.intermediate_size, kvd = c.n_kv_heads * c.head_dim;
  const size_t V = c.vocab_size;
  float *X = nullptr, *Q = nullptr, *A = nullptr;
  uint32_t* dids = nullptr;
  int rc = dev_alloc(s->allocs, (void**)&X, n * D * 4);
  if (rc == IFX_OK) rc = dev_alloc(s->allocs, (void**)&Q, n * D * 4);
  if (rc == IFX_OK) rc = dev_alloc(s->allocs, (void**)&A, n * D * 4);
  if (rc == IFX_OK) rc = dev_alloc(s->allocs, (void**)&dids, n * 4);
  hipStream_t st = s->stream;
  auto hip = [&](hipError_t e) {
    if (rc == IFX_OK && e != hipSuccess) rc = set_error(IFX_E_HIP, "forward: %s", hipGetErrorString(e));
  };
  if (rc == IFX_OK) {
    hip(hipMemcpyAsync(dids, ids, n * 4, hipMemcpyHostToDevice, st));
    hip(launch_embed_rows(devw(m->embd), dids, n, X, st));
  }
  for (size_t l = 0; l < m->layers.size() && rc == IFX_OK; l++) {
    const LayerDev& L = m->layers[l];
    void* kc = s->kc + l * s->max_seq * kvd * s->kv_es;
    void* vc = s->vc + l * s->max_seq * kvd * s->kv_es;
    const uint32_t kv16 = s->kv_es == 2;
    for (uint64_t t = 0; t < n && rc == IFX_OK; t++) {
      hip(launch_state(s->state, StateOp{STATE_TOKEN_AT, (uint32_t)t, (uint32_t)n}, st));
      GemvLaunch g;
      g.seg[0] = seg_of(L.q); g.seg[1] = seg_of(L.k); g.seg[2] = seg_of(L.v);
      g.nseg = 3; g.cols = (uint32_t)D; g.x = X + t * D; g.norm_w = L.attn_norm; g.eps = c.norm_eps;
      QkvEpi e{Q + t * D, kc, vc, s->rope_cs, s->state, (uint32_t)c.head_dim, (uint32_t)c.rope_dim, (uint32_t)kvd,
               (uint32_t)s->max_seq, kv16};
      hip(gemv_qkv(g, e, st));
    }
    for (uint64_t t = 0; t < n && rc == IFX_OK; t++) {
      hip(launch_state(s->state, StateOp{STATE_TOKEN_AT, (uint32_t)t, (uint32_t)n}, st));
      AttnArgs a{Q + t * D, kc, vc, A + t * D, s->partial, s->state, (uint32_t)c.n_heads,
                 (uint32_t)c.n_kv_heads, (uint32_t)c.head_dim, s->max_chunks, s->attn_chunk,
                 (uint32_t)s->max_seq, kv16};
      hip(launch_attn_decode(a, st));
    }
    for (uint64_t t = 0; t < n && rc == IFX_OK; t++) {
      GemvLaunch go;
      go.seg[0] = seg_of(L.o); go.nseg = 1; go.cols = (uint32_t)D; go.x = A + t * D;
      hip(gemv_residual(go, X + t * D, st));
      GemvLaunch gf;
      gf.seg[0] = seg_of(L.gate); gf.seg[1] = seg_of(L.up); gf.nseg = 2; gf.paired = true;
      gf.cols = (uint32_t)D; gf.x = X + t * D; gf.norm_w = L.ffn_norm; gf.eps = c.norm_eps;
      hip(gemv_swiglu(gf, s->mid, st));
      GemvLaunch gd;
      gd.seg[0] = seg_of(L.down); gd.nseg = 1; gd.cols = (uint32_t)F; gd.x = s->mid;
      hip(gemv_residual(gd, X + t * D, st));
    }
  }
  for (uint64_t t = last_only ? n - 1 : 0; t < n && rc == IFX_OK; t++) {
    GemvLaunch gh;
    gh.seg[0] = seg_of(m->output); gh.nseg = 1; gh.cols = (uint32_t)D; gh.x = X + t * D;
    gh.norm_w = m->out_norm; gh.eps = c.norm_eps;
    hip(gemv_logits(gh, s->logits, s->state, st));
    hip(hipMemcpyAsync(logits_out + (last_only ? 0 : t) * V, s->logits, V * 4, hipMemcpyDeviceToHost, st));
  }
  hip(hipStreamSynchronize(st));
  session_free(s);
  return rc;
}

int ifx_forward(ifx_model* m, const uint32_t* ids, uint64_t n, float* logits_out) {
  clear_error();
  return forward_rows(m, ids, n, logits_out, false);
}

int ifx_forward_last_token_logits(ifx_model* m, const uint32_t* ids, uint64_t n, float* logits_out) {
  clear_error();
  // the reference slices the last vocab_size logits, which an empty prompt does not have
  if (n == 0) return set_error(IFX_E_INVALID_ARG, "forward_last_token_logits of an empty prompt");
  return forward_rows(m, ids, n, logits_out, true);
}

}  // extern "C"
