// host_config.cpp — model metadata and weight resolution (host only).
#include "host_config.h"

#include <stdio.h>

#include <string>

namespace ifx {

const char* const kLayerRoleNames[R_COUNT] = {"attn_norm", "attn_q",   "attn_k", "attn_v", "attn_output",
                                              "ffn_norm",  "ffn_gate", "ffn_up", "ffn_down"};

int plan_model(const GgufFile& f, ModelPlan* out) {
  ModelPlan p;
  ifx_config& c = p.cfg;
  std::string arch;
  if (!f.get_string("general.architecture", &arch)) return set_error(IFX_E_TENSOR_NOT_FOUND, "general.architecture");
  if (arch != "llama") return set_error(IFX_E_UNSUPPORTED_ARCH, "unsupported model architecture: %s", arch.c_str());
  snprintf(c.architecture, sizeof c.architecture, "%s", arch.c_str());
  const char* req[3] = {"llama.embedding_length", "llama.block_count", "llama.attention.head_count"};
  uint64_t* dst[3] = {&c.hidden_size, &c.n_layers, &c.n_heads};
  for (int i = 0; i < 3; i++)
    if (!f.get_u64(req[i], dst[i])) return set_error(IFX_E_TENSOR_NOT_FOUND, "%s", req[i]);
  uint32_t u;
  c.n_kv_heads = f.get_u32("llama.attention.head_count_kv", &u) ? u : c.n_heads;
  if (c.n_heads == 0) return set_error(IFX_E_INVALID_ARG, "head_count is 0");
  c.head_dim = f.get_u32("llama.attention.key_length", &u) ? u : c.hidden_size / c.n_heads;
  if (!f.get_u64("llama.feed_forward_length", &c.intermediate_size))
    return set_error(IFX_E_TENSOR_NOT_FOUND, "llama.feed_forward_length");
  if (!f.get_f32("llama.attention.layer_norm_rms_epsilon", &c.norm_eps)) c.norm_eps = 1e-5f;
  if (!f.get_f32("llama.rope.freq_base", &c.rope_base)) c.rope_base = 10000.0f;
  c.rope_dim = f.get_u32("llama.rope.dimension_count", &u) ? u : c.head_dim;
  c.context_length = f.get_u32("llama.context_length", &u) ? u : 4096;
  c.vocab_size = f.get_u32("llama.vocab_size", &u) ? u : 0;

  // block_count comes from the file: the indices grow one layer at a time, so
  // a count larger than the file's tensors can hold ends at the first missing
  // blk.N tensor (TensorNotFound, as the reference reports it) without sizing
  // anything by it
  for (uint64_t l = 0; l < c.n_layers; l++)
    for (int r = 0; r < R_COUNT; r++) {
      char nm[128];
      snprintf(nm, sizeof nm, "blk.%llu.%s.weight", (unsigned long long)l, kLayerRoleNames[r]);
      const int64_t ti = f.tensor_index(nm);
      if (ti < 0) return set_error(IFX_E_TENSOR_NOT_FOUND, "blk.%llu.*", (unsigned long long)l);
      p.layers.push_back(ti);
    }
  p.embd.idx = f.tensor_index("token_embd.weight");
  if (p.embd.idx < 0) return set_error(IFX_E_TENSOR_NOT_FOUND, "token_embd.weight");
  p.out_norm = f.tensor_index("output_norm.weight");
  if (p.out_norm < 0) return set_error(IFX_E_TENSOR_NOT_FOUND, "output_norm.weight");
  p.output.idx = f.tensor_index("output.weight");
  *out = std::move(p);
  return IFX_OK;
}

int plan_shapes(const GgufFile& f, ModelPlan* p, uint64_t shapes[R_COUNT][2]) {
  const ifx_config& c = p->cfg;
  const uint64_t D = c.hidden_size, F = c.intermediate_size;
  uint64_t KV;
  if (!mul_u64(c.n_kv_heads, c.head_dim, &KV))
    return set_error(IFX_E_INVALID_ARG, "kv dim %llu x %llu overflows", (unsigned long long)c.n_kv_heads,
                     (unsigned long long)c.head_dim);
  const uint64_t sh[R_COUNT][2] = {{1, D}, {D, D}, {KV, D}, {KV, D}, {D, D}, {1, D}, {F, D}, {F, D}, {D, F}};
  for (int r = 0; r < R_COUNT; r++) {
    shapes[r][0] = sh[r][0];
    shapes[r][1] = sh[r][1];
  }
  // token_embd and output: [* x hidden]
  const uint64_t embd_n = f.tensors[p->embd.idx].n_elements();
  if (D == 0 || embd_n % D)
    return set_error(IFX_E_INVALID_ARG, "token_embd.weight is not [*, %llu]", (unsigned long long)D);
  p->embd.rows = embd_n / D;
  p->embd.cols = D;
  if (p->output.idx >= 0) {
    const uint64_t n = f.tensors[p->output.idx].n_elements();
    if (n % D) return set_error(IFX_E_INVALID_ARG, "output.weight is not [*, %llu]", (unsigned long long)D);
    p->output.rows = n / D;
    p->output.cols = D;
  }
  if (f.tensors[p->out_norm].n_elements() != D)
    return set_error(IFX_E_INVALID_ARG, "output_norm.weight has %llu elements, expected %llu",
                     (unsigned long long)f.tensors[p->out_norm].n_elements(), (unsigned long long)D);
  for (size_t i = 0; i < p->layers.size(); i++) {
    const int r = (int)(i % R_COUNT);
    const GgufTensor& t = f.tensors[p->layers[i]];
    uint64_t n;
    if (!mul_u64(sh[r][0], sh[r][1], &n) || t.n_elements() != n)
      return set_error(IFX_E_INVALID_ARG, "%s has %llu elements, expected %llu x %llu", t.name.c_str(),
                       (unsigned long long)t.n_elements(), (unsigned long long)sh[r][0],
                       (unsigned long long)sh[r][1]);
  }
  return IFX_OK;
}

}  // namespace ifx
