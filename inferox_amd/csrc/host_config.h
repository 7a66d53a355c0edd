// host_config.h — Config::from_gguf (src/model/config.rs:34-84) and the weight
// resolution of Model::open / Layer::from_weights (src/model/mod.rs:34-92),
// host only: everything a model open decides from the file's metadata and
// tensor table before any device work.
#pragma once

#include <stdint.h>

#include <vector>

#include "host_gguf.h"
#include "ifx_common.h"

namespace ifx {

// The nine per-layer tensors, in the order of ModelPlan::layers.
enum LayerRole { R_ATTN_NORM, R_Q, R_K, R_V, R_O, R_FFN_NORM, R_GATE, R_UP, R_DOWN, R_COUNT };
extern const char* const kLayerRoleNames[R_COUNT];

struct PlanMatrix {
  int64_t idx = -1;  // index into GgufFile::tensors
  uint64_t rows = 0, cols = 0;
};

struct ModelPlan {
  ifx_config cfg{};
  PlanMatrix embd, output;     // output.idx < 0: tied to token_embd (src/model/forward.rs:573)
  int64_t out_norm = -1;
  std::vector<int64_t> layers;  // [n_layers][R_COUNT] tensor indices
};

// Config + name resolution.  Statuses as Model::open reports them:
// TENSOR_NOT_FOUND for a missing required key or tensor (the first missing
// blk.N.* ends the walk over block_count, so a huge or wrapping count sizes
// nothing), UNSUPPORTED_ARCH, INVALID_ARG for head_count 0.
int plan_model(const GgufFile& f, ModelPlan* out);

// The matrix shapes every weight must have ([rows x cols], cols contiguous):
// token_embd / output [* x hidden], q/o [hidden x hidden], k/v [kv_dim x
// hidden], gate/up [ffn x hidden], down [hidden x ffn], norms [hidden];
// INVALID_ARG when a tensor's element count differs or a product overflows.
// rows_of(role) of a layer matrix is stored in *shapes ([R_COUNT] of {rows, cols}).
int plan_shapes(const GgufFile& f, ModelPlan* plan, uint64_t shapes[R_COUNT][2]);

}  // namespace ifx
