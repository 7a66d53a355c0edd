// kern_dequant.hip — bit-exact dequantization kernels and the embedding gather.
// Compiled with -ffp-contract=off (see inferox_amd/build.py).
#include <algorithm>

#include "kernels.h"

namespace ifx {

// Raw GGUF stream -> f32 (gguf::dequantize_f32, src/gguf/dequant.rs:10-31).
__global__ void __launch_bounds__(256) k_dequant_raw(uint32_t type, const uint8_t* __restrict__ p,
                                                     uint64_t n, float* __restrict__ out) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) out[i] = raw_elem(type, p, i);
}

// Device-layout matrix -> f32.
__global__ void __launch_bounds__(256) k_dequant_dev(DevW w, uint64_t n, float* __restrict__ out) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) out[i] = dev_elem(w, i);
}

// out[r][:] = row ids[r] of the table (embedding_lookup, src/ops.rs:246-258,
// over the dequantized table as src/model/forward.rs:505-507 builds it).
__global__ void __launch_bounds__(256) k_embed_rows(DevW w, const uint32_t* __restrict__ ids,
                                                    float* __restrict__ out) {
  uint64_t row = ids[blockIdx.y];
  float* o = out + (uint64_t)blockIdx.y * w.cols;
  for (uint64_t c = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; c < w.cols;
       c += (uint64_t)gridDim.x * blockDim.x)
    o[c] = dev_elem(w, row * w.cols + c);
}

// hidden = row cur_token (Model::decode_step, src/model/forward.rs:556-558).
// It also clears the rows of the step's first K-split q/k/v launch (clr).
__global__ void __launch_bounds__(256) k_embed_state(DevW w, const DevState* __restrict__ s,
                                                     float* __restrict__ hidden, QkvClear clr) {
  uint64_t row = s->cur_token;
  const uint32_t len = s->len;
  qkv_clear(clr, len, blockIdx.x, gridDim.x, threadIdx.x, blockDim.x);
  for (uint64_t c = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; c < w.cols;
       c += (uint64_t)gridDim.x * blockDim.x)
    hidden[c] = dev_elem(w, row * w.cols + c);
}

static unsigned grid_for(uint64_t n) {
  uint64_t g = (n + 255) / 256;
  return (unsigned)(g < 8192 ? (g ? g : 1) : 8192);
}

hipError_t launch_dequant_raw(uint32_t type, const uint8_t* bytes, uint64_t n, float* out,
                              hipStream_t st) {
  hipLaunchKernelGGL(k_dequant_raw, dim3(grid_for(n)), dim3(256), 0, st, type, bytes, n, out);
  return hipGetLastError();
}

hipError_t launch_dequant_dev(const DevW& w, uint64_t n, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_dequant_dev, dim3(grid_for(n)), dim3(256), 0, st, w, n, out);
  return hipGetLastError();
}

hipError_t launch_embed_rows(const DevW& w, const uint32_t* ids, uint64_t n_ids, float* out,
                             hipStream_t st) {
  if (n_ids == 0) return hipSuccess;
  unsigned gx = (unsigned)((w.cols + 255) / 256);
  hipLaunchKernelGGL(k_embed_rows, dim3(gx, (unsigned)n_ids), dim3(256), 0, st, w, ids, out);
  return hipGetLastError();
}

hipError_t launch_embed_state(const DevW& w, const DevState* state, float* hidden, hipStream_t st,
                              const QkvClear& clr) {
  const unsigned gx = (unsigned)std::max<uint64_t>((w.cols + 255) / 256, (clr.floats() + 1023) / 1024);
  hipLaunchKernelGGL(k_embed_state, dim3(gx), dim3(256), 0, st, w, state, hidden, clr);
  return hipGetLastError();
}

}  // namespace ifx
