// kern_ops.hip — f32 operators (src/ops.rs) on device buffers, greedy argmax
// and the per-step state kernels.  Compiled with -ffp-contract=off.
#include "kernels.h"

namespace ifx {

namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Block-wide reduction (256 threads) through LDS.
template <bool MAX>
__device__ float block_reduce(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = MAX ? wave_max(v) : wave_sum(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
  for (int w = 1; w < nw; w++) t = MAX ? fmaxf(t, red[w]) : t + red[w];
  return t;
}

// ops::matmul_t (src/ops.rs:33-44): c[i][j] = sum_l a[i][l] * b[j][l].
// One wave per output element; lanes stride over l.
__global__ void __launch_bounds__(256) k_matmul_t(const float* __restrict__ a, const float* __restrict__ b,
                                                  float* __restrict__ c, uint64_t m, uint64_t n, uint64_t k) {
  const uint64_t out = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (out >= m * n) return;
  const uint64_t i = out / n, j = out % n;
  float s = 0.f;
  for (uint64_t l = lane; l < k; l += 64) s = fmaf(a[i * k + l], b[j * k + l], s);
  s = wave_sum(s);
  if (lane == 0) c[out] = s;
}

// ops::rms_norm_rows (src/ops.rs:155-180).
__global__ void __launch_bounds__(256) k_rms_norm(float* __restrict__ x, const float* __restrict__ w,
                                                  uint64_t n, float eps) {
  __shared__ float red[4];
  float* row = x + (uint64_t)blockIdx.x * n;
  float ss = 0.f;
  for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(row[i], row[i], ss);
  ss = block_reduce<false>(ss, red);
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
  for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) row[i] = (row[i] * scale) * w[i];
}

__device__ __forceinline__ float silu_ref(float g) {
  float c = fminf(fmaxf(g, -80.f), 80.f);
  if (g != g) c = g;
  return g * (1.0f / (1.0f + expf(-c)));
}

__global__ void k_swiglu(const float* g, const float* u, float* o, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    o[i] = silu_ref(g[i]) * u[i];
}

__global__ void k_add(float* o, const float* b, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    o[i] = o[i] + b[i];
}

// ops::softmax_rows (src/ops.rs:223-239): max (NaN-skipping, like f32::max),
// exp(v - max), sum, divide.
__global__ void __launch_bounds__(256) k_softmax(float* __restrict__ x, uint64_t cols) {
  __shared__ float red[4];
  float* row = x + (uint64_t)blockIdx.x * cols;
  float mx = -INFINITY;
  for (uint64_t i = threadIdx.x; i < cols; i += blockDim.x) mx = fmaxf(mx, row[i]);
  mx = block_reduce<true>(mx, red);
  float s = 0.f;
  for (uint64_t i = threadIdx.x; i < cols; i += blockDim.x) {
    const float e = expf(row[i] - mx);
    row[i] = e;
    s += e;
  }
  s = block_reduce<false>(s, red);
  for (uint64_t i = threadIdx.x; i < cols; i += blockDim.x) row[i] = row[i] / s;
}

// ops::rope (src/ops.rs:265-287) with positions pos0 + p.
__global__ void k_rope(float* x, uint64_t seq, uint64_t heads, uint64_t hd, uint64_t rope_dim,
                       float base, uint64_t pos0) {
  const uint64_t pairs = rope_dim / 2, total = seq * heads * pairs;
  for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t p = t / (heads * pairs), h = (t / pairs) % heads, i = 2 * (t % pairs);
    float* v = x + (p * heads + h) * hd + i;
    const float a = v[0], b = v[1];
    const float inv = 1.0f / powf(base, (float)i / (float)rope_dim);
    const float ang = (float)(pos0 + p) * inv;
    const float sn = sinf(ang), cs = cosf(ang);
    v[0] = a * cs - b * sn;
    v[1] = a * sn + b * cs;
  }
}

__device__ __forceinline__ unsigned long long order_key(float v, uint32_t idx) {
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | idx;
}

// argmax (src/model/forward.rs:615-622): the last index of the maximum; a NaN
// sets *status.  One workgroup.
__global__ void __launch_bounds__(1024) k_argmax(const float* __restrict__ x, uint64_t n,
                                                 uint32_t* out, int* status) {
  __shared__ unsigned long long best[16];
  __shared__ int nan_seen;
  if (threadIdx.x == 0) nan_seen = 0;
  __syncthreads();
  unsigned long long b = 0;
  bool nan = false;
  for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = x[i];
    if (v != v) nan = true;
    const unsigned long long k = order_key(v, (uint32_t)i);
    b = k > b ? k : b;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(b, off, 64);
    b = o > b ? o : b;
  }
  if (nan) nan_seen = 1;
  if ((threadIdx.x & 63) == 0) best[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long t = 0;
    for (unsigned w = 0; w < blockDim.x / 64; w++) t = best[w] > t ? best[w] : t;
    *out = n <= 1 ? 0u : (uint32_t)(t & 0xffffffffu);
    if (status) *status = (nan_seen && n > 1) ? (int)IFX_E_NAN_LOGIT : (int)IFX_OK;
  }
}

// End of one token: record the greedy pick, advance the cache length and set
// the position rule of the next token.
__global__ void k_finalize(DevState* s) {
  const uint32_t tok = (uint32_t)(s->argmax_key & 0xffffffffull);
  const uint32_t nan_bit = s->status == IFX_E_NAN_LOGIT ? 0x80000000u : 0u;
  if (s->step < s->out_cap) s->out_tokens[s->step] = tok | nan_bit;
  s->status = IFX_OK;
  s->step += 1;
  s->argmax_key = 0ull;
  s->len += 1;
  uint32_t next = tok;
  if (s->prefill) {
    const uint32_t t = s->len - s->chunk_start;
    if (t < s->feed_n) next = s->feed_ids[t];
    else s->prefill = 0;
  }
  s->cur_token = next;
  if (s->prefill) {
    s->rope_pos = s->rope_mode == IFX_ROPE_ABSOLUTE ? s->len : s->len - s->chunk_start;
    s->attn_lo = s->chunk_start;
  } else {
    s->rope_pos = s->rope_mode == IFX_ROPE_ABSOLUTE ? s->len : 0u;
    s->attn_lo = 0u;
  }
}

// Host-requested state transitions (a kernel, so they order with the step
// kernels on the stream and are safe to use around captured graphs).
__global__ void k_state(DevState* s, StateOp op) {
  switch (op.kind) {
    case STATE_RESET:
      s->len = op.len;
      s->step = 0;
      s->prefill = 0;
      s->argmax_key = 0ull;
      s->status = IFX_OK;
      s->attn_lo = 0;
      s->attn_end = 0;
      s->rope_pos = s->rope_mode == IFX_ROPE_ABSOLUTE ? op.len : 0u;
      break;
    case STATE_MODE:
      s->rope_mode = op.value;
      break;
    case STATE_SAMPLER:
      s->temperature = op.f0;
      s->top_k = op.value;
      s->top_p = op.f1;
      s->seed = op.seed;
      break;
    case STATE_DECODE:  // decode_step at the current length
      s->cur_token = op.value;
      s->prefill = 0;
      s->attn_lo = 0;
      s->attn_end = 0;
      s->rope_pos = s->rope_mode == IFX_ROPE_ABSOLUTE ? s->len : 0u;
      break;
    case STATE_PREFILL:  // a chunk of op.len ids at feed_ids, cache_start = len
      s->prefill = 1;
      s->chunk_start = s->len;
      s->feed_n = op.len;
      s->cur_token = s->feed_ids[0];
      s->attn_lo = s->len;
      s->attn_end = 0;
      s->rope_pos = s->rope_mode == IFX_ROPE_ABSOLUTE ? s->len : 0u;
      break;
    case STATE_BATCH:  // a batched prefill of op.len rows wrote its K/V rows: the next
                       // finalize records the last row's greedy pick as a step would
      s->len += op.len - 1u;
      s->step += op.len - 1u;
      s->prefill = 0;
      s->attn_lo = 0;
      s->attn_end = 0;
      s->argmax_key = 0ull;
      s->status = IFX_OK;
      break;
    case STATE_TOKEN_AT:  // non-causal forward: token op.value of a chunk of op.len rows
      s->len = op.value;
      s->prefill = 0;
      s->attn_lo = 0;
      s->attn_end = op.len;
      s->rope_pos = op.value;
      break;
  }
}

__global__ void k_fill_u32(uint32_t* p, uint32_t v, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

unsigned blocks_for(uint64_t n, unsigned per = 256) {
  uint64_t g = (n + per - 1) / per;
  return (unsigned)(g == 0 ? 1 : (g > 4096 ? 4096 : g));
}

}  // namespace

hipError_t launch_matmul_t_f32(const float* a, const float* b, float* c, uint64_t m, uint64_t n,
                               uint64_t k, hipStream_t st) {
  if (m * n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_matmul_t, dim3((unsigned)((m * n + 3) / 4)), dim3(256), 0, st, a, b, c, m, n, k);
  return hipGetLastError();
}

hipError_t launch_rms_norm_rows(float* x, const float* w, uint64_t n, uint64_t rows, float eps,
                                hipStream_t st) {
  if (rows == 0 || n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rms_norm, dim3((unsigned)rows), dim3(256), 0, st, x, w, n, eps);
  return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, float* o, uint64_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_swiglu, dim3(blocks_for(n)), dim3(256), 0, st, g, u, o, n);
  return hipGetLastError();
}

hipError_t launch_add(float* o, const float* b, uint64_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_add, dim3(blocks_for(n)), dim3(256), 0, st, o, b, n);
  return hipGetLastError();
}

hipError_t launch_softmax_rows(float* x, uint64_t rows, uint64_t cols, hipStream_t st) {
  if (rows == 0 || cols == 0) return hipSuccess;
  hipLaunchKernelGGL(k_softmax, dim3((unsigned)rows), dim3(256), 0, st, x, cols);
  return hipGetLastError();
}

hipError_t launch_rope(float* x, uint64_t seq, uint64_t heads, uint64_t hd, uint64_t rope_dim,
                       float base, uint64_t pos0, hipStream_t st) {
  hipLaunchKernelGGL(k_rope, dim3(blocks_for(seq * heads * (rope_dim / 2))), dim3(256), 0, st, x, seq,
                     heads, hd, rope_dim, base, pos0);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* x, uint64_t n, uint32_t* out, int* status, hipStream_t st) {
  hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, st, x, n, out, status);
  return hipGetLastError();
}

hipError_t launch_finalize(DevState* state, hipStream_t st) {
  hipLaunchKernelGGL(k_finalize, dim3(1), dim3(1), 0, st, state);
  return hipGetLastError();
}

hipError_t launch_state(DevState* state, const StateOp& op, hipStream_t st) {
  hipLaunchKernelGGL(k_state, dim3(1), dim3(1), 0, st, state, op);
  return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t v, uint64_t n, hipStream_t st) {
  hipLaunchKernelGGL(k_fill_u32, dim3(blocks_for(n)), dim3(256), 0, st, p, v, n);
  return hipGetLastError();
}

}  // namespace ifx
