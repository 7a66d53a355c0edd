// capi_ops.cpp — device plumbing, dequantization, uploaded matrices, GEMV and
// the f32 operators of include/inferox.h.
#include <string.h>

#include <algorithm>
#include <mutex>
#include <thread>
#include <vector>

#include "ifx_common.h"
#include "kernels.h"

using namespace ifx;

namespace ifx {

static std::once_flag g_init_once;
static int g_init_status = IFX_OK;
static hipStream_t g_stream = nullptr;
static hipEvent_t g_ev0 = nullptr, g_ev1 = nullptr;

// The library targets gfx950 only: refuse any other device loudly.
int device_init() {
  std::call_once(g_init_once, [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
      g_init_status = IFX_E_NO_DEVICE;
      return;
    }
    hipDeviceProp_t prop;
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess || strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
      g_init_status = IFX_E_NO_DEVICE;
      return;
    }
    if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&g_ev0) != hipSuccess || hipEventCreate(&g_ev1) != hipSuccess)
      g_init_status = IFX_E_HIP;
  });
  if (g_init_status != IFX_OK)
    return set_error(g_init_status, "no usable gfx950 device (HIP device count / arch check failed)");
  return IFX_OK;
}

static hipStream_t stream_of(void* s) { return s ? (hipStream_t)s : g_stream; }
hipStream_t library_stream() { return g_stream; }
hipStream_t ops_stream(void* s) { return stream_of(s); }

DevW devw(const ifx_tensor* t) {
  DevW w{t->L.type, t->L.cols, t->L.body, t->L.scal, t->L.q6_signed, 0, 0};
  if (t->L.type == T_Q4K || t->L.type == T_Q6K)
    tile_strides(t->L.type, t->L.rows, &w.tstride, &w.bstride);
  return w;
}

// Runs fn(i0, i1) over [0, n) in contiguous ranges, one worker per core share.
template <class F>
static void parallel_ranges(uint64_t n, uint64_t min_per_worker, F fn) {
  unsigned nt = std::thread::hardware_concurrency();
  nt = nt == 0 ? 1 : (nt > 16 ? 16 : nt);
  if (n < (uint64_t)nt * min_per_worker) nt = (unsigned)std::max<uint64_t>(1, n / min_per_worker);
  std::vector<std::thread> th;
  const uint64_t per = (n + nt - 1) / nt;
  for (unsigned i = 0; i < nt; i++) {
    const uint64_t a = i * per, b = a + per < n ? a + per : n;
    if (a >= b) break;
    th.emplace_back([=] { fn(a, b); });
  }
  for (auto& t : th) t.join();
}

int upload_matrix(uint32_t type, const uint8_t* src, uint64_t nbytes, uint64_t rows, uint64_t cols,
                  ifx_tensor** out, uint32_t flags) {
  *out = nullptr;
  std::vector<uint8_t> converted;  // ggml K-quant blocks rewritten as the reference's
  const bool ggml = (flags & IFX_OPEN_GGML_KQUANTS) != 0;
  if (ggml && type == T_Q8K)
    return set_error(IFX_E_UNKNOWN_TENSOR_TYPE, "ggml's Q8_K is not a storage type of the reference's layout");
  if (!gemv_supported(type))
    return set_error(IFX_E_UNKNOWN_TENSOR_TYPE, "tensor type %u has no device layout", type);
  // the kernels index rows and columns in 32 bits; the product is checked so
  // that no size below is taken modulo 2^64
  uint64_t n_el;
  if (rows == 0 || cols == 0 || rows >= (1ull << 31) || cols >= (1ull << 31) || !mul_u64(rows, cols, &n_el))
    return set_error(IFX_E_INVALID_ARG, "matrix shape [%llu x %llu] out of range", (unsigned long long)rows,
                     (unsigned long long)cols);
  uint64_t expect;
  if (!byte_size(type, n_el, &expect))
    return set_error(IFX_E_UNKNOWN_TENSOR_TYPE, "tensor type %u", type);
  if (expect != nbytes)
    return set_error(IFX_E_UNEXPECTED_EOF, "%llu bytes for a %s [%llu x %llu] matrix, %llu expected",
                     (unsigned long long)nbytes, type_name(type), (unsigned long long)rows,
                     (unsigned long long)cols, (unsigned long long)expect);
  if (ggml && (type == T_Q4K || type == T_Q6K)) {
    const uint64_t bb = type == T_Q4K ? 144 : 210, nb = nbytes / bb;
    converted.resize(nbytes);
    parallel_ranges(nb, 65536, [&](uint64_t b0, uint64_t b1) {
      ggml_kquant_to_reference(type, src + b0 * bb, b1 - b0, converted.data() + b0 * bb);
    });
    src = converted.data();
  }
  uint64_t body, scal;
  if (!layout_sizes(type, rows, cols, &body, &scal))
    return set_error(IFX_E_INVALID_ARG, "%s rows of %llu columns are not whole blocks", type_name(type),
                     (unsigned long long)cols);
  ifx_tensor* t = new ifx_tensor();
  const uint64_t body_al = (body + 255) / 256 * 256;
  if (hipMalloc(&t->alloc, body_al + scal + 16) != hipSuccess) {
    delete t;
    return set_error(IFX_E_OOM, "hipMalloc of %llu bytes failed", (unsigned long long)(body_al + scal));
  }
  t->L.type = type;
  t->L.rows = rows;
  t->L.cols = cols;
  t->L.body = (uint8_t*)t->alloc;
  t->L.scal = scal ? (uint8_t*)t->alloc + body_al : nullptr;
  t->L.body_bytes = body;
  t->L.scal_bytes = scal;
  t->L.gguf_bytes = nbytes;
  t->L.q6_signed = ggml && type == T_Q6K;
  uint64_t be = 1, bb = 0;
  if (type == T_F32 || type == T_F16) { be = 1; bb = element_size(type); }
  else block_layout(type, &be, &bb);
  t->L.n_blocks = rows * cols / be;
  t->L.blocks_per_row = cols / be;
  hipError_t e;
  if (type == T_F32 || type == T_F16) {
    e = hipMemcpy(t->L.body, src, nbytes, hipMemcpyHostToDevice);
  } else {
    std::vector<uint8_t> stage(body + scal);
    if (type == T_Q4K || type == T_Q6K) {
      const uint64_t tiles = (rows + kTileRows - 1) / kTileRows;
      parallel_ranges(tiles, 64, [&](uint64_t t0, uint64_t t1) {
        repack_tiles(type, src, rows, cols, t0, t1, stage.data());
      });
    } else {
      const uint64_t nb = t->L.n_blocks, body_bb = body / nb, scal_bb = scal / nb;
      uint8_t* sp = scal ? stage.data() + body : nullptr;
      parallel_ranges(nb, 65536, [&](uint64_t b0, uint64_t b1) {
        repack_to_device_layout(type, src + b0 * bb, b1 - b0, stage.data() + b0 * body_bb,
                                sp ? sp + b0 * scal_bb : nullptr);
      });
    }
    e = hipMemcpy(t->L.body, stage.data(), body, hipMemcpyHostToDevice);
    if (e == hipSuccess && scal) e = hipMemcpy(t->L.scal, stage.data() + body, scal, hipMemcpyHostToDevice);
    std::mutex mu;
    float bound = 0.f;
    parallel_ranges(t->L.n_blocks, 65536, [&](uint64_t b0, uint64_t b1) {
      const float v = block_abs_bound(type, src, b0, b1);
      std::lock_guard<std::mutex> g(mu);
      bound = (v > bound || v != v) ? v : bound;
    });
    t->L.abs_bound = bound;
    if (type == T_Q4K) {
      float dm = 0.f;
      parallel_ranges(t->L.n_blocks, 65536, [&](uint64_t b0, uint64_t b1) {
        const float v = block_dmin_max(src, b0, b1);
        std::lock_guard<std::mutex> g(mu);
        dm = (v > dm || v != v) ? v : dm;
      });
      t->L.dmin_max = dm;
    }
  }
  if (type == T_F32 || type == T_F16) t->L.abs_bound = INFINITY;
  if (e != hipSuccess) {
    (void)hipFree(t->alloc);
    delete t;
    return set_error(IFX_E_HIP, "upload failed: %s", hipGetErrorString(e));
  }
  *out = t;
  return IFX_OK;
}

}  // namespace ifx

extern "C" {

const char* ifx_last_error(void) { return last_error(); }

const char* ifx_status_string(int s) {
  switch (s) {
    case IFX_OK: return "ok";
    case IFX_E_IO: return "io error";
    case IFX_E_INVALID_MAGIC: return "invalid magic";
    case IFX_E_UNSUPPORTED_VERSION: return "unsupported GGUF version";
    case IFX_E_UNKNOWN_VALUE_TYPE: return "unknown metadata value type";
    case IFX_E_UNKNOWN_TENSOR_TYPE: return "unknown tensor type";
    case IFX_E_INVALID_UTF8: return "invalid utf-8 string";
    case IFX_E_INVALID_SHAPE: return "invalid tensor shape";
    case IFX_E_UNEXPECTED_EOF: return "unexpected end of file";
    case IFX_E_TENSOR_NOT_FOUND: return "tensor not found";
    case IFX_E_INVALID_TENSOR_INDEX: return "tensor index out of bounds";
    case IFX_E_TENSOR_OFFSET_OVERFLOW: return "tensor byte range overflows file bounds";
    case IFX_E_UNSUPPORTED_ARCH: return "unsupported model architecture";
    case IFX_E_JSON: return "json error";
    case IFX_E_UNSUPPORTED_TOKENIZER: return "unsupported tokenizer model";
    case IFX_E_INVALID_ARG: return "invalid argument";
    case IFX_E_KV_FULL: return "KV cache full";
    case IFX_E_HIP: return "HIP runtime error";
    case IFX_E_OOM: return "out of memory";
    case IFX_E_NAN_LOGIT: return "NaN logit in argmax";
    case IFX_E_NO_DEVICE: return "no gfx950 device";
    default: return "unknown status";
  }
}

int ifx_device_info(char* name, uint64_t cap, int* n_cu, uint64_t* hbm) {
  IFX_TRY(device_init());
  int dev = 0;
  IFX_HIP(hipGetDevice(&dev));
  hipDeviceProp_t p;
  IFX_HIP(hipGetDeviceProperties(&p, dev));
  if (name && cap) snprintf(name, cap, "%s (%s)", p.name, p.gcnArchName);
  if (n_cu) *n_cu = p.multiProcessorCount;
  if (hbm) *hbm = p.totalGlobalMem;
  return IFX_OK;
}

int ifx_malloc(void** p, uint64_t bytes) {
  IFX_TRY(device_init());
  if (!p) return set_error(IFX_E_INVALID_ARG, "null pointer");
  if (hipMalloc(p, bytes ? bytes : 4) != hipSuccess) return set_error(IFX_E_OOM, "hipMalloc(%llu)", (unsigned long long)bytes);
  return IFX_OK;
}

int ifx_free(void* p) {
  if (p) IFX_HIP(hipFree(p));
  return IFX_OK;
}

int ifx_memcpy_h2d(void* d, const void* s, uint64_t n) { IFX_TRY(device_init()); IFX_HIP(hipMemcpy(d, s, n, hipMemcpyHostToDevice)); return IFX_OK; }
int ifx_memcpy_d2h(void* d, const void* s, uint64_t n) { IFX_TRY(device_init()); IFX_HIP(hipStreamSynchronize(g_stream)); IFX_HIP(hipMemcpy(d, s, n, hipMemcpyDeviceToHost)); return IFX_OK; }
int ifx_memcpy_d2d(void* d, const void* s, uint64_t n) { IFX_TRY(device_init()); IFX_HIP(hipMemcpyAsync(d, s, n, hipMemcpyDeviceToDevice, g_stream)); return IFX_OK; }
int ifx_stream_synchronize(void* s) { IFX_TRY(device_init()); IFX_HIP(hipStreamSynchronize(stream_of(s))); return IFX_OK; }

int ifx_timer_start(void* s) {
  IFX_TRY(device_init());
  IFX_HIP(hipEventRecord(g_ev0, stream_of(s)));
  return IFX_OK;
}

int ifx_timer_stop(void* s, float* ms) {
  IFX_TRY(device_init());
  IFX_HIP(hipEventRecord(g_ev1, stream_of(s)));
  IFX_HIP(hipEventSynchronize(g_ev1));
  IFX_HIP(hipEventElapsedTime(ms, g_ev0, g_ev1));
  return IFX_OK;
}

// gguf::dequantize_f32 (src/gguf/dequant.rs:10-31), same check order.
int ifx_dequantize_f32(uint32_t type, uint64_t n_elements, const void* bytes, uint64_t n_bytes,
                       float* out, uint64_t n_out, void* stream) {
  clear_error();
  IFX_TRY(device_init());
  uint64_t expected;
  if (!byte_size(type, n_elements, &expected))
    return set_error(IFX_E_UNKNOWN_TENSOR_TYPE, "unknown tensor type id: %u", type);
  if (n_bytes != expected) return set_error(IFX_E_UNEXPECTED_EOF, "unexpected end of file");
  if (n_out != n_elements) return set_error(IFX_E_INVALID_TENSOR_INDEX, "tensor index out of bounds: %llu", (unsigned long long)n_out);
  if (!dequant_supported(type)) return set_error(IFX_E_UNKNOWN_TENSOR_TYPE, "unknown tensor type id: %u", type);
  uint64_t be = 1, bb;
  if (type != T_F32 && type != T_F16) block_layout(type, &be, &bb);
  if (n_elements % be) return set_error(IFX_E_INVALID_ARG, "%llu elements is not a whole number of blocks", (unsigned long long)n_elements);
  if (n_elements == 0) return IFX_OK;
  IFX_HIP(launch_dequant_raw(type, (const uint8_t*)bytes, n_elements, out, stream_of(stream)));
  return IFX_OK;
}

int ifx_tensor_upload(uint32_t type, const void* host, uint64_t n_bytes, uint64_t rows, uint64_t cols,
                      ifx_tensor** out) {
  clear_error();
  IFX_TRY(device_init());
  if (!out || (!host && n_bytes)) return set_error(IFX_E_INVALID_ARG, "null argument");
  return upload_matrix(type, (const uint8_t*)host, n_bytes, rows, cols, out, 0);
}

int ifx_tensor_upload_ex(uint32_t type, const void* host, uint64_t n_bytes, uint64_t rows, uint64_t cols,
                         uint32_t flags, ifx_tensor** out) {
  clear_error();
  IFX_TRY(device_init());
  if (!out || (!host && n_bytes)) return set_error(IFX_E_INVALID_ARG, "null argument");
  if (flags & ~(uint32_t)IFX_OPEN_GGML_KQUANTS) return set_error(IFX_E_INVALID_ARG, "unknown flags %#x", flags);
  return upload_matrix(type, (const uint8_t*)host, n_bytes, rows, cols, out, flags);
}

void ifx_tensor_free(ifx_tensor* t) {
  if (!t) return;
  if (t->alloc) (void)hipFree(t->alloc);
  delete t;
}

int ifx_tensor_bytes(const ifx_tensor* t, uint64_t* dev, uint64_t* gguf) {
  if (!t) return set_error(IFX_E_INVALID_ARG, "null tensor");
  if (dev) *dev = t->L.body_bytes + t->L.scal_bytes;
  if (gguf) *gguf = t->L.gguf_bytes;
  return IFX_OK;
}

int ifx_tensor_dequant(const ifx_tensor* t, float* out, void* stream) {
  IFX_TRY(device_init());
  if (!t || !out) return set_error(IFX_E_INVALID_ARG, "null argument");
  IFX_HIP(launch_dequant_dev(devw(t), t->L.rows * t->L.cols, out, stream_of(stream)));
  return IFX_OK;
}

int ifx_gemv(const ifx_tensor* w, const float* x, float* y, void* stream) {
  IFX_TRY(device_init());
  if (!w || !x || !y) return set_error(IFX_E_INVALID_ARG, "null argument");
  GemvLaunch L;
  L.seg[0] = gemv_seg(w->L);
  L.nseg = 1;
  L.cols = (uint32_t)w->L.cols;
  L.x = x;
  IFX_HIP(gemv_store(L, y, stream_of(stream)));
  return IFX_OK;
}

int ifx_matmul_qt(const float* a, uint64_t m, const ifx_tensor* w, float* c, void* stream) {
  IFX_TRY(device_init());
  if (!w || (m && (!a || !c))) return set_error(IFX_E_INVALID_ARG, "null argument");
  // two rows or more: the prefill GEMM (fp16 matrix cores, hi/lo activation
  // pairs) for the matrices it takes; the GEMV row by row otherwise
  if (m >= 2 && m <= 0xffffffffull && w->L.cols <= 0xffffffffull && gemm_type(w->L.type) && gemm_layout_ok(w->L)) {
    hipStream_t st = stream_of(stream);
    const uint64_t k = w->L.cols;
    const uint64_t part_bytes = 64ull << 20;  // split-K partial tiles of short inputs
    // one allocation: hi, lo planes, group sums, row exponents, partial tiles
    const uint64_t bh = (m * k * 2 + 255) & ~255ull, bg = (m * (k / 256 + 1) * 32 + 255) & ~255ull,
                   br = (m * 4 + 255) & ~255ull;
    uint8_t* buf = nullptr;
    IFX_HIP(hipMallocAsync((void**)&buf, 2 * bh + bg + br + part_bytes, st));
    const GemmIn in{(const uint16_t*)buf, (const uint16_t*)(buf + bh), (const uint16_t*)(buf + 2 * bh),
                    (const int*)(buf + 2 * bh + bg), (uint32_t)m, (uint32_t)k, (float*)(buf + 2 * bh + bg + br),
                    part_bytes};
    hipError_t e = launch_prep_rows(a, (uint32_t)m, (uint32_t)k, (uint32_t)k, nullptr, 0.f, in, st);
    if (e == hipSuccess) {
      const GemmW gw = gemm_w(w->L);
      e = gemm_store(in, gw, c, (uint32_t)w->L.rows, st);
    }
    const hipError_t ef = hipFreeAsync(buf, st);
    IFX_HIP(e);
    IFX_HIP(ef);
    return IFX_OK;
  }
  for (uint64_t i = 0; i < m; i++) {
    GemvLaunch L;
    L.seg[0] = gemv_seg(w->L);
    L.nseg = 1;
    L.cols = (uint32_t)w->L.cols;
    L.x = a + i * w->L.cols;
    IFX_HIP(gemv_store(L, c + i * w->L.rows, stream_of(stream)));
  }
  return IFX_OK;
}

int ifx_ops_matmul_t(const float* a, const float* b, float* c, uint64_t m, uint64_t n, uint64_t k,
                     void* stream) {
  IFX_TRY(device_init());
  IFX_HIP(launch_matmul_t_f32(a, b, c, m, n, k, stream_of(stream)));
  return IFX_OK;
}

int ifx_ops_rms_norm_rows(float* x, const float* w, uint64_t n, uint64_t rows, float eps, void* stream) {
  IFX_TRY(device_init());
  IFX_HIP(launch_rms_norm_rows(x, w, n, rows, eps, stream_of(stream)));
  return IFX_OK;
}

int ifx_ops_swiglu(const float* g, const float* u, float* o, uint64_t n, void* stream) {
  IFX_TRY(device_init());
  IFX_HIP(launch_swiglu(g, u, o, n, stream_of(stream)));
  return IFX_OK;
}

int ifx_ops_add_in_place(float* o, const float* b, uint64_t n, void* stream) {
  IFX_TRY(device_init());
  IFX_HIP(launch_add(o, b, n, stream_of(stream)));
  return IFX_OK;
}

int ifx_ops_softmax_rows(float* x, uint64_t rows, uint64_t cols, void* stream) {
  IFX_TRY(device_init());
  IFX_HIP(launch_softmax_rows(x, rows, cols, stream_of(stream)));
  return IFX_OK;
}

int ifx_ops_rope(float* x, uint64_t seq, uint64_t heads, uint64_t hd, uint64_t rope_dim, float base,
                 uint64_t pos0, void* stream) {
  IFX_TRY(device_init());
  if (rope_dim > hd || (rope_dim & 1)) return set_error(IFX_E_INVALID_ARG, "rope_dim must be even and <= head_dim");
  if (seq * heads * (rope_dim / 2) == 0) return IFX_OK;
  IFX_HIP(launch_rope(x, seq, heads, hd, rope_dim, base, pos0, stream_of(stream)));
  return IFX_OK;
}

int ifx_ops_embedding_lookup(const ifx_tensor* table, const uint32_t* ids, uint64_t n_ids, float* out,
                             void* stream) {
  IFX_TRY(device_init());
  if (!table) return set_error(IFX_E_INVALID_ARG, "null table");
  IFX_HIP(launch_embed_rows(devw(table), ids, n_ids, out, stream_of(stream)));
  return IFX_OK;
}

int ifx_ops_argmax(const float* x, uint64_t n, uint32_t* out, int* status, void* stream) {
  IFX_TRY(device_init());
  IFX_HIP(launch_argmax(x, n, out, status, stream_of(stream)));
  return IFX_OK;
}

}  // extern "C"
