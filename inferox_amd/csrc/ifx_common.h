// ifx_common.h — shared definitions of the inferox HIP library (host + device).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/inferox.h"

namespace ifx {

// ---------------------------------------------------------------------------
// Errors: a per-thread message beside the int status of the C ABI.
// ---------------------------------------------------------------------------
int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
const char* last_error();
void clear_error();

#define IFX_HIP(call)                                                                   \
  do {                                                                                  \
    hipError_t e_ = (call);                                                             \
    if (e_ != hipSuccess)                                                               \
      return ::ifx::set_error(IFX_E_HIP, "%s failed: %s (%s:%d)", #call,                \
                              hipGetErrorString(e_), __FILE__, __LINE__);               \
  } while (0)

#define IFX_TRY(expr)            \
  do {                           \
    int s_ = (expr);             \
    if (s_ != IFX_OK) return s_; \
  } while (0)

// ---------------------------------------------------------------------------
// GGML tensor types (src/gguf/types.rs:70-229)
// ---------------------------------------------------------------------------
enum GgmlType : uint32_t {
  T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 7, T_Q4K = 12, T_Q6K = 14, T_Q8K = 15
};

bool type_known(uint32_t t);                                   // TensorType::from_u32
bool block_layout(uint32_t t, uint64_t* elems, uint64_t* bytes);  // TensorType::block_layout
uint64_t element_size(uint32_t t);                             // TensorType::element_size
bool byte_size(uint32_t t, uint64_t n_elements, uint64_t* bytes); // TensorInfo::byte_size
bool dequant_supported(uint32_t t);  // the types dequantize_f32 accepts (src/gguf/dequant.rs:21-30)
const char* type_name(uint32_t t);

// ---------------------------------------------------------------------------
// Device weight layout of a [rows x cols] matrix (cols contiguous), as read by
// the GEMV / embedding / device-dequant kernels.  Same bits as the GGUF blocks;
// only the placement of block fields changes, so the bytes streamed per row
// equal the GGUF bytes.
//   F32, F16 : row-major elements.
//   Q4_K     : GGUF blocks unchanged (144 B = 9 x 16 B, rows are whole blocks).
//   Q4_0     : qs[nb][16] | d[nb] (f16).
//   Q8_0     : qs[nb][32] | d[nb] (f16).
//   Q6_K     : body[nb][208] = ql[128] | qh'[64] | sc[16]  and  d[nb] (f16).
//              qh' holds the same 2-bit high parts, re-ordered per 16 elements
//              so that a 32-bit word lines up with the nibble split of ql.
//   Q8_K     : body[nb][288] = sc[32] | qs[256]  and  dd[nb] = {d, dmin} (f16 x 2).
// ---------------------------------------------------------------------------
struct DevLayout {
  uint32_t type = 0;
  uint64_t rows = 0, cols = 0;
  uint64_t n_blocks = 0;      // blocks (or elements for F32/F16) in the matrix
  uint64_t blocks_per_row = 0;
  uint8_t* body = nullptr;    // device: main array
  uint8_t* scal = nullptr;    // device: scale array (Q4_0/Q8_0/Q6_K/Q8_K), else null
  uint64_t body_bytes = 0, scal_bytes = 0;
  uint64_t gguf_bytes = 0;    // stored GGUF bytes of the same matrix
};

// Host-side repack of one matrix from GGUF block bytes into the device layout
// (dst_body/dst_scal sized by layout_sizes).
bool layout_sizes(uint32_t type, uint64_t rows, uint64_t cols, uint64_t* body, uint64_t* scal);
void repack_to_device_layout(uint32_t type, const uint8_t* src, uint64_t n_blocks, uint8_t* body,
                             uint8_t* scal);

}  // namespace ifx

struct ifx_tensor {
  ifx::DevLayout L;
  void* alloc = nullptr;  // one device allocation holding body and scal
};
