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

// a * b when it fits in 64 bits (sizes taken from a file are multiplied with this)
inline bool mul_u64(uint64_t a, uint64_t b, uint64_t* out) { return !__builtin_mul_overflow(a, b, out); }

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
// the GEMV / embedding / device-dequant kernels.  The same bits as the GGUF
// blocks, placed for the kernel that streams them.
//   F32, F16 : row-major elements.
//   Q4_0     : qs[nb][16] | d[nb] (f16).
//   Q8_0     : qs[nb][32] | d[nb] (f16).
//   Q8_K     : body[nb][288] = sc[32] | qs[256]  and  dd[nb] = {d, dmin} (f16 x 2).
//   Q4_K, Q6_K (tiled, for the int8-MFMA GEMV): rows are grouped in tiles of
//     16 (the last tile padded with zero blocks); unit (t, b) holds block b of
//     rows 16t..16t+15 at unit tile_unit(t, b, tiles), block-major: the
//     units of block b of all tiles are consecutive (the kernels take the
//     byte strides of tile_strides).  The GEMV, K-split GEMV and GEMM
//     launches read a block of many tiles at a time, so the whole GPU streams
//     one contiguous region (a 48 MB Q6_K stream with nontemporal loads:
//     7.3 us, against 9.2 us when each wave streams the units of its own tile
//     in a tile-major order).  Lane L = n + 16g
//     (row n, group g = 0..3) owns sub-blocks g and g + 4 (32 elements each)
//     of row n; its bytes sit where one 16-byte load per lane fetches them.
//     Q4_K unit (2304 B = 16 x 144):
//       [0, 256)      row n: d, dmin, 12 scale bytes (the block's first 16 B)
//       [256, 2304)   [q = 0, 1][lane L][16]: the qs bytes of sub-block g + 4q
//     Q6_K unit (3360 B = 16 x 210):
//       [0, 2048)     [q][lane L][16]: the ql bytes of sub-block g + 4q
//       [2048, 3072)  [lane L][c = 0..3]: 32-bit word of the 2-bit high parts
//                     of part c (sub-block g + 4 (c >> 1), half c & 1): element
//                     k of the part at byte (k & 7) / 2, bits 2 (k & 1) + 4 (k >> 3)
//       [3072, 3328)  [lane L][c]: the part's u8 scale
//       [3328, 3360)  row n: d (f16)
// ---------------------------------------------------------------------------
constexpr uint64_t kTileRows = 16;
constexpr uint64_t kUnitQ4K = 16 * 144, kUnitQ6K = 16 * 210;
__host__ __device__ inline uint64_t row_tiles(uint64_t rows) { return (rows + kTileRows - 1) / kTileRows; }
// unit index of (tile t, 256-column block b) in a matrix of `tiles` row tiles
__host__ __device__ inline uint64_t tile_unit(uint64_t t, uint64_t b, uint64_t tiles) { return b * tiles + t; }
// byte strides of a tile and of a block of a tiled Q4_K / Q6_K matrix: unit
// (t, b) at body + t tstride + b bstride
__host__ __device__ inline void tile_strides(uint32_t type, uint64_t rows, uint64_t* tstride, uint64_t* bstride) {
  const uint64_t unit = type == 12 ? kUnitQ4K : kUnitQ6K;
  *tstride = unit;
  *bstride = row_tiles(rows) * unit;
}

struct DevLayout {
  uint32_t type = 0;
  uint64_t rows = 0, cols = 0;
  uint64_t n_blocks = 0;      // blocks (or elements for F32/F16) in the matrix
  uint64_t blocks_per_row = 0;
  uint8_t* body = nullptr;    // device: main array
  uint8_t* scal = nullptr;    // device: scale array (Q4_0/Q8_0/Q6_K/Q8_K), else null
  uint64_t body_bytes = 0, scal_bytes = 0;
  uint64_t gguf_bytes = 0;    // stored GGUF bytes of the same matrix
  float abs_bound = 0.f;      // bound on |element| from the block scales (inf: unbounded or non-finite)
  float dmin_max = 0.f;       // Q4_K: largest |dmin| (NaN if any is NaN)
  uint32_t q6_signed = 0;     // Q6_K: scale bytes are int8 (ggml's layout), not the reference's u8
};

// ggml's K-quant blocks (llama.cpp ggml-common.h block_q4_K / block_q6_K)
// rewritten as the reference's blocks: Q4_K loses nothing (only the
// nibble-to-element order differs); Q6_K moves d first and re-places ql/qh
// in the reference's element order, keeping the int8 scale bytes as they are
// (the tensor is then read with q6_signed).  n_blocks blocks, in -> out.
void ggml_kquant_to_reference(uint32_t type, const uint8_t* in, uint64_t n_blocks, uint8_t* out);

// Host-side repack of one matrix from GGUF block bytes into the device layout
// (dst_body/dst_scal sized by layout_sizes); the block-wise types.
bool layout_sizes(uint32_t type, uint64_t rows, uint64_t cols, uint64_t* body, uint64_t* scal);
void repack_to_device_layout(uint32_t type, const uint8_t* src, uint64_t n_blocks, uint8_t* body,
                             uint8_t* scal);
// Q4_K / Q6_K: row tiles [t0, t1) of the tiled layout into body (the whole
// matrix's body; src is the whole matrix's GGUF bytes).
void repack_tiles(uint32_t type, const uint8_t* src, uint64_t rows, uint64_t cols, uint64_t t0, uint64_t t1,
                  uint8_t* body);
// Bound on |element| over GGUF blocks [b0, b1) of a quantized type, from the
// block scales alone (Q4_K: |d| 63 15 + |dmin| 63; Q6_K: |d| 255 32; Q8_0:
// |d| 128; Q4_0: |d| 8); +inf for F32/F16/Q8_K or a non-finite scale.
float block_abs_bound(uint32_t type, const uint8_t* src, uint64_t b0, uint64_t b1);
// Largest |dmin| over Q4_K blocks [b0, b1) (NaN if one is NaN).
float block_dmin_max(const uint8_t* src, uint64_t b0, uint64_t b1);
// The batched prefill GEMM carries this matrix exactly: finite block scales,
// whole blocks per row, and (Q4_K) -32 dmin mn or (Q6_K) the weights inside
// the fp16 range.
bool gemm_layout_ok(const DevLayout& L);

}  // namespace ifx

struct ifx_tensor {
  ifx::DevLayout L;
  void* alloc = nullptr;  // one device allocation holding body and scal
};
