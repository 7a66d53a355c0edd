// host_types.cpp — GGML type table, error plumbing and the host-side repack of
// GGUF blocks into the device layout described in ifx_common.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "ifx_common.h"

namespace ifx {

static thread_local std::string g_err;

int set_error(int status, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return status;
}
const char* last_error() { return g_err.c_str(); }
void clear_error() { g_err.clear(); }

// TensorType::from_u32 (src/gguf/types.rs:110-143): ids 0-3, 5-8, 10-30.
bool type_known(uint32_t t) { return t <= 3 || (t >= 5 && t <= 8) || (t >= 10 && t <= 30); }

// TensorType::element_size (src/gguf/types.rs:181-192).
uint64_t element_size(uint32_t t) {
  switch (t) {
    case 0: return 4; case 1: return 2; case 16: return 1; case 17: return 2;
    case 18: return 4; case 19: return 8; case 20: return 8; default: return 0;
  }
}

// TensorType::block_layout (src/gguf/types.rs:197-229).
bool block_layout(uint32_t t, uint64_t* e, uint64_t* b) {
  struct Row { uint32_t t, e, b; };
  static const Row tab[] = {{2, 32, 18},    {3, 32, 20},    {5, 32, 22},    {6, 32, 24},
                            {7, 32, 34},    {8, 32, 36},    {29, 32, 18},   {10, 256, 96},
                            {11, 256, 110}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210},
                            {15, 256, 292}, {21, 256, 166}, {22, 256, 184}, {23, 256, 66},
                            {24, 256, 104}, {25, 256, 176}, {26, 256, 98},  {27, 256, 166},
                            {28, 256, 136}, {30, 256, 116}};
  for (const Row& r : tab)
    if (r.t == t) { *e = r.e; *b = r.b; return true; }
  return false;
}

// TensorInfo::byte_size (src/gguf/tensor.rs:30-40).
bool byte_size(uint32_t t, uint64_t n, uint64_t* bytes) {
  uint64_t es = element_size(t), be, bb;
  if (es) { *bytes = n * es; return true; }
  if (block_layout(t, &be, &bb)) { *bytes = (n + be - 1) / be * bb; return true; }
  return false;
}

bool dequant_supported(uint32_t t) {
  return t == T_F32 || t == T_F16 || t == T_Q4_0 || t == T_Q8_0 || t == T_Q4K || t == T_Q6K ||
         t == T_Q8K;
}

const char* type_name(uint32_t t) {
  switch (t) {
    case 0: return "F32"; case 1: return "F16"; case 2: return "Q4_0"; case 7: return "Q8_0";
    case 12: return "Q4_K"; case 14: return "Q6_K"; case 15: return "Q8_K"; default: return "?";
  }
}

bool layout_sizes(uint32_t type, uint64_t rows, uint64_t cols, uint64_t* body, uint64_t* scal) {
  uint64_t n = rows * cols;
  switch (type) {
    case T_F32: *body = n * 4; *scal = 0; return true;
    case T_F16: *body = n * 2; *scal = 0; return true;
    case T_Q4_0: if (cols % 32) return false; *body = n / 32 * 16; *scal = n / 32 * 2; return true;
    case T_Q8_0: if (cols % 32) return false; *body = n / 32 * 32; *scal = n / 32 * 2; return true;
    case T_Q4K: if (cols % 256) return false; *body = n / 256 * 144; *scal = 0; return true;
    case T_Q6K: if (cols % 256) return false; *body = n / 256 * 208; *scal = n / 256 * 2; return true;
    case T_Q8K: if (cols % 256) return false; *body = n / 256 * 288; *scal = n / 256 * 4; return true;
    default: return false;
  }
}

// Spread the four nibbles of a 16-bit value into the low nibbles of four bytes.
static inline uint32_t spread_nibbles(uint32_t x) {
  x = (x | (x << 8)) & 0x00FF00FFu;
  return (x | (x << 4)) & 0x0F0F0F0Fu;
}

// Q6_K qh re-order for one 32-element group.  The original 64 bits hold element
// e at bits 2e..2e+1.  For each 16-element half the new 32-bit word holds the
// high bits of elements 0..7 in the high nibble of byte b (element 2b at bits
// 4-5, 2b+1 at 6-7) and of elements 8..15 in the low nibble (8+2b at 0-1,
// 8+2b+1 at 2-3), matching the even/odd nibble split of the two ql words.
static inline void q6_reorder_group(const uint8_t* qh8, uint8_t* out8) {
  uint64_t q;
  memcpy(&q, qh8, 8);
  for (int h = 0; h < 2; h++) {
    uint32_t s = (uint32_t)(q >> (32 * h));
    uint32_t w = (spread_nibbles(s & 0xFFFFu) << 4) | spread_nibbles(s >> 16);
    memcpy(out8 + 4 * h, &w, 4);
  }
}

void repack_to_device_layout(uint32_t type, const uint8_t* src, uint64_t nb, uint8_t* body,
                             uint8_t* scal) {
  switch (type) {
    case T_F32: memcpy(body, src, nb * 4); return;
    case T_F16: memcpy(body, src, nb * 2); return;
    case T_Q4K: memcpy(body, src, nb * 144); return;
    case T_Q4_0:
      for (uint64_t b = 0; b < nb; b++) {
        memcpy(scal + 2 * b, src + 18 * b, 2);
        memcpy(body + 16 * b, src + 18 * b + 2, 16);
      }
      return;
    case T_Q8_0:
      for (uint64_t b = 0; b < nb; b++) {
        memcpy(scal + 2 * b, src + 34 * b, 2);
        memcpy(body + 32 * b, src + 34 * b + 2, 32);
      }
      return;
    case T_Q8K:
      for (uint64_t b = 0; b < nb; b++) {
        memcpy(scal + 4 * b, src + 292 * b, 4);
        memcpy(body + 288 * b, src + 292 * b + 4, 288);
      }
      return;
    case T_Q6K:
      for (uint64_t b = 0; b < nb; b++) {
        const uint8_t* s = src + 210 * b;
        uint8_t* o = body + 208 * b;
        memcpy(scal + 2 * b, s, 2);          // d
        memcpy(o, s + 18, 128);              // ql
        memcpy(o + 192, s + 2, 16);          // u8 scales
        for (int g = 0; g < 8; g++) q6_reorder_group(s + 146 + 8 * g, o + 128 + 8 * g);
      }
      return;
    default: return;
  }
}

}  // namespace ifx
