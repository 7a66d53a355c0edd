// host_types.cpp — GGML type table, error plumbing and the host-side repack of
// GGUF blocks into the device layout described in ifx_common.h.
#include <stdarg.h>
#include <stdio.h>
#include <math.h>
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

// TensorType::name (src/gguf/types.rs:146-178), indexed by the type id.
const char* type_name(uint32_t t) {
  static const char* names[31] = {"F32",    "F16",     "Q4_0",   "Q4_1",  "?",     "Q5_0",    "Q5_1",   "Q8_0",
                                  "Q8_1",   "?",       "Q2_K",   "Q3_K",  "Q4_K",  "Q5_K",    "Q6_K",   "Q8_K",
                                  "I8",     "I16",     "I32",    "I64",   "F64",   "IQ1_S",   "IQ1_M",  "IQ2_XXS",
                                  "IQ2_XS", "IQ2_S",   "IQ3_XXS", "IQ3_S", "IQ4_XS", "IQ4_NL", "IQ4_XSS"};
  return t < 31 ? names[t] : "?";
}

bool layout_sizes(uint32_t type, uint64_t rows, uint64_t cols, uint64_t* body, uint64_t* scal) {
  uint64_t n = rows * cols;
  const uint64_t tiled = (rows + kTileRows - 1) / kTileRows * kTileRows * (cols / 256);  // blocks incl. padding
  switch (type) {
    case T_F32: *body = n * 4; *scal = 0; return true;
    case T_F16: *body = n * 2; *scal = 0; return true;
    case T_Q4_0: if (cols % 32) return false; *body = n / 32 * 16; *scal = n / 32 * 2; return true;
    case T_Q8_0: if (cols % 32) return false; *body = n / 32 * 32; *scal = n / 32 * 2; return true;
    case T_Q4K: if (cols % 256) return false; *body = tiled * 144; *scal = 0; return true;
    case T_Q6K: if (cols % 256) return false; *body = tiled * 210; *scal = 0; return true;
    case T_Q8K: if (cols % 256) return false; *body = n / 256 * 288; *scal = n / 256 * 4; return true;
    default: return false;
  }
}

void repack_to_device_layout(uint32_t type, const uint8_t* src, uint64_t nb, uint8_t* body,
                             uint8_t* scal) {
  switch (type) {
    case T_F32: memcpy(body, src, nb * 4); return;
    case T_F16: memcpy(body, src, nb * 2); return;
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
    default: return;
  }
}

// Bit position, in a Q6_K lane word, of the 2-bit high part of element k
// (0..15) of a 16-element part: byte (k & 7) / 2, bits 2 (k & 1) + 4 (k >> 3).
static inline int q6_word_bitpos(int k) { return 8 * ((k & 7) >> 1) + 2 * (k & 1) + 4 * (k >> 3); }

// One (tile, block) unit of the tiled K-quant layout; blk[n] is row n's GGUF
// block, or null for a padding row (zero bytes).
static void pack_unit(uint32_t type, const uint8_t* const* blk, uint8_t* u) {
  if (type == T_Q4K) {
    memset(u, 0, kUnitQ4K);
    for (uint64_t n = 0; n < kTileRows; n++) {
      if (!blk[n]) continue;
      memcpy(u + 16 * n, blk[n], 16);  // d, dmin, 12 scale bytes
      for (int q = 0; q < 2; q++)
        for (int g = 0; g < 4; g++)    // lane n + 16g: the 16 qs bytes of sub-block g + 4q
          memcpy(u + 256 + 1024 * q + 16 * (n + 16 * g), blk[n] + 16 + 16 * (g + 4 * q), 16);
    }
    return;
  }
  // Q6_K, reference block: d @0, u8 scales @2, ql @18, qh @146 (src/gguf/dequant.rs:165-199)
  memset(u, 0, kUnitQ6K);
  for (uint64_t n = 0; n < kTileRows; n++) {
    const uint8_t* b = blk[n];
    if (!b) continue;
    memcpy(u + 3328 + 2 * n, b, 2);
    for (int g = 0; g < 4; g++) {
      const uint64_t lane = n + 16 * g;
      for (int q = 0; q < 2; q++) memcpy(u + 1024 * q + 16 * lane, b + 18 + 16 * (g + 4 * q), 16);
      for (int c = 0; c < 4; c++) {  // part c of the lane: sub-block g + 4 (c >> 1), half c & 1
        const int part = 2 * (g + 4 * (c >> 1)) + (c & 1);
        uint32_t w = 0;
        for (int k = 0; k < 16; k++) {
          const int e = 16 * part + k;
          const uint32_t hi = (b[146 + e / 4] >> (2 * (e % 4))) & 3u;
          w |= hi << q6_word_bitpos(k);
        }
        memcpy(u + 2048 + 16 * lane + 4 * c, &w, 4);
        u[3072 + 4 * lane + c] = b[2 + part];
      }
    }
  }
}

// ggml's blocks (llama.cpp ggml-quants.c dequantize_row_q4_K / _q6_K) as the
// reference's (src/gguf/dequant.rs:133-161, 182-197):
//   Q4_K: same header; ggml's element 64 i + l is the low nibble of qs[32 i + l]
//         (sub-block 2 i), element 64 i + 32 + l its high nibble (sub-block
//         2 i + 1); the reference's element 32 g + l is nibble l % 2 of
//         qs[16 g + l / 2].
//   Q6_K: ggml: ql[128], qh[64], int8 scales[16], d; element 128 h + 32 j + l
//         (j < 4, l < 32) has its low 4 bits in ql[64 h + l + 32 (j & 1)]
//         (low nibble for j < 2, high for j >= 2) and its high 2 bits at bit
//         2 j of qh[32 h + l]; its scale is scales[(128 h + 32 j + l) / 16].
//         The reference: d, scales, ql (element e: nibble e % 2 of byte e / 2),
//         qh (element e: bits 2 (e % 4) of byte e / 4); scales by e / 16.
void ggml_kquant_to_reference(uint32_t type, const uint8_t* in, uint64_t n_blocks, uint8_t* out) {
  for (uint64_t b = 0; b < n_blocks; b++) {
    if (type == T_Q4K) {
      const uint8_t* g = in + 144 * b;
      uint8_t* r = out + 144 * b;
      memcpy(r, g, 16);
      memset(r + 16, 0, 128);
      for (int sb = 0; sb < 8; sb++)
        for (int l = 0; l < 32; l++) {
          const uint8_t byte = g[16 + 32 * (sb / 2) + l];
          const uint8_t v = (sb & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15);
          r[16 + 16 * sb + l / 2] |= (uint8_t)(v << (4 * (l & 1)));
        }
    } else {
      const uint8_t* g = in + 210 * b;
      uint8_t* r = out + 210 * b;
      memset(r, 0, 210);
      memcpy(r, g + 208, 2);       // d
      memcpy(r + 2, g + 192, 16);  // the int8 scale bytes, unchanged
      for (int e = 0; e < 256; e++) {
        const int h = e / 128, j = (e % 128) / 32, l = e % 32;
        const uint8_t lb = g[64 * h + l + 32 * (j & 1)];
        const uint32_t lo = j < 2 ? (lb & 15u) : (uint32_t)(lb >> 4);
        const uint32_t hi = (g[128 + 32 * h + l] >> (2 * j)) & 3u;
        r[18 + e / 2] |= (uint8_t)(lo << (4 * (e & 1)));
        r[146 + e / 4] |= (uint8_t)(hi << (2 * (e & 3)));
      }
    }
  }
}

void repack_tiles(uint32_t type, const uint8_t* src, uint64_t rows, uint64_t cols, uint64_t t0, uint64_t t1,
                  uint8_t* body) {
  const uint64_t nbr = cols / 256, bb = type == T_Q4K ? 144 : 210, tiles = row_tiles(rows);
  const uint64_t unit = type == T_Q4K ? kUnitQ4K : kUnitQ6K;
  const uint8_t* blk[kTileRows];
  for (uint64_t t = t0; t < t1; t++)
    for (uint64_t b = 0; b < nbr; b++) {
      for (uint64_t n = 0; n < kTileRows; n++) {
        const uint64_t r = t * kTileRows + n;
        blk[n] = r < rows ? src + (r * nbr + b) * bb : nullptr;
      }
      pack_unit(type, blk, body + tile_unit(t, b, tiles) * unit);
    }
}

static float host_f16(const uint8_t* p) {
  const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
  const uint32_t e = (h >> 10) & 31u, f = h & 1023u;
  float v;
  if (e == 31) v = f ? NAN : INFINITY;
  else if (e == 0) v = ldexpf((float)f, -24);
  else v = ldexpf((float)(f | 1024u), (int)e - 25);
  return (h & 0x8000u) ? -v : v;
}

float block_dmin_max(const uint8_t* src, uint64_t b0, uint64_t b1) {
  float m = 0.f;
  for (uint64_t b = b0; b < b1; b++) {
    const float v = fabsf(host_f16(src + 144 * b + 2));
    if (v != v) return v;
    m = v > m ? v : m;
  }
  return m;
}

bool gemm_layout_ok(const DevLayout& L) {
  if (!(L.abs_bound <= 3.0e38f)) return false;  // a non-finite block scale
  switch (L.type) {
    case T_Q4K: return L.cols % 256 == 0 && L.dmin_max * 2016.f <= 65504.f;  // 63 * 32 * dmin
    case T_Q6K: return L.cols % 256 == 0 && L.abs_bound <= 32768.f;  // w = (d sc)(q - 32) as fp16 hi + lo
    case T_Q8_0:
    case T_Q4_0: return L.cols % 32 == 0;
    default: return false;
  }
}

float block_abs_bound(uint32_t type, const uint8_t* src, uint64_t b0, uint64_t b1) {
  float m = 0.f;
  for (uint64_t b = b0; b < b1; b++) {
    float v;
    switch (type) {
      case T_Q4K: v = fabsf(host_f16(src + 144 * b)) * 945.f + fabsf(host_f16(src + 144 * b + 2)) * 63.f; break;
      case T_Q6K: v = fabsf(host_f16(src + 210 * b)) * 8160.f; break;
      case T_Q8_0: v = fabsf(host_f16(src + 34 * b)) * 128.f; break;
      case T_Q4_0: v = fabsf(host_f16(src + 18 * b)) * 8.f; break;
      default: return INFINITY;
    }
    if (!(v <= 3.0e38f)) return INFINITY;
    m = v > m ? v : m;
  }
  return m;
}

}  // namespace ifx
