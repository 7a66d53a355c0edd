// dev_quant.h — device-side element decoding, bit-exact with the reference
// dequantizers (src/gguf/dequant.rs).  This translation unit family is compiled
// with -ffp-contract=off, so `a * b - c` stays two roundings as in Rust.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ifx_common.h"

namespace ifx {

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffffu));
}

__device__ __forceinline__ uint32_t ld_u8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t ld_u16_unaligned(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

// Q4_K 6-bit (scale, min) of group g from the 12 packed bytes s[0..12)
// (src/gguf/dequant.rs:141-149).
__device__ __forceinline__ void q4k_scale_min(const uint8_t* s, int g, uint32_t* sc, uint32_t* mn) {
  if (g < 4) {
    *sc = s[g] & 63u;
    *mn = s[g + 4] & 63u;
  } else {
    *sc = (s[g + 4] & 15u) | ((uint32_t)(s[g - 4] >> 6) << 4);
    *mn = (uint32_t)(s[g + 4] >> 4) | ((uint32_t)(s[g] >> 6) << 4);
  }
}

// Element e of a raw GGUF block stream of the given type.
__device__ __forceinline__ float raw_elem(uint32_t type, const uint8_t* p, uint64_t e) {
  switch (type) {
    case 0: {  // F32: little-endian copy
      const uint8_t* q = p + 4 * e;
      uint32_t u = (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
      return __uint_as_float(u);
    }
    case 1:  // F16
      return h2f(ld_u16_unaligned(p + 2 * e));
    case 2: {  // Q4_0 (dequant.rs:70-82)
      const uint8_t* blk = p + (e / 32) * 18;
      int j = (int)(e % 32);
      float delta = h2f(ld_u16_unaligned(blk));
      uint32_t byte = blk[2 + (j & 15)];
      int q = (int)(j < 16 ? (byte & 15u) : (byte >> 4)) - 8;
      return (float)q * delta;
    }
    case 7: {  // Q8_0 (dequant.rs:101-109)
      const uint8_t* blk = p + (e / 32) * 34;
      float delta = h2f(ld_u16_unaligned(blk));
      return (float)(int8_t)blk[2 + e % 32] * delta;
    }
    case 12: {  // Q4_K (dequant.rs:133-161)
      const uint8_t* blk = p + (e / 256) * 144;
      int j = (int)(e % 256), g = j / 32, l = j % 32;
      float d = h2f(ld_u16_unaligned(blk)), dmin = h2f(ld_u16_unaligned(blk + 2));
      uint32_t sc, mn;
      q4k_scale_min(blk + 4, g, &sc, &mn);
      float dall = d * (float)sc;
      float dm = dmin * (float)mn;
      uint32_t byte = blk[16 + 16 * g + l / 2];
      uint32_t q = (l & 1) ? (byte >> 4) : (byte & 15u);
      return dall * (float)q - dm;
    }
    case 14: {  // Q6_K (dequant.rs:182-197)
      const uint8_t* blk = p + (e / 256) * 210;
      int j = (int)(e % 256);
      float d = h2f(ld_u16_unaligned(blk));
      uint32_t qlb = blk[18 + j / 2];
      uint32_t lo = (j & 1) ? (qlb >> 4) : (qlb & 15u);
      uint32_t hi = (blk[146 + j / 4] >> (2 * (j % 4))) & 3u;
      int q = (int)(lo | (hi << 4));
      return d * (float)blk[2 + j / 16] * (float)(q - 32);
    }
    case 15: {  // Q8_K (dequant.rs:218-230)
      const uint8_t* blk = p + (e / 256) * 292;
      int j = (int)(e % 256);
      float d = h2f(ld_u16_unaligned(blk)), dmin = h2f(ld_u16_unaligned(blk + 2));
      return d * (float)blk[4 + j / 8] * (float)(int8_t)blk[36 + j] - dmin;
    }
    default:
      return 0.0f;
  }
}

struct DevW {
  uint32_t type;
  uint64_t cols;
  const uint8_t* body;
  const uint8_t* scal;
  uint32_t q6_signed;  // Q6_K: int8 scale bytes (ggml's), else u8 (the reference's)
  uint64_t tstride, bstride;  // Q4_K / Q6_K: unit (t, b) at body + t tstride + b bstride (tile_strides)
};

// Element e (row-major flat index) of a matrix in the device layout; same
// arithmetic as raw_elem, so bit-exact with the reference.
__device__ __forceinline__ float dev_elem(const DevW& w, uint64_t e) {
  switch (w.type) {
    case 0: return ((const float*)w.body)[e];
    case 1: return h2f(((const uint16_t*)w.body)[e]);
    case 2: {
      uint64_t b = e / 32;
      int j = (int)(e % 32);
      float delta = h2f(((const uint16_t*)w.scal)[b]);
      uint32_t byte = w.body[b * 16 + (j & 15)];
      int q = (int)(j < 16 ? (byte & 15u) : (byte >> 4)) - 8;
      return (float)q * delta;
    }
    case 7: {
      uint64_t b = e / 32;
      float delta = h2f(((const uint16_t*)w.scal)[b]);
      return (float)(int8_t)w.body[b * 32 + e % 32] * delta;
    }
    case 12: {  // tiled Q4_K (ifx_common.h): same arithmetic as raw_elem
      const uint64_t row = e / w.cols, col = e % w.cols;
      const uint8_t* u = w.body + (row >> 4) * w.tstride + (col >> 8) * w.bstride;
      const int n = (int)(row & 15), j = (int)(col & 255), g = j / 32, l = j % 32;
      const uint8_t* h = u + 16 * n;
      float d = h2f(ld_u16_unaligned(h)), dmin = h2f(ld_u16_unaligned(h + 2));
      uint32_t sc, mn;
      q4k_scale_min(h + 4, g, &sc, &mn);
      float dall = d * (float)sc;
      float dm = dmin * (float)mn;
      uint32_t byte = u[256 + (g >> 2) * 1024 + (n + 16 * (g & 3)) * 16 + l / 2];
      uint32_t q = (l & 1) ? (byte >> 4) : (byte & 15u);
      return dall * (float)q - dm;
    }
    case 14: {  // tiled Q6_K
      const uint64_t row = e / w.cols, col = e % w.cols;
      const uint8_t* u = w.body + (row >> 4) * w.tstride + (col >> 8) * w.bstride;
      const int n = (int)(row & 15), j = (int)(col & 255), s = j / 32, k = j & 15;
      const int lane = n + 16 * (s & 3), c = 2 * (s >> 2) + ((j >> 4) & 1);
      uint32_t qlb = u[(s >> 2) * 1024 + lane * 16 + ((j >> 1) & 15)];
      uint32_t lo = (j & 1) ? (qlb >> 4) : (qlb & 15u);
      const uint8_t* hw = u + 2048 + lane * 16 + 4 * c;
      uint32_t word = (uint32_t)hw[0] | ((uint32_t)hw[1] << 8) | ((uint32_t)hw[2] << 16) | ((uint32_t)hw[3] << 24);
      uint32_t hi = (word >> (8 * ((k & 7) >> 1) + 2 * (k & 1) + 4 * (k >> 3))) & 3u;
      int q = (int)(lo | (hi << 4));
      float d = h2f(ld_u16_unaligned(u + 3328 + 2 * n));
      const uint32_t sb = u[3072 + 4 * lane + c];
      const float sc = w.q6_signed ? (float)(int8_t)sb : (float)sb;
      return d * sc * (float)(q - 32);
    }
    case 15: {
      uint64_t b = e / 256;
      int j = (int)(e % 256);
      const uint8_t* blk = w.body + b * 288;
      const uint16_t* dd = (const uint16_t*)w.scal + 2 * b;
      float d = h2f(dd[0]), dmin = h2f(dd[1]);
      return d * (float)blk[j / 8] * (float)(int8_t)blk[32 + j] - dmin;
    }
    default:
      return 0.0f;
  }
}

}  // namespace ifx
