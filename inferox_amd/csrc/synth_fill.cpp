// synth_fill.cpp — seeded payload generator for synthetic GGUF models.
//
// Fills the data bytes of one tensor in the reference's block layouts
// (src/gguf/dequant.rs: Q4_K at :113-163, Q6_K with d first and u8 scales at
// :165-199, Q8_0 at :86-111, Q4_0 at :54-84).  Every block draws from its own
// counter-based stream (splitmix64 of seed and block index), so the output does
// not depend on the thread count.  Host-only; built with g++ -fopenmp.
#include <stdint.h>
#include <string.h>
#include <math.h>

namespace {

inline uint64_t splitmix64(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

struct Rng {
  uint64_t s;
  Rng(uint64_t seed, uint64_t idx) : s(seed ^ (idx * 0xD1B54A32D192ED03ull)) { splitmix64(s); }
  uint64_t next() { return splitmix64(s); }
  double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }  // [0,1)
  double normal() {
    double u1 = uniform(), u2 = uniform();
    if (u1 < 1e-300) u1 = 1e-300;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
  }
  void bytes(uint8_t* p, size_t n) {
    while (n >= 8) { uint64_t v = next(); memcpy(p, &v, 8); p += 8; n -= 8; }
    if (n) { uint64_t v = next(); memcpy(p, &v, n); }
  }
};

// f32 -> f16 bits with round-to-nearest-even (IEEE binary16).
inline uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t e = (x >> 23) & 0xffu;
  uint32_t m = x & 0x7fffffu;
  if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
  int ee = (int)e - 127 + 15;
  if (ee >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (ee <= 0) {
    if (ee < -10) return (uint16_t)sign;
    m |= 0x800000u;
    uint32_t shift = (uint32_t)(14 - ee);
    uint32_t hm = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (hm & 1u))) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t hm = m >> 13, rem = m & 0x1fffu;
  uint32_t h = sign | ((uint32_t)ee << 10) | hm;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h++;
  return (uint16_t)h;
}

inline void put_f16(uint8_t* p, double v) {
  uint16_t h = f32_to_f16((float)v);
  p[0] = (uint8_t)(h & 0xff);
  p[1] = (uint8_t)(h >> 8);
}

}  // namespace

extern "C" {

uint16_t ifx_synth_f32_to_f16(float f) { return f32_to_f16(f); }

// Fill `dst` with a tensor of `n_elements` of ggml `type`.
// Parameters by type:
//   F32 / F16 : normal(p0, p1)
//   Q8_0      : delta f16 ~ U[p0,p1], quants i8 ~ U[-127,127]
//   Q4_0      : delta f16 ~ U[p0,p1], 16 uniform nibble bytes
//   Q4_K      : d f16 ~ U[p0,p1], dmin f16 ~ U[p2,p3], 12 uniform scale bytes, 128 uniform qs
//   Q6_K      : d f16 ~ U[p0,p1] at byte 0, scales i8 ~ U[-32,31] at 2..18, ql 18..146, qh 146..210 uniform
// Returns 0, or -1 for an unsupported type / partial block.
int ifx_synth_fill(uint8_t* dst, uint32_t type, uint64_t n_elements, uint64_t seed, double p0,
                   double p1, double p2, double p3) {
  if (type == 0 || type == 1) {
    const uint64_t chunk = 256;
    uint64_t nchunks = (n_elements + chunk - 1) / chunk;
#pragma omp parallel for schedule(static)
    for (uint64_t c = 0; c < nchunks; c++) {
      Rng r(seed, c);
      uint64_t e1 = (c + 1) * chunk < n_elements ? (c + 1) * chunk : n_elements;
      for (uint64_t e = c * chunk; e < e1; e++) {
        float v = (float)(p0 + p1 * r.normal());
        if (type == 0) memcpy(dst + 4 * e, &v, 4);
        else put_f16(dst + 2 * e, v);
      }
    }
    return 0;
  }
  uint64_t be, bb;
  switch (type) {
    case 2: be = 32; bb = 18; break;
    case 7: be = 32; bb = 34; break;
    case 12: be = 256; bb = 144; break;
    case 14: be = 256; bb = 210; break;
    default: return -1;
  }
  if (n_elements % be) return -1;
  uint64_t nb = n_elements / be;
#pragma omp parallel for schedule(static, 4096)
  for (uint64_t b = 0; b < nb; b++) {
    Rng r(seed, b);
    uint8_t* blk = dst + b * bb;
    switch (type) {
      case 2:
        put_f16(blk, p0 + (p1 - p0) * r.uniform());
        r.bytes(blk + 2, 16);
        break;
      case 7:
        put_f16(blk, p0 + (p1 - p0) * r.uniform());
        for (int j = 0; j < 32; j++) blk[2 + j] = (uint8_t)(int8_t)((int)(r.next() % 255u) - 127);
        break;
      case 12:
        put_f16(blk, p0 + (p1 - p0) * r.uniform());
        put_f16(blk + 2, p2 + (p3 - p2) * r.uniform());
        r.bytes(blk + 4, 140);
        break;
      case 14:
        put_f16(blk, p0 + (p1 - p0) * r.uniform());
        for (int j = 0; j < 16; j++) blk[2 + j] = (uint8_t)(int8_t)((int)(r.next() % 64u) - 32);
        r.bytes(blk + 18, 192);
        break;
    }
  }
  return 0;
}

// Zero-mean K-quant blocks (test models whose attention carries weight in
// the logits; the benchmark models keep the uniform bytes above).
//   Q4_K : d f16 ~ U[p0,p1]; per 32-element group a 6-bit scale sc ~ U{0..63}
//          and min mn = sc, dmin = f16(7.5 d): w = (d sc) q - (dmin sc),
//          about d sc (q - 7.5), q uniform nibbles.  The 12 scale bytes are
//          packed as the reference unpacks them (src/gguf/dequant.rs:139-152).
//   Q6_K : d f16 ~ U[p0,p1] at byte 0, u8 scales ~ U{1..p2} (p2 <= 127),
//          uniform ql/qh: w = (d sc)(q - 32), mean -d sc / 2.
// Other types as ifx_synth_fill.  Returns 0, or -1 as ifx_synth_fill.
int ifx_synth_fill_centred(uint8_t* dst, uint32_t type, uint64_t n_elements, uint64_t seed, double p0, double p1,
                           double p2) {
  if (type != 12 && type != 14) return ifx_synth_fill(dst, type, n_elements, seed, p0, p1, p2, 0.0);
  if (n_elements % 256) return -1;
  const uint64_t nb = n_elements / 256, bb = type == 12 ? 144 : 210;
  const int sc_hi = p2 < 1.0 ? 1 : (p2 > 127.0 ? 127 : (int)p2);
#pragma omp parallel for schedule(static, 4096)
  for (uint64_t b = 0; b < nb; b++) {
    Rng r(seed, b);
    uint8_t* blk = dst + b * bb;
    const uint16_t dh = f32_to_f16((float)(p0 + (p1 - p0) * r.uniform()));
    blk[0] = (uint8_t)(dh & 0xff);
    blk[1] = (uint8_t)(dh >> 8);
    if (type == 12) {
      // the f16 value of d, widened (normal range: p0 >= 6.2e-5)
      uint32_t e = (dh >> 10) & 31u, m = dh & 1023u;
      float d = e ? ldexpf((float)(1024u + m), (int)e - 25) : ldexpf((float)m, -24);
      put_f16(blk + 2, 7.5 * (double)d);
      uint8_t sc[8];
      for (int g = 0; g < 8; g++) sc[g] = (uint8_t)(r.next() % 64u);
      uint8_t* s = blk + 4;
      for (int g = 0; g < 4; g++) {
        s[g] = (uint8_t)((sc[g] & 63u) | ((sc[g + 4] >> 4) << 6));      // sc_g, top bits of sc_{g+4}
        s[g + 4] = (uint8_t)((sc[g] & 63u) | ((sc[g + 4] >> 4) << 6));  // mn_g = sc_g, top bits of mn_{g+4}
        s[g + 8] = (uint8_t)((sc[g + 4] & 15u) | ((sc[g + 4] & 15u) << 4));
      }
      r.bytes(blk + 16, 128);
    } else {
      for (int j = 0; j < 16; j++) blk[2 + j] = (uint8_t)(1 + r.next() % (uint64_t)sc_hi);
      r.bytes(blk + 18, 192);
    }
  }
  return 0;
}

// Seeded uniform token ids in [0, vocab).
void ifx_synth_token_ids(uint32_t* out, uint64_t n, uint32_t vocab, uint64_t seed) {
  Rng r(seed, 0x70ull);
  for (uint64_t i = 0; i < n; i++) out[i] = (uint32_t)(r.next() % vocab);
}

// Seeded N(mean, std) f32 values (KV fills).
void ifx_synth_normal_f32(float* out, uint64_t n, uint64_t seed, float mean, float std) {
  const uint64_t chunk = 4096;
  uint64_t nchunks = (n + chunk - 1) / chunk;
#pragma omp parallel for schedule(static)
  for (uint64_t c = 0; c < nchunks; c++) {
    Rng r(seed, c);
    uint64_t e1 = (c + 1) * chunk < n ? (c + 1) * chunk : n;
    for (uint64_t e = c * chunk; e < e1; e++) out[e] = (float)(mean + std * r.normal());
  }
}

}  // extern "C"
