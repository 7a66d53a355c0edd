/*
 * oracle.c — CPU restatement of the inferox reference token loop.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never the product.
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.
 *
 * Build: oracle/Makefile (gcc -O2 -mavx2 -mfma -ffp-contract=off -fopenmp).
 * -ffp-contract=off matters: the reference (Rust) never fuses a*b+c, so every
 * scalar multiply and add below is one IEEE single rounding.  The only fused
 * operations are the explicit 8-lane FMAs of matmul_t, as in the reference.
 *
 * Citations are path:line in the reference tree (phraakture/inferox).
 *
 * How each part is pinned (tests/test_oracle_kats.py, test_oracle_crosscheck.py):
 *   dequant, every type   reference KATs (src/gguf/dequant.rs:248-392) + an
 *                         independent numpy restatement, bit-equal on random and
 *                         edge blocks (every 6-bit Q4_K scale/min value, Q6_K
 *                         unsigned scales, all 65536 f16 values)
 *   matmul_t              reference KATs (src/ops.rs:293-346), float64 bound, a
 *                         lane-order vector that separates the hsum tree from a
 *                         sequential sum
 *   rms_norm, swiglu,     reference KATs (src/ops.rs:348-416), float64 within
 *   softmax, add, argmax  tolerance, closed forms (softmax rows sum to 1, last
 *                         index on ties, NaN -> error)
 *   rope                  identity at position 0 (the decode case), rotation by
 *                         the float64 angle elsewhere
 *   decode/prefill/       float64 brute force of a small model, invariants
 *   forward/generate      (prefill([t]) == decode(t), KV-row permutation), the
 *                         all-zero-weight generate KAT (src/model/forward.rs)
 * parity unpinned: the bit patterns of the libm-dependent values (expf in
 * silu/softmax, powf/sinf/cosf in rope) equal the reference's only if Rust std
 * and this glibc agree, which no reference test checks; they are pinned to
 * tolerance above.  The same holds for whole token streams of decode/generate.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <fcntl.h>
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ------------------------------------------------------------------------- */
/* GGML type ids and block layouts (src/gguf/types.rs:70-229)                */
/* ------------------------------------------------------------------------- */
enum {
  T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 5, T_Q5_1 = 6, T_Q8_0 = 7,
  T_Q8_1 = 8, T_Q2K = 10, T_Q3K = 11, T_Q4K = 12, T_Q5K = 13, T_Q6K = 14, T_Q8K = 15,
  T_I8 = 16, T_I16 = 17, T_I32 = 18, T_I64 = 19, T_F64 = 20
  /* 21..30: IQ types */
};

/* TensorType::from_u32 (src/gguf/types.rs:110-143): ids 0-3, 5-8 and 10-30 are known. */
static int type_known(uint32_t t) { return t <= 3 || (t >= 5 && t <= 8) || (t >= 10 && t <= 30); }

/* TensorType::element_size (src/gguf/types.rs:181-192). */
static uint64_t element_size(uint32_t t) {
  switch (t) {
    case T_F32: return 4; case T_F16: return 2; case T_I8: return 1; case T_I16: return 2;
    case T_I32: return 4; case T_I64: return 8; case T_F64: return 8; default: return 0;
  }
}

/* TensorType::block_layout (src/gguf/types.rs:197-229): {elements, bytes}. */
int orc_block_layout(uint32_t t, uint64_t* be, uint64_t* bb) {
  static const struct { uint32_t t, e, b; } tab[] = {
      {2, 32, 18},   {3, 32, 20},   {5, 32, 22},   {6, 32, 24},   {7, 32, 34},   {8, 32, 36},
      {29, 32, 18},  {10, 256, 96}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
      {14, 256, 210}, {15, 256, 292}, {21, 256, 166}, {22, 256, 184}, {23, 256, 66},
      {24, 256, 104}, {25, 256, 176}, {26, 256, 98}, {27, 256, 166}, {28, 256, 136},
      {30, 256, 116}};
  for (size_t i = 0; i < sizeof(tab) / sizeof(tab[0]); i++)
    if (tab[i].t == t) { *be = tab[i].e; *bb = tab[i].b; return ORC_OK; }
  return ORC_E_UNKNOWN_TENSOR_TYPE;
}

/* TensorInfo::byte_size (src/gguf/tensor.rs:30-40). */
int orc_byte_size(uint32_t t, uint64_t n, uint64_t* bytes) {
  uint64_t es = element_size(t), be, bb;
  if (es) { *bytes = n * es; return ORC_OK; }
  if (orc_block_layout(t, &be, &bb) == ORC_OK) { *bytes = ((n + be - 1) / be) * bb; return ORC_OK; }
  return ORC_E_UNKNOWN_TENSOR_TYPE;
}

/* ------------------------------------------------------------------------- */
/* f16 -> f32, exact (half 2.7.1 f16::to_f32, used at src/gguf/dequant.rs:49,71,...) */
/* NaNs keep their payload and come out quiet, as with F16C vcvtph2ps.        */
/* ------------------------------------------------------------------------- */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ffu, bits;
  if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13) | (man ? 0x00400000u : 0u);
  } else if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24, renormalise */
      int e = -1;
      do { man <<= 1; e++; } while (!(man & 0x400u));
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else {
    bits = sign | ((exp + (127 - 15)) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static inline float ld_f16(const uint8_t* p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ------------------------------------------------------------------------- */
/* Dequantizers: src/gguf/dequant.rs. Each works on whole blocks.             */
/* ------------------------------------------------------------------------- */

/* dequantize_q4_0 (src/gguf/dequant.rs:62-84): low nibble -> j, high -> j+16. */
static void dq_q4_0(const uint8_t* src, uint64_t nb, float* out) {
  for (uint64_t b = 0; b < nb; b++) {
    const uint8_t* blk = src + b * 18;
    float delta = ld_f16(blk);
    float* o = out + b * 32;
    for (int j = 0; j < 16; j++) {
      int q0 = (blk[2 + j] & 0x0f) - 8, q1 = (blk[2 + j] >> 4) - 8;
      o[j] = (float)q0 * delta;
      o[j + 16] = (float)q1 * delta;
    }
  }
}

/* dequantize_q8_0 (src/gguf/dequant.rs:93-111): y = f32(i8) * delta. */
static void dq_q8_0(const uint8_t* src, uint64_t nb, float* out) {
  for (uint64_t b = 0; b < nb; b++) {
    const uint8_t* blk = src + b * 34;
    float delta = ld_f16(blk);
    for (int j = 0; j < 32; j++) out[b * 32 + j] = (float)(int8_t)blk[2 + j] * delta;
  }
}

/* dequantize_q4_k (src/gguf/dequant.rs:123-163).  Group g owns qs[16g..16g+16];
 * element 32g+l is nibble (l&1) of qs[16g + l/2].  y = (d*sc)*q - (dmin*mn). */
static void dq_q4_k(const uint8_t* src, uint64_t nb, float* out) {
  for (uint64_t b = 0; b < nb; b++) {
    const uint8_t* blk = src + b * 144;
    float d = ld_f16(blk), dmin = ld_f16(blk + 2);
    const uint8_t* s = blk + 4;
    const uint8_t* qs = blk + 16;
    for (int g = 0; g < 8; g++) {
      uint32_t sc, mn;
      if (g < 4) {
        sc = s[g] & 63u;
        mn = s[g + 4] & 63u;
      } else {
        sc = (s[g + 4] & 15u) | ((uint32_t)(s[g - 4] >> 6) << 4);
        mn = (uint32_t)(s[g + 4] >> 4) | ((uint32_t)(s[g] >> 6) << 4);
      }
      float dall = d * (float)sc;
      float dm = dmin * (float)mn;
      for (int l = 0; l < 32; l++) {
        uint8_t byte = qs[16 * g + l / 2];
        uint32_t q = (l & 1) ? (byte >> 4) : (byte & 15u);
        out[b * 256 + 32 * g + l] = dall * (float)q - dm;
      }
    }
  }
}

/* dequantize_q6_k (src/gguf/dequant.rs:174-199).  d@0, u8 scales@2..18,
 * ql@18..146, qh@146..210;  y = (d * f32(u8 sc)) * f32(q - 32). */
static void dq_q6_k(const uint8_t* src, uint64_t nb, float* out) {
  for (uint64_t b = 0; b < nb; b++) {
    const uint8_t* blk = src + b * 210;
    float d = ld_f16(blk);
    const uint8_t *sc = blk + 2, *ql = blk + 18, *qh = blk + 146;
    for (int j = 0; j < 256; j++) {
      uint32_t lo = (j & 1) ? (ql[j / 2] >> 4) : (ql[j / 2] & 15u);
      uint32_t hi = (qh[j / 4] >> (2 * (j % 4))) & 3u;
      int q = (int)(lo | (hi << 4));
      out[b * 256 + j] = d * (float)sc[j / 16] * (float)(q - 32);
    }
  }
}

/* dequantize_q8_k (src/gguf/dequant.rs:210-232): y = ((d*sc[j/8])*f32(i8 q)) - dmin. */
static void dq_q8_k(const uint8_t* src, uint64_t nb, float* out) {
  for (uint64_t b = 0; b < nb; b++) {
    const uint8_t* blk = src + b * 292;
    float d = ld_f16(blk), dmin = ld_f16(blk + 2);
    const uint8_t *sc = blk + 4, *qs = blk + 36;
    for (int j = 0; j < 256; j++) out[b * 256 + j] = d * (float)sc[j / 8] * (float)(int8_t)qs[j] - dmin;
  }
}

/* dequantize_f32_f32 / dequantize_f16_f32 (src/gguf/dequant.rs:40-52). */
static void dq_f32(const uint8_t* src, uint64_t n, float* out) { memcpy(out, src, n * 4); }
static void dq_f16(const uint8_t* src, uint64_t n, float* out) {
  for (uint64_t i = 0; i < n; i++) out[i] = ld_f16(src + 2 * i);
}

/* Dequantize `nblk` whole units (blocks, or elements for F32/F16) starting at src. */
static int dq_units(uint32_t t, const uint8_t* src, uint64_t nunits, float* out) {
  switch (t) {
    case T_F32: dq_f32(src, nunits, out); return ORC_OK;
    case T_F16: dq_f16(src, nunits, out); return ORC_OK;
    case T_Q4_0: dq_q4_0(src, nunits, out); return ORC_OK;
    case T_Q8_0: dq_q8_0(src, nunits, out); return ORC_OK;
    case T_Q4K: dq_q4_k(src, nunits, out); return ORC_OK;
    case T_Q6K: dq_q6_k(src, nunits, out); return ORC_OK;
    case T_Q8K: dq_q8_k(src, nunits, out); return ORC_OK;
    default: return ORC_E_UNKNOWN_TENSOR_TYPE;
  }
}

/* elements and bytes of one dequant unit of a supported type */
static int unit_of(uint32_t t, uint64_t* ue, uint64_t* ub) {
  if (t == T_F32) { *ue = 1; *ub = 4; return ORC_OK; }
  if (t == T_F16) { *ue = 1; *ub = 2; return ORC_OK; }
  if (t == T_Q4_0 || t == T_Q8_0 || t == T_Q4K || t == T_Q6K || t == T_Q8K)
    return orc_block_layout(t, ue, ub);
  return ORC_E_UNKNOWN_TENSOR_TYPE;
}

/* dequantize_f32 (src/gguf/dequant.rs:10-31): same check order and errors.
 * A trailing partial block makes the reference index past `out` (a panic);
 * here that is ORC_E_INVALID_ARG. */
int orc_dequantize_f32(uint32_t t, uint64_t n_elements, const uint8_t* bytes, uint64_t n_bytes,
                       float* out, uint64_t n_out) {
  uint64_t expected;
  if (orc_byte_size(t, n_elements, &expected) != ORC_OK) return ORC_E_UNKNOWN_TENSOR_TYPE;
  if (n_bytes != expected) return ORC_E_UNEXPECTED_EOF;
  if (n_out != n_elements) return ORC_E_INVALID_TENSOR_INDEX;
  uint64_t ue, ub;
  if (unit_of(t, &ue, &ub) != ORC_OK) return ORC_E_UNKNOWN_TENSOR_TYPE;
  if (n_elements % ue) return ORC_E_INVALID_ARG;
  return dq_units(t, bytes, n_elements / ue, out);
}

/* Dequantize elements [e0, e0+n) of a flat tensor into out (row slice). */
static int dq_range(uint32_t t, const uint8_t* data, uint64_t e0, uint64_t n, float* out,
                    float* scratch) {
  uint64_t ue, ub;
  int rc = unit_of(t, &ue, &ub);
  if (rc) return rc;
  uint64_t u0 = e0 / ue, u1 = (e0 + n + ue - 1) / ue;
  if (u0 * ue == e0 && u1 * ue == e0 + n) return dq_units(t, data + u0 * ub, u1 - u0, out);
  rc = dq_units(t, data + u0 * ub, u1 - u0, scratch);
  memcpy(out, scratch + (e0 - u0 * ue), n * 4);
  return rc;
}

/* ------------------------------------------------------------------------- */
/* Ops: src/ops.rs                                                           */
/* ------------------------------------------------------------------------- */

/* Dot product in the order of matmul_t_avx2 (src/ops.rs:104-134): eight lane
 * accumulators, each a chain of exact FMAs over l = r, r+8, ...; then the
 * hsum256_ps tree (src/ops.rs:136-149) = (s0+s1)+(s2+s3) with s_r = acc_r + acc_{r+4};
 * then the scalar tail as sum = sum + (a*b). */
static inline float dot_ref(const float* a, const float* b, uint64_t k) {
  __m256 acc = _mm256_setzero_ps();
  uint64_t l = 0;
  for (; l + 8 <= k; l += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + l), _mm256_loadu_ps(b + l), acc);
  float lane[8];
  _mm256_storeu_ps(lane, acc);
  float s0 = lane[0] + lane[4], s1 = lane[1] + lane[5], s2 = lane[2] + lane[6], s3 = lane[3] + lane[7];
  float sum = (s0 + s1) + (s2 + s3);
  for (; l < k; l++) sum = sum + a[l] * b[l];
  return sum;
}

/* matmul_t (src/ops.rs:33-44) taking the AVX2+FMA path, as on any x86-64 host
 * with both features (the dispatch at src/ops.rs:38-43). */
void orc_matmul_t(const float* a, const float* b, float* c, uint64_t m, uint64_t n, uint64_t k) {
  for (uint64_t i = 0; i < m; i++)
    for (uint64_t j = 0; j < n; j++) c[i * n + j] = dot_ref(a + i * k, b + j * k, k);
}

/* matmul_t_scalar (src/ops.rs:61-71): the non-AVX2 fallback. */
void orc_matmul_t_scalar(const float* a, const float* b, float* c, uint64_t m, uint64_t n,
                         uint64_t k) {
  for (uint64_t i = 0; i < m; i++)
    for (uint64_t j = 0; j < n; j++) {
      float s = 0.0f;
      for (uint64_t l = 0; l < k; l++) s = s + a[i * k + l] * b[j * k + l];
      c[i * n + j] = s;
    }
}

/* rms_norm (src/ops.rs:155-168): sequential sum of squares, 1/sqrt, (x*scale)*w. */
void orc_rms_norm(float* x, const float* w, uint64_t n, float eps) {
  if (n == 0) return;
  float ss = -0.0f;
  for (uint64_t i = 0; i < n; i++) ss = ss + x[i] * x[i];
  float mean_sq = ss / (float)n;
  float scale = 1.0f / sqrtf(mean_sq + eps);
  for (uint64_t i = 0; i < n; i++) x[i] = x[i] * scale * w[i];
}

/* rms_norm_rows (src/ops.rs:173-180). */
void orc_rms_norm_rows(float* x, const float* w, uint64_t n, uint64_t rows, float eps) {
  for (uint64_t r = 0; r < rows; r++) orc_rms_norm(x + r * n, w, n, eps);
}

/* sigmoid / silu_scalar (src/ops.rs:199-209): clamp to +-80, 1/(1+exp(-x)). */
static inline float sigmoid_ref(float x) {
  float c = x;
  if (!(c != c)) { /* f32::clamp keeps NaN */
    if (c < -80.0f) c = -80.0f;
    if (c > 80.0f) c = 80.0f;
  }
  return 1.0f / (1.0f + expf(-c));
}
static inline float silu_ref(float x) { return x * sigmoid_ref(x); }

/* silu (src/ops.rs:183-187). */
void orc_silu(float* x, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) x[i] = silu_ref(x[i]);
}

/* swiglu (src/ops.rs:190-197): out = silu(g) * u. */
void orc_swiglu(const float* g, const float* u, float* out, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) out[i] = silu_ref(g[i]) * u[i];
}

/* add_in_place (src/ops.rs:212-217): out = out + b. */
void orc_add_in_place(float* out, const float* b, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) out[i] = out[i] + b[i];
}

/* f32::max (IEEE maxNum: a NaN operand yields the other operand). */
static inline float fmax_rust(float a, float b) {
  if (a != a) return b;
  if (b != b) return a;
  return a > b ? a : b;
}

/* softmax_rows (src/ops.rs:223-239): max fold from -inf, exp(v-max), sequential
 * sum, divide. */
void orc_softmax_rows(float* x, uint64_t rows, uint64_t cols) {
  for (uint64_t r = 0; r < rows; r++) {
    float* row = x + r * cols;
    float mx = -INFINITY;
    for (uint64_t c = 0; c < cols; c++) mx = fmax_rust(mx, row[c]);
    float sum = -0.0f;
    for (uint64_t c = 0; c < cols; c++) {
      row[c] = expf(row[c] - mx);
      sum = sum + row[c];
    }
    for (uint64_t c = 0; c < cols; c++) row[c] = row[c] / sum;
  }
}

/* embedding_lookup (src/ops.rs:246-258); an out-of-range id panics there. */
int orc_embedding_lookup(const float* emb, uint64_t vocab, const uint32_t* ids, uint64_t n_ids,
                         uint64_t hidden, float* out) {
  for (uint64_t p = 0; p < n_ids; p++) {
    if ((uint64_t)ids[p] >= vocab) return ORC_E_INVALID_ARG;
    memcpy(out + p * hidden, emb + (uint64_t)ids[p] * hidden, hidden * 4);
  }
  return ORC_OK;
}

/* rope (src/ops.rs:265-287): adjacent pairs (2i, 2i+1) of the first rope_dim
 * dims of each head; inv = 1/powf(base, i/rope_dim); angle = pos*inv.
 * The reference uses pos = 0..seq; pos0 shifts that for the ABSOLUTE mode. */
void orc_rope(float* x, uint64_t seq, uint64_t heads, uint64_t hd, uint64_t rope_dim, float base,
              uint64_t pos0) {
  for (uint64_t p = 0; p < seq; p++) {
    float pos = (float)(pos0 + p);
    for (uint64_t h = 0; h < heads; h++) {
      uint64_t off = (p * heads + h) * hd;
      for (uint64_t i = 0; i < rope_dim; i += 2) {
        float a = x[off + i], b = x[off + i + 1];
        float inv = 1.0f / powf(base, (float)i / (float)rope_dim);
        float ang = pos * inv;
        float sn = sinf(ang), cs = cosf(ang);
        x[off + i] = a * cs - b * sn;
        x[off + i + 1] = a * sn + b * cs;
      }
    }
  }
}

/* argmax (src/model/forward.rs:615-622, src/sampler.rs:75-82): Iterator::max_by
 * with partial_cmp: the LAST of equal maxima wins; any NaN compared panics
 * (here ORC_E_NAN_LOGIT); an empty slice gives 0. */
int orc_argmax(const float* x, uint64_t n, uint32_t* out) {
  *out = 0;
  if (n == 0) return ORC_OK;
  if (n == 1) return ORC_OK;
  for (uint64_t i = 0; i < n; i++)
    if (x[i] != x[i]) return ORC_E_NAN_LOGIT;
  uint64_t best = 0;
  for (uint64_t i = 1; i < n; i++)
    if (x[i] >= x[best]) best = i;
  *out = (uint32_t)best;
  return ORC_OK;
}

/* ------------------------------------------------------------------------- */
/* GGUF parsing: src/gguf/file.rs, tensor.rs, value.rs                        */
/* ------------------------------------------------------------------------- */
typedef struct {
  char* key;
  uint32_t type; /* ValueType id, src/gguf/types.rs:7-21 */
  union { uint64_t u; int64_t i; double f; } num;
  char* str;
} orc_meta;

typedef struct {
  char* name;
  uint32_t type;
  uint32_t n_dims;
  uint64_t shape[4];
  uint64_t offset;
} orc_tinfo;

typedef struct {
  int64_t attn_norm, attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down;
} orc_layer;

struct orc_model {
  uint8_t* map;
  size_t map_len;
  uint64_t n_meta, n_tensors;
  orc_meta* meta;
  orc_tinfo* tensors;
  uint64_t data_offset;
  orc_config cfg;
  orc_layer* layers;
  int64_t token_embd, output_norm, output; /* output = -1 when absent */
};

struct orc_kv {
  uint64_t n_layers, max_seq_len, kv_dim, len;
  float** k;
  float** v;
  int f16; /* rows rounded to binary16 as they are stored (the f16-KV session mode) */
};

/* x rounded to the nearest IEEE binary16 value (ties to even), returned as a
 * float: the grid spacing of x's binade, 2^(e - 11) for x = m 2^e with m in
 * [0.5, 1), no finer than the subnormal step 2^-24; rintf rounds half to even
 * in the default rounding mode; beyond the largest finite half (65504) the
 * result is infinite.  Not part of the reference (its cache is f32): the
 * emulation of the f16 cache mode. */
float orc_round_f16(float x) {
  if (!isfinite(x) || x == 0.0f) return x;
  int e;
  frexpf(x, &e);
  int q = e - 11;
  if (q < -24) q = -24;
  const float r = ldexpf(rintf(ldexpf(x, -q)), q);
  return fabsf(r) > 65504.0f ? copysignf(INFINITY, x) : r;
}

static void round_f16_n(float* p, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) p[i] = orc_round_f16(p[i]);
}

typedef struct {
  const uint8_t* p;
  size_t len, pos;
} rd_t;

static int rd_bytes(rd_t* r, void* dst, size_t n) {
  if (n > r->len - r->pos) return ORC_E_IO; /* read_exact on a short file: io::Error */
  memcpy(dst, r->p + r->pos, n);
  r->pos += n;
  return ORC_OK;
}
#define RD(r, var) rd_bytes((r), &(var), sizeof(var))

static int utf8_valid(const uint8_t* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    uint8_t c = s[i];
    size_t len;
    uint32_t cp;
    if (c < 0x80) { i++; continue; }
    if ((c & 0xe0) == 0xc0) { len = 2; cp = c & 0x1f; }
    else if ((c & 0xf0) == 0xe0) { len = 3; cp = c & 0x0f; }
    else if ((c & 0xf8) == 0xf0) { len = 4; cp = c & 0x07; }
    else return 0;
    if (i + len > n) return 0;
    for (size_t k = 1; k < len; k++) {
      if ((s[i + k] & 0xc0) != 0x80) return 0;
      cp = (cp << 6) | (s[i + k] & 0x3f);
    }
    if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
        cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff))
      return 0;
    i += len;
  }
  return 1;
}

/* read_string (src/gguf/value.rs:108-113): u64 length + UTF-8 bytes. */
static int rd_string(rd_t* r, char** out) {
  uint64_t n;
  int rc = RD(r, n);
  if (rc) return rc;
  if (n > r->len - r->pos) return ORC_E_IO;
  if (!utf8_valid(r->p + r->pos, n)) return ORC_E_INVALID_UTF8;
  char* s = (char*)malloc(n + 1);
  memcpy(s, r->p + r->pos, n);
  s[n] = 0;
  r->pos += n;
  *out = s;
  return ORC_OK;
}

/* Value::read (src/gguf/value.rs:45-71).  Scalars are kept for the typed getters;
 * arrays are parsed (recursively) and dropped. */
static int rd_value(rd_t* r, uint32_t ty, orc_meta* m) {
  int rc = ORC_OK;
  switch (ty) {
    case 0: { uint8_t v = 0; rc = RD(r, v); if (m) m->num.u = v; break; }
    case 1: { int8_t v = 0; rc = RD(r, v); if (m) m->num.i = v; break; }
    case 2: { uint16_t v = 0; rc = RD(r, v); if (m) m->num.u = v; break; }
    case 3: { int16_t v = 0; rc = RD(r, v); if (m) m->num.i = v; break; }
    case 4: { uint32_t v = 0; rc = RD(r, v); if (m) m->num.u = v; break; }
    case 5: { int32_t v = 0; rc = RD(r, v); if (m) m->num.i = v; break; }
    case 6: { float v = 0; rc = RD(r, v); if (m) m->num.f = v; break; }
    case 7: { uint8_t v = 0; rc = RD(r, v); if (m) m->num.u = v != 0; break; }
    case 8: { char* s = NULL; rc = rd_string(r, &s); if (m) m->str = s; else free(s); break; }
    case 9: {
      uint32_t it;
      uint64_t n;
      if ((rc = RD(r, it))) return rc;
      if (it > 12) return ORC_E_UNKNOWN_VALUE_TYPE;
      if ((rc = RD(r, n))) return rc;
      for (uint64_t i = 0; i < n && rc == ORC_OK; i++) rc = rd_value(r, it, NULL);
      break;
    }
    case 10: { uint64_t v = 0; rc = RD(r, v); if (m) m->num.u = v; break; }
    case 11: { int64_t v = 0; rc = RD(r, v); if (m) m->num.i = v; break; }
    case 12: { double v = 0; rc = RD(r, v); if (m) m->num.f = v; break; }
    default: return ORC_E_UNKNOWN_VALUE_TYPE;
  }
  return rc;
}

static const orc_meta* meta_get(const orc_model* m, const char* key) {
  for (uint64_t i = 0; i < m->n_meta; i++)
    if (strcmp(m->meta[i].key, key) == 0) return &m->meta[i];
  return NULL;
}

/* GgufFile::get_u32 / get_u64 / get_f32 (src/gguf/file.rs:142-186): integer
 * types cast with `as` (truncate / sign-extend), floats only for get_f32. */
static int meta_int(const orc_meta* e, int64_t* v) {
  if (!e) return 0;
  switch (e->type) {
    case 0: case 2: case 4: case 10: *v = (int64_t)e->num.u; return 1;
    case 1: case 3: case 5: case 11: *v = e->num.i; return 1;
    default: return 0;
  }
}
static int get_u32(const orc_model* m, const char* k, uint32_t* out) {
  int64_t v;
  if (!meta_int(meta_get(m, k), &v)) return 0;
  *out = (uint32_t)v;
  return 1;
}
static int get_u64(const orc_model* m, const char* k, uint64_t* out) {
  int64_t v;
  if (!meta_int(meta_get(m, k), &v)) return 0;
  *out = (uint64_t)v;
  return 1;
}
static int get_f32(const orc_model* m, const char* k, float* out) {
  const orc_meta* e = meta_get(m, k);
  if (!e) return 0;
  if (e->type == 6 || e->type == 12) { *out = (float)e->num.f; return 1; }
  if (e->type == 0 || e->type == 2 || e->type == 4 || e->type == 10) { *out = (float)e->num.u; return 1; }
  if (e->type == 1 || e->type == 3 || e->type == 5 || e->type == 11) { *out = (float)e->num.i; return 1; }
  return 0;
}

static int64_t tensor_index(const orc_model* m, const char* name) {
  for (uint64_t i = 0; i < m->n_tensors; i++)
    if (strcmp(m->tensors[i].name, name) == 0) return (int64_t)i;
  return -1;
}

static uint64_t t_nelem(const orc_tinfo* t) {
  uint64_t n = 1;
  for (uint32_t d = 0; d < t->n_dims; d++) n *= t->shape[d];
  return n;
}

/* Weights::tensor_bytes (src/gguf/weights.rs:97-112). */
static int tensor_bytes(const orc_model* m, int64_t idx, const uint8_t** data, uint64_t* n) {
  if (idx < 0 || (uint64_t)idx >= m->n_tensors) return ORC_E_INVALID_TENSOR_INDEX;
  const orc_tinfo* t = &m->tensors[idx];
  uint64_t size;
  if (orc_byte_size(t->type, t_nelem(t), &size)) return ORC_E_UNKNOWN_TENSOR_TYPE;
  uint64_t start = m->data_offset + t->offset;
  if (start < m->data_offset) return ORC_E_TENSOR_OFFSET_OVERFLOW;
  uint64_t end = start + size;
  if (end < start) return ORC_E_TENSOR_OFFSET_OVERFLOW;
  if (end > m->map_len) return ORC_E_UNEXPECTED_EOF;
  *data = m->map + start;
  *n = size;
  return ORC_OK;
}

int orc_model_tensor_bytes(const orc_model* m, uint64_t idx, const uint8_t** data, uint64_t* n) {
  return tensor_bytes(m, (int64_t)idx, data, n);
}

static void model_free(orc_model* m) {
  if (!m) return;
  for (uint64_t i = 0; i < m->n_meta; i++) { free(m->meta[i].key); free(m->meta[i].str); }
  for (uint64_t i = 0; i < m->n_tensors; i++) free(m->tensors[i].name);
  free(m->meta);
  free(m->tensors);
  free(m->layers);
  if (m->map) munmap(m->map, m->map_len);
  free(m);
}

void orc_model_close(orc_model* m) { model_free(m); }

/* GgufFile::read (src/gguf/file.rs:57-116) + Config::from_gguf
 * (src/model/config.rs:34-84) + Model::open (src/model/mod.rs:64-92). */
int orc_model_open(const char* path, orc_model** out) {
  *out = NULL;
  int fd = open(path, O_RDONLY);
  if (fd < 0) return ORC_E_IO;
  struct stat st;
  if (fstat(fd, &st) != 0) { close(fd); return ORC_E_IO; }
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  m->map_len = (size_t)st.st_size;
  if (m->map_len) {
    void* p = mmap(NULL, m->map_len, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) { close(fd); free(m); return ORC_E_IO; }
    m->map = (uint8_t*)p;
  }
  close(fd);
  rd_t r = {m->map, m->map_len, 0};
  int rc;
  uint8_t magic[4];
  uint32_t version;
  if ((rc = rd_bytes(&r, magic, 4))) goto fail;
  if (memcmp(magic, "GGUF", 4) != 0) { rc = ORC_E_INVALID_MAGIC; goto fail; }
  if ((rc = RD(&r, version))) goto fail;
  if (version != 2 && version != 3) { rc = ORC_E_UNSUPPORTED_VERSION; goto fail; }
  uint64_t n_tensors, n_kv;
  if ((rc = RD(&r, n_tensors)) || (rc = RD(&r, n_kv))) goto fail;
  if (n_kv > r.len || n_tensors > r.len) { rc = ORC_E_IO; goto fail; }
  m->meta = (orc_meta*)calloc(n_kv ? n_kv : 1, sizeof(orc_meta));
  for (uint64_t i = 0; i < n_kv; i++) {
    orc_meta* e = &m->meta[i];
    if ((rc = rd_string(&r, &e->key))) goto fail;
    m->n_meta = i + 1;
    if ((rc = RD(&r, e->type))) goto fail;
    if (e->type > 12) { rc = ORC_E_UNKNOWN_VALUE_TYPE; goto fail; }
    if ((rc = rd_value(&r, e->type, e))) goto fail;
  }
  m->tensors = (orc_tinfo*)calloc(n_tensors ? n_tensors : 1, sizeof(orc_tinfo));
  for (uint64_t i = 0; i < n_tensors; i++) { /* TensorInfo::read (src/gguf/tensor.rs:52-75) */
    orc_tinfo* t = &m->tensors[i];
    if ((rc = rd_string(&r, &t->name))) goto fail;
    m->n_tensors = i + 1;
    if ((rc = RD(&r, t->n_dims))) goto fail;
    if (t->n_dims > 4) { rc = ORC_E_INVALID_SHAPE; goto fail; }
    for (uint32_t d = 0; d < t->n_dims; d++)
      if ((rc = RD(&r, t->shape[d]))) goto fail;
    if ((rc = RD(&r, t->type))) goto fail;
    if (!type_known(t->type)) { rc = ORC_E_UNKNOWN_TENSOR_TYPE; goto fail; }
    if ((rc = RD(&r, t->offset))) goto fail;
  }
  m->data_offset = (r.pos + 31) / 32 * 32; /* fixed 32-byte alignment, src/gguf/file.rs:112-116 */

  /* Config::from_gguf */
  const orc_meta* arch = meta_get(m, "general.architecture");
  if (!arch || arch->type != 8) { rc = ORC_E_TENSOR_NOT_FOUND; goto fail; }
  if (strcmp(arch->str, "llama") != 0) { rc = ORC_E_UNSUPPORTED_ARCH; goto fail; }
  orc_config* c = &m->cfg;
  if (!get_u64(m, "llama.embedding_length", &c->hidden_size) ||
      !get_u64(m, "llama.block_count", &c->n_layers) ||
      !get_u64(m, "llama.attention.head_count", &c->n_heads)) {
    rc = ORC_E_TENSOR_NOT_FOUND;
    goto fail;
  }
  uint32_t u;
  c->n_kv_heads = get_u32(m, "llama.attention.head_count_kv", &u) ? u : c->n_heads;
  if (c->n_heads == 0) { rc = ORC_E_INVALID_ARG; goto fail; }
  c->head_dim = get_u32(m, "llama.attention.key_length", &u) ? u : c->hidden_size / c->n_heads;
  if (!get_u64(m, "llama.feed_forward_length", &c->intermediate_size)) { rc = ORC_E_TENSOR_NOT_FOUND; goto fail; }
  if (!get_f32(m, "llama.attention.layer_norm_rms_epsilon", &c->norm_eps)) c->norm_eps = 1e-5f;
  if (!get_f32(m, "llama.rope.freq_base", &c->rope_base)) c->rope_base = 10000.0f;
  c->rope_dim = get_u32(m, "llama.rope.dimension_count", &u) ? u : c->head_dim;
  c->context_length = get_u32(m, "llama.context_length", &u) ? u : 4096;
  c->vocab_size = get_u32(m, "llama.vocab_size", &u) ? u : 0;

  /* Model::open / Layer::from_weights name resolution.  Every layer needs 9
   * distinct tensors, so a block_count beyond n_tensors / 9 meets a missing
   * blk.N tensor (TensorNotFound) before the array sized here runs out. */
  {
    uint64_t cap = c->n_layers < m->n_tensors / 9 + 1 ? c->n_layers : m->n_tensors / 9 + 1;
    m->layers = (orc_layer*)calloc(cap ? cap : 1, sizeof(orc_layer));
    if (!m->layers) { rc = ORC_E_OOM; goto fail; }
  }
  static const char* names[9] = {"attn_norm", "attn_q",   "attn_k", "attn_v",  "attn_output",
                                 "ffn_norm",  "ffn_gate", "ffn_up", "ffn_down"};
  for (uint64_t l = 0; l < c->n_layers; l++) {
    int64_t* slots = &m->layers[l].attn_norm;
    for (int k = 0; k < 9; k++) {
      char nm[128];
      snprintf(nm, sizeof nm, "blk.%llu.%s.weight", (unsigned long long)l, names[k]);
      slots[k] = tensor_index(m, nm);
      if (slots[k] < 0) { rc = ORC_E_TENSOR_NOT_FOUND; goto fail; }
    }
  }
  m->token_embd = tensor_index(m, "token_embd.weight");
  if (m->token_embd < 0) { rc = ORC_E_TENSOR_NOT_FOUND; goto fail; }
  m->output_norm = tensor_index(m, "output_norm.weight");
  if (m->output_norm < 0) { rc = ORC_E_TENSOR_NOT_FOUND; goto fail; }
  m->output = tensor_index(m, "output.weight");
  *out = m;
  return ORC_OK;
fail:
  model_free(m);
  return rc;
}

int orc_model_config(const orc_model* m, orc_config* out) {
  *out = m->cfg;
  return ORC_OK;
}

int orc_model_n_tensors(const orc_model* m, uint64_t* n) {
  *n = m->n_tensors;
  return ORC_OK;
}

int orc_model_tensor_info(const orc_model* m, uint64_t idx, char* name, uint64_t cap,
                          uint32_t* type, uint64_t* n_dims, uint64_t* shape4, uint64_t* offset) {
  if (idx >= m->n_tensors) return ORC_E_INVALID_TENSOR_INDEX;
  const orc_tinfo* t = &m->tensors[idx];
  if (name && cap) { strncpy(name, t->name, cap - 1); name[cap - 1] = 0; }
  *type = t->type;
  *n_dims = t->n_dims;
  for (int d = 0; d < 4; d++) shape4[d] = d < (int)t->n_dims ? t->shape[d] : 0;
  *offset = t->offset;
  return ORC_OK;
}

/* ------------------------------------------------------------------------- */
/* KvCache (src/model/cache.rs:8-38)                                          */
/* ------------------------------------------------------------------------- */
orc_kv* orc_kv_new(const orc_model* m, uint64_t max_seq_len) {
  orc_kv* kv = (orc_kv*)calloc(1, sizeof(orc_kv));
  kv->n_layers = m->cfg.n_layers;
  kv->max_seq_len = max_seq_len;
  kv->kv_dim = m->cfg.n_kv_heads * m->cfg.head_dim;
  kv->k = (float**)calloc(kv->n_layers ? kv->n_layers : 1, sizeof(float*));
  kv->v = (float**)calloc(kv->n_layers ? kv->n_layers : 1, sizeof(float*));
  for (uint64_t l = 0; l < kv->n_layers; l++) {
    kv->k[l] = (float*)calloc(max_seq_len * kv->kv_dim + 1, 4);
    kv->v[l] = (float*)calloc(max_seq_len * kv->kv_dim + 1, 4);
  }
  return kv;
}

void orc_kv_free(orc_kv* kv) {
  if (!kv) return;
  for (uint64_t l = 0; l < kv->n_layers; l++) { free(kv->k[l]); free(kv->v[l]); }
  free(kv->k);
  free(kv->v);
  free(kv);
}

void orc_kv_clear(orc_kv* kv) { kv->len = 0; }
void orc_kv_set_f16(orc_kv* kv, int on) { kv->f16 = on != 0; }
uint64_t orc_kv_len(const orc_kv* kv) { return kv->len; }

/* Import/export in the reference layout [layer][t][kv_dim], t < len. */
int orc_kv_import(orc_kv* kv, const float* k, const float* v, uint64_t len) {
  if (len > kv->max_seq_len) return ORC_E_KV_FULL;
  for (uint64_t l = 0; l < kv->n_layers; l++) {
    memcpy(kv->k[l], k + l * len * kv->kv_dim, len * kv->kv_dim * 4);
    memcpy(kv->v[l], v + l * len * kv->kv_dim, len * kv->kv_dim * 4);
  }
  kv->len = len;
  return ORC_OK;
}

int orc_kv_export(const orc_kv* kv, float* k, float* v, uint64_t len) {
  if (len > kv->len) return ORC_E_INVALID_ARG;
  for (uint64_t l = 0; l < kv->n_layers; l++) {
    memcpy(k + l * len * kv->kv_dim, kv->k[l], len * kv->kv_dim * 4);
    memcpy(v + l * len * kv->kv_dim, kv->v[l], len * kv->kv_dim * 4);
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------------- */
/* Model forward (src/model/forward.rs)                                      */
/* ------------------------------------------------------------------------- */
void orc_set_threads(int n) {
  if (n > 0) omp_set_num_threads(n);
}

/* Weights::tensor_f32_by_index (src/gguf/weights.rs:66-74): full dequant into a
 * freshly zero-allocated vector. */
static int tensor_f32(const orc_model* m, int64_t idx, float** out, uint64_t* n_out) {
  const uint8_t* data;
  uint64_t nb;
  int rc = tensor_bytes(m, idx, &data, &nb);
  if (rc) return rc;
  uint64_t n = t_nelem(&m->tensors[idx]);
  float* buf = (float*)calloc(n ? n : 1, 4);
  if (!buf) return ORC_E_INVALID_ARG;
  rc = orc_dequantize_f32(m->tensors[idx].type, n, data, nb, buf, n);
  if (rc) { free(buf); return rc; }
  *out = buf;
  if (n_out) *n_out = n;
  return ORC_OK;
}

/* ------------------------------------------------------------------------- */
/* FAST-mode kernels.  Same values as the restatements above, computed with    */
/* AVX2: every element and every output sees the same IEEE operations in the  */
/* same order (no fusion beyond the explicit 8-lane FMA of matmul_t), so FAST  */
/* equals FAITHFUL bit for bit; only independent work is interleaved.          */
/* ------------------------------------------------------------------------- */

/* 8 bytes (low half of v) as 8 floats */
static inline __m256 u8x8_to_ps(__m128i v) { return _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(v)); }

/* dq_q4_k: per group y = (dall * f32(q)) - dm with the nibble order of
 * dequant.rs:155-159 (element 2i = low nibble of byte i, 2i+1 = high). */
static void dq_q4_k_fast(const uint8_t* src, uint64_t nb, float* out) {
  const __m128i m4 = _mm_set1_epi8(15);
  for (uint64_t b = 0; b < nb; b++) {
    const uint8_t* blk = src + b * 144;
    const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
    const uint8_t* s = blk + 4;
    const uint8_t* qs = blk + 16;
    for (int g = 0; g < 8; g++) {
      uint32_t sc, mn;
      if (g < 4) {
        sc = s[g] & 63u;
        mn = s[g + 4] & 63u;
      } else {
        sc = (s[g + 4] & 15u) | ((uint32_t)(s[g - 4] >> 6) << 4);
        mn = (uint32_t)(s[g + 4] >> 4) | ((uint32_t)(s[g] >> 6) << 4);
      }
      const __m256 vd = _mm256_set1_ps(d * (float)sc), vm = _mm256_set1_ps(dmin * (float)mn);
      const __m128i raw = _mm_loadu_si128((const __m128i*)(qs + 16 * g));
      const __m128i lo = _mm_and_si128(raw, m4), hi = _mm_and_si128(_mm_srli_epi16(raw, 4), m4);
      const __m128i e0 = _mm_unpacklo_epi8(lo, hi), e1 = _mm_unpackhi_epi8(lo, hi);
      float* o = out + b * 256 + 32 * g;
      _mm256_storeu_ps(o, _mm256_sub_ps(_mm256_mul_ps(vd, u8x8_to_ps(e0)), vm));
      _mm256_storeu_ps(o + 8, _mm256_sub_ps(_mm256_mul_ps(vd, u8x8_to_ps(_mm_srli_si128(e0, 8))), vm));
      _mm256_storeu_ps(o + 16, _mm256_sub_ps(_mm256_mul_ps(vd, u8x8_to_ps(e1)), vm));
      _mm256_storeu_ps(o + 24, _mm256_sub_ps(_mm256_mul_ps(vd, u8x8_to_ps(_mm_srli_si128(e1, 8))), vm));
    }
  }
}

/* the four 2-bit fields of a qh byte, one per byte of the word (element j of
 * the four takes bits 2j, 2j+1: dequant.rs:189-192) */
static uint32_t g_qh4[256];
__attribute__((constructor)) static void qh4_init(void) {
  for (int v = 0; v < 256; v++)
    g_qh4[v] = (uint32_t)(v & 3) | ((uint32_t)((v >> 2) & 3) << 8) | ((uint32_t)((v >> 4) & 3) << 16) |
               ((uint32_t)((v >> 6) & 3) << 24);
}

/* dq_q6_k: y = (d * f32(u8 sc)) * f32(q - 32) per 16-element part */
static void dq_q6_k_fast(const uint8_t* src, uint64_t nb, float* out) {
  const __m128i m4 = _mm_set1_epi8(15);
  const __m256i c32 = _mm256_set1_epi32(32);
  for (uint64_t b = 0; b < nb; b++) {
    const uint8_t* blk = src + b * 210;
    const float d = ld_f16(blk);
    const uint8_t *sc = blk + 2, *ql = blk + 18, *qh = blk + 146;
    for (int part = 0; part < 16; part++) {
      /* elements 16 part .. +15: ql bytes 8 part .. +7, qh bytes 4 part .. +3 */
      const __m128i raw = _mm_loadl_epi64((const __m128i*)(ql + 8 * part));
      const __m128i lo = _mm_unpacklo_epi8(_mm_and_si128(raw, m4), _mm_and_si128(_mm_srli_epi16(raw, 4), m4));
      const __m128i hi = _mm_set_epi32((int)g_qh4[qh[4 * part + 3]], (int)g_qh4[qh[4 * part + 2]],
                                       (int)g_qh4[qh[4 * part + 1]], (int)g_qh4[qh[4 * part]]);
      const __m128i q = _mm_or_si128(lo, _mm_slli_epi16(hi, 4));
      const __m256 vs = _mm256_set1_ps(d * (float)sc[part]);
      float* o = out + b * 256 + 16 * part;
      _mm256_storeu_ps(o, _mm256_mul_ps(vs, _mm256_cvtepi32_ps(_mm256_sub_epi32(_mm256_cvtepu8_epi32(q), c32))));
      _mm256_storeu_ps(o + 8, _mm256_mul_ps(vs, _mm256_cvtepi32_ps(
                                                    _mm256_sub_epi32(_mm256_cvtepu8_epi32(_mm_srli_si128(q, 8)), c32))));
    }
  }
}

/* dq_q8_0: y = f32(i8 q) * delta */
static void dq_q8_0_fast(const uint8_t* src, uint64_t nb, float* out) {
  for (uint64_t b = 0; b < nb; b++) {
    const uint8_t* blk = src + b * 34;
    const __m256 vd = _mm256_set1_ps(ld_f16(blk));
    for (int h = 0; h < 4; h++) {
      const __m128i raw = _mm_loadl_epi64((const __m128i*)(blk + 2 + 8 * h));
      _mm256_storeu_ps(out + b * 32 + 8 * h, _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(raw)), vd));
    }
  }
}

static int dq_units_fast(uint32_t t, const uint8_t* src, uint64_t nunits, float* out) {
  switch (t) {
    case T_Q4K: dq_q4_k_fast(src, nunits, out); return ORC_OK;
    case T_Q6K: dq_q6_k_fast(src, nunits, out); return ORC_OK;
    case T_Q8_0: dq_q8_0_fast(src, nunits, out); return ORC_OK;
    default: return dq_units(t, src, nunits, out);
  }
}

static int dq_range_fast(uint32_t t, const uint8_t* data, uint64_t e0, uint64_t n, float* out,
                         float* scratch) {
  uint64_t ue, ub;
  int rc = unit_of(t, &ue, &ub);
  if (rc) return rc;
  uint64_t u0 = e0 / ue, u1 = (e0 + n + ue - 1) / ue;
  if (u0 * ue == e0 && u1 * ue == e0 + n) return dq_units_fast(t, data + u0 * ub, u1 - u0, out);
  rc = dq_units_fast(t, data + u0 * ub, u1 - u0, scratch);
  memcpy(out, scratch + (e0 - u0 * ue), n * 4);
  return rc;
}

/* Test hook: dequantize_f32 through the FAST routines (must equal the restatement). */
int orc_dequantize_fast(uint32_t t, uint64_t n_elements, const uint8_t* bytes, float* out) {
  uint64_t ue, ub;
  if (unit_of(t, &ue, &ub) != ORC_OK || n_elements % ue) return ORC_E_INVALID_ARG;
  return dq_units_fast(t, bytes, n_elements / ue, out);
}

/* dot_ref's hsum tree and scalar tail, from a finished 8-lane accumulator */
static inline float finish_ref(__m256 acc, const float* a, const float* b, uint64_t l, uint64_t k) {
  float lane[8];
  _mm256_storeu_ps(lane, acc);
  float s0 = lane[0] + lane[4], s1 = lane[1] + lane[5], s2 = lane[2] + lane[6], s3 = lane[3] + lane[7];
  float sum = (s0 + s1) + (s2 + s3);
  for (; l < k; l++) sum = sum + a[l] * b[l];
  return sum;
}

/* 3 rows of a x 4 rows of w: twelve dot_ref chains advanced together */
static inline void tile_3x4(const float* a0, const float* a1, const float* a2, const float* w0, const float* w1,
                            const float* w2, const float* w3, uint64_t k, float* c, uint64_t ldc) {
  __m256 c00 = _mm256_setzero_ps(), c01 = c00, c02 = c00, c03 = c00, c10 = c00, c11 = c00, c12 = c00, c13 = c00,
         c20 = c00, c21 = c00, c22 = c00, c23 = c00;
  uint64_t l = 0;
  for (; l + 8 <= k; l += 8) {
    const __m256 x0 = _mm256_loadu_ps(a0 + l), x1 = _mm256_loadu_ps(a1 + l), x2 = _mm256_loadu_ps(a2 + l);
    __m256 y = _mm256_loadu_ps(w0 + l);
    c00 = _mm256_fmadd_ps(x0, y, c00); c10 = _mm256_fmadd_ps(x1, y, c10); c20 = _mm256_fmadd_ps(x2, y, c20);
    y = _mm256_loadu_ps(w1 + l);
    c01 = _mm256_fmadd_ps(x0, y, c01); c11 = _mm256_fmadd_ps(x1, y, c11); c21 = _mm256_fmadd_ps(x2, y, c21);
    y = _mm256_loadu_ps(w2 + l);
    c02 = _mm256_fmadd_ps(x0, y, c02); c12 = _mm256_fmadd_ps(x1, y, c12); c22 = _mm256_fmadd_ps(x2, y, c22);
    y = _mm256_loadu_ps(w3 + l);
    c03 = _mm256_fmadd_ps(x0, y, c03); c13 = _mm256_fmadd_ps(x1, y, c13); c23 = _mm256_fmadd_ps(x2, y, c23);
  }
  c[0] = finish_ref(c00, a0, w0, l, k); c[1] = finish_ref(c01, a0, w1, l, k);
  c[2] = finish_ref(c02, a0, w2, l, k); c[3] = finish_ref(c03, a0, w3, l, k);
  c[ldc] = finish_ref(c10, a1, w0, l, k); c[ldc + 1] = finish_ref(c11, a1, w1, l, k);
  c[ldc + 2] = finish_ref(c12, a1, w2, l, k); c[ldc + 3] = finish_ref(c13, a1, w3, l, k);
  c[2 * ldc] = finish_ref(c20, a2, w0, l, k); c[2 * ldc + 1] = finish_ref(c21, a2, w1, l, k);
  c[2 * ldc + 2] = finish_ref(c22, a2, w2, l, k); c[2 * ldc + 3] = finish_ref(c23, a2, w3, l, k);
}

/* 1 row of a x 4 rows of w */
static inline void tile_1x4(const float* a0, const float* w0, const float* w1, const float* w2, const float* w3,
                            uint64_t k, float* c) {
  __m256 c0 = _mm256_setzero_ps(), c1 = c0, c2 = c0, c3 = c0;
  uint64_t l = 0;
  for (; l + 8 <= k; l += 8) {
    const __m256 x = _mm256_loadu_ps(a0 + l);
    c0 = _mm256_fmadd_ps(x, _mm256_loadu_ps(w0 + l), c0);
    c1 = _mm256_fmadd_ps(x, _mm256_loadu_ps(w1 + l), c1);
    c2 = _mm256_fmadd_ps(x, _mm256_loadu_ps(w2 + l), c2);
    c3 = _mm256_fmadd_ps(x, _mm256_loadu_ps(w3 + l), c3);
  }
  c[0] = finish_ref(c0, a0, w0, l, k); c[1] = finish_ref(c1, a0, w1, l, k);
  c[2] = finish_ref(c2, a0, w2, l, k); c[3] = finish_ref(c3, a0, w3, l, k);
}

/* c[m x n] = a . W^T for W rows [j0, j0 + jn) held dequantized in wb (jn x k) */
static void tiles(const float* a, uint64_t m, uint64_t k, const float* wb, uint64_t jn, uint64_t j0, float* c,
                  uint64_t n) {
  uint64_t i = 0;
  for (; i + 3 <= m; i += 3) {
    uint64_t r = 0;
    for (; r + 4 <= jn; r += 4)
      tile_3x4(a + i * k, a + (i + 1) * k, a + (i + 2) * k, wb + r * k, wb + (r + 1) * k, wb + (r + 2) * k,
               wb + (r + 3) * k, k, c + i * n + j0 + r, n);
    for (; r < jn; r++)
      for (uint64_t ii = i; ii < i + 3; ii++) c[ii * n + j0 + r] = dot_ref(a + ii * k, wb + r * k, k);
  }
  for (; i < m; i++) {
    uint64_t r = 0;
    for (; r + 4 <= jn; r += 4)
      tile_1x4(a + i * k, wb + r * k, wb + (r + 1) * k, wb + (r + 2) * k, wb + (r + 3) * k, k, c + i * n + j0 + r);
    for (; r < jn; r++) c[i * n + j0 + r] = dot_ref(a + i * k, wb + r * k, k);
  }
}

/* c[m x n] = a[m x k] . W^T with W = tensor idx ([n, k]) in the matmul_t order.
 * FAITHFUL dequantizes the whole tensor first (as the reference does on every
 * call); FAST dequantizes one row at a time inside a parallel loop.  Each c[i][j]
 * sees the same operation sequence either way. */
static int linear(const orc_model* mdl, int64_t idx, const float* a, uint64_t m, uint64_t n,
                  uint64_t k, float* c, int mode) {
  const uint8_t* data;
  uint64_t nb;
  int rc = tensor_bytes(mdl, idx, &data, &nb);
  if (rc) return rc;
  const orc_tinfo* t = &mdl->tensors[idx];
  if (t_nelem(t) != n * k) return ORC_E_INVALID_ARG; /* matmul_t shape assert */
  if (mode == ORC_MODE_FAITHFUL) {
    float* w;
    if ((rc = tensor_f32(mdl, idx, &w, NULL))) return rc;
    orc_matmul_t(a, w, c, m, n, k);
    free(w);
    return ORC_OK;
  }
  uint64_t ue, ub;
  if ((rc = unit_of(t->type, &ue, &ub))) return rc;
  /* blocks of JB weight rows, dequantized once and swept by every row of a in
   * 3 x 4 register tiles (the block stays in cache while a streams past) */
  const uint64_t JB = m == 1 ? 16 : 64, nblk = (n + JB - 1) / JB;
  int err = ORC_OK;
#pragma omp parallel
  {
    float* wb = (float*)malloc((JB * k + 2 * ue) * 4);
    float* scratch = (float*)malloc((k + 2 * ue) * 4);
#pragma omp for schedule(dynamic, 1)
    for (uint64_t bj = 0; bj < nblk; bj++) {
      const uint64_t j0 = bj * JB, jn = n - j0 < JB ? n - j0 : JB;
      int bad = 0;
      for (uint64_t r = 0; r < jn; r++)
        if (dq_range_fast(t->type, data, (j0 + r) * k, k, wb + r * k, scratch) != ORC_OK) bad = 1;
      if (bad) {
        err = ORC_E_UNKNOWN_TENSOR_TYPE;
        continue;
      }
      tiles(a, m, k, wb, jn, j0, c, n);
    }
    free(wb);
    free(scratch);
  }
  return err;
}

/* The norm weight tensor as f32 (F32 copy, or dequant for other types). */
static int norm_weight(const orc_model* m, int64_t idx, uint64_t n, float** w) {
  uint64_t cnt;
  int rc = tensor_f32(m, idx, w, &cnt);
  if (rc) return rc;
  if (cnt != n) { free(*w); return ORC_E_INVALID_ARG; }
  return ORC_OK;
}

/* Embedding row `tok` of token_embd: FAITHFUL dequantizes the whole table as
 * src/model/forward.rs:556-558 does; FAST only the blocks covering the row. */
static int embed_row(const orc_model* m, uint32_t tok, float* dst, int mode) {
  uint64_t H = m->cfg.hidden_size;
  const orc_tinfo* t = &m->tensors[m->token_embd];
  if ((uint64_t)tok * H + H > t_nelem(t)) return ORC_E_INVALID_ARG;
  if (mode == ORC_MODE_FAITHFUL) {
    float* emb;
    int rc = tensor_f32(m, m->token_embd, &emb, NULL);
    if (rc) return rc;
    memcpy(dst, emb + (uint64_t)tok * H, H * 4);
    free(emb);
    return ORC_OK;
  }
  const uint8_t* data;
  uint64_t nb, ue, ub;
  int rc = tensor_bytes(m, m->token_embd, &data, &nb);
  if (rc) return rc;
  if ((rc = unit_of(t->type, &ue, &ub))) return rc;
  float* scratch = (float*)malloc((H + 2 * ue) * 4);
  rc = dq_range(t->type, data, (uint64_t)tok * H, H, dst, scratch);
  free(scratch);
  return rc;
}

static int64_t out_weight(const orc_model* m) { return m->output >= 0 ? m->output : m->token_embd; }

static int check_dims(const orc_model* m) {
  const orc_config* c = &m->cfg;
  if (c->n_kv_heads == 0 || c->n_heads % c->n_kv_heads || c->n_heads * c->head_dim != c->hidden_size ||
      c->rope_dim > c->head_dim || (c->rope_dim & 1))
    return ORC_E_INVALID_ARG; /* shape asserts of matmul_t / rope */
  return ORC_OK;
}

/* One query head of the decode attention (src/model/forward.rs:383-414):
 * s_t = (sum_d q_d k_td) / sqrt(hd) in sequence, softmax_rows, o_d = sum_t p_t v_td. */
static void decode_head(const float* q, const float* kc, const float* vc, uint64_t nl, uint64_t h, uint64_t grp,
                        uint64_t hd, uint64_t kvd, float* scores, float* head_out, float* attn) {
  uint64_t hk = h / grp;
  const float* qh = q + h * hd;
  float rs = sqrtf((float)hd);
  for (uint64_t t = 0; t < nl; t++) {
    const float* kh = kc + t * kvd + hk * hd;
    float s = 0.0f;
    for (uint64_t d = 0; d < hd; d++) s = s + qh[d] * kh[d];
    scores[t] = s / rs;
  }
  orc_softmax_rows(scores, 1, nl);
  for (uint64_t d = 0; d < hd; d++) head_out[d] = 0.0f;
  for (uint64_t t = 0; t < nl; t++) {
    const float* vh = vc + t * kvd + hk * hd;
    for (uint64_t d = 0; d < hd; d++) head_out[d] = head_out[d] + scores[t] * vh[d];
  }
  memcpy(attn + h * hd, head_out, hd * 4);
}

/* Layer::decode_step (src/model/forward.rs:344-440). */
static int layer_decode(const orc_model* m, const orc_layer* L, float* kc, float* vc,
                        uint64_t cache_len, float* hidden, int mode, int rope_mode, int kv16) {
  const orc_config* c = &m->cfg;
  uint64_t H = c->hidden_size, hd = c->head_dim, kvd = c->n_kv_heads * hd, F = c->intermediate_size;
  uint64_t grp = c->n_heads / c->n_kv_heads;
  int rc = ORC_OK;
  float *residual = malloc(H * 4), *q = malloc(H * 4), *k = malloc(kvd * 4), *v = malloc(kvd * 4);
  float *scores = malloc((cache_len + 1) * 4), *head_out = malloc(hd * 4), *attn = calloc(H, 4);
  float *gate = malloc(F * 4), *up = malloc(F * 4), *mid = malloc(F * 4), *down = malloc(H * 4);
  float* w = NULL;
  memcpy(residual, hidden, H * 4);
  if ((rc = norm_weight(m, L->attn_norm, H, &w))) goto done;
  orc_rms_norm(hidden, w, H, c->norm_eps);
  free(w); w = NULL;
  if ((rc = linear(m, L->attn_q, hidden, 1, H, H, q, mode))) goto done;
  if ((rc = linear(m, L->attn_k, hidden, 1, kvd, H, k, mode))) goto done;
  if ((rc = linear(m, L->attn_v, hidden, 1, kvd, H, v, mode))) goto done;
  /* rope(.., 1, ..): position 0 in the reference (src/model/forward.rs:371-372) */
  uint64_t pos0 = rope_mode == ORC_ROPE_ABSOLUTE ? cache_len : 0;
  orc_rope(q, 1, c->n_heads, hd, c->rope_dim, c->rope_base, pos0);
  orc_rope(k, 1, c->n_kv_heads, hd, c->rope_dim, c->rope_base, pos0);
  if (kv16) {
    round_f16_n(k, kvd);
    round_f16_n(v, kvd);
  }
  memcpy(kc + cache_len * kvd, k, kvd * 4);
  memcpy(vc + cache_len * kvd, v, kvd * 4);
  uint64_t nl = cache_len + 1;
  if (mode == ORC_MODE_FAITHFUL) {
    for (uint64_t h = 0; h < c->n_heads; h++)
      decode_head(q, kc, vc, nl, h, grp, hd, kvd, scores, head_out, attn);
  } else {
    /* the heads are independent: FAST runs them in parallel, each exactly as above */
#pragma omp parallel
    {
      float* sc_t = (float*)malloc(nl * 4);
      float* ho_t = (float*)malloc(hd * 4);
#pragma omp for schedule(static)
      for (uint64_t h = 0; h < c->n_heads; h++) decode_head(q, kc, vc, nl, h, grp, hd, kvd, sc_t, ho_t, attn);
      free(sc_t);
      free(ho_t);
    }
  }
  if ((rc = linear(m, L->attn_output, attn, 1, H, H, hidden, mode))) goto done;
  orc_add_in_place(hidden, residual, H);
  memcpy(residual, hidden, H * 4);
  if ((rc = norm_weight(m, L->ffn_norm, H, &w))) goto done;
  orc_rms_norm(hidden, w, H, c->norm_eps);
  free(w); w = NULL;
  if ((rc = linear(m, L->ffn_gate, hidden, 1, F, H, gate, mode))) goto done;
  if ((rc = linear(m, L->ffn_up, hidden, 1, F, H, up, mode))) goto done;
  orc_swiglu(gate, up, mid, F);
  if ((rc = linear(m, L->ffn_down, mid, 1, H, F, down, mode))) goto done;
  memcpy(hidden, down, H * 4);
  orc_add_in_place(hidden, residual, H);
done:
  free(w); free(residual); free(q); free(k); free(v); free(scores); free(head_out); free(attn);
  free(gate); free(up); free(mid); free(down);
  return rc;
}

/* Model::decode_step (src/model/forward.rs:543-586). */
int orc_decode_step(const orc_model* m, orc_kv* kv, uint32_t token, float* logits, int mode,
                    int rope_mode) {
  const orc_config* c = &m->cfg;
  int rc;
  if ((uint64_t)token >= (uint64_t)c->vocab_size) return ORC_E_INVALID_TENSOR_INDEX;
  if ((rc = check_dims(m))) return rc;
  if (kv->len >= kv->max_seq_len) return ORC_E_KV_FULL; /* slice panic at forward.rs:376 */
  uint64_t H = c->hidden_size, V = c->vocab_size;
  float* hidden = (float*)malloc(H * 4);
  float* w = NULL;
  if ((rc = embed_row(m, token, hidden, mode))) goto done;
  for (uint64_t l = 0; l < c->n_layers; l++)
    if ((rc = layer_decode(m, &m->layers[l], kv->k[l], kv->v[l], kv->len, hidden, mode, rope_mode, kv->f16)))
      goto done;
  if ((rc = norm_weight(m, m->output_norm, H, &w))) goto done;
  orc_rms_norm(hidden, w, H, c->norm_eps);
  if ((rc = linear(m, out_weight(m), hidden, 1, V, H, logits, mode))) goto done;
  kv->len += 1;
done:
  free(w);
  free(hidden);
  return rc;
}

/* The chunk attention of layer_batch in FAST mode: query heads in parallel;
 * the scores of 8 keys at once from the head's K transposed (lane t holds key
 * t), each score the same sequential s = s + q_d k_d then / sqrt(hd) as the
 * scalar loop; softmax_rows per head as before; p . V over 8 head-dim lanes,
 * each the same sequential sum over keys. */
static void batch_attention_fast(const float* q, const float* k, const float* v, float* attn, uint64_t seq,
                                 uint64_t nh, uint64_t nkv, uint64_t hd, uint64_t H, int causal) {
  const uint64_t grp = nh / nkv, seq8 = (seq + 7) / 8 * 8;
  const __m256 vrs = _mm256_set1_ps(sqrtf((float)hd));
#pragma omp parallel
  {
    float* scores = (float*)malloc(seq * seq * 4 + 4);
    float* kt = (float*)malloc(hd * seq8 * 4 + 4);
    float* row = (float*)malloc(seq8 * 4 + 4);
    float* ho = (float*)malloc(hd * 4 + 4);
#pragma omp for schedule(dynamic, 1)
    for (uint64_t h = 0; h < nh; h++) {
      const uint64_t hk = h / grp;
      for (uint64_t d = 0; d < hd; d++) {
        for (uint64_t t = 0; t < seq; t++) kt[d * seq8 + t] = k[(t * nkv + hk) * hd + d];
        for (uint64_t t = seq; t < seq8; t++) kt[d * seq8 + t] = 0.0f;
      }
      for (uint64_t p = 0; p < seq; p++) {
        const float* qh = q + (p * nh + h) * hd;
        const uint64_t tend = causal ? p + 1 : seq;
        for (uint64_t t0 = 0; t0 < tend; t0 += 8) {
          __m256 sv = _mm256_setzero_ps();
          for (uint64_t d = 0; d < hd; d++)
            sv = _mm256_add_ps(sv, _mm256_mul_ps(_mm256_set1_ps(qh[d]), _mm256_loadu_ps(kt + d * seq8 + t0)));
          _mm256_storeu_ps(row + t0, _mm256_div_ps(sv, vrs));
        }
        for (uint64_t t = tend; t < seq; t++) row[t] = -INFINITY;
        memcpy(scores + p * seq, row, seq * 4);
      }
      orc_softmax_rows(scores, seq, seq);
      for (uint64_t p = 0; p < seq; p++) {
        const uint64_t tend = causal ? p + 1 : seq;
        for (uint64_t d = 0; d < hd; d++) ho[d] = 0.0f;
        for (uint64_t t = 0; t < tend; t++) {
          const __m256 sc = _mm256_set1_ps(scores[p * seq + t]);
          const float* vh = v + (t * nkv + hk) * hd;
          uint64_t d = 0;
          for (; d + 8 <= hd; d += 8)
            _mm256_storeu_ps(ho + d, _mm256_add_ps(_mm256_loadu_ps(ho + d), _mm256_mul_ps(sc, _mm256_loadu_ps(vh + d))));
          for (; d < hd; d++) ho[d] = ho[d] + scores[p * seq + t] * vh[d];
        }
        memcpy(attn + p * H + h * hd, ho, hd * 4);
      }
    }
    free(scores);
    free(kt);
    free(row);
    free(ho);
  }
}

/* The chunk attention of Layer::prefill (src/model/forward.rs:255-303, causal)
 * and Layer::forward (src/model/forward.rs:104-156, no mask), one query head
 * after another: s_pt = (sum_d q_d k_td) / sqrt(hd) in sequence (masked keys
 * -inf), softmax_rows over the whole row, o_pd = sum_{t <= p} p_pt v_td.
 * q, attn: [seq][H] (head h at h*hd); k, v: [seq][nkv*hd].  scores: seq*seq
 * floats of scratch, head_out: seq*hd. */
static void batch_attention_ref(const float* q, const float* k, const float* v, float* attn, uint64_t seq,
                                uint64_t nh, uint64_t nkv, uint64_t hd, uint64_t H, int causal, float* scores,
                                float* head_out) {
  const uint64_t grp = nh / nkv;
  float rs = sqrtf((float)hd);
  for (uint64_t h = 0; h < nh; h++) {
    uint64_t hk = h / grp;
    for (uint64_t p = 0; p < seq; p++) {
      const float* qh = q + (p * nh + h) * hd;
      for (uint64_t t = 0; t < seq; t++) {
        if (causal && t > p) { scores[p * seq + t] = -INFINITY; continue; }
        const float* kh = k + (t * nkv + hk) * hd;
        float s = 0.0f;
        for (uint64_t d = 0; d < hd; d++) s = s + qh[d] * kh[d];
        scores[p * seq + t] = s / rs;
      }
    }
    orc_softmax_rows(scores, seq, seq);
    for (uint64_t p = 0; p < seq; p++) {
      float* ho = head_out + p * hd;
      for (uint64_t d = 0; d < hd; d++) ho[d] = 0.0f;
      uint64_t tend = causal ? p + 1 : seq;
      for (uint64_t t = 0; t < tend; t++) {
        float sc = scores[p * seq + t];
        const float* vh = v + (t * nkv + hk) * hd;
        for (uint64_t d = 0; d < hd; d++) ho[d] = ho[d] + sc * vh[d];
      }
      memcpy(attn + p * H + h * hd, ho, hd * 4);
    }
  }
}

/* The decode attention of Layer::decode_step (src/model/forward.rs:383-414)
 * on its own: every query head of q [n_heads*hd] over cache rows 0..nl-1 of k,
 * v in the KvCache layout [t][n_kv_heads*hd] (src/model/cache.rs:8-24); out
 * [n_heads*hd].  The same decode_head the decode step runs. */
int orc_attention_decode(const float* q, const float* k, const float* v, uint64_t nl, uint64_t n_heads,
                         uint64_t n_kv_heads, uint64_t hd, float* out) {
  if (!q || !k || !v || !out || nl == 0 || hd == 0 || n_kv_heads == 0 || n_heads % n_kv_heads)
    return ORC_E_INVALID_ARG;
  const uint64_t grp = n_heads / n_kv_heads, kvd = n_kv_heads * hd;
  float *scores = malloc(nl * 4), *head_out = malloc(hd * 4);
  if (!scores || !head_out) { free(scores); free(head_out); return ORC_E_OOM; }
  for (uint64_t h = 0; h < n_heads; h++) decode_head(q, k, v, nl, h, grp, hd, kvd, scores, head_out, out);
  free(scores);
  free(head_out);
  return ORC_OK;
}

/* The chunk attention of Layer::prefill / Layer::forward on its own (the
 * loops layer_batch runs): q, out [seq][n_heads*hd]; k, v [seq][n_kv_heads*hd]
 * (the chunk's rows).  FAITHFUL: batch_attention_ref; FAST: the threaded form
 * (the same bits). */
int orc_attention_batch(const float* q, const float* k, const float* v, uint64_t seq, uint64_t n_heads,
                        uint64_t n_kv_heads, uint64_t hd, int causal, float* out, int mode) {
  if (!q || !k || !v || !out || seq == 0 || hd == 0 || n_kv_heads == 0 || n_heads % n_kv_heads)
    return ORC_E_INVALID_ARG;
  const uint64_t H = n_heads * hd;
  if (mode == ORC_MODE_FAST) {
    batch_attention_fast(q, k, v, out, seq, n_heads, n_kv_heads, hd, H, causal);
    return ORC_OK;
  }
  float *scores = malloc(seq * seq * 4), *head_out = malloc(seq * hd * 4);
  if (!scores || !head_out) { free(scores); free(head_out); return ORC_E_OOM; }
  batch_attention_ref(q, k, v, out, seq, n_heads, n_kv_heads, hd, H, causal, scores, head_out);
  free(scores);
  free(head_out);
  return ORC_OK;
}

/* Shared body of Layer::prefill (src/model/forward.rs:215-337, causal, writes
 * the cache) and Layer::forward (src/model/forward.rs:62-207, no mask, no cache). */
static int layer_batch(const orc_model* m, const orc_layer* L, float* x, uint64_t seq, float* kc,
                       float* vc, uint64_t cache_start, int causal, int mode, int rope_mode, int kv16) {
  const orc_config* c = &m->cfg;
  uint64_t H = c->hidden_size, hd = c->head_dim, kvd = c->n_kv_heads * hd, F = c->intermediate_size;
  uint64_t nh = c->n_heads;
  int rc = ORC_OK;
  float *residual = malloc(seq * H * 4), *q = malloc(seq * H * 4), *k = malloc(seq * kvd * 4);
  float *v = malloc(seq * kvd * 4), *scores = malloc(seq * seq * 4), *head_out = malloc(seq * hd * 4);
  float *attn = calloc(seq * H, 4), *gate = malloc(seq * F * 4), *up = malloc(seq * F * 4);
  float *mid = malloc(seq * F * 4), *down = malloc(seq * H * 4);
  float* w = NULL;
  memcpy(residual, x, seq * H * 4);
  if ((rc = norm_weight(m, L->attn_norm, H, &w))) goto done;
  orc_rms_norm_rows(x, w, H, seq, c->norm_eps);
  free(w); w = NULL;
  if ((rc = linear(m, L->attn_q, x, seq, H, H, q, mode))) goto done;
  if ((rc = linear(m, L->attn_k, x, seq, kvd, H, k, mode))) goto done;
  if ((rc = linear(m, L->attn_v, x, seq, kvd, H, v, mode))) goto done;
  uint64_t pos0 = (causal && rope_mode == ORC_ROPE_ABSOLUTE) ? cache_start : 0;
  orc_rope(q, seq, nh, hd, c->rope_dim, c->rope_base, pos0);
  orc_rope(k, seq, c->n_kv_heads, hd, c->rope_dim, c->rope_base, pos0);
  if (kv16) { /* the chunk attends to its rows as the cache holds them */
    round_f16_n(k, seq * kvd);
    round_f16_n(v, seq * kvd);
  }
  if (kc) {
    for (uint64_t t = 0; t < seq; t++) {
      memcpy(kc + (cache_start + t) * kvd, k + t * kvd, kvd * 4);
      memcpy(vc + (cache_start + t) * kvd, v + t * kvd, kvd * 4);
    }
  }
  if (mode == ORC_MODE_FAITHFUL) {
    batch_attention_ref(q, k, v, attn, seq, nh, c->n_kv_heads, hd, H, causal, scores, head_out);
  } else {
    batch_attention_fast(q, k, v, attn, seq, nh, c->n_kv_heads, hd, H, causal);
  }
  if ((rc = linear(m, L->attn_output, attn, seq, H, H, x, mode))) goto done;
  orc_add_in_place(x, residual, seq * H);
  memcpy(residual, x, seq * H * 4);
  if ((rc = norm_weight(m, L->ffn_norm, H, &w))) goto done;
  orc_rms_norm_rows(x, w, H, seq, c->norm_eps);
  free(w); w = NULL;
  if ((rc = linear(m, L->ffn_gate, x, seq, F, H, gate, mode))) goto done;
  if ((rc = linear(m, L->ffn_up, x, seq, F, H, up, mode))) goto done;
  orc_swiglu(gate, up, mid, seq * F);
  if ((rc = linear(m, L->ffn_down, mid, seq, H, F, down, mode))) goto done;
  memcpy(x, down, seq * H * 4);
  orc_add_in_place(x, residual, seq * H);
done:
  free(w); free(residual); free(q); free(k); free(v); free(scores); free(head_out); free(attn);
  free(gate); free(up); free(mid); free(down);
  return rc;
}

/* Model::prefill (src/model/forward.rs:496-538) when kv != NULL, else
 * Model::forward (src/model/forward.rs:448-482).  Logits for every row. */
static int batch_forward(const orc_model* m, orc_kv* kv, const uint32_t* ids, uint64_t n,
                         float* logits, int mode, int rope_mode, const uint64_t* rows, uint64_t n_rows) {
  const orc_config* c = &m->cfg;
  uint64_t H = c->hidden_size, V = c->vocab_size;
  int rc;
  for (uint64_t i = 0; i < n; i++)
    if ((uint64_t)ids[i] >= V) return ORC_E_INVALID_TENSOR_INDEX;
  if ((rc = check_dims(m))) return rc;
  if (kv && kv->len + n > kv->max_seq_len) return ORC_E_KV_FULL;
  float* x = (float*)malloc((n ? n : 1) * H * 4);
  float* w = NULL;
  for (uint64_t i = 0; i < n; i++)
    if ((rc = embed_row(m, ids[i], x + i * H, mode))) goto done;
  for (uint64_t l = 0; l < c->n_layers; l++) {
    rc = layer_batch(m, &m->layers[l], x, n, kv ? kv->k[l] : NULL, kv ? kv->v[l] : NULL,
                     kv ? kv->len : 0, kv != NULL, mode, rope_mode, kv ? kv->f16 : 0);
    if (rc) goto done;
  }
  if (kv) kv->len += n;
  if ((rc = norm_weight(m, m->output_norm, H, &w))) goto done;
  orc_rms_norm_rows(x, w, H, n, c->norm_eps);
  if (rows) {
    /* logits of the listed rows only (matmul_t's rows are independent) */
    for (uint64_t r = 0; r < n_rows; r++)
      if (rows[r] >= n) { rc = ORC_E_INVALID_ARG; goto done; }
    float* xs = (float*)malloc((n_rows ? n_rows : 1) * H * 4);
    for (uint64_t r = 0; r < n_rows; r++) memcpy(xs + r * H, x + rows[r] * H, H * 4);
    rc = linear(m, out_weight(m), xs, n_rows, V, H, logits, mode);
    free(xs);
  } else {
    rc = linear(m, out_weight(m), x, n, V, H, logits, mode);
  }
done:
  free(w);
  free(x);
  return rc;
}

int orc_prefill(const orc_model* m, orc_kv* kv, const uint32_t* ids, uint64_t n, float* logits,
                int mode, int rope_mode) {
  return batch_forward(m, kv, ids, n, logits, mode, rope_mode, NULL, 0);
}

/* orc_prefill with the logits of rows[0 .. n_rows) only, in that order
 * ([n_rows x vocab]); the cache and every row's hidden state as orc_prefill. */
int orc_prefill_rows(const orc_model* m, orc_kv* kv, const uint32_t* ids, uint64_t n, const uint64_t* rows,
                     uint64_t n_rows, float* logits, int mode, int rope_mode) {
  return batch_forward(m, kv, ids, n, logits, mode, rope_mode, rows, n_rows);
}

int orc_forward(const orc_model* m, const uint32_t* ids, uint64_t n, float* logits, int mode) {
  return batch_forward(m, NULL, ids, n, logits, mode, ORC_ROPE_REFERENCE, NULL, 0);
}

/* orc_forward with the logits of rows[0 .. n_rows) only. */
int orc_forward_rows(const orc_model* m, const uint32_t* ids, uint64_t n, const uint64_t* rows, uint64_t n_rows,
                     float* logits, int mode) {
  return batch_forward(m, NULL, ids, n, logits, mode, ORC_ROPE_REFERENCE, rows, n_rows);
}

/* Model::generate (src/model/forward.rs:592-612): clear, prefill, then
 * max_tokens x (argmax of the last row -> decode_step). */
int orc_generate(const orc_model* m, orc_kv* kv, const uint32_t* prompt, uint64_t n,
                 uint64_t max_tokens, uint32_t* out, int mode, int rope_mode) {
  uint64_t V = m->cfg.vocab_size;
  if (n == 0) return ORC_E_INVALID_ARG; /* logits.len() - vocab underflows */
  orc_kv_clear(kv);
  float* logits = (float*)malloc(n * V * 4 + 4);
  int rc = orc_prefill(m, kv, prompt, n, logits, mode, rope_mode);
  const float* last = logits + (n - 1) * V;
  for (uint64_t s = 0; s < max_tokens && rc == ORC_OK; s++) {
    uint32_t tok;
    if ((rc = orc_argmax(last, V, &tok))) break;
    out[s] = tok;
    rc = orc_decode_step(m, kv, tok, logits, mode, rope_mode);
    last = logits;
  }
  free(logits);
  return rc;
}
