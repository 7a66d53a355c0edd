/*
 * oracle.h — CPU restatement of the inferox reference token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load it.  The product library (inferox_amd) never links,
 * loads or calls it, and has no CPU fallback through it.
 *
 * Every function restates one reference function; the citation is given at the
 * definition in oracle.c.  Floating-point order follows the reference exactly:
 * the library is compiled with -ffp-contract=off, uses the same AVX2 FMA lane
 * order as the reference matmul_t, and calls glibc expf/powf/sinf/cosf.
 */
#ifndef INFEROX_ORACLE_H
#define INFEROX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: one per reference gguf::Error variant (src/gguf/error.rs:6-42),
 * plus codes for conditions the reference turns into panics. Same numbering as
 * include/inferox.h. */
enum {
  ORC_OK = 0,
  ORC_E_IO = 1,
  ORC_E_INVALID_MAGIC = 2,
  ORC_E_UNSUPPORTED_VERSION = 3,
  ORC_E_UNKNOWN_VALUE_TYPE = 4,
  ORC_E_UNKNOWN_TENSOR_TYPE = 5,
  ORC_E_INVALID_UTF8 = 6,
  ORC_E_INVALID_SHAPE = 7,
  ORC_E_UNEXPECTED_EOF = 8,
  ORC_E_TENSOR_NOT_FOUND = 9,
  ORC_E_INVALID_TENSOR_INDEX = 10,
  ORC_E_TENSOR_OFFSET_OVERFLOW = 11,
  ORC_E_UNSUPPORTED_ARCH = 12,
  ORC_E_INVALID_ARG = 20,
  ORC_E_KV_FULL = 21,
  ORC_E_OOM = 23,
  ORC_E_NAN_LOGIT = 24,
};

/* Execution mode of the model-level oracle. Both give bit-identical results. */
enum {
  ORC_MODE_FAITHFUL = 0, /* per-step full-tensor dequant into fresh buffers, 1 thread */
  ORC_MODE_FAST = 1      /* per-row dequant fused with the same dot, threaded over rows */
};

/* RoPE position rule. REFERENCE reproduces the reference (decode at position 0,
 * prefill positions 0..seq relative to the chunk). ABSOLUTE uses the cache index. */
enum { ORC_ROPE_REFERENCE = 0, ORC_ROPE_ABSOLUTE = 1 };

/* ---- element conversion and dequantization ---- */
float orc_f16_to_f32(uint16_t h);
int orc_block_layout(uint32_t type, uint64_t* block_elems, uint64_t* block_bytes);
int orc_byte_size(uint32_t type, uint64_t n_elements, uint64_t* bytes);
int orc_dequantize_f32(uint32_t type, uint64_t n_elements, const uint8_t* bytes,
                       uint64_t n_bytes, float* out, uint64_t n_out);
/* dequantize through the FAST-mode routines (a test hook: equals orc_dequantize_f32) */
int orc_dequantize_fast(uint32_t type, uint64_t n_elements, const uint8_t* bytes, float* out);

/* ---- ops ---- */
void orc_matmul_t(const float* a, const float* b, float* c, uint64_t m, uint64_t n, uint64_t k);
void orc_matmul_t_scalar(const float* a, const float* b, float* c, uint64_t m, uint64_t n,
                         uint64_t k);
void orc_rms_norm(float* x, const float* w, uint64_t n, float eps);
void orc_rms_norm_rows(float* x, const float* w, uint64_t n, uint64_t rows, float eps);
void orc_silu(float* x, uint64_t n);
void orc_swiglu(const float* gate, const float* up, float* out, uint64_t n);
void orc_add_in_place(float* out, const float* b, uint64_t n);
void orc_softmax_rows(float* x, uint64_t rows, uint64_t cols);
int orc_embedding_lookup(const float* emb, uint64_t vocab, const uint32_t* ids, uint64_t n_ids,
                         uint64_t hidden, float* out);
void orc_rope(float* x, uint64_t seq, uint64_t heads, uint64_t head_dim, uint64_t rope_dim,
              float base, uint64_t pos0);
int orc_argmax(const float* x, uint64_t n, uint32_t* out);
/* The attention loops of the decode step and of a prefill/forward chunk on
 * their own.  Decode: q [n_heads*hd] over rows 0..nl-1 of k, v
 * [t][n_kv_heads*hd]; batch: q, out [seq][n_heads*hd], k, v [seq][n_kv*hd],
 * mode ORC_MODE_FAITHFUL or ORC_MODE_FAST (same bits). */
int orc_attention_decode(const float* q, const float* k, const float* v, uint64_t nl, uint64_t n_heads,
                         uint64_t n_kv_heads, uint64_t hd, float* out);
int orc_attention_batch(const float* q, const float* k, const float* v, uint64_t seq, uint64_t n_heads,
                        uint64_t n_kv_heads, uint64_t hd, int causal, float* out, int mode);

/* ---- GGUF + model ---- */
typedef struct orc_model orc_model;
typedef struct orc_kv orc_kv;

typedef struct {
  uint32_t vocab_size;
  uint64_t hidden_size, n_layers, n_heads, n_kv_heads, head_dim, intermediate_size;
  float norm_eps, rope_base;
  uint64_t rope_dim, context_length;
} orc_config;

int orc_model_open(const char* path, orc_model** out);
void orc_model_close(orc_model* m);
int orc_model_config(const orc_model* m, orc_config* out);
/* metadata / tensor-table inspection for parser tests */
int orc_model_n_tensors(const orc_model* m, uint64_t* n);
int orc_model_tensor_info(const orc_model* m, uint64_t idx, char* name, uint64_t name_cap,
                          uint32_t* type, uint64_t* n_dims, uint64_t* shape4, uint64_t* offset);
int orc_model_tensor_bytes(const orc_model* m, uint64_t idx, const uint8_t** data, uint64_t* n);

orc_kv* orc_kv_new(const orc_model* m, uint64_t max_seq_len);
void orc_kv_free(orc_kv* kv);
void orc_kv_clear(orc_kv* kv);
/* The f16-KV session mode (no reference counterpart): rows stored from now on
 * are rounded to binary16 (orc_round_f16) before any attention reads them;
 * import stores what it is given. */
void orc_kv_set_f16(orc_kv* kv, int on);
float orc_round_f16(float x);
uint64_t orc_kv_len(const orc_kv* kv);
int orc_kv_import(orc_kv* kv, const float* k, const float* v, uint64_t len);
int orc_kv_export(const orc_kv* kv, float* k, float* v, uint64_t len);

void orc_set_threads(int n);
int orc_decode_step(const orc_model* m, orc_kv* kv, uint32_t token, float* logits, int mode,
                    int rope_mode);
int orc_prefill(const orc_model* m, orc_kv* kv, const uint32_t* ids, uint64_t n, float* logits,
                int mode, int rope_mode);
int orc_prefill_rows(const orc_model* m, orc_kv* kv, const uint32_t* ids, uint64_t n, const uint64_t* rows,
                     uint64_t n_rows, float* logits, int mode, int rope_mode);
int orc_forward(const orc_model* m, const uint32_t* ids, uint64_t n, float* logits, int mode);
int orc_forward_rows(const orc_model* m, const uint32_t* ids, uint64_t n, const uint64_t* rows, uint64_t n_rows,
                     float* logits, int mode);
int orc_generate(const orc_model* m, orc_kv* kv, const uint32_t* prompt, uint64_t n,
                 uint64_t max_tokens, uint32_t* out, int mode, int rope_mode);

#ifdef __cplusplus
}
#endif
#endif
