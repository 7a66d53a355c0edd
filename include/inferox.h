/*
 * inferox.h — C ABI of the MI355X (gfx950) inferox token loop.
 *
 * This is the drop-in boundary: every entry point replaces one reference
 * interface (phraakture/inferox, cited as path:line) that a Rust crate would
 * bind through `extern "C"`.  Plain pointers and sizes only.
 *
 * Conventions
 *  - Every call returns an int status (IFX_OK = 0).  Nothing aborts: the
 *    conditions for which the reference panics (shape asserts, a full KV cache,
 *    a NaN met by argmax) come back as IFX_E_INVALID_ARG / IFX_E_KV_FULL /
 *    IFX_E_NAN_LOGIT.  ifx_last_error() gives a message for the calling thread.
 *  - `ifx_model` is immutable after open and may be shared by threads.  An
 *    `ifx_session` (KV cache + scratch + one HIP stream) is used by one thread
 *    at a time, like the reference's `&mut KvCache` / `&mut DecodeBuffers`.
 *  - Host-pointer outputs are complete when the call returns.
 *  - Kernel-level entry points (ifx_dequantize_f32, ifx_gemv, ifx_ops_*) take
 *    device pointers and a stream (NULL = the library's own stream) and are
 *    asynchronous; ifx_stream_synchronize() waits.
 */
#ifndef INFEROX_H
#define INFEROX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * Status codes.  1..12 map one-to-one onto the variants of the reference's
 * gguf::Error (src/gguf/error.rs:6-42); 20.. replace reference panics.
 * ------------------------------------------------------------------------- */
enum {
  IFX_OK = 0,
  IFX_E_IO = 1,                   /* Error::Io */
  IFX_E_INVALID_MAGIC = 2,        /* Error::InvalidMagic */
  IFX_E_UNSUPPORTED_VERSION = 3,  /* Error::UnsupportedVersion */
  IFX_E_UNKNOWN_VALUE_TYPE = 4,   /* Error::UnknownValueType */
  IFX_E_UNKNOWN_TENSOR_TYPE = 5,  /* Error::UnknownTensorType */
  IFX_E_INVALID_UTF8 = 6,         /* Error::InvalidUtf8 */
  IFX_E_INVALID_SHAPE = 7,        /* Error::InvalidShape */
  IFX_E_UNEXPECTED_EOF = 8,       /* Error::UnexpectedEof */
  IFX_E_TENSOR_NOT_FOUND = 9,     /* Error::TensorNotFound */
  IFX_E_INVALID_TENSOR_INDEX = 10,/* Error::InvalidTensorIndex */
  IFX_E_TENSOR_OFFSET_OVERFLOW = 11, /* Error::TensorOffsetOverflow */
  IFX_E_UNSUPPORTED_ARCH = 12,    /* Error::UnsupportedArchitecture */
  IFX_E_JSON = 13,                /* TokenizerError::Json (src/tokenizer/mod.rs:228-232) */
  IFX_E_UNSUPPORTED_TOKENIZER = 14, /* TokenizerError::UnsupportedModel */
  IFX_E_INVALID_ARG = 20,         /* a reference assert!/slice panic */
  IFX_E_KV_FULL = 21,             /* KV append past max_seq_len (src/model/forward.rs:376) */
  IFX_E_HIP = 22,                 /* a HIP runtime call failed */
  IFX_E_OOM = 23,                 /* device or host allocation failed */
  IFX_E_NAN_LOGIT = 24,           /* argmax met a NaN (src/model/forward.rs:619 unwrap) */
  IFX_E_NO_DEVICE = 25            /* no usable gfx950 device */
};

/* GGML tensor type ids (src/gguf/types.rs:70-100). */
enum {
  IFX_TYPE_F32 = 0, IFX_TYPE_F16 = 1, IFX_TYPE_Q4_0 = 2, IFX_TYPE_Q8_0 = 7,
  IFX_TYPE_Q4_K = 12, IFX_TYPE_Q6_K = 14, IFX_TYPE_Q8_K = 15
};

/* RoPE position rule of a session.
 * REFERENCE (default) reproduces the reference exactly: decode rotates q/k at
 * position 0 (src/model/forward.rs:371-372 with src/ops.rs:270) and prefill at
 * positions 0..n relative to the chunk (src/model/forward.rs:243-244).
 * ABSOLUTE rotates at the cache index (len + t). */
enum { IFX_ROPE_REFERENCE = 0, IFX_ROPE_ABSOLUTE = 1 };

const char* ifx_last_error(void);
const char* ifx_status_string(int status);

/* ---------------------------------------------------------------------------
 * Model and session — replaces src/model/{mod,cache,forward}.rs
 * ------------------------------------------------------------------------- */
typedef struct ifx_model ifx_model;
typedef struct ifx_session ifx_session;

/* Config (src/model/config.rs:5-30). */
typedef struct {
  uint32_t vocab_size;
  uint64_t hidden_size;
  uint64_t n_layers;
  uint64_t n_heads;
  uint64_t n_kv_heads;
  uint64_t head_dim;
  uint64_t intermediate_size;
  float norm_eps;
  float rope_base;
  uint64_t rope_dim;
  uint64_t context_length;
  char architecture[32];
} ifx_config;

/* Model::open (src/model/mod.rs:64-92): mmap + parse (src/gguf/weights.rs:24-32,
 * src/gguf/file.rs:57-116), Config::from_gguf (src/model/config.rs:34-84), name
 * resolution (src/model/mod.rs:34-48).  In addition every weight is uploaded to
 * HBM once, in its quantized form; nothing is dequantized to f32 in HBM. */
int ifx_model_open(const char* path, ifx_model** out);
/* Open flags (no reference counterpart).  IFX_OPEN_GGML_KQUANTS reads Q4_K
 * and Q6_K tensors in ggml's block layout (llama.cpp block_q4_K: ggml's
 * nibble-to-element order; block_q6_K: ql, qh, int8 scales, then d) instead of
 * the reference's (Q4_K group-contiguous nibbles, Q6_K d first with u8
 * scales), for GGUF files written by llama.cpp.  Q4_0, Q8_0, F32 and F16 read
 * the same either way; a Q8_K tensor is refused (IFX_E_UNKNOWN_TENSOR_TYPE). */
enum { IFX_OPEN_GGML_KQUANTS = 1 };
int ifx_model_open_ex(const char* path, uint32_t flags, ifx_model** out);
void ifx_model_close(ifx_model* model);
int ifx_model_config(const ifx_model* model, ifx_config* out);
/* Bytes of weights resident in HBM, and the stored GGUF bytes they came from. */
int ifx_model_weight_bytes(const ifx_model* model, uint64_t* device_bytes, uint64_t* gguf_bytes);

/* KvCache::new + DecodeBuffers::new (src/model/cache.rs:16-24,62-83): a device
 * KV cache of max_seq_len rows per layer, scratch and one HIP stream. */
int ifx_session_create(ifx_model* model, uint64_t max_seq_len, ifx_session** out);
/* Element type of a session's KV cache. */
enum { IFX_KV_F32 = 0, IFX_KV_F16 = 1 };
/* ifx_session_create with the KV cache stored as kv_type.  IFX_KV_F32 is the
 * reference's f32 KvCache (what ifx_session_create makes).  IFX_KV_F16 has no
 * reference counterpart: keys (after RoPE) and values are rounded to IEEE
 * binary16 (to nearest, ties to even) as they are stored, which halves the
 * cache and the attention's HBM traffic at long contexts; attention arithmetic
 * stays f32, so results differ from the reference by that rounding.
 * ifx_kv_import rounds the same way, ifx_kv_export widens exactly.  Needs
 * head_dim % 8 == 0 (IFX_E_INVALID_ARG otherwise). */
int ifx_session_create_kv(ifx_model* model, uint64_t max_seq_len, int kv_type, ifx_session** out);
void ifx_session_destroy(ifx_session* s);
int ifx_session_clear(ifx_session* s);                 /* KvCache::clear (cache.rs:26-28) */
int ifx_session_len(const ifx_session* s, uint64_t* len);  /* KvCache::len (cache.rs:31-33) */
int ifx_session_set_rope_mode(ifx_session* s, int mode);

/* Prefill path of a session.  Model::prefill (src/model/forward.rs:496-538)
 * runs chunks of at least min_rows ids (default 64; 0 = never) layer by layer
 * as dequant-to-LDS GEMMs on the fp16 matrix cores and a batched causal
 * attention, when the model is eligible (ifx_model_batched_prefill); shorter
 * chunks replay the decode step per id.  Both give the reference's semantics
 * (chunk-relative RoPE, chunk-only attention, logits of every row) within
 * f32-level rounding. */
int ifx_session_set_prefill_batch(ifx_session* s, uint64_t min_rows);
/* *eligible = 1 if every layer matrix and the output matrix have a type the
 * prefill GEMM reads (Q4_K, Q6_K, Q8_0, Q4_0) with elements inside the fp16
 * range, and the head dim is one the prefill attention is built for. */
int ifx_model_batched_prefill(const ifx_model* m, int* eligible);

/* Model::decode_step (src/model/forward.rs:543-586).  logits_out: host buffer of
 * vocab_size floats, or NULL to leave the logits on the device. */
int ifx_decode_step(ifx_session* s, uint32_t token, float* logits_out);

/* Model::prefill (src/model/forward.rs:496-538): causal over the chunk, writes
 * K/V at len..len+n, len += n.  logits_out: host [n x vocab], or NULL. */
int ifx_prefill(ifx_session* s, const uint32_t* ids, uint64_t n, float* logits_out);

/* Model::forward (src/model/forward.rs:448-482): non-causal, no cache; logits
 * for every row into host logits_out [n x vocab]. */
int ifx_forward(ifx_model* model, const uint32_t* ids, uint64_t n, float* logits_out);

/* Model::forward_last_token_logits (src/model/forward.rs:484-489): the
 * forward's last row into host logits_out [vocab].  The output head runs for
 * that row only.  n == 0 is IFX_E_INVALID_ARG (the reference's slice panics). */
int ifx_forward_last_token_logits(ifx_model* model, const uint32_t* ids, uint64_t n, float* logits_out);

/* Model::generate (src/model/forward.rs:592-612): clear, prefill, then
 * max_tokens greedy steps (argmax ties -> last index, src/model/forward.rs:615-622).
 * The argmax runs on the device; the loop runs without host round trips. */
int ifx_generate(ifx_session* s, const uint32_t* prompt, uint64_t n, uint64_t max_tokens,
                 uint32_t* out_tokens);

/* The decode half of generate: feeds `token`, then n_steps-1 of its own greedy
 * picks; out_tokens[i] = argmax of step i's logits.  len grows by n_steps. */
int ifx_decode_greedy(ifx_session* s, uint32_t token, uint64_t n_steps, uint32_t* out_tokens);

/* Sampler::sample (src/sampler.rs:28-76) for ifx_generate_sampled: temperature
 * (0: greedy argmax), top_k (0: off), top_p (1: off), and the seed of the
 * draws.  Diverges from the reference by design: the logits are shifted by
 * their maximum before exp (the reference's exp(z/T) overflows past 88) and
 * the draws come from splitmix64(seed, step) instead of rand's thread_rng, so
 * a run is reproducible.  Default: temperature 0.  No reference counterpart
 * as a C entry point: the reference passes a Sampler to its CLI loop. */
int ifx_session_set_sampler(ifx_session* s, float temperature, uint32_t top_k, float top_p, uint64_t seed);

/* ifx_generate with every generated token drawn by the session's sampler on
 * the device (three sampler launches between the logits and the state
 * update). */
int ifx_generate_sampled(ifx_session* s, const uint32_t* prompt, uint64_t n, uint64_t max_tokens,
                         uint32_t* out_tokens);

/* One-off draws from host logits[vocab] (tests): n_draws draws, draw i with
 * counter i, as generate step i would.  IFX_E_NAN_LOGIT if a logit is NaN. */
int ifx_sample_logits(const float* logits, uint32_t vocab, float temperature, uint32_t top_k, float top_p,
                      uint64_t seed, uint32_t n_draws, uint32_t* out);

/* KV state in the reference layout: k,v = [n_layers][len][n_kv_heads*head_dim]
 * f32 (src/model/cache.rs:8-24), host memory.  Import sets len. */
int ifx_kv_import(ifx_session* s, const float* k, const float* v, uint64_t len);
int ifx_kv_export(ifx_session* s, float* k, float* v, uint64_t len);

/* ---- text path: the byte-level BPE tokenizer (host only, no device) ---- */
typedef struct ifx_tokenizer ifx_tokenizer;
/* BpeTokenizer::from_file / from_json (src/tokenizer/mod.rs:61-114): a
 * Hugging Face tokenizer.json of model type "BPE".  IFX_E_IO (unreadable, not
 * UTF-8), IFX_E_JSON (malformed, a missing or mistyped field),
 * IFX_E_UNSUPPORTED_TOKENIZER (another model type). */
int ifx_tokenizer_from_file(const char* path, ifx_tokenizer** out);
int ifx_tokenizer_from_json(const char* json, uint64_t len, ifx_tokenizer** out);
void ifx_tokenizer_free(ifx_tokenizer* t);
/* Tokenizer::encode (src/tokenizer/mod.rs:196-205) of len bytes of UTF-8
 * text (IFX_E_INVALID_UTF8 otherwise): *n_ids = the id count, the first
 * min(cap, count) ids written. */
int ifx_tokenizer_encode(const ifx_tokenizer* t, const char* text, uint64_t len, uint32_t* ids, uint64_t cap,
                         uint64_t* n_ids);
/* Tokenizer::decode (src/tokenizer/mod.rs:207-225): the UTF-8 text (lossy, as
 * String::from_utf8_lossy) of n ids; *len_out = its byte length, the first
 * min(cap, length) bytes written, no terminator. */
int ifx_tokenizer_decode(const ifx_tokenizer* t, const uint32_t* ids, uint64_t n, char* text, uint64_t cap,
                         uint64_t* len_out);
/* Entries of the vocabulary (no reference counterpart; for callers sizing buffers). */
int ifx_tokenizer_vocab_size(const ifx_tokenizer* t, uint64_t* n);

/* argmax (src/model/forward.rs:615-622) of the logits of the most recent
 * step — for a prefill, of its last row: the token generate feeds next. */
int ifx_session_last_token(ifx_session* s, uint32_t* token);

/* Device time of the last ifx_decode_greedy / ifx_prefill call, measured with
 * HIP events on the session stream (milliseconds). */
int ifx_session_last_elapsed_ms(const ifx_session* s, float* ms);

/* Measurement hook (no reference counterpart; the reference has no timers):
 * n_steps greedy decode steps from `token` (launched directly), then every
 * kernel class launched back to back, once per layer or once, n_steps times
 * over, between one HIP event pair on the session stream.  Arrays of 8, one
 * per kernel class: 0 embedding gather, 1 QKV GEMV (+RMSNorm, RoPE, KV
 * append), 2 attention (chunk records + merge), 3 attn_output GEMV
 * (+residual), 4 ffn gate/up GEMV (+RMSNorm, SwiGLU), 5 ffn_down GEMV
 * (+residual), 6 output head GEMV (+RMSNorm, argmax), 7 finalize (not timed:
 * it advances the state; reported as 0).  avg_ms: mean time per launch;
 * launches: per step; bytes: stored weight bytes each launch streams
 * (attention: the f32 K/V rows it reads).  len grows by n_steps and one more
 * row must be free; scratch is left overwritten. */
int ifx_session_profile(ifx_session* s, uint32_t token, uint64_t n_steps, float* avg_ms,
                        uint64_t* launches, uint64_t* bytes);

/* Measurement hook (no reference counterpart): n_steps greedy decode steps
 * from `token`, each launched kernel by kernel with a HIP event pair around
 * every launch, so each kernel is timed in the order and cache state of a real
 * step (the captured step replays the same launches with no events between
 * them).  avg_ms[8]: the mean duration of one launch of each kernel class of
 * ifx_session_profile (class 7, finalize, is timed too).  len grows by n_steps. */
int ifx_session_profile_ordered(ifx_session* s, uint32_t token, uint64_t n_steps, float* avg_ms);

/* ---------------------------------------------------------------------------
 * Device memory and streams (plumbing for the kernel-level entry points)
 * ------------------------------------------------------------------------- */
int ifx_device_info(char* name, uint64_t name_cap, int* n_cu, uint64_t* hbm_bytes);
int ifx_malloc(void** dptr, uint64_t bytes);
int ifx_free(void* dptr);
int ifx_memcpy_h2d(void* dst, const void* src, uint64_t bytes);
int ifx_memcpy_d2h(void* dst, const void* src, uint64_t bytes);
int ifx_memcpy_d2d(void* dst, const void* src, uint64_t bytes);
int ifx_stream_synchronize(void* stream);
/* HIP event timing on a stream (NULL = library stream). */
int ifx_timer_start(void* stream);
int ifx_timer_stop(void* stream, float* ms);

/* ---------------------------------------------------------------------------
 * Dequantization — replaces gguf::dequantize_f32 (src/gguf/dequant.rs:10-31)
 * Bit-exact with the reference for F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K; the
 * same checks in the same order (UnknownTensorType, UnexpectedEof,
 * InvalidTensorIndex).  `bytes` is the raw GGUF block stream on the device.
 * ------------------------------------------------------------------------- */
int ifx_dequantize_f32(uint32_t type, uint64_t n_elements, const void* bytes, uint64_t n_bytes,
                       float* out, uint64_t n_out, void* stream);

/* ---------------------------------------------------------------------------
 * Quantized weight matrices on the device and the fused dequant-GEMV — the
 * decode (m = 1) case of ops::matmul_t (src/ops.rs:33-44) fed by
 * Weights::tensor_f32_by_index (src/gguf/weights.rs:66-74), without the f32
 * copy: y[rows] = W[rows x cols] . x[cols].
 * ------------------------------------------------------------------------- */
typedef struct ifx_tensor ifx_tensor;

/* Upload a host GGUF block stream holding a [rows x cols] matrix (row-major,
 * cols contiguous) into the device layout the GEMV kernels read. */
int ifx_tensor_upload(uint32_t type, const void* host_bytes, uint64_t n_bytes, uint64_t rows,
                      uint64_t cols, ifx_tensor** out);
/* ifx_tensor_upload with IFX_OPEN_* flags (IFX_OPEN_GGML_KQUANTS: ggml's
 * Q4_K / Q6_K block layout). */
int ifx_tensor_upload_ex(uint32_t type, const void* host_bytes, uint64_t n_bytes, uint64_t rows, uint64_t cols,
                         uint32_t flags, ifx_tensor** out);
void ifx_tensor_free(ifx_tensor* t);
int ifx_tensor_bytes(const ifx_tensor* t, uint64_t* device_bytes, uint64_t* gguf_bytes);
/* Dequantize an uploaded matrix to f32 [rows x cols] on the device (bit-exact). */
int ifx_tensor_dequant(const ifx_tensor* t, float* out, void* stream);
/* y = W x  (x: device f32 [cols], y: device f32 [rows]). */
int ifx_gemv(const ifx_tensor* w, const float* x, float* y, void* stream);
/* C[m x rows] = A[m x cols] . W^T for m >= 1 (the prefill form of matmul_t). */
int ifx_matmul_qt(const float* a, uint64_t m, const ifx_tensor* w, float* c, void* stream);
/* ifx_matmul_qt without device allocation.  No reference counterpart: for
 * callers that cannot call hipMalloc (code under HIP graph capture, serving
 * loops, harnesses that forbid allocation).  The GEMM's activation operand and
 * split-K workspace live in a fixed ~23 MiB device array that each GPU holds
 * until the process ends; m <= 16384 and m * cols <= 2^22 for the GEMM path
 * (IFX_E_INVALID_ARG beyond).  All calls on one GPU share that array: calls
 * that overlap on one GPU (two streams or threads) race.  m = 1 and matrices
 * the GEMM does not take use the GEMV, as ifx_matmul_qt does. */
int ifx_matmul_qt_noalloc(const float* a, uint64_t m, const ifx_tensor* w, float* c, void* stream);

/* ---------------------------------------------------------------------------
 * f32 operators on device buffers — replaces src/ops.rs
 * ------------------------------------------------------------------------- */
/* ops::matmul_t (src/ops.rs:33-44): C[m x n] = A[m x k] . B[n x k]^T. */
int ifx_ops_matmul_t(const float* a, const float* b, float* c, uint64_t m, uint64_t n, uint64_t k,
                     void* stream);
/* ops::rms_norm_rows (src/ops.rs:155-180), in place, x = [rows x n]. */
int ifx_ops_rms_norm_rows(float* x, const float* w, uint64_t n, uint64_t rows, float eps,
                          void* stream);
/* ops::swiglu (src/ops.rs:190-197). */
int ifx_ops_swiglu(const float* gate, const float* up, float* out, uint64_t n, void* stream);
/* ops::add_in_place (src/ops.rs:212-217). */
int ifx_ops_add_in_place(float* out, const float* b, uint64_t n, void* stream);
/* ops::softmax_rows (src/ops.rs:223-239), in place. */
int ifx_ops_softmax_rows(float* x, uint64_t rows, uint64_t cols, void* stream);
/* ops::rope (src/ops.rs:265-287), x = [seq x heads x head_dim], positions pos0..pos0+seq. */
int ifx_ops_rope(float* x, uint64_t seq, uint64_t heads, uint64_t head_dim, uint64_t rope_dim,
                 float base, uint64_t pos0, void* stream);
/* ops::embedding_lookup (src/ops.rs:246-258) over an uploaded (quantized) table:
 * out[n_ids x cols] = dequantized rows ids[i] (bit-exact). ids: device u32. */
int ifx_ops_embedding_lookup(const ifx_tensor* table, const uint32_t* ids, uint64_t n_ids,
                             float* out, void* stream);
/* argmax (src/model/forward.rs:615-622): last index of the maximum; *status_out
 * (device int) becomes IFX_E_NAN_LOGIT if a NaN is present. out: device u32. */
int ifx_ops_argmax(const float* x, uint64_t n, uint32_t* out, int* status_out, void* stream);

/* ---------------------------------------------------------------------------
 * The decode step's attention, q/k/v and residual launches as operators, on
 * caller buffers (device pointers).  A device KV cache here is head-major,
 * [n_kv_heads][max_seq][head_dim] of kv_type (IFX_KV_F32 or IFX_KV_F16), the
 * layout a session keeps.  Each call allocates its small device state, runs
 * on `stream` (NULL = the library's) and returns when its work is complete.
 * ------------------------------------------------------------------------- */
/* The decode attention of Layer::decode_step (src/model/forward.rs:383-414,
 * softmax_rows src/ops.rs:223-239): query head h (kv head h / (n_heads /
 * n_kv_heads)) of q [n_heads*head_dim] attends to cache rows 0 .. n_rows-1:
 * out[h] = sum_t softmax_t(q_h . k_t / sqrt(head_dim)) v_t, through the
 * step's launches (records of 64-row chunks, then their merge).  head_dim a
 * multiple of 4 (f32 cache) or 8 (f16) up to 256; at most 8 query heads per
 * kv head. */
int ifx_ops_attention_decode(const float* q, const void* k_cache, const void* v_cache, int kv_type, uint64_t max_seq,
                             uint64_t n_rows, uint64_t n_heads, uint64_t n_kv_heads, uint64_t head_dim, float* out,
                             void* stream);
/* ifx_ops_attention_decode, then h += W_o . attn: the attn_output projection
 * and residual add of Layer::decode_step (src/model/forward.rs:415-419), h of
 * W_o's rows.  merge_bound > 0: the step's fused form, the chunk records
 * merged inside the O projection's prologue, which loads merge_bound records
 * per kv head up front (rounded up to a multiple of 8, at most 48) and any
 * further ones in a loop; needs 8 kv heads, head dim 128, 4 or 8 query heads
 * per kv head and a Q4_K/Q6_K W_o of n_heads*head_dim = 1024*group columns
 * (IFX_E_INVALID_ARG otherwise).  merge_bound 0: the separate merge launch,
 * then the O launch the step takes.  attn_out: NULL, or a device buffer of
 * n_heads*head_dim floats for the attention output (separate form only). */
int ifx_ops_attention_decode_o(const float* q, const void* k_cache, const void* v_cache, int kv_type,
                               uint64_t max_seq, uint64_t n_rows, uint64_t n_heads, uint64_t n_kv_heads,
                               uint64_t head_dim, const ifx_tensor* w_o, float* h, uint32_t merge_bound,
                               float* attn_out, void* stream);
/* The attention of a prefill chunk (Layer::prefill, src/model/forward.rs:
 * 255-303; causal) or of Layer::forward (src/model/forward.rs:104-156;
 * causal = 0) over its own cache rows: query row t of q [n][n_heads*head_dim]
 * attends to cache rows row0 .. row0+t (causal) or row0 .. row0+n-1; out
 * [n][n_heads*head_dim].  The batched prefill's kernels; head_dim 48, 64, 96
 * or 128. */
int ifx_ops_attention_prefill(const float* q, const void* k_cache, const void* v_cache, int kv_type,
                              uint64_t max_seq, uint64_t row0, uint64_t n, uint64_t n_heads, uint64_t n_kv_heads,
                              uint64_t head_dim, int causal, float* out, void* stream);
/* h[rows] += W . x[cols]: matmul_t + add_in_place of the attn_output and
 * ffn_down projections (src/model/forward.rs:415-419,432-437).  mode 0: the
 * decode step's launch (for Q4_K/Q6_K matrices it takes, K split over 8
 * workgroup slices whose partial sums are added with atomics); mode 1: the
 * tiled launch, each row summed in one fixed order.  *path_out (optional):
 * 1 if the K-split launch ran, else 0. */
int ifx_ops_gemv_residual(const ifx_tensor* w, const float* x, float* h, int mode, int* path_out, void* stream);
/* q/k/v of one decode token (src/model/forward.rs:357-378): x_n =
 * rms_norm(x, norm_w, eps); q = Wq x_n, k = Wk x_n, v = Wv x_n; RoPE of q and
 * k at position pos (base rope_base over the first rope_dim dims of each
 * head, src/ops.rs:265-287); q -> q_out; k, v -> row `row` of the caches.
 * pos < 131072.  mode 0: the decode step's launch (for Q4_K/Q6_K matrices
 * and an f32 cache, K split over 8 slices whose RoPE-rotated partial sums are
 * added into q and the cache rows with atomics); mode 1: the tiled launch.
 * *path_out (optional): 1 if the K-split launch ran. */
int ifx_ops_qkv(const ifx_tensor* wq, const ifx_tensor* wk, const ifx_tensor* wv, const float* x, const float* norm_w,
                float eps, uint64_t head_dim, uint64_t rope_dim, float rope_base, uint64_t pos, float* q_out,
                void* k_cache, void* v_cache, int kv_type, uint64_t max_seq, uint64_t row, int mode, int* path_out,
                void* stream);

/* Fixed summation order for a session (no reference counterpart; the
 * reference adds in one order, src/ops.rs:212-217, src/model/forward.rs:
 * 419,437).  on = 1: q/k/v, attn_output and ffn_down take the tiled launches
 * and the attention merge its own launch, so two runs of the same calls give
 * bit-identical logits, tokens and draws.  on = 0 (default): the faster
 * K-split launches, whose atomic adds of partial sums can differ in the last
 * bits between runs.  Takes effect from the next step. */
int ifx_session_set_deterministic(ifx_session* s, int on);

#ifdef __cplusplus
}
#endif
#endif /* INFEROX_H */
