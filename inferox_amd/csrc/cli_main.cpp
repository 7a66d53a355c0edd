// cli_main.cpp — the `inferox` command (src/main.rs): with a model alone it
// prints the GGUF inspection report; with a tokenizer and a prompt it
// generates text through the device token loop.
//
//   inferox <model.gguf>                                   inspect (main.rs:91-107)
//   inferox <model.gguf> <tokenizer.json> <prompt> [max_tokens=32] [temperature=0.0]
//
// generate (main.rs:38-89): every prompt token goes through decode_step (not
// prefill), the cache holds context_length rows, then max_tokens tokens are
// picked and each is fed back through decode_step; the picks are decoded and
// printed without a trailing newline.  Temperature 0 is the greedy argmax on
// the device (ifx_decode_greedy).  Above 0 each pick is a draw from the step's
// logits by the device sampler (ifx_sample_logits: temperature softmax, no
// top-k, top-p 1, as the CLI's Sampler); the reference draws from thread_rng,
// this command from splitmix64 of a seed (IFX_SEED, else the clock) and the
// step, so a run repeats from its seed.  IFX_GGML=1 in the environment opens
// the model with IFX_OPEN_GGML_KQUANTS (a GGUF written by llama.cpp).
#include <inttypes.h>
#include <stdint.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <string>
#include <vector>

#include "host_gguf.h"
#include "ifx_common.h"

using namespace ifx;

namespace {

const char* value_type_name(uint32_t t) {  // ValueType's Display (src/gguf/types.rs:44-63)
  static const char* names[] = {"uint8", "int8",   "uint16", "int16", "uint32", "int32", "float32",
                                "bool",  "string", "array",  "uint64", "int64", "float64"};
  return t < 13 ? names[t] : "?";
}

// Rust's Display of a float: the shortest decimal that reads back as the same
// value, written out positionally (no exponent), "NaN", "inf", "-inf".
std::string rust_float(double v, bool f32) {
  if (isnan(v)) return "NaN";
  if (isinf(v)) return v > 0 ? "inf" : "-inf";
  char buf[64];
  for (int prec = 1; prec <= 17; prec++) {
    snprintf(buf, sizeof buf, "%.*e", prec - 1, v);
    if (f32 ? strtof(buf, nullptr) == (float)v : strtod(buf, nullptr) == v) break;
  }
  const char* p = buf;
  std::string sign;
  if (*p == '-') {
    sign = "-";
    p++;
  }
  std::string digits;
  while (*p && *p != 'e') {
    if (*p != '.') digits += *p;
    p++;
  }
  const int e = atoi(p + 1);  // value = d.ddd x 10^e
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  std::string out;
  if (e >= 0) {
    if ((int)digits.size() <= e + 1) {
      out = digits + std::string(e + 1 - digits.size(), '0');
    } else {
      out = digits.substr(0, e + 1) + "." + digits.substr(e + 1);
    }
  } else {
    out = "0." + std::string(-e - 1, '0') + digits;
  }
  if (out == "0" || out.find_first_not_of("0.") == std::string::npos) out = "0";
  return sign + out;
}

// Value's Display (src/gguf/value.rs:74-104)
std::string value_str(const GgufValue& v) {
  char b[64];
  switch (v.type) {
    case 0: case 2: case 4: case 10:
      snprintf(b, sizeof b, "%" PRIu64, v.u);
      return b;
    case 1: case 3: case 5: case 11:
      snprintf(b, sizeof b, "%" PRId64, v.i);
      return b;
    case 6: return rust_float(v.f, true);
    case 12: return rust_float(v.f, false);
    case 7: return v.u ? "true" : "false";
    case 8: return v.s;
    case 9: {
      std::string out = std::string(value_type_name(v.item_type)) + "[" + std::to_string(v.items.size()) + "] [";
      const size_t max_preview = 8;
      for (size_t i = 0; i < v.items.size(); i++) {
        if (i >= max_preview && v.items.size() > max_preview + 1) {
          out += ", ...";
          break;
        }
        if (i > 0) out += ", ";
        out += value_str(v.items[i]);
      }
      return out + "]";
    }
    default: return "?";
  }
}

void section(const char* title) {
  const std::string rule(72, '-');
  printf("%s\n%s\n%s\n", rule.c_str(), title, rule.c_str());
}

// inspect (src/main.rs:91-182)
int inspect(const char* path) {
  MappedFile m;
  GgufFile f;
  int rc = m.open(path);
  if (rc == IFX_OK) rc = gguf_parse(m.data, m.size, &f);
  if (rc != IFX_OK) {
    fprintf(stderr, "error: failed to open '%s': %s\n", path, ifx_last_error());
    return 1;
  }
  section("Header");
  printf("  version:     %u\n", f.version);
  printf("  n_tensors:   %zu\n", f.tensors.size());
  printf("  n_kv:        %zu\n", f.meta.size());
  char title[96];
  snprintf(title, sizeof title, "Metadata (%zu entries)", f.meta.size());
  section(title);
  for (size_t i = 0; i < f.meta.size(); i++)
    printf("  [%3zu] %-50s (%s) => %s\n", i, f.meta[i].key.c_str(), value_type_name(f.meta[i].value.type),
           value_str(f.meta[i].value).c_str());
  snprintf(title, sizeof title, "Tensors (%zu tensors)", f.tensors.size());
  section(title);
  bool all_sized = true;
  uint64_t total = 0;
  for (size_t i = 0; i < f.tensors.size(); i++) {
    const GgufTensor& t = f.tensors[i];
    std::string shape;
    for (size_t d = 0; d < t.shape.size(); d++) shape += (d ? " x " : "") + std::to_string(t.shape[d]);
    printf("  [%3zu] %s\n", i, t.name.c_str());
    printf("        type:    %s (id=%u)\n", type_name(t.type), t.type);
    printf("        shape:   [%s]\n", shape.c_str());
    printf("        elems:   %" PRIu64 "\n", t.n_elements());
    printf("        offset:  %" PRIu64 " bytes\n", t.offset);
    uint64_t sz;
    if (byte_size(t.type, t.n_elements(), &sz)) {
      printf("        size:    %" PRIu64 " bytes\n", sz);
      total += sz;
    } else {
      printf("        size:    <unknown type size>\n");
      all_sized = false;
    }
  }
  section("Layout");
  printf("  file:                 %s\n", path);
  printf("  tensor data offset:   %" PRIu64 " bytes\n", f.data_offset);
  if (all_sized) printf("  total tensor bytes:   %" PRIu64 " bytes\n", total);
  else printf("  total tensor bytes:   <unknown>\n");
  section("Raw tensor bytes (mmap)");
  if (f.tensors.empty()) {
    printf("  (no tensors)\n");
    return 0;
  }
  for (size_t i = 0; i < f.tensors.size() && i < 5; i++) {
    const uint8_t* data;
    uint64_t n;
    if (gguf_tensor_bytes(f, m, (int64_t)i, &data, &n) == IFX_OK)
      printf("  %-40s -> %" PRIu64 " bytes\n", f.tensors[i].name.c_str(), n);
    else
      printf("  %-40s -> error: %s\n", f.tensors[i].name.c_str(), ifx_last_error());
  }
  if (f.tensors.size() > 5) printf("  ... and %zu more tensor(s)\n", f.tensors.size() - 5);
  return 0;
}

// generate (src/main.rs:38-89)
int generate(const char* model_path, const char* tok_path, const char* prompt, uint64_t max_tokens,
             float temperature) {
  ifx_model* model = nullptr;
  const char* ggml_env = getenv("IFX_GGML");
  const uint32_t flags = ggml_env && strcmp(ggml_env, "1") == 0 ? (uint32_t)IFX_OPEN_GGML_KQUANTS : 0u;
  if (ifx_model_open_ex(model_path, flags, &model) != IFX_OK) {
    fprintf(stderr, "error: failed to load model '%s': %s\n", model_path, ifx_last_error());
    return 1;
  }
  ifx_tokenizer* tok = nullptr;
  if (ifx_tokenizer_from_file(tok_path, &tok) != IFX_OK) {
    fprintf(stderr, "error: failed to load tokenizer '%s': %s\n", tok_path, ifx_last_error());
    ifx_model_close(model);
    return 1;
  }
  uint64_t n_prompt = 0;
  const uint64_t plen = strlen(prompt);
  std::vector<uint32_t> ids;
  int rc = ifx_tokenizer_encode(tok, prompt, plen, nullptr, 0, &n_prompt);
  if (rc == IFX_OK) {
    ids.resize(n_prompt);
    rc = ifx_tokenizer_encode(tok, prompt, plen, ids.data(), n_prompt, &n_prompt);
  }
  ifx_config cfg;
  ifx_session* s = nullptr;
  if (rc == IFX_OK) rc = ifx_model_config(model, &cfg);
  if (rc == IFX_OK) rc = ifx_session_create(model, cfg.context_length, &s);
  const uint32_t V = rc == IFX_OK ? cfg.vocab_size : 0;
  std::vector<float> logits(V ? V : 1, 0.0f);  // DecodeBuffers start zeroed
  std::vector<uint32_t> gen;
  // the prompt: every token through decode_step (main.rs:68-73); the last
  // step's logits (or the zeroed buffer of an empty prompt) feed the first pick
  for (uint64_t i = 0; i < n_prompt && rc == IFX_OK; i++)
    rc = ifx_decode_step(s, ids[i], (temperature != 0.0f && i + 1 == n_prompt) ? logits.data() : nullptr);
  if (rc == IFX_OK && max_tokens > 0) {
    if (temperature == 0.0f) {
      uint32_t first = V - 1;  // argmax of all-zero logits: the last index
      if (n_prompt) rc = ifx_session_last_token(s, &first);
      std::vector<uint32_t> out(max_tokens);
      if (rc == IFX_OK) rc = ifx_decode_greedy(s, first, max_tokens, out.data());
      if (rc == IFX_OK) {
        gen.push_back(first);
        gen.insert(gen.end(), out.begin(), out.end() - 1);
      }
    } else {
      const char* env = getenv("IFX_SEED");
      const uint64_t seed = env ? strtoull(env, nullptr, 0) : (uint64_t)time(nullptr) ^ ((uint64_t)clock() << 32);
      for (uint64_t i = 0; i < max_tokens && rc == IFX_OK; i++) {
        uint32_t next = 0;
        rc = ifx_sample_logits(logits.data(), V, temperature, 0, 1.0f, seed + i, 1, &next);
        if (rc == IFX_OK) {
          gen.push_back(next);
          rc = ifx_decode_step(s, next, logits.data());
        }
      }
    }
  }
  if (rc != IFX_OK) {
    fprintf(stderr, "error: decode failed: %s\n", ifx_last_error());
  } else {
    uint64_t n = 0;
    ifx_tokenizer_decode(tok, gen.data(), gen.size(), nullptr, 0, &n);
    std::string text(n, '\0');
    ifx_tokenizer_decode(tok, gen.data(), gen.size(), text.data(), n, &n);
    fwrite(text.data(), 1, text.size(), stdout);
    fflush(stdout);
  }
  if (s) ifx_session_destroy(s);
  ifx_tokenizer_free(tok);
  ifx_model_close(model);
  return rc == IFX_OK ? 0 : 1;
}

// str::parse::<usize>: an optional '+', then one or more decimal digits, in range
bool parse_u64(const char* s, uint64_t* v) {
  if (*s == '+') s++;
  if (!*s) return false;
  uint64_t x = 0;
  for (const char* p = s; *p; p++) {
    if (*p < '0' || *p > '9') return false;
    const uint64_t d = (uint64_t)(*p - '0');
    if (x > (UINT64_MAX - d) / 10) return false;
    x = x * 10 + d;
  }
  *v = x;
  return true;
}

// str::parse::<f32>: a decimal number with optional sign and exponent, or
// inf / infinity / nan (any case); no blanks, no hexadecimal (which strtof
// alone would take)
bool parse_f32(const char* s, float* v) {
  if (!*s || strchr(s, 'x') || strchr(s, 'X') || strchr(s, ' ') || strchr(s, '\t') || strchr(s, '\n')) return false;
  char* end;
  *v = strtof(s, &end);
  return *end == 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: %s <model.gguf> [tokenizer.json] [prompt] [max_tokens] [temperature]\n", argv[0]);
    return 1;
  }
  if (argc < 4) return inspect(argv[1]);
  uint64_t max_tokens = 32;
  float temperature = 0.0f;
  if (argc > 4 && !parse_u64(argv[4], &max_tokens)) max_tokens = 32;
  if (argc > 5 && !parse_f32(argv[5], &temperature)) temperature = 0.0f;
  return generate(argv[1], argv[2], argv[3], max_tokens, temperature);
}
