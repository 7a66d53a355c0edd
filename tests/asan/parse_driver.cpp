// Host-only driver for the AddressSanitizer run of the untrusted-input
// parsers (GGUF: host_gguf.cpp with the type tables of host_types.cpp; the
// tokenizer.json reader and BPE of host_tokenizer.cpp).  Test infrastructure:
// built with g++ -fsanitize=address by tests/test_asan_parsers.py.
//
// Arguments: g:<path> parses a GGUF file and walks its metadata and tensor
// byte ranges; m:<path> parses it and runs the model loader's host half
// (host_config.cpp: Config::from_gguf, the blk.N name walk, the weight shape
// plan); t:<path> loads a tokenizer.json and round-trips a sample text.
// Prints one status per argument, in order.
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../inferox_amd/csrc/host_config.h"
#include "../../inferox_amd/csrc/host_gguf.h"
#include "../../inferox_amd/csrc/ifx_common.h"

static int run_gguf(const char* path) {
  ifx::MappedFile m;
  int rc = m.open(path);
  if (rc != IFX_OK) return rc;
  ifx::GgufFile f;
  rc = ifx::gguf_parse(m.data, m.size, &f);
  if (rc != IFX_OK) return rc;
  // the getters the model loader uses, on every key, and every tensor's bytes
  for (const ifx::GgufMeta& e : f.meta) {
    uint32_t u32;
    uint64_t u64;
    float f32;
    std::string s;
    (void)f.get_u32(e.key.c_str(), &u32);
    (void)f.get_u64(e.key.c_str(), &u64);
    (void)f.get_f32(e.key.c_str(), &f32);
    (void)f.get_string(e.key.c_str(), &s);
  }
  unsigned long long sum = 0;
  for (size_t i = 0; i < f.tensors.size(); i++) {
    const uint8_t* data;
    uint64_t n;
    if (ifx::gguf_tensor_bytes(f, m, (int64_t)i, &data, &n) == IFX_OK && n) sum += data[0] + data[n - 1];
  }
  return sum == 0xffffffffffffffffull ? -1 : IFX_OK;
}

static int run_model_plan(const char* path) {
  ifx::MappedFile m;
  int rc = m.open(path);
  if (rc != IFX_OK) return rc;
  ifx::GgufFile f;
  rc = ifx::gguf_parse(m.data, m.size, &f);
  if (rc != IFX_OK) return rc;
  ifx::ModelPlan plan;
  rc = ifx::plan_model(f, &plan);
  if (rc != IFX_OK) return rc;
  uint64_t shapes[ifx::R_COUNT][2];
  rc = ifx::plan_shapes(f, &plan, shapes);
  if (rc != IFX_OK) return rc;
  // every resolved tensor's bytes, as the upload reads them
  unsigned long long sum = 0;
  for (int64_t i : plan.layers) {
    const uint8_t* data;
    uint64_t n;
    if (ifx::gguf_tensor_bytes(f, m, i, &data, &n) == IFX_OK && n) sum += data[0] + data[n - 1];
  }
  return sum == 0xffffffffffffffffull ? -1 : IFX_OK;
}

static int run_tokenizer(const char* path) {
  ifx_tokenizer* t = nullptr;
  int rc = ifx_tokenizer_from_file(path, &t);
  if (rc != IFX_OK) return rc;
  const char* text = "Hello, world!  <|endoftext|> caf\xc3\xa9 \xe2\x82\xac 123";
  std::vector<uint32_t> ids(256);
  uint64_t n = 0;
  rc = ifx_tokenizer_encode(t, text, strlen(text), ids.data(), ids.size(), &n);
  if (rc == IFX_OK) {
    std::vector<char> out(1024);
    uint64_t len = 0;
    ids.push_back(0xffffffffu);  // an id past the vocabulary decodes to nothing
    rc = ifx_tokenizer_decode(t, ids.data(), n < ids.size() ? n : ids.size(), out.data(), out.size(), &len);
  }
  ifx_tokenizer_free(t);
  return rc;
}

int main(int argc, char** argv) {
  for (int i = 1; i < argc; i++) {
    const char* a = argv[i];
    int rc = -1;
    if (!strncmp(a, "g:", 2)) rc = run_gguf(a + 2);
    else if (!strncmp(a, "m:", 2)) rc = run_model_plan(a + 2);
    else if (!strncmp(a, "t:", 2)) rc = run_tokenizer(a + 2);
    printf("%d\n", rc);
  }
  return 0;
}
