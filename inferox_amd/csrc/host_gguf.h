// host_gguf.h — GGUF parsing and the read-only file mapping (the product-side
// restatement of src/gguf/{file,tensor,value,weights}.rs).
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace ifx {

struct GgufValue {
  uint32_t type = 0;  // ValueType id (src/gguf/types.rs:7-21)
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0.0;
  std::string s;
  uint32_t item_type = 0;        // arrays: Value::Array(item type, items)
  std::vector<GgufValue> items;
};

struct GgufMeta {
  std::string key;
  GgufValue value;
};

struct GgufTensor {
  std::string name;
  std::vector<uint64_t> shape;
  uint32_t type = 0;
  uint64_t offset = 0;
  uint64_t n_elements() const;
};

struct GgufFile {
  uint32_t version = 0;
  std::vector<GgufMeta> meta;
  std::vector<GgufTensor> tensors;
  uint64_t data_offset = 0;

  const GgufValue* get(const char* key) const;
  bool get_u32(const char* key, uint32_t* v) const;
  bool get_u64(const char* key, uint64_t* v) const;
  bool get_f32(const char* key, float* v) const;
  bool get_string(const char* key, std::string* v) const;
  int64_t tensor_index(const char* name) const;
};

// Read-only mmap of a whole file (Weights::open, src/gguf/weights.rs:24-32).
struct MappedFile {
  const uint8_t* data = nullptr;
  size_t size = 0;
  int open(const char* path);
  void close();
  ~MappedFile() { close(); }
};

// GgufFile::read (src/gguf/file.rs:57-116); returns an IFX_* status.
int gguf_parse(const uint8_t* p, size_t n, GgufFile* out);

// Weights::tensor_bytes (src/gguf/weights.rs:97-112).
int gguf_tensor_bytes(const GgufFile& f, const MappedFile& m, int64_t idx, const uint8_t** data,
                      uint64_t* size);

}  // namespace ifx
