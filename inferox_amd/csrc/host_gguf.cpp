// host_gguf.cpp — GGUF parser and file mapping.
#include "host_gguf.h"

#include <fcntl.h>

#include <algorithm>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "ifx_common.h"

namespace ifx {

uint64_t GgufTensor::n_elements() const {
  uint64_t n = 1;
  for (uint64_t d : shape) n *= d;
  return n;
}

const GgufValue* GgufFile::get(const char* key) const {
  for (const GgufMeta& m : meta)
    if (m.key == key) return &m.value;
  return nullptr;
}

// Integer getters cast like Rust `as` (src/gguf/file.rs:142-169).
static bool as_int(const GgufValue* v, int64_t* out) {
  if (!v) return false;
  switch (v->type) {
    case 0: case 2: case 4: case 10: *out = (int64_t)v->u; return true;
    case 1: case 3: case 5: case 11: *out = v->i; return true;
    default: return false;
  }
}

bool GgufFile::get_u32(const char* key, uint32_t* v) const {
  int64_t x;
  if (!as_int(get(key), &x)) return false;
  *v = (uint32_t)x;
  return true;
}

bool GgufFile::get_u64(const char* key, uint64_t* v) const {
  int64_t x;
  if (!as_int(get(key), &x)) return false;
  *v = (uint64_t)x;
  return true;
}

// GgufFile::get_f32 (src/gguf/file.rs:172-186).
bool GgufFile::get_f32(const char* key, float* v) const {
  const GgufValue* g = get(key);
  if (!g) return false;
  if (g->type == 6 || g->type == 12) { *v = (float)g->f; return true; }
  int64_t x;
  if (!as_int(g, &x)) return false;
  bool is_unsigned = g->type == 0 || g->type == 2 || g->type == 4 || g->type == 10;
  *v = is_unsigned ? (float)g->u : (float)x;
  return true;
}

bool GgufFile::get_string(const char* key, std::string* v) const {
  const GgufValue* g = get(key);
  if (!g || g->type != 8) return false;
  *v = g->s;
  return true;
}

int64_t GgufFile::tensor_index(const char* name) const {
  for (size_t i = 0; i < tensors.size(); i++)
    if (tensors[i].name == name) return (int64_t)i;
  return -1;
}

int MappedFile::open(const char* path) {
  close();
  int fd = ::open(path, O_RDONLY);
  if (fd < 0) return set_error(IFX_E_IO, "cannot open %s", path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return set_error(IFX_E_IO, "cannot stat %s", path);
  }
  size = (size_t)st.st_size;
  if (size) {
    void* p = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      ::close(fd);
      size = 0;
      return set_error(IFX_E_IO, "mmap of %s failed", path);
    }
    data = (const uint8_t*)p;
  }
  ::close(fd);
  return IFX_OK;
}

void MappedFile::close() {
  if (data) munmap((void*)data, size);
  data = nullptr;
  size = 0;
}

namespace {

struct Reader {
  const uint8_t* p;
  size_t n, pos = 0;
  // read_exact past the end is an io::Error in the reference
  int bytes(void* dst, size_t k) {
    if (k > n - pos) return set_error(IFX_E_IO, "unexpected end of file at byte %zu", pos);
    memcpy(dst, p + pos, k);
    pos += k;
    return IFX_OK;
  }
  template <class T>
  int get(T* v) { return bytes(v, sizeof(T)); }
};

bool valid_utf8(const uint8_t* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    uint8_t c = s[i];
    size_t len;
    uint32_t cp;
    if (c < 0x80) { i++; continue; }
    if ((c & 0xe0) == 0xc0) { len = 2; cp = c & 0x1f; }
    else if ((c & 0xf0) == 0xe0) { len = 3; cp = c & 0x0f; }
    else if ((c & 0xf8) == 0xf0) { len = 4; cp = c & 0x07; }
    else return false;
    if (i + len > n) return false;
    for (size_t k = 1; k < len; k++) {
      if ((s[i + k] & 0xc0) != 0x80) return false;
      cp = (cp << 6) | (s[i + k] & 0x3fu);
    }
    if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
        cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff))
      return false;
    i += len;
  }
  return true;
}

// read_string (src/gguf/value.rs:108-113)
int read_string(Reader& r, std::string* out) {
  uint64_t len;
  IFX_TRY(r.get(&len));
  if (len > r.n - r.pos) return set_error(IFX_E_IO, "string of %llu bytes past end of file", (unsigned long long)len);
  if (!valid_utf8(r.p + r.pos, len)) return set_error(IFX_E_INVALID_UTF8, "invalid utf-8 string");
  out->assign((const char*)r.p + r.pos, len);
  r.pos += len;
  return IFX_OK;
}

// Value::read (src/gguf/value.rs:45-71)
int read_value(Reader& r, uint32_t type, GgufValue* v) {
  v->type = type;
  switch (type) {
    case 0: { uint8_t x; IFX_TRY(r.get(&x)); v->u = x; return IFX_OK; }
    case 1: { int8_t x; IFX_TRY(r.get(&x)); v->i = x; return IFX_OK; }
    case 2: { uint16_t x; IFX_TRY(r.get(&x)); v->u = x; return IFX_OK; }
    case 3: { int16_t x; IFX_TRY(r.get(&x)); v->i = x; return IFX_OK; }
    case 4: { uint32_t x; IFX_TRY(r.get(&x)); v->u = x; return IFX_OK; }
    case 5: { int32_t x; IFX_TRY(r.get(&x)); v->i = x; return IFX_OK; }
    case 6: { float x; IFX_TRY(r.get(&x)); v->f = x; return IFX_OK; }
    case 7: { uint8_t x; IFX_TRY(r.get(&x)); v->u = x != 0; return IFX_OK; }
    case 8: return read_string(r, &v->s);
    case 9: {
      uint32_t it;
      uint64_t n;
      IFX_TRY(r.get(&it));
      if (it > 12) return set_error(IFX_E_UNKNOWN_VALUE_TYPE, "unknown array item type %u", it);
      IFX_TRY(r.get(&n));
      // every item takes at least one byte: a longer count runs past the end,
      // which the reference meets as an io error while reading the items
      if (n > r.n - r.pos) return set_error(IFX_E_IO, "unexpected end of file in an array of %llu items",
                                            (unsigned long long)n);
      v->item_type = it;
      // grown item by item from a capped reservation (src/gguf/value.rs:60): a
      // count the file cannot back ends in an io error, not in a huge allocation
      v->items.reserve(std::min<uint64_t>(n, 1u << 20));
      for (uint64_t k = 0; k < n; k++) {
        v->items.emplace_back();
        IFX_TRY(read_value(r, it, &v->items.back()));
      }
      return IFX_OK;
    }
    case 10: { uint64_t x; IFX_TRY(r.get(&x)); v->u = x; return IFX_OK; }
    case 11: { int64_t x; IFX_TRY(r.get(&x)); v->i = x; return IFX_OK; }
    case 12: { double x; IFX_TRY(r.get(&x)); v->f = x; return IFX_OK; }
    default: return set_error(IFX_E_UNKNOWN_VALUE_TYPE, "unknown metadata value type %u", type);
  }
}

}  // namespace

int gguf_parse(const uint8_t* p, size_t n, GgufFile* out) {
  Reader r{p, n};
  uint8_t magic[4];
  IFX_TRY(r.bytes(magic, 4));
  if (memcmp(magic, "GGUF", 4) != 0)
    return set_error(IFX_E_INVALID_MAGIC, "invalid magic %02x%02x%02x%02x", magic[0], magic[1], magic[2], magic[3]);
  IFX_TRY(r.get(&out->version));
  if (out->version != 2 && out->version != 3)
    return set_error(IFX_E_UNSUPPORTED_VERSION, "unsupported GGUF version %u", out->version);
  uint64_t n_tensors, n_kv;
  IFX_TRY(r.get(&n_tensors));
  IFX_TRY(r.get(&n_kv));
  if (n_kv > n || n_tensors > n) return set_error(IFX_E_IO, "counts exceed the file size");
  // capped reservations, entries appended as they are read (src/gguf/file.rs:94,105)
  out->meta.reserve(std::min<uint64_t>(n_kv, 1u << 20));
  for (uint64_t k = 0; k < n_kv; k++) {
    out->meta.emplace_back();
    GgufMeta& m = out->meta.back();
    IFX_TRY(read_string(r, &m.key));
    uint32_t type;
    IFX_TRY(r.get(&type));
    if (type > 12) return set_error(IFX_E_UNKNOWN_VALUE_TYPE, "unknown metadata value type %u", type);
    IFX_TRY(read_value(r, type, &m.value));
  }
  out->tensors.reserve(std::min<uint64_t>(n_tensors, 1u << 20));
  for (uint64_t k = 0; k < n_tensors; k++) {  // TensorInfo::read (src/gguf/tensor.rs:52-75)
    out->tensors.emplace_back();
    GgufTensor& t = out->tensors.back();
    IFX_TRY(read_string(r, &t.name));
    uint32_t n_dims;
    IFX_TRY(r.get(&n_dims));
    if (n_dims > 4) return set_error(IFX_E_INVALID_SHAPE, "tensor %s has %u dims", t.name.c_str(), n_dims);
    t.shape.resize(n_dims);
    for (uint32_t d = 0; d < n_dims; d++) IFX_TRY(r.get(&t.shape[d]));
    IFX_TRY(r.get(&t.type));
    if (!type_known(t.type)) return set_error(IFX_E_UNKNOWN_TENSOR_TYPE, "unknown tensor type %u", t.type);
    IFX_TRY(r.get(&t.offset));
  }
  out->data_offset = (r.pos + 31) / 32 * 32;  // fixed 32-byte alignment (src/gguf/file.rs:112-116)
  return IFX_OK;
}

int gguf_tensor_bytes(const GgufFile& f, const MappedFile& m, int64_t idx, const uint8_t** data,
                      uint64_t* size) {
  if (idx < 0 || (uint64_t)idx >= f.tensors.size())
    return set_error(IFX_E_INVALID_TENSOR_INDEX, "tensor index %lld", (long long)idx);
  const GgufTensor& t = f.tensors[idx];
  uint64_t sz;
  if (!byte_size(t.type, t.n_elements(), &sz))
    return set_error(IFX_E_UNKNOWN_TENSOR_TYPE, "tensor %s: unknown type %u", t.name.c_str(), t.type);
  uint64_t start = f.data_offset + t.offset;
  if (start < f.data_offset) return set_error(IFX_E_TENSOR_OFFSET_OVERFLOW, "offset overflow");
  uint64_t end = start + sz;
  if (end < start) return set_error(IFX_E_TENSOR_OFFSET_OVERFLOW, "size overflow");
  if (end > m.size) return set_error(IFX_E_UNEXPECTED_EOF, "tensor %s ends past the file", t.name.c_str());
  *data = m.data + start;
  *size = sz;
  return IFX_OK;
}

}  // namespace ifx
