// host_tokenizer.cpp — the byte-level BPE tokenizer of the text path
// (src/tokenizer/mod.rs, src/tokenizer/bytes.rs) behind the C ABI.
//
// Loads a Hugging Face tokenizer.json the way BpeTokenizer::from_json
// (src/tokenizer/mod.rs:67-114) deserializes it: `model` must be an object
// with `type` == "BPE", `vocab` (string -> u32) and `merges` (strings "a b");
// `unk_token` is optional; `added_tokens[].content` become the special tokens;
// unknown fields are ignored, a missing required field, a wrongly typed value
// or trailing characters are a JSON error, as with serde_json.  The JSON
// reader below is this file's own (no JSON library is part of the build).
//
// Two places where the reference's behaviour depends on hash-set iteration
// order are fixed here: when two special tokens match at the same earliest
// position the longer one is taken (src/tokenizer/mod.rs:165-172 takes
// whichever the set yields first), and when two vocab entries share an id the
// later one in the file decodes (src/tokenizer/mod.rs:75-78).  Empty special
// tokens are ignored (the reference's split loop would not advance on one).
#include <stdio.h>
#include <string.h>

#include <new>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "ifx_common.h"

using namespace ifx;

namespace {

// ---------------------------------------------------------------------------
// UTF-8 helpers
// ---------------------------------------------------------------------------
void put_utf8(std::string& out, uint32_t cp) {
  if (cp < 0x80) {
    out += (char)cp;
  } else if (cp < 0x800) {
    out += (char)(0xC0 | (cp >> 6));
    out += (char)(0x80 | (cp & 0x3F));
  } else if (cp < 0x10000) {
    out += (char)(0xE0 | (cp >> 12));
    out += (char)(0x80 | ((cp >> 6) & 0x3F));
    out += (char)(0x80 | (cp & 0x3F));
  } else {
    out += (char)(0xF0 | (cp >> 18));
    out += (char)(0x80 | ((cp >> 12) & 0x3F));
    out += (char)(0x80 | ((cp >> 6) & 0x3F));
    out += (char)(0x80 | (cp & 0x3F));
  }
}

// Length of the valid UTF-8 sequence starting at p[i] (0 if invalid): the
// well-formed byte sequences of the Unicode standard, table 3-7.
size_t utf8_valid_len(const uint8_t* p, size_t n, size_t i) {
  const uint8_t b = p[i];
  auto cont = [&](size_t k) { return i + k < n && (p[i + k] & 0xC0) == 0x80; };
  if (b < 0x80) return 1;
  if (b >= 0xC2 && b <= 0xDF) return cont(1) ? 2 : 0;
  if (b >= 0xE0 && b <= 0xEF) {
    if (i + 1 >= n) return 0;
    const uint8_t c = p[i + 1];
    const bool ok = (b == 0xE0) ? (c >= 0xA0 && c <= 0xBF) : (b == 0xED) ? (c >= 0x80 && c <= 0x9F)
                                                                         : (c >= 0x80 && c <= 0xBF);
    return ok && cont(2) ? 3 : 0;
  }
  if (b >= 0xF0 && b <= 0xF4) {
    if (i + 1 >= n) return 0;
    const uint8_t c = p[i + 1];
    const bool ok = (b == 0xF0) ? (c >= 0x90 && c <= 0xBF) : (b == 0xF4) ? (c >= 0x80 && c <= 0x8F)
                                                                         : (c >= 0x80 && c <= 0xBF);
    return ok && cont(2) && cont(3) ? 4 : 0;
  }
  return 0;
}

bool utf8_valid(const char* s, size_t n) {
  const uint8_t* p = (const uint8_t*)s;
  for (size_t i = 0; i < n;) {
    const size_t l = utf8_valid_len(p, n, i);
    if (!l) return false;
    i += l;
  }
  return true;
}

// Code points of a valid UTF-8 string.
std::vector<uint32_t> code_points(const std::string& s) {
  std::vector<uint32_t> out;
  const uint8_t* p = (const uint8_t*)s.data();
  for (size_t i = 0; i < s.size();) {
    const uint8_t b = p[i];
    uint32_t cp;
    size_t l;
    if (b < 0x80) { cp = b; l = 1; }
    else if (b < 0xE0) { cp = b & 0x1F; l = 2; }
    else if (b < 0xF0) { cp = b & 0x0F; l = 3; }
    else { cp = b & 0x07; l = 4; }
    for (size_t k = 1; k < l && i + k < s.size(); k++) cp = (cp << 6) | (p[i + k] & 0x3F);
    out.push_back(cp);
    i += l;
  }
  return out;
}

// String::from_utf8_lossy: every maximal prefix of an ill-formed sequence
// becomes one U+FFFD (the Unicode "substitution of maximal subparts").
std::string utf8_lossy(const std::string& in) {
  std::string out;
  const uint8_t* p = (const uint8_t*)in.data();
  const size_t n = in.size();
  size_t i = 0;
  while (i < n) {
    const size_t l = utf8_valid_len(p, n, i);
    if (l) {
      out.append(in, i, l);
      i += l;
      continue;
    }
    // the ill-formed subpart: the lead byte plus the continuation bytes that
    // can still follow it in a well-formed sequence
    const uint8_t b = p[i];
    size_t k = 1;
    if (b >= 0xE0 && b <= 0xF4 && i + 1 < n) {
      const uint8_t c = p[i + 1];
      bool second_ok;
      if (b == 0xE0) second_ok = c >= 0xA0 && c <= 0xBF;
      else if (b == 0xED) second_ok = c >= 0x80 && c <= 0x9F;
      else if (b == 0xF0) second_ok = c >= 0x90 && c <= 0xBF;
      else if (b == 0xF4) second_ok = c >= 0x80 && c <= 0x8F;
      else second_ok = c >= 0x80 && c <= 0xBF;
      if (second_ok) {
        k = 2;
        if (b >= 0xF0 && i + 2 < n && (p[i + 2] & 0xC0) == 0x80) k = 3;
      }
    }
    out += "\xEF\xBF\xBD";
    i += k;
  }
  return out;
}

// GPT-2 byte table (src/tokenizer/bytes.rs:9-27): printable bytes map to
// themselves, the other 68 to U+0100, U+0101, ... in byte order.
struct ByteTable {
  uint32_t enc[256];
  std::unordered_map<uint32_t, uint8_t> dec;
  ByteTable() {
    uint32_t n = 0;
    for (uint32_t b = 0; b < 256; b++) {
      const bool keep = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
      enc[b] = keep ? b : 0x100 + n++;
      dec[enc[b]] = (uint8_t)b;
    }
  }
};
const ByteTable& bytes_table() {
  static const ByteTable t;
  return t;
}

// ---------------------------------------------------------------------------
// JSON (RFC 8259), as far as tokenizer.json needs it
// ---------------------------------------------------------------------------
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  std::string text;  // NUM: the literal; STR: the decoded string
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
};

struct JParser {
  const char* p;
  const char* e;
  std::string err;
  int depth = 0;

  bool fail(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool lit(const char* w) {
    const size_t n = strlen(w);
    if ((size_t)(e - p) < n || memcmp(p, w, n)) return fail("invalid literal");
    p += n;
    return true;
  }
  bool hex4(uint32_t& v) {
    if (e - p < 4) return fail("truncated \\u escape");
    v = 0;
    for (int k = 0; k < 4; k++) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return fail("invalid \\u escape");
    }
    return true;
  }
  bool str(std::string& out) {
    if (p >= e || *p != '"') return fail("expected a string");
    p++;
    out.clear();
    while (true) {
      if (p >= e) return fail("unterminated string");
      const unsigned char c = (unsigned char)*p;
      if (c == '"') {
        p++;
        return true;
      }
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') {
        out += (char)c;
        p++;
        continue;
      }
      p++;
      if (p >= e) return fail("unterminated escape");
      const char x = *p++;
      switch (x) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t u;
          if (!hex4(u)) return false;
          if (u >= 0xD800 && u <= 0xDBFF) {  // a surrogate pair
            uint32_t lo;
            if (e - p < 2 || p[0] != '\\' || p[1] != 'u') return fail("lone leading surrogate");
            p += 2;
            if (!hex4(lo)) return false;
            if (lo < 0xDC00 || lo > 0xDFFF) return fail("invalid low surrogate");
            u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
          } else if (u >= 0xDC00 && u <= 0xDFFF) {
            return fail("lone trailing surrogate");
          }
          put_utf8(out, u);
          break;
        }
        default: return fail("invalid escape");
      }
    }
  }
  bool num(std::string& out) {
    const char* s = p;
    if (p < e && *p == '-') p++;
    if (p >= e) return fail("invalid number");
    if (*p == '0') p++;
    else if (*p >= '1' && *p <= '9') while (p < e && *p >= '0' && *p <= '9') p++;
    else return fail("invalid number");
    if (p < e && *p == '.') {
      p++;
      if (p >= e || *p < '0' || *p > '9') return fail("invalid number");
      while (p < e && *p >= '0' && *p <= '9') p++;
    }
    if (p < e && (*p == 'e' || *p == 'E')) {
      p++;
      if (p < e && (*p == '+' || *p == '-')) p++;
      if (p >= e || *p < '0' || *p > '9') return fail("invalid number");
      while (p < e && *p >= '0' && *p <= '9') p++;
    }
    out.assign(s, p);
    return true;
  }
  bool value(JVal& v) {
    ws();
    if (p >= e) return fail("unexpected end of input");
    const char c = *p;
    if (c == '{' || c == '[') {
      if (++depth > 128) return fail("recursion limit exceeded");
      p++;
      ws();
      const char close = c == '{' ? '}' : ']';
      v.kind = c == '{' ? JVal::OBJ : JVal::ARR;
      if (p < e && *p == close) {
        p++;
        depth--;
        return true;
      }
      while (true) {
        if (v.kind == JVal::OBJ) {
          ws();
          std::string key;
          if (!str(key)) return false;
          ws();
          if (p >= e || *p != ':') return fail("expected ':'");
          p++;
          v.obj.emplace_back(std::move(key), JVal());
          if (!value(v.obj.back().second)) return false;
        } else {
          v.arr.emplace_back();
          if (!value(v.arr.back())) return false;
        }
        ws();
        if (p < e && *p == ',') {
          p++;
          continue;
        }
        if (p < e && *p == close) {
          p++;
          depth--;
          return true;
        }
        return fail("expected ',' or a closing bracket");
      }
    }
    if (c == '"') {
      v.kind = JVal::STR;
      return str(v.text);
    }
    if (c == 't') { v.kind = JVal::BOOL; v.b = true; return lit("true"); }
    if (c == 'f') { v.kind = JVal::BOOL; v.b = false; return lit("false"); }
    if (c == 'n') { v.kind = JVal::NUL; return lit("null"); }
    v.kind = JVal::NUM;
    return num(v.text);
  }
};

// A struct field as serde reads it: absent -> nullptr; present twice -> error.
bool field(const JVal& o, const char* name, const JVal** out, std::string& err) {
  *out = nullptr;
  for (const auto& kv : o.obj)
    if (kv.first == name) {
      if (*out) {
        err = std::string("duplicate field `") + name + "`";
        return false;
      }
      *out = &kv.second;
    }
  return true;
}

// serde's u32 from a JSON number: a non-negative integer literal in range.
bool as_u32(const JVal& v, uint32_t* out) {
  if (v.kind != JVal::NUM) return false;
  const std::string& t = v.text;
  if (t.empty() || t.find_first_of(".eE") != std::string::npos) return false;
  if (t[0] == '-') {
    if (t == "-0") { *out = 0; return true; }  // serde_json reads -0 as the integer 0
    return false;
  }
  uint64_t x = 0;
  for (char ch : t) {
    x = x * 10 + (uint64_t)(ch - '0');
    if (x > 0xFFFFFFFFull) return false;
  }
  *out = (uint32_t)x;
  return true;
}

}  // namespace

// ---------------------------------------------------------------------------
// BpeTokenizer (src/tokenizer/mod.rs:23-226)
// ---------------------------------------------------------------------------
struct ifx_tokenizer {
  std::unordered_map<std::string, uint32_t> vocab;
  std::unordered_map<uint32_t, std::string> id_to_token;
  std::unordered_map<std::string, size_t> merges;  // key: a + '\xff' + b (0xFF never occurs in UTF-8)
  std::vector<std::string> special;                // distinct, non-empty
  std::unordered_set<std::string> special_set;
  uint32_t unk_id = 0;

  // src/tokenizer/mod.rs:116-139: merge the lowest-ranked adjacent pair
  // (the leftmost on equal ranks) until none is in the merge table.
  std::vector<std::string> bpe(std::vector<std::string> pieces) const {
    if (pieces.size() < 2) return pieces;
    std::string key;
    while (true) {
      size_t best_rank = 0, best_idx = 0;
      bool found = false;
      for (size_t i = 0; i + 1 < pieces.size(); i++) {
        key.assign(pieces[i]);
        key += '\xff';
        key += pieces[i + 1];
        const auto it = merges.find(key);
        if (it != merges.end() && (!found || it->second < best_rank)) {
          best_rank = it->second;
          best_idx = i;
          found = true;
        }
      }
      if (!found) break;
      pieces[best_idx] += pieces[best_idx + 1];
      pieces.erase(pieces.begin() + (long)best_idx + 1);
    }
    return pieces;
  }

  // src/tokenizer/mod.rs:141-153
  void encode_piece(const std::string& text, std::vector<uint32_t>& ids) const {
    const ByteTable& bt = bytes_table();
    std::vector<std::string> init;
    init.reserve(text.size());
    for (unsigned char b : text) {
      std::string s;
      put_utf8(s, bt.enc[b]);
      init.push_back(std::move(s));
    }
    for (const std::string& s : bpe(std::move(init))) {
      const auto it = vocab.find(s);
      ids.push_back(it == vocab.end() ? unk_id : it->second);
    }
  }

  // src/tokenizer/mod.rs:155-193 + 196-205
  std::vector<uint32_t> encode(const std::string& text) const {
    std::vector<uint32_t> ids;
    std::vector<std::string> pieces;
    if (special.empty()) {
      pieces.push_back(text);
    } else {
      size_t at = 0;
      while (at < text.size()) {
        size_t best = std::string::npos;
        const std::string* tok = nullptr;
        for (const std::string& t : special) {
          const size_t pos = text.find(t, at);
          if (pos == std::string::npos) continue;
          if (pos < best || (pos == best && t.size() > tok->size())) {
            best = pos;
            tok = &t;
          }
        }
        if (!tok) {
          pieces.push_back(text.substr(at));
          break;
        }
        if (best > at) pieces.push_back(text.substr(at, best - at));
        pieces.push_back(*tok);
        at = best + tok->size();
      }
    }
    for (const std::string& piece : pieces) {
      if (special_set.count(piece)) {
        const auto it = vocab.find(piece);
        ids.push_back(it == vocab.end() ? unk_id : it->second);
      } else {
        encode_piece(piece, ids);
      }
    }
    return ids;
  }

  // src/tokenizer/mod.rs:207-225
  std::string decode(const uint32_t* ids, uint64_t n) const {
    const ByteTable& bt = bytes_table();
    std::string bytes;
    for (uint64_t i = 0; i < n; i++) {
      const auto it = id_to_token.find(ids[i]);
      if (it == id_to_token.end()) continue;
      for (uint32_t cp : code_points(it->second)) {
        const auto d = bt.dec.find(cp);
        if (d != bt.dec.end()) bytes += (char)d->second;
        else put_utf8(bytes, cp);  // a non-byte character: its own UTF-8 bytes
      }
    }
    return utf8_lossy(bytes);
  }
};

namespace {

int tokenizer_from_json(const char* json, size_t len, ifx_tokenizer** out) {
  if (!utf8_valid(json, len)) return set_error(IFX_E_IO, "tokenizer.json: stream did not contain valid UTF-8");
  JParser jp{json, json + len};
  JVal root;
  bool ok = jp.value(root);
  if (ok) {
    jp.ws();
    if (jp.p != jp.e) ok = jp.fail("trailing characters");
  }
  if (!ok) return set_error(IFX_E_JSON, "json error: %s at byte %zu", jp.err.c_str(), (size_t)(jp.p - json));
  std::string err;
  auto bad = [&](const std::string& what) { return set_error(IFX_E_JSON, "json error: %s", what.c_str()); };
  if (root.kind != JVal::OBJ) return bad("invalid type: expected struct TokenizerJson");
  const JVal *added = nullptr, *model = nullptr;
  if (!field(root, "added_tokens", &added, err) || !field(root, "model", &model, err)) return bad(err);
  if (!model) return bad("missing field `model`");
  if (model->kind != JVal::OBJ) return bad("invalid type: expected struct Model");
  const JVal *type = nullptr, *vocab = nullptr, *merges = nullptr, *unk = nullptr;
  if (!field(*model, "type", &type, err) || !field(*model, "vocab", &vocab, err) ||
      !field(*model, "merges", &merges, err) || !field(*model, "unk_token", &unk, err))
    return bad(err);
  if (!type) return bad("missing field `type`");
  if (!vocab) return bad("missing field `vocab`");
  if (!merges) return bad("missing field `merges`");
  if (type->kind != JVal::STR) return bad("invalid type for `type`: expected a string");
  if (vocab->kind != JVal::OBJ) return bad("invalid type for `vocab`: expected a map");
  if (merges->kind != JVal::ARR) return bad("invalid type for `merges`: expected a sequence");
  if (unk && unk->kind != JVal::STR && unk->kind != JVal::NUL) return bad("invalid type for `unk_token`");
  if (added && added->kind != JVal::ARR) return bad("invalid type for `added_tokens`: expected a sequence");

  ifx_tokenizer* t = new ifx_tokenizer();
  auto drop = [&](const std::string& what) {
    delete t;
    return bad(what);
  };
  // vocab: a later duplicate key replaces the earlier one (HashMap insert)
  for (const auto& kv : vocab->obj) {
    uint32_t id;
    if (!as_u32(kv.second, &id)) return drop("invalid value in `vocab`: expected u32");
    t->vocab[kv.first] = id;
  }
  for (const auto& kv : vocab->obj) {
    const auto it = t->vocab.find(kv.first);
    t->id_to_token[it->second] = kv.first;  // file order: the later token of a shared id decodes
  }
  // merges: "a b" (split on whitespace, the first two fields), rank = index
  for (size_t rank = 0; rank < merges->arr.size(); rank++) {
    const JVal& m = merges->arr[rank];
    if (m.kind != JVal::STR) return drop("invalid type in `merges`: expected a string");
    std::vector<std::string> parts;
    size_t i = 0;
    const std::string& s = m.text;
    while (i < s.size() && parts.size() < 2) {
      while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r' || s[i] == '\f' ||
                              s[i] == '\v'))
        i++;
      const size_t j0 = i;
      while (i < s.size() && !(s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r' || s[i] == '\f' ||
                               s[i] == '\v'))
        i++;
      if (i > j0) parts.push_back(s.substr(j0, i - j0));
    }
    if (parts.size() == 2) t->merges[parts[0] + '\xff' + parts[1]] = rank;
  }
  if (added) {
    for (const JVal& a : added->arr) {
      if (a.kind != JVal::OBJ) return drop("invalid type in `added_tokens`: expected struct AddedToken");
      const JVal* content = nullptr;
      if (!field(a, "content", &content, err)) return drop(err);
      if (!content) return drop("missing field `content`");
      if (content->kind != JVal::STR) return drop("invalid type for `content`: expected a string");
      if (!content->text.empty() && t->special_set.insert(content->text).second) t->special.push_back(content->text);
    }
  }
  if (unk && unk->kind == JVal::STR) {
    const auto it = t->vocab.find(unk->text);
    if (it != t->vocab.end()) t->unk_id = it->second;
  }
  if (type->text != "BPE") {
    delete t;
    return set_error(IFX_E_UNSUPPORTED_TOKENIZER, "unsupported tokenizer model: %s", type->text.c_str());
  }
  *out = t;
  return IFX_OK;
}

}  // namespace

extern "C" {

int ifx_tokenizer_from_json(const char* json, uint64_t len, ifx_tokenizer** out) {
  clear_error();
  if (!out || (!json && len)) return set_error(IFX_E_INVALID_ARG, "null argument");
  *out = nullptr;
  try {
    return tokenizer_from_json(json ? json : "", (size_t)len, out);
  } catch (const std::bad_alloc&) {
    return set_error(IFX_E_OOM, "out of memory reading a tokenizer");
  }
}

int ifx_tokenizer_from_file(const char* path, ifx_tokenizer** out) {
  clear_error();
  if (!path || !out) return set_error(IFX_E_INVALID_ARG, "null argument");
  *out = nullptr;
  FILE* f = fopen(path, "rb");
  if (!f) return set_error(IFX_E_IO, "io error: cannot open %s", path);
  try {
    std::string raw;
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) raw.append(buf, n);
    const bool err = ferror(f) != 0;
    fclose(f);
    f = nullptr;
    if (err) return set_error(IFX_E_IO, "io error: reading %s", path);
    return tokenizer_from_json(raw.data(), raw.size(), out);
  } catch (const std::bad_alloc&) {
    if (f) fclose(f);
    return set_error(IFX_E_OOM, "out of memory reading %s", path);
  }
}

void ifx_tokenizer_free(ifx_tokenizer* t) { delete t; }

int ifx_tokenizer_encode(const ifx_tokenizer* t, const char* text, uint64_t len, uint32_t* ids, uint64_t cap,
                         uint64_t* n_ids) {
  clear_error();
  if (!t || !n_ids || (!text && len) || (!ids && cap)) return set_error(IFX_E_INVALID_ARG, "null argument");
  if (!utf8_valid(text ? text : "", (size_t)len)) return set_error(IFX_E_INVALID_UTF8, "text is not valid UTF-8");
  const std::vector<uint32_t> v = t->encode(std::string(text ? text : "", (size_t)len));
  *n_ids = v.size();
  for (size_t i = 0; i < v.size() && i < cap; i++) ids[i] = v[i];
  return IFX_OK;
}

int ifx_tokenizer_decode(const ifx_tokenizer* t, const uint32_t* ids, uint64_t n, char* text, uint64_t cap,
                         uint64_t* len_out) {
  clear_error();
  if (!t || !len_out || (!ids && n) || (!text && cap)) return set_error(IFX_E_INVALID_ARG, "null argument");
  const std::string s = t->decode(ids, n);
  *len_out = s.size();
  if (cap) memcpy(text, s.data(), s.size() < cap ? s.size() : cap);
  return IFX_OK;
}

int ifx_tokenizer_vocab_size(const ifx_tokenizer* t, uint64_t* n) {
  if (!t || !n) return set_error(IFX_E_INVALID_ARG, "null argument");
  *n = t->vocab.size();
  return IFX_OK;
}

}  // extern "C"
