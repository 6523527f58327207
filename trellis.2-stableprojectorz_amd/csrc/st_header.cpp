// Safetensors header parser (declared in st_header.h): a small recursive-descent JSON reader
// (strings with escapes, integers, arrays, objects, literals) and the checks of every entry.
// Host-only C++; built into the library and, with -fsanitize=address,undefined, into the fuzz
// harness tests/fuzz/st_header_fuzz.cpp.

#include "st_header.h"

#include <stdint.h>
#include <string.h>

#include <string>
#include <vector>

namespace tsc {
namespace {

// True when [s, s + n) is well-formed UTF-8 (RFC 3629: no overlong forms, no surrogates, nothing
// past U+10FFFF).  The reference format's reader decodes the header as UTF-8 text before it parses
// the JSON, so a header that is not UTF-8 is rejected as a whole.
bool valid_utf8(const char* s, size_t n) {
  const unsigned char* u = (const unsigned char*)s;
  size_t i = 0;
  while (i < n) {
    const unsigned c = u[i];
    if (c < 0x80) { ++i; continue; }
    int len;
    unsigned cp, min;
    if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; min = 0x80; }
    else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; min = 0x800; }
    else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; min = 0x10000; }
    else return false;
    if (n - i < (size_t)len) return false;
    for (int k = 1; k < len; ++k) {
      if ((u[i + k] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (u[i + k] & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp < 0xE000)) return false;
    i += (size_t)len;
  }
  return true;
}

struct Json {
  const char* start;
  const char* p;
  const char* end;
  std::string err;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool peek(char c) {
    ws();
    return p < end && *p == c;
  }
  bool expect(char c) {
    if (peek(c)) {
      ++p;
      return true;
    }
    err = std::string("expected '") + c + "' at byte " + std::to_string(p - start);
    return false;
  }
  static void utf8(unsigned v, std::string* out) {
    if (v < 0x80) {
      out->push_back((char)v);
    } else if (v < 0x800) {
      out->push_back((char)(0xC0 | (v >> 6)));
      out->push_back((char)(0x80 | (v & 0x3F)));
    } else if (v < 0x10000) {
      out->push_back((char)(0xE0 | (v >> 12)));
      out->push_back((char)(0x80 | ((v >> 6) & 0x3F)));
      out->push_back((char)(0x80 | (v & 0x3F)));
    } else {
      out->push_back((char)(0xF0 | (v >> 18)));
      out->push_back((char)(0x80 | ((v >> 12) & 0x3F)));
      out->push_back((char)(0x80 | ((v >> 6) & 0x3F)));
      out->push_back((char)(0x80 | (v & 0x3F)));
    }
  }
  bool hex4(unsigned* v) {
    if (end - p < 4) return false;
    *v = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = *p++;
      *v <<= 4;
      if (h >= '0' && h <= '9') *v |= (unsigned)(h - '0');
      else if (h >= 'a' && h <= 'f') *v |= (unsigned)(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') *v |= (unsigned)(h - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string* out) {
    if (!expect('"')) return false;
    out->clear();
    while (p < end && *p != '"') {
      const char c = *p++;
      if ((unsigned char)c < 0x20) { err = "control character in a string"; return false; }
      if (c != '\\') {
        out->push_back(c);
        continue;
      }
      if (p >= end) break;
      const char e = *p++;
      switch (e) {
        case '"': out->push_back('"'); break;
        case '\\': out->push_back('\\'); break;
        case '/': out->push_back('/'); break;
        case 'b': out->push_back('\b'); break;
        case 'f': out->push_back('\f'); break;
        case 'n': out->push_back('\n'); break;
        case 'r': out->push_back('\r'); break;
        case 't': out->push_back('\t'); break;
        case 'u': {
          unsigned v;
          if (!hex4(&v)) { err = "bad \\u escape"; return false; }
          if (v >= 0xDC00 && v < 0xE000) { err = "lone low surrogate"; return false; }
          if (v >= 0xD800 && v < 0xDC00) {  // surrogate pair
            unsigned lo;
            if (end - p < 6 || p[0] != '\\' || p[1] != 'u') { err = "lone surrogate"; return false; }
            p += 2;
            if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) { err = "bad surrogate pair"; return false; }
            v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(v, out);
          break;
        }
        default: err = "bad escape"; return false;
      }
    }
    if (p >= end) { err = "unterminated string"; return false; }
    ++p;
    return true;
  }
  bool integer(int64_t* out) {
    ws();
    bool neg = false;
    if (p < end && *p == '-') { neg = true; ++p; }
    if (p >= end || *p < '0' || *p > '9') { err = "expected an integer"; return false; }
    int64_t v = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      if (v > (INT64_MAX - 9) / 10) { err = "integer overflow"; return false; }
      v = v * 10 + (*p++ - '0');
    }
    if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) { err = "expected an integer"; return false; }
    *out = neg ? -v : v;
    return true;
  }
  bool int_array(std::vector<int64_t>* out) {
    out->clear();
    if (!expect('[')) return false;
    if (peek(']')) { ++p; return true; }
    for (;;) {
      int64_t v;
      if (!integer(&v)) return false;
      out->push_back(v);
      if (peek(',')) { ++p; continue; }
      return expect(']');
    }
  }
  // Skips one JSON value of any kind (unknown entry fields).
  bool skip(int depth = 0) {
    if (depth > 64) { err = "nesting too deep"; return false; }
    ws();
    if (p >= end) { err = "unexpected end of header"; return false; }
    if (*p == '"') {
      std::string s;
      return string(&s);
    }
    if (*p == '{' || *p == '[') {
      const char close = *p == '{' ? '}' : ']';
      const bool obj = *p == '{';
      ++p;
      if (peek(close)) { ++p; return true; }
      for (;;) {
        if (obj) {
          std::string k;
          if (!string(&k) || !expect(':')) return false;
        }
        if (!skip(depth + 1)) return false;
        if (peek(',')) { ++p; continue; }
        return expect(close);
      }
    }
    for (const char* lit : {"true", "false", "null"}) {
      const size_t n = strlen(lit);
      if ((size_t)(end - p) >= n && !memcmp(p, lit, n)) {
        p += n;
        return true;
      }
    }
    // a number: sign, digits, fraction, exponent
    const char* s = p;
    while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' ||
                       *p == '+' || *p == '-'))
      ++p;
    if (p == s) { err = "unexpected character at byte " + std::to_string(p - start); return false; }
    return true;
  }
};

// Element size of each TSC_ST_* code; the names are the header's dtype strings.
struct DtypeInfo {
  const char* name;
  int size;
};
constexpr DtypeInfo kDtypes[] = {{"F32", 4}, {"F16", 2},  {"BF16", 2},   {"F64", 8},     {"I64", 8},
                                 {"I32", 4}, {"I16", 2},  {"I8", 1},     {"U8", 1},      {"BOOL", 1},
                                 {"U16", 2}, {"U32", 4},  {"U64", 8},    {"F8_E4M3", 1}, {"F8_E5M2", 1}};
constexpr int kNumDtypes = (int)(sizeof(kDtypes) / sizeof(kDtypes[0]));
static_assert(kNumDtypes == kStNumDtypes, "dtype table matches enum tsc_st_dtype");

int dtype_code(const std::string& s) {
  for (int i = 0; i < kNumDtypes; ++i)
    if (s == kDtypes[i].name) return i;
  return -1;
}

}  // namespace

const char* st_dtype_name(int code) { return code >= 0 && code < kNumDtypes ? kDtypes[code].name : ""; }
int st_dtype_size(int code) { return code >= 0 && code < kNumDtypes ? kDtypes[code].size : 0; }

bool st_parse_header(tsc_st* f, const char* text, size_t len, std::string* err) {
  const int64_t data_bytes = f->file_size - f->data_begin;
  Json j{text, text, text + len, {}};
  auto bad = [&](const std::string& what) {
    *err = what;
    return false;
  };
  if (!valid_utf8(text, len)) return bad("header is not UTF-8");
  if (!j.expect('{')) return bad(j.err);
  if (j.peek('}')) {
    ++j.p;
  } else {
    for (;;) {
      std::string key;
      if (!j.string(&key) || !j.expect(':')) return bad(j.err);
      if (key == "__metadata__") {
        // string -> string map (weights.ts:94); other value types are rejected
        if (!j.expect('{')) return bad(j.err);
        if (j.peek('}')) {
          ++j.p;
        } else {
          for (;;) {
            std::string k, v;
            if (!j.string(&k) || !j.expect(':') || !j.string(&v))
              return bad("__metadata__: " + j.err);
            f->metadata.emplace_back(std::move(k), std::move(v));
            if (j.peek(',')) { ++j.p; continue; }
            if (!j.expect('}')) return bad(j.err);
            break;
          }
        }
      } else {
        tsc_st::Entry e;
        bool have_dtype = false, have_shape = false, have_offsets = false;
        if (!j.expect('{')) return bad(j.err);
        if (!j.peek('}')) {
          for (;;) {
            std::string field;
            if (!j.string(&field) || !j.expect(':')) return bad(j.err);
            if (field == "dtype") {
              std::string d;
              if (!j.string(&d)) return bad(j.err);
              e.dtype = dtype_code(d);
              if (e.dtype < 0) return bad("unsupported dtype \"" + d + "\" of " + key);
              have_dtype = true;
            } else if (field == "shape") {
              if (!j.int_array(&e.shape)) return bad("shape of " + key + ": " + j.err);
              have_shape = true;
            } else if (field == "data_offsets") {
              std::vector<int64_t> o;
              if (!j.int_array(&o) || o.size() != 2) return bad("data_offsets of " + key);
              e.begin = o[0];
              e.end = o[1];
              have_offsets = true;
            } else if (!j.skip()) {
              return bad(j.err);
            }
            if (j.peek(',')) { ++j.p; continue; }
            break;
          }
        }
        if (!j.expect('}')) return bad(j.err);
        if (!have_dtype || !have_shape || !have_offsets) return bad("incomplete entry " + key);
        int64_t numel = 1;
        for (int64_t d : e.shape) {
          if (d < 0 || (d && numel > INT64_MAX / 8 / d)) return bad("bad shape of " + key);
          numel *= d;
        }
        if (e.begin < 0 || e.end < e.begin || e.end > data_bytes ||
            e.end - e.begin != numel * kDtypes[e.dtype].size)
          return bad("data_offsets of " + key + " do not match its shape, dtype and the file size");
        if (f->index.count(key)) return bad("duplicate tensor " + key);
        f->index.emplace(key, f->names.size());
        f->names.push_back(std::move(key));
        f->entries.push_back(std::move(e));
      }
      if (j.peek(',')) { ++j.p; continue; }
      if (!j.expect('}')) return bad(j.err);
      break;
    }
  }
  j.ws();
  if (j.p != j.end) return bad("trailing bytes after the header object");
  return true;
}


}  // namespace tsc
