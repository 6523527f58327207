// Sanitizer / fuzz harness of the safetensors header parser (st_header.cpp), built on the CPU with
// g++ -fsanitize=address,undefined by tests/test_st_header_sanitized.py.
//
//   st_header_fuzz ITERATIONS SEED FILE...
//
// Each FILE is a complete .safetensors file (8-byte length + JSON header + data).  The harness
// parses every file as the library does (st_open: header length checked against the file size,
// then st_parse_header over the JSON text), then runs ITERATIONS mutations of randomly chosen
// files (byte flips, insertions and deletions of bytes and of JSON tokens, truncations, splices
// of two files, length-field rewrites) through the same path.  For every accepted header it
// checks what the parser promises: each tensor's [begin, end) lies inside the data block, its
// length is numel x element size, names are unique and the index maps each name to its entry.
// Memory errors and undefined behaviour abort through the sanitizers; a broken promise exits 1.
// Prints one summary line: files, iterations, accepted headers.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../trellis.2-stableprojectorz_amd/csrc/st_header.h"

namespace {

uint64_t g_state = 1;
uint64_t rnd() {  // xorshift64*
  g_state ^= g_state >> 12;
  g_state ^= g_state << 25;
  g_state ^= g_state >> 27;
  return g_state * 2685821657736338717ull;
}
size_t below(size_t n) { return n ? (size_t)(rnd() % n) : 0; }

bool read_file(const char* path, std::string* out) {
  FILE* f = fopen(path, "rb");
  if (!f) return false;
  char buf[65536];
  size_t n;
  out->clear();
  while ((n = fread(buf, 1, sizeof(buf), f)) > 0) out->append(buf, n);
  fclose(f);
  return true;
}

int g_failures = 0;
void broken(const char* what, const std::string& name) {
  fprintf(stderr, "broken promise: %s (%s)\n", what, name.c_str());
  ++g_failures;
}

// The library's st_open on an in-memory file image; returns true when the header is accepted.
bool open_image(const std::string& file) {
  if (file.size() < 8) return false;
  uint64_t h = 0;
  for (int k = 7; k >= 0; --k) h = (h << 8) | (uint8_t)file[k];
  if (h > (uint64_t)file.size() - 8 || h > ((uint64_t)100 << 20)) return false;
  tsc_st f;
  f.data_begin = 8 + (int64_t)h;
  f.file_size = (int64_t)file.size();
  // the parser gets exactly the header bytes, in a buffer of that size (ASan sees any overread)
  std::vector<char> text(file.begin() + 8, file.begin() + 8 + (ptrdiff_t)h);
  std::string err;
  if (!tsc::st_parse_header(&f, text.data(), text.size(), &err)) {
    if (err.empty()) broken("rejected without a message", "");
    return false;
  }
  const int64_t data = f.file_size - f.data_begin;
  if (f.names.size() != f.entries.size() || f.index.size() != f.names.size())
    broken("names, entries and index differ in size", "");
  for (size_t i = 0; i < f.names.size(); ++i) {
    const tsc_st::Entry& e = f.entries[i];
    int64_t numel = 1;
    for (int64_t d : e.shape) {
      if (d < 0) broken("negative dimension", f.names[i]);
      numel *= d;
    }
    const int size = tsc::st_dtype_size(e.dtype);
    if (size <= 0) broken("unknown dtype accepted", f.names[i]);
    if (e.begin < 0 || e.end < e.begin || e.end > data) broken("range outside the data", f.names[i]);
    if (e.end - e.begin != numel * size) broken("range length != numel x size", f.names[i]);
    auto it = f.index.find(f.names[i]);
    if (it == f.index.end() || it->second != i) broken("index does not map the name", f.names[i]);
  }
  return true;
}

const char* kTokens[] = {"{", "}", "[", "]", ",", ":", "\"", "\\", "\\u", "\\ud800", "\\udc00",
                         "-", "0", "9999999999999999999", "1e5", "true", "null", "\"dtype\"",
                         "\"shape\"", "\"data_offsets\"", "\"BF16\"", "\"F8_E5M2\"",
                         "\"__metadata__\"", " ", "\n", "\x80", "\xff"};

std::string mutate(const std::vector<std::string>& corpus) {
  std::string s = corpus[below(corpus.size())];
  const int edits = 1 + (int)below(4);
  for (int k = 0; k < edits; ++k) {
    const size_t hdr_end = s.size();
    switch (below(8)) {
      case 0:  // flip a byte
        if (!s.empty()) s[below(s.size())] ^= (char)(1 + below(255));
        break;
      case 1:  // insert a token
        s.insert(below(hdr_end + 1), kTokens[below(sizeof(kTokens) / sizeof(kTokens[0]))]);
        break;
      case 2:  // delete a run
        if (!s.empty()) {
          const size_t a = below(s.size());
          s.erase(a, 1 + below(16));
        }
        break;
      case 3:  // truncate
        s.resize(below(s.size() + 1));
        break;
      case 4: {  // splice the tail of another file
        const std::string& o = corpus[below(corpus.size())];
        const size_t a = below(s.size() + 1), b = below(o.size() + 1);
        s = s.substr(0, a) + o.substr(b);
        break;
      }
      case 5:  // duplicate a run
        if (!s.empty()) {
          const size_t a = below(s.size());
          s.insert(a, s.substr(a, 1 + below(32)));
        }
        break;
      case 6:  // rewrite the header length (keeps the text, moves the data block)
        if (s.size() >= 8) {
          uint64_t h = 0;
          for (int q = 7; q >= 0; --q) h = (h << 8) | (uint8_t)s[q];
          h += (uint64_t)(int64_t)((int)below(17) - 8);
          for (int q = 0; q < 8; ++q) s[q] = (char)(h >> (8 * q));
        }
        break;
      default:  // replace a digit run inside the header
        if (s.size() > 8) {
          const size_t a = 8 + below(s.size() - 8);
          if (s[a] >= '0' && s[a] <= '9') s[a] = (char)('0' + below(10));
        }
        break;
    }
  }
  return s;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 4) {
    fprintf(stderr, "usage: %s ITERATIONS SEED FILE...\n", argv[0]);
    return 2;
  }
  const long iters = atol(argv[1]);
  g_state = (uint64_t)atoll(argv[2]) * 0x9E3779B97F4A7C15ull + 1;
  std::vector<std::string> corpus;
  long accepted = 0;
  for (int i = 3; i < argc; ++i) {
    std::string s;
    if (!read_file(argv[i], &s)) {
      fprintf(stderr, "cannot read %s\n", argv[i]);
      return 2;
    }
    accepted += open_image(s);
    corpus.push_back(std::move(s));
  }
  const long seeds_accepted = accepted;
  for (long it = 0; it < iters; ++it) accepted += open_image(mutate(corpus));
  printf("files %zu (accepted %ld) iterations %ld accepted %ld failures %d\n", corpus.size(),
         seeds_accepted, iters, accepted - seeds_accepted, g_failures);
  return g_failures ? 1 : 0;
}
