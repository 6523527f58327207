// Safetensors header parsing: host-only C++ (no HIP), shared by the library (safetensors.hip) and
// the sanitizer / fuzz harness under tests/fuzz.  The header is untrusted input: an 8-byte
// little-endian length H, then H bytes of JSON
//   {"name": {"dtype": "BF16", "shape": [..], "data_offsets": [begin, end]}, ...,
//    "__metadata__": {"key": "value", ...}}
// (the format SafetensorsFile reads, src/runtime/weights.ts:67-99).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

struct tsc_st {
  int fd = -1;
  int64_t data_begin = 0;  // file offset of the data block (8 + header length)
  int64_t file_size = 0;
  struct Entry {
    int32_t dtype = 0;  // TSC_ST_* code
    std::vector<int64_t> shape;
    int64_t begin = 0, end = 0;  // relative to the data block
  };
  std::vector<std::string> names;  // header order
  std::vector<Entry> entries;      // parallel to names
  std::unordered_map<std::string, size_t> index;
  std::vector<std::pair<std::string, std::string>> metadata;
};

namespace tsc {

// Number of safetensors dtype codes (TSC_ST_F32 .. TSC_ST_F8_E5M2) and each code's header name and
// element size.
constexpr int kStNumDtypes = 15;
const char* st_dtype_name(int code);
int st_dtype_size(int code);

// Parses the JSON header text[0, len) into f (f->file_size and f->data_begin must be set: every
// tensor's byte range must lie inside the data block).  Returns true, or false with a message in
// *err.  Rejects malformed JSON, unknown dtypes, missing fields, shapes whose element count
// overflows, offsets that disagree with shape x element size or lie outside the data block,
// duplicate names, non-string metadata values and anything after the header object.
bool st_parse_header(tsc_st* f, const char* text, size_t len, std::string* err);

}  // namespace tsc
