// The bounded GGUF v3 header reader (gguf/gguf.go) and ConfigFrom
// (config.go): host code only, no HIP, so that it also builds on its own with
// the address and undefined-behaviour sanitizers (tests/test_gguf_sanitized.py).
#pragma once

#include <stdint.h>

#include <functional>
#include <map>
#include <string>
#include <vector>

#include "errors.h"

namespace llm {

namespace gguf {

// Bounds on a header, gguf/gguf.go:18-26.
constexpr uint64_t MaxTensors = 1 << 16, MaxKV = 1 << 16, MaxString = 1 << 24, MaxArray = 1 << 22,
                   MaxHeader = 256ull << 20, MaxDims = 4, MaxAlignment = 1 << 20;

enum Kind { K_UINT, K_INT, K_FLOAT, K_STRING, K_BOOL, K_ARRAY };

struct Value {
  Kind kind = K_UINT;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0;
  bool b = false;
  std::string s;
  uint64_t n = 0;  // array length (elements are not kept: nothing reads them)
};

struct Tensor {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  uint64_t offset = 0, size = 0;
};

struct File {
  uint32_t version = 0;
  std::map<std::string, Value> meta;
  std::vector<Tensor> tensors;
  std::map<std::string, size_t> by_name;
  uint64_t data_offset = 0, alignment = 32, size = 0;
};

using ReaderAt = std::function<int64_t(void* dst, uint64_t n, uint64_t off)>;

// gguf.Type.BlockSize, gguf/gguf.go:72-92.
bool block_size(uint32_t t, uint64_t* elems, uint64_t* bytes);
// Parse, gguf/gguf.go:292-407: the header of a file of `size` bytes read
// through r; *kind is the LLM_GGUF_* class of a refusal.
int parse(ReaderAt r, uint64_t size, File* f, int* kind);
// File.Uint / Float / Str, gguf/gguf.go:410-432.
bool meta_uint(const File& f, const std::string& k, uint64_t* v);
bool meta_float(const File& f, const std::string& k, double* v);
bool meta_str(const File& f, const std::string& k, std::string* v);

}  // namespace gguf

// ConfigFrom, config.go:29-73.
int config_from(const gguf::File& f, llmhip_config* c);

}  // namespace llm

struct llm_gguf {
  llm::gguf::File f;
};

namespace llm {
// The header of the open file fd (read with pread), as llm_gguf_parse_file.
int parse_fd(int fd, llm_gguf** out, int* kind);
}  // namespace llm
