// gguf.h -- GGUF v3 reader and writer (host).
//
// The reference reads its GGUF with offsets baked at compile time
// (src/model.cpp:78-133, include/minicpm_metadata.h) and walks the key/value
// section only to find the vocabulary (src/tokenizer.cpp:10-60, value sizes
// :275-292).  This reader parses the header, the key/value section and the
// tensor table at run time.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace mcpm {

enum GgufValueType : uint32_t {
  GGUF_UINT8 = 0, GGUF_INT8 = 1, GGUF_UINT16 = 2, GGUF_INT16 = 3, GGUF_UINT32 = 4, GGUF_INT32 = 5,
  GGUF_FLOAT32 = 6, GGUF_BOOL = 7, GGUF_STRING = 8, GGUF_ARRAY = 9, GGUF_UINT64 = 10, GGUF_INT64 = 11,
  GGUF_FLOAT64 = 12,
};

struct GgufValue {
  uint32_t type = 0;
  double num = 0.0;     // every numeric scalar, widened
  int64_t inum = 0;     // integer scalars
  std::string str;      // GGUF_STRING
  uint32_t arr_type = 0;  // GGUF_ARRAY element type
  uint64_t arr_len = 0;
  std::vector<std::string> strs;  // string arrays (kept by the reader and the writer)
};

struct GgufTensor {
  std::string name;
  std::vector<uint64_t> dims;  // dims[0] = columns (fastest), dims[1] = rows
  uint32_t type = 0;
  uint64_t offset = 0;         // from the start of the data section
  size_t bytes = 0;
  const uint8_t* data = nullptr;
};

struct GgufFile {
  uint32_t version = 0;
  uint64_t alignment = 32;
  std::map<std::string, GgufValue> kv;
  std::vector<GgufTensor> tensors;
  const GgufTensor* find(const std::string& name) const;
  bool get_int(const std::string& key, int64_t& out) const;
  bool get_float(const std::string& key, double& out) const;
  bool get_str(const std::string& key, std::string& out) const;
};

// Bytes of a tensor of `type` with dims; 0 for unknown types.
size_t gguf_tensor_bytes(uint32_t type, const std::vector<uint64_t>& dims);

// Parses an in-memory image (file contents).  Tensor data pointers point into
// `data`, which must outlive the result.  Returns false with `err` set.
bool gguf_parse(const uint8_t* data, size_t size, GgufFile& out, std::string& err);

// Writer: collect key/values and tensors, then serialise.
class GgufWriter {
 public:
  void kv_u32(const std::string& k, uint32_t v);
  void kv_f32(const std::string& k, float v);
  void kv_str(const std::string& k, const std::string& v);
  // An array of strings (as tokenizer.ggml.tokens, src/tokenizer.cpp:33-48).
  void kv_str_array(const std::string& k, const std::vector<std::string>& v);
  // Adds a tensor; its bytes are produced later by the fill callback of
  // write(), in tensor order, at the given offset of the output image.
  void add_tensor(const std::string& name, uint32_t type, const std::vector<uint64_t>& dims);
  // Lays out the image; returns its size and each tensor's absolute offset.
  size_t layout(std::vector<size_t>& abs_offsets);
  // Writes header + tensor table into `image` (size from layout()); tensor
  // bytes are left for the caller to fill at abs_offsets.
  void write_header(uint8_t* image) const;
  const std::vector<GgufTensor>& tensors() const { return tensors_; }

 private:
  std::vector<std::pair<std::string, GgufValue>> kv_;
  std::vector<GgufTensor> tensors_;
  size_t header_bytes_ = 0;
};

}  // namespace mcpm
