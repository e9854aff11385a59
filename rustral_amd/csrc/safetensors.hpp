// safetensors.hpp -- the safetensors reader shared by the host loaders
// (safetensors.cpp) and the loaders that copy straight into device memory
// (weights.hip).  Host code only.
//
// File format: 8-byte little-endian header length N, N bytes of JSON
// {"<name>": {"dtype": "F32", "shape": [..], "data_offsets": [begin, end]},
//  ..., "__metadata__": {"<key>": "<value>"}}, then the data section;
// offsets are relative to its start.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "../../include/rustral_model.h"

namespace rkv {
namespace st {

struct Tensor {
  std::string name, dtype;
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;  // byte range in the data section
};

// A file mapped read-only, its header parsed.  open() checks every entry:
// dtype a string, shape non-negative integers, data_offsets two integers
// with begin <= end <= the data section, and end - begin equal to the
// element count times the element size for the dtypes it knows (F64, F32,
// F16, BF16, I64, I32, I16, I8, U8, BOOL).
struct File {
  const uint8_t* data = nullptr;
  uint64_t data_len = 0;
  std::vector<Tensor> tensors;  // header order; __metadata__ is not a tensor
  void* map = nullptr;
  size_t map_len = 0;
  File() = default;
  File(const File&) = delete;
  File& operator=(const File&) = delete;
  ~File();
  const Tensor* find(const std::string& name) const;
};

std::unique_ptr<File> open(const char* path, std::string& err);

struct Want {
  std::string name;
  std::vector<int64_t> shape;
};

// The strict rules of the reference's load_model
// (crates/runtime/src/model_io.rs:36-105): every wanted name present
// ("missing keys: ..."), no other tensor in the file ("unexpected extra
// keys: ..."), each shape equal ("shape mismatch for ..."), dtype F32
// ("dtype mismatch for ...").  found[i] is the tensor of want[i].
bool match(const File& f, const std::vector<Want>& want, std::vector<const Tensor*>& found,
           std::string& err);

// The decoder's names and shapes in parameter order, with each one's float
// offset into the packed parameter array.
std::vector<Want> decoder_layout(const rkv_decoder_config& c, std::vector<int64_t>* offsets);

std::string shape_str(const std::vector<int64_t>& s);

}  // namespace st
}  // namespace rkv

// The C ABI's opaque handle (include/rustral_model.h).
struct rkv_st_file {
  std::unique_ptr<rkv::st::File> f;
};
