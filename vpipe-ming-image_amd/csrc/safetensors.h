// safetensors files: a little-endian u64 header length, a JSON header
// mapping each tensor name to {dtype, shape, data_offsets [begin, end)}
// relative to the byte after the header, an optional "__metadata__" map of
// strings, then the raw data. Files are memory-mapped read-only; nothing is
// copied until a caller narrows a tensor.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace ming::st {

struct Tensor {
  std::string name;
  std::string dtype;           // "BF16", "F16", "F32", "U32", ...
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  size_t bytes = 0;
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

// Bytes per element of a safetensors dtype; 0 for one this reader refuses.
size_t dtype_size(const std::string& dtype);

class File {
 public:
  File() = default;
  ~File();
  File(const File&) = delete;
  File& operator=(const File&) = delete;
  // Maps and validates `path`: header length within the file, every tensor's
  // dtype known, its offsets inside the data region and its byte count equal
  // to numel * dtype size.
  bool open(const std::string& path, std::string* why);
  const std::string& path() const { return path_; }
  const std::vector<Tensor>& tensors() const { return tensors_; }
  const std::map<std::string, std::string>& metadata() const { return meta_; }

 private:
  std::string path_;
  void* map_ = nullptr;
  size_t map_bytes_ = 0;
  std::vector<Tensor> tensors_;
  std::map<std::string, std::string> meta_;
};

// Every tensor of a checkpoint directory (all its *.safetensors files, a
// sharded diffusers checkpoint included) or of one file, by name.
class Set {
 public:
  bool open_dir(const std::string& dir, std::string* why);
  bool open_file(const std::string& path, std::string* why);
  const Tensor* find(const std::string& name) const;
  const std::vector<const Tensor*>& all() const { return order_; }
  // The metadata of the first file (adapters are one file).
  const std::map<std::string, std::string>* metadata() const {
    return files_.empty() ? nullptr : &files_.front()->metadata();
  }

 private:
  bool add(const std::string& path, std::string* why);
  std::vector<std::unique_ptr<File>> files_;
  std::map<std::string, const Tensor*> by_name_;
  std::vector<const Tensor*> order_;
};

// f32 -> bf16 as the checkpoint loader narrows (ming-dit.cc:173-181):
// round to nearest even on the bit pattern, no special case for NaN.
uint16_t f32_to_bf16_narrow(float f);
// A float tensor (BF16 copied, F16 and F32 narrowed as above) as bf16 bits.
bool to_bf16(const Tensor& t, std::vector<uint16_t>* out, std::string* why);
// A float tensor as f32 (BF16 and F16 widened exactly).
bool to_f32(const Tensor& t, std::vector<float>* out, std::string* why);

struct OutTensor {
  std::string name;
  std::string dtype;
  std::vector<int64_t> shape;
  const void* data = nullptr;
  size_t bytes = 0;
};
// Writes a safetensors file (header padded with spaces to a multiple of 8).
bool write(const std::string& path, const std::vector<OutTensor>& ts,
           const std::map<std::string, std::string>& metadata, std::string* why);

}  // namespace ming::st
