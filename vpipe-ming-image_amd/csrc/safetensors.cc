// safetensors reader (mmap) and writer for checkpoints, packs and adapters.
#include "safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <filesystem>
#include <fstream>

#include "json.h"

namespace ming::st {

namespace fs = std::filesystem;

size_t dtype_size(const std::string& d) {
  if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
  if (d == "F32" || d == "U32" || d == "I32") return 4;
  if (d == "F64" || d == "I64" || d == "U64") return 8;
  if (d == "U8" || d == "I8" || d == "BOOL") return 1;
  return 0;
}

File::~File() {
  if (map_) munmap(map_, map_bytes_);
}

bool File::open(const std::string& path, std::string* why) {
  auto no = [&](const std::string& m) {
    if (why) *why = "'" + path + "': " + m;
    return false;
  };
  path_ = path;
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) return no("cannot be opened");
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    ::close(fd);
    return no("cannot be read");
  }
  const size_t size = (size_t)sb.st_size;
  if (size < 8) {
    ::close(fd);
    return no("is not a safetensors file (shorter than its header length)");
  }
  void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return no("cannot be mapped");
  map_ = m;
  map_bytes_ = size;
  const uint8_t* base = static_cast<const uint8_t*>(m);
  uint64_t hl = 0;
  std::memcpy(&hl, base, 8);  // little-endian on every host this builds for
  if (hl == 0 || hl > size - 8 || hl > (100ull << 20))
    return no("the header length does not fit the file");
  json::Value h;
  std::string jerr;
  if (!json::parse(reinterpret_cast<const char*>(base + 8), (size_t)hl, &h, &jerr) ||
      !h.is_obj())
    return no("the header is not a JSON object (" + jerr + ")");
  const uint8_t* data = base + 8 + hl;
  const size_t data_bytes = size - 8 - (size_t)hl;
  for (const auto& kv : h.obj) {
    if (kv.first == "__metadata__") {
      if (!kv.second.is_obj()) return no("__metadata__ is not an object");
      for (const auto& mv : kv.second.obj)
        if (mv.second.is_str()) meta_[mv.first] = mv.second.str;
      continue;
    }
    const json::Value& e = kv.second;
    const json::Value* dt = e.get("dtype");
    const json::Value* sh = e.get("shape");
    const json::Value* off = e.get("data_offsets");
    if (!dt || !dt->is_str() || !sh || !sh->is_arr() || !off || !off->is_arr() ||
        off->arr.size() != 2)
      return no("tensor '" + kv.first + "' has a malformed entry");
    Tensor t;
    t.name = kv.first;
    t.dtype = dt->str;
    const size_t es = dtype_size(t.dtype);
    if (es == 0) return no("tensor '" + kv.first + "' has the unknown dtype " + t.dtype);
    for (const auto& d : sh->arr) {
      if (!d.is_num() || d.num < 0 || d.num != (double)(int64_t)d.num || d.num > 9.0e15)
        return no("tensor '" + kv.first + "' has a bad shape");
      t.shape.push_back((int64_t)d.num);
    }
    const json::Value& b0 = off->arr[0];
    const json::Value& b1 = off->arr[1];
    if (!b0.is_num() || !b1.is_num() || b0.num < 0 || b1.num < b0.num ||
        b1.num > (double)data_bytes)
      return no("tensor '" + kv.first + "' has offsets outside the data");
    const size_t begin = (size_t)b0.num, end = (size_t)b1.num;
    double elems = 1.0;
    for (int64_t d : t.shape) elems *= (double)d;
    if ((double)(end - begin) != elems * (double)es)
      return no("tensor '" + kv.first + "' holds " + std::to_string(end - begin) +
                " bytes, not the " + std::to_string((long long)(elems * (double)es)) +
                " its shape and dtype need");
    t.data = data + begin;
    t.bytes = end - begin;
    tensors_.push_back(std::move(t));
  }
  return true;
}

bool Set::add(const std::string& path, std::string* why) {
  auto f = std::make_unique<File>();
  if (!f->open(path, why)) return false;
  for (const Tensor& t : f->tensors()) {
    if (!by_name_.emplace(t.name, &t).second) {
      if (why) *why = "tensor '" + t.name + "' appears in more than one file ('" + path + "')";
      return false;
    }
    order_.push_back(&t);
  }
  files_.push_back(std::move(f));
  return true;
}

bool Set::open_dir(const std::string& dir, std::string* why) {
  std::error_code ec;
  if (!fs::is_directory(dir, ec)) {
    if (why) *why = "'" + dir + "' is not a directory";
    return false;
  }
  std::vector<std::string> files;
  for (const auto& e : fs::directory_iterator(dir, ec))
    if (e.is_regular_file() && e.path().extension() == ".safetensors")
      files.push_back(e.path().string());
  if (files.empty()) {
    if (why) *why = "'" + dir + "' holds no .safetensors file";
    return false;
  }
  std::sort(files.begin(), files.end());
  for (const auto& f : files)
    if (!add(f, why)) return false;
  return true;
}

bool Set::open_file(const std::string& path, std::string* why) { return add(path, why); }

const Tensor* Set::find(const std::string& name) const {
  auto it = by_name_.find(name);
  return it == by_name_.end() ? nullptr : it->second;
}

uint16_t f32_to_bf16_narrow(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

namespace {

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else {  // subnormal: renormalise
      exp = 127 - 15 + 1;
      while ((man & 0x400u) == 0) {
        man <<= 1;
        --exp;
      }
      man &= 0x3ffu;
      u = sign | (exp << 23) | (man << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

}  // namespace

bool to_bf16(const Tensor& t, std::vector<uint16_t>* out, std::string* why) {
  const size_t n = (size_t)t.numel();
  out->resize(n);
  if (t.dtype == "BF16") {
    std::memcpy(out->data(), t.data, n * 2);
  } else if (t.dtype == "F32") {
    for (size_t i = 0; i < n; ++i) {
      float f;
      std::memcpy(&f, t.data + 4 * i, 4);
      (*out)[i] = f32_to_bf16_narrow(f);
    }
  } else if (t.dtype == "F16") {
    for (size_t i = 0; i < n; ++i) {
      uint16_t h;
      std::memcpy(&h, t.data + 2 * i, 2);
      (*out)[i] = f32_to_bf16_narrow(f16_to_f32(h));
    }
  } else {
    if (why) *why = "tensor '" + t.name + "' is " + t.dtype + ", not a float tensor";
    return false;
  }
  return true;
}

bool to_f32(const Tensor& t, std::vector<float>* out, std::string* why) {
  const size_t n = (size_t)t.numel();
  out->resize(n);
  if (t.dtype == "F32") {
    std::memcpy(out->data(), t.data, n * 4);
  } else if (t.dtype == "BF16") {
    for (size_t i = 0; i < n; ++i) {
      uint16_t h;
      std::memcpy(&h, t.data + 2 * i, 2);
      const uint32_t u = (uint32_t)h << 16;
      std::memcpy(&(*out)[i], &u, 4);
    }
  } else if (t.dtype == "F16") {
    for (size_t i = 0; i < n; ++i) {
      uint16_t h;
      std::memcpy(&h, t.data + 2 * i, 2);
      (*out)[i] = f16_to_f32(h);
    }
  } else if (t.dtype == "F64") {
    for (size_t i = 0; i < n; ++i) {
      double d;
      std::memcpy(&d, t.data + 8 * i, 8);
      (*out)[i] = (float)d;
    }
  } else {
    if (why) *why = "tensor '" + t.name + "' is " + t.dtype + ", not a float tensor";
    return false;
  }
  return true;
}

bool write(const std::string& path, const std::vector<OutTensor>& ts,
           const std::map<std::string, std::string>& metadata, std::string* why) {
  json::Value h = json::Value::object();
  if (!metadata.empty()) {
    json::Value m = json::Value::object();
    for (const auto& kv : metadata) m.set(kv.first, json::Value::string(kv.second));
    h.set("__metadata__", std::move(m));
  }
  size_t off = 0;
  for (const OutTensor& t : ts) {
    json::Value e = json::Value::object();
    e.set("dtype", json::Value::string(t.dtype));
    json::Value sh = json::Value::array();
    for (int64_t d : t.shape) sh.arr.push_back(json::Value::number((double)d));
    e.set("shape", std::move(sh));
    json::Value o = json::Value::array();
    o.arr.push_back(json::Value::number((double)off));
    o.arr.push_back(json::Value::number((double)(off + t.bytes)));
    e.set("data_offsets", std::move(o));
    h.set(t.name, std::move(e));
    off += t.bytes;
  }
  std::string hdr = json::dump(h);
  while (hdr.size() % 8) hdr.push_back(' ');
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) {
    if (why) *why = "'" + path + "' cannot be written";
    return false;
  }
  const uint64_t hl = hdr.size();
  f.write(reinterpret_cast<const char*>(&hl), 8);
  f.write(hdr.data(), (std::streamsize)hdr.size());
  for (const OutTensor& t : ts) f.write(static_cast<const char*>(t.data), (std::streamsize)t.bytes);
  f.close();
  if (!f) {
    if (why) *why = "'" + path + "' could not be written in full";
    return false;
  }
  return true;
}

}  // namespace ming::st
