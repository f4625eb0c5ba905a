// Read-only safetensors file (memory-mapped) with a minimal header parser.
//
// Keeps the reference loader's surface (src/io/safetensors.hpp:108-150):
// names() in dictionary order, contains(name), dtype(name), shape(name) as
// std::vector<size_t>, tensor_bytes(name, nbytes); an unknown name throws
// std::runtime_error.  Format:
// 8-byte little-endian header length, a JSON object mapping each tensor name
// to {"dtype", "shape", "data_offsets": [begin, end]} (offsets relative to
// the end of the header), optional "__metadata__", then the raw data.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace dollama {

enum class StDtype { F64, F32, F16, BF16, I64, I32, I16, I8, U8, BOOL, Unknown };

class SafeTensors {
 public:
  explicit SafeTensors(const std::string& path);
  ~SafeTensors();
  SafeTensors(const SafeTensors&) = delete;
  SafeTensors& operator=(const SafeTensors&) = delete;

  const std::vector<std::string>& names() const { return names_; }
  bool contains(const std::string& name) const { return entries_.count(name) != 0; }
  StDtype dtype(const std::string& name) const;
  const std::vector<size_t>& shape(const std::string& name) const;
  // the same shape as signed extents (the UNet / VAE weight specs' type)
  const std::vector<int64_t>& shape_i64(const std::string& name) const;
  const uint8_t* tensor_bytes(const std::string& name, size_t& nbytes) const;
  // whole data region (for a single upload)
  const uint8_t* data() const { return data_; }
  size_t data_bytes() const { return data_bytes_; }
  size_t offset(const std::string& name) const;

 private:
  struct Entry {
    StDtype dtype = StDtype::Unknown;
    std::vector<int64_t> shape;
    std::vector<size_t> shape_u;
    size_t begin = 0, end = 0;
  };
  const Entry& entry(const std::string& name) const;
  void parse_header(const std::string& json);

  void* map_ = nullptr;
  size_t map_bytes_ = 0;
  const uint8_t* data_ = nullptr;
  size_t data_bytes_ = 0;
  std::unordered_map<std::string, Entry> entries_;
  std::vector<std::string> names_;
};

}  // namespace dollama
