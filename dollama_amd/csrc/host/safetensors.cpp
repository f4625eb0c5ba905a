// safetensors reader (see safetensors.hpp).
#include "safetensors.hpp"

#include <algorithm>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cstring>
#include <stdexcept>

namespace dollama {
namespace {

StDtype parse_dtype(const std::string& s) {
  if (s == "F64") return StDtype::F64;
  if (s == "F32") return StDtype::F32;
  if (s == "F16") return StDtype::F16;
  if (s == "BF16") return StDtype::BF16;
  if (s == "I64") return StDtype::I64;
  if (s == "I32") return StDtype::I32;
  if (s == "I16") return StDtype::I16;
  if (s == "I8") return StDtype::I8;
  if (s == "U8") return StDtype::U8;
  if (s == "BOOL") return StDtype::BOOL;
  return StDtype::Unknown;
}

size_t dtype_size(StDtype d) {
  switch (d) {
    case StDtype::F64: case StDtype::I64: return 8;
    case StDtype::F32: case StDtype::I32: return 4;
    case StDtype::F16: case StDtype::BF16: case StDtype::I16: return 2;
    case StDtype::I8: case StDtype::U8: case StDtype::BOOL: return 1;
    default: return 0;
  }
}

// Minimal JSON cursor sufficient for the safetensors header grammar.
struct Json {
  const std::string& s;
  size_t i = 0;
  explicit Json(const std::string& str) : s(str) {}
  [[noreturn]] void fail(const char* what) const {
    throw std::runtime_error(std::string("safetensors header: ") + what + " at byte " + std::to_string(i));
  }
  void ws() {
    while (i < s.size() && std::isspace((unsigned char)s[i])) ++i;
  }
  bool peek(char c) {
    ws();
    return i < s.size() && s[i] == c;
  }
  void expect(char c) {
    ws();
    if (i >= s.size() || s[i] != c) fail("unexpected character");
    ++i;
  }
  std::string str() {
    expect('"');
    std::string out;
    while (i < s.size() && s[i] != '"') {
      if (s[i] == '\\') {
        ++i;
        if (i >= s.size()) fail("bad escape");
        const char e = s[i];
        if (e == 'u') {
          if (i + 4 >= s.size()) fail("bad unicode escape");
          const unsigned cp = (unsigned)std::stoul(s.substr(i + 1, 4), nullptr, 16);
          if (cp < 0x80) out += (char)cp;
          else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 0x3F)); }
          else { out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 0x3F)); out += (char)(0x80 | (cp & 0x3F)); }
          i += 4;
        } else {
          out += e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e == 'b' ? '\b' : e == 'f' ? '\f' : e;
        }
        ++i;
      } else {
        out += s[i++];
      }
    }
    if (i >= s.size()) fail("unterminated string");
    ++i;
    return out;
  }
  int64_t integer() {
    ws();
    size_t j = i;
    if (j < s.size() && s[j] == '-') ++j;
    while (j < s.size() && std::isdigit((unsigned char)s[j])) ++j;
    if (j == i) fail("expected integer");
    const int64_t v = std::stoll(s.substr(i, j - i));
    i = j;
    return v;
  }
  void skip_value() {
    ws();
    if (peek('"')) { (void)str(); return; }
    if (peek('{')) {
      expect('{');
      if (peek('}')) { expect('}'); return; }
      while (true) {
        (void)str();
        expect(':');
        skip_value();
        if (peek(',')) { expect(','); continue; }
        expect('}');
        return;
      }
    }
    if (peek('[')) {
      expect('[');
      if (peek(']')) { expect(']'); return; }
      while (true) {
        skip_value();
        if (peek(',')) { expect(','); continue; }
        expect(']');
        return;
      }
    }
    while (i < s.size() && s[i] != ',' && s[i] != '}' && s[i] != ']') ++i;
  }
  std::vector<int64_t> int_list() {
    std::vector<int64_t> v;
    expect('[');
    if (peek(']')) { expect(']'); return v; }
    while (true) {
      v.push_back(integer());
      if (peek(',')) { expect(','); continue; }
      expect(']');
      return v;
    }
  }
};

}  // namespace

SafeTensors::SafeTensors(const std::string& path) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) throw std::runtime_error("safetensors: cannot open " + path);
  struct stat st {};
  if (::fstat(fd, &st) != 0) {
    ::close(fd);
    throw std::runtime_error("safetensors: cannot stat " + path);
  }
  map_bytes_ = (size_t)st.st_size;
  if (map_bytes_ < 8) {
    ::close(fd);
    throw std::runtime_error("safetensors: file too small: " + path);
  }
  map_ = ::mmap(nullptr, map_bytes_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map_ == MAP_FAILED) {
    map_ = nullptr;
    throw std::runtime_error("safetensors: mmap failed: " + path);
  }
  const uint8_t* base = static_cast<const uint8_t*>(map_);
  uint64_t hlen = 0;
  std::memcpy(&hlen, base, 8);
  if (hlen > map_bytes_ - 8) {
    ::munmap(map_, map_bytes_);
    map_ = nullptr;
    throw std::runtime_error("safetensors: header length exceeds file size");
  }
  data_ = base + 8 + hlen;
  data_bytes_ = map_bytes_ - 8 - hlen;
  try {
    parse_header(std::string(reinterpret_cast<const char*>(base + 8), (size_t)hlen));
  } catch (...) {
    ::munmap(map_, map_bytes_);
    map_ = nullptr;
    throw;
  }
}

SafeTensors::~SafeTensors() {
  if (map_) ::munmap(map_, map_bytes_);
}

void SafeTensors::parse_header(const std::string& json) {
  Json j(json);
  j.expect('{');
  if (j.peek('}')) return;
  struct SortNames {  // names() lists tensors in dictionary order on return
    std::vector<std::string>& v;
    ~SortNames() { std::sort(v.begin(), v.end()); }
  } sort_names{names_};
  while (true) {
    const std::string key = j.str();
    j.expect(':');
    if (key == "__metadata__") {
      j.skip_value();
    } else {
      Entry e;
      bool have_dtype = false, have_shape = false, have_off = false;
      j.expect('{');
      while (!j.peek('}')) {
        const std::string f = j.str();
        j.expect(':');
        if (f == "dtype") { e.dtype = parse_dtype(j.str()); have_dtype = true; }
        else if (f == "shape") { e.shape = j.int_list(); have_shape = true; }
        else if (f == "data_offsets") {
          const auto o = j.int_list();
          if (o.size() != 2 || o[0] < 0 || o[1] < o[0]) j.fail("bad data_offsets");
          e.begin = (size_t)o[0];
          e.end = (size_t)o[1];
          have_off = true;
        } else {
          j.skip_value();
        }
        if (j.peek(',')) j.expect(',');
      }
      j.expect('}');
      if (!have_dtype || !have_shape || !have_off) j.fail("tensor entry missing a field");
      if (e.end > data_bytes_) throw std::runtime_error("safetensors: tensor '" + key + "' beyond file end");
      // element count and byte size with overflow checks: a crafted header
      // must not wrap n * es around to the stored byte range
      size_t n = 1;
      for (int64_t d : e.shape) {
        if (d < 0) j.fail("negative dimension");
        if (__builtin_mul_overflow(n, (size_t)d, &n))
          throw std::runtime_error("safetensors: tensor '" + key + "' shape overflows");
        e.shape_u.push_back((size_t)d);
      }
      const size_t es = dtype_size(e.dtype);
      size_t nbytes = 0;
      if (es != 0 && __builtin_mul_overflow(n, es, &nbytes))
        throw std::runtime_error("safetensors: tensor '" + key + "' byte size overflows");
      if (es != 0 && nbytes != e.end - e.begin)
        throw std::runtime_error("safetensors: tensor '" + key + "' size does not match shape");
      if (entries_.count(key)) j.fail("duplicate tensor name");
      entries_[key] = e;
      names_.push_back(key);
    }
    if (j.peek(',')) {
      j.expect(',');
      continue;
    }
    j.expect('}');
    break;
  }
}

const SafeTensors::Entry& SafeTensors::entry(const std::string& name) const {
  auto it = entries_.find(name);
  if (it == entries_.end()) throw std::runtime_error("safetensors: no tensor named '" + name + "'");
  return it->second;
}

StDtype SafeTensors::dtype(const std::string& name) const { return entry(name).dtype; }
const std::vector<size_t>& SafeTensors::shape(const std::string& name) const { return entry(name).shape_u; }
const std::vector<int64_t>& SafeTensors::shape_i64(const std::string& name) const { return entry(name).shape; }
size_t SafeTensors::offset(const std::string& name) const { return entry(name).begin; }

const uint8_t* SafeTensors::tensor_bytes(const std::string& name, size_t& nbytes) const {
  const Entry& e = entry(name);
  nbytes = e.end - e.begin;
  return data_ + e.begin;
}

}  // namespace dollama
