#include "lora.hpp"

#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>

#include "check.hpp"

namespace dollama {

uint16_t f32_to_f16_rne(float v) {
  uint32_t x;
  std::memcpy(&x, &v, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));  // nan / inf
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds past the largest half
  if (ax < 0x33000001u) return (uint16_t)sign;              // below half the smallest subnormal
  const int e = (int)(ax >> 23) - 127;
  uint32_t mant = (ax & 0x7fffffu) | 0x800000u;  // 24-bit significand
  uint32_t h;
  if (e < -14) {  // subnormal half: keep (e + 24) bits
    const int shift = -e - 1;  // 14..24
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    h = mant >> shift;
    if (rem > half || (rem == half && (h & 1u))) ++h;
  } else {
    const uint32_t rem = mant & 0x1fffu, half = 0x1000u;
    h = ((uint32_t)(e + 15) << 10) | ((mant >> 13) & 0x3ffu);
    if (rem > half || (rem == half && (h & 1u))) ++h;  // may carry into the exponent: correct
  }
  return (uint16_t)(sign | h);
}

namespace {

bool ends_with(const std::string& s, const std::string& suf) {
  return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

float half_to_float(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
  if (e == 0) {
    if (m == 0) {
      x = s;
    } else {  // subnormal
      e = 113;
      while (!(m & 0x400u)) {
        m <<= 1;
        --e;
      }
      x = s | (e << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (e == 31) {
    x = s | 0x7f800000u | (m << 13);
  } else {
    x = s | ((e + 112) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

float read_scalar(const SafeTensors& st, const std::string& key) {
  size_t n = 0;
  const uint8_t* p = st.tensor_bytes(key, n);
  if (st.dtype(key) == StDtype::F32 && n == 4) {
    float v;
    std::memcpy(&v, p, 4);
    return v;
  }
  if (st.dtype(key) == StDtype::F16 && n == 2) {
    uint16_t h;
    std::memcpy(&h, p, 2);
    return half_to_float(h);
  }
  throw std::runtime_error("lora: alpha '" + key + "' must be an F32 or F16 scalar");
}

std::vector<uint16_t> read_f16(const SafeTensors& st, const std::string& key) {
  size_t n = 0;
  const uint8_t* p = st.tensor_bytes(key, n);
  if (st.dtype(key) == StDtype::F16) {
    std::vector<uint16_t> out(n / 2);
    std::memcpy(out.data(), p, n);
    return out;
  }
  if (st.dtype(key) == StDtype::F32) {
    std::vector<uint16_t> out(n / 4);
    for (size_t i = 0; i < out.size(); ++i) {
      float v;
      std::memcpy(&v, p + 4 * i, 4);
      out[i] = f32_to_f16_rne(v);
    }
    return out;
  }
  throw std::runtime_error("lora: tensor '" + key + "' must be F16 or F32");
}

int64_t tail(const std::vector<int64_t>& s) {
  int64_t n = 1;
  for (size_t i = 1; i < s.size(); ++i) n *= s[i];
  return n;
}

struct Group {
  std::string down, up;
  bool has_alpha = false;
  float alpha = 0.0f;
};

}  // namespace

std::vector<LoraModule> load_lora_modules(const std::vector<WeightSpec>& base,
                                          const SafeTensors& lora, float strength,
                                          LoraReport* report) {
  LoraReport rep;
  std::map<std::string, Group> groups;
  for (const std::string& k : lora.names()) {
    if (k.rfind("lora_te1_", 0) == 0 || k.rfind("lora_te2_", 0) == 0 || k.rfind("lora_te_", 0) == 0) {
      ++rep.te_skipped;
      continue;
    }
    if (k.rfind("lora_unet_", 0) != 0) {
      ++rep.other_keys;
      continue;
    }
    const std::string body = k.substr(10);
    static const char* kSuffix[6] = {".lora_down.weight", ".lora_up.weight", ".alpha",
                                     "_lora_down_weight", "_lora_up_weight", "_alpha"};
    int which = -1;
    for (int i = 0; i < 6 && which < 0; ++i)
      if (ends_with(body, kSuffix[i])) which = i;
    if (which < 0) {
      ++rep.other_keys;
      continue;
    }
    Group& g = groups[body.substr(0, body.size() - std::strlen(kSuffix[which]))];
    if (which % 3 == 0) g.down = k;
    else if (which % 3 == 1) g.up = k;
    else {  // read as soon as seen: a malformed alpha is an error even in a skipped module
      g.alpha = read_scalar(lora, k);
      g.has_alpha = true;
    }
  }
  // base names with every '.' replaced by '_' ("a.b.weight" -> "a_b_weight")
  std::map<std::string, const WeightSpec*> index;
  for (const WeightSpec& w : base) {
    std::string flat = w.name;
    for (char& ch : flat)
      if (ch == '.') ch = '_';
    index[flat] = &w;
  }
  std::vector<LoraModule> mods;
  for (const auto& kv : groups) {
    const std::string& mod = kv.first;
    const Group& g = kv.second;
    if (g.down.empty() || g.up.empty()) {
      ++rep.incomplete;
      continue;
    }
    auto hit = index.find(mod + "_weight");
    if (hit == index.end())
      throw std::runtime_error("lora: module 'lora_unet_" + mod + "' matches no UNet weight");
    const WeightSpec& w = *hit->second;
    const std::vector<int64_t>& as = lora.shape_i64(g.down);
    const std::vector<int64_t>& bs = lora.shape_i64(g.up);
    if (as.empty() || bs.empty()) throw std::runtime_error("lora: module '" + mod + "' has an empty shape");
    const int64_t rank = as[0], in_flat = tail(as), out_dim = bs[0];
    if (tail(bs) != rank)
      throw std::runtime_error("lora: module '" + mod + "' up tensor does not match the rank");
    if (rank <= 0 || in_flat <= 0 || out_dim <= 0)
      throw std::runtime_error("lora: module '" + mod + "' has a zero dimension");
    int64_t wn = 1;
    for (int64_t d : w.shape) wn *= d;
    if (w.shape.size() == 2 ? (w.shape[0] != out_dim || w.shape[1] != in_flat) : wn != out_dim * in_flat)
      throw std::runtime_error("lora: module '" + mod + "' does not match the shape of '" + w.name + "'");
    const float alpha = g.has_alpha ? g.alpha : (float)rank;
    LoraModule m;
    m.base_key = w.name;
    m.a_fp16 = read_f16(lora, g.down);
    m.b_fp16 = read_f16(lora, g.up);
    m.rank = (int)rank;
    m.in_flat = (int)in_flat;
    m.out_dim = (int)out_dim;
    m.scale = strength * (alpha / (float)rank);
    mods.push_back(std::move(m));
  }
  rep.modules = mods.size();
  if (report) *report = rep;
  return mods;
}

void unet_apply_lora_file(UNet& u, const std::string& path, float strength, LoraReport* report,
                          void* stream) {
  SafeTensors st(path);
  LoraReport rep;
  const std::vector<LoraModule> mods = load_lora_modules(unet_weight_specs(u.config()), st, strength, &rep);
  for (const LoraModule& m : mods) unet_apply_lora_module(u, m, stream);
  if (report) *report = rep;
}

void unet_apply_lora_module(UNet& u, const LoraModule& m, void* stream) {
  const size_t na = m.a_fp16.size(), nb = m.b_fp16.size();
  if (m.rank <= 0 || na != (size_t)m.rank * m.in_flat || nb != (size_t)m.out_dim * m.rank)
    throw std::runtime_error("lora: module '" + m.base_key + "' has inconsistent A / B sizes");
  void* dev = nullptr;
  DLM_CALL(dlm_malloc(&dev, (na + nb) * 2));
  std::unique_ptr<void, void (*)(void*)> hold(dev, [](void* p) { (void)dlm_free(p); });
  DLM_CALL(dlm_memcpy(dev, m.a_fp16.data(), na * 2, 0));
  DLM_CALL(dlm_memcpy(static_cast<uint16_t*>(dev) + na, m.b_fp16.data(), nb * 2, 0));
  u.apply_lora(m.base_key, dev, static_cast<uint16_t*>(dev) + na, m.rank, m.in_flat, m.out_dim, m.scale,
               stream);
}

}  // namespace dollama
