// SDXL AutoencoderKL decoder driver (channels-last, fused epilogues).
#include "vae.hpp"

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <utility>

#include "check.hpp"
#include "device_arena.hpp"
#include "lora.hpp"

namespace dollama {

// Channels of post_quant_conv's output as conv_in reads it (the latent's 4,
// zero-padded): a multiple of 64 puts conv_in on the DMA implicit-GEMM core.
static constexpr int kPqPad = 64;

#define LAUNCH(cls, flops, bytes, expr)          \
  do {                                           \
    prof_begin((cls), (flops), (bytes), stream); \
    try {                                        \
      DLM_CALL(expr);                            \
    } catch (...) {                              \
      if (prof_on_) (void)dlm_prof_disarm();     \
      throw;                                     \
    }                                            \
    prof_end(stream);                            \
  } while (0)

namespace {
using Shape = std::vector<int64_t>;
constexpr size_t kH = 2;      // bytes per fp16
constexpr float kEps = 1e-6f;  // GroupNorm eps (src/kernels/vae_decode.cu:579, :621, :665, :704)
// An fp32 activation becomes a conv operand as fp16(x * kWideIn); the weight
// columns it meets are multiplied by 1 / kWideIn.  Both are exact powers of
// two, so the product is unchanged and fp16 overflows only beyond 65504 / kWideIn.
constexpr float kWideIn = 1.0f / 256.0f;

std::string shape_str(const Shape& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? "," : "") + std::to_string(s[i]);
  return r + "]";
}

// ResnetBlock2D without time embedding (src/kernels/vae_decode.cu:608-652)
void add_resnet(std::vector<WeightSpec>& v, const std::string& p, int Ci, int Co) {
  v.push_back({p + "norm1.weight", {Ci}});
  v.push_back({p + "norm1.bias", {Ci}});
  v.push_back({p + "conv1.weight", {Co, Ci, 3, 3}});
  v.push_back({p + "conv1.bias", {Co}});
  v.push_back({p + "norm2.weight", {Co}});
  v.push_back({p + "norm2.bias", {Co}});
  v.push_back({p + "conv2.weight", {Co, Co, 3, 3}});
  v.push_back({p + "conv2.bias", {Co}});
  if (Ci != Co) {
    v.push_back({p + "conv_shortcut.weight", {Co, Ci, 1, 1}});
    v.push_back({p + "conv_shortcut.bias", {Co}});
  }
}

std::string up_prefix(int i) { return "decoder.up_blocks." + std::to_string(i) + "."; }
}  // namespace

std::vector<WeightSpec> vae_weight_specs(const VaeConfig& c) {
  std::vector<WeightSpec> v;
  const int L = c.latent_channels, Cm = c.up_ch(0);
  v.push_back({"post_quant_conv.weight", {L, L, 1, 1}});
  v.push_back({"post_quant_conv.bias", {L}});
  v.push_back({"decoder.conv_in.weight", {Cm, L, 3, 3}});
  v.push_back({"decoder.conv_in.bias", {Cm}});
  add_resnet(v, "decoder.mid_block.resnets.0.", Cm, Cm);
  const std::string a = "decoder.mid_block.attentions.0.";
  v.push_back({a + "group_norm.weight", {Cm}});
  v.push_back({a + "group_norm.bias", {Cm}});
  for (const char* n : {"to_q", "to_k", "to_v", "to_out.0"}) {
    v.push_back({a + n + ".weight", {Cm, Cm}});
    v.push_back({a + n + ".bias", {Cm}});
  }
  add_resnet(v, "decoder.mid_block.resnets.1.", Cm, Cm);
  int prev = Cm;
  for (int i = 0; i < 4; ++i) {
    const int Co = c.up_ch(i);
    for (int r = 0; r < c.layers; ++r)
      add_resnet(v, up_prefix(i) + "resnets." + std::to_string(r) + ".", r == 0 ? prev : Co, Co);
    if (i < 3) {
      v.push_back({up_prefix(i) + "upsamplers.0.conv.weight", {Co, Co, 3, 3}});
      v.push_back({up_prefix(i) + "upsamplers.0.conv.bias", {Co}});
    }
    prev = Co;
  }
  v.push_back({"decoder.conv_norm_out.weight", {c.up_ch(3)}});
  v.push_back({"decoder.conv_norm_out.bias", {c.up_ch(3)}});
  v.push_back({"decoder.conv_out.weight", {c.out_channels, c.up_ch(3), 3, 3}});
  v.push_back({"decoder.conv_out.bias", {c.out_channels}});
  return v;
}

VAE::VAE(const VaeConfig& cfg) : cfg_(cfg) {
  for (int C : cfg_.ch) {
    if (C <= 0 || C % 64 != 0) throw std::invalid_argument("VAE: channel counts must be multiples of 64");
    if (cfg_.groups <= 0 || C % cfg_.groups != 0)
      throw std::invalid_argument("VAE: channels not divisible by groups");
  }
  if (cfg_.latent_channels <= 0 || cfg_.latent_channels > 8)
    throw std::invalid_argument("VAE: latent_channels must be in [1, 8]");
  if (cfg_.out_channels <= 0 || cfg_.out_channels > 64)
    throw std::invalid_argument("VAE: out_channels must be in [1, 64]");
  if (cfg_.layers <= 0) throw std::invalid_argument("VAE: layers must be positive");
  if (cfg_.fp32_from < 0 || cfg_.fp32_from > 4) throw std::invalid_argument("VAE: fp32_from must be in [0, 4]");
}

VAE::~VAE() {
  if (packed_) (void)dlm_free(packed_);
  for (void* e : prof_events_) (void)dlm_event_destroy(e);
}

// ------------------------------------------------------------------ profiling

void VAE::prof_begin(int cls, double flops, double bytes, void* stream) {
  if (!prof_on_) return;
  if (prof_next_ * 2 + 2 > prof_events_.size()) {
    for (int i = 0; i < 2; ++i) {
      void* e = nullptr;
      DLM_CALL(dlm_event_create(&e));
      prof_events_.push_back(e);
    }
  }
  if (prof_recs_.size() <= prof_next_) prof_recs_.resize(prof_next_ + 1);
  prof_recs_[prof_next_] = ProfRec{cls, flops, bytes};
  // the kernels of the call carry the event pair in their own dispatches
  DLM_CALL(dlm_prof_arm(prof_events_[prof_next_ * 2], prof_events_[prof_next_ * 2 + 1]));
  (void)stream;
}

void VAE::prof_end(void* stream) {
  if (!prof_on_) return;
  if (dlm_prof_disarm() == 0) {  // no kernel in the call: an empty interval
    DLM_CALL(dlm_event_record(prof_events_[prof_next_ * 2], stream));
    DLM_CALL(dlm_event_record(prof_events_[prof_next_ * 2 + 1], stream));
  }
  ++prof_next_;
}

std::vector<VAE::ClassStats> VAE::profile_report(void* stream) {
  DLM_CALL(dlm_stream_synchronize(stream));
  std::vector<ClassStats> out(kClassCount);
  for (size_t i = 0; i < prof_next_ && i < prof_recs_.size(); ++i) {
    float ms = 0.0f;
    DLM_CALL(dlm_event_elapsed_ms(&ms, prof_events_[2 * i], prof_events_[2 * i + 1]));
    ClassStats& c = out[prof_recs_[i].cls];
    c.count += 1;
    c.ms += ms;
    c.flops += prof_recs_[i].flops;
    c.bytes += prof_recs_[i].bytes;
  }
  return out;
}

// ------------------------------------------------------------------ weights

void VAE::set_weight(const std::string& name, const void* dptr, const Shape& shape) {
  if (!dptr) throw std::invalid_argument("VAE::set_weight: NULL pointer for " + name);
  Shape s = shape;
  // attention projections stored as 1x1 convs by some checkpoints
  if (name.find(".attentions.") != std::string::npos && s.size() == 4 && s[2] == 1 && s[3] == 1)
    s.resize(2);
  srcs_[name] = Src{dptr, s};
}

const VAE::Src& VAE::src(const std::string& name, const Shape& shape) const {
  auto it = srcs_.find(name);
  if (it == srcs_.end()) throw std::runtime_error("VAE: missing weight '" + name + "'");
  if (it->second.shape != shape)
    throw std::runtime_error("VAE: weight '" + name + "' has shape " + shape_str(it->second.shape) +
                             ", expected " + shape_str(shape));
  return it->second;
}

void* VAE::take(size_t elems) {
  const size_t off = cursor_;
  cursor_ += (elems * kH + 255) & ~size_t(255);
  return sizing_ ? nullptr : packed_ + off;
}

const void* VAE::copy_of(const std::string& name, const Shape& shape, void* stream) {
  const Src& s = src(name, shape);
  size_t n = 1;
  for (int64_t d : shape) n *= (size_t)d;
  void* dst = take(n);
  if (!sizing_) DLM_CALL(dlm_memcpy_async(dst, s.ptr, n * kH, 2, stream));
  return dst;
}

void VAE::pack_weight(const std::string& name, void* dst, int Co, int Ci, int k, int cin_pad, int ld,
                      int col0, float scale, void* stream) {
  const Src& s = src(name, {Co, Ci, k, k});
  const size_t n = (size_t)Co * Ci * k * k;
  if (sizing_) {
    if (scale == 1.0f) return;
    // the scaled copy below is exact (a power of two) if no scaled element
    // leaves the fp16 range; checked on the host before anything is packed
    // (magnitudes of finite fp16 values order like their bit patterns
    // without the sign)
    std::vector<uint16_t> hw(n);
    DLM_CALL(dlm_stream_synchronize(stream));
    DLM_CALL(dlm_memcpy(hw.data(), s.ptr, n * kH, 1));
    const uint16_t limit = f32_to_f16_rne(65504.0f / scale);
    for (uint16_t b : hw)
      if ((b & 0x7fff) > limit)
        throw std::runtime_error("VAE: weight '" + name + "' has an element beyond 65504 / " +
                                 std::to_string(scale) + " (its fp32-stage operand scaling would overflow)");
    return;
  }
  if (scale == 1.0f) {
    DLM_CALL(dlm_conv_weight_pack_fp16(s.ptr, dst, Co, Ci, k, k, cin_pad, ld, col0, stream));
    return;
  }
  DeviceArenaScope sc(DeviceArenaId::VAE);
  void* tmp = sc.alloc<uint16_t>(n);
  DLM_CALL(dlm_memcpy_async(tmp, s.ptr, n * kH, 2, stream));
  DLM_CALL(dlm_scale_fp16(tmp, (long long)n, scale, stream));
  DLM_CALL(dlm_conv_weight_pack_fp16(tmp, dst, Co, Ci, k, k, cin_pad, ld, col0, stream));
}

VAE::Conv VAE::pack_conv(const std::string& p, int Co, int Ci, int k, int cin_pad, float scale,
                         void* stream) {
  Conv c;
  c.ldw = k * k * cin_pad;
  void* w = take((size_t)Co * c.ldw);
  pack_weight(p + "weight", w, Co, Ci, k, cin_pad, c.ldw, 0, scale, stream);
  c.w = w;
  c.b = copy_of(p + "bias", {Co}, stream);
  return c;
}

VAE::Resnet VAE::pack_resnet(const std::string& p, int Ci, int Co, bool in_f32, bool out_f32,
                             void* stream) {
  Resnet r;
  r.Ci = Ci;
  r.Co = Co;
  r.shortcut = Ci != Co;
  r.in_f32 = in_f32;
  r.out_f32 = out_f32;
  r.n1g = copy_of(p + "norm1.weight", {Ci}, stream);
  r.n1b = copy_of(p + "norm1.bias", {Ci}, stream);
  void* c1 = take((size_t)Co * 9 * Ci);
  pack_weight(p + "conv1.weight", c1, Co, Ci, 3, Ci, 9 * Ci, 0, 1.0f, stream);
  r.c1w = c1;
  r.c1b = copy_of(p + "conv1.bias", {Co}, stream);
  r.n2g = copy_of(p + "norm2.weight", {Co}, stream);
  r.n2b = copy_of(p + "norm2.bias", {Co}, stream);
  // conv2 (+ conv_shortcut appended as a second K segment; its operand is
  // the block input, scaled by kWideIn when that input is fp32)
  r.c2_ldw = 9 * Co + (r.shortcut ? Ci : 0);
  void* c2 = take((size_t)Co * r.c2_ldw);
  pack_weight(p + "conv2.weight", c2, Co, Co, 3, Co, r.c2_ldw, 0, 1.0f, stream);
  r.c2w = c2;
  if (r.shortcut) {
    pack_weight(p + "conv_shortcut.weight", c2, Co, Ci, 1, Ci, r.c2_ldw, 9 * Co,
                in_f32 ? 1.0f / kWideIn : 1.0f, stream);
    void* b = take(Co);
    const Src& b2 = src(p + "conv2.bias", {Co});
    const Src& bs = src(p + "conv_shortcut.bias", {Co});
    if (!sizing_) DLM_CALL(dlm_add_fp16(b2.ptr, bs.ptr, b, Co, stream));
    r.c2b = b;
  } else {
    r.c2b = copy_of(p + "conv2.bias", {Co}, stream);
  }
  return r;
}

VAE::Attn VAE::pack_attn(const std::string& p, int C, void* stream) {
  Attn a;
  a.C = C;
  a.ng = copy_of(p + "group_norm.weight", {C}, stream);
  a.nb = copy_of(p + "group_norm.bias", {C}, stream);
  // fused q|k|v projection [3C, C] and bias [3C]
  char* w = static_cast<char*>(take((size_t)3 * C * C));
  char* b = static_cast<char*>(take((size_t)3 * C));
  const char* names[3] = {"to_q", "to_k", "to_v"};
  for (int i = 0; i < 3; ++i) {
    const Src& sw = src(p + names[i] + ".weight", {C, C});
    const Src& sb = src(p + names[i] + ".bias", {C});
    if (!sizing_) {
      DLM_CALL(dlm_memcpy_async(w + (size_t)i * C * C * kH, sw.ptr, (size_t)C * C * kH, 2, stream));
      DLM_CALL(dlm_memcpy_async(b + (size_t)i * C * kH, sb.ptr, (size_t)C * kH, 2, stream));
    }
  }
  a.wqkv = w;
  a.bqkv = b;
  a.wo = copy_of(p + "to_out.0.weight", {C, C}, stream);
  a.bo = copy_of(p + "to_out.0.bias", {C}, stream);
  return a;
}

void VAE::pack_all(void* stream) {
  const VaeConfig& c = cfg_;
  cursor_ = 0;
  const int L = c.latent_channels, Cm = c.up_ch(0);
  pqc_ = pack_conv("post_quant_conv.", L, L, 1, 8, 1.0f, stream);
  // conv_in reads post_quant_conv's output zero-padded to 64 channels, so it
  // runs on the DMA implicit-GEMM core (K = 9 x 64)
  conv_in_ = pack_conv("decoder.conv_in.", Cm, L, 3, kPqPad, 1.0f, stream);
  res_.clear();
  ups_.clear();
  res_.push_back(pack_resnet("decoder.mid_block.resnets.0.", Cm, Cm, false, false, stream));
  attn_ = pack_attn("decoder.mid_block.attentions.0.", Cm, stream);
  res_.push_back(pack_resnet("decoder.mid_block.resnets.1.", Cm, Cm, false, false, stream));
  int prev = Cm;
  for (int i = 0; i < 4; ++i) {
    const int Co = c.up_ch(i);
    const bool f32 = i >= c.fp32_from;
    for (int r = 0; r < c.layers; ++r) {
      const bool in_f32 = r > 0 ? f32 : i > c.fp32_from;
      res_.push_back(pack_resnet(up_prefix(i) + "resnets." + std::to_string(r) + ".",
                                 r == 0 ? prev : Co, Co, in_f32, f32, stream));
    }
    if (i < 3)
      ups_.push_back(pack_conv(up_prefix(i) + "upsamplers.0.conv.", Co, Co, 3, Co,
                               f32 ? 1.0f / kWideIn : 1.0f, stream));
    prev = Co;
  }
  norm_out_g_ = copy_of("decoder.conv_norm_out.weight", {c.up_ch(3)}, stream);
  norm_out_b_ = copy_of("decoder.conv_norm_out.bias", {c.up_ch(3)}, stream);
  conv_out_ = pack_conv("decoder.conv_out.", c.out_channels, c.up_ch(3), 3, c.up_ch(3), 1.0f, stream);
}

void VAE::prepare(void* stream) {
  sizing_ = true;
  pack_all(stream);
  const size_t bytes = cursor_;
  sizing_ = false;
  if (packed_) {
    DLM_CALL(dlm_free(packed_));
    packed_ = nullptr;
  }
  void* p = nullptr;
  DLM_CALL(dlm_malloc(&p, bytes));
  packed_ = static_cast<char*>(p);
  packed_bytes_ = bytes;
  try {
    pack_all(stream);
    if (cursor_ != bytes) throw std::logic_error("VAE::prepare: sizing pass disagrees with fill pass");
  } catch (...) {
    (void)dlm_stream_synchronize(stream);
    (void)dlm_free(packed_);
    packed_ = nullptr;
    packed_bytes_ = 0;
    throw;
  }
  DLM_CALL(dlm_stream_synchronize(stream));
  srcs_.clear();
}

// ------------------------------------------------------------------ forward

void VAE::stage(const char* name, const void* p, size_t n, int C, bool f32, void* stream) {
  if (!hook_) return;
  DLM_CALL(dlm_stream_synchronize(stream));
  hook_(name, p, n, C, f32 ? 1 : 0, hook_user_);
}

void VAE::gn(const void* x, bool f32, int C, const void* g, const void* b, void* out, int N, int HW,
             bool silu, void* stream) {
  DeviceArenaScope sc(DeviceArenaId::VAE);
  void* ws = sc.alloc_bytes(dlm_group_norm_nhwc_workspace_bytes(N, C, HW));
  const double bytes = (double)N * HW * C * ((f32 ? 4.0 : 2.0) * 2 + 2.0);
  if (f32)
    LAUNCH(kGroupNorm, 0.0, bytes,
           dlm_group_norm_nhwc_f32in(static_cast<const float*>(x), C, g, b, out, C, N, HW, C,
                                     cfg_.groups, kEps, silu ? 1 : 0, ws, stream));
  else
    LAUNCH(kGroupNorm, 0.0, bytes,
           dlm_group_norm_nhwc_fp16(x, C, C, nullptr, 8, g, b, out, C, N, HW, C, cfg_.groups, kEps,
                                    silu ? 1 : 0, ws, stream));
}

void VAE::conv(const Conv& c, const void* x, int Ci, int ldx, void* out, int Co, int ldy,
               bool out_f32, int N, int H, int W, int k, bool up, void* stream) {
  dlm_conv_nhwc_args a{};
  a.src0a = x;
  a.C0a = Ci;
  a.ld0a = ldx;
  a.N = N;
  a.H = H;
  a.W = W;
  a.KH = k;
  a.KW = k;
  a.stride = 1;
  a.pad = k / 2;
  a.upsample = up ? 1 : 0;
  a.weight = c.w;
  a.ldw = c.ldw;
  a.Cout = Co;
  a.bias = c.b;
  a.out = out;
  a.ldy = ldy;
  a.out_f32 = out_f32 ? 1 : 0;
  const double px = (double)N * H * W * (up ? 4 : 1);
  LAUNCH(kConv, 2.0 * px * Co * k * k * Ci, 0.0, dlm_conv2d_nhwc_fp16(&a, stream));
}

void VAE::resnet(const Resnet& r, const void* x, void* out, int N, int H, int W, void* stream) {
  const int HW = H * W, Ci = r.Ci, Co = r.Co;
  const size_t px = (size_t)N * HW;
  const size_t ob = r.out_f32 ? 4 : 2;
  DeviceArenaScope sc(DeviceArenaId::VAE);
  void* h = sc.alloc<uint16_t>(px * std::max(Ci, Co));
  gn(x, r.in_f32, Ci, r.n1g, r.n1b, h, N, HW, true, stream);
  void* c1 = sc.alloc_bytes(px * Co * ob);
  {
    Conv c{r.c1w, r.c1b, 9 * Ci};
    conv(c, h, Ci, Ci, c1, Co, Co, r.out_f32, N, H, W, 3, false, stream);
  }
  gn(c1, r.out_f32, Co, r.n2g, r.n2b, h, N, HW, true, stream);
  dlm_conv_nhwc_args a{};
  a.src0a = h;
  a.C0a = Co;
  a.ld0a = Co;
  a.N = N;
  a.H = H;
  a.W = W;
  a.KH = 3;
  a.KW = 3;
  a.stride = 1;
  a.pad = 1;
  a.weight = r.c2w;
  a.ldw = r.c2_ldw;
  a.Cout = Co;
  a.bias = r.c2b;
  a.out = out;
  a.ldy = Co;
  a.out_f32 = r.out_f32 ? 1 : 0;
  if (r.shortcut) {
    const void* xs = x;
    if (r.in_f32) {
      void* t = sc.alloc<uint16_t>(px * Ci);
      LAUNCH(kOther, 0.0, px * Ci * 6.0,
             dlm_cast_f32_to_f16(static_cast<const float*>(x), t, (long long)(px * Ci), kWideIn, stream));
      xs = t;
    }
    a.src1a = xs;
    a.C1a = Ci;
    a.ld1a = Ci;
  } else {
    a.residual = x;
    a.res_ld = Co;
    a.res_f32 = r.in_f32 ? 1 : 0;
  }
  LAUNCH(kConv, 2.0 * px * Co * (9.0 * Co + (r.shortcut ? Ci : 0)), 0.0,
         dlm_conv2d_nhwc_fp16(&a, stream));
}

// Single-head attention over all pixels (src/kernels/vae_decode.cu:654-692):
// x + to_out(softmax(q k^T / sqrt(C)) v), q|k|v = GroupNorm(x) W^T + b.
void VAE::attention(const Attn& at, const void* x, void* out, int N, int HW, void* stream) {
  const int C = at.C;
  const size_t px = (size_t)N * HW;
  DeviceArenaScope sc(DeviceArenaId::VAE);
  void* hn = sc.alloc<uint16_t>(px * C);
  gn(x, false, C, at.ng, at.nb, hn, N, HW, false, stream);
  // Q|K as [N*HW, 2C], V^T as [N, C, HW]
  char* qk = static_cast<char*>(sc.alloc_bytes(px * 2 * C * kH));
  char* vt = static_cast<char*>(sc.alloc_bytes(px * C * kH));
  LAUNCH(kLinear, 2.0 * px * 3 * C * C, 0.0,
         dlm_linear_vt_fp16(hn, C, at.wqkv, C, at.bqkv, qk, 2 * C, vt, 2 * C, HW, HW, (int)px, 3 * C,
                            C, stream));
  // query rows per pass: fp32 scores for one pass stay within 1 GiB
  const long long cap = std::max<long long>(256, ((1LL << 30) / ((long long)HW * 4)) & ~7LL);
  const int rows = (int)std::min<long long>(HW, cap);
  float* scores = static_cast<float*>(sc.alloc_bytes((size_t)rows * HW * 4));
  void* P = sc.alloc_bytes((size_t)rows * HW * kH);
  char* o = static_cast<char*>(sc.alloc_bytes(px * C * kH));
  const float scale = 1.0f / std::sqrt((float)C);
  for (int b = 0; b < N; ++b) {
    const char* qb = qk + (size_t)b * HW * 2 * C * kH;
    const char* kb = qb + (size_t)C * kH;
    const char* vb = vt + (size_t)b * C * HW * kH;
    for (int r0 = 0; r0 < HW; r0 += rows) {
      const int m = std::min(rows, HW - r0);
      LAUNCH(kAttention, 2.0 * m * HW * C, 0.0,
             dlm_linear_f32out_fp16(qb + (size_t)r0 * 2 * C * kH, 2 * C, kb, 2 * C, nullptr, nullptr,
                                    0, scores, HW, m, HW, C, scale, 0.0f, DLM_ACT_NONE, stream));
      LAUNCH(kAttention, 0.0, (double)m * HW * 6.0,
             dlm_softmax_rows_f32_fp16(scores, HW, P, HW, m, HW, stream));
      LAUNCH(kAttention, 2.0 * m * HW * C, 0.0,
             dlm_linear_fp16(P, HW, vb, HW, nullptr, nullptr, 0,
                             o + ((size_t)b * HW + r0) * C * kH, C, m, C, HW, 1.0f, 0.0f, DLM_ACT_NONE,
                             stream));
    }
  }
  LAUNCH(kLinear, 2.0 * px * C * C, 0.0,
         dlm_linear_fp16(o, C, at.wo, C, at.bo, x, C, out, C, (int)px, C, C, 1.0f, 1.0f, DLM_ACT_NONE,
                         stream));
}

void VAE::decode(int N, int h, int w, const void* latent, void* image, void* stream) {
  if (!packed_) throw std::runtime_error("VAE::decode: prepare() has not run");
  if (N <= 0 || N > 16) throw std::invalid_argument("VAE::decode: N must be in [1, 16]");
  if (h <= 0 || w <= 0 || ((long long)h * w) % 8 != 0)
    throw std::invalid_argument("VAE::decode: h * w must be a positive multiple of 8");
  if (!latent || !image) throw std::invalid_argument("VAE::decode: NULL input");
  const VaeConfig& c = cfg_;
  const int L = c.latent_channels, Cm = c.up_ch(0);
  const int HW0 = h * w;
  prof_next_ = 0;
  // two carry buffers sized for the widest activation of the walk
  size_t carry = (size_t)N * HW0 * Cm * kH;
  {
    size_t hw = HW0;
    for (int i = 0; i < 4; ++i) {
      const size_t eb = i >= c.fp32_from ? 4 : 2;
      carry = std::max(carry, (size_t)N * hw * c.up_ch(i) * eb);
      if (i < 3) {
        hw *= 4;
        carry = std::max(carry, (size_t)N * hw * c.up_ch(i) * eb);
      }
    }
  }
  if (carry / 4 >= (size_t(1) << 31))
    throw std::invalid_argument("VAE::decode: activation too large (> 2^31 fp32 elements)");
  DeviceArenaScope scope(DeviceArenaId::VAE);
  void* A = scope.alloc_bytes(carry);
  void* B = scope.alloc_bytes(carry);
  // latent NCHW -> channels-last, 8 channels (zero padded); post_quant_conv's
  // output zero-padded to 64 channels for conv_in
  {
    DeviceArenaScope sc(DeviceArenaId::VAE);
    void* x8 = sc.alloc<uint16_t>((size_t)N * HW0 * 8);
    void* pq = sc.alloc<uint16_t>((size_t)N * HW0 * kPqPad);
    LAUNCH(kOther, 0.0, 0.0, dlm_nchw_to_nhwc_fp16(latent, x8, N, L, HW0, 8, stream));
    DLM_CALL(dlm_memset_async(pq, 0, (size_t)N * HW0 * kPqPad * kH, stream));
    conv(pqc_, x8, 8, 8, pq, L, kPqPad, false, N, h, w, 1, false, stream);
    stage("post_quant_conv_out", pq, (size_t)N * HW0 * kPqPad, kPqPad, false, stream);
    conv(conv_in_, pq, kPqPad, kPqPad, A, Cm, Cm, false, N, h, w, 3, false, stream);
  }
  stage("conv_in_out", A, (size_t)N * HW0 * Cm, Cm, false, stream);
  // mid block
  resnet(res_[0], A, B, N, h, w, stream);
  attention(attn_, B, A, N, HW0, stream);
  resnet(res_[1], A, B, N, h, w, stream);
  void* cur = B;
  void* nxt = A;
  stage("mid_block_out", cur, (size_t)N * HW0 * Cm, Cm, false, stream);
  // up blocks
  size_t ri = 2;
  int H = h, W = w;
  for (int i = 0; i < 4; ++i) {
    const int C = c.up_ch(i);
    const bool f32 = i >= c.fp32_from;
    for (int r = 0; r < c.layers; ++r) {
      resnet(res_[ri++], cur, nxt, N, H, W, stream);
      std::swap(cur, nxt);
    }
    if (i < 3) {
      DeviceArenaScope sc(DeviceArenaId::VAE);
      const void* x = cur;
      if (f32) {
        const size_t n = (size_t)N * H * W * C;
        void* t = sc.alloc<uint16_t>(n);
        LAUNCH(kOther, 0.0, n * 6.0,
               dlm_cast_f32_to_f16(static_cast<const float*>(cur), t, (long long)n, kWideIn, stream));
        x = t;
      }
      conv(ups_[i], x, C, C, nxt, C, C, f32, N, H, W, 3, true, stream);
      std::swap(cur, nxt);
      H *= 2;
      W *= 2;
    }
    static const char* names[4] = {"up_block_0_out", "up_block_1_out", "up_block_2_out",
                                   "up_block_3_out"};
    stage(names[i], cur, (size_t)N * H * W * C, C, f32, stream);
  }
  if (ri != res_.size()) throw std::logic_error("VAE::decode: graph walk does not match the packed weights");
  // conv_norm_out + SiLU + conv_out, written NCHW
  {
    const int C = c.up_ch(3);
    DeviceArenaScope sc(DeviceArenaId::VAE);
    void* g = sc.alloc<uint16_t>((size_t)N * H * W * C);
    gn(cur, 3 >= c.fp32_from, C, norm_out_g_, norm_out_b_, g, N, H * W, true, stream);
    dlm_conv_nhwc_args a{};
    a.src0a = g;
    a.C0a = C;
    a.ld0a = C;
    a.N = N;
    a.H = H;
    a.W = W;
    a.KH = 3;
    a.KW = 3;
    a.stride = 1;
    a.pad = 1;
    a.weight = conv_out_.w;
    a.ldw = conv_out_.ldw;
    a.Cout = c.out_channels;
    a.bias = conv_out_.b;
    a.out = image;
    a.ldy = c.out_channels;
    a.out_nchw = 1;
    LAUNCH(kConv, 2.0 * N * H * W * c.out_channels * 9.0 * C, 0.0, dlm_conv2d_nhwc_fp16(&a, stream));
  }
  stage("final_image", image, (size_t)N * c.out_channels * H * W, c.out_channels, false, stream);
}

}  // namespace dollama
