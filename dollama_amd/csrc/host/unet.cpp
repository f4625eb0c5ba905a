// SDXL UNet driver (see unet.hpp).  Host C++ only: every device operation is
// a call into the C ABI of include/dlm.h.
#include "unet.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <stdexcept>

#include "check.hpp"
#include "device_arena.hpp"

namespace dollama {

// Input channels of conv_in after padding (the latent's 4 channels, zero
// filled): a multiple of 64 puts the conv on the DMA implicit-GEMM core.
static constexpr int kConvInPad = 64;

// Launch one C-ABI kernel call; when profiling, its kernels carry an event
// pair in their own dispatches (dlm_prof_arm).
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
constexpr size_t kH = 2;  // bytes per fp16

// Algorithmic HBM bytes of one fp16 linear Y[M, Ny] = X[M, K] W[N, K]^T
// (+ residual [M, Ny]): each operand read once, the output written once.
double lin_bytes(double M, double N, double K, double Ny, bool residual) {
  return 2.0 * (M * K + N * K + M * Ny + (residual ? M * Ny : 0.0));
}

std::string shape_str(const Shape& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? "," : "") + std::to_string(s[i]);
  return r + "]";
}

void add_resnet(std::vector<WeightSpec>& v, const std::string& p, int Ci, int Co, int T) {
  v.push_back({p + "norm1.weight", {Ci}});
  v.push_back({p + "norm1.bias", {Ci}});
  v.push_back({p + "conv1.weight", {Co, Ci, 3, 3}});
  v.push_back({p + "conv1.bias", {Co}});
  v.push_back({p + "time_emb_proj.weight", {Co, T}});
  v.push_back({p + "time_emb_proj.bias", {Co}});
  v.push_back({p + "norm2.weight", {Co}});
  v.push_back({p + "norm2.bias", {Co}});
  v.push_back({p + "conv2.weight", {Co, Co, 3, 3}});
  v.push_back({p + "conv2.bias", {Co}});
  if (Ci != Co) {
    v.push_back({p + "conv_shortcut.weight", {Co, Ci, 1, 1}});
    v.push_back({p + "conv_shortcut.bias", {Co}});
  }
}

void add_t2d(std::vector<WeightSpec>& v, const std::string& p, int C, int depth, int cross) {
  v.push_back({p + "norm.weight", {C}});
  v.push_back({p + "norm.bias", {C}});
  v.push_back({p + "proj_in.weight", {C, C}});
  v.push_back({p + "proj_in.bias", {C}});
  for (int l = 0; l < depth; ++l) {
    const std::string b = p + "transformer_blocks." + std::to_string(l) + ".";
    for (const char* n : {"norm1", "norm2", "norm3"}) {
      v.push_back({b + n + ".weight", {C}});
      v.push_back({b + n + ".bias", {C}});
    }
    for (const char* n : {"to_q", "to_k", "to_v"}) v.push_back({b + "attn1." + n + ".weight", {C, C}});
    v.push_back({b + "attn1.to_out.0.weight", {C, C}});
    v.push_back({b + "attn1.to_out.0.bias", {C}});
    v.push_back({b + "attn2.to_q.weight", {C, C}});
    v.push_back({b + "attn2.to_k.weight", {C, cross}});
    v.push_back({b + "attn2.to_v.weight", {C, cross}});
    v.push_back({b + "attn2.to_out.0.weight", {C, C}});
    v.push_back({b + "attn2.to_out.0.bias", {C}});
    v.push_back({b + "ff.net.0.proj.weight", {8 * C, C}});
    v.push_back({b + "ff.net.0.proj.bias", {8 * C}});
    v.push_back({b + "ff.net.2.weight", {C, 4 * C}});
    v.push_back({b + "ff.net.2.bias", {C}});
  }
  v.push_back({p + "proj_out.weight", {C, C}});
  v.push_back({p + "proj_out.bias", {C}});
}

// Resnet (Ci, Co) list and transformer placement in forward order.
struct LevelPlan {
  // up-block resnet input channels: current + popped skip
  static std::vector<std::pair<int, int>> up_res(const UNetConfig& c, int level) {
    const int C0 = c.C0, C1 = c.C1, C2 = c.C2;
    if (level == 0) return {{C2 + C2, C2}, {C2 + C2, C2}, {C2 + C1, C2}};
    if (level == 1) return {{C2 + C1, C1}, {C1 + C1, C1}, {C1 + C0, C1}};
    return {{C1 + C0, C0}, {C0 + C0, C0}, {C0 + C0, C0}};
  }
};
}  // namespace

std::vector<WeightSpec> unet_weight_specs(const UNetConfig& c) {
  std::vector<WeightSpec> v;
  const int T = c.time_dim();
  v.push_back({"conv_in.weight", {c.C0, c.in_channels, 3, 3}});
  v.push_back({"conv_in.bias", {c.C0}});
  v.push_back({"time_embedding.linear_1.weight", {T, c.C0}});
  v.push_back({"time_embedding.linear_1.bias", {T}});
  v.push_back({"time_embedding.linear_2.weight", {T, T}});
  v.push_back({"time_embedding.linear_2.bias", {T}});
  v.push_back({"add_embedding.linear_1.weight", {T, c.add_dim()}});
  v.push_back({"add_embedding.linear_1.bias", {T}});
  v.push_back({"add_embedding.linear_2.weight", {T, T}});
  v.push_back({"add_embedding.linear_2.bias", {T}});
  // down
  add_resnet(v, "down_blocks.0.resnets.0.", c.C0, c.C0, T);
  add_resnet(v, "down_blocks.0.resnets.1.", c.C0, c.C0, T);
  v.push_back({"down_blocks.0.downsamplers.0.conv.weight", {c.C0, c.C0, 3, 3}});
  v.push_back({"down_blocks.0.downsamplers.0.conv.bias", {c.C0}});
  add_resnet(v, "down_blocks.1.resnets.0.", c.C0, c.C1, T);
  add_t2d(v, "down_blocks.1.attentions.0.", c.C1, c.depth1, c.cross_dim);
  add_resnet(v, "down_blocks.1.resnets.1.", c.C1, c.C1, T);
  add_t2d(v, "down_blocks.1.attentions.1.", c.C1, c.depth1, c.cross_dim);
  v.push_back({"down_blocks.1.downsamplers.0.conv.weight", {c.C1, c.C1, 3, 3}});
  v.push_back({"down_blocks.1.downsamplers.0.conv.bias", {c.C1}});
  add_resnet(v, "down_blocks.2.resnets.0.", c.C1, c.C2, T);
  add_t2d(v, "down_blocks.2.attentions.0.", c.C2, c.depth2, c.cross_dim);
  add_resnet(v, "down_blocks.2.resnets.1.", c.C2, c.C2, T);
  add_t2d(v, "down_blocks.2.attentions.1.", c.C2, c.depth2, c.cross_dim);
  // mid
  add_resnet(v, "mid_block.resnets.0.", c.C2, c.C2, T);
  add_t2d(v, "mid_block.attentions.0.", c.C2, c.depth2, c.cross_dim);
  add_resnet(v, "mid_block.resnets.1.", c.C2, c.C2, T);
  // up
  for (int u = 0; u < 3; ++u) {
    const auto rs = LevelPlan::up_res(c, u);
    const int C = u == 0 ? c.C2 : (u == 1 ? c.C1 : c.C0);
    const int depth = u == 0 ? c.depth2 : (u == 1 ? c.depth1 : 0);
    for (int r = 0; r < 3; ++r) {
      const std::string p = "up_blocks." + std::to_string(u) + ".";
      add_resnet(v, p + "resnets." + std::to_string(r) + ".", rs[r].first, rs[r].second, T);
      if (depth > 0) add_t2d(v, p + "attentions." + std::to_string(r) + ".", C, depth, c.cross_dim);
    }
    if (u < 2) {
      const std::string p = "up_blocks." + std::to_string(u) + ".upsamplers.0.conv.";
      v.push_back({p + "weight", {C, C, 3, 3}});
      v.push_back({p + "bias", {C}});
    }
  }
  v.push_back({"conv_norm_out.weight", {c.C0}});
  v.push_back({"conv_norm_out.bias", {c.C0}});
  v.push_back({"conv_out.weight", {c.out_channels, c.C0, 3, 3}});
  v.push_back({"conv_out.bias", {c.out_channels}});
  return v;
}

UNet::UNet(const UNetConfig& cfg) : cfg_(cfg) {
  const UNetConfig& c = cfg_;
  for (int C : {c.C0, c.C1, c.C2}) {
    if (C <= 0 || C % 64 != 0) throw std::invalid_argument("UNet: channel counts must be multiples of 64");
    if (C % c.groups != 0) throw std::invalid_argument("UNet: channels not divisible by groups");
    if (C % c.head_dim != 0) throw std::invalid_argument("UNet: channels not divisible by head_dim");
  }
  if (c.head_dim != 64) throw std::invalid_argument("UNet: head_dim must be 64");
  if (c.cross_dim % 8 || c.text_dim % 8 || c.id_dim % 8)
    throw std::invalid_argument("UNet: cross/text/id dims must be multiples of 8");
  if (c.in_channels > kConvInPad)
    throw std::invalid_argument("UNet: more than 64 input channels not supported");
}

UNet::~UNet() {
  clear_graphs();
  for (Backup& b : backups_) (void)dlm_free(b.copy);
  if (packed_) (void)dlm_free(packed_);
  for (void* e : prof_events_) (void)dlm_event_destroy(e);
}

// ---------------------------------------------------------------------------
// Runtime LoRA (reference src/infer/unet.cu:373-458): W += scale * (B @ A) on
// the resident weights.  delta = scale * (B @ A) is formed in fp16 by the
// MFMA GEMM (fp32 accumulate), packed exactly like the weight it patches
// (plain rows, GEGLU interleave or the per-tap conv layout) and added
// element-wise (fp32 add, fp16 round), so W' = f16(W + f16(delta)) as in the
// reference.  The packed region is copied aside before its first patch;
// clear_loras() copies every saved region back (bit-exact revert).
// ---------------------------------------------------------------------------
void UNet::apply_lora(const std::string& key, const void* dA, const void* dB, int rank,
                      int in_flat, int out_dim, float scale, void* stream) {
  if (!prepared()) throw std::logic_error("UNet::apply_lora before prepare()");
  auto it = placed_.find(key);
  if (it == placed_.end()) throw std::invalid_argument("lora: '" + key + "' is not a UNet weight");
  const Placement& pl = it->second;
  const size_t n = (size_t)out_dim * in_flat;
  size_t wn = pl.elems;
  if (pl.kind == Placement::kConv) wn = (size_t)pl.Co * pl.Ci * pl.k * pl.k;
  if (rank <= 0 || n != wn)
    throw std::invalid_argument("lora: '" + key + "' delta shape does not match the weight");
  if (!patched_.count(key)) {  // save the packed region once
    Backup bk;
    bk.dst = pl.dst;
    bk.bytes = pl.elems * kH;
    DLM_CALL(dlm_malloc(&bk.copy, bk.bytes));
    DLM_CALL(dlm_memcpy_async(bk.copy, bk.dst, bk.bytes, 2, stream));
    backups_.push_back(bk);
    patched_.insert(key);
  }
  DeviceArenaScope sc(DeviceArenaId::UNet);
  void* delta = sc.alloc<uint16_t>(n);
  DLM_CALL(dlm_gemm_fp16(dB, dA, delta, out_dim, in_flat, rank, scale, 0.0f, 0, 0, stream));
  if (pl.kind == Placement::kCopy) {
    DLM_CALL(dlm_add_fp16(pl.dst, delta, pl.dst, (int)n, stream));
  } else if (pl.kind == Placement::kGeglu) {
    void* packed = sc.alloc<uint16_t>(n);
    DLM_CALL(dlm_geglu_pack_fp16(delta, nullptr, packed, nullptr, pl.Co / 2, pl.Ci, stream));
    DLM_CALL(dlm_add_fp16(pl.dst, packed, pl.dst, (int)n, stream));
  } else {
    DLM_CALL(dlm_conv_weight_pack_add_fp16(delta, pl.dst, pl.Co, pl.Ci, pl.k, pl.k, pl.cin_pad,
                                           pl.ld, pl.col0, stream));
  }
  auto fd = fold_deps_.find(key);
  if (fd != fold_deps_.end())
    for (const LnFold& f : fd->second) refold(f, stream);
  DLM_CALL(dlm_stream_synchronize(stream));  // the arena scope ends here
}

void UNet::clear_loras(void* stream) {
  for (auto it = backups_.rbegin(); it != backups_.rend(); ++it)
    DLM_CALL(dlm_memcpy_async(it->dst, it->copy, it->bytes, 2, stream));
  for (const std::string& key : patched_) {  // folds of restored weights
    auto fd = fold_deps_.find(key);
    if (fd != fold_deps_.end())
      for (const LnFold& f : fd->second) refold(f, stream);
  }
  DLM_CALL(dlm_stream_synchronize(stream));
  for (Backup& b : backups_) dlm_free(b.copy);
  backups_.clear();
  patched_.clear();
}

void UNet::read_weight(const std::string& key, void* host, size_t bytes, void* stream) const {
  if (!prepared()) throw std::logic_error("UNet::read_weight before prepare()");
  auto it = placed_.find(key);
  if (it == placed_.end()) throw std::invalid_argument("'" + key + "' is not a resident weight");
  const Placement& pl = it->second;
  const size_t n = pl.kind == Placement::kConv ? (size_t)pl.Co * pl.Ci * pl.k * pl.k : pl.elems;
  if (bytes != n * kH) throw std::invalid_argument("'" + key + "' holds " + std::to_string(n * kH) + " bytes");
  std::vector<uint16_t> raw(pl.elems);
  DLM_CALL(dlm_memcpy_async(raw.data(), pl.dst, pl.elems * kH, 1, stream));
  DLM_CALL(dlm_stream_synchronize(stream));
  uint16_t* out = static_cast<uint16_t*>(host);
  if (pl.kind == Placement::kCopy) {
    std::copy(raw.begin(), raw.end(), out);
  } else if (pl.kind == Placement::kGeglu) {  // packed row 8q+s <- value 4q+s | gate d+4q+s-4
    const int d = pl.Co / 2, K = pl.Ci;
    for (int r = 0; r < pl.Co; ++r) {
      const int q = r / 8, s = r % 8;
      const int src = s < 4 ? 4 * q + s : d + 4 * q + (s - 4);
      std::copy(raw.begin() + (size_t)r * K, raw.begin() + (size_t)(r + 1) * K, out + (size_t)src * K);
    }
  } else {  // packed conv segment (dlm_conv_weight_pack_fp16's column order) <- [co][ci][tap]
    const int taps = pl.k * pl.k;
    auto col = [&](int t, int ci) -> size_t {
      if (pl.cin_pad % 64 == 0) return ((size_t)(ci / 64) * taps + t) * 64 + ci % 64;
      return (size_t)t * pl.cin_pad + ci;
    };
    for (int co = 0; co < pl.Co; ++co)
      for (int ci = 0; ci < pl.Ci; ++ci)
        for (int t = 0; t < taps; ++t)
          out[((size_t)co * pl.Ci + ci) * taps + t] = raw[(size_t)co * pl.ld + pl.col0 + col(t, ci)];
  }
}

void UNet::set_profiling(bool on) { prof_on_ = on; }

void UNet::prof_begin(int cls, double flops, double bytes, void* stream) {
  if (!prof_on_) return;
  if (prof_next_ * 2 + 2 > prof_events_.size()) {
    for (int i = 0; i < 2; ++i) {
      void* e = nullptr;
      DLM_CALL(dlm_event_create(&e));
      prof_events_.push_back(e);
    }
  }
  if (prof_recs_.size() <= prof_next_) prof_recs_.resize(prof_next_ + 1);
  prof_recs_[prof_next_] = ProfRec{cls, flops, bytes, std::string(), {0, 0, 0, 0}};
  (void)dlm_last_kernel(1);
  // the kernels of the call carry the event pair in their own dispatches
  DLM_CALL(dlm_prof_arm(prof_events_[prof_next_ * 2], prof_events_[prof_next_ * 2 + 1]));
  (void)stream;
}

void UNet::prof_end(void* stream) {
  if (!prof_on_) return;
  if (dlm_prof_disarm() == 0) {  // no kernel in the call: an empty interval
    DLM_CALL(dlm_event_record(prof_events_[prof_next_ * 2], stream));
    DLM_CALL(dlm_event_record(prof_events_[prof_next_ * 2 + 1], stream));
  }
  DLM_CALL(dlm_last_kernel_dims(prof_recs_[prof_next_].dims));
  prof_recs_[prof_next_].kernel = dlm_last_kernel(1);
  ++prof_next_;
}

std::vector<UNet::KernelStats> UNet::profile_kernels(void* stream) {
  DLM_CALL(dlm_stream_synchronize(stream));
  std::vector<KernelStats> out;
  std::map<std::string, size_t> at;
  for (size_t i = 0; i < prof_next_ && i < prof_recs_.size(); ++i) {
    float ms = 0.0f;
    DLM_CALL(dlm_event_elapsed_ms(&ms, prof_events_[2 * i], prof_events_[2 * i + 1]));
    const ProfRec& r = prof_recs_[i];
    const std::string name = r.kernel.empty() ? "?" : r.kernel;
    auto it = at.find(name);
    if (it == at.end()) {
      it = at.emplace(name, out.size()).first;
      out.push_back(KernelStats{name, r.cls, 0, 0.0, 0.0, 0.0});
    }
    KernelStats& k = out[it->second];
    k.count += 1;
    k.ms += ms;
    k.flops += r.flops;
    k.bytes += r.bytes;
    if (r.dims[0] > 0) ++k.dims[std::vector<int>(r.dims, r.dims + 4)];
  }
  return out;
}

std::vector<UNet::ClassStats> UNet::profile_report(void* stream) {
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

void UNet::set_weight(const std::string& name, const void* dptr, const Shape& shape) {
  if (!dptr) throw std::invalid_argument("UNet::set_weight: NULL pointer for " + name);
  srcs_[name] = Src{dptr, shape};
}

const UNet::Src& UNet::src(const std::string& name, const Shape& shape) const {
  auto it = srcs_.find(name);
  if (it == srcs_.end()) throw std::runtime_error("UNet: missing weight '" + name + "'");
  if (it->second.shape != shape)
    throw std::runtime_error("UNet: weight '" + name + "' has shape " + shape_str(it->second.shape) +
                             ", expected " + shape_str(shape));
  return it->second;
}

void* UNet::take(size_t elems) {
  const size_t off = cursor_;
  cursor_ += (elems * kH + 255) & ~size_t(255);
  return sizing_ ? nullptr : packed_ + off;
}

const void* UNet::copy_of(const std::string& name, const Shape& shape, void* stream) {
  const Src& s = src(name, shape);
  size_t n = 1;
  for (int64_t d : shape) n *= (size_t)d;
  void* dst = take(n);
  if (!sizing_) {
    DLM_CALL(dlm_memcpy_async(dst, s.ptr, n * kH, 2, stream));
    place_copy(name, dst, n);
  }
  return dst;
}

UNet::LnFold UNet::make_fold(const void* w, const void* g, const void* b, const void* bias, int N,
                             int K, const std::vector<std::string>& deps, void* stream) {
  LnFold f;
  f.w = w;
  f.g = g;
  f.b = b;
  f.bias = bias;
  f.N = N;
  f.K = K;
  f.wf = take((size_t)N * K);
  f.c1 = static_cast<float*>(take((size_t)2 * N));  // fp32: two halves per element
  f.c2 = static_cast<float*>(take((size_t)2 * N));
  if (!sizing_) {
    refold(f, stream);
    for (const std::string& d : deps) fold_deps_[d].push_back(f);
  }
  return f;
}

void UNet::refold(const LnFold& f, void* stream) {
  DLM_CALL(dlm_ln_fold_fp16(f.w, f.K, f.N, f.K, f.g, f.b, f.bias, f.wf, f.K, f.c1, f.c2, stream));
}

void UNet::set_ln_fold(int mask) {
  if (mask < 0 || mask > 3) throw std::invalid_argument("UNet::set_ln_fold: mask must be in [0, 3]");
  if (mask != ln_fold_) clear_graphs();
  ln_fold_ = mask;
}

void UNet::set_gn_fold(bool on) {
  if (on != gn_fold_) clear_graphs();
  gn_fold_ = on;
}

void UNet::place_copy(const std::string& name, void* dst, size_t n) {
  Placement pl;
  pl.kind = Placement::kCopy;
  pl.dst = static_cast<char*>(dst);
  pl.elems = n;
  placed_[name] = pl;
}

void UNet::place_conv(const std::string& name, void* dst, int Co, int Ci, int k, int cin_pad,
                      int ld, int col0) {
  Placement pl;
  pl.kind = Placement::kConv;
  pl.dst = static_cast<char*>(dst);
  pl.elems = (size_t)Co * ld;  // the whole packed rows (shared with a second K segment)
  pl.Co = Co;
  pl.Ci = Ci;
  pl.k = k;
  pl.cin_pad = cin_pad;
  pl.ld = ld;
  pl.col0 = col0;
  placed_[name] = pl;
}

UNet::Conv UNet::pack_conv(const std::string& p, int Co, int Ci, int k, int cin_pad, void* stream) {
  Conv c;
  c.ldw = k * k * cin_pad;
  void* w = take((size_t)Co * c.ldw);
  const Src& s = src(p + "weight", {Co, Ci, k, k});
  if (!sizing_) {
    DLM_CALL(dlm_conv_weight_pack_fp16(s.ptr, w, Co, Ci, k, k, cin_pad, c.ldw, 0, stream));
    place_conv(p + "weight", w, Co, Ci, k, cin_pad, c.ldw, 0);
  }
  c.w = w;
  c.b = copy_of(p + "bias", {Co}, stream);
  return c;
}

UNet::Resnet UNet::pack_resnet(const std::string& p, int Ci, int Co, void* stream) {
  Resnet r;
  r.Ci = Ci;
  r.Co = Co;
  r.shortcut = Ci != Co;
  r.n1g = copy_of(p + "norm1.weight", {Ci}, stream);
  r.n1b = copy_of(p + "norm1.bias", {Ci}, stream);
  void* c1 = take((size_t)Co * 9 * Ci);
  const Src& s1 = src(p + "conv1.weight", {Co, Ci, 3, 3});
  if (!sizing_) {
    DLM_CALL(dlm_conv_weight_pack_fp16(s1.ptr, c1, Co, Ci, 3, 3, Ci, 9 * Ci, 0, stream));
    place_conv(p + "conv1.weight", c1, Co, Ci, 3, Ci, 9 * Ci, 0);
  }
  r.c1w = c1;
  r.c1b = copy_of(p + "conv1.bias", {Co}, stream);
  r.n2g = copy_of(p + "norm2.weight", {Co}, stream);
  r.n2b = copy_of(p + "norm2.bias", {Co}, stream);
  // conv2 (+ conv_shortcut appended as a second K segment)
  r.c2_ldw = 9 * Co + (r.shortcut ? Ci : 0);
  void* c2 = take((size_t)Co * r.c2_ldw);
  const Src& s2 = src(p + "conv2.weight", {Co, Co, 3, 3});
  if (!sizing_) {
    DLM_CALL(dlm_conv_weight_pack_fp16(s2.ptr, c2, Co, Co, 3, 3, Co, r.c2_ldw, 0, stream));
    place_conv(p + "conv2.weight", c2, Co, Co, 3, Co, r.c2_ldw, 0);
  }
  r.c2w = c2;
  if (r.shortcut) {
    const Src& ss = src(p + "conv_shortcut.weight", {Co, Ci, 1, 1});
    if (!sizing_) {
      DLM_CALL(dlm_conv_weight_pack_fp16(ss.ptr, c2, Co, Ci, 1, 1, Ci, r.c2_ldw, 9 * Co, stream));
      place_conv(p + "conv_shortcut.weight", c2, Co, Ci, 1, Ci, r.c2_ldw, 9 * Co);
    }
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

UNet::T2D UNet::pack_t2d(const std::string& p, int C, int depth, void* stream) {
  T2D t;
  t.C = C;
  t.ng = copy_of(p + "norm.weight", {C}, stream);
  t.nb = copy_of(p + "norm.bias", {C}, stream);
  t.pin_w = copy_of(p + "proj_in.weight", {C, C}, stream);
  t.pin_b = copy_of(p + "proj_in.bias", {C}, stream);
  for (int l = 0; l < depth; ++l) {
    const std::string b = p + "transformer_blocks." + std::to_string(l) + ".";
    Block k;
    k.ln1g = copy_of(b + "norm1.weight", {C}, stream);
    k.ln1b = copy_of(b + "norm1.bias", {C}, stream);
    k.ln2g = copy_of(b + "norm2.weight", {C}, stream);
    k.ln2b = copy_of(b + "norm2.bias", {C}, stream);
    k.ln3g = copy_of(b + "norm3.weight", {C}, stream);
    k.ln3b = copy_of(b + "norm3.bias", {C}, stream);
    // fused q/k/v rows
    char* qkv = static_cast<char*>(take((size_t)3 * C * C));
    int i = 0;
    for (const char* n : {"to_q", "to_k", "to_v"}) {
      const Src& s = src(b + "attn1." + n + ".weight", {C, C});
      if (!sizing_) {
        DLM_CALL(dlm_memcpy_async(qkv + (size_t)i * C * C * kH, s.ptr, (size_t)C * C * kH, 2, stream));
        place_copy(b + "attn1." + n + ".weight", qkv + (size_t)i * C * C * kH, (size_t)C * C);
      }
      ++i;
    }
    k.wqkv = qkv;
    k.wo1 = copy_of(b + "attn1.to_out.0.weight", {C, C}, stream);
    k.bo1 = copy_of(b + "attn1.to_out.0.bias", {C}, stream);
    k.wq2 = copy_of(b + "attn2.to_q.weight", {C, C}, stream);
    k.wo2 = copy_of(b + "attn2.to_out.0.weight", {C, C}, stream);
    k.bo2 = copy_of(b + "attn2.to_out.0.bias", {C}, stream);
    // GEGLU projection in the 4-row value/gate interleave
    void* w1 = take((size_t)8 * C * C);
    void* b1 = take((size_t)8 * C);
    const Src& sw = src(b + "ff.net.0.proj.weight", {8 * C, C});
    const Src& sb = src(b + "ff.net.0.proj.bias", {8 * C});
    if (!sizing_) {
      DLM_CALL(dlm_geglu_pack_fp16(sw.ptr, sb.ptr, w1, b1, 4 * C, C, stream));
      Placement pl;
      pl.kind = Placement::kGeglu;
      pl.dst = static_cast<char*>(w1);
      pl.elems = (size_t)8 * C * C;
      pl.Co = 8 * C;
      pl.Ci = C;
      placed_[b + "ff.net.0.proj.weight"] = pl;
    }
    k.wff1 = w1;
    k.bff1 = b1;
    k.wff2 = copy_of(b + "ff.net.2.weight", {C, 4 * C}, stream);
    k.bff2 = copy_of(b + "ff.net.2.bias", {C}, stream);
    // folded copies of the LayerNorm-consuming linears
    k.fqkv = make_fold(k.wqkv, k.ln1g, k.ln1b, nullptr, 3 * C, C,
                       {b + "attn1.to_q.weight", b + "attn1.to_k.weight", b + "attn1.to_v.weight",
                        b + "norm1.weight", b + "norm1.bias"},
                       stream);
    k.fq2 = make_fold(k.wq2, k.ln2g, k.ln2b, nullptr, C, C,
                      {b + "attn2.to_q.weight", b + "norm2.weight", b + "norm2.bias"}, stream);
    k.kv_off = kv_total_ / 2;  // row offset of this block's K (and, past all K rows, its V)
    kv_total_ += 2 * C;
    t.blocks.push_back(k);
  }
  t.pout_w = copy_of(p + "proj_out.weight", {C, C}, stream);
  t.pout_b = copy_of(p + "proj_out.bias", {C}, stream);
  return t;
}

void UNet::pack_all(void* stream) {
  const UNetConfig& c = cfg_;
  const int T = c.time_dim();
  res_.clear();
  t2d_.clear();
  res_names_.clear();
  t2d_names_.clear();
  kv_total_ = 0;
  tproj_total_ = 0;
  cursor_ = 0;
  // the latent's channels padded to 64: the conv then runs on the DMA core's
  // implicit GEMM (K = 9 x 64) instead of the register-staged small-channel
  // kernel
  conv_in_ = pack_conv("conv_in.", c.C0, c.in_channels, 3, kConvInPad, stream);
  te1w_ = copy_of("time_embedding.linear_1.weight", {T, c.C0}, stream);
  te1b_ = copy_of("time_embedding.linear_1.bias", {T}, stream);
  te2w_ = copy_of("time_embedding.linear_2.weight", {T, T}, stream);
  te2b_ = copy_of("time_embedding.linear_2.bias", {T}, stream);
  ae1w_ = copy_of("add_embedding.linear_1.weight", {T, c.add_dim()}, stream);
  ae1b_ = copy_of("add_embedding.linear_1.bias", {T}, stream);
  ae2w_ = copy_of("add_embedding.linear_2.weight", {T, T}, stream);
  ae2b_ = copy_of("add_embedding.linear_2.bias", {T}, stream);

  auto R = [&](const std::string& p, int Ci, int Co) {
    res_names_.push_back(p);
    res_.push_back(pack_resnet(p, Ci, Co, stream));
    res_.back().tproj_off = tproj_total_;
    tproj_total_ += Co;
  };
  auto A = [&](const std::string& p, int C, int depth) {
    t2d_names_.push_back(p);
    t2d_.push_back(pack_t2d(p, C, depth, stream));
  };

  R("down_blocks.0.resnets.0.", c.C0, c.C0);
  R("down_blocks.0.resnets.1.", c.C0, c.C0);
  down0_ = pack_conv("down_blocks.0.downsamplers.0.conv.", c.C0, c.C0, 3, c.C0, stream);
  R("down_blocks.1.resnets.0.", c.C0, c.C1);
  A("down_blocks.1.attentions.0.", c.C1, c.depth1);
  R("down_blocks.1.resnets.1.", c.C1, c.C1);
  A("down_blocks.1.attentions.1.", c.C1, c.depth1);
  down1_ = pack_conv("down_blocks.1.downsamplers.0.conv.", c.C1, c.C1, 3, c.C1, stream);
  R("down_blocks.2.resnets.0.", c.C1, c.C2);
  A("down_blocks.2.attentions.0.", c.C2, c.depth2);
  R("down_blocks.2.resnets.1.", c.C2, c.C2);
  A("down_blocks.2.attentions.1.", c.C2, c.depth2);
  R("mid_block.resnets.0.", c.C2, c.C2);
  A("mid_block.attentions.0.", c.C2, c.depth2);
  R("mid_block.resnets.1.", c.C2, c.C2);
  for (int u = 0; u < 3; ++u) {
    const auto rs = LevelPlan::up_res(c, u);
    const int C = u == 0 ? c.C2 : (u == 1 ? c.C1 : c.C0);
    const int depth = u == 0 ? c.depth2 : (u == 1 ? c.depth1 : 0);
    const std::string p = "up_blocks." + std::to_string(u) + ".";
    for (int r = 0; r < 3; ++r) {
      R(p + "resnets." + std::to_string(r) + ".", rs[r].first, rs[r].second);
      if (depth > 0) A(p + "attentions." + std::to_string(r) + ".", C, depth);
    }
    if (u == 0) up0_ = pack_conv(p + "upsamplers.0.conv.", C, C, 3, C, stream);
    if (u == 1) up1_ = pack_conv(p + "upsamplers.0.conv.", C, C, 3, C, stream);
  }
  norm_out_g_ = copy_of("conv_norm_out.weight", {c.C0}, stream);
  norm_out_b_ = copy_of("conv_norm_out.bias", {c.C0}, stream);
  conv_out_ = pack_conv("conv_out.", c.out_channels, c.C0, 3, c.C0, stream);

  // all resnets' time_emb_proj rows, concatenated in forward order
  {
    char* w = static_cast<char*>(take((size_t)tproj_total_ * T));
    char* b = static_cast<char*>(take((size_t)tproj_total_));
    if (!sizing_) {
      std::vector<std::string> names;
      for (const WeightSpec& s : unet_weight_specs(c))
        if (s.name.find("time_emb_proj.weight") != std::string::npos) names.push_back(s.name);
      // unet_weight_specs lists resnets in forward order, same as res_
      if (names.size() != res_.size()) throw std::logic_error("UNet: resnet count mismatch");
      for (size_t i = 0; i < res_.size(); ++i) {
        const int Co = res_[i].Co;
        const std::string p = names[i].substr(0, names[i].size() - std::string("weight").size());
        const Src& sw = src(p + "weight", {Co, T});
        const Src& sb = src(p + "bias", {Co});
        DLM_CALL(dlm_memcpy_async(w + (size_t)res_[i].tproj_off * T * kH, sw.ptr, (size_t)Co * T * kH, 2, stream));
        place_copy(p + "weight", w + (size_t)res_[i].tproj_off * T * kH, (size_t)Co * T);
        DLM_CALL(dlm_memcpy_async(b + (size_t)res_[i].tproj_off * kH, sb.ptr, (size_t)Co * kH, 2, stream));
      }
    }
    tproj_w_ = w;
    tproj_b_ = b;
  }
  // every transformer block's cross-attention K and V rows, concatenated
  {
    char* w = static_cast<char*>(take((size_t)kv_total_ * c.cross_dim));
    if (!sizing_) {
      std::vector<std::string> prefixes;
      for (const WeightSpec& s : unet_weight_specs(c))
        if (s.name.find("attn2.to_k.weight") != std::string::npos)
          prefixes.push_back(s.name.substr(0, s.name.size() - std::string("to_k.weight").size()));
      size_t bi = 0;
      for (const T2D& t : t2d_) {
        for (const Block& k : t.blocks) {
          const int C = t.C;
          const Src& sk = src(prefixes[bi] + "to_k.weight", {C, c.cross_dim});
          const Src& sv = src(prefixes[bi] + "to_v.weight", {C, c.cross_dim});
          const size_t row = (size_t)c.cross_dim * kH;
          DLM_CALL(dlm_memcpy_async(w + (size_t)k.kv_off * row, sk.ptr, (size_t)C * row, 2, stream));
          DLM_CALL(dlm_memcpy_async(w + (size_t)(kv_total_ / 2 + k.kv_off) * row, sv.ptr,
                                    (size_t)C * row, 2, stream));
          place_copy(prefixes[bi] + "to_k.weight", w + (size_t)k.kv_off * row, (size_t)C * c.cross_dim);
          place_copy(prefixes[bi] + "to_v.weight", w + (size_t)(kv_total_ / 2 + k.kv_off) * row,
                     (size_t)C * c.cross_dim);
          ++bi;
        }
      }
    }
    kv_w_ = w;
  }
}

void UNet::set_graphs(bool on) {
  graphs_on_ = on;
  if (!on) clear_graphs();
}

void UNet::clear_graphs() {
  for (auto& kv : graphs_) (void)dlm_graph_destroy(kv.second);
  graphs_.clear();
  seen_.clear();
}

void UNet::prepare(void* stream) {
  clear_graphs();  // captured graphs hold the old packed weight addresses
  // a re-pack starts from the registered weights: earlier LoRA state is void
  for (Backup& b : backups_) (void)dlm_free(b.copy);
  backups_.clear();
  patched_.clear();
  placed_.clear();
  fold_deps_.clear();
  // pass 1: sizes and validation
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
  // pass 2: fill
  pack_all(stream);
  if (cursor_ != bytes) throw std::logic_error("UNet::prepare: sizing pass disagrees with fill pass");
  DLM_CALL(dlm_stream_synchronize(stream));
  srcs_.clear();
}

// ------------------------------------------------------------------ forward

void UNet::stage(const char* name, const void* p, size_t n, int C, void* stream) {
  if (!hook_) return;
  DLM_CALL(dlm_stream_synchronize(stream));
  hook_(name, p, n, C, hook_user_);
}

// A GroupNorm workspace whose statistics a producer fills (null where the
// chunk statistics do not apply: more than 16384 pixels per sample, or the
// fold is off).
static void* gn_stats_ws(DeviceArenaScope& sc, int B, int C, int HW, bool on = true) {
  if (!on || HW > 16384) return nullptr;
  return sc.alloc_bytes(dlm_group_norm_nhwc_workspace_bytes(B, C, HW));
}

void UNet::gn(const void* xa, int Ca, const void* xb, int Cb, const void* g, const void* b,
              void* out, int B, int HW, float eps, bool silu, void* stream, const void* prestats,
              const void* prestats_b) {
  const int C = Ca + Cb;
  if (xb && prestats && prestats_b) {  // concat(xa, xb), each source's producer statistics
    DeviceArenaScope sc(DeviceArenaId::UNet);
    void* ws = sc.alloc_bytes(dlm_group_norm_nhwc_workspace_bytes(B, C, HW));
    LAUNCH(kGroupNorm, 0.0, 4.0 * B * HW * C,
           dlm_group_norm_nhwc_prestats2_fp16(xa, Ca, Ca, xb, Cb, prestats, prestats_b, g, b, out, C, B, HW, C,
                                              cfg_.groups, eps, silu ? 1 : 0, ws, stream));
    return;
  }
  if (xb) prestats = nullptr;  // one source's statistics do not cover the concatenation
  if (prestats) {
    LAUNCH(kGroupNorm, 0.0, 4.0 * B * HW * C,
           dlm_group_norm_nhwc_prestats_fp16(xa, C, g, b, out, C, B, HW, C, cfg_.groups, eps,
                                             silu ? 1 : 0, const_cast<void*>(prestats), stream));
    return;
  }
  DeviceArenaScope sc(DeviceArenaId::UNet);
  void* ws = sc.alloc_bytes(dlm_group_norm_nhwc_workspace_bytes(B, C, HW));
  LAUNCH(kGroupNorm, 0.0, 4.0 * B * HW * C,
         dlm_group_norm_nhwc_fp16(xa, Ca, Ca, xb, Cb > 0 ? Cb : 8, g, b, out, C, B, HW, C,
                                  cfg_.groups, eps, silu ? 1 : 0, ws, stream));
}

void UNet::conv3(const Conv& c, const void* x, int C, const void* xb, int Cb, void* out, int Co,
                 int B, int H, int W, int stride, bool up, void* stream, int flop_cin, void* gn_stats) {
  dlm_conv_nhwc_args a{};
  a.src0a = x;
  a.C0a = C;
  a.ld0a = C;
  a.src0b = xb;
  a.C0b = Cb;
  a.ld0b = Cb;
  a.N = B;
  a.H = H;
  a.W = W;
  a.KH = 3;
  a.KW = 3;
  a.stride = stride;
  a.pad = 1;
  a.upsample = up ? 1 : 0;
  a.weight = c.w;
  a.ldw = c.ldw;
  a.Cout = Co;
  a.bias = c.b;
  a.out = out;
  a.ldy = Co;
  a.gn_stats = gn_stats;
  const int Ho = (up ? 2 * H : (H + 2 - 3) / stride + 1), Wo = (up ? 2 * W : (W + 2 - 3) / stride + 1);
  const double cin = flop_cin > 0 ? flop_cin : (double)(C + Cb);
  LAUNCH(kConv, 2.0 * B * Ho * Wo * Co * 9.0 * cin,
         2.0 * ((double)B * H * W * (C + Cb) + (double)Co * 9.0 * (C + Cb) + (double)B * Ho * Wo * Co),
         dlm_conv2d_nhwc_fp16(&a, stream));
}

void UNet::resnet(const Resnet& r, const void* xa, int Ca, const void* xb, int Cb, void* out,
                  int B, int H, int W, const void* tproj, void* stream, const void* in_stats,
                  void* out_stats, const void* in_stats_b) {
  const int HW = H * W;
  const int Ci = Ca + Cb, Co = r.Co;
  if (Ci != r.Ci) throw std::logic_error("UNet::resnet: input channel mismatch");
  DeviceArenaScope sc(DeviceArenaId::UNet);
  void* h = sc.alloc<uint16_t>((size_t)B * HW * std::max(Ci, Co));
  void* h2 = sc.alloc<uint16_t>((size_t)B * HW * Co);
  // conv1 writes norm2's statistics
  void* st2 = gn_stats_ws(sc, B, Co, HW, gn_fold_);
  // norm1 + SiLU over concat(xa, xb)
  gn(xa, Ca, xb, Cb, r.n1g, r.n1b, h, B, HW, 1e-5f, true, stream, in_stats, in_stats_b);
  // conv1 + bias + time_emb_proj(silu(temb)) per (n, c)
  {
    dlm_conv_nhwc_args a{};
    a.src0a = h;
    a.C0a = Ci;
    a.ld0a = Ci;
    a.N = B;
    a.H = H;
    a.W = W;
    a.KH = 3;
    a.KW = 3;
    a.stride = 1;
    a.pad = 1;
    a.weight = r.c1w;
    a.ldw = 9 * Ci;
    a.Cout = Co;
    a.bias = r.c1b;
    a.tbias = static_cast<const char*>(tproj) + (size_t)r.tproj_off * kH;
    a.tbias_ld = tproj_total_;
    a.out = h2;
    a.ldy = Co;
    a.gn_stats = st2;
    LAUNCH(kConv, 2.0 * B * HW * Co * 9.0 * Ci,
           2.0 * ((double)B * HW * Ci + (double)Co * 9.0 * Ci + (double)B * HW * Co),
           dlm_conv2d_nhwc_fp16(&a, stream));
  }
  // norm2 + SiLU
  gn(h2, Co, nullptr, 0, r.n2g, r.n2b, h, B, HW, 1e-5f, true, stream, st2);
  // conv2 + bias + (fused 1x1 shortcut over the block input | identity residual)
  {
    dlm_conv_nhwc_args a{};
    a.src0a = h;
    a.C0a = Co;
    a.ld0a = Co;
    a.N = B;
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
    a.gn_stats = out_stats;
    if (r.shortcut) {
      a.src1a = xa;
      a.C1a = Ca;
      a.ld1a = Ca;
      a.src1b = xb;
      a.C1b = Cb;
      a.ld1b = Cb;
    } else {
      if (xb) throw std::logic_error("UNet::resnet: identity residual over a concatenated input");
      a.residual = xa;
      a.res_ld = Co;
    }
    LAUNCH(kConv, 2.0 * B * HW * Co * (9.0 * Co + (r.shortcut ? Ci : 0)),
           2.0 * ((double)B * HW * Co * 2.0 + (double)Co * (9.0 * Co + (r.shortcut ? Ci : 0)) +
                  (double)B * HW * (r.shortcut ? Ci : Co)),
           dlm_conv2d_nhwc_fp16(&a, stream));
  }
}

void UNet::tblock(const Block& k, int C, void* h, const TScratch& ts, int B, int HW,
                  const CrossKV& kv, int kv_off, int kv_stride, int ctx_len, void* stream) {
  const int M = B * HW;
  const int heads = C / 64;
  const float scale = 1.0f / std::sqrt(64.0f);
  void* n = ts.n;
  void* qkv = ts.qkv;
  void* vt = ts.vt;
  const int vt_ld = ts.vt_ld;
  void* o = ts.o;
  void* f = ts.f;
  // self-attention: Q|K as [M, 2C] and V transposed per sample as
  // [B, heads, 64, HW], of norm1(h) (folded into the GEMM, or a separate
  // LayerNorm launch)
  if (ln_fold_ & 1) {
    LAUNCH(kLinear, 2.0 * M * 3 * C * C, lin_bytes(M, 3 * C, C, 3 * C, false),
           dlm_linear_vt_ln_fp16(h, C, k.fqkv.wf, C, k.fqkv.c1, k.fqkv.c2, 1e-5f, qkv, 2 * C, vt,
                                 2 * C, HW, vt_ld, M, 3 * C, C, stream));
  } else {
    LAUNCH(kLayerNorm, 0.0, 4.0 * M * C, dlm_layer_norm_fp16(h, k.ln1g, k.ln1b, n, M, C, 1e-5f, stream));
    LAUNCH(kLinear, 2.0 * M * 3 * C * C, lin_bytes(M, 3 * C, C, 3 * C, false),
           dlm_linear_vt_fp16(n, C, k.wqkv, C, nullptr, qkv, 2 * C, vt, 2 * C, HW, vt_ld, M,
                              3 * C, C, stream));
  }
  {
    dlm_attention_vt_args a{};
    const char* base = static_cast<const char*>(qkv);
    a.q = base;
    a.k = base + (size_t)C * kH;
    a.vt = vt;
    a.q_sb = a.k_sb = (long long)HW * 2 * C;
    a.q_ss = a.k_ss = 2 * C;
    a.q_sh = a.k_sh = 64;
    a.vt_sb = (long long)C * vt_ld;
    a.vt_sh = 64LL * vt_ld;
    a.vt_ld = vt_ld;
    a.o = o;
    a.o_sb = (long long)HW * C;
    a.o_ss = C;
    a.o_sh = 64;
    a.B = B;
    a.H = heads;
    a.Sq = HW;
    a.Sk = HW;
    a.scale = scale;
    a.k_bytes = ((size_t)M * 2 * C - C) * kH;
    a.vt_bytes = (size_t)B * C * vt_ld * kH;
    LAUNCH(kAttention, 4.0 * B * heads * (double)HW * HW * 64, 0.0,
           dlm_attention_vt_fp16(&a, stream));
  }
  LAUNCH(kLinear, 2.0 * M * C * C, lin_bytes(M, C, C, C, true),
       dlm_linear_fp16(o, C, k.wo1, C, k.bo1, h, C, h, C, M, C, C, 1.0f, 1.0f, DLM_ACT_NONE,
                           stream));
  // cross-attention over the context's K / V^T (rows kv_off.. of stride kv_stride)
  if (ln_fold_ & 2) {
    LAUNCH(kLinear, 2.0 * M * C * C, lin_bytes(M, C, C, C, false),
           dlm_linear_ln_fp16(h, C, k.fq2.wf, C, k.fq2.c1, k.fq2.c2, 1e-5f, nullptr, 0, qkv, C, M, C, C,
                              0.0f, DLM_ACT_NONE, stream));
  } else {
    LAUNCH(kLayerNorm, 0.0, 4.0 * M * C, dlm_layer_norm_fp16(h, k.ln2g, k.ln2b, n, M, C, 1e-5f, stream));
    LAUNCH(kLinear, 2.0 * M * C * C, lin_bytes(M, C, C, C, false),
           dlm_linear_fp16(n, C, k.wq2, C, nullptr, nullptr, 0, qkv, C, M, C, C, 1.0f, 0.0f,
                           DLM_ACT_NONE, stream));
  }
  {
    dlm_attention_vt_args a{};
    a.q = qkv;
    a.q_sb = (long long)HW * C;
    a.q_ss = C;
    a.q_sh = 64;
    a.k = static_cast<const char*>(kv.k) + (size_t)kv_off * kH;
    a.k_sb = (long long)ctx_len * kv_stride;
    a.k_ss = kv_stride;
    a.k_sh = 64;
    a.vt = static_cast<const char*>(kv.vt) + (size_t)kv_off * kv.ld * kH;
    a.vt_sb = (long long)kv_stride * kv.ld;
    a.vt_sh = 64LL * kv.ld;
    a.vt_ld = kv.ld;
    a.o = o;
    a.o_sb = (long long)HW * C;
    a.o_ss = C;
    a.o_sh = 64;
    a.B = B;
    a.H = heads;
    a.Sq = HW;
    a.Sk = ctx_len;
    a.scale = scale;
    a.k_bytes = ((size_t)B * ctx_len * kv_stride - kv_off) * kH;
    a.vt_bytes = ((size_t)B * kv_stride - kv_off) * kv.ld * kH;
    LAUNCH(kAttention, 4.0 * B * heads * (double)HW * ctx_len * 64, 0.0,
           dlm_attention_vt_fp16(&a, stream));
  }
  LAUNCH(kLinear, 2.0 * M * C * C, lin_bytes(M, C, C, C, true),
       dlm_linear_fp16(o, C, k.wo2, C, k.bo2, h, C, h, C, M, C, C, 1.0f, 1.0f, DLM_ACT_NONE,
                           stream));
  // GEGLU feed-forward (norm3 stays a separate launch: folded into the
  // GEGLU projection it made the step slower, 23.07 -> 23.54 ms)
  LAUNCH(kLayerNorm, 0.0, 4.0 * M * C, dlm_layer_norm_fp16(h, k.ln3g, k.ln3b, n, M, C, 1e-5f, stream));
  LAUNCH(kLinear, 2.0 * M * 8 * C * C, lin_bytes(M, 8 * C, C, 4 * C, false),
         dlm_linear_fp16(n, C, k.wff1, C, k.bff1, nullptr, 0, f, 4 * C, M, 8 * C, C, 1.0f,
                         0.0f, DLM_ACT_GEGLU, stream));
  LAUNCH(kLinear, 2.0 * M * 4 * C * C, lin_bytes(M, C, 4 * C, C, true),
       dlm_linear_fp16(f, 4 * C, k.wff2, 4 * C, k.bff2, h, C, h, C, M, C, 4 * C, 1.0f, 1.0f,
                           DLM_ACT_NONE, stream));
}

void UNet::t2d(const T2D& t, void* x, int B, int HW, const CrossKV& kv, int ctx_len, void* stream,
               const void* in_stats, void* out_stats) {
  const int C = t.C;
  const int M = B * HW;
  DeviceArenaScope sc(DeviceArenaId::UNet);
  void* g = sc.alloc<uint16_t>((size_t)M * C);
  void* h = sc.alloc<uint16_t>((size_t)M * C);
  void* n = sc.alloc<uint16_t>((size_t)M * C);
  void* qkv = sc.alloc<uint16_t>((size_t)M * 2 * C);
  // V^T rows are padded to a multiple of 8 tokens (the attention kernel's
  // key granularity); the QKV epilogue writes zeros into the padding
  const int vt_ld = (HW + 7) & ~7;
  void* vt = sc.alloc<uint16_t>((size_t)B * C * vt_ld);
  void* o = sc.alloc<uint16_t>((size_t)M * C);
  void* f = sc.alloc<uint16_t>((size_t)M * 4 * C);

  gn(x, C, nullptr, 0, t.ng, t.nb, g, B, HW, 1e-6f, false, stream, in_stats);
  LAUNCH(kLinear, 2.0 * M * C * C, lin_bytes(M, C, C, C, false),
         dlm_linear_fp16(g, C, t.pin_w, C, t.pin_b, nullptr, 0, h, C, M, C, C, 1.0f, 0.0f,
                           DLM_ACT_NONE, stream));
  const TScratch ts{n, qkv, vt, vt_ld, o, f};
  for (const Block& k : t.blocks) tblock(k, C, h, ts, B, HW, kv, k.kv_off, kv_total_ / 2, ctx_len, stream);
  // proj_out + residual (the block input), written back in place (with the
  // next GroupNorm's statistics when out_stats is given)
  if (out_stats) {
    LAUNCH(kLinear, 2.0 * M * C * C, lin_bytes(M, C, C, C, true),
           dlm_linear_gn_stats_fp16(h, C, t.pout_w, C, t.pout_b, x, C, x, C, M, C, C, 1.0f, 1.0f,
                                    DLM_ACT_NONE, HW, out_stats, stream));
  } else {
    LAUNCH(kLinear, 2.0 * M * C * C, lin_bytes(M, C, C, C, true),
           dlm_linear_fp16(h, C, t.pout_w, C, t.pout_b, x, C, x, C, M, C, C, 1.0f, 1.0f,
                           DLM_ACT_NONE, stream));
  }
}

static std::string with_dot(const std::string& p) {
  return (!p.empty() && p.back() == '.') ? p : p + ".";
}

void UNet::run_resnet(const std::string& prefix, const void* xa, int Ca, const void* xb, int Cb,
                      void* out, int B, int H, int W, const void* temb, void* stream) {
  if (!packed_) throw std::runtime_error("UNet::run_resnet: prepare() has not run");
  if (!xa || !out || !temb || (Cb > 0 && !xb)) throw std::invalid_argument("UNet::run_resnet: NULL input");
  if (B <= 0 || H <= 0 || W <= 0) throw std::invalid_argument("UNet::run_resnet: bad shape");
  const std::string p = with_dot(prefix);
  size_t i = 0;
  while (i < res_names_.size() && res_names_[i] != p) ++i;
  if (i == res_names_.size()) throw std::out_of_range("UNet::run_resnet: no resnet '" + prefix + "'");
  const Resnet& r = res_[i];
  if (Ca + Cb != r.Ci) throw std::invalid_argument("UNet::run_resnet: input channels != block input");
  const int T = cfg_.time_dim();
  DeviceArenaScope persist(DeviceArenaId::UNetPersist);
  // this block's time_emb_proj(silu(temb)), laid out as the forward's tproj
  // rows would be (row stride tproj_total_, the block's columns at tproj_off)
  void* tproj = persist.alloc<uint16_t>((size_t)B * tproj_total_);
  const char* w = static_cast<const char*>(tproj_w_) + (size_t)r.tproj_off * T * kH;
  const char* b = static_cast<const char*>(tproj_b_) + (size_t)r.tproj_off * kH;
  DLM_CALL(dlm_linear_small_fp16(temb, T, w, b, static_cast<char*>(tproj) + (size_t)r.tproj_off * kH,
                                 tproj_total_, B, r.Co, T, 1, DLM_ACT_NONE, 0, stream));
  resnet(r, xa, Ca, xb, Cb, out, B, H, W, tproj, stream);
}

void UNet::run_transformer_block(const std::string& prefix, void* x, int B, int HW, const void* ehs,
                                 int ctx_len, void* stream) {
  if (!packed_) throw std::runtime_error("UNet::run_transformer_block: prepare() has not run");
  if (!x || !ehs) throw std::invalid_argument("UNet::run_transformer_block: NULL input");
  if (B <= 0 || HW <= 0 || ctx_len <= 0) throw std::invalid_argument("UNet::run_transformer_block: bad shape");
  const std::string p = with_dot(prefix);
  const std::string tag = "transformer_blocks.";
  const size_t at = p.rfind(tag);
  if (at == std::string::npos) throw std::out_of_range("UNet::run_transformer_block: not a block prefix");
  const std::string owner = p.substr(0, at);
  const int l = std::atoi(p.c_str() + at + tag.size());
  size_t ti = 0;
  while (ti < t2d_names_.size() && t2d_names_[ti] != owner) ++ti;
  if (ti == t2d_names_.size() || l < 0 || l >= (int)t2d_[ti].blocks.size())
    throw std::out_of_range("UNet::run_transformer_block: no block '" + prefix + "'");
  const T2D& t = t2d_[ti];
  const Block& k = t.blocks[l];
  const int C = t.C, M = B * HW, cross = cfg_.cross_dim;
  const int kv_half = kv_total_ / 2;
  DeviceArenaScope sc(DeviceArenaId::UNet);
  // this block's context K [B*ctx, C] and V^T [B, C, ctx_pad] from its rows
  // of the concatenated projection weight
  const int ctx_pad = (ctx_len + 7) & ~7;
  CrossKV kv{sc.alloc<uint16_t>((size_t)B * ctx_len * C), sc.alloc<uint16_t>((size_t)B * C * ctx_pad),
             ctx_pad};
  const char* kw = static_cast<const char*>(kv_w_) + (size_t)k.kv_off * cross * kH;
  const char* vw = static_cast<const char*>(kv_w_) + (size_t)(kv_half + k.kv_off) * cross * kH;
  LAUNCH(kLinear, 2.0 * B * ctx_len * C * cross, lin_bytes(B * ctx_len, C, cross, C, false),
         dlm_linear_fp16(ehs, cross, kw, cross, nullptr, nullptr, 0, kv.k, C, B * ctx_len, C, cross,
                         1.0f, 0.0f, DLM_ACT_NONE, stream));
  LAUNCH(kLinear, 2.0 * B * ctx_len * C * cross, lin_bytes(B * ctx_len, C, cross, C, false),
         dlm_linear_vt_fp16(ehs, cross, vw, cross, nullptr, kv.vt, 0, kv.vt, 0, ctx_len, ctx_pad,
                            B * ctx_len, C, cross, stream));
  const int vt_ld = (HW + 7) & ~7;
  const TScratch ts{sc.alloc<uint16_t>((size_t)M * C), sc.alloc<uint16_t>((size_t)M * 2 * C),
                    sc.alloc<uint16_t>((size_t)B * C * vt_ld), vt_ld,
                    sc.alloc<uint16_t>((size_t)M * C), sc.alloc<uint16_t>((size_t)M * 4 * C)};
  tblock(k, C, x, ts, B, HW, kv, 0, C, ctx_len, stream);
}

void UNet::forward(int B, int H, int W, const void* latent, const float* d_timesteps,
                   const void* ehs, int ctx_len, const void* text, const void* time_ids,
                   int ids_bstride, void* out, void* stream) {
  if (!graphs_on_ || hook_ || prof_on_ || !stream || !packed_) {
    forward_impl(B, H, W, latent, d_timesteps, ehs, ctx_len, text, time_ids, ids_bstride, out, stream);
    return;
  }
  auto words = [](const void* p) { return (uint64_t)(uintptr_t)p; };
  const DeviceArenaMark m0 = device_arena_mark(DeviceArenaId::UNet);
  const DeviceArenaMark m1 = device_arena_mark(DeviceArenaId::UNetPersist);
  const uint64_t e0 = device_arena_epoch(DeviceArenaId::UNet);
  const uint64_t e1 = device_arena_epoch(DeviceArenaId::UNetPersist);
  const std::vector<uint64_t> key = {
      (uint64_t)B, (uint64_t)H, (uint64_t)W, (uint64_t)ctx_len, (uint64_t)ids_bstride, words(latent),
      words(d_timesteps), words(ehs), words(text), words(time_ids), words(out), words(stream),
      m0.chunk, m0.offset, m1.chunk, m1.offset, e0, e1};
  auto it = graphs_.find(key);
  if (it != graphs_.end()) {
    DLM_CALL(dlm_graph_launch(it->second, stream));
    return;
  }
  if (!seen_.count(key)) {  // first sight: run eagerly (allocates chunks and workspaces)
    if (seen_.size() >= 64) clear_graphs();
    seen_.insert(key);
    forward_impl(B, H, W, latent, d_timesteps, ehs, ctx_len, text, time_ids, ids_bstride, out, stream);
    return;
  }
  DLM_CALL(dlm_graph_begin_capture(stream));
  void* exec = nullptr;
  try {
    forward_impl(B, H, W, latent, d_timesteps, ehs, ctx_len, text, time_ids, ids_bstride, out, stream);
  } catch (...) {
    void* junk = nullptr;
    (void)dlm_graph_end_capture(stream, &junk);
    (void)dlm_graph_destroy(junk);
    throw;
  }
  DLM_CALL(dlm_graph_end_capture(stream, &exec));
  if (device_arena_epoch(DeviceArenaId::UNet) != e0 ||
      device_arena_epoch(DeviceArenaId::UNetPersist) != e1) {
    // an arena grew during the capture: do not keep the graph, run eagerly
    (void)dlm_graph_destroy(exec);
    forward_impl(B, H, W, latent, d_timesteps, ehs, ctx_len, text, time_ids, ids_bstride, out, stream);
    return;
  }
  graphs_[key] = exec;
  DLM_CALL(dlm_graph_launch(exec, stream));
}

void UNet::forward_impl(int B, int H, int W, const void* latent, const float* d_timesteps,
                        const void* ehs, int ctx_len, const void* text, const void* time_ids,
                        int ids_bstride, void* out, void* stream) {
  if (!packed_) throw std::runtime_error("UNet::forward: prepare() has not run");
  if (B <= 0 || B > 16) throw std::invalid_argument("UNet::forward: B must be in [1, 16]");
  if (H % 4 != 0 || W % 4 != 0 || H < 8 || W < 8)
    throw std::invalid_argument("UNet::forward: H and W must be multiples of 4 and >= 8");
  if (ctx_len <= 0) throw std::invalid_argument("UNet::forward: ctx_len must be positive");
  if (!latent || !d_timesteps || !ehs || !text || !time_ids || !out)
    throw std::invalid_argument("UNet::forward: NULL input");
  const UNetConfig& c = cfg_;
  const int T = c.time_dim();
  const int C0 = c.C0, C1 = c.C1, C2 = c.C2;
  const int H1 = H / 2, W1 = W / 2, H2 = H / 4, W2 = W / 4;
  const int HW0 = H * W, HW1 = H1 * W1, HW2 = H2 * W2;

  prof_next_ = 0;
  DeviceArenaScope persist(DeviceArenaId::UNetPersist);
  auto P = [&](size_t elems) { return persist.alloc<uint16_t>(elems); };

  // ---- time / add embeddings, every resnet's time projection
  void* t_emb = P((size_t)B * C0);
  void* add_in = P((size_t)B * c.add_dim());
  LAUNCH(kOther, 0.0, 0.0,
         dlm_sdxl_embed_inputs_fp16(d_timesteps, text, c.text_dim, time_ids, ids_bstride, c.id_dim,
                                    t_emb, C0, add_in, B, stream));
  void* th = P((size_t)B * T);
  void* temb = P((size_t)B * T);
  LAUNCH(kOther, 0.0, 0.0, dlm_linear_small_fp16(t_emb, C0, te1w_, te1b_, th, T, B, T, C0, 0, DLM_ACT_SILU, 0, stream));
  LAUNCH(kOther, 0.0, 0.0, dlm_linear_small_fp16(th, T, te2w_, te2b_, temb, T, B, T, T, 0, DLM_ACT_NONE, 0, stream));
  LAUNCH(kOther, 0.0, 0.0, dlm_linear_small_fp16(add_in, c.add_dim(), ae1w_, ae1b_, th, T, B, T, c.add_dim(), 0,
                                 DLM_ACT_SILU, 0, stream));
  LAUNCH(kOther, 0.0, 0.0, dlm_linear_small_fp16(th, T, ae2w_, ae2b_, temb, T, B, T, T, 0, DLM_ACT_NONE, 1, stream));
  stage("temb", temb, (size_t)B * T, T, stream);
  void* tproj = P((size_t)B * tproj_total_);
  LAUNCH(kOther, 0.0, 0.0, dlm_linear_small_fp16(temb, T, tproj_w_, tproj_b_, tproj, tproj_total_, B, tproj_total_, T,
                                 1, DLM_ACT_NONE, 0, stream));
  // ---- cross-attention K/V of every transformer block, one GEMM: K as
  // [B*ctx, sumC] row-major, V transposed as [B, sumC, ctx_pad] (zero padded)
  const int kv_half = kv_total_ / 2;
  const int ctx_pad = (ctx_len + 7) & ~7;
  CrossKV ckv{P((size_t)B * ctx_len * kv_half), P((size_t)B * kv_half * ctx_pad), ctx_pad};
  LAUNCH(kLinear, 2.0 * B * ctx_len * kv_total_ * c.cross_dim,
         lin_bytes(B * ctx_len, kv_total_, c.cross_dim, kv_total_, false),
         dlm_linear_vt_fp16(ehs, c.cross_dim, kv_w_, c.cross_dim, nullptr, ckv.k, kv_half, ckv.vt,
                            kv_half, ctx_len, ctx_pad, B * ctx_len, kv_total_, c.cross_dim, stream));

  size_t ri = 0, ai = 0;
  // down-path outputs the up path concatenates, with their producers' GroupNorm
  // statistics (null where not written)
  struct Skip {
    void* x;
    int C;
    void* st;
  };
  std::vector<Skip> skips;
  // ---- conv_in (latent NCHW -> channels-last, zero-padded to 64 channels)
  void* xin = P((size_t)B * HW0 * kConvInPad);
  LAUNCH(kOther, 0.0, 0.0, dlm_nchw_to_nhwc_fp16(latent, xin, B, c.in_channels, HW0, kConvInPad, stream));
  // GroupNorm statistics written by the conv (or proj_out) that produces a
  // GroupNorm's input (conv1 -> norm2 inside each resnet; here: conv_in, the
  // downsamplers, resnet and transformer outputs that feed a GroupNorm, and
  // both sources of every up-path concatenation: each skip and the h it is
  // concatenated with)
  auto S = [&](int C, int HWs) { return gn_stats_ws(persist, B, C, HWs, gn_fold_); };
  void* cur = P((size_t)B * HW0 * C0);
  void* cur_st = S(C0, HW0);
  conv3(conv_in_, xin, kConvInPad, nullptr, 0, cur, C0, B, H, W, 1, false, stream, c.in_channels, cur_st);
  stage("conv_in_out", cur, (size_t)B * HW0 * C0, C0, stream);
  skips.push_back({cur, C0, cur_st});

  // ---- down_blocks.0
  for (int r = 0; r < 2; ++r) {
    void* o = P((size_t)B * HW0 * C0);
    void* o_st = S(C0, HW0);  // the next norm1, or (second resnet) up_blocks.2's last concatenation
    resnet(res_[ri++], cur, C0, nullptr, 0, o, B, H, W, tproj, stream, cur_st, o_st);
    skips.push_back({o, C0, o_st});
    cur = o;
    cur_st = o_st;
  }
  {
    void* d = P((size_t)B * HW1 * C0);
    cur_st = S(C0, HW1);
    conv3(down0_, cur, C0, nullptr, 0, d, C0, B, H, W, 2, false, stream, -1, cur_st);
    skips.push_back({d, C0, cur_st});
    cur = d;
  }
  stage("down_block_0_out", cur, (size_t)B * HW1 * C0, C0, stream);
  // ---- down_blocks.1 (each transformer's proj_out writes the statistics of
  // its output: the second resnet's norm1, and both skips)
  int curC = C0;
  for (int r = 0; r < 2; ++r) {
    void* o = P((size_t)B * HW1 * C1);
    void* o_st = S(C1, HW1);
    void* t_st = S(C1, HW1);
    resnet(res_[ri++], cur, curC, nullptr, 0, o, B, H1, W1, tproj, stream, cur_st, o_st);
    t2d(t2d_[ai++], o, B, HW1, ckv, ctx_len, stream, o_st, t_st);
    skips.push_back({o, C1, t_st});
    cur = o;
    cur_st = t_st;
    curC = C1;
  }
  {
    void* d = P((size_t)B * HW2 * C1);
    cur_st = S(C1, HW2);
    conv3(down1_, cur, C1, nullptr, 0, d, C1, B, H1, W1, 2, false, stream, -1, cur_st);
    skips.push_back({d, C1, cur_st});
    cur = d;
  }
  stage("down_block_1_out", cur, (size_t)B * HW2 * C1, C1, stream);
  // ---- down_blocks.2
  // (both transformers' proj_out write the next resnet's norm1 statistics:
  // the second resnet's, then the mid block's first)
  for (int r = 0; r < 2; ++r) {
    void* o = P((size_t)B * HW2 * C2);
    void* o_st = S(C2, HW2);
    void* t_st = S(C2, HW2);
    resnet(res_[ri++], cur, curC, nullptr, 0, o, B, H2, W2, tproj, stream, cur_st, o_st);
    t2d(t2d_[ai++], o, B, HW2, ckv, ctx_len, stream, o_st, t_st);
    skips.push_back({o, C2, t_st});
    cur = o;
    cur_st = t_st;
    curC = C2;
  }
  stage("down_block_2_out", cur, (size_t)B * HW2 * C2, C2, stream);
  // ---- mid_block
  {
    void* m0 = P((size_t)B * HW2 * C2);
    void* m0_st = S(C2, HW2);
    void* t_st = S(C2, HW2);
    resnet(res_[ri++], cur, C2, nullptr, 0, m0, B, H2, W2, tproj, stream, cur_st, m0_st);
    t2d(t2d_[ai++], m0, B, HW2, ckv, ctx_len, stream, m0_st, t_st);
    void* m1 = P((size_t)B * HW2 * C2);
    void* m1_st = S(C2, HW2);  // h of up_blocks.0's first concatenation
    resnet(res_[ri++], m0, C2, nullptr, 0, m1, B, H2, W2, tproj, stream, t_st, m1_st);
    cur = m1;
    cur_st = m1_st;
  }
  stage("mid_block_out", cur, (size_t)B * HW2 * C2, C2, stream);
  // ---- up_blocks
  const int upC[3] = {C2, C1, C0};
  const int upH[3] = {H2, H1, H}, upW[3] = {W2, W1, W};
  const int depth[3] = {c.depth2, c.depth1, 0};
  for (int u = 0; u < 3; ++u) {
    const int Hh = upH[u], Ww = upW[u], HWu = Hh * Ww, C = upC[u];
    for (int r = 0; r < 3; ++r) {
      const Skip sk = skips.back();
      skips.pop_back();
      void* o = P((size_t)B * HWu * C);
      // the output's next GroupNorm: the transformer's, the next
      // concatenation's (h), or conv_norm_out
      void* o_st = S(C, HWu);
      resnet(res_[ri++], cur, curC, sk.x, sk.C, o, B, Hh, Ww, tproj, stream, cur_st, o_st, sk.st);
      cur_st = o_st;
      if (depth[u] > 0) {
        // the transformer rewrites o in place; its proj_out writes the
        // statistics of the next concatenation's h (none before the upsampler)
        void* t_st = r < 2 ? S(C, HWu) : nullptr;
        t2d(t2d_[ai++], o, B, HWu, ckv, ctx_len, stream, o_st, t_st);
        cur_st = t_st;
      }
      cur = o;
      curC = C;
    }
    if (u < 2) {
      void* up = P((size_t)B * 4 * HWu * C);
      cur_st = S(C, 4 * HWu);  // h of the next up block's first concatenation
      conv3(u == 0 ? up0_ : up1_, cur, C, nullptr, 0, up, C, B, Hh, Ww, 1, true, stream, -1, cur_st);
      cur = up;
    }
    static const char* names[3] = {"up_block_0_out", "up_block_1_out", "up_block_2_out"};
    const int HWo = u < 2 ? 4 * HWu : HWu;
    stage(names[u], cur, (size_t)B * HWo * C, C, stream);
  }
  if (ri != res_.size() || ai != t2d_.size() || !skips.empty())
    throw std::logic_error("UNet::forward: graph walk does not match the packed weights");
  // ---- conv_norm_out + SiLU + conv_out (written NCHW)
  {
    DeviceArenaScope sc(DeviceArenaId::UNet);
    void* g = sc.alloc<uint16_t>((size_t)B * HW0 * C0);
    gn(cur, C0, nullptr, 0, norm_out_g_, norm_out_b_, g, B, HW0, 1e-5f, true, stream, cur_st);
    dlm_conv_nhwc_args a{};
    a.src0a = g;
    a.C0a = C0;
    a.ld0a = C0;
    a.N = B;
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
    a.out = out;
    a.ldy = c.out_channels;
    a.out_nchw = 1;
    LAUNCH(kConv, 2.0 * B * HW0 * c.out_channels * 9.0 * C0, 0.0, dlm_conv2d_nhwc_fp16(&a, stream));
  }
  stage("noise_pred", out, (size_t)B * c.out_channels * HW0, c.out_channels, stream);
}

}  // namespace dollama
