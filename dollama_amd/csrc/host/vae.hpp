// SDXL AutoencoderKL decoder on channels-last activations.
//
// Graph, weight names and numerics policy follow the reference's decoder
// (src/kernels/vae_decode.cuh:20-77, vae_decode.cu:575-875):
// post_quant_conv 1x1 -> conv_in 3x3 -> mid (resnet, single-head attention
// over all pixels, resnet) -> four up blocks of `layers` resnets (nearest-2x
// upsample + 3x3 conv after the first three) -> GroupNorm + SiLU -> conv_out,
// GroupNorm eps 1e-6, attention scale 1/sqrt(C).  Up blocks from `fp32_from`
// on keep their activations in fp32, because the conv2 and conv_shortcut
// outputs there leave the fp16 range before the residual add cancels them
// (vae_decode.cu:9-19).
//
// What differs by design (MI355X-first, same arithmetic up to rounding):
//   - every conv is one implicit-GEMM launch with fp16 operands and fp32
//     accumulation; bias, residual add and the 1x1 conv_shortcut (as a second
//     K segment) run in its epilogue, so a pre-residual sum is never stored;
//     nearest-2x upsampling happens in the operand loader;
//   - in the fp32 stages the residual stream, the conv outputs and the
//     GroupNorm inputs are fp32, while conv operands are fp16 (GroupNorm+SiLU
//     output, or an fp32 activation scaled by 2^-8 with the matching weight
//     columns scaled by 2^8, which moves the fp16 overflow point to 1.7e7);
//   - the mid-block attention (Dh = C = 512, S = h*w) runs as three launches:
//     fp32 scores GEMM, row softmax to fp16, P V GEMM (V^T written by the QKV
//     GEMM), with the residual add in the output projection's epilogue.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "dlm.h"
#include "unet.hpp"

namespace dollama {

struct VaeConfig {
  int ch[4] = {128, 256, 512, 512};  // block_out_channels (encoder order)
  int latent_channels = 4;
  int out_channels = 3;
  int layers = 3;     // resnets per decoder up block (layers_per_block + 1)
  int groups = 32;
  int fp32_from = 2;  // decoder up blocks with index >= fp32_from run in fp32
  // output channels of decoder up block i (decode order)
  int up_ch(int i) const { return ch[3 - i]; }
};

std::vector<WeightSpec> vae_weight_specs(const VaeConfig& cfg);

using VaeStageHook = void (*)(const char* name, const void* dptr, size_t n, int C, int is_f32,
                              void* user);

class VAE {
 public:
  explicit VAE(const VaeConfig& cfg);
  ~VAE();
  VAE(const VAE&) = delete;
  VAE& operator=(const VAE&) = delete;

  const VaeConfig& config() const { return cfg_; }

  // Register a device fp16 weight (borrowed until prepare()).  Attention
  // projections are accepted as [C, C] or [C, C, 1, 1].
  void set_weight(const std::string& name, const void* dptr, const std::vector<int64_t>& shape);
  // Pack every registered weight into the handle's own device memory.
  void prepare(void* stream);
  bool prepared() const { return packed_ != nullptr; }
  size_t packed_bytes() const { return packed_bytes_; }

  // image [N, out_channels, 8h, 8w] fp16 NCHW from latent
  // [N, latent_channels, h, w] fp16 NCHW (already divided by the scaling
  // factor).  h * w must be a multiple of 8.
  void decode(int N, int h, int w, const void* latent, void* image, void* stream);

  void set_stage_hook(VaeStageHook hook, void* user) {
    hook_ = hook;
    hook_user_ = user;
  }

  // Per-launch timing by kernel class, as UNet::set_profiling.
  enum KernelClass { kConv = 0, kLinear, kAttention, kGroupNorm, kOther, kClassCount };
  void set_profiling(bool on) { prof_on_ = on; }
  struct ClassStats {
    int count = 0;
    double ms = 0.0, flops = 0.0, bytes = 0.0;
  };
  std::vector<ClassStats> profile_report(void* stream);

 private:
  struct Conv {
    const void *w = nullptr, *b = nullptr;
    int ldw = 0;
  };
  struct Resnet {
    int Ci = 0, Co = 0;
    bool shortcut = false;
    bool in_f32 = false;   // block input is fp32
    bool out_f32 = false;  // conv outputs (and the block output) are fp32
    const void *n1g, *n1b, *c1w, *c1b, *n2g, *n2b, *c2w, *c2b;
    int c2_ldw = 0;
  };
  struct Attn {
    int C = 0;
    const void *ng, *nb, *wqkv, *bqkv, *wo, *bo;
  };
  struct Src {
    const void* ptr;
    std::vector<int64_t> shape;
  };

  const Src& src(const std::string& name, const std::vector<int64_t>& shape) const;
  void* take(size_t elems);
  const void* copy_of(const std::string& name, const std::vector<int64_t>& shape, void* stream);
  void pack_weight(const std::string& name, void* dst, int Co, int Ci, int k, int cin_pad, int ld,
                   int col0, float scale, void* stream);
  Conv pack_conv(const std::string& p, int Co, int Ci, int k, int cin_pad, float scale,
                 void* stream);
  Resnet pack_resnet(const std::string& p, int Ci, int Co, bool in_f32, bool out_f32,
                     void* stream);
  Attn pack_attn(const std::string& p, int C, void* stream);
  void pack_all(void* stream);

  void gn(const void* x, bool f32, int C, const void* g, const void* b, void* out, int N, int HW,
          bool silu, void* stream);
  void conv(const Conv& c, const void* x, int Ci, int ldx, void* out, int Co, int ldy, bool out_f32,
            int N, int H, int W, int k, bool up, void* stream);
  void resnet(const Resnet& r, const void* x, void* out, int N, int H, int W, void* stream);
  void attention(const Attn& a, const void* x, void* out, int N, int HW, void* stream);
  void stage(const char* name, const void* p, size_t n, int C, bool f32, void* stream);

  VaeConfig cfg_;
  std::unordered_map<std::string, Src> srcs_;
  bool sizing_ = false;
  char* packed_ = nullptr;
  size_t packed_bytes_ = 0;
  size_t cursor_ = 0;
  Conv pqc_, conv_in_, conv_out_;
  std::vector<Conv> ups_;       // upsampler convs of up blocks 0..2
  std::vector<Resnet> res_;     // mid (2), then up blocks in decode order
  Attn attn_{};
  const void *norm_out_g_ = nullptr, *norm_out_b_ = nullptr;
  VaeStageHook hook_ = nullptr;
  void* hook_user_ = nullptr;

  struct ProfRec {
    int cls;
    double flops, bytes;
  };
  bool prof_on_ = false;
  std::vector<void*> prof_events_;
  std::vector<ProfRec> prof_recs_;
  size_t prof_next_ = 0;
  void prof_begin(int cls, double flops, double bytes, void* stream);
  void prof_end(void* stream);
};

}  // namespace dollama
