// Text-to-image pipeline around the dense path: seeded initial latent, the
// Euler denoise loop on the device (with or without classifier-free
// guidance), VAE decode and RGB8 conversion.
//
// The reference runs its loop on the host (src/infer/diffusion.cu:551-1000):
// per step an H2D of the scaled latent, the UNet forward(s), a D2H of the
// noise predictions, the CFG combine u + g (c - u) and the Euler step in host
// floats, then a host latent / scaling_factor -> VAE -> D2H -> RGB8.  Here
// the latent stays on the device in fp32: one fused kernel does CFG + Euler +
// the next step's scale_model_input, the per-step timesteps are uploaded
// once, and the only transfers are the conditioning (in) and the RGB8 image
// (out).  Batch layout follows the reference's B=2 path: slice 0 = cond,
// slice 1 = uncond (B=2 == 2 x B=1 bit for bit in this UNet, so the
// reference's batch2 switch does not change results here).
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "safetensors.hpp"
#include "unet.hpp"
#include "vae.hpp"

namespace dollama {

constexpr float kDefaultVaeScalingFactor = 0.13025f;  // SDXL VAE

// Switches of the reference's FAST mode (src/server/fast_config.hpp).  They
// select reference code paths (fused attention, B=2 CFG, fused epilogues,
// CUDA graphs); this build always runs its fused paths, so the fields are
// accepted and carried for API compatibility only.
struct FastConfig {
  bool fast = false;
  bool fp8 = false;
  bool attn_fast = false;
  bool batch2 = false;
  bool graphs = false;
  bool epilogue = false;
};

// Standard normal samples of the reference's initial-noise generator
// (src/infer/diffusion.cu:80-136): xorshift128+ (Vigna, shifts 23/17/26)
// seeded by two splitmix64 outputs (of seed and seed + 0x9E3779B97F4A7C15),
// the top 53 bits as a double in [0, 1), and the Box-Muller transform
// (u1 <= 1e-12 redrawn), returning the cos sample, then the sin sample.  The
// same seed gives the same latent as the reference.
class Randn {
 public:
  explicit Randn(uint64_t seed);
  double next();

 private:
  double uniform();
  uint64_t s0_, s1_;
  bool has_spare_ = false;
  double spare_ = 0.0;
};

// latent[k] = float(z_k * sigma0) for k < n (the reference's initial latent).
void randn_latent(uint64_t seed, double sigma0, float* out, size_t n);

struct DenoiseArgs {
  int steps = 20;
  float guidance = 7.5f;
  int H = 128, W = 128;
  float* latent = nullptr;  // device fp32 [C, H, W]: in = randn * sigma_0, out = final latent
  const void* ehs = nullptr;       // device fp16 [2, ctx_len, cross_dim] (cond, uncond)
  int ctx_len = 77;
  const void* text = nullptr;      // device fp16 [2, text_dim]
  const void* time_ids = nullptr;  // device fp16 [6] (shared)
};

// CFG loop (B=2 forwards).  With cfg = false the forwards are B=1 on ehs[0]
// / text[0] and the Euler step uses the prediction as is (guidance unused).
void denoise(UNet& unet, const DenoiseArgs& a, void* stream, bool cfg = true);

// Load every tensor the network reads from a diffusers-named fp16
// safetensors file and prepare the handle.
void load_unet_safetensors(UNet& u, const std::string& path, void* stream);
void load_unet_safetensors(UNet& u, const SafeTensors& st, void* stream);
void load_vae_safetensors(VAE& v, const std::string& path, void* stream);

// Reference DiffusionPipeline (src/infer/diffusion.cuh:62-178) over the
// resident UNet and VAE handles.
class DiffusionPipeline {
 public:
  // embeds_path: safetensors with the conditioning of generate()
  // (input_encoder_hidden_states_f16 [ctx*cross_dim], input_text_embeds_f16
  // [text_dim], input_time_ids_f16 [6]; reference diffusion.cu:305-312).
  // latent_h / latent_w: the latent size (SDXL 1024x1024 -> 128 x 128).
  DiffusionPipeline(const std::string& unet_weights, const std::string& vae_weights,
                    const std::string& embeds_path, const FastConfig& fast = FastConfig{},
                    float vae_scaling_factor = kDefaultVaeScalingFactor,
                    const UNetConfig& ucfg = UNetConfig{}, const VaeConfig& vcfg = VaeConfig{},
                    int latent_h = 128, int latent_w = 128);
  ~DiffusionPipeline();
  DiffusionPipeline(const DiffusionPipeline&) = delete;
  DiffusionPipeline& operator=(const DiffusionPipeline&) = delete;

  // No guidance (guidance_scale must be 1), conditioning from the embeds file.
  void generate(int steps, uint64_t seed, float guidance_scale, std::vector<uint8_t>& rgb_out, int& w,
                int& h);
  // CFG with caller conditioning (host fp32; ehs [ctx_len * cross_dim], text
  // [text_dim], time_ids [6]).
  void generate_txt2img(int steps, uint64_t seed, float guidance_scale, const float* cond_ehs,
                        const float* cond_text_embeds, const float* uncond_ehs,
                        const float* uncond_text_embeds, const float* time_ids,
                        std::vector<uint8_t>& rgb_out, int& w, int& h);
  void apply_lora_file(const std::string& path, float strength);
  void clear_loras();

  float vae_scaling_factor() const { return vae_scaling_; }
  int ctx_len() const { return ctx_len_; }
  const UNetConfig& unet_config() const { return unet_.config(); }
  UNet& unet() { return unet_; }
  VAE& vae() { return vae_; }

 private:
  void run(int steps, uint64_t seed, float guidance, bool cfg, const void* d_ehs, const void* d_text,
           const void* d_ids, std::vector<uint8_t>& rgb_out, int& w, int& h);

  UNet unet_;
  VAE vae_;
  FastConfig fast_;
  float vae_scaling_ = kDefaultVaeScalingFactor;
  int lh_, lw_;
  int ctx_len_ = 0;
  void* d_ehs_ = nullptr;  // embeds-file conditioning, fp16
  void* d_text_ = nullptr;
  void* d_ids_ = nullptr;
};

}  // namespace dollama
