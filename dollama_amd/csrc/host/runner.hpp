// Diffusion backend plugin surface: IDiffusionRunner (the reference's GPU
// txt2img runner, src/server/diffusion_runner.hpp:33-79) and
// IDiffusionBackend with its "sdxl" registration (src/server/
// diffusion_backend.hpp:40-126, sdxl_backend.hpp), over DiffusionPipeline.
//
// Same contracts: make_diffusion_runner returns nullptr (with a message on
// stderr) when a weight / embeddings file is unreadable or construction
// fails; make_backend returns nullptr for an unknown name or a failed
// construction; apply_loras applies every file or, on any failure, clears
// all LoRAs and rethrows; generate() defaults steps <= 0 to 20 and cfg <= 0
// to 7.5 and returns the backend's native resolution.
//
// What differs: the reference's "sdxl" backend encodes the prompt with the
// CLIP-L / CLIP-G text encoders (OpenVINO, outside this build's scope).  The
// backend here takes its conditioning from precomputed embeddings: the
// embeddings file's cond tensors (input_encoder_hidden_states_f16,
// input_text_embeds_f16, input_time_ids_f16) and, when present, uncond
// tensors (uncond_encoder_hidden_states_f16, uncond_text_embeds_f16);
// without them the uncond conditioning is zero, as SDXL does for an empty
// negative prompt (force_zeros_for_empty_prompt).  The prompt strings are
// not read.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "pipeline.hpp"

namespace dollama {

constexpr float kServerDefaultVaeScalingFactor = kDefaultVaeScalingFactor;

struct LoraFileRequest {
  std::string path;
  float strength = 1.0f;
};

struct IDiffusionRunner {
  virtual ~IDiffusionRunner() = default;
  virtual void apply_loras(const std::vector<LoraFileRequest>& reqs) { (void)reqs; }
  virtual void clear_loras() {}
  // host fp32 conditioning: ehs [ctx_len * cross_dim], text [text_dim],
  // time_ids [6]; rgb_out [h, w, 3]
  virtual void run_txt2img(int steps, uint64_t seed, float guidance_scale, const float* cond_ehs,
                           const float* cond_text_embeds, const float* uncond_ehs,
                           const float* uncond_text_embeds, const float* time_ids,
                           std::vector<uint8_t>& rgb_out, int& w, int& h) = 0;
};

// The GPU runner: DiffusionPipeline behind IDiffusionRunner (reference
// DiffusionRunner, src/server/diffusion_runner.cu:33-110).
class DiffusionRunner : public IDiffusionRunner {
 public:
  DiffusionRunner(const std::string& unet, const std::string& vae, const std::string& embeds,
                  const FastConfig& fast, float vae_scaling_factor, const UNetConfig& ucfg,
                  const VaeConfig& vcfg, int latent_h, int latent_w);
  DiffusionRunner(const DiffusionRunner&) = delete;
  DiffusionRunner& operator=(const DiffusionRunner&) = delete;
  void run_txt2img(int steps, uint64_t seed, float guidance_scale, const float* cond_ehs,
                   const float* cond_text_embeds, const float* uncond_ehs,
                   const float* uncond_text_embeds, const float* time_ids,
                   std::vector<uint8_t>& rgb_out, int& w, int& h) override;
  void apply_loras(const std::vector<LoraFileRequest>& reqs) override;
  void clear_loras() override;
  DiffusionPipeline& pipeline() { return pipe_; }

 private:
  DiffusionPipeline pipe_;
};

// ucfg / vcfg / latent size default to SDXL at 1024x1024.
std::unique_ptr<IDiffusionRunner> make_diffusion_runner(
    const std::string& unet_weights, const std::string& vae_weights, const std::string& embeds_path,
    const FastConfig& fast_cfg = FastConfig{}, float vae_scaling_factor = kServerDefaultVaeScalingFactor,
    const UNetConfig& ucfg = UNetConfig{}, const VaeConfig& vcfg = VaeConfig{}, int latent_h = 128,
    int latent_w = 128);

struct BackendInfo {
  std::string name;
  int latent_channels = 0;
  int native_resolution = 0;
  bool needs_t5 = false;
};

struct LoraRequest {
  std::string name;
  float strength = 1.0f;
};

struct IDiffusionBackend {
  virtual ~IDiffusionBackend() = default;
  virtual void apply_loras(const std::vector<LoraRequest>& reqs) { (void)reqs; }
  virtual void clear_loras() {}
  virtual void generate(const std::string& prompt, const std::string& negative, int steps,
                        uint64_t seed, float cfg, int w, int h, std::vector<uint8_t>& rgb_out,
                        int& w_out, int& h_out) = 0;
  virtual BackendInfo info() const = 0;
  virtual std::string model_id() const = 0;
};

struct BackendConfig {
  std::string backend_name;
  std::string preset;
  std::string unet_weights;
  std::string vae_weights;
  std::string embeds;
  // text-encoder files of the reference's OpenVINO conditioner; not read here
  std::string tok_l, tok_g, enc_l, enc_g, tok_dll, device_l, device_g;
  FastConfig fast_cfg;
  float vae_scaling_factor = kServerDefaultVaeScalingFactor;
  // network shapes (SDXL defaults) and latent size of the native resolution
  UNetConfig unet_cfg;
  VaeConfig vae_cfg;
  int latent_size = 128;
};

// "sdxl" -> the precomputed-conditioning SDXL backend; anything else -> nullptr.
std::unique_ptr<IDiffusionBackend> make_backend(const BackendConfig& cfg);

// "sdxl-1.0" or "sdxl-1.0/<preset>" (reference compose_model_id).
std::string compose_model_id(const std::string& preset);

// LoRA name -> "<DOLLAMA_LORA_DIR or models/loras>/<name>.safetensors";
// names may hold [A-Za-z0-9_.-] and must not start with '.'.
std::string resolve_lora_path(const std::string& name);

}  // namespace dollama
