// Diffusion runner and backend registry (see runner.hpp).
#include "runner.hpp"

#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <stdexcept>

#include "safetensors.hpp"

namespace dollama {

namespace {

bool file_readable(const std::string& path) {
  if (path.empty()) return false;
  std::ifstream f(path, std::ios::binary);
  return f.good();
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      uint32_t m = man;
      do {
        ++e;
        m <<= 1;
      } while (!(m & 0x400u));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

std::vector<float> f32_of(const SafeTensors& st, const std::string& name, size_t expect) {
  if (!st.contains(name)) throw std::runtime_error("embeds: missing '" + name + "'");
  if (st.dtype(name) != StDtype::F16) throw std::runtime_error("embeds: '" + name + "' is not F16");
  size_t nbytes = 0;
  const uint8_t* p = st.tensor_bytes(name, nbytes);
  if (nbytes != expect * 2) throw std::runtime_error("embeds: '" + name + "' size mismatch");
  std::vector<float> v(expect);
  for (size_t i = 0; i < expect; ++i) v[i] = f16_to_f32((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
  return v;
}

// "sdxl" backend over precomputed conditioning.
class SdxlBackend : public IDiffusionBackend {
 public:
  static constexpr float kGuidanceScale = 7.5f;

  explicit SdxlBackend(const BackendConfig& c) : preset_(c.preset), cfg_(c) {
    runner_ = make_diffusion_runner(c.unet_weights, c.vae_weights, c.embeds, c.fast_cfg,
                                    c.vae_scaling_factor, c.unet_cfg, c.vae_cfg, c.latent_size,
                                    c.latent_size);
    if (!runner_) throw std::runtime_error("SdxlBackend: the diffusion runner could not be built");
    SafeTensors st(c.embeds);
    const size_t nt = (size_t)c.unet_cfg.text_dim;
    size_t nbytes = 0;
    st.tensor_bytes("input_encoder_hidden_states_f16", nbytes);
    const size_t ne = nbytes / 2;
    cond_ehs_ = f32_of(st, "input_encoder_hidden_states_f16", ne);
    cond_txt_ = f32_of(st, "input_text_embeds_f16", nt);
    ids_ = f32_of(st, "input_time_ids_f16", 6);
    uncond_ehs_ = st.contains("uncond_encoder_hidden_states_f16")
                      ? f32_of(st, "uncond_encoder_hidden_states_f16", ne)
                      : std::vector<float>(ne, 0.0f);
    uncond_txt_ = st.contains("uncond_text_embeds_f16") ? f32_of(st, "uncond_text_embeds_f16", nt)
                                                   : std::vector<float>(nt, 0.0f);
  }

  void generate(const std::string& prompt, const std::string& negative, int steps, uint64_t seed,
                float cfg, int w, int h, std::vector<uint8_t>& rgb_out, int& w_out,
                int& h_out) override {
    (void)prompt;
    (void)negative;
    (void)w;
    (void)h;
    const int real_steps = steps > 0 ? steps : 20;
    const float scale = cfg > 0.0f ? cfg : kGuidanceScale;
    rgb_out.clear();
    w_out = 0;
    h_out = 0;
    runner_->run_txt2img(real_steps, seed, scale, cond_ehs_.data(), cond_txt_.data(), uncond_ehs_.data(),
                         uncond_txt_.data(), ids_.data(), rgb_out, w_out, h_out);
  }

  void apply_loras(const std::vector<LoraRequest>& reqs) override {
    if (reqs.empty()) return;
    std::vector<LoraFileRequest> files;
    files.reserve(reqs.size());
    for (const LoraRequest& r : reqs) {
      const std::string path = resolve_lora_path(r.name);
      if (!file_readable(path))
        throw std::invalid_argument("SdxlBackend: LoRA '" + r.name + "' not found: " + path);
      files.push_back(LoraFileRequest{path, r.strength});
    }
    runner_->apply_loras(files);
  }

  void clear_loras() override { runner_->clear_loras(); }

  BackendInfo info() const override {
    return {"sdxl", cfg_.unet_cfg.in_channels, 8 * cfg_.latent_size, false};
  }

  std::string model_id() const override { return compose_model_id(preset_); }

 private:
  std::string preset_;
  BackendConfig cfg_;
  std::unique_ptr<IDiffusionRunner> runner_;
  std::vector<float> cond_ehs_, cond_txt_, uncond_ehs_, uncond_txt_, ids_;
};

}  // namespace

DiffusionRunner::DiffusionRunner(const std::string& unet, const std::string& vae,
                                 const std::string& embeds, const FastConfig& fast, float sf,
                                 const UNetConfig& ucfg, const VaeConfig& vcfg, int lh, int lw)
    : pipe_(unet, vae, embeds, fast, sf, ucfg, vcfg, lh, lw) {}

void DiffusionRunner::run_txt2img(int steps, uint64_t seed, float guidance_scale, const float* cond_ehs,
                                  const float* cond_text_embeds, const float* uncond_ehs,
                                  const float* uncond_text_embeds, const float* time_ids,
                                  std::vector<uint8_t>& rgb_out, int& w, int& h) {
  pipe_.generate_txt2img(steps, seed, guidance_scale, cond_ehs, cond_text_embeds, uncond_ehs,
                         uncond_text_embeds, time_ids, rgb_out, w, h);
}

void DiffusionRunner::apply_loras(const std::vector<LoraFileRequest>& reqs) {
  try {
    for (const LoraFileRequest& r : reqs) pipe_.apply_lora_file(r.path, r.strength);
  } catch (...) {
    pipe_.clear_loras();
    throw;
  }
}

void DiffusionRunner::clear_loras() { pipe_.clear_loras(); }

std::unique_ptr<IDiffusionRunner> make_diffusion_runner(const std::string& unet_weights,
                                                        const std::string& vae_weights,
                                                        const std::string& embeds_path,
                                                        const FastConfig& fast_cfg,
                                                        float vae_scaling_factor,
                                                        const UNetConfig& ucfg, const VaeConfig& vcfg,
                                                        int latent_h, int latent_w) {
  if (!file_readable(unet_weights) || !file_readable(vae_weights) || !file_readable(embeds_path)) {
    std::cerr << "[diffusion_runner] weights or embeddings missing\n"
              << "  unet  = " << unet_weights << (file_readable(unet_weights) ? " [OK]" : " [MISSING]") << "\n"
              << "  vae   = " << vae_weights << (file_readable(vae_weights) ? " [OK]" : " [MISSING]") << "\n"
              << "  embed = " << embeds_path << (file_readable(embeds_path) ? " [OK]" : " [MISSING]") << "\n";
    return nullptr;
  }
  try {
    return std::make_unique<DiffusionRunner>(unet_weights, vae_weights, embeds_path, fast_cfg,
                                             vae_scaling_factor, ucfg, vcfg, latent_h, latent_w);
  } catch (const std::exception& e) {
    std::cerr << "[diffusion_runner] construction failed: " << e.what() << "\n";
    return nullptr;
  }
}

std::unique_ptr<IDiffusionBackend> make_backend(const BackendConfig& cfg) {
  if (cfg.backend_name == "sdxl") {
    try {
      return std::make_unique<SdxlBackend>(cfg);
    } catch (const std::exception& e) {
      std::cerr << "[make_backend] sdxl: " << e.what() << "\n";
      return nullptr;
    }
  }
  return nullptr;
}

std::string compose_model_id(const std::string& preset) {
  return preset.empty() ? "sdxl-1.0" : "sdxl-1.0/" + preset;
}

std::string resolve_lora_path(const std::string& name) {
  if (name.empty() || name[0] == '.') throw std::invalid_argument("invalid LoRA name: '" + name + "'");
  for (const char c : name) {
    const bool ok = (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') ||
                    c == '_' || c == '-' || c == '.';
    if (!ok) throw std::invalid_argument("invalid LoRA name: '" + name + "'");
  }
  const char* env = std::getenv("DOLLAMA_LORA_DIR");
  const std::string dir = (env && env[0]) ? env : "models/loras";
  return dir + "/" + name + ".safetensors";
}

}  // namespace dollama
