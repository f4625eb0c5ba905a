// Text-to-image pipeline: device-resident denoise loop, VAE decode, RGB8.
#include "pipeline.hpp"

#include <cmath>
#include <memory>
#include <stdexcept>
#include <vector>

#include "check.hpp"
#include "device_arena.hpp"
#include "lora.hpp"
#include "safetensors.hpp"
#include "scheduler.hpp"

namespace dollama {

// ------------------------------------------------------------------ noise

namespace {
// splitmix64 output function of state x (Steele, Lea, Flood 2014)
uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ULL;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
  return x ^ (x >> 31);
}
}  // namespace

Randn::Randn(uint64_t seed) : s0_(splitmix64(seed)), s1_(splitmix64(seed + 0x9E3779B97F4A7C15ULL)) {}

double Randn::uniform() {
  // xorshift128+ (Vigna 2014: a = 23, b = 17, c = 26), result s1 + s0_old
  uint64_t a = s0_;
  const uint64_t b = s1_;
  s0_ = b;
  a ^= a << 23;
  s1_ = a ^ b ^ (a >> 17) ^ (b >> 26);
  return (double)((s1_ + b) >> 11) * (1.0 / 9007199254740992.0);  // 53 bits / 2^53
}

double Randn::next() {
  if (has_spare_) {
    has_spare_ = false;
    return spare_;
  }
  double u1;
  do {
    u1 = uniform();
  } while (u1 <= 1e-12);
  const double u2 = uniform();
  const double r = std::sqrt(-2.0 * std::log(u1));
  const double th = 2.0 * 3.14159265358979323846 * u2;
  spare_ = r * std::sin(th);
  has_spare_ = true;
  return r * std::cos(th);
}

void randn_latent(uint64_t seed, double sigma0, float* out, size_t n) {
  Randn g(seed);
  for (size_t k = 0; k < n; ++k) out[k] = (float)(g.next() * sigma0);
}

// ------------------------------------------------------------------ loop

void denoise(UNet& unet, const DenoiseArgs& a, void* stream, bool cfg) {
  if (a.steps <= 0) throw std::invalid_argument("denoise: steps must be positive");
  if (!a.latent || !a.ehs || !a.text || !a.time_ids) throw std::invalid_argument("denoise: NULL input");
  const UNetConfig& c = unet.config();
  const int n = c.in_channels * a.H * a.W;
  if (c.in_channels != c.out_channels) throw std::invalid_argument("denoise: in/out channels differ");
  const int B = cfg ? 2 : 1;

  EulerDiscreteScheduler sched;
  sched.set_timesteps(a.steps);
  const auto& ts = sched.timesteps();
  const auto& sg = sched.sigmas();

  DeviceArenaScope scope(DeviceArenaId::UNetPersist);
  // per-step timesteps [steps][B] (cond and uncond share t)
  std::vector<float> host_t((size_t)B * a.steps);
  for (int i = 0; i < a.steps; ++i)
    for (int b = 0; b < B; ++b) host_t[(size_t)B * i + b] = ts[i];
  float* d_t = scope.alloc<float>(host_t.size());
  DLM_CALL(dlm_memcpy(d_t, host_t.data(), host_t.size() * sizeof(float), 0));
  void* model_in = scope.alloc<uint16_t>((size_t)B * n);
  void* noise = scope.alloc<uint16_t>((size_t)B * n);
  // the step's timesteps are copied into one slot, so every forward of the
  // loop has the same arguments (one captured graph serves all steps)
  float* d_tslot = scope.alloc<float>(B);

  DLM_CALL(dlm_scale_latent_fp16(a.latent, model_in, n, (float)sched.input_scale(0), B, stream));
  for (int i = 0; i < a.steps; ++i) {
    DLM_CALL(dlm_memcpy_async(d_tslot, d_t + (size_t)B * i, B * sizeof(float), 2, stream));
    unet.forward(B, a.H, a.W, model_in, d_tslot, a.ehs, a.ctx_len, a.text, a.time_ids, 0, noise, stream);
    const float next_scale = i + 1 < a.steps ? (float)sched.input_scale(i + 1) : 1.0f;
    if (cfg)
      DLM_CALL(dlm_euler_cfg_step(a.latent, noise, model_in, n, a.guidance, sg[i], sg[i + 1], next_scale,
                                  stream));
    else
      DLM_CALL(dlm_euler_step(a.latent, noise, model_in, n, sg[i], sg[i + 1], next_scale, stream));
  }
}

// ------------------------------------------------------------------ weights

namespace {
template <class Net>
void load_safetensors(Net& net, const std::vector<WeightSpec>& specs, const SafeTensors& st,
                      const std::string& what, void* stream) {
  // one upload of the whole data region, tensors registered in place
  void* dev = nullptr;
  DLM_CALL(dlm_malloc(&dev, st.data_bytes()));
  std::unique_ptr<void, void (*)(void*)> hold(dev, [](void* p) { (void)dlm_free(p); });
  DLM_CALL(dlm_memcpy(dev, st.data(), st.data_bytes(), 0));
  for (const WeightSpec& s : specs) {
    if (!st.contains(s.name)) throw std::runtime_error("safetensors: missing '" + s.name + "' in " + what);
    if (st.dtype(s.name) != StDtype::F16)
      throw std::runtime_error("safetensors: '" + s.name + "' is not F16");
    if (st.offset(s.name) % 2 != 0) throw std::runtime_error("safetensors: misaligned tensor");
    net.set_weight(s.name, static_cast<char*>(dev) + st.offset(s.name), st.shape_i64(s.name));
  }
  net.prepare(stream);  // packs into the handle's memory and synchronises
}

std::vector<uint16_t> f16_tensor(const SafeTensors& st, const std::string& name, size_t expect) {
  if (!st.contains(name)) throw std::runtime_error("embeds: missing '" + name + "'");
  if (st.dtype(name) != StDtype::F16) throw std::runtime_error("embeds: '" + name + "' is not F16");
  size_t nbytes = 0;
  const uint8_t* p = st.tensor_bytes(name, nbytes);
  if (expect && nbytes != expect * 2) throw std::runtime_error("embeds: '" + name + "' size mismatch");
  std::vector<uint16_t> v(nbytes / 2);
  for (size_t i = 0; i < v.size(); ++i) v[i] = (uint16_t)(p[2 * i] | (p[2 * i + 1] << 8));
  return v;
}

void* upload(const std::vector<uint16_t>& v) {
  void* d = nullptr;
  DLM_CALL(dlm_malloc(&d, v.size() * 2));
  DLM_CALL(dlm_memcpy(d, v.data(), v.size() * 2, 0));
  return d;
}

std::vector<uint16_t> to_f16(const float* x, size_t n) {
  std::vector<uint16_t> v(n);
  for (size_t i = 0; i < n; ++i) v[i] = f32_to_f16_rne(x[i]);
  return v;
}
}  // namespace

void load_unet_safetensors(UNet& u, const std::string& path, void* stream) {
  const SafeTensors st(path);
  load_safetensors(u, unet_weight_specs(u.config()), st, path, stream);
}

void load_unet_safetensors(UNet& u, const SafeTensors& st, void* stream) {
  load_safetensors(u, unet_weight_specs(u.config()), st, "the safetensors file", stream);
}

void load_vae_safetensors(VAE& v, const std::string& path, void* stream) {
  const SafeTensors st(path);
  load_safetensors(v, vae_weight_specs(v.config()), st, path, stream);
}

// ------------------------------------------------------------------ pipeline

DiffusionPipeline::DiffusionPipeline(const std::string& unet_weights, const std::string& vae_weights,
                                     const std::string& embeds_path, const FastConfig& fast,
                                     float vae_scaling_factor, const UNetConfig& ucfg,
                                     const VaeConfig& vcfg, int latent_h, int latent_w)
    : unet_(ucfg), vae_(vcfg), fast_(fast), lh_(latent_h), lw_(latent_w) {
  // an invalid scaling factor falls back to the default (reference diffusion.cu:293-303)
  vae_scaling_ = (vae_scaling_factor > 0.0f && std::isfinite(vae_scaling_factor)) ? vae_scaling_factor
                                                                                  : kDefaultVaeScalingFactor;
  if (lh_ <= 0 || lw_ <= 0 || lh_ % 4 || lw_ % 4)
    throw std::invalid_argument("DiffusionPipeline: latent size must be positive multiples of 4");
  if (vcfg.latent_channels != ucfg.out_channels)
    throw std::invalid_argument("DiffusionPipeline: VAE latent channels != UNet channels");
  try {
    SafeTensors emb(embeds_path);
    const std::vector<uint16_t> ehs = f16_tensor(emb, "input_encoder_hidden_states_f16", 0);
    if (ehs.empty() || ehs.size() % ucfg.cross_dim)
      throw std::runtime_error("embeds: encoder hidden states not a multiple of cross_dim");
    ctx_len_ = (int)(ehs.size() / ucfg.cross_dim);
    d_ehs_ = upload(ehs);
    d_text_ = upload(f16_tensor(emb, "input_text_embeds_f16", ucfg.text_dim));
    d_ids_ = upload(f16_tensor(emb, "input_time_ids_f16", 6));
    load_unet_safetensors(unet_, unet_weights, nullptr);
    load_vae_safetensors(vae_, vae_weights, nullptr);
  } catch (...) {
    for (void* p : {d_ehs_, d_text_, d_ids_})
      if (p) (void)dlm_free(p);
    throw;
  }
}

DiffusionPipeline::~DiffusionPipeline() {
  for (void* p : {d_ehs_, d_text_, d_ids_})
    if (p) (void)dlm_free(p);
}

void DiffusionPipeline::run(int steps, uint64_t seed, float guidance, bool cfg, const void* d_ehs,
                            const void* d_text, const void* d_ids, std::vector<uint8_t>& rgb_out,
                            int& w, int& h) {
  const UNetConfig& c = unet_.config();
  const size_t n = (size_t)c.in_channels * lh_ * lw_;
  EulerDiscreteScheduler sched;
  sched.set_timesteps(steps);
  std::vector<float> lat(n);
  randn_latent(seed, (double)sched.sigmas()[0], lat.data(), n);

  void* stream = nullptr;
  DeviceArenaScope scope(DeviceArenaId::UNetPersist);
  float* d_lat = scope.alloc<float>(n);
  DLM_CALL(dlm_memcpy(d_lat, lat.data(), n * sizeof(float), 0));
  DenoiseArgs a;
  a.steps = steps;
  a.guidance = guidance;
  a.H = lh_;
  a.W = lw_;
  a.latent = d_lat;
  a.ehs = d_ehs;
  a.ctx_len = ctx_len_;
  a.text = d_text;
  a.time_ids = d_ids;
  denoise(unet_, a, stream, cfg);
  // latent / scaling_factor -> VAE -> RGB8 (reference diffusion.cu:980-998)
  const int W = 8 * lw_, H = 8 * lh_;
  void* d_z = scope.alloc<uint16_t>(n);
  void* d_img = scope.alloc<uint16_t>((size_t)3 * H * W);
  uint8_t* d_rgb = scope.alloc<uint8_t>((size_t)3 * H * W);
  DLM_CALL(dlm_latent_to_vae_fp16(d_lat, d_z, (long long)n, vae_scaling_, stream));
  vae_.decode(1, lh_, lw_, d_z, d_img, stream);
  DLM_CALL(dlm_image_to_rgb8(d_img, d_rgb, 1, H, W, stream));
  rgb_out.resize((size_t)3 * H * W);
  DLM_CALL(dlm_stream_synchronize(stream));
  DLM_CALL(dlm_memcpy(rgb_out.data(), d_rgb, rgb_out.size(), 1));
  w = W;
  h = H;
}

void DiffusionPipeline::generate(int steps, uint64_t seed, float guidance_scale,
                                 std::vector<uint8_t>& rgb_out, int& w, int& h) {
  if (steps <= 0) throw std::runtime_error("DiffusionPipeline::generate: steps must be > 0");
  if (std::fabs(guidance_scale - 1.0f) > 1e-6f)
    throw std::runtime_error(
        "DiffusionPipeline::generate: guidance_scale != 1.0 is not supported (use generate_txt2img for CFG)");
  run(steps, seed, 1.0f, false, d_ehs_, d_text_, d_ids_, rgb_out, w, h);
}

void DiffusionPipeline::generate_txt2img(int steps, uint64_t seed, float guidance_scale,
                                         const float* cond_ehs, const float* cond_text_embeds,
                                         const float* uncond_ehs, const float* uncond_text_embeds,
                                         const float* time_ids, std::vector<uint8_t>& rgb_out, int& w,
                                         int& h) {
  if (steps <= 0) throw std::runtime_error("DiffusionPipeline::generate_txt2img: steps must be > 0");
  if (!cond_ehs || !cond_text_embeds || !uncond_ehs || !uncond_text_embeds || !time_ids)
    throw std::runtime_error("DiffusionPipeline::generate_txt2img: null embedding pointer");
  const UNetConfig& c = unet_.config();
  const size_t ne = (size_t)ctx_len_ * c.cross_dim, nt = (size_t)c.text_dim;
  // fp32 -> fp16 (round to nearest even) on the host, as the reference does
  std::vector<uint16_t> ehs2(2 * ne), txt2(2 * nt);
  {
    const std::vector<uint16_t> ce = to_f16(cond_ehs, ne), ue = to_f16(uncond_ehs, ne);
    const std::vector<uint16_t> ct = to_f16(cond_text_embeds, nt), ut = to_f16(uncond_text_embeds, nt);
    std::copy(ce.begin(), ce.end(), ehs2.begin());
    std::copy(ue.begin(), ue.end(), ehs2.begin() + ne);
    std::copy(ct.begin(), ct.end(), txt2.begin());
    std::copy(ut.begin(), ut.end(), txt2.begin() + nt);
  }
  const std::vector<uint16_t> ids = to_f16(time_ids, 6);
  DeviceArenaScope scope(DeviceArenaId::UNetPersist);
  void* d_ehs = scope.alloc<uint16_t>(ehs2.size());
  void* d_txt = scope.alloc<uint16_t>(txt2.size());
  void* d_ids = scope.alloc<uint16_t>(8);
  DLM_CALL(dlm_memcpy(d_ehs, ehs2.data(), ehs2.size() * 2, 0));
  DLM_CALL(dlm_memcpy(d_txt, txt2.data(), txt2.size() * 2, 0));
  DLM_CALL(dlm_memcpy(d_ids, ids.data(), ids.size() * 2, 0));
  run(steps, seed, guidance_scale, true, d_ehs, d_txt, d_ids, rgb_out, w, h);
}

void DiffusionPipeline::apply_lora_file(const std::string& path, float strength) {
  unet_apply_lora_file(unet_, path, strength, nullptr, nullptr);
}

void DiffusionPipeline::clear_loras() { unet_.clear_loras(nullptr); }

}  // namespace dollama
