// C ABI of the host layer (include/dollama.h).  Every entry point catches
// C++ exceptions and turns them into a status plus dlm_last_error() text.
#include "dollama.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>

#include "check.hpp"
#include "device_arena.hpp"
#include "lora.hpp"
#include "pipeline.hpp"
#include "runner.hpp"
#include "safetensors.hpp"
#include "scheduler.hpp"
#include "unet.hpp"
#include "vae.hpp"

using namespace dollama;

namespace {

int guard_status(const std::exception& e, int code) {
  dlm_set_last_error(e.what());
  return code;
}

template <class F>
int guarded(F&& f) {
  try {
    f();
    return DLM_OK;
  } catch (const std::invalid_argument& e) {
    return guard_status(e, DLM_ERR_INVALID_ARG);
  } catch (const std::bad_alloc& e) {
    return guard_status(e, DLM_ERR_OUT_OF_MEMORY);
  } catch (const std::out_of_range& e) {
    return guard_status(e, DLM_ERR_NOT_FOUND);
  } catch (const std::exception& e) {
    return guard_status(e, DLM_ERR_STATE);
  }
}

UNetConfig to_cfg(const dlm_unet_config* c) {
  UNetConfig u;
  u.C0 = c->C0;
  u.C1 = c->C1;
  u.C2 = c->C2;
  u.depth1 = c->depth1;
  u.depth2 = c->depth2;
  u.head_dim = c->head_dim;
  u.cross_dim = c->cross_dim;
  u.text_dim = c->text_dim;
  u.id_dim = c->id_dim;
  u.in_channels = c->in_channels;
  u.out_channels = c->out_channels;
  u.groups = c->groups;
  return u;
}

VaeConfig to_vcfg(const dlm_vae_config* c) {
  VaeConfig v;
  for (int i = 0; i < 4; ++i) v.ch[i] = c->ch[i];
  v.latent_channels = c->latent_channels;
  v.out_channels = c->out_channels;
  v.layers = c->layers;
  v.groups = c->groups;
  v.fp32_from = c->fp32_from;
  return v;
}

void spec_out(const std::vector<WeightSpec>& specs, int index, char* name, int name_len, int* ndim,
              int64_t* shape) {
  if (!name || name_len <= 0 || !ndim || !shape) throw std::invalid_argument("NULL argument");
  if (index < 0 || index >= (int)specs.size()) throw std::invalid_argument("index out of range");
  const WeightSpec& s = specs[index];
  if ((int)s.name.size() >= name_len) throw std::invalid_argument("name buffer too small");
  std::memcpy(name, s.name.c_str(), s.name.size() + 1);
  *ndim = (int)s.shape.size();
  for (int i = 0; i < 4; ++i) shape[i] = i < *ndim ? s.shape[i] : 0;
}

DeviceArenaId arena_id(int id) {
  if (id < 0 || id >= kDeviceArenaCount) throw std::invalid_argument("bad arena id");
  return static_cast<DeviceArenaId>(id);
}

}  // namespace

extern "C" {

int dlm_unet_config_sdxl(dlm_unet_config* cfg) {
  if (!cfg) {
    dlm_set_last_error("dlm_unet_config_sdxl: NULL cfg");
    return DLM_ERR_INVALID_ARG;
  }
  const UNetConfig u;
  cfg->C0 = u.C0;
  cfg->C1 = u.C1;
  cfg->C2 = u.C2;
  cfg->depth1 = u.depth1;
  cfg->depth2 = u.depth2;
  cfg->head_dim = u.head_dim;
  cfg->cross_dim = u.cross_dim;
  cfg->text_dim = u.text_dim;
  cfg->id_dim = u.id_dim;
  cfg->in_channels = u.in_channels;
  cfg->out_channels = u.out_channels;
  cfg->groups = u.groups;
  return DLM_OK;
}

int dlm_unet_weight_count(const dlm_unet_config* cfg, int* count) {
  return guarded([&] {
    if (!cfg || !count) throw std::invalid_argument("NULL argument");
    *count = (int)unet_weight_specs(to_cfg(cfg)).size();
  });
}

int dlm_unet_weight_spec(const dlm_unet_config* cfg, int index, char* name, int name_len, int* ndim,
                         int64_t* shape) {
  return guarded([&] {
    if (!cfg || !name || name_len <= 0 || !ndim || !shape) throw std::invalid_argument("NULL argument");
    const auto specs = unet_weight_specs(to_cfg(cfg));
    if (index < 0 || index >= (int)specs.size()) throw std::invalid_argument("index out of range");
    const WeightSpec& s = specs[index];
    if ((int)s.name.size() >= name_len) throw std::invalid_argument("name buffer too small");
    std::memcpy(name, s.name.c_str(), s.name.size() + 1);
    *ndim = (int)s.shape.size();
    for (int i = 0; i < 4; ++i) shape[i] = i < *ndim ? s.shape[i] : 0;
  });
}

int dlm_unet_create(const dlm_unet_config* cfg, void** handle) {
  return guarded([&] {
    if (!cfg || !handle) throw std::invalid_argument("NULL argument");
    *handle = nullptr;
    *handle = new UNet(to_cfg(cfg));
  });
}

int dlm_unet_destroy(void* handle) {
  return guarded([&] { delete static_cast<UNet*>(handle); });
}

int dlm_unet_set_weight(void* handle, const char* name, const void* dptr, int ndim,
                        const int64_t* shape) {
  return guarded([&] {
    if (!handle || !name || ndim < 0 || ndim > 8 || (ndim > 0 && !shape))
      throw std::invalid_argument("bad argument");
    std::vector<int64_t> s(shape, shape + ndim);
    static_cast<UNet*>(handle)->set_weight(name, dptr, s);
  });
}

int dlm_unet_prepare(void* handle, void* stream) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<UNet*>(handle)->prepare(stream);
  });
}

int dlm_unet_load_safetensors(void* handle, const char* path, void* stream) {
  return guarded([&] {
    if (!handle || !path) throw std::invalid_argument("NULL argument");
    load_unet_safetensors(*static_cast<UNet*>(handle), path, stream);
  });
}

int dlm_unet_apply_lora(void* handle, const char* base_key, const void* A, const void* B, int rank,
                        int in_flat, int out_dim, float scale, void* stream) {
  return guarded([&] {
    if (!handle || !base_key || !A || !B) throw std::invalid_argument("NULL argument");
    static_cast<UNet*>(handle)->apply_lora(base_key, A, B, rank, in_flat, out_dim, scale, stream);
  });
}

static void fill_counts(int* counts, const LoraReport& r) {
  if (!counts) return;
  counts[0] = (int)r.modules;
  counts[1] = (int)r.te_skipped;
  counts[2] = (int)r.other_keys;
  counts[3] = (int)r.incomplete;
}

int dlm_unet_load_lora(void* handle, const char* path, float strength, int* counts, void* stream) {
  return guarded([&] {
    if (!handle || !path) throw std::invalid_argument("NULL argument");
    LoraReport rep;
    unet_apply_lora_file(*static_cast<UNet*>(handle), path, strength, &rep, stream);
    fill_counts(counts, rep);
  });
}

int dlm_unet_clear_loras(void* handle, void* stream) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<UNet*>(handle)->clear_loras(stream);
  });
}

int dlm_lora_scan(const dlm_unet_config* cfg, const char* path, float strength, int* counts,
                  dlm_lora_module_fn fn, void* user) {
  return guarded([&] {
    if (!cfg || !path) throw std::invalid_argument("NULL argument");
    SafeTensors st(path);
    LoraReport rep;
    const std::vector<LoraModule> mods =
        load_lora_modules(unet_weight_specs(to_cfg(cfg)), st, strength, &rep);
    fill_counts(counts, rep);
    if (fn)
      for (const LoraModule& m : mods) fn(m.base_key.c_str(), m.rank, m.in_flat, m.out_dim, m.scale, user);
  });
}

int dlm_unet_read_weight(void* handle, const char* name, void* host_out, size_t bytes, void* stream) {
  return guarded([&] {
    if (!handle || !name || !host_out) throw std::invalid_argument("NULL argument");
    static_cast<UNet*>(handle)->read_weight(name, host_out, bytes, stream);
  });
}

int dlm_f32_to_f16(const float* in, uint16_t* out, size_t n) {
  return guarded([&] {
    if ((!in || !out) && n) throw std::invalid_argument("NULL argument");
    for (size_t i = 0; i < n; ++i) out[i] = f32_to_f16_rne(in[i]);
  });
}

int dlm_unet_packed_bytes(void* handle, size_t* bytes) {
  return guarded([&] {
    if (!handle || !bytes) throw std::invalid_argument("NULL argument");
    *bytes = static_cast<UNet*>(handle)->packed_bytes();
  });
}

int dlm_unet_forward(void* handle, int B, int H, int W, const void* latent, const float* timesteps,
                     const void* ehs, int ctx_len, const void* text, const void* time_ids,
                     int ids_bstride, void* out, void* stream) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<UNet*>(handle)->forward(B, H, W, latent, timesteps, ehs, ctx_len, text, time_ids,
                                        ids_bstride, out, stream);
  });
}

int dlm_unet_run_resnet(void* handle, const char* prefix, const void* xa, int Ca, const void* xb,
                        int Cb, void* out, int B, int H, int W, const void* temb, void* stream) {
  return guarded([&] {
    if (!handle || !prefix) throw std::invalid_argument("NULL argument");
    static_cast<UNet*>(handle)->run_resnet(prefix, xa, Ca, xb, Cb, out, B, H, W, temb, stream);
  });
}

int dlm_unet_run_transformer_block(void* handle, const char* prefix, void* x, int B, int HW,
                                   const void* ehs, int ctx_len, void* stream) {
  return guarded([&] {
    if (!handle || !prefix) throw std::invalid_argument("NULL argument");
    static_cast<UNet*>(handle)->run_transformer_block(prefix, x, B, HW, ehs, ctx_len, stream);
  });
}

int dlm_unet_set_stage_hook(void* handle, dlm_unet_stage_hook hook, void* user) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<UNet*>(handle)->set_stage_hook(hook, user);
  });
}

int dlm_unet_set_graphs(void* handle, int on) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<UNet*>(handle)->set_graphs(on != 0);
  });
}

int dlm_unet_set_ln_fold(void* handle, int on) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<UNet*>(handle)->set_ln_fold(on);
  });
}

int dlm_unet_set_gn_fold(void* handle, int on) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<UNet*>(handle)->set_gn_fold(on != 0);
  });
}

int dlm_unet_graphs_captured(void* handle, size_t* count) {
  return guarded([&] {
    if (!handle || !count) throw std::invalid_argument("NULL argument");
    *count = static_cast<UNet*>(handle)->graphs_captured();
  });
}

int dlm_unet_set_profiling(void* handle, int on) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<UNet*>(handle)->set_profiling(on != 0);
  });
}

int dlm_unet_profile_report(void* handle, double* out, void* stream) {
  return guarded([&] {
    if (!handle || !out) throw std::invalid_argument("NULL argument");
    const auto r = static_cast<UNet*>(handle)->profile_report(stream);
    for (size_t c = 0; c < r.size() && c < 6; ++c) {
      out[4 * c + 0] = r[c].count;
      out[4 * c + 1] = r[c].ms;
      out[4 * c + 2] = r[c].flops;
      out[4 * c + 3] = r[c].bytes;
    }
  });
}

int dlm_unet_profile_kernels(void* handle, char* buf, size_t len, size_t* needed, void* stream) {
  return guarded([&] {
    if (!handle || !needed) throw std::invalid_argument("NULL argument");
    std::string text;
    char line[512];
    for (const auto& k : static_cast<UNet*>(handle)->profile_kernels(stream)) {
      std::snprintf(line, sizeof(line), "%s\t%d\t%d\t%.6f\t%.6e\t%.6e\t", k.name.c_str(), k.cls,
                    k.count, k.ms, k.flops, k.bytes);
      text += line;
      for (const auto& d : k.dims) {
        std::snprintf(line, sizeof(line), "%d,%d,%d,%d:%d;", d.first[0], d.first[1], d.first[2],
                      d.first[3], d.second);
        text += line;
      }
      text += "\n";
    }
    *needed = text.size() + 1;
    if (buf && len > 0) {
      const size_t n = std::min(len - 1, text.size());
      std::memcpy(buf, text.data(), n);
      buf[n] = 0;
    }
  });
}

int dlm_euler_schedule(int steps, float* sigmas, float* timesteps) {
  return guarded([&] {
    if (!sigmas || !timesteps) throw std::invalid_argument("NULL argument");
    EulerDiscreteScheduler s;
    s.set_timesteps(steps);
    for (int i = 0; i <= steps; ++i) sigmas[i] = s.sigmas()[i];
    for (int i = 0; i < steps; ++i) timesteps[i] = s.timesteps()[i];
  });
}

int dlm_pipeline_denoise(void* unet, int steps, float guidance, int H, int W, float* latent,
                         const void* ehs, int ctx_len, const void* text, const void* time_ids,
                         void* stream) {
  return guarded([&] {
    if (!unet) throw std::invalid_argument("NULL handle");
    DenoiseArgs a;
    a.steps = steps;
    a.guidance = guidance;
    a.H = H;
    a.W = W;
    a.latent = latent;
    a.ehs = ehs;
    a.ctx_len = ctx_len;
    a.text = text;
    a.time_ids = time_ids;
    denoise(*static_cast<UNet*>(unet), a, stream);
  });
}

int dlm_vae_config_sdxl(dlm_vae_config* cfg) {
  return guarded([&] {
    if (!cfg) throw std::invalid_argument("NULL cfg");
    const VaeConfig v;
    for (int i = 0; i < 4; ++i) cfg->ch[i] = v.ch[i];
    cfg->latent_channels = v.latent_channels;
    cfg->out_channels = v.out_channels;
    cfg->layers = v.layers;
    cfg->groups = v.groups;
    cfg->fp32_from = v.fp32_from;
  });
}

int dlm_vae_weight_count(const dlm_vae_config* cfg, int* count) {
  return guarded([&] {
    if (!cfg || !count) throw std::invalid_argument("NULL argument");
    *count = (int)vae_weight_specs(to_vcfg(cfg)).size();
  });
}

int dlm_vae_weight_spec(const dlm_vae_config* cfg, int index, char* name, int name_len, int* ndim,
                        int64_t* shape) {
  return guarded([&] {
    if (!cfg) throw std::invalid_argument("NULL cfg");
    spec_out(vae_weight_specs(to_vcfg(cfg)), index, name, name_len, ndim, shape);
  });
}

int dlm_vae_create(const dlm_vae_config* cfg, void** handle) {
  return guarded([&] {
    if (!cfg || !handle) throw std::invalid_argument("NULL argument");
    *handle = nullptr;
    *handle = new VAE(to_vcfg(cfg));
  });
}

int dlm_vae_destroy(void* handle) {
  return guarded([&] { delete static_cast<VAE*>(handle); });
}

int dlm_vae_set_weight(void* handle, const char* name, const void* dptr, int ndim,
                       const int64_t* shape) {
  return guarded([&] {
    if (!handle || !name || ndim < 0 || ndim > 8 || (ndim > 0 && !shape))
      throw std::invalid_argument("bad argument");
    std::vector<int64_t> s(shape, shape + ndim);
    static_cast<VAE*>(handle)->set_weight(name, dptr, s);
  });
}

int dlm_vae_prepare(void* handle, void* stream) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<VAE*>(handle)->prepare(stream);
  });
}

int dlm_vae_load_safetensors(void* handle, const char* path, void* stream) {
  return guarded([&] {
    if (!handle || !path) throw std::invalid_argument("NULL argument");
    load_vae_safetensors(*static_cast<VAE*>(handle), path, stream);
  });
}

int dlm_vae_packed_bytes(void* handle, size_t* bytes) {
  return guarded([&] {
    if (!handle || !bytes) throw std::invalid_argument("NULL argument");
    *bytes = static_cast<VAE*>(handle)->packed_bytes();
  });
}

int dlm_vae_decode(void* handle, int N, int h, int w, const void* latent, void* image, void* stream) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<VAE*>(handle)->decode(N, h, w, latent, image, stream);
  });
}

int dlm_vae_set_stage_hook(void* handle, dlm_vae_stage_hook hook, void* user) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<VAE*>(handle)->set_stage_hook(hook, user);
  });
}

int dlm_vae_set_profiling(void* handle, int on) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<VAE*>(handle)->set_profiling(on != 0);
  });
}

int dlm_vae_profile_report(void* handle, double* out, void* stream) {
  return guarded([&] {
    if (!handle || !out) throw std::invalid_argument("NULL argument");
    const auto r = static_cast<VAE*>(handle)->profile_report(stream);
    for (size_t c = 0; c < r.size() && c < 5; ++c) {
      out[4 * c + 0] = r[c].count;
      out[4 * c + 1] = r[c].ms;
      out[4 * c + 2] = r[c].flops;
      out[4 * c + 3] = r[c].bytes;
    }
  });
}

// ------------------------------------------------------------------ runner / backend

static void copy_rgb(const std::vector<uint8_t>& rgb, uint8_t* out, size_t cap) {
  if (rgb.size() > cap) throw std::invalid_argument("rgb_out holds " + std::to_string(cap) +
                                                    " bytes, the image needs " + std::to_string(rgb.size()));
  std::memcpy(out, rgb.data(), rgb.size());
}

int dlm_runner_create(const char* unet_weights, const char* vae_weights, const char* embeds,
                      float vae_scaling_factor, const dlm_unet_config* ucfg, const dlm_vae_config* vcfg,
                      int latent_h, int latent_w, void** handle) {
  return guarded([&] {
    if (!unet_weights || !vae_weights || !embeds || !handle) throw std::invalid_argument("NULL argument");
    *handle = nullptr;
    std::unique_ptr<IDiffusionRunner> r = make_diffusion_runner(
        unet_weights, vae_weights, embeds, FastConfig{}, vae_scaling_factor,
        ucfg ? to_cfg(ucfg) : UNetConfig{}, vcfg ? to_vcfg(vcfg) : VaeConfig{}, latent_h, latent_w);
    if (!r) throw std::runtime_error("make_diffusion_runner returned no runner (see stderr)");
    *handle = r.release();
  });
}

int dlm_runner_destroy(void* handle) {
  return guarded([&] { delete static_cast<IDiffusionRunner*>(handle); });
}

int dlm_runner_txt2img(void* handle, int steps, uint64_t seed, float guidance, const float* cond_ehs,
                       const float* cond_text, const float* uncond_ehs, const float* uncond_text,
                       const float* time_ids, uint8_t* rgb_out, size_t rgb_capacity, int* w, int* h) {
  return guarded([&] {
    if (!handle || !rgb_out || !w || !h) throw std::invalid_argument("NULL argument");
    std::vector<uint8_t> rgb;
    static_cast<IDiffusionRunner*>(handle)->run_txt2img(steps, seed, guidance, cond_ehs, cond_text,
                                                        uncond_ehs, uncond_text, time_ids, rgb, *w, *h);
    copy_rgb(rgb, rgb_out, rgb_capacity);
  });
}

int dlm_runner_generate(void* handle, int steps, uint64_t seed, uint8_t* rgb_out, size_t rgb_capacity,
                        int* w, int* h) {
  return guarded([&] {
    if (!handle || !rgb_out || !w || !h) throw std::invalid_argument("NULL argument");
    auto* r = dynamic_cast<DiffusionRunner*>(static_cast<IDiffusionRunner*>(handle));
    if (!r) throw std::invalid_argument("not a DiffusionRunner handle");
    std::vector<uint8_t> rgb;
    r->pipeline().generate(steps, seed, 1.0f, rgb, *w, *h);
    copy_rgb(rgb, rgb_out, rgb_capacity);
  });
}

int dlm_runner_apply_loras(void* handle, const char* const* paths, const float* strengths, int n) {
  return guarded([&] {
    if (!handle || n < 0 || (n > 0 && (!paths || !strengths))) throw std::invalid_argument("bad argument");
    std::vector<LoraFileRequest> reqs;
    for (int i = 0; i < n; ++i) reqs.push_back(LoraFileRequest{paths[i], strengths[i]});
    static_cast<IDiffusionRunner*>(handle)->apply_loras(reqs);
  });
}

int dlm_runner_clear_loras(void* handle) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<IDiffusionRunner*>(handle)->clear_loras();
  });
}

int dlm_backend_create(const dlm_backend_config* c, void** handle) {
  return guarded([&] {
    if (!c || !handle || !c->backend_name) throw std::invalid_argument("NULL argument");
    *handle = nullptr;
    BackendConfig b;
    b.backend_name = c->backend_name;
    b.preset = c->preset ? c->preset : "";
    b.unet_weights = c->unet_weights ? c->unet_weights : "";
    b.vae_weights = c->vae_weights ? c->vae_weights : "";
    b.embeds = c->embeds ? c->embeds : "";
    b.vae_scaling_factor = c->vae_scaling_factor;
    if (c->unet_cfg) b.unet_cfg = to_cfg(c->unet_cfg);
    if (c->vae_cfg) b.vae_cfg = to_vcfg(c->vae_cfg);
    if (c->latent_size > 0) b.latent_size = c->latent_size;
    std::unique_ptr<IDiffusionBackend> be = make_backend(b);
    if (!be) throw std::out_of_range("make_backend: no backend for '" + b.backend_name + "' (see stderr)");
    *handle = be.release();
  });
}

int dlm_backend_destroy(void* handle) {
  return guarded([&] { delete static_cast<IDiffusionBackend*>(handle); });
}

int dlm_backend_generate(void* handle, const char* prompt, const char* negative, int steps, uint64_t seed,
                         float cfg, int w, int h, uint8_t* rgb_out, size_t rgb_capacity, int* w_out,
                         int* h_out) {
  return guarded([&] {
    if (!handle || !rgb_out || !w_out || !h_out) throw std::invalid_argument("NULL argument");
    std::vector<uint8_t> rgb;
    static_cast<IDiffusionBackend*>(handle)->generate(prompt ? prompt : "", negative ? negative : "", steps,
                                                      seed, cfg, w, h, rgb, *w_out, *h_out);
    copy_rgb(rgb, rgb_out, rgb_capacity);
  });
}

int dlm_backend_info(void* handle, char* name, int name_len, int* latent_channels, int* native_resolution,
                     int* needs_t5) {
  return guarded([&] {
    if (!handle || !name || name_len <= 0 || !latent_channels || !native_resolution || !needs_t5)
      throw std::invalid_argument("NULL argument");
    const BackendInfo i = static_cast<IDiffusionBackend*>(handle)->info();
    if ((int)i.name.size() >= name_len) throw std::invalid_argument("name buffer too small");
    std::memcpy(name, i.name.c_str(), i.name.size() + 1);
    *latent_channels = i.latent_channels;
    *native_resolution = i.native_resolution;
    *needs_t5 = i.needs_t5 ? 1 : 0;
  });
}

int dlm_backend_model_id(void* handle, char* buf, int len) {
  return guarded([&] {
    if (!handle || !buf || len <= 0) throw std::invalid_argument("NULL argument");
    const std::string id = static_cast<IDiffusionBackend*>(handle)->model_id();
    if ((int)id.size() >= len) throw std::invalid_argument("buffer too small");
    std::memcpy(buf, id.c_str(), id.size() + 1);
  });
}

int dlm_backend_apply_loras(void* handle, const char* const* names, const float* strengths, int n) {
  return guarded([&] {
    if (!handle || n < 0 || (n > 0 && (!names || !strengths))) throw std::invalid_argument("bad argument");
    std::vector<LoraRequest> reqs;
    for (int i = 0; i < n; ++i) reqs.push_back(LoraRequest{names[i], strengths[i]});
    static_cast<IDiffusionBackend*>(handle)->apply_loras(reqs);
  });
}

int dlm_backend_clear_loras(void* handle) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<IDiffusionBackend*>(handle)->clear_loras();
  });
}

int dlm_randn_latent(uint64_t seed, double sigma0, float* out, size_t n) {
  return guarded([&] {
    if (!out && n) throw std::invalid_argument("NULL out");
    randn_latent(seed, sigma0, out, n);
  });
}

// ------------------------------------------------------------------ safetensors

int dlm_st_open(const char* path, void** handle) {
  return guarded([&] {
    if (!path || !handle) throw std::invalid_argument("NULL argument");
    *handle = nullptr;
    *handle = new SafeTensors(path);
  });
}

int dlm_st_close(void* handle) {
  return guarded([&] { delete static_cast<SafeTensors*>(handle); });
}

int dlm_st_count(void* handle, int* count) {
  return guarded([&] {
    if (!handle || !count) throw std::invalid_argument("NULL argument");
    *count = (int)static_cast<SafeTensors*>(handle)->names().size();
  });
}

int dlm_st_name(void* handle, int index, char* buf, int len) {
  return guarded([&] {
    if (!handle || !buf || len <= 0) throw std::invalid_argument("NULL argument");
    const auto& ns = static_cast<SafeTensors*>(handle)->names();
    if (index < 0 || index >= (int)ns.size()) throw std::invalid_argument("index out of range");
    if ((int)ns[index].size() >= len) throw std::invalid_argument("buffer too small");
    std::memcpy(buf, ns[index].c_str(), ns[index].size() + 1);
  });
}

int dlm_st_info(void* handle, const char* name, int* dtype, int* ndim, int64_t* shape, size_t* nbytes) {
  return guarded([&] {
    if (!handle || !name || !dtype || !ndim || !shape || !nbytes) throw std::invalid_argument("NULL argument");
    const SafeTensors& st = *static_cast<SafeTensors*>(handle);
    if (!st.contains(name)) throw std::out_of_range(std::string("safetensors: no tensor '") + name + "'");
    *dtype = (int)st.dtype(name);
    const auto& sh = st.shape(name);
    if (sh.size() > 8) throw std::invalid_argument("more than 8 dimensions");
    *ndim = (int)sh.size();
    for (size_t i = 0; i < sh.size(); ++i) shape[i] = sh[i];
    st.tensor_bytes(name, *nbytes);
  });
}

int dlm_st_read(void* handle, const char* name, void* out, size_t bytes) {
  return guarded([&] {
    if (!handle || !name || (!out && bytes)) throw std::invalid_argument("NULL argument");
    const SafeTensors& st = *static_cast<SafeTensors*>(handle);
    size_t nb = 0;
    const uint8_t* p = st.tensor_bytes(name, nb);
    if (bytes != nb) throw std::invalid_argument("byte count mismatch");
    std::memcpy(out, p, nb);
  });
}

int dlm_arena_stats(int id, uint64_t* out) {
  return guarded([&] {
    if (!out) throw std::invalid_argument("NULL out");
    const DeviceArenaStats s = device_arena_stats(arena_id(id));
    const uint64_t v[11] = {s.cuda_malloc_calls, s.cuda_free_calls, s.chunk_alloc_calls, s.alloc_calls,
                            s.total_capacity, s.live_chunks, s.bytes_in_use, s.peak_bytes_in_use,
                            s.live_request_bytes, s.peak_request_bytes, s.reserved_bytes};
    for (int i = 0; i < 11; ++i) out[i] = v[i];
  });
}

int dlm_arena_release(int id) {
  return guarded([&] { device_arena_release(arena_id(id)); });
}

int dlm_arena_reserve(int id, size_t bytes) {
  return guarded([&] { device_arena_reserve(arena_id(id), bytes); });
}

int dlm_arena_fill(int id, int pattern) {
  return guarded([&] { device_arena_fill(arena_id(id), pattern); });
}

}  // extern "C"
