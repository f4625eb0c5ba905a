// C ABI of the host layer (include/dollama.h).  Every entry point catches
// C++ exceptions and turns them into a status plus dlm_last_error() text.
#include "dollama.h"

#include <cstring>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>

#include "check.hpp"
#include "device_arena.hpp"
#include "lora.hpp"
#include "pipeline.hpp"
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
    UNet* u = static_cast<UNet*>(handle);
    SafeTensors st(path);
    // one upload of the whole data region, tensors registered in place
    void* dev = nullptr;
    DLM_CALL(dlm_malloc(&dev, st.data_bytes()));
    std::unique_ptr<void, void (*)(void*)> hold(dev, [](void* p) { (void)dlm_free(p); });
    DLM_CALL(dlm_memcpy(dev, st.data(), st.data_bytes(), 0));
    for (const WeightSpec& s : unet_weight_specs(u->config())) {
      if (!st.has(s.name)) throw std::runtime_error("safetensors: missing '" + s.name + "'");
      if (st.dtype(s.name) != StDtype::F16)
        throw std::runtime_error("safetensors: '" + s.name + "' is not F16");
      if (st.offset(s.name) % 2 != 0) throw std::runtime_error("safetensors: misaligned tensor");
      u->set_weight(s.name, static_cast<char*>(dev) + st.offset(s.name), st.shape(s.name));
    }
    u->prepare(stream);
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
    UNet* u = static_cast<UNet*>(handle);
    SafeTensors st(path);
    LoraReport rep;
    std::vector<LoraModule> mods = load_lora_modules(unet_weight_specs(u->config()), st, strength, &rep);
    for (const LoraModule& m : mods) {
      void* dev = nullptr;
      const size_t na = m.a_fp16.size(), nb = m.b_fp16.size();
      DLM_CALL(dlm_malloc(&dev, (na + nb) * 2));
      std::unique_ptr<void, void (*)(void*)> hold(dev, [](void* p) { (void)dlm_free(p); });
      DLM_CALL(dlm_memcpy(dev, m.a_fp16.data(), na * 2, 0));
      DLM_CALL(dlm_memcpy(static_cast<uint16_t*>(dev) + na, m.b_fp16.data(), nb * 2, 0));
      u->apply_lora(m.base_key, dev, static_cast<uint16_t*>(dev) + na, m.rank, m.in_flat, m.out_dim,
                    m.scale, stream);
    }
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

int dlm_unet_set_stage_hook(void* handle, dlm_unet_stage_hook hook, void* user) {
  return guarded([&] {
    if (!handle) throw std::invalid_argument("NULL handle");
    static_cast<UNet*>(handle)->set_stage_hook(hook, user);
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
    VAE* v = static_cast<VAE*>(handle);
    SafeTensors st(path);
    void* dev = nullptr;
    DLM_CALL(dlm_malloc(&dev, st.data_bytes()));
    std::unique_ptr<void, void (*)(void*)> hold(dev, [](void* p) { (void)dlm_free(p); });
    DLM_CALL(dlm_memcpy(dev, st.data(), st.data_bytes(), 0));
    for (const WeightSpec& s : vae_weight_specs(v->config())) {
      if (!st.has(s.name)) throw std::runtime_error("safetensors: missing '" + s.name + "'");
      if (st.dtype(s.name) != StDtype::F16)
        throw std::runtime_error("safetensors: '" + s.name + "' is not F16");
      if (st.offset(s.name) % 2 != 0) throw std::runtime_error("safetensors: misaligned tensor");
      v->set_weight(s.name, static_cast<char*>(dev) + st.offset(s.name), st.shape(s.name));
    }
    v->prepare(stream);
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

}  // extern "C"
