// The reference's UNet host API (src/infer/unet.cuh:53-146) over UNet and
// the C ABI: see unet_api.hpp for the contract.
#include "unet_api.hpp"

#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>

#include "check.hpp"
#include "pipeline.hpp"

namespace dollama {

namespace {

constexpr int kMaxBatch = 16;

std::mutex g_hook_mu;
UnetStageHookFn g_hook = nullptr;

UnetStageHookFn current_hook() {
  std::lock_guard<std::mutex> lk(g_hook_mu);
  return g_hook;
}

struct Handle {
  std::unique_ptr<UNet> net;
  void* stream = nullptr;  // the handle's own stream: graphs need a created stream
  float* d_t = nullptr;    // device timesteps [kMaxBatch] (one slot per sample)
  float* h_t = nullptr;    // pinned host staging of the same
  int H = 128, W = 128, ctx_len = 77;
  // stage-hook adapter state (NCHW copies handed to a reference-style hook)
  UnetStageHookFn hook = nullptr;
  int B = 0;
  void* tmp = nullptr;
  size_t tmp_bytes = 0;

  ~Handle() {
    net.reset();
    if (tmp) (void)dlm_free(tmp);
    if (d_t) (void)dlm_free(d_t);
    if (h_t) (void)dlm_host_free_pinned(h_t);
    if (stream) {
      (void)dlm_scratch_release(stream);
      (void)dlm_stream_destroy(stream);
    }
  }
};

Handle& handle_of(UnetWeightsHandle h) {
  if (!h) throw std::invalid_argument("UNet handle is null");
  return *static_cast<Handle*>(h);
}

size_t dim_of(const SafeTensors& st, const std::string& name, size_t i) {
  if (!st.contains(name)) throw std::runtime_error("unet_weights_create: missing '" + name + "'");
  const auto& s = st.shape(name);
  if (s.size() <= i) throw std::runtime_error("unet_weights_create: '" + name + "' has too few dimensions");
  return s[i];
}

int count_blocks(const SafeTensors& st, const std::string& prefix) {
  int n = 0;
  while (st.contains(prefix + std::to_string(n) + ".norm1.weight")) ++n;
  return n;
}

// Channels-last stage -> NCHW copy -> the reference-style hook (test only:
// the copy buffer grows by allocation).
void stage_adapter(const char* name, const void* dptr, size_t n, int C, void* user) {
  Handle& h = *static_cast<Handle*>(user);
  if (!h.hook) return;
  const std::string nm(name);
  if (nm == "temb") {  // [B, time_dim]: the reference's "temb_final"
    h.hook("temb_final", dptr, n);
    return;
  }
  if (nm == "noise_pred") {  // already NCHW
    h.hook(name, dptr, n);
    return;
  }
  if (n * 2 > h.tmp_bytes) {
    if (h.tmp) DLM_CALL(dlm_free(h.tmp));
    h.tmp = nullptr;
    h.tmp_bytes = 0;
    DLM_CALL(dlm_malloc(&h.tmp, n * 2));
    h.tmp_bytes = n * 2;
  }
  const int HW = (int)(n / ((size_t)h.B * C));
  DLM_CALL(dlm_nhwc_to_nchw_fp16(dptr, h.tmp, h.B, C, HW, C, h.stream));
  DLM_CALL(dlm_stream_synchronize(h.stream));
  h.hook(name, h.tmp, n);
}

void run(Handle& h, int B, const void* latent, float timestep, const void* ehs, const void* text,
         const void* time_ids, void* out) {
  if (B < 1 || B > kMaxBatch) throw std::invalid_argument("launch_unet_batched: B must be in [1, 16]");
  if (!latent || !ehs || !text || !time_ids || !out) throw std::invalid_argument("launch_unet: null pointer");
  // the caller's earlier default-stream work (input copies) is done before
  // the handle's stream reads the inputs
  DLM_CALL(dlm_stream_synchronize(nullptr));
  for (int b = 0; b < B; ++b) h.h_t[b] = timestep;
  DLM_CALL(dlm_memcpy_async(h.d_t, h.h_t, (size_t)B * sizeof(float), 0, h.stream));
  h.hook = current_hook();
  h.B = B;
  h.net->set_stage_hook(h.hook ? stage_adapter : nullptr, &h);
  h.net->forward(B, h.H, h.W, latent, h.d_t, ehs, h.ctx_len, text, time_ids, 0, out, h.stream);
  DLM_CALL(dlm_stream_synchronize(h.stream));
}

}  // namespace

UNetConfig unet_config_from_weights(const SafeTensors& st) {
  UNetConfig c;
  c.C0 = (int)dim_of(st, "conv_in.weight", 0);
  c.in_channels = (int)dim_of(st, "conv_in.weight", 1);
  c.out_channels = (int)dim_of(st, "conv_out.weight", 0);
  c.C1 = (int)dim_of(st, "down_blocks.1.resnets.0.conv1.weight", 0);
  c.C2 = (int)dim_of(st, "down_blocks.2.resnets.0.conv1.weight", 0);
  c.depth1 = count_blocks(st, "down_blocks.1.attentions.0.transformer_blocks.");
  c.depth2 = count_blocks(st, "down_blocks.2.attentions.0.transformer_blocks.");
  c.cross_dim = (int)dim_of(st, "down_blocks.1.attentions.0.transformer_blocks.0.attn2.to_k.weight", 1);
  c.id_dim = 256;  // addition_time_embed_dim of SDXL (the reference's fixed 6 x 256)
  c.text_dim = (int)dim_of(st, "add_embedding.linear_1.weight", 1) - 6 * c.id_dim;
  if (c.depth1 <= 0 || c.depth2 <= 0 || c.text_dim <= 0)
    throw std::runtime_error("unet_weights_create: the tensors do not describe an SDXL-topology UNet");
  return c;
}

UnetWeightsHandle unet_weights_create(const SafeTensors& weights) {
  return unet_weights_create(weights, unet_config_from_weights(weights));
}

UnetWeightsHandle unet_weights_create(const SafeTensors& weights, const UNetConfig& cfg) {
  auto h = std::make_unique<Handle>();
  h->net = std::make_unique<UNet>(cfg);
  DLM_CALL(dlm_stream_create(&h->stream));
  void* p = nullptr;
  DLM_CALL(dlm_malloc(&p, kMaxBatch * sizeof(float)));
  h->d_t = static_cast<float*>(p);
  DLM_CALL(dlm_host_malloc_pinned(&p, kMaxBatch * sizeof(float)));
  h->h_t = static_cast<float*>(p);
  load_unet_safetensors(*h->net, weights, h->stream);
  return h.release();
}

void unet_weights_destroy(UnetWeightsHandle handle) { delete static_cast<Handle*>(handle); }

void unet_apply_loras(UnetWeightsHandle handle, const LoraModule* mods, int n) {
  Handle& h = handle_of(handle);
  if (n > 0 && !mods) throw std::invalid_argument("unet_apply_loras: null module array");
  for (int i = 0; i < n; ++i) unet_apply_lora_module(*h.net, mods[i], h.stream);
}

void unet_clear_loras(UnetWeightsHandle handle) {
  Handle& h = handle_of(handle);
  h.net->clear_loras(h.stream);
}

std::vector<uint16_t> unet_read_weight(UnetWeightsHandle handle, const std::string& name) {
  Handle& h = handle_of(handle);
  for (const WeightSpec& s : unet_weight_specs(h.net->config())) {
    if (s.name != name) continue;
    size_t n = 1;
    for (int64_t d : s.shape) n *= (size_t)d;
    std::vector<uint16_t> out(n);
    h.net->read_weight(name, out.data(), n * 2, h.stream);
    return out;
  }
  throw std::runtime_error("unet_read_weight: no weight named '" + name + "'");
}

void launch_unet(UnetWeightsHandle handle, const void* d_latent, float timestep,
                 const void* d_encoder_hidden_states, const void* d_text_embeds,
                 const void* d_time_ids, void* d_noise_pred_out, bool /*attn_fast*/,
                 bool /*epilogue*/) {
  run(handle_of(handle), 1, d_latent, timestep, d_encoder_hidden_states, d_text_embeds, d_time_ids,
      d_noise_pred_out);
}

void launch_unet_batched(UnetWeightsHandle handle, int B, const void* d_latent, float timestep,
                         const void* d_encoder_hidden_states, const void* d_text_embeds,
                         const void* d_time_ids, void* d_noise_pred_out, bool /*attn_fast*/,
                         bool /*epilogue*/) {
  run(handle_of(handle), B, d_latent, timestep, d_encoder_hidden_states, d_text_embeds, d_time_ids,
      d_noise_pred_out);
}

void launch_unet(const SafeTensors& weights, const void* d_latent, float timestep,
                 const void* d_encoder_hidden_states, const void* d_text_embeds,
                 const void* d_time_ids, void* d_noise_pred_out, bool attn_fast, bool epilogue) {
  std::unique_ptr<Handle> h(static_cast<Handle*>(unet_weights_create(weights)));
  launch_unet(h.get(), d_latent, timestep, d_encoder_hidden_states, d_text_embeds, d_time_ids,
              d_noise_pred_out, attn_fast, epilogue);
}

void unet_set_stage_hook(UnetStageHookFn hook) {
  std::lock_guard<std::mutex> lk(g_hook_mu);
  g_hook = hook;
}

void unet_set_geometry(UnetWeightsHandle handle, int latent_h, int latent_w, int ctx_len) {
  Handle& h = handle_of(handle);
  if (latent_h <= 0 || latent_w <= 0 || latent_h % 4 || latent_w % 4 || ctx_len <= 0)
    throw std::invalid_argument("unet_set_geometry: H, W positive multiples of 4 and ctx_len > 0");
  h.H = latent_h;
  h.W = latent_w;
  h.ctx_len = ctx_len;
}

void unet_set_graphs(UnetWeightsHandle handle, bool on) { handle_of(handle).net->set_graphs(on); }

UNet& unet_model(UnetWeightsHandle handle) { return *handle_of(handle).net; }

}  // namespace dollama
