// The reference's UNet host API, with its signatures, over this library.
//
// Replaces src/infer/unet.cuh:53-146 for a caller that keeps the reference's
// DiffusionPipeline: the same names, argument order and meaning, so swapping
// the UNet is a change of include and link line.  Device pointers are fp16
// buffers in the reference's layouts (latent / noise_pred NCHW b-major,
// encoder hidden states [B, 77, 2048], text embeds [B, 1280], time ids [6]
// shared by the batch); the reference's `const __half*` / `__half*`
// arguments convert implicitly to the `const void*` / `void*` taken here.
//
// Behaviour, as the reference's:
//   - the default stream's earlier work is complete before the forward reads
//     its inputs, and the output is complete when the call returns (the
//     reference's launch_unet is followed by a blocking cudaMemcpy; here the
//     forward runs on the handle's own stream between two synchronisations);
//   - errors throw std::runtime_error (reference: CUDA_CHECK);
//   - unet_apply_loras: W += scale * (B @ A) per module, in order; a module
//     that fails leaves the ones before it applied (callers clear, then
//     retry); unet_clear_loras restores every patched weight bit-exactly.
// Differences, by design:
//   - the handle uploads and packs every weight at create time (the
//     reference uploads lazily on the first launch), so it does not borrow
//     the SafeTensors: the file may be closed after create;
//   - the host timestep goes into a device slot owned by the handle, stream
//     ordered before the forward, so a handle with graphs on replays one
//     captured graph for every step (unet_set_graphs);
//   - attn_fast / epilogue select nothing: the reference's FAST modes are
//     alternative kernels for the same function, and this library has one
//     path, always the fused one;
//   - the stage hook is called at the block boundaries the fused forward
//     materialises (temb_final, conv_in_out, down_block_{0,1,2}_out,
//     mid_block_out, up_block_{0,1,2}_out, noise_pred), each as an NCHW
//     (or [B, C] for temb_final) device copy the hook may read during the
//     call; the reference's finer stages (resnet0_out, attn0_out, ...) have no
//     buffer of their own here.
// unet_weight_device_ptr (reference: a device pointer into the resident
// diffusers-layout weight) has no counterpart: weights are resident in packed
// forms (fused q/k/v, GEGLU interleave, per-tap channels-last convs);
// unet_read_weight copies one back to host memory in its diffusers layout.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "lora.hpp"
#include "safetensors.hpp"
#include "unet.hpp"

namespace dollama {

using UnetWeightsHandle = void*;

// Resident weight handle from a diffusers-named fp16 safetensors file
// (reference unet_weights_create, src/infer/unet.cuh:90).  The configuration
// is read from the tensors' shapes (channel widths, transformer depths,
// cross-attention width, in / out channels); the time-id sinusoid width is
// SDXL's 256.  Latent 128 x 128 and 77 context tokens until
// unet_set_geometry says otherwise.
UnetWeightsHandle unet_weights_create(const SafeTensors& weights);
// Same, with an explicit configuration (any UNetConfig this library runs).
UnetWeightsHandle unet_weights_create(const SafeTensors& weights, const UNetConfig& cfg);
// Frees every device buffer of the handle; nullptr is ignored
// (reference unet_weights_destroy, :93).
void unet_weights_destroy(UnetWeightsHandle handle);

// Runtime LoRA (reference unet_apply_loras / unet_clear_loras, :106-111).
void unet_apply_loras(UnetWeightsHandle handle, const LoraModule* mods, int n);
void unet_clear_loras(UnetWeightsHandle handle);
// Host copy of a resident weight in its diffusers layout, fp16 bits.
std::vector<uint16_t> unet_read_weight(UnetWeightsHandle handle, const std::string& name);

// One forward, B = 1 (reference launch_unet(handle, ...), :119-127).
void launch_unet(UnetWeightsHandle handle, const void* d_latent, float timestep,
                 const void* d_encoder_hidden_states, const void* d_text_embeds,
                 const void* d_time_ids, void* d_noise_pred_out, bool attn_fast = false,
                 bool epilogue = false);
// One forward over B b-major samples sharing timestep and time ids
// (reference launch_unet_batched, :137-146); 1 <= B <= 16.
void launch_unet_batched(UnetWeightsHandle handle, int B, const void* d_latent, float timestep,
                         const void* d_encoder_hidden_states, const void* d_text_embeds,
                         const void* d_time_ids, void* d_noise_pred_out, bool attn_fast = false,
                         bool epilogue = false);
// Per-call form that creates a handle from the file, runs one B = 1
// forward and destroys it (reference launch_unet(const SafeTensors&, ...),
// :63-71: it re-uploads every weight per call, as this does).
void launch_unet(const SafeTensors& weights, const void* d_latent, float timestep,
                 const void* d_encoder_hidden_states, const void* d_text_embeds,
                 const void* d_time_ids, void* d_noise_pred_out, bool attn_fast = false,
                 bool epilogue = false);

// Stage hook for tests (reference unet_set_stage_hook, :53-54): global, as
// the reference's; nullptr removes it.  A hook declared with the reference's
// `const __half*` parameter binds through the template overload.
using UnetStageHookFn = void (*)(const char* name, const void* d_buf, size_t n);
void unet_set_stage_hook(UnetStageHookFn hook);
template <class Half>
void unet_set_stage_hook(void (*hook)(const char*, const Half*, size_t)) {
  static_assert(sizeof(Half) == 2, "the stage hook receives fp16 buffers");
  unet_set_stage_hook(reinterpret_cast<UnetStageHookFn>(hook));
}

// Extensions with no reference counterpart.
// Latent size (H, W multiples of 4) and context length of later launches.
void unet_set_geometry(UnetWeightsHandle handle, int latent_h, int latent_w, int ctx_len);
// HIP-graph replay of the forward (the reference's FastConfig::graphs).
void unet_set_graphs(UnetWeightsHandle handle, bool on);
// The native model, for the C-ABI calls (profiling, block runners).
UNet& unet_model(UnetWeightsHandle handle);
// The configuration unet_weights_create(weights) reads from the shapes.
UNetConfig unet_config_from_weights(const SafeTensors& weights);

}  // namespace dollama
