/*
 * dollama.h — C ABI of the C++20 host layer (libdollama.so): the SDXL UNet
 * driver with a resident weight handle, and the VRAM arena statistics.
 *
 * Replaces the reference's UNet host API (src/infer/unet.cuh:53-146:
 * unet_weights_create / unet_weights_destroy / launch_unet_batched /
 * unet_set_stage_hook) for callers that bind through a C FFI.  Same status
 * convention as include/dlm.h (0 = DLM_OK, text in dlm_last_error()).
 */
#ifndef DOLLAMA_H
#define DOLLAMA_H

#include <stddef.h>
#include <stdint.h>

#include "dlm.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dlm_unet_config {
  int C0, C1, C2;          /* block_out_channels (SDXL 320, 640, 1280) */
  int depth1, depth2;      /* transformer depth at levels 1, 2 (SDXL 2, 10) */
  int head_dim;            /* 64 */
  int cross_dim;           /* encoder hidden width (2048) */
  int text_dim;            /* pooled text embedding width (1280) */
  int id_dim;              /* sinusoid width per time id (256) */
  int in_channels, out_channels; /* 4, 4 */
  int groups;              /* GroupNorm groups (32) */
} dlm_unet_config;

/* SDXL base configuration. */
int dlm_unet_config_sdxl(dlm_unet_config* cfg);

/* Enumerate the parameters the forward reads (diffusers key names). */
int dlm_unet_weight_count(const dlm_unet_config* cfg, int* count);
int dlm_unet_weight_spec(const dlm_unet_config* cfg, int index, char* name, int name_len,
                         int* ndim, int64_t* shape /* [4] */);

/* Resident weight handle.  set_weight registers fp16 device buffers
 * (borrowed until prepare); prepare packs them into the handle's own device
 * memory (conv weights channels-last per tap, fused q/k/v, GEGLU interleave,
 * batched time and cross-K/V projections), after which the caller may free
 * the registered buffers.  Replaces unet_weights_create / _destroy
 * (src/infer/unet.cuh:90-93). */
int dlm_unet_create(const dlm_unet_config* cfg, void** handle);
int dlm_unet_destroy(void* handle);
int dlm_unet_set_weight(void* handle, const char* name, const void* dptr, int ndim,
                        const int64_t* shape);
/* Load every fp16 tensor of a safetensors file (diffusers key names) and
 * prepare the handle from it. */
int dlm_unet_load_safetensors(void* handle, const char* path, void* stream);
int dlm_unet_prepare(void* handle, void* stream);
int dlm_unet_packed_bytes(void* handle, size_t* bytes);

/* One UNet forward, B-major, replaces launch_unet_batched
 * (src/infer/unet.cuh:137-146):
 *   latent [B, in, H, W] fp16 NCHW, timesteps device fp32 [B],
 *   ehs [B, ctx_len, cross_dim] fp16, text [B, text_dim] fp16,
 *   time_ids fp16 [6] (ids_bstride 0, shared) or [B, 6] (ids_bstride 6),
 *   out [B, out, H, W] fp16 NCHW.  H, W multiples of 4; 1 <= B <= 16. */
int dlm_unet_forward(void* handle, int B, int H, int W, const void* latent,
                     const float* timesteps, const void* ehs, int ctx_len, const void* text,
                     const void* time_ids, int ids_bstride, void* out, void* stream);

/* Stage hook for tests (src/infer/unet.cuh:53-54): called after the stream
 * is synchronised with (name, device pointer, element count, channel count);
 * activations are channels-last [B, H, W, C] except noise_pred (NCHW). */
typedef void (*dlm_unet_stage_hook)(const char* name, const void* dptr, size_t n, int C,
                                    void* user);
int dlm_unet_set_stage_hook(void* handle, dlm_unet_stage_hook hook, void* user);

/* Per-launch kernel timing (device events around every launch of a
 * forward).  Classes: 0 conv, 1 linear, 2 attention, 3 groupnorm,
 * 4 layernorm, 5 other.  report fills, per class, out[4*c + 0..3] =
 * launches, summed kernel ms, algorithmic FLOPs, algorithmic bytes of the
 * last forward run with profiling on.  Synchronises the stream. */
int dlm_unet_set_profiling(void* handle, int on);
int dlm_unet_profile_report(void* handle, double* out /* [24] */, void* stream);

/* Euler discrete scheduler (reference src/infer/scheduler.hpp:31-197:
 * scaled_linear betas 0.00085..0.012, leading spacing, steps_offset 1):
 * sigmas[steps + 1] (last = 0) and timesteps[steps], descending. */
int dlm_euler_schedule(int steps, float* sigmas, float* timesteps);

/* Full CFG denoise loop on the device (reference
 * src/infer/diffusion.cu:896-978, B=2 path): latent is device fp32
 * [in_channels, H, W] holding randn * sigmas[0] on entry and the final latent
 * on return; ehs [2, ctx_len, cross_dim] and text [2, text_dim] hold the cond
 * then uncond rows; time_ids [6] shared. */
int dlm_pipeline_denoise(void* unet, int steps, float guidance, int H, int W, float* latent,
                         const void* ehs, int ctx_len, const void* text, const void* time_ids,
                         void* stream);

/* VRAM arena statistics (src/kernels/device_arena.cuh DeviceArenaStats):
 * out[0..10] = cuda_malloc_calls, cuda_free_calls, chunk_alloc_calls,
 * alloc_calls, total_capacity, live_chunks, bytes_in_use, peak_bytes_in_use,
 * live_request_bytes, peak_request_bytes, reserved_bytes. */
int dlm_arena_stats(int arena_id, uint64_t* out /* [11] */);
int dlm_arena_release(int arena_id);
int dlm_arena_reserve(int arena_id, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* DOLLAMA_H */
