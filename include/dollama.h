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

/* One block of the prepared model on its own, for block-level tests and
 * timing (the reference's resnet_block / transformer_block,
 * src/infer/unet.cu:537-797, are file-local; these run the same code the
 * forward runs for that block).
 *   dlm_unet_run_resnet: prefix e.g. "down_blocks.1.resnets.0"; input
 *   channels-last concat(xa [B,H,W,Ca], xb [B,H,W,Cb]) (xb NULL when Cb = 0);
 *   temb [B, time_dim] fp16 before the SiLU (the time MLP's output; SiLU and
 *   the block's time_emb_proj are applied inside); out [B,H,W,Co].
 *   dlm_unet_run_transformer_block: prefix e.g.
 *   "down_blocks.1.attentions.0.transformer_blocks.0"; x [B*HW, C] updated in
 *   place; ehs [B, ctx_len, cross_dim] (the block's cross K / V projections
 *   run inside).
 * An unknown prefix is DLM_ERR_NOT_FOUND. */
int dlm_unet_run_resnet(void* handle, const char* prefix, const void* xa, int Ca, const void* xb,
                        int Cb, void* out, int B, int H, int W, const void* temb, void* stream);
int dlm_unet_run_transformer_block(void* handle, const char* prefix, void* x, int B, int HW,
                                   const void* ehs, int ctx_len, void* stream);

/* Runtime LoRA (reference src/infer/unet.cuh:97-114, unet.cu:373-458):
 * W += scale * (B @ A) on the resident weight named base_key (diffusers
 * name), A device fp16 [rank, in_flat], B device fp16 [out_dim, rank]
 * (out_dim * in_flat = the weight's element count; 4-D conv weights are
 * flattened as [Cout, Cin*KH*KW]).  The delta is rounded to fp16 before the
 * add, as in the reference.  Synchronises the stream. */
int dlm_unet_apply_lora(void* handle, const char* base_key, const void* A, const void* B, int rank,
                        int in_flat, int out_dim, float scale, void* stream);
/* Load a kohya-named LoRA safetensors file (lora_unet_<flat>.lora_down /
 * .lora_up / .alpha; reference src/infer/lora.hpp:265-445) and apply every
 * UNet module with scale = strength * alpha / rank.  counts (may be NULL)
 * receives modules applied, text-encoder modules skipped, keys not
 * understood, modules missing a half.  A module that matches no UNet weight
 * is an error (DLM_ERR_STATE) and nothing after it is applied. */
int dlm_unet_load_lora(void* handle, const char* path, float strength, int* counts /* [4] */,
                       void* stream);
/* Restore every weight patched since the last clear, bit-exactly. */
int dlm_unet_clear_loras(void* handle, void* stream);
/* Host only: resolve a LoRA file against the weight list of cfg without
 * touching a device (reference load_lora_modules, src/infer/lora.hpp:265-445;
 * same counts as dlm_unet_load_lora); fails like it on an unresolvable
 * module.  fn (may be NULL) is called once per module that would be applied. */
typedef void (*dlm_lora_module_fn)(const char* base_key, int rank, int in_flat, int out_dim,
                                   float scale, void* user);
int dlm_lora_scan(const dlm_unet_config* cfg, const char* path, float strength,
                  int* counts /* [4] */, dlm_lora_module_fn fn, void* user);
/* Copy a resident weight back to host memory as fp16 in its diffusers
 * layout (reference unet_weight_device_ptr, src/infer/unet.cuh:114, the
 * accessor its LoRA tests read weights through); bytes = 2 * numel. */
int dlm_unet_read_weight(void* handle, const char* name, void* host_out, size_t bytes,
                         void* stream);
/* Host only: fp32 -> fp16 bits with round-to-nearest-even (the conversion
 * the LoRA loader applies to F32 tensors). */
int dlm_f32_to_f16(const float* in, uint16_t* out, size_t n);

/* Stage hook for tests (src/infer/unet.cuh:53-54): called after the stream
 * is synchronised with (name, device pointer, element count, channel count);
 * activations are channels-last [B, H, W, C] except noise_pred (NCHW). */
typedef void (*dlm_unet_stage_hook)(const char* name, const void* dptr, size_t n, int C,
                                    void* user);
int dlm_unet_set_stage_hook(void* handle, dlm_unet_stage_hook hook, void* user);

/* HIP-graph replay of the forward (the reference's CUDA-graph mode,
 * FastConfig::graphs).  With graphs on, a forward on a created stream whose
 * arguments and arena state equal an earlier forward's replays that
 * forward's captured graph: the first such call runs eagerly, the second is
 * captured and launched, later ones launch (about 850 kernels per SDXL
 * step in one hipGraphLaunch).  Results equal the eager forward's bit for
 * bit.  Inactive on the null stream, with a stage hook or with profiling;
 * dlm_unet_prepare drops the captured graphs.  The denoise loop passes the
 * same arguments every step, so one graph serves the whole loop. */
int dlm_unet_set_graphs(void* handle, int on);
int dlm_unet_graphs_captured(void* handle, size_t* count);

/* Which of the transformer blocks' LayerNorms are folded into the linears
 * that consume them (see dlm_linear_ln_fp16), as a bit mask in [0, 3]: bit 0
 * norm1 -> fused QKV, bit 1 norm2 -> cross-attention Q (3, both, is the
 * default); an unfolded LayerNorm, and norm3 always, runs as its own launch.
 * No counterpart in the reference (its forward is the unfolded one; the
 * folded form computes the same function).  The folded weight copies are
 * kept in step with LoRA patches and their removal. */
int dlm_unet_set_ln_fold(void* handle, int mask);

/* GroupNorm statistics from the producers (on = 1, the default): a conv
 * whose output feeds a GroupNorm directly writes that GroupNorm's chunk
 * statistics from its epilogue (dlm_conv_nhwc_args::gn_stats) and the
 * GroupNorm runs no statistics pass; on = 0 runs the pass everywhere.  The
 * output is the same bit for bit.  No counterpart in the reference. */
int dlm_unet_set_gn_fold(void* handle, int on);

/* Per-launch kernel timing (device events around every launch of a
 * forward).  Classes: 0 conv, 1 linear, 2 attention, 3 groupnorm,
 * 4 layernorm, 5 other.  report fills, per class, out[4*c + 0..3] =
 * launches, summed kernel ms, algorithmic FLOPs, algorithmic bytes of the
 * last forward run with profiling on.  Synchronises the stream. */
int dlm_unet_set_profiling(void* handle, int on);
int dlm_unet_profile_report(void* handle, double* out /* [24] */, void* stream);
/* The last profiled forward grouped by kernel (the instantiation each launch
 * ran last, dlm_last_kernel): one line per kernel, tab-separated
 * "name class launches ms flops bytes dims", dims = "M,N,K,flags:launches;"
 * for each GEMM problem the kernel ran (dlm_last_kernel_dims), in
 * first-launch order.  *needed
 * receives the text size including the terminating zero; buf (len bytes)
 * may be NULL to query it. */
int dlm_unet_profile_kernels(void* handle, char* buf, size_t len, size_t* needed, void* stream);

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

/* ------------------------------------------------------------------ */
/* SDXL VAE decoder (AutoencoderKL decoder + post_quant_conv)          */
/* ------------------------------------------------------------------ */

typedef struct dlm_vae_config {
  int ch[4];            /* block_out_channels, encoder order (SDXL 128, 256, 512, 512) */
  int latent_channels;  /* 4 */
  int out_channels;     /* 3 */
  int layers;           /* resnets per decoder up block (3) */
  int groups;           /* GroupNorm groups (32) */
  int fp32_from;        /* decoder up blocks >= this keep fp32 activations (2) */
} dlm_vae_config;

int dlm_vae_config_sdxl(dlm_vae_config* cfg);
int dlm_vae_weight_count(const dlm_vae_config* cfg, int* count);
int dlm_vae_weight_spec(const dlm_vae_config* cfg, int index, char* name, int name_len,
                        int* ndim, int64_t* shape /* [4] */);

/* Resident weight handle (replaces vae_weights_create / vae_weights_destroy,
 * src/kernels/vae_decode.cuh:59-69): set_weight registers fp16 device
 * buffers (decoder.* and post_quant_conv.* diffusers names, borrowed until
 * prepare), prepare packs them into the handle's own memory. */
int dlm_vae_create(const dlm_vae_config* cfg, void** handle);
int dlm_vae_destroy(void* handle);
int dlm_vae_set_weight(void* handle, const char* name, const void* dptr, int ndim,
                       const int64_t* shape);
int dlm_vae_load_safetensors(void* handle, const char* path, void* stream);
int dlm_vae_prepare(void* handle, void* stream);
int dlm_vae_packed_bytes(void* handle, size_t* bytes);

/* image [N, out_channels, 8h, 8w] fp16 NCHW (values in about [-1, 1]) from
 * latent [N, latent_channels, h, w] fp16 NCHW already divided by the scaling
 * factor (dlm_latent_to_vae_fp16); h * w a multiple of 8, 1 <= N <= 16.
 * Replaces launch_vae_decode(handle, d_latent, d_image_out)
 * (src/kernels/vae_decode.cuh:71-75), which decodes one 128x128 latent and
 * synchronises; this call is stream-ordered. */
int dlm_vae_decode(void* handle, int N, int h, int w, const void* latent, void* image,
                   void* stream);

/* Stage hook for tests (the reference's golden stages, src/tests/
 * test_vae_decode.cu): post_quant_conv_out (64 channels, the last 60 zero),
 * conv_in_out, mid_block_out, up_block_{0..3}_out (channels-last, fp32
 * when is_f32), final_image (NCHW fp16). */
typedef void (*dlm_vae_stage_hook)(const char* name, const void* dptr, size_t n, int C,
                                   int is_f32, void* user);
int dlm_vae_set_stage_hook(void* handle, dlm_vae_stage_hook hook, void* user);
/* Kernel timing by class: 0 conv, 1 linear, 2 attention, 3 groupnorm,
 * 4 other; out[4*c + 0..3] as dlm_unet_profile_report. */
int dlm_vae_set_profiling(void* handle, int on);
int dlm_vae_profile_report(void* handle, double* out /* [20] */, void* stream);

/* ------------------------------------------------------------------ */
/* Text-to-image runner and backend plugin                             */
/* ------------------------------------------------------------------ */

/* IDiffusionRunner over the device pipeline (reference make_diffusion_runner
 * + DiffusionRunner, src/server/diffusion_runner.hpp:33-79 and
 * diffusion_runner.cu:33-160).  Loads the UNet and VAE safetensors (diffusers
 * keys) and the embeddings file (input_encoder_hidden_states_f16,
 * input_text_embeds_f16, input_time_ids_f16; src/infer/diffusion.cu:305-312).
 * ucfg / vcfg NULL = SDXL; latent 128 x 128 = a 1024 x 1024 image.  Where the
 * reference returns nullptr (unreadable file, failed construction) this
 * returns a non-zero status and *handle = NULL.  An invalid
 * vae_scaling_factor (<= 0 or not finite) falls back to 0.13025. */
int dlm_runner_create(const char* unet_weights, const char* vae_weights, const char* embeds,
                      float vae_scaling_factor, const dlm_unet_config* ucfg,
                      const dlm_vae_config* vcfg, int latent_h, int latent_w, void** handle);
int dlm_runner_destroy(void* handle);
/* run_txt2img: CFG with guidance, host fp32 conditioning (ehs [ctx_len *
 * cross_dim], text [text_dim], time_ids [6]); the seed gives the reference's
 * initial latent (dlm_randn_latent); rgb_out receives [h, w, 3] bytes
 * (rgb_capacity >= 3 * w * h). */
int dlm_runner_txt2img(void* handle, int steps, uint64_t seed, float guidance,
                       const float* cond_ehs, const float* cond_text, const float* uncond_ehs,
                       const float* uncond_text, const float* time_ids, uint8_t* rgb_out,
                       size_t rgb_capacity, int* w, int* h);
/* DiffusionPipeline::generate (guidance 1, conditioning from the embeddings
 * file, B=1 forwards; src/infer/diffusion.cu:551-700). */
int dlm_runner_generate(void* handle, int steps, uint64_t seed, uint8_t* rgb_out,
                        size_t rgb_capacity, int* w, int* h);
/* Apply LoRA files in order; on any failure every LoRA is cleared and the
 * error returned (reference DiffusionRunner::apply_loras). */
int dlm_runner_apply_loras(void* handle, const char* const* paths, const float* strengths, int n);
int dlm_runner_clear_loras(void* handle);

/* IDiffusionBackend registry (reference make_backend,
 * src/server/diffusion_backend.cpp): backend_name "sdxl" builds the SDXL
 * backend; any other name, or a failed construction, returns
 * DLM_ERR_NOT_FOUND with *handle = NULL.  The "sdxl" backend here takes its
 * conditioning from the embeddings file (cond tensors as above, optional
 * uncond_encoder_hidden_states_f16 / uncond_text_embeds_f16, zero when
 * absent) instead of the reference's CLIP text encoders; generate() does not
 * read the prompt strings, defaults steps <= 0 to 20 and cfg <= 0 to 7.5, and
 * returns the native resolution (8 * latent_size). */
typedef struct dlm_backend_config {
  const char* backend_name;
  const char* preset;
  const char* unet_weights;
  const char* vae_weights;
  const char* embeds;
  float vae_scaling_factor;
  const dlm_unet_config* unet_cfg; /* NULL = SDXL */
  const dlm_vae_config* vae_cfg;   /* NULL = SDXL */
  int latent_size;                 /* <= 0: 128 */
} dlm_backend_config;
int dlm_backend_create(const dlm_backend_config* cfg, void** handle);
int dlm_backend_destroy(void* handle);
int dlm_backend_generate(void* handle, const char* prompt, const char* negative, int steps,
                         uint64_t seed, float cfg, int w, int h, uint8_t* rgb_out,
                         size_t rgb_capacity, int* w_out, int* h_out);
int dlm_backend_info(void* handle, char* name, int name_len, int* latent_channels,
                     int* native_resolution, int* needs_t5);
/* "sdxl-1.0" or "sdxl-1.0/<preset>" (reference compose_model_id). */
int dlm_backend_model_id(void* handle, char* buf, int len);
/* LoRA names resolve to $DOLLAMA_LORA_DIR (default models/loras)/<name>.safetensors;
 * names hold [A-Za-z0-9_.-] and do not start with '.'. */
int dlm_backend_apply_loras(void* handle, const char* const* names, const float* strengths, int n);
int dlm_backend_clear_loras(void* handle);

/* Host only: out[k] = float(z_k * sigma0), z the reference's seeded normal
 * stream (xorshift128+ seeded by splitmix64, Box-Muller;
 * src/infer/diffusion.cu:80-136, :828-835). */
int dlm_randn_latent(uint64_t seed, double sigma0, float* out, size_t n);

/* ------------------------------------------------------------------ */
/* safetensors reader (host)                                           */
/* ------------------------------------------------------------------ */

/* Memory-mapped read-only safetensors file (reference SafeTensors,
 * src/io/safetensors.hpp:108: names / dtype / shape / tensor_bytes).  A
 * missing file, a header length beyond the file or malformed JSON fails at
 * open; an unknown name is DLM_ERR_NOT_FOUND.  dtype codes: 0 F64, 1 F32,
 * 2 F16, 3 BF16, 4 I64, 5 I32, 6 I16, 7 I8, 8 U8, 9 BOOL, 10 other.
 * __metadata__ is not a tensor. */
int dlm_st_open(const char* path, void** handle);
int dlm_st_close(void* handle);
int dlm_st_count(void* handle, int* count);
int dlm_st_name(void* handle, int index, char* buf, int len);
int dlm_st_info(void* handle, const char* name, int* dtype, int* ndim, int64_t* shape /* [8] */,
                size_t* nbytes);
int dlm_st_read(void* handle, const char* name, void* out, size_t bytes);

/* VRAM arena statistics (src/kernels/device_arena.cuh DeviceArenaStats):
 * out[0..10] = cuda_malloc_calls, cuda_free_calls, chunk_alloc_calls,
 * alloc_calls, total_capacity, live_chunks, bytes_in_use, peak_bytes_in_use,
 * live_request_bytes, peak_request_bytes, reserved_bytes. */
int dlm_arena_stats(int arena_id, uint64_t* out /* [11] */);
int dlm_arena_release(int arena_id);
int dlm_arena_reserve(int arena_id, size_t bytes);
/* Fill all memory the arena holds with the byte `pattern` (synchronous);
 * DLM_ERR_STATE-class failure while allocations are live.  Test support for
 * the reference's poisoned-arena determinism gate
 * (src/tests/test_unet_fast.cu:136-172): a forward that reads scratch before
 * writing it gives different results after fills with different patterns. */
int dlm_arena_fill(int arena_id, int pattern);

#ifdef __cplusplus
}
#endif

#endif /* DOLLAMA_H */
