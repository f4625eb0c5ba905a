// Runtime LoRA: kohya-named LoRA tensors resolved against the UNet's
// diffusers parameter names.
//
// Same contract as the reference's loader (src/infer/lora.hpp:136-445):
//   W' = W + scale * (B @ A), scale = strength * alpha / rank, rank = A.rows;
//   A = lora_unet_<flat>.lora_down.weight [rank, in(*kh*kw)],
//   B = lora_unet_<flat>.lora_up.weight [out, rank(,1,1)],
//   alpha = lora_unet_<flat>.alpha (scalar, default rank); the fully flat
//   spellings _lora_down_weight / _lora_up_weight / _alpha are accepted too;
//   <flat> + "_weight" must equal a base key with every '.' replaced by '_'
//   (unresolvable modules are an error, never silently dropped);
//   text-encoder modules (lora_te1_*, lora_te2_*, lora_te_*) are skipped and counted; modules missing
//   their down or up half are skipped and counted; F32 tensors are rounded to
//   F16 (round to nearest even).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "safetensors.hpp"
#include "unet.hpp"

namespace dollama {

struct LoraModule {
  std::string base_key;
  std::vector<uint16_t> a_fp16;  // [rank, in_flat]
  std::vector<uint16_t> b_fp16;  // [out_dim, rank]
  int rank = 0, in_flat = 0, out_dim = 0;
  float scale = 1.0f;
};

struct LoraReport {
  size_t te_skipped = 0;
  size_t other_keys = 0;
  size_t incomplete = 0;
  size_t modules = 0;
};

std::vector<LoraModule> load_lora_modules(const std::vector<WeightSpec>& base,
                                          const SafeTensors& lora, float strength,
                                          LoraReport* report);

uint16_t f32_to_f16_rne(float v);

// Load a LoRA file and merge every UNet module into the resident weights
// (reference DiffusionPipeline::apply_lora_file, src/infer/diffusion.cu).
// Modules applied before a failing one stay applied.
void unet_apply_lora_file(UNet& u, const std::string& path, float strength, LoraReport* report,
                          void* stream);
// Merge one resolved module (W += scale * (B @ A)) into the resident weights.
void unet_apply_lora_module(UNet& u, const LoraModule& m, void* stream);

}  // namespace dollama
