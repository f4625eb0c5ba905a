// CFG denoise loop on the device.
//
// The reference runs this loop on the host (src/infer/diffusion.cu:896-978):
// per step an H2D of the scaled latent, one B=2 UNet forward, a D2H of both
// noise predictions, the CFG combine u + g (c - u) and the Euler step in host
// floats.  Here the latent stays on the device in fp32: one fused kernel does
// CFG + Euler + the next step's scale_model_input, and the per-step
// timesteps are uploaded once before the loop.  Batch layout follows the
// reference's B=2 path: slice 0 = cond, slice 1 = uncond.
#pragma once

#include "unet.hpp"

namespace dollama {

struct DenoiseArgs {
  int steps = 20;
  float guidance = 7.5f;
  int H = 128, W = 128;
  float* latent = nullptr;  // device fp32 [C, H, W]: in = randn * sigma_0, out = final latent
  const void* ehs = nullptr;       // device fp16 [2, ctx_len, cross_dim] (cond, uncond)
  int ctx_len = 77;
  const void* text = nullptr;      // device fp16 [2, text_dim]
  const void* time_ids = nullptr;  // device fp16 [6] (shared)
};

void denoise(UNet& unet, const DenoiseArgs& a, void* stream);

}  // namespace dollama
