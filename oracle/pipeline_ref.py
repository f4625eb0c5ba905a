"""fp32 CPU restatement of the text-to-image pipeline (test oracle only).

Follows the reference's DiffusionPipeline (src/infer/diffusion.cu:551-1000):
initial latent = Randn(seed) * sigma_0 (:828-835), per step
scale_model_input x / sqrt(sigma_i^2 + 1) (src/infer/scheduler.hpp:112-120),
UNet on [cond; uncond] (B=2 path, :908-955), eps = u + g (c - u) (:968-973),
Euler x += eps (sigma_{i+1} - sigma_i) (scheduler.hpp:122-143); without
guidance a B=1 UNet on the cond embeddings and eps = its prediction
(:551-700); then latent / scaling_factor -> VAE decode -> RGB8 (:980-998,
image_f16_to_rgb_u8 :146-165).  Everything in fp32 (no fp16 rounding of
the model input, the conditioning or the image).
"""
from __future__ import annotations

import math

import torch

from . import naive
from . import noise_ref as NR
from . import unet_ref as OR
from . import vae_ref as OV


def txt2img(unet_w, ucfg, vae_w, vcfg, *, seed, steps, lh, lw, cond_ehs, cond_text, time_ids,
            uncond_ehs=None, uncond_text=None, guidance=7.5, cfg=True, scaling_factor=0.13025):
    """RGB8 [1, 8 lh, 8 lw, 3] (torch uint8) and the final latent."""
    sig, ts = naive.euler_schedule(steps)
    C = ucfg.in_channels
    lat = torch.from_numpy(NR.randn_latent(seed, float(sig[0]), C * lh * lw)).float().reshape(1, C, lh, lw)
    ehs = cond_ehs.reshape(1, -1, ucfg.cross_dim).float()
    txt = cond_text.reshape(1, -1).float()
    if cfg:
        ehs = torch.cat([ehs, uncond_ehs.reshape(1, -1, ucfg.cross_dim).float()], 0)
        txt = torch.cat([txt, uncond_text.reshape(1, -1).float()], 0)
    B = 2 if cfg else 1
    ids = time_ids.reshape(6).float()
    for i in range(steps):
        x = lat / math.sqrt(float(sig[i]) ** 2 + 1.0)
        t = torch.full((B,), float(ts[i]))
        out = OR.unet_forward(unet_w, ucfg, x.expand(B, -1, -1, -1).contiguous(), t, ehs, txt, ids)
        eps = out[1:2] + guidance * (out[0:1] - out[1:2]) if cfg else out
        lat = lat + eps * (float(sig[i + 1]) - float(sig[i]))
    img = OV.vae_decode(vae_w, vcfg, lat / scaling_factor)
    return OV.image_to_rgb8(img), lat
