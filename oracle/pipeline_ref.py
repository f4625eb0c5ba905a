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

The per-step pieces (scale_model_input, cfg_combine, euler_step) are
separate functions so the tests can pin each one: the first and last
against the reference's own scheduler header compiled on the CPU, the CFG
combine and its slot order against a stub noise predictor.
"""
from __future__ import annotations

import math

import torch

from . import naive
from . import noise_ref as NR
from . import unet_ref as OR
from . import vae_ref as OV


def scale_model_input(sample, sigma):
    """sample / sqrt(sigma^2 + 1) (src/infer/scheduler.hpp:112-120)."""
    return sample / math.sqrt(float(sigma) ** 2 + 1.0)


def cfg_combine(noise, guidance):
    """Classifier-free guidance over a batch-2 prediction whose slot 0 ran on
    the cond embeddings and slot 1 on the uncond ones (the reference copies
    cond into the first half of d_ehs2 / d_txt2 and uncond into the second,
    diffusion.cu:878-883, and reads d_noise2 back the same way, :928-931):
    u + g (c - u) (:968-973)."""
    c, u = noise[0:1], noise[1:2]
    return u + guidance * (c - u)


def euler_step(sample, eps, sigma, sigma_next):
    """Euler step with an epsilon prediction: sample + eps * (sigma_next -
    sigma) (src/infer/scheduler.hpp:122-143)."""
    return sample + eps * (float(sigma_next) - float(sigma))


def denoise(unet_fn, sig, ts, lat, ehs, txt, ids, *, guidance=7.5, cfg=True):
    """The sampling loop on an fp32 latent [1, C, h, w]; unet_fn(x, t, ehs,
    txt, ids) returns the noise prediction for a batch (B = 2 with cond then
    uncond rows when cfg, else 1).  Returns the final latent."""
    B = 2 if cfg else 1
    for i in range(len(ts)):
        x = scale_model_input(lat, sig[i])
        t = torch.full((B,), float(ts[i]))
        out = unet_fn(x.expand(B, -1, -1, -1).contiguous(), t, ehs, txt, ids)
        eps = cfg_combine(out, guidance) if cfg else out
        lat = euler_step(lat, eps, sig[i], sig[i + 1])
    return lat


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
    ids = time_ids.reshape(6).float()

    def unet_fn(x, t, e, tx, i):
        return OR.unet_forward(unet_w, ucfg, x, t, e, tx, i)

    lat = denoise(unet_fn, sig, ts, lat, ehs, txt, ids, guidance=guidance, cfg=cfg)
    img = OV.vae_decode(vae_w, vcfg, lat / scaling_factor)
    return OV.image_to_rgb8(img), lat
