"""fp32 torch-CPU restatement of the SDXL AutoencoderKL decoder (test oracle
only).

Follows the reference's decoder as a structural spec
(src/kernels/vae_decode.cuh:20-48, vae_decode.cu:699-875):
post_quant_conv 1x1 (:721-724) -> conv_in 3x3 (:727-728) -> mid block
resnet / attention / resnet (:733-753) -> up blocks 0..3, each `layers`
resnets and, for blocks 0..2, nearest-2x upsample + 3x3 conv (:756-842) ->
conv_norm_out GroupNorm(32, eps 1e-6) + SiLU -> conv_out 3x3 (:845-869).
ResnetBlock2D: vae_decode.cu:608-652; AttnBlock: :654-692 (one head over
all h*w pixels, scale 1/sqrt(C)).  The whole graph runs in fp32 (the
reference keeps fp16 activations up to up block 1; the oracle does not
round them).  Parameter names are diffusers' (the reference reads them by
name); the list below is written independently of the GPU driver's own
list, and the tests compare the two.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import ref_ops as R

EPS = 1e-6
GROUPS = 32


@dataclass(frozen=True)
class VaeCfg:
    ch: Tuple[int, int, int, int] = (128, 256, 512, 512)
    latent_channels: int = 4
    out_channels: int = 3
    layers: int = 3


SDXL_VAE = VaeCfg()
# small channel counts, same topology (shortcut in the last two blocks)
TINY_VAE = VaeCfg(ch=(64, 128, 192, 192))


def decoder_channels(cfg: VaeCfg):
    """Output channels of decoder up blocks 0..3 (block_out_channels reversed)."""
    return list(reversed(cfg.ch))


def param_shapes(cfg: VaeCfg) -> dict:
    """name -> shape for every parameter the decoder reads."""
    P = {}
    L = cfg.latent_channels
    dec = decoder_channels(cfg)
    mid = dec[0]

    def conv(name, o, i, k):
        P[name + ".weight"] = (o, i, k, k)
        P[name + ".bias"] = (o,)

    def norm(name, c):
        P[name + ".weight"] = (c,)
        P[name + ".bias"] = (c,)

    def resnet(p, i, o):
        norm(p + "norm1", i)
        conv(p + "conv1", o, i, 3)
        norm(p + "norm2", o)
        conv(p + "conv2", o, o, 3)
        if i != o:
            conv(p + "conv_shortcut", o, i, 1)

    conv("post_quant_conv", L, L, 1)
    conv("decoder.conv_in", mid, L, 3)
    resnet("decoder.mid_block.resnets.0.", mid, mid)
    a = "decoder.mid_block.attentions.0."
    norm(a + "group_norm", mid)
    for n in ("to_q", "to_k", "to_v", "to_out.0"):
        P[a + n + ".weight"] = (mid, mid)
        P[a + n + ".bias"] = (mid,)
    resnet("decoder.mid_block.resnets.1.", mid, mid)
    cin = mid
    for b, co in enumerate(dec):
        for r in range(cfg.layers):
            resnet(f"decoder.up_blocks.{b}.resnets.{r}.", cin if r == 0 else co, co)
        if b < 3:
            conv(f"decoder.up_blocks.{b}.upsamplers.0.conv", co, co, 3)
        cin = co
    norm("decoder.conv_norm_out", dec[3])
    conv("decoder.conv_out", cfg.out_channels, dec[3], 3)
    return P


def random_weights(cfg: VaeCfg, seed: int) -> dict:
    """fp32 CPU weights on the fp16 grid: conv / linear weights ~N(0, 1/fan_in),
    biases ~N(0, 0.02^2), norm scales 1 + N(0, 0.02^2), shifts N(0, 0.02^2)."""
    g = torch.Generator().manual_seed(seed)
    W = {}
    for name, shape in param_shapes(cfg).items():
        x = torch.randn(shape, generator=g, dtype=torch.float32)
        if len(shape) >= 2:
            fan_in = 1
            for d in shape[1:]:
                fan_in *= d
            x = x / fan_in ** 0.5
        else:
            x = x * 0.02
            if "norm" in name.split(".")[-2] and name.endswith(".weight"):
                x = x + 1.0
        W[name] = x.to(torch.float16).to(torch.float32)
    return W


def resnet_block(w, p, x):
    """ResnetBlock2D without time embedding (src/kernels/vae_decode.cu:608-652)."""
    h = R.silu(R.group_norm(x, GROUPS, w[p + "norm1.weight"], w[p + "norm1.bias"], EPS))
    h = R.conv2d(h, w[p + "conv1.weight"], w[p + "conv1.bias"], 1, 1)
    h = R.silu(R.group_norm(h, GROUPS, w[p + "norm2.weight"], w[p + "norm2.bias"], EPS))
    h = R.conv2d(h, w[p + "conv2.weight"], w[p + "conv2.bias"], 1, 1)
    if p + "conv_shortcut.weight" in w:
        x = R.conv2d(x, w[p + "conv_shortcut.weight"], w[p + "conv_shortcut.bias"], 1, 0)
    return x + h


def attn_block(w, p, x):
    """Single-head spatial self-attention (src/kernels/vae_decode.cu:654-692)."""
    N, C, H, W = x.shape
    h = R.group_norm(x, GROUPS, w[p + "group_norm.weight"], w[p + "group_norm.bias"], EPS)
    h = h.reshape(N, C, H * W).transpose(1, 2)  # [N, S, C]
    q = R.linear(h, w[p + "to_q.weight"], w[p + "to_q.bias"])
    k = R.linear(h, w[p + "to_k.weight"], w[p + "to_k.bias"])
    v = R.linear(h, w[p + "to_v.weight"], w[p + "to_v.bias"])
    o = R.attention(q[:, None], k[:, None], v[:, None], 1.0 / C ** 0.5)[:, 0]
    o = R.linear(o, w[p + "to_out.0.weight"], w[p + "to_out.0.bias"])
    return x + o.transpose(1, 2).reshape(N, C, H, W)


def vae_decode(w, cfg: VaeCfg, latent, stages: Optional[dict] = None):
    """image [N, out, 8h, 8w] from latent [N, L, h, w] (already divided by the
    scaling factor), fp32.  `stages` (if given) receives the reference's
    golden stage tensors by name."""
    def keep(name, t):
        if stages is not None:
            stages[name] = t

    x = R.conv2d(latent, w["post_quant_conv.weight"], w["post_quant_conv.bias"], 1, 0)
    keep("post_quant_conv_out", x)
    x = R.conv2d(x, w["decoder.conv_in.weight"], w["decoder.conv_in.bias"], 1, 1)
    keep("conv_in_out", x)
    x = resnet_block(w, "decoder.mid_block.resnets.0.", x)
    x = attn_block(w, "decoder.mid_block.attentions.0.", x)
    x = resnet_block(w, "decoder.mid_block.resnets.1.", x)
    keep("mid_block_out", x)
    for b in range(4):
        for r in range(cfg.layers):
            x = resnet_block(w, f"decoder.up_blocks.{b}.resnets.{r}.", x)
        if b < 3:
            p = f"decoder.up_blocks.{b}.upsamplers.0.conv"
            x = R.conv2d(R.upsample_nearest2x(x), w[p + ".weight"], w[p + ".bias"], 1, 1)
        keep(f"up_block_{b}_out", x)
    x = R.silu(R.group_norm(x, GROUPS, w["decoder.conv_norm_out.weight"],
                            w["decoder.conv_norm_out.bias"], EPS))
    x = R.conv2d(x, w["decoder.conv_out.weight"], w["decoder.conv_out.bias"], 1, 1)
    keep("final_image", x)
    return x


def image_to_rgb8(img):
    """[N, 3, H, W] in [-1, 1] -> uint8 [N, H, W, 3]: q = int(clamp(v/2 + 1/2, 0, 1)
    * 255 + 0.5) (src/infer/diffusion.cu:146-165)."""
    n01 = (img.float() * 0.5 + 0.5).clamp(0.0, 1.0)
    q = torch.floor(n01 * 255.0 + 0.5).to(torch.int32).clamp(0, 255)
    return q.to(torch.uint8).permute(0, 2, 3, 1).contiguous()
