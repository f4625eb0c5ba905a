"""fp32 torch-CPU restatement of the SDXL UNet2DConditionModel forward
(test oracle only).

Follows the reference's UNet driver as a structural spec
(src/infer/unet.cu:537-1309): NCHW activations, resnet_block (:537-664),
transformer_block (:677-797), transformer2d (:810-858), downsample /
upsample (:863-881), the skip stack and concat order (:1035-1266),
conv_norm_out + SiLU + conv_out (:1270-1291); time / add embeddings
(:976-1031).  Parameter names are diffusers' (the reference reads them by
name).  The parameter list below is written independently of the GPU
driver's own list; the tests compare the two.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ref_ops as R


@dataclass(frozen=True)
class UNetCfg:
    C0: int = 320
    C1: int = 640
    C2: int = 1280
    depth1: int = 2
    depth2: int = 10
    head_dim: int = 64
    cross_dim: int = 2048
    text_dim: int = 1280
    id_dim: int = 256
    in_channels: int = 4
    out_channels: int = 4
    groups: int = 32

    @property
    def T(self):
        return 4 * self.C0


SDXL = UNetCfg()
# a small configuration of the same topology for fast full-graph checks
TINY = UNetCfg(C0=64, C1=128, C2=192, depth1=1, depth2=2, cross_dim=96, text_dim=64, id_dim=16)


def _level_channels(cfg):
    return [cfg.C0, cfg.C1, cfg.C2]


def param_shapes(cfg: UNetCfg) -> dict:
    """name -> shape for every parameter the forward reads."""
    P = {}
    T = cfg.T

    def lin(name, o, i, bias=True):
        P[name + ".weight"] = (o, i)
        if bias:
            P[name + ".bias"] = (o,)

    def conv(name, o, i, k):
        P[name + ".weight"] = (o, i, k, k)
        P[name + ".bias"] = (o,)

    def norm(name, c):
        P[name + ".weight"] = (c,)
        P[name + ".bias"] = (c,)

    def resnet(p, ci, co):
        norm(p + "norm1", ci)
        conv(p + "conv1", co, ci, 3)
        lin(p + "time_emb_proj", co, T)
        norm(p + "norm2", co)
        conv(p + "conv2", co, co, 3)
        if ci != co:
            conv(p + "conv_shortcut", co, ci, 1)

    def t2d(p, c, depth):
        norm(p + "norm", c)
        lin(p + "proj_in", c, c)
        for l in range(depth):
            b = f"{p}transformer_blocks.{l}."
            for n in ("norm1", "norm2", "norm3"):
                norm(b + n, c)
            for n in ("to_q", "to_k", "to_v"):
                lin(b + "attn1." + n, c, c, bias=False)
            lin(b + "attn1.to_out.0", c, c)
            lin(b + "attn2.to_q", c, c, bias=False)
            lin(b + "attn2.to_k", c, cfg.cross_dim, bias=False)
            lin(b + "attn2.to_v", c, cfg.cross_dim, bias=False)
            lin(b + "attn2.to_out.0", c, c)
            lin(b + "ff.net.0.proj", 8 * c, c)
            lin(b + "ff.net.2", c, 4 * c)
        lin(p + "proj_out", c, c)

    C = _level_channels(cfg)
    depths = [0, cfg.depth1, cfg.depth2]
    conv("conv_in", cfg.C0, cfg.in_channels, 3)
    lin("time_embedding.linear_1", T, cfg.C0)
    lin("time_embedding.linear_2", T, T)
    lin("add_embedding.linear_1", T, cfg.text_dim + 6 * cfg.id_dim)
    lin("add_embedding.linear_2", T, T)
    prev = cfg.C0
    for lv in range(3):
        for r in range(2):
            resnet(f"down_blocks.{lv}.resnets.{r}.", prev if r == 0 else C[lv], C[lv])
            if depths[lv]:
                t2d(f"down_blocks.{lv}.attentions.{r}.", C[lv], depths[lv])
        prev = C[lv]
        if lv < 2:
            conv(f"down_blocks.{lv}.downsamplers.0.conv", C[lv], C[lv], 3)
    resnet("mid_block.resnets.0.", C[2], C[2])
    t2d("mid_block.attentions.0.", C[2], cfg.depth2)
    resnet("mid_block.resnets.1.", C[2], C[2])
    # skip channels in push order: conv_in, down0 r0 r1 ds, down1 r0 r1 ds, down2 r0 r1
    skips = [C[0], C[0], C[0], C[0], C[1], C[1], C[1], C[2], C[2]]
    cur = C[2]
    for u in range(3):
        lv = 2 - u
        for r in range(3):
            sk = skips.pop()
            resnet(f"up_blocks.{u}.resnets.{r}.", cur + sk, C[lv])
            cur = C[lv]
            if depths[lv]:
                t2d(f"up_blocks.{u}.attentions.{r}.", C[lv], depths[lv])
        if u < 2:
            conv(f"up_blocks.{u}.upsamplers.0.conv", C[lv], C[lv], 3)
    norm("conv_norm_out", cfg.C0)
    conv("conv_out", cfg.out_channels, cfg.C0, 3)
    return P


def random_weights(cfg: UNetCfg, seed: int, std: float = 0.02) -> dict:
    """fp32 CPU weights on the fp16 grid: matrices / conv kernels / biases
    ~N(0, std^2); norm scales 1 + N(0, std^2), norm shifts N(0, std^2)."""
    g = torch.Generator().manual_seed(seed)
    W = {}
    for name, shape in param_shapes(cfg).items():
        x = torch.randn(shape, generator=g, dtype=torch.float32) * std
        if ("norm" in name.split(".")[-2]) and name.endswith(".weight") and len(shape) == 1:
            x = x + 1.0
        W[name] = x.to(torch.float16).to(torch.float32)
    return W


# ------------------------------------------------------------------ blocks --
def resnet_block(w, p, x, temb_silu):
    """src/infer/unet.cu:537-664."""
    h = R.silu(R.group_norm(x, 32, w[p + "norm1.weight"], w[p + "norm1.bias"], 1e-5))
    h = R.conv2d(h, w[p + "conv1.weight"], w[p + "conv1.bias"], 1, 1)
    tp = R.linear(temb_silu, w[p + "time_emb_proj.weight"], w[p + "time_emb_proj.bias"])
    h = h + tp[:, :, None, None]
    h = R.silu(R.group_norm(h, 32, w[p + "norm2.weight"], w[p + "norm2.bias"], 1e-5))
    h = R.conv2d(h, w[p + "conv2.weight"], w[p + "conv2.bias"], 1, 1)
    if p + "conv_shortcut.weight" in w:
        x = R.conv2d(x, w[p + "conv_shortcut.weight"], w[p + "conv_shortcut.bias"], 1, 0)
    return x + h


def _heads(t, heads):
    B, S, C = t.shape
    return t.reshape(B, S, heads, C // heads).permute(0, 2, 1, 3).contiguous()


def _merge(t):
    B, H, S, D = t.shape
    return t.permute(0, 2, 1, 3).reshape(B, S, H * D)


def _attn(q, k, v, heads):
    out = []
    for b in range(q.shape[0]):
        out.append(R.attention(_heads(q[b:b + 1], heads), _heads(k[b:b + 1], heads),
                               _heads(v[b:b + 1], heads), 1.0 / 8.0))
    return _merge(torch.cat(out))


def transformer_block(w, p, x, ctx, heads):
    """src/infer/unet.cu:677-797; x [B, S, C]."""
    C = x.shape[-1]
    n = R.layer_norm(x, w[p + "norm1.weight"], w[p + "norm1.bias"], 1e-5)
    q = R.linear(n, w[p + "attn1.to_q.weight"])
    k = R.linear(n, w[p + "attn1.to_k.weight"])
    v = R.linear(n, w[p + "attn1.to_v.weight"])
    o = _attn(q, k, v, heads)
    x = x + R.linear(o, w[p + "attn1.to_out.0.weight"], w[p + "attn1.to_out.0.bias"])
    n = R.layer_norm(x, w[p + "norm2.weight"], w[p + "norm2.bias"], 1e-5)
    q = R.linear(n, w[p + "attn2.to_q.weight"])
    k = R.linear(ctx, w[p + "attn2.to_k.weight"])
    v = R.linear(ctx, w[p + "attn2.to_v.weight"])
    o = _attn(q, k, v, heads)
    x = x + R.linear(o, w[p + "attn2.to_out.0.weight"], w[p + "attn2.to_out.0.bias"])
    n = R.layer_norm(x, w[p + "norm3.weight"], w[p + "norm3.bias"], 1e-5)
    h = R.linear(n, w[p + "ff.net.0.proj.weight"], w[p + "ff.net.0.proj.bias"])
    h = R.geglu(h)
    x = x + R.linear(h, w[p + "ff.net.2.weight"], w[p + "ff.net.2.bias"])
    assert x.shape[-1] == C
    return x


def transformer2d(w, p, x, ctx, depth):
    """src/infer/unet.cu:810-858; x NCHW."""
    B, C, H, W = x.shape
    h = R.group_norm(x, 32, w[p + "norm.weight"], w[p + "norm.bias"], 1e-6)
    h = h.permute(0, 2, 3, 1).reshape(B, H * W, C)
    h = R.linear(h, w[p + "proj_in.weight"], w[p + "proj_in.bias"])
    for l in range(depth):
        h = transformer_block(w, f"{p}transformer_blocks.{l}.", h, ctx, C // 64)
    h = R.linear(h, w[p + "proj_out.weight"], w[p + "proj_out.bias"])
    return h.reshape(B, H, W, C).permute(0, 3, 1, 2) + x


def embeddings(w, cfg, timesteps, text, time_ids):
    """time + add embedding -> temb [B, T] (src/infer/unet.cu:976-1031)."""
    t_emb = R.timestep_embedding(timesteps, cfg.C0)
    h = R.silu(R.linear(t_emb, w["time_embedding.linear_1.weight"], w["time_embedding.linear_1.bias"]))
    temb = R.linear(h, w["time_embedding.linear_2.weight"], w["time_embedding.linear_2.bias"])
    B = text.shape[0]
    ids = time_ids.reshape(-1, 6)
    if ids.shape[0] == 1:
        ids = ids.expand(B, 6)
    emb = R.timestep_embedding(ids.reshape(-1), cfg.id_dim).reshape(B, 6 * cfg.id_dim)
    a = torch.cat([text, emb], dim=1)
    a = R.silu(R.linear(a, w["add_embedding.linear_1.weight"], w["add_embedding.linear_1.bias"]))
    a = R.linear(a, w["add_embedding.linear_2.weight"], w["add_embedding.linear_2.bias"])
    return temb + a


@torch.no_grad()
def unet_forward(w, cfg: UNetCfg, latent, timesteps, ehs, text, time_ids, stages=None):
    """noise_pred for latent [B, in, H, W]; timesteps [B]; ehs [B, L, cross];
    text [B, text_dim]; time_ids [6] or [B, 6].  ``stages`` (dict) receives
    named intermediate outputs (NCHW)."""
    def stage(name, t):
        if stages is not None:
            stages[name] = t.clone()

    C = _level_channels(cfg)
    depths = [0, cfg.depth1, cfg.depth2]
    temb = embeddings(w, cfg, timesteps, text, time_ids)
    stage("temb", temb)
    ts = R.silu(temb)
    x = R.conv2d(latent, w["conv_in.weight"], w["conv_in.bias"], 1, 1)
    stage("conv_in_out", x)
    skips = [x]
    for lv in range(3):
        for r in range(2):
            x = resnet_block(w, f"down_blocks.{lv}.resnets.{r}.", x, ts)
            if depths[lv]:
                x = transformer2d(w, f"down_blocks.{lv}.attentions.{r}.", x, ehs, depths[lv])
            skips.append(x)
        if lv < 2:
            x = R.conv2d(x, w[f"down_blocks.{lv}.downsamplers.0.conv.weight"],
                         w[f"down_blocks.{lv}.downsamplers.0.conv.bias"], 2, 1)
            skips.append(x)
        stage(f"down_block_{lv}_out", x)
    x = resnet_block(w, "mid_block.resnets.0.", x, ts)
    x = transformer2d(w, "mid_block.attentions.0.", x, ehs, cfg.depth2)
    x = resnet_block(w, "mid_block.resnets.1.", x, ts)
    stage("mid_block_out", x)
    for u in range(3):
        lv = 2 - u
        for r in range(3):
            x = torch.cat([x, skips.pop()], dim=1)
            x = resnet_block(w, f"up_blocks.{u}.resnets.{r}.", x, ts)
            if depths[lv]:
                x = transformer2d(w, f"up_blocks.{u}.attentions.{r}.", x, ehs, depths[lv])
        if u < 2:
            x = R.upsample_nearest2x(x)
            x = R.conv2d(x, w[f"up_blocks.{u}.upsamplers.0.conv.weight"],
                         w[f"up_blocks.{u}.upsamplers.0.conv.bias"], 1, 1)
        stage(f"up_block_{u}_out", x)
    assert not skips
    x = R.silu(R.group_norm(x, 32, w["conv_norm_out.weight"], w["conv_norm_out.bias"], 1e-5))
    x = R.conv2d(x, w["conv_out.weight"], w["conv_out.bias"], 1, 1)
    stage("noise_pred", x)
    return x
