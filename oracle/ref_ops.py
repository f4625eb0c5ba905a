"""fp32 torch-CPU restatement of the hot-path kernels (test oracle only).

Every function takes and returns float32 CPU tensors.  Inputs that the GPU
sees as fp16 are rounded to fp16 first by the caller and decoded back to
fp32, so the oracle measures only kernel error (the reference's test
convention, src/tests/test_conv2d.cu:47-69).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def conv2d(x, w, b=None, stride=1, pad=1, dilation=1):
    """NCHW conv, zero padding; stride / pad / dilation an int or an (h, w)
    pair.  Reference formula: src/kernels/conv2d.cu:88-164 (direct conv with
    per-axis stride, padding and dilation, fp32 accumulate) and
    src/kernels/conv2d.cuh:21-40."""
    return F.conv2d(x, w, b, stride=stride, padding=pad, dilation=dilation)


def gemm(a, b, c=None, alpha=1.0, beta=0.0, trans_a=False, trans_b=False):
    """C = alpha op(A) op(B) + beta C (src/kernels/gemm.cuh:30-53)."""
    A = a.t() if trans_a else a
    B = b.t() if trans_b else b
    out = alpha * (A @ B)
    if c is not None and beta != 0.0:
        out = out + beta * c
    return out


def linear(x, w, b=None):
    """y = x W^T + b, W [out, in] (src/infer/unet.cu:517-525)."""
    return F.linear(x, w, b)


def group_norm(x, num_groups, gamma, beta, eps):
    """GroupNorm on NCHW (src/kernels/groupnorm.cu:91-148: per-(n,g) mean/var,
    biased variance, var clamped at 0, y = (x-mean)*rsqrt(var+eps)*gamma+beta)."""
    return F.group_norm(x, num_groups, gamma, beta, eps)


def silu(x):
    """x * sigmoid(x) (src/kernels/activation.cu:25-35)."""
    return x * torch.sigmoid(x)


def gelu_erf(x):
    """0.5 x (1 + erf(x / sqrt 2)) (src/kernels/activation.cu:37-50)."""
    return 0.5 * x * (1.0 + torch.erf(x * (1.0 / math.sqrt(2.0))))


def gelu_tanh(x):
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) (src/kernels/activation.cu:54-70,
    src/tests/test_activation.cu:127-131)."""
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def layer_norm(x, gamma, beta, eps=1e-5):
    """LayerNorm over the last dim (src/kernels/layernorm.cu:78-126)."""
    C = x.shape[-1]
    return F.layer_norm(x, (C,), gamma, beta, eps)


def attention(q, k, v, scale):
    """softmax(scale Q K^T) V in fp32, [B,H,S,Dh] (src/kernels/attention.cu:137-219,
    src/tests/test_attention.cu:99-161).  Written out, not via SDPA."""
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    s = s - s.amax(dim=-1, keepdim=True)
    p = torch.exp(s)
    p = p / p.sum(dim=-1, keepdim=True)
    return torch.matmul(p, v)


def geglu(h):
    """h [T, 2d] -> h[:, :d] * gelu_erf(h[:, d:]) (src/kernels/geglu.cuh:13-19,
    geglu.cu:26-48: value = first half, gate = second half)."""
    d = h.shape[-1] // 2
    return h[..., :d] * gelu_erf(h[..., d:])


def timestep_embedding(t, dim, max_period=10000.0):
    """Sinusoid with cos first (flip_sin_to_cos), shift 0
    (src/kernels/timeembed.cuh:14-24, timeembed.cu:30-49).  t: 1-D tensor."""
    half = dim // 2
    exponent = -math.log(max_period) * torch.arange(half, dtype=torch.float32) / half
    args = t.float()[:, None] * torch.exp(exponent)[None, :]
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1)


def upsample_nearest2x(x):
    """NCHW nearest 2x (src/kernels/elementwise.cu:40-73)."""
    return F.interpolate(x, scale_factor=2.0, mode="nearest")


def add_embedding_input(text_embeds, time_ids):
    """[B,1280] text_embeds ++ 6 x sinusoid_256(time_ids) -> [B,2816]
    (src/infer/unet.cu:995-1024)."""
    B = text_embeds.shape[0]
    ids = time_ids.reshape(-1, 6)
    if ids.shape[0] == 1 and B > 1:
        ids = ids.expand(B, 6)
    emb = timestep_embedding(ids.reshape(-1), 256).reshape(B, 6 * 256)
    return torch.cat([text_embeds, emb], dim=1)


def to_fp16_grid(x):
    """Round to fp16 and decode back to fp32 (what the GPU stores)."""
    return x.to(torch.float16).to(torch.float32)
