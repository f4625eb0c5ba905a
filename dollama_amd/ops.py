"""Python mirror of the reference kernel host API, over the C ABI.

The ``launch_*`` functions keep the names, argument order and meaning of the
reference's ``dollama::launch_*`` wrappers (src/kernels/*.cuh) and raise
``DlmError`` (a RuntimeError) where those throw.  Device buffers are torch
CUDA tensors (fp16 unless stated); torch is used only to own device memory and
to name the stream, every computation runs in the HIP kernels of
``libdlm_hip.so``.

Before each launch the wrapper checks on the host that every tensor is a
contiguous fp16 tensor on the GPU holding at least the elements the kernel
will touch, so a shape mistake raises instead of reaching the device.

The channels-last helpers at the bottom (``linear``, ``conv2d_nhwc``,
``group_norm_nhwc``, ``attention_strided``...) expose the fused native forms
the UNet driver uses.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _lib
from ._lib import (ACT_GEGLU, ACT_GELU, ACT_NONE, ACT_SILU, AttentionArgs, AttentionVtArgs,
                   ConvNhwcArgs, call)

__all__ = [
    "launch_conv2d", "launch_gemm_fp16", "launch_group_norm", "launch_group_norm_mb",
    "launch_group_norm_silu", "launch_layer_norm", "launch_attention", "launch_attention_fast",
    "launch_geglu", "launch_silu", "launch_gelu", "launch_add", "launch_upsample_nearest2x",
    "launch_bias_add_rowvec", "launch_bias_add_channel", "launch_conv_bias_biasch",
    "launch_conv_bias_residual", "launch_timestep_embedding", "linear", "pack_conv_weight",
    "conv2d_nhwc", "group_norm_nhwc", "attention_strided", "pack_geglu", "nchw_to_nhwc",
    "nhwc_to_nchw", "linear_small", "sdxl_embed_inputs",
    "ACT_NONE", "ACT_SILU", "ACT_GEGLU", "ACT_GELU",
]


def stream_handle() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t: Optional[torch.Tensor], numel: int, name: str, dtype=torch.float16, optional=False):
    if t is None:
        if optional:
            return
        raise ValueError(f"{name} is None")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < numel:
        raise ValueError(f"{name} holds {t.numel()} elements, the call needs {numel}")


def _conv_out_dim(x, k, s, p, d):
    return (x + 2 * p - d * (k - 1) - 1) // s + 1


# ---------------------------------------------------------------------------
# Reference-layout API
# ---------------------------------------------------------------------------
def launch_conv2d(d_in, d_weight, d_bias, d_out, N, Cin, H, W, Cout, KH, KW,
                  stride_h, stride_w, pad_h, pad_w, dilation_h=1, dilation_w=1):
    """reference src/kernels/conv2d.cuh:38-40 (NCHW, optional bias)."""
    if min(N, Cin, H, W, Cout, KH, KW) <= 0:
        return
    Ho = _conv_out_dim(H, KH, stride_h, pad_h, dilation_h)
    Wo = _conv_out_dim(W, KW, stride_w, pad_w, dilation_w)
    if Ho <= 0 or Wo <= 0:
        return
    _need(d_in, N * Cin * H * W, "d_in")
    _need(d_weight, Cout * Cin * KH * KW, "d_weight")
    _need(d_bias, Cout, "d_bias", optional=True)
    _need(d_out, N * Cout * Ho * Wo, "d_out")
    call("dlm_conv2d_fp16", _p(d_in), _p(d_weight), _p(d_bias), _p(d_out), N, Cin, H, W, Cout,
         KH, KW, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w, stream_handle())


def launch_gemm_fp16(d_A, d_B, d_C, M, N, K, alpha=1.0, beta=0.0, transA=False, transB=False):
    """reference src/kernels/gemm.cuh:44-53: C = alpha op(A) op(B) + beta C."""
    if min(M, N, K) <= 0:
        return
    _need(d_A, M * K, "d_A")
    _need(d_B, K * N, "d_B")
    _need(d_C, M * N, "d_C")
    call("dlm_gemm_fp16", _p(d_A), _p(d_B), _p(d_C), M, N, K, float(alpha), float(beta),
         int(bool(transA)), int(bool(transB)), stream_handle())


def _gn(d_in, d_gamma, d_beta, d_out, N, C, H, W, num_groups, eps, silu):
    if min(N, C, H, W, num_groups) <= 0:
        return
    _need(d_in, N * C * H * W, "d_in")
    _need(d_out, N * C * H * W, "d_out")
    _need(d_gamma, C, "d_gamma", optional=True)
    _need(d_beta, C, "d_beta", optional=True)
    call("dlm_group_norm_fp16", _p(d_in), _p(d_gamma), _p(d_beta), _p(d_out), N, C, H, W,
         num_groups, float(eps), int(silu), stream_handle())


def launch_group_norm(d_in, d_gamma, d_beta, d_out, N, C, H, W, num_groups, eps):
    """reference src/kernels/groupnorm.cuh:51-60."""
    _gn(d_in, d_gamma, d_beta, d_out, N, C, H, W, num_groups, eps, 0)


def launch_group_norm_mb(d_in, d_gamma, d_beta, d_out, N, C, H, W, num_groups, eps):
    """reference src/kernels/groupnorm.cuh:75-84 (same numerics as launch_group_norm)."""
    _gn(d_in, d_gamma, d_beta, d_out, N, C, H, W, num_groups, eps, 0)


def launch_group_norm_silu(d_in, d_gamma, d_beta, d_out, N, C, H, W, num_groups, eps):
    """reference src/kernels/groupnorm.cuh:99-108."""
    _gn(d_in, d_gamma, d_beta, d_out, N, C, H, W, num_groups, eps, 1)


def launch_layer_norm(d_in, d_gamma, d_beta, d_out, rows, C, eps=1e-5):
    """reference src/kernels/layernorm.cuh:51-57."""
    if rows <= 0 or C <= 0:
        return
    _need(d_in, rows * C, "d_in")
    _need(d_out, rows * C, "d_out")
    _need(d_gamma, C, "d_gamma", optional=True)
    _need(d_beta, C, "d_beta", optional=True)
    call("dlm_layer_norm_fp16", _p(d_in), _p(d_gamma), _p(d_beta), _p(d_out), rows, C,
         float(eps), stream_handle())


def launch_attention(d_q, d_k, d_v, d_out, B, H, Sq, Sk, Dh, scale):
    """reference src/kernels/attention.cuh:53-54, layout [B,H,S,Dh]."""
    if min(B, H, Sq, Sk, Dh) <= 0:
        return
    _need(d_q, B * H * Sq * Dh, "d_q")
    _need(d_k, B * H * Sk * Dh, "d_k")
    _need(d_v, B * H * Sk * Dh, "d_v")
    _need(d_out, B * H * Sq * Dh, "d_out")
    call("dlm_attention_fp16", _p(d_q), _p(d_k), _p(d_v), _p(d_out), B, H, Sq, Sk, Dh,
         float(scale), stream_handle())


launch_attention_fast = launch_attention


def launch_geglu(d_in, d_out, tokens, d):
    """reference src/kernels/geglu.cuh:42."""
    if tokens <= 0 or d <= 0:
        return
    _need(d_in, tokens * 2 * d, "d_in")
    _need(d_out, tokens * d, "d_out")
    call("dlm_geglu_fp16", _p(d_in), _p(d_out), tokens, d, stream_handle())


def _unary(name, d_in, d_out, n):
    if n <= 0:
        return
    _need(d_in, n, "d_in")
    _need(d_out, n, "d_out")
    call(name, _p(d_in), _p(d_out), n, stream_handle())


def launch_silu(d_in, d_out, n):
    """reference src/kernels/activation.cuh:33."""
    _unary("dlm_silu_fp16", d_in, d_out, n)


def launch_gelu(d_in, d_out, n):
    """reference src/kernels/activation.cuh:37."""
    _unary("dlm_gelu_fp16", d_in, d_out, n)


def launch_gelu_tanh(d_in, d_out, n):
    """Reference launch_gelu_tanh (src/kernels/activation.cuh:41)."""
    _unary("dlm_gelu_tanh_fp16", d_in, d_out, n)


def launch_add(d_a, d_b, d_out, n):
    """reference src/kernels/elementwise.cuh:26."""
    if n <= 0:
        return
    _need(d_a, n, "d_a")
    _need(d_b, n, "d_b")
    _need(d_out, n, "d_out")
    call("dlm_add_fp16", _p(d_a), _p(d_b), _p(d_out), n, stream_handle())


def launch_upsample_nearest2x(d_in, d_out, N, C, H, W):
    """reference src/kernels/elementwise.cuh:37."""
    if min(N, C, H, W) <= 0:
        return
    _need(d_in, N * C * H * W, "d_in")
    _need(d_out, N * C * 4 * H * W, "d_out")
    call("dlm_upsample_nearest2x_fp16", _p(d_in), _p(d_out), N, C, H, W, stream_handle())


def launch_bias_add_rowvec(d_in, d_bias, d_out, tokens, C):
    """reference src/kernels/bias_add.cuh:32-36."""
    if tokens <= 0 or C <= 0:
        return
    _need(d_in, tokens * C, "d_in")
    _need(d_bias, C, "d_bias")
    _need(d_out, tokens * C, "d_out")
    call("dlm_bias_add_rowvec_fp16", _p(d_in), _p(d_bias), _p(d_out), tokens, C, stream_handle())


def launch_bias_add_channel(d_in, d_bias, d_out, N, C, H, W):
    """reference src/kernels/bias_add.cuh:51-57."""
    if min(N, C, H, W) <= 0:
        return
    _need(d_in, N * C * H * W, "d_in")
    _need(d_bias, C, "d_bias")
    _need(d_out, N * C * H * W, "d_out")
    call("dlm_bias_add_channel_fp16", _p(d_in), _p(d_bias), _p(d_out), N, C, H, W,
         stream_handle())


def launch_conv_bias_biasch(d_conv, d_convbias, d_tproj, d_out, B, Cout, H, W):
    """reference src/kernels/bias_add.cuh:75-82."""
    if min(B, Cout, H, W) <= 0:
        return
    _need(d_conv, B * Cout * H * W, "d_conv")
    _need(d_convbias, Cout, "d_convbias")
    _need(d_tproj, B * Cout, "d_tproj")
    _need(d_out, B * Cout * H * W, "d_out")
    call("dlm_conv_bias_biasch_fp16", _p(d_conv), _p(d_convbias), _p(d_tproj), _p(d_out), B, Cout,
         H, W, stream_handle())


def launch_conv_bias_residual(d_conv, d_convbias, d_residual, d_out, B, Cout, H, W):
    """reference src/kernels/bias_add.cuh:96-103."""
    if min(B, Cout, H, W) <= 0:
        return
    _need(d_conv, B * Cout * H * W, "d_conv")
    _need(d_convbias, Cout, "d_convbias")
    _need(d_residual, B * Cout * H * W, "d_residual")
    _need(d_out, B * Cout * H * W, "d_out")
    call("dlm_conv_bias_residual_fp16", _p(d_conv), _p(d_convbias), _p(d_residual), _p(d_out), B,
         Cout, H, W, stream_handle())


def launch_timestep_embedding(d_out, timestep, dim, max_period=10000.0):
    """reference src/kernels/timeembed.cuh:44-47 (cos first)."""
    if dim <= 1:
        return
    _need(d_out, (dim // 2) * 2, "d_out")
    call("dlm_timestep_embedding_fp16", _p(d_out), float(timestep), dim, float(max_period),
         stream_handle())


# ---------------------------------------------------------------------------
# Channels-last fused helpers (native forms)
# ---------------------------------------------------------------------------
def linear(x: torch.Tensor, w: torch.Tensor, bias=None, residual=None, act=ACT_NONE,
           out=None, alpha=1.0, beta=1.0, gn_stats: Optional[torch.Tensor] = None,
           tokens: int = 0) -> torch.Tensor:
    """y = act(alpha * x @ w.T + bias) + beta * residual.  x [M,K], w [N,K].
    For ACT_GEGLU, w/bias must be packed with ``pack_geglu`` and y has N/2 columns.
    gn_stats: a GroupNorm workspace that receives y's chunk statistics, y
    holding M / tokens samples of `tokens` rows."""
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError("w.shape[1] != K")
    ncols = N // 2 if act == ACT_GEGLU else N
    if out is None:
        out = torch.empty(M, ncols, dtype=torch.float16, device=x.device)
    _need(x, M * K, "x")
    _need(w, N * K, "w")
    _need(bias, N, "bias", optional=True)
    _need(residual, M * ncols, "residual", optional=True)
    _need(out, M * ncols, "out")
    if gn_stats is not None:
        if tokens <= 0 or M % tokens:
            raise ValueError("gn_stats needs M = samples x tokens")
        _need(gn_stats, group_norm_workspace_bytes(M // tokens, N, tokens), "gn_stats", dtype=torch.uint8)
        call("dlm_linear_gn_stats_fp16", _p(x), K, _p(w), K, _p(bias), _p(residual), ncols, _p(out), ncols,
             M, N, K, float(alpha), float(beta), int(act), int(tokens), _p(gn_stats), stream_handle())
        return out
    call("dlm_linear_fp16", _p(x), K, _p(w), K, _p(bias), _p(residual), ncols, _p(out), ncols,
         M, N, K, float(alpha), float(beta), int(act), stream_handle())
    return out


def linear_f32out(x: torch.Tensor, w: torch.Tensor, bias=None, residual=None, act=ACT_NONE,
                  out=None, alpha=1.0, beta=1.0) -> torch.Tensor:
    """fp32 y = act(alpha * x @ w.T + bias) + beta * residual (fp32 residual);
    x [M,K], w [N,K] fp16."""
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError("w.shape[1] != K")
    if out is None:
        out = torch.empty(M, N, dtype=torch.float32, device=x.device)
    _need(x, M * K, "x")
    _need(w, N * K, "w")
    _need(bias, N, "bias", optional=True)
    _need(residual, M * N, "residual", optional=True, dtype=torch.float32)
    _need(out, M * N, "out", dtype=torch.float32)
    call("dlm_linear_f32out_fp16", _p(x), K, _p(w), K, _p(bias), _p(residual), N, _p(out), N,
         M, N, K, float(alpha), float(beta), int(act), stream_handle())
    return out


def softmax_rows(s: torch.Tensor, out=None) -> torch.Tensor:
    """fp16 softmax over the last dim of fp32 [rows, cols]."""
    rows, cols = s.shape
    if out is None:
        out = torch.empty(rows, cols, dtype=torch.float16, device=s.device)
    _need(s, rows * cols, "s", dtype=torch.float32)
    _need(out, rows * cols, "out")
    call("dlm_softmax_rows_f32_fp16", _p(s), cols, _p(out), cols, rows, cols, stream_handle())
    return out


def cast_f32_to_f16(x: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """fp16(x * scale)."""
    _need(x, x.numel(), "x", dtype=torch.float32)
    out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    call("dlm_cast_f32_to_f16", _p(x), _p(out), x.numel(), float(scale), stream_handle())
    return out


def linear_vt(x: torch.Tensor, w: torch.Tensor, vt_col0: int, tokens: int, bias=None, vt_ld=None):
    """y = x @ w.T for columns [0, vt_col0) as [M, vt_col0], and the remaining
    columns transposed per sample as vt [M // tokens, N - vt_col0, vt_ld]
    (vt_ld >= tokens; positions past `tokens` are zero)."""
    vt_ld = vt_ld or tokens
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K or M % tokens != 0:
        raise ValueError("shape mismatch")
    y = torch.empty(M, vt_col0, dtype=torch.float16, device=x.device)
    vt = torch.empty(M // tokens, N - vt_col0, vt_ld, dtype=torch.float16, device=x.device)
    _need(x, M * K, "x")
    _need(w, N * K, "w")
    _need(bias, N, "bias", optional=True)
    call("dlm_linear_vt_fp16", _p(x), K, _p(w), K, _p(bias), _p(y), vt_col0, _p(vt), vt_col0,
         tokens, vt_ld, M, N, K, stream_handle())
    return y, vt


def ln_fold(w: torch.Tensor, gamma=None, beta=None, bias=None):
    """Weight side of a LayerNorm folded into the linear w [N, K] (bias [N]):
    (fp16 w * gamma, fp32 c1 = row sums of it, fp32 c2 = w @ beta + bias)."""
    N, K = w.shape
    wo = torch.empty_like(w)
    c1 = torch.empty(N, dtype=torch.float32, device=w.device)
    c2 = torch.empty(N, dtype=torch.float32, device=w.device)
    _need(w, N * K, "w")
    _need(gamma, K, "gamma", optional=True)
    _need(beta, K, "beta", optional=True)
    _need(bias, N, "bias", optional=True)
    call("dlm_ln_fold_fp16", _p(w), K, N, K, _p(gamma), _p(beta), _p(bias), _p(wo), K, _p(c1),
         _p(c2), stream_handle())
    return wo, c1, c2


def linear_ln(x: torch.Tensor, w_folded, c1, c2, eps: float, residual=None, act=ACT_NONE,
              out=None, beta=1.0) -> torch.Tensor:
    """y = act(LayerNorm(x) @ w.T + b) + beta * residual with the LayerNorm
    computed inside the GEMM; w_folded, c1, c2 from ``ln_fold``."""
    M, K = x.shape
    N = w_folded.shape[0]
    ncols = N // 2 if act == ACT_GEGLU else N
    if out is None:
        out = torch.empty(M, ncols, dtype=torch.float16, device=x.device)
    _need(x, M * K, "x")
    _need(w_folded, N * K, "w")
    _need(c1, N, "c1", dtype=torch.float32)
    _need(c2, N, "c2", dtype=torch.float32)
    _need(residual, M * ncols, "residual", optional=True)
    _need(out, M * ncols, "out")
    call("dlm_linear_ln_fp16", _p(x), K, _p(w_folded), K, _p(c1), _p(c2), float(eps), _p(residual),
         ncols, _p(out), ncols, M, N, K, float(beta), int(act), stream_handle())
    return out


def linear_vt_ln(x: torch.Tensor, w_folded, c1, c2, eps: float, vt_col0: int, tokens: int,
                 vt_ld=None):
    """``linear_vt`` of LayerNorm(x), the LayerNorm computed inside the GEMM."""
    vt_ld = vt_ld or tokens
    M, K = x.shape
    N = w_folded.shape[0]
    y = torch.empty(M, vt_col0, dtype=torch.float16, device=x.device)
    vt = torch.empty(M // tokens, N - vt_col0, vt_ld, dtype=torch.float16, device=x.device)
    _need(x, M * K, "x")
    _need(w_folded, N * K, "w")
    _need(c1, N, "c1", dtype=torch.float32)
    _need(c2, N, "c2", dtype=torch.float32)
    call("dlm_linear_vt_ln_fp16", _p(x), K, _p(w_folded), K, _p(c1), _p(c2), float(eps), _p(y),
         vt_col0, _p(vt), vt_col0, tokens, vt_ld, M, N, K, stream_handle())
    return y, vt


def pack_geglu(w: torch.Tensor, b: Optional[torch.Tensor]):
    """[2d, K] value-first GEGLU projection -> 4-row value/gate interleave for ACT_GEGLU."""
    two_d, K = w.shape
    d = two_d // 2
    wo = torch.empty_like(w)
    bo = None if b is None else torch.empty_like(b)
    _need(w, two_d * K, "w")
    _need(b, two_d, "b", optional=True)
    call("dlm_geglu_pack_fp16", _p(w), _p(b), _p(wo), _p(bo), d, K, stream_handle())
    return wo, bo


def pack_conv_weight(w: torch.Tensor, cin_pad: Optional[int] = None, out=None, ld=None, col0=0):
    """[Cout, Cin, KH, KW] -> [Cout, KH*KW*Cin_pad]: channel blocks of 64, then
    taps, then channels when Cin_pad % 64 == 0, else taps then channels."""
    Cout, Cin, KH, KW = w.shape
    cp = cin_pad or Cin
    ld = ld or KH * KW * cp
    if out is None:
        out = torch.zeros(Cout, ld, dtype=torch.float16, device=w.device)
    _need(w, w.numel(), "w")
    _need(out, Cout * ld, "out")
    call("dlm_conv_weight_pack_fp16", _p(w), _p(out), Cout, Cin, KH, KW, cp, ld, col0,
         stream_handle())
    return out


def nchw_to_nhwc(x: torch.Tensor, c_pad: Optional[int] = None) -> torch.Tensor:
    N, C, H, W = x.shape
    cp = c_pad or C
    out = torch.empty(N, H, W, cp, dtype=torch.float16, device=x.device)
    _need(x, x.numel(), "x")
    call("dlm_nchw_to_nhwc_fp16", _p(x), _p(out), N, C, H * W, cp, stream_handle())
    return out


def nhwc_to_nchw(x: torch.Tensor, C: Optional[int] = None) -> torch.Tensor:
    N, H, W, cp = x.shape
    C = C or cp
    out = torch.empty(N, C, H, W, dtype=torch.float16, device=x.device)
    _need(x, x.numel(), "x")
    call("dlm_nhwc_to_nchw_fp16", _p(x), _p(out), N, C, H * W, cp, stream_handle())
    return out


def conv2d_nhwc(x: torch.Tensor, w_packed: torch.Tensor, *, KH: int, KW: int, stride=1, pad=1,
                bias=None, tbias=None, residual=None, x_b: Optional[torch.Tensor] = None,
                upsample=False, shortcut: Optional[torch.Tensor] = None,
                shortcut_b: Optional[torch.Tensor] = None, act=ACT_NONE, out=None,
                out_nchw=False, cout: Optional[int] = None, out_f32=False,
                gn_stats: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Channels-last implicit-GEMM conv.  x [N,H,W,Ca] (+ x_b [N,H,W,Cb] concatenated),
    optional fused 1x1 shortcut over concat(shortcut, shortcut_b), weight from
    ``pack_conv_weight`` (segment-1 columns appended).  The residual may be
    fp16 or fp32; out_f32 gives an fp32 output.  gn_stats: a GroupNorm
    workspace (``group_norm_workspace``) that receives the output's chunk
    statistics, for ``group_norm_nhwc_prestats``."""
    N, H, W, Ca = x.shape
    Cb = 0 if x_b is None else x_b.shape[3]
    C1a = 0 if shortcut is None else shortcut.shape[3]
    C1b = 0 if shortcut_b is None else shortcut_b.shape[3]
    Cout = cout or w_packed.shape[0]
    Hv, Wv = (2 * H, 2 * W) if upsample else (H, W)
    Ho = (Hv + 2 * pad - KH) // stride + 1
    Wo = (Wv + 2 * pad - KW) // stride + 1
    K = KH * KW * (Ca + Cb) + C1a + C1b
    if w_packed.shape[1] < K:
        raise ValueError(f"packed weight has {w_packed.shape[1]} columns, need {K}")
    _need(x, N * H * W * Ca, "x")
    _need(x_b, N * H * W * Cb, "x_b", optional=True)
    _need(shortcut, N * Ho * Wo * C1a, "shortcut", optional=True)
    _need(shortcut_b, N * Ho * Wo * C1b, "shortcut_b", optional=True)
    _need(w_packed, Cout * w_packed.shape[1], "w_packed")
    _need(bias, Cout, "bias", optional=True)
    _need(tbias, N * Cout, "tbias", optional=True)
    res_f32 = residual is not None and residual.dtype == torch.float32
    _need(residual, N * Ho * Wo * Cout, "residual", optional=True,
          dtype=torch.float32 if res_f32 else torch.float16)
    odt = torch.float32 if out_f32 else torch.float16
    if out is None:
        shape = (N, Cout, Ho, Wo) if out_nchw else (N, Ho, Wo, Cout)
        out = torch.empty(shape, dtype=odt, device=x.device)
    _need(out, N * Ho * Wo * Cout, "out", dtype=odt)
    a = ConvNhwcArgs()
    a.src0a, a.src0b, a.C0a, a.C0b, a.ld0a, a.ld0b = _p(x), _p(x_b), Ca, Cb, Ca, max(Cb, 0)
    a.src1a, a.src1b, a.C1a, a.C1b, a.ld1a, a.ld1b = _p(shortcut), _p(shortcut_b), C1a, C1b, C1a, C1b
    a.N, a.H, a.W, a.KH, a.KW, a.stride, a.pad, a.upsample = N, H, W, KH, KW, stride, pad, int(upsample)
    a.weight, a.ldw, a.Cout = _p(w_packed), w_packed.shape[1], Cout
    a.bias, a.tbias, a.tbias_ld = _p(bias), _p(tbias), Cout
    a.residual, a.res_ld = _p(residual), Cout
    a.out, a.ldy, a.out_nchw, a.act = _p(out), Cout, int(out_nchw), int(act)
    a.out_f32, a.res_f32 = int(out_f32), int(res_f32)
    if gn_stats is not None:
        _need(gn_stats, group_norm_workspace_bytes(N, Cout, Ho * Wo), "gn_stats", dtype=torch.uint8)
    a.gn_stats = _p(gn_stats)
    call("dlm_conv2d_nhwc_fp16", ctypes.byref(a), stream_handle())
    return out


_ws_cache: dict = {}


def group_norm_nhwc(x: torch.Tensor, gamma, beta, groups: int, eps: float, silu: bool,
                    x_b: Optional[torch.Tensor] = None, out=None) -> torch.Tensor:
    """GroupNorm on [N,H,W,Ca] (+ x_b [N,H,W,Cb] concatenated) -> [N,H,W,Ca+Cb]."""
    N, H, W, Ca = x.shape
    Cb = 0 if x_b is None else x_b.shape[3]
    C = Ca + Cb
    HW = H * W
    _need(x, N * HW * Ca, "x", dtype=x.dtype if x.dtype == torch.float32 else torch.float16)
    _need(x_b, N * HW * Cb, "x_b", optional=True)
    _need(gamma, C, "gamma", optional=True)
    _need(beta, C, "beta", optional=True)
    if out is None:
        out = torch.empty(N, H, W, C, dtype=torch.float16, device=x.device)
    _need(out, N * HW * C, "out")
    nbytes = _lib.hip_lib().dlm_group_norm_nhwc_workspace_bytes(N, C, HW)
    ws = _ws_cache.get(x.device)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        _ws_cache[x.device] = ws
    if x.dtype == torch.float32:
        if x_b is not None:
            raise ValueError("fp32 GroupNorm takes one source")
        call("dlm_group_norm_nhwc_f32in", _p(x), C, _p(gamma), _p(beta), _p(out), C, N, HW, C,
             groups, float(eps), int(silu), _p(ws), stream_handle())
        return out
    call("dlm_group_norm_nhwc_fp16", _p(x), Ca, Ca, _p(x_b), max(Cb, 8), _p(gamma), _p(beta),
         _p(out), C, N, HW, C, groups, float(eps), int(silu), _p(ws), stream_handle())
    return out


def group_norm_workspace_bytes(N: int, C: int, HW: int) -> int:
    return int(_lib.hip_lib().dlm_group_norm_nhwc_workspace_bytes(N, C, HW))


def group_norm_workspace(N: int, C: int, HW: int, device) -> torch.Tensor:
    """A GroupNorm workspace; its first bytes hold the chunk statistics."""
    return torch.empty(group_norm_workspace_bytes(N, C, HW), dtype=torch.uint8, device=device)


def group_norm_chunk_stats(x: torch.Tensor, ws: torch.Tensor) -> torch.Tensor:
    """Chunk statistics of fp16 [N,H,W,C] into the workspace ws (returned)."""
    N, H, W, C = x.shape
    _need(x, N * H * W * C, "x")
    _need(ws, group_norm_workspace_bytes(N, C, H * W), "ws", dtype=torch.uint8)
    call("dlm_group_norm_chunk_stats_fp16", _p(x), C, N, H * W, C, _p(ws), stream_handle())
    return ws


def group_norm_nhwc_prestats(x: torch.Tensor, gamma, beta, groups: int, eps: float, silu: bool,
                             ws: torch.Tensor, out=None) -> torch.Tensor:
    """GroupNorm of fp16 [N,H,W,C] whose chunk statistics are already in ws."""
    N, H, W, C = x.shape
    HW = H * W
    _need(x, N * HW * C, "x")
    _need(gamma, C, "gamma", optional=True)
    _need(beta, C, "beta", optional=True)
    _need(ws, group_norm_workspace_bytes(N, C, HW), "ws", dtype=torch.uint8)
    if out is None:
        out = torch.empty(N, H, W, C, dtype=torch.float16, device=x.device)
    _need(out, N * HW * C, "out")
    call("dlm_group_norm_nhwc_prestats_fp16", _p(x), C, _p(gamma), _p(beta), _p(out), C, N, HW, C,
         groups, float(eps), int(silu), _p(ws), stream_handle())
    return out


def group_norm_nhwc_prestats2(x: torch.Tensor, x_b: torch.Tensor, gamma, beta, groups: int, eps: float,
                              silu: bool, ws_a: torch.Tensor, ws_b: torch.Tensor, out=None) -> torch.Tensor:
    """GroupNorm of concat(x [N,H,W,Ca], x_b [N,H,W,Cb]) from each source's chunk
    statistics (the first bytes of ws_a, ws_b: GroupNorm workspaces for Ca and
    Cb channels)."""
    N, H, W, Ca = x.shape
    Cb = x_b.shape[3]
    C, HW = Ca + Cb, H * W
    _need(x, N * HW * Ca, "x")
    _need(x_b, N * HW * Cb, "x_b")
    _need(gamma, C, "gamma", optional=True)
    _need(beta, C, "beta", optional=True)
    _need(ws_a, group_norm_workspace_bytes(N, Ca, HW), "ws_a", dtype=torch.uint8)
    _need(ws_b, group_norm_workspace_bytes(N, Cb, HW), "ws_b", dtype=torch.uint8)
    if out is None:
        out = torch.empty(N, H, W, C, dtype=torch.float16, device=x.device)
    _need(out, N * HW * C, "out")
    ws = group_norm_workspace(N, C, HW, x.device)
    call("dlm_group_norm_nhwc_prestats2_fp16", _p(x), Ca, Ca, _p(x_b), Cb, _p(ws_a), _p(ws_b), _p(gamma),
         _p(beta), _p(out), C, N, HW, C, groups, float(eps), int(silu), _p(ws), stream_handle())
    return out


def attention_strided(q, k, v, o, *, B, H, Sq, Sk, q_strides, k_strides, v_strides, o_strides,
                      scale, Dh=64):
    """Flash attention with (batch, token, head) strides in elements per tensor."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (o, "o")):
        if not t.is_cuda or t.dtype != torch.float16:
            raise ValueError(f"{nm} must be a GPU fp16 tensor")
    def _span(strides, S):
        sb, ss, sh = strides
        return (B - 1) * sb + (S - 1) * ss + (H - 1) * sh + Dh
    for t, st, S, nm in ((q, q_strides, Sq, "q"), (k, k_strides, Sk, "k"), (v, v_strides, Sk, "v"),
                         (o, o_strides, Sq, "o")):
        base = t.storage_offset()
        if base + _span(st, S) > t.untyped_storage().nbytes() // 2:
            raise ValueError(f"{nm}: strides reach beyond the tensor's storage")
    a = AttentionArgs()
    a.q, (a.q_sb, a.q_ss, a.q_sh) = _p(q), q_strides
    a.k, (a.k_sb, a.k_ss, a.k_sh) = _p(k), k_strides
    a.v, (a.v_sb, a.v_ss, a.v_sh) = _p(v), v_strides
    a.o, (a.o_sb, a.o_ss, a.o_sh) = _p(o), o_strides
    a.B, a.H, a.Sq, a.Sk, a.Dh, a.scale = B, H, Sq, Sk, Dh, float(scale)
    call("dlm_attention_strided_fp16", ctypes.byref(a), stream_handle())
    return o


def attention_vt(q, k, vt, o, *, B, H, Sq, Sk, q_strides, k_strides, vt_strides, vt_ld,
                 o_strides, scale):
    """Flash attention (Dh = 64) with V given transposed: V^T element
    (b, h, d, key) at vt[b*vt_sb + h*vt_sh + d*vt_ld + key]."""
    for t, nm in ((q, "q"), (k, "k"), (vt, "vt"), (o, "o")):
        if not t.is_cuda or t.dtype != torch.float16:
            raise ValueError(f"{nm} must be a GPU fp16 tensor")
    def _span(strides, S):
        sb, ss, sh = strides
        return (B - 1) * sb + (S - 1) * ss + (H - 1) * sh + 64
    vspan = (B - 1) * vt_strides[0] + (H - 1) * vt_strides[1] + 63 * vt_ld + ((Sk + 7) & ~7)
    for t, span, nm in ((q, _span(q_strides, Sq), "q"), (k, _span(k_strides, Sk), "k"),
                        (vt, vspan, "vt"), (o, _span(o_strides, Sq), "o")):
        if t.storage_offset() + span > t.untyped_storage().nbytes() // 2:
            raise ValueError(f"{nm}: strides reach beyond the tensor's storage")
    a = AttentionVtArgs()
    a.q, a.k, a.vt, a.o = _p(q), _p(k), _p(vt), _p(o)
    a.q_sb, a.q_ss, a.q_sh = q_strides
    a.k_sb, a.k_ss, a.k_sh = k_strides
    a.vt_sb, a.vt_sh = vt_strides
    a.o_sb, a.o_ss, a.o_sh = o_strides
    a.vt_ld, a.B, a.H, a.Sq, a.Sk, a.scale = vt_ld, B, H, Sq, Sk, float(scale)
    a.k_bytes = k.untyped_storage().nbytes() - k.storage_offset() * 2
    a.vt_bytes = vt.untyped_storage().nbytes() - vt.storage_offset() * 2
    call("dlm_attention_vt_fp16", ctypes.byref(a), stream_handle())
    return o


def linear_small(x, w, bias=None, silu_in=False, act=ACT_NONE, out=None, accumulate=False):
    """Skinny linear for M <= 16 rows."""
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.float16, device=x.device)
    _need(x, M * K, "x")
    _need(w, N * K, "w")
    _need(bias, N, "bias", optional=True)
    _need(out, M * N, "out")
    call("dlm_linear_small_fp16", _p(x), K, _p(w), _p(bias), _p(out), N, M, N, K, int(silu_in),
         int(act), int(accumulate), stream_handle())
    return out


def sdxl_embed_inputs(timesteps: torch.Tensor, text_embeds: torch.Tensor, time_ids: torch.Tensor):
    """-> (t_emb [B,320], add_in [B,2816]).  time_ids [6] shared or [B,6]."""
    B = text_embeds.shape[0]
    _need(timesteps, B, "timesteps", dtype=torch.float32)
    _need(text_embeds, B * 1280, "text_embeds")
    stride = 6 if time_ids.dim() == 2 else 0
    _need(time_ids, 6 * (B if stride else 1), "time_ids")
    t_emb = torch.empty(B, 320, dtype=torch.float16, device=text_embeds.device)
    add_in = torch.empty(B, 2816, dtype=torch.float16, device=text_embeds.device)
    call("dlm_sdxl_embed_inputs_fp16", _p(timesteps), _p(text_embeds), 1280, _p(time_ids), stride,
         256, _p(t_emb), 320, _p(add_in), B, stream_handle())
    return t_emb, add_in


def euler_cfg_step(latent: torch.Tensor, noise: torch.Tensor, model_in: torch.Tensor, guidance: float,
                   sigma: float, sigma_next: float, in_scale: float):
    """In place: latent (fp32 [n]) += (u + g (c - u)) * (sigma_next - sigma)
    with noise fp16 [2, n] (cond first); model_in fp16 [2, n] receives
    fp16(latent * in_scale) twice (reference src/infer/diffusion.cu:968-973,
    src/infer/scheduler.hpp:112-143)."""
    n = latent.numel()
    _need(latent, n, "latent", dtype=torch.float32)
    _need(noise, 2 * n, "noise")
    _need(model_in, 2 * n, "model_in")
    call("dlm_euler_cfg_step", _p(latent), _p(noise), _p(model_in), n, float(guidance), float(sigma),
         float(sigma_next), float(in_scale), stream_handle())


def euler_step(latent: torch.Tensor, noise: torch.Tensor, model_in: torch.Tensor, sigma: float,
               sigma_next: float, in_scale: float):
    """In place: latent += noise * (sigma_next - sigma), model_in =
    fp16(latent * in_scale) (one prediction, no guidance)."""
    n = latent.numel()
    _need(latent, n, "latent", dtype=torch.float32)
    _need(noise, n, "noise")
    _need(model_in, n, "model_in")
    call("dlm_euler_step", _p(latent), _p(noise), _p(model_in), n, float(sigma), float(sigma_next),
         float(in_scale), stream_handle())


def scale_latent(latent: torch.Tensor, model_in: torch.Tensor, scale: float, copies: int):
    """model_in[c, :] = fp16(latent * scale) for c < copies."""
    n = latent.numel()
    _need(latent, n, "latent", dtype=torch.float32)
    _need(model_in, copies * n, "model_in")
    call("dlm_scale_latent_fp16", _p(latent), _p(model_in), n, float(scale), int(copies), stream_handle())
