"""Kernels the VAE decoder adds to the dense path, against fp32 references:
fp32-output GEMM (attention scores), row softmax to fp16, conv with fp32
output / fp32 residual, GroupNorm over fp32 input, and the scaled
fp32 -> fp16 cast (bit-exact)."""
import math

import pytest
import torch

from dollama_amd import ops
from oracle import ref_ops as R
from tests._util import assert_close, randn, to_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K", [(512, 1024, 512), (300, 260, 64), (2048, 2048, 512)])
def test_linear_f32out(gpu, M, N, K):
    x = randn((M, K), 1)
    w = randn((N, K), 2, std=1 / math.sqrt(K))
    b = randn((N,), 3, std=0.1)
    r = torch.randn(M, N, generator=torch.Generator().manual_seed(4)) * 1e5
    got = ops.linear_f32out(to_gpu(x), to_gpu(w), bias=to_gpu(b), residual=r.cuda(), alpha=0.5,
                            beta=1.0)
    ref = 0.5 * (x @ w.t()) + b + r
    assert got.dtype == torch.float32
    assert_close(got, ref, f"linear_f32out {M}x{N}x{K} (fp32 residual 1e5)")
    # the part below the residual's magnitude
    assert_close(got.cpu() - r, ref - r, f"linear_f32out {M}x{N}x{K} product part")


@pytest.mark.parametrize("rows,cols", [(64, 1024), (16, 4096), (32, 16384), (8, 20000), (5, 36)])
def test_softmax_rows(gpu, rows, cols):
    s = torch.randn(rows, cols, generator=torch.Generator().manual_seed(cols)) * 8.0
    got = ops.softmax_rows(s.cuda().contiguous())
    ref = torch.softmax(s.double(), dim=-1).float()
    assert_close(got, ref, f"softmax_rows {rows}x{cols}")
    sums = got.float().sum(-1).cpu()
    assert (sums - 1).abs().max() < 2e-2


def test_vae_attention_pipeline_16384(gpu):
    """scores (fp32 GEMM, scale 1/sqrt(512)) -> softmax -> P V at the VAE's
    full mid-block shape S = 16384, Dh = 512, against torch fp32."""
    S, D = 16384, 512
    g = torch.Generator().manual_seed(7)
    q = (torch.randn(S, D, generator=g) * 0.5).half().cuda()
    k = (torch.randn(S, D, generator=g) * 0.5).half().cuda()
    v = torch.randn(S, D, generator=g).half().cuda()
    sc = ops.linear_f32out(q, k, alpha=1 / math.sqrt(D))
    p = ops.softmax_rows(sc)
    del sc
    vt = v.t().contiguous()
    o = ops.linear(p, vt)
    del p
    qf, kf, vf = q.float(), k.float(), v.float()
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        ref = torch.softmax(torch.matmul(qf, kf.t().contiguous()) / math.sqrt(D), dim=-1)
        ref = torch.matmul(ref, vf)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    assert_close(o.float().cpu(), ref.cpu(), "VAE attention S=16384 Dh=512")


@pytest.mark.parametrize("res_f32", [False, True])
def test_conv_f32_out_and_residual(gpu, res_f32):
    N, C, Co, H, W = 1, 128, 192, 24, 20
    x = randn((N, C, H, W), 11)
    w = randn((Co, C, 3, 3), 12, std=1 / math.sqrt(9 * C)) * 4096
    w = w.half().float()
    b = randn((Co,), 13, std=0.1)
    res = torch.randn(N, Co, H, W, generator=torch.Generator().manual_seed(14)) * 3e5
    if not res_f32:
        res = res.clamp(-6e4, 6e4).half().float()
    xg = ops.nchw_to_nhwc(to_gpu(x))
    rg = res.permute(0, 2, 3, 1).contiguous().cuda()
    rg = rg if res_f32 else rg.half()
    y = ops.conv2d_nhwc(xg, ops.pack_conv_weight(to_gpu(w)), KH=3, KW=3, bias=to_gpu(b),
                        residual=rg, out_f32=True)
    assert y.dtype == torch.float32
    ref = R.conv2d(x, w, b) + res
    assert ref.abs().max() > 65504
    assert_close(y.permute(0, 3, 1, 2).cpu(), ref, f"conv3x3 fp32 out, res_f32={res_f32}")


def test_group_norm_f32_input(gpu):
    N, C, H, W = 2, 256, 32, 24
    x = torch.randn(N, C, H, W, generator=torch.Generator().manual_seed(21)) * 2e5 + 7e4
    gm = randn((C,), 22, std=0.1, mean=1.0)
    bt = randn((C,), 23, std=0.1)
    xg = x.permute(0, 2, 3, 1).contiguous().cuda()
    y = ops.group_norm_nhwc(xg, to_gpu(gm), to_gpu(bt), 32, 1e-6, True)
    ref = R.silu(R.group_norm(x, 32, gm, bt, 1e-6))
    assert_close(y.permute(0, 3, 1, 2).float().cpu(), ref, "GroupNorm+SiLU over fp32 input")


def test_cast_f32_to_f16_scaled_exact(gpu):
    x = torch.randn(1000003, generator=torch.Generator().manual_seed(31)) * 1e6
    got = ops.cast_f32_to_f16(x.cuda(), 1.0 / 256).cpu()
    assert torch.equal(got, (x * (1.0 / 256)).half())
