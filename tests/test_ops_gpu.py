"""GPU parity of each hot-path kernel against the fp32 CPU oracle.

Every case prints its name and shape before it launches.  Gates: relative
error max|g-r|/max|r| <= 1e-2 and cosine >= 0.9999 (per-op tolerance of this
path), on seeded inputs rounded to fp16 that the oracle sees decoded.
"""
import math

import pytest
import torch

from dollama_amd import ops
from oracle import ref_ops as R
from tests._util import assert_close, from_gpu, randn, to_gpu

pytestmark = pytest.mark.gpu


def announce(msg):
    print(f"[case] {msg}", flush=True)


# ------------------------------------------------------------------ GEMM ---
@pytest.mark.parametrize("M,N,K", [(32, 32, 16), (64, 64, 64), (130, 96, 72), (154, 640, 2048),
                                   (2048, 1280, 1280), (8192, 640, 640), (1000, 40, 64)])
def test_linear_plain(gpu, M, N, K):
    announce(f"linear M={M} N={N} K={K}")
    x = randn((M, K), 1)
    w = randn((N, K), 2, std=0.02 * math.sqrt(640 / K) * 5)
    y = ops.linear(to_gpu(x), to_gpu(w))
    assert_close(y, R.linear(x, w), f"linear {M}x{N}x{K}")


def test_linear_bias_residual_act(gpu):
    M, N, K = 300, 192, 320
    announce(f"linear bias/residual/silu/gelu M={M} N={N} K={K}")
    x, w = randn((M, K), 3), randn((N, K), 4, std=0.05)
    b, r = randn((N,), 5, std=0.1), randn((M, N), 6)
    y = ops.linear(to_gpu(x), to_gpu(w), bias=to_gpu(b), residual=to_gpu(r))
    assert_close(y, R.linear(x, w, b) + r, "linear+bias+residual")
    y = ops.linear(to_gpu(x), to_gpu(w), bias=to_gpu(b), act=ops.ACT_SILU)
    assert_close(y, R.silu(R.linear(x, w, b)), "linear+bias+silu")
    y = ops.linear(to_gpu(x), to_gpu(w), bias=to_gpu(b), act=ops.ACT_GELU)
    assert_close(y, R.gelu_erf(R.linear(x, w, b)), "linear+bias+gelu")


@pytest.mark.parametrize("M,d,K", [(96, 64, 128), (8192, 2560, 640), (2048, 5120, 1280)])
def test_linear_geglu(gpu, M, d, K):
    announce(f"linear geglu M={M} d={d} K={K}")
    x, w = randn((M, K), 7), randn((2 * d, K), 8, std=0.02)
    b = randn((2 * d,), 9, std=0.01)
    wp, bp = ops.pack_geglu(to_gpu(w), to_gpu(b))
    y = ops.linear(to_gpu(x), wp, bias=bp, act=ops.ACT_GEGLU)
    assert y.shape == (M, d)
    assert_close(y, R.geglu(R.linear(x, w, b)), f"geglu {M}x{d}x{K}")


@pytest.mark.parametrize("tile", list(range(8, 45)))
def test_dma_tile_configs(gpu, tile):
    """Every LDS-DMA tile configuration (dlm_gemm_force_tile 8-44, the
    fragment-prefetch forms 27-34, two-slice stages 35-39, the 16-column
    tiles 42-43 and the 192-row tile 44 included),
    whole and split-K, on ragged shapes with an odd slice count and a K tail:
    bias + SiLU + residual, GEGLU, and a 3x3 conv with residual."""
    from dollama_amd import _lib
    announce(f"forced DMA tile {tile}")
    M, N, K = 300, 240, 648  # 11 K slices: odd, with a tail
    x, w = randn((M, K), 13), randn((N, K), 14, std=0.04)
    b, r = randn((N,), 15, std=0.1), randn((M, N), 16)
    ref = R.silu(R.linear(x, w, b)) + r
    wg, bg = randn((2 * 80, K), 17, std=0.04), randn((2 * 80,), 18, std=0.01)
    xc, wc = randn((2, 128, 12, 10), 19), randn((160, 128, 3, 3), 20, std=0.03)
    rc = randn((2, 160, 12, 10), 21)
    try:
        _lib.call("dlm_gemm_force_tile", tile)
        for splits in (0, 3):
            _lib.call("dlm_gemm_force_split", splits)
            y = ops.linear(to_gpu(x), to_gpu(w), bias=to_gpu(b), residual=to_gpu(r), act=ops.ACT_SILU)
            assert_close(y, ref, f"tile {tile} splits {splits} linear+bias+silu+res {M}x{N}x{K}")
            yc = ops.conv2d_nhwc(ops.nchw_to_nhwc(to_gpu(xc)), ops.pack_conv_weight(to_gpu(wc)), KH=3, KW=3,
                                 residual=ops.nchw_to_nhwc(to_gpu(rc)))
            assert_close(ops.nhwc_to_nchw(yc), R.conv2d(xc, wc, None) + rc, f"tile {tile} splits {splits} conv")
        _lib.call("dlm_gemm_force_split", 0)
        wp, bp = ops.pack_geglu(to_gpu(wg), to_gpu(bg))
        yg = ops.linear(to_gpu(x), wp, bias=bp, act=ops.ACT_GEGLU)
        assert_close(yg, R.geglu(R.linear(x, wg, bg)), f"tile {tile} geglu")
    finally:
        _lib.call("dlm_gemm_force_tile", 0)
        _lib.call("dlm_gemm_force_split", 0)


@pytest.mark.parametrize("transA,transB", [(False, True), (False, False), (True, True), (True, False)])
def test_gemm_reference_api(gpu, transA, transB):
    M, N, K = 70, 50, 36
    announce(f"launch_gemm_fp16 transA={transA} transB={transB}")
    A = randn((K, M) if transA else (M, K), 10)
    B = randn((N, K) if transB else (K, N), 11)
    C0 = randn((M, N), 12)
    dA, dB, dC = to_gpu(A), to_gpu(B), to_gpu(C0)
    ops.launch_gemm_fp16(dA, dB, dC, M, N, K, 0.5, 0.25, transA, transB)
    ref = R.gemm(A, B, C0, 0.5, 0.25, transA, transB)
    assert_close(dC, ref, "gemm ref api")


# ------------------------------------------------------------------ conv ---
def test_conv2d_config1_bias_silu(gpu):
    """Single conv 3x3 s1 p1, N=1, 320->320 @128x128 with fused bias+SiLU."""
    N, C, H, W = 1, 320, 128, 128
    announce("conv config1 320->320 @128 bias+silu (NHWC entry)")
    x = randn((N, C, H, W), 20)
    w = randn((C, C, 3, 3), 21, std=0.02)
    b = randn((C,), 22, std=0.01)
    xg = ops.nchw_to_nhwc(to_gpu(x))
    wp = ops.pack_conv_weight(to_gpu(w))
    y = ops.conv2d_nhwc(xg, wp, KH=3, KW=3, bias=to_gpu(b), act=ops.ACT_SILU)
    ref = R.silu(R.conv2d(x, w, b))
    assert_close(ops.nhwc_to_nchw(y), ref, "conv config1 bias+silu")


@pytest.mark.parametrize("N,Cin,H,W,Cout,k,s,p", [
    (1, 320, 128, 128, 320, 3, 1, 1),
    (2, 64, 17, 23, 96, 3, 1, 1),
    (2, 320, 64, 64, 320, 3, 2, 1),
    (2, 640, 32, 32, 1280, 1, 1, 0),
    (1, 3, 9, 11, 5, 3, 1, 1),
    (2, 4, 32, 32, 320, 3, 1, 1),
    (2, 320, 32, 32, 4, 3, 1, 1),
    (1, 16, 8, 8, 16, 5, 2, 2),
])
def test_conv2d_reference_api(gpu, N, Cin, H, W, Cout, k, s, p):
    announce(f"launch_conv2d N={N} Cin={Cin} {H}x{W} Cout={Cout} k={k} s={s} p={p}")
    x = randn((N, Cin, H, W), 30)
    w = randn((Cout, Cin, k, k), 31, std=1.0 / math.sqrt(Cin * k * k))
    b = randn((Cout,), 32, std=0.1)
    Ho = (H + 2 * p - k) // s + 1
    Wo = (W + 2 * p - k) // s + 1
    out = torch.empty(N, Cout, Ho, Wo, dtype=torch.float16, device=gpu)
    ops.launch_conv2d(to_gpu(x), to_gpu(w), to_gpu(b), out, N, Cin, H, W, Cout, k, k, s, s, p, p, 1, 1)
    assert_close(out, R.conv2d(x, w, b, s, p), "launch_conv2d")


@pytest.mark.parametrize("N,Cin,H,W,Cout,KH,KW,sh,sw,ph,pw,dh,dw", [
    (1, 320, 64, 64, 320, 3, 3, 1, 1, 2, 2, 2, 2),      # channel-aligned (LDS-DMA) path
    (2, 128, 33, 31, 64, 3, 3, 2, 1, 3, 1, 3, 1),       # anisotropic, dilated
    (2, 64, 17, 23, 96, 3, 5, 1, 2, 1, 4, 2, 2),        # KH != KW
    (1, 4, 20, 18, 8, 3, 3, 2, 1, 1, 0, 1, 3),          # small-channel (generic loader) path
    (2, 3, 9, 11, 5, 3, 3, 1, 1, 0, 0, 4, 4),           # dilation larger than the padding
])
def test_conv2d_reference_api_geometry(gpu, N, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, dh, dw):
    """Per-axis stride / pad and dilation of launch_conv2d (src/kernels/conv2d.cu:88-164)."""
    announce(f"launch_conv2d geometry N={N} Cin={Cin} {H}x{W} Cout={Cout} k={KH}x{KW} "
             f"s=({sh},{sw}) p=({ph},{pw}) d=({dh},{dw})")
    x = randn((N, Cin, H, W), 33)
    w = randn((Cout, Cin, KH, KW), 34, std=1.0 / math.sqrt(Cin * KH * KW))
    b = randn((Cout,), 35, std=0.1)
    Ho = (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1
    Wo = (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1
    out = torch.empty(N, Cout, Ho, Wo, dtype=torch.float16, device=gpu)
    ops.launch_conv2d(to_gpu(x), to_gpu(w), to_gpu(b), out, N, Cin, H, W, Cout, KH, KW,
                      sh, sw, ph, pw, dh, dw)
    assert_close(out, R.conv2d(x, w, b, (sh, sw), (ph, pw), (dh, dw)), "launch_conv2d geometry")


def test_conv_nhwc_concat_shortcut_residual_tbias(gpu):
    """ResnetBlock2D conv2 form: 3x3 over h, fused 1x1 shortcut over concat(x_a, x_b),
    per-(n,c) time bias."""
    N, H, W = 2, 16, 16
    Ca, Cb, Cout = 128, 64, 128
    announce("conv nhwc 3x3 + fused 1x1 shortcut over concat + tbias")
    h = randn((N, Cout, H, W), 40)
    xa, xb = randn((N, Ca, H, W), 41), randn((N, Cb, H, W), 42)
    w2 = randn((Cout, Cout, 3, 3), 43, std=0.03)
    wsc = randn((Cout, Ca + Cb, 1, 1), 44, std=0.05)
    b = randn((Cout,), 45, std=0.1)
    tb = randn((N, Cout), 46, std=0.5)
    K0 = 9 * Cout
    wp = torch.zeros(Cout, K0 + Ca + Cb, dtype=torch.float16, device=gpu)
    ops.pack_conv_weight(to_gpu(w2), out=wp, ld=wp.shape[1], col0=0)
    ops.pack_conv_weight(to_gpu(wsc), out=wp, ld=wp.shape[1], col0=K0)
    y = ops.conv2d_nhwc(ops.nchw_to_nhwc(to_gpu(h)), wp, KH=3, KW=3, bias=to_gpu(b),
                        tbias=to_gpu(tb), shortcut=ops.nchw_to_nhwc(to_gpu(xa)),
                        shortcut_b=ops.nchw_to_nhwc(to_gpu(xb)))
    xc = torch.cat([xa, xb], 1)
    ref = R.conv2d(h, w2, b) + tb[:, :, None, None] + R.conv2d(xc, wsc, None, 1, 0)
    assert_close(ops.nhwc_to_nchw(y), ref, "conv+shortcut+tbias")


def test_conv_nhwc_concat_upsample_residual(gpu):
    N, H, W, Ca, Cb, Cout = 2, 8, 12, 64, 128, 64
    announce("conv nhwc concat input + nearest2x upsample + residual")
    xa, xb = randn((N, Ca, H, W), 50), randn((N, Cb, H, W), 51)
    w = randn((Cout, Ca + Cb, 3, 3), 52, std=0.03)
    b = randn((Cout,), 53, std=0.1)
    res = randn((N, Cout, 2 * H, 2 * W), 54)
    wp = ops.pack_conv_weight(to_gpu(w))
    y = ops.conv2d_nhwc(ops.nchw_to_nhwc(to_gpu(xa)), wp, KH=3, KW=3, bias=to_gpu(b),
                        x_b=ops.nchw_to_nhwc(to_gpu(xb)), upsample=True,
                        residual=ops.nchw_to_nhwc(to_gpu(res)))
    xc = R.upsample_nearest2x(torch.cat([xa, xb], 1))
    assert_close(ops.nhwc_to_nchw(y), R.conv2d(xc, w, b) + res, "conv concat+upsample+res")


def test_conv_out_nchw_small_cout(gpu):
    N, C, H, W = 2, 320, 32, 32
    announce("conv nhwc -> nchw out, Cout=4")
    x = randn((N, C, H, W), 60)
    w = randn((4, C, 3, 3), 61, std=0.02)
    b = randn((4,), 62, std=0.1)
    y = ops.conv2d_nhwc(ops.nchw_to_nhwc(to_gpu(x)), ops.pack_conv_weight(to_gpu(w)), KH=3, KW=3,
                        bias=to_gpu(b), out_nchw=True)
    assert_close(y, R.conv2d(x, w, b), "conv_out nchw")


@pytest.mark.parametrize("Cin,cin_pad,k", [(128, 128, 3), (120, 128, 3), (72, 72, 3), (4, 8, 3), (320, 320, 1)])
def test_conv_weight_pack_layout(gpu, Cin, cin_pad, k):
    """dlm_conv_weight_pack_fp16's column order as include/dlm.h states it:
    [Cin_pad/64][KH][KW][64] when Cin_pad % 64 == 0, else [KH][KW][Cin_pad];
    zero padding channels."""
    announce(f"conv weight pack Cin={Cin} pad={cin_pad} k={k}")
    w = randn((16, Cin, k, k), 90)
    got = ops.pack_conv_weight(to_gpu(w), cin_pad=cin_pad).float().cpu()
    taps = k * k
    wt = w.reshape(16, Cin, taps)
    ref = torch.zeros(16, taps * cin_pad)
    for ci in range(Cin):
        for t in range(taps):
            col = ((ci // 64) * taps + t) * 64 + ci % 64 if cin_pad % 64 == 0 else t * cin_pad + ci
            ref[:, col] = wt[:, ci, t]
    assert torch.equal(got, ref)


# ------------------------------------------------------------- GroupNorm ---
@pytest.mark.parametrize("N,C,H,W,G,eps,silu", [
    (2, 640, 64, 64, 32, 1e-5, True),
    (2, 1280, 32, 32, 32, 1e-6, False),
    (2, 320, 128, 128, 32, 1e-5, True),
    (1, 64, 7, 9, 8, 1e-5, False),
])
def test_group_norm_reference_api(gpu, N, C, H, W, G, eps, silu):
    announce(f"launch_group_norm{'_silu' if silu else ''} N={N} C={C} {H}x{W} G={G}")
    x = randn((N, C, H, W), 70, std=2.0, mean=0.5)
    gm, bt = randn((C,), 71, std=0.5, mean=1.0), randn((C,), 72, std=0.5)
    out = torch.empty(N, C, H, W, dtype=torch.float16, device=gpu)
    fn = ops.launch_group_norm_silu if silu else ops.launch_group_norm
    fn(to_gpu(x), to_gpu(gm), to_gpu(bt), out, N, C, H, W, G, eps)
    ref = R.group_norm(x, G, gm, bt, eps)
    if silu:
        ref = R.silu(ref)
    assert_close(out, ref, "group_norm")


def test_group_norm_nhwc_concat(gpu):
    N, H, W, Ca, Cb, G = 2, 32, 32, 1280, 640, 32
    announce("group_norm nhwc over concat 1280+640")
    xa, xb = randn((N, Ca, H, W), 80), randn((N, Cb, H, W), 81, std=3.0)
    gm, bt = randn((Ca + Cb,), 82, std=0.3, mean=1.0), randn((Ca + Cb,), 83, std=0.3)
    y = ops.group_norm_nhwc(ops.nchw_to_nhwc(to_gpu(xa)), to_gpu(gm), to_gpu(bt), G, 1e-5, True,
                            x_b=ops.nchw_to_nhwc(to_gpu(xb)))
    ref = R.silu(R.group_norm(torch.cat([xa, xb], 1), G, gm, bt, 1e-5))
    assert_close(ops.nhwc_to_nchw(y), ref, "group_norm nhwc concat")


def test_group_norm_large_offset(gpu):
    """Mean 40 against std 0.5 (a ratio of 80): the chunk statistics must be
    combined without cancellation (E[x^2] - mean^2 in fp32 would lose about
    four digits here); the reference runs in float64 on the same fp16 values.
    A second call on the same input gives the same bits."""
    N, C, H, W, G = 2, 640, 64, 64, 32
    announce("group_norm nhwc, mean 40 / std 0.5")
    x = randn((N, C, H, W), 84, std=0.5, mean=40.0)
    gm, bt = randn((C,), 85, std=0.3, mean=1.0), randn((C,), 86, std=0.3)
    xg = ops.nchw_to_nhwc(to_gpu(x))
    y = ops.group_norm_nhwc(xg, to_gpu(gm), to_gpu(bt), G, 1e-5, False)
    y2 = ops.group_norm_nhwc(xg, to_gpu(gm), to_gpu(bt), G, 1e-5, False)
    assert torch.equal(y, y2)
    ref = R.group_norm(x.double(), G, gm.double(), bt.double(), 1e-5).float()
    assert_close(ops.nhwc_to_nchw(y), ref, "group_norm large offset")


def test_group_norm_many_samples(gpu):
    """A batch of 4100 small samples: one statistics chunk per sample, one
    merge wave per (sample, group)."""
    N, C, H, W, G = 4100, 16, 3, 3, 4
    announce("group_norm nhwc, N=4100")
    x = randn((N, C, H, W), 87, std=1.5, mean=-0.5)
    gm, bt = randn((C,), 88, std=0.3, mean=1.0), randn((C,), 89, std=0.3)
    y = ops.group_norm_nhwc(ops.nchw_to_nhwc(to_gpu(x)), to_gpu(gm), to_gpu(bt), G, 1e-5, True)
    ref = R.silu(R.group_norm(x, G, gm, bt, 1e-5))
    assert_close(ops.nhwc_to_nchw(y), ref, "group_norm many samples")


# ------------------------------------------------------------- LayerNorm ---
@pytest.mark.parametrize("rows,C", [(8192, 640), (2048, 1280), (77, 2048), (5, 100), (13, 520), (3, 8), (6, 1032)])
def test_layer_norm(gpu, rows, C):
    announce(f"launch_layer_norm rows={rows} C={C}")
    x = randn((rows, C), 90, std=1.5, mean=0.3)
    gm, bt = randn((C,), 91, std=0.3, mean=1.0), randn((C,), 92, std=0.3)
    out = torch.empty(rows, C, dtype=torch.float16, device=gpu)
    ops.launch_layer_norm(to_gpu(x), to_gpu(gm), to_gpu(bt), out, rows, C, 1e-5)
    assert_close(out, R.layer_norm(x, gm, bt, 1e-5), "layer_norm")


# ------------------------------------------------------------- attention ---
@pytest.mark.parametrize("B,H,Sq,Sk", [(1, 1, 32, 64), (1, 2, 100, 33), (2, 10, 4096, 4096),
                                       (2, 20, 1024, 1024), (2, 10, 4096, 77), (2, 20, 1024, 77)])
def test_attention_reference_api(gpu, B, H, Sq, Sk):
    Dh = 64
    announce(f"launch_attention B={B} H={H} Sq={Sq} Sk={Sk}")
    q, k, v = randn((B, H, Sq, Dh), 100), randn((B, H, Sk, Dh), 101), randn((B, H, Sk, Dh), 102)
    out = torch.empty(B, H, Sq, Dh, dtype=torch.float16, device=gpu)
    ops.launch_attention(to_gpu(q), to_gpu(k), to_gpu(v), out, B, H, Sq, Sk, Dh, 1.0 / 8.0)
    ref = torch.cat([R.attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], 1.0 / 8.0) for b in range(B)])
    assert_close(out, ref, "attention")


@pytest.mark.parametrize("B,H,Sq,Sk,Dh", [(1, 2, 100, 33, 40), (2, 3, 257, 77, 80), (1, 1, 1024, 1024, 512),
                                          (2, 2, 65, 129, 20), (1, 3, 48, 5, 128), (2, 1, 96, 96, 8),
                                          (1, 1, 300, 1, 36)])
def test_attention_reference_api_any_head_dim(gpu, B, H, Sq, Sk, Dh):
    """launch_attention for head dims other than 64 (src/kernels/attention.cu:602-700 accepts
    any Dh; the VAE mid block uses Dh = 512): odd key counts, Dh not a multiple of 8, Sk = 1."""
    announce(f"launch_attention B={B} H={H} Sq={Sq} Sk={Sk} Dh={Dh}")
    q, k, v = randn((B, H, Sq, Dh), 103), randn((B, H, Sk, Dh), 104), randn((B, H, Sk, Dh), 105)
    scale = 1.0 / math.sqrt(Dh)
    out = torch.empty(B, H, Sq, Dh, dtype=torch.float16, device=gpu)
    ops.launch_attention(to_gpu(q), to_gpu(k), to_gpu(v), out, B, H, Sq, Sk, Dh, scale)
    ref = torch.cat([R.attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], scale) for b in range(B)])
    assert_close(out, ref, f"attention Dh={Dh}")


def test_attention_reference_api_unaligned(gpu):
    """Q / K / V / O that start 2 bytes into their allocation take the general path."""
    B, H, Sq, Sk, Dh = 1, 2, 70, 45, 64
    announce("launch_attention unaligned operands")
    q, k, v = randn((B, H, Sq, Dh), 106), randn((B, H, Sk, Dh), 107), randn((B, H, Sk, Dh), 108)
    def shifted(t):
        buf = torch.zeros(t.numel() + 1, dtype=torch.float16, device=gpu)
        buf[1:] = t.reshape(-1).to(torch.float16)
        return buf[1:]
    out_buf = torch.zeros(B * H * Sq * Dh + 1, dtype=torch.float16, device=gpu)
    out = out_buf[1:]
    ops.launch_attention(shifted(q), shifted(k), shifted(v), out, B, H, Sq, Sk, Dh, 0.125)
    ref = R.attention(q, k, v, 0.125)
    assert_close(out.reshape(B, H, Sq, Dh), ref, "attention unaligned")


def test_attention_strided_fused_qkv(gpu):
    """Q/K/V read in place from a fused [B, S, 3C] projection, O written to [B, S, C]."""
    B, S, Hh, Dh = 2, 256, 4, 64
    C = Hh * Dh
    announce("attention strided fused qkv")
    qkv = randn((B, S, 3 * C), 110)
    dq = to_gpu(qkv)
    o = torch.empty(B, S, C, dtype=torch.float16, device=gpu)
    st = (S * 3 * C, 3 * C, Dh)
    ops.attention_strided(dq, dq[:, :, C:], dq[:, :, 2 * C:], o, B=B, H=Hh, Sq=S, Sk=S,
                          q_strides=st, k_strides=st, v_strides=st, o_strides=(S * C, C, Dh),
                          scale=0.125)
    def heads(t):
        return t.reshape(B, S, Hh, Dh).permute(0, 2, 1, 3).contiguous()
    ref = R.attention(heads(qkv[:, :, :C]), heads(qkv[:, :, C:2 * C]), heads(qkv[:, :, 2 * C:]), 0.125)
    ref = ref.permute(0, 2, 1, 3).reshape(B, S, C)
    assert_close(o, ref, "attention strided")


@pytest.mark.parametrize("B,H,Sq,Sk", [(1, 1, 32, 64), (1, 2, 300, 136), (2, 10, 4096, 4096),
                                       (2, 20, 1024, 1024), (1, 3, 1000, 8), (2, 10, 4096, 77),
                                       (2, 20, 1024, 77), (1, 2, 64, 5), (1, 2, 70, 96), (2, 1, 40, 32),
                                       (2, 1, 33, 1), (1, 2, 130, 97)])
def test_attention_vt(gpu, B, H, Sq, Sk):
    """Flash attention over V^T [B, H, 64, Sk] with Q/K read from a fused
    [B, S, 2C] buffer; partial last key tiles, Sq not a multiple of the
    query block, both query-block widths, and short key sets (one, two and three
    32-key blocks, full and partial, Sk = 1) are covered."""
    Dh = 64
    C = H * Dh
    announce(f"attention_vt B={B} H={H} Sq={Sq} Sk={Sk}")
    q, k, v = randn((B, H, Sq, Dh), 120), randn((B, H, Sk, Dh), 121), randn((B, H, Sk, Dh), 122)
    dq = to_gpu(q.permute(0, 2, 1, 3).reshape(B, Sq, C))
    dk = to_gpu(k.permute(0, 2, 1, 3).reshape(B, Sk, C))
    ld = (Sk + 7) // 8 * 8
    vt = torch.zeros(B, H, Dh, ld, dtype=torch.float16, device=gpu)  # [B, H, 64, ld], zero padded
    vt[..., :Sk] = to_gpu(v.transpose(2, 3).contiguous())
    o = torch.empty(B, Sq, C, dtype=torch.float16, device=gpu)
    ops.attention_vt(dq, dk, vt, o, B=B, H=H, Sq=Sq, Sk=Sk, q_strides=(Sq * C, C, Dh),
                     k_strides=(Sk * C, C, Dh), vt_strides=(H * Dh * ld, Dh * ld), vt_ld=ld,
                     o_strides=(Sq * C, C, Dh), scale=0.125)
    ref = torch.cat([R.attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], 0.125) for b in range(B)])
    assert_close(o, ref.permute(0, 2, 1, 3).reshape(B, Sq, C), "attention_vt")


@pytest.mark.parametrize("mode,B,H,Sq,Sk", [("wide", 2, 4, 1024, 1024), ("wide", 1, 2, 130, 97),
                                            ("negative", 2, 4, 1024, 1024), ("negative", 1, 2, 300, 77),
                                            ("negative", 1, 2, 130, 33), ("growing", 1, 2, 256, 1000)])
def test_attention_vt_rebase_paths(gpu, mode, B, H, Sq, Sk):
    """The flash kernel's running base in the online softmax: scores with a
    spread of ~11 in the exponent's units (the base moves whenever a tile's
    max passes it by more than 2^8), scores that are all far below 0 (the
    first tile moves the base down, or every p would underflow in fp16),
    and keys whose scores grow along the sequence (a move on many tiles).
    Same bar as every attention case."""
    Dh = 64
    C = H * Dh
    announce(f"attention_vt rebase {mode} B={B} H={H} Sq={Sq} Sk={Sk}")
    q, k, v = randn((B, H, Sq, Dh), 130), randn((B, H, Sk, Dh), 131), randn((B, H, Sk, Dh), 132)
    if mode == "wide":
        q = (q * 8).half().float()
    elif mode == "negative":
        q = (1.0 + 0.1 * q).half().float()
        k = (-1.5 + 0.3 * k).half().float()
    else:  # key j's score against a query grows like 2 j / Sk in raw units
        q = (0.5 + 0.1 * q).half().float()
        k = (torch.linspace(0.0, 2.0, Sk).reshape(1, 1, Sk, 1) + 0.1 * k).half().float()
    dq = to_gpu(q.permute(0, 2, 1, 3).reshape(B, Sq, C))
    dk = to_gpu(k.permute(0, 2, 1, 3).reshape(B, Sk, C))
    ld = (Sk + 7) // 8 * 8
    vt = torch.zeros(B, H, Dh, ld, dtype=torch.float16, device=gpu)
    vt[..., :Sk] = to_gpu(v.transpose(2, 3).contiguous())
    o = torch.empty(B, Sq, C, dtype=torch.float16, device=gpu)
    ops.attention_vt(dq, dk, vt, o, B=B, H=H, Sq=Sq, Sk=Sk, q_strides=(Sq * C, C, Dh),
                     k_strides=(Sk * C, C, Dh), vt_strides=(H * Dh * ld, Dh * ld), vt_ld=ld,
                     o_strides=(Sq * C, C, Dh), scale=0.125)
    ref = torch.cat([R.attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], 0.125) for b in range(B)])
    assert_close(o, ref.permute(0, 2, 1, 3).reshape(B, Sq, C), f"attention_vt {mode}")


@pytest.mark.parametrize("mode", ["first", "late", "spike"])
@pytest.mark.parametrize("B,H,Sq,Sk", [(1, 2, 1024, 1024), (1, 64, 1024, 1024), (1, 2, 300, 333)])
def test_attention_vt_overflow_rebase(gpu, mode, B, H, Sq, Sk):
    """The flash kernel's base moves only when some p = 2^(s - m) of a tile
    would overflow fp16 (s - m >= 16 in the exponent's units): scores whose
    first tile already overflows (Q x 16: a spread of ~23 per score), keys whose scores
    grow by ~35 along the sequence (the base moves up on many tiles), and one
    key in a late tile whose score jumps ~40 above all others.  Both
    query-block widths (2 heads: 64-query workgroups; 64 heads: 128-query
    workgroups) and a partial last tile.  Same bar as every attention case."""
    Dh = 64
    C = H * Dh
    announce(f"attention_vt overflow rebase {mode} B={B} H={H} Sq={Sq} Sk={Sk}")
    q, k, v = randn((B, H, Sq, Dh), 150), randn((B, H, Sk, Dh), 151), randn((B, H, Sk, Dh), 152)
    if mode == "first":
        q = (q * 16).half().float()
    elif mode == "late":  # key j's score grows like 24 j / Sk in raw units (~35 in log2 units)
        q = (0.5 + 0.1 * q).half().float()
        k = (torch.linspace(0.0, 6.0, Sk).reshape(1, 1, Sk, 1) + 0.1 * k).half().float()
    else:  # key 3 Sk / 4 aligned with every query: raw score ~28 above the rest
        q = (0.5 + 0.1 * q).half().float()
        j = 3 * Sk // 4
        k[:, :, j, :] = 7.0
        k = k.half().float()
    dq = to_gpu(q.permute(0, 2, 1, 3).reshape(B, Sq, C))
    dk = to_gpu(k.permute(0, 2, 1, 3).reshape(B, Sk, C))
    ld = (Sk + 7) // 8 * 8
    vt = torch.zeros(B, H, Dh, ld, dtype=torch.float16, device=gpu)
    vt[..., :Sk] = to_gpu(v.transpose(2, 3).contiguous())
    o = torch.empty(B, Sq, C, dtype=torch.float16, device=gpu)
    ops.attention_vt(dq, dk, vt, o, B=B, H=H, Sq=Sq, Sk=Sk, q_strides=(Sq * C, C, Dh),
                     k_strides=(Sk * C, C, Dh), vt_strides=(H * Dh * ld, Dh * ld), vt_ld=ld,
                     o_strides=(Sq * C, C, Dh), scale=0.125)
    assert torch.isfinite(o).all(), f"attention_vt overflow {mode}: non-finite output"
    ref = torch.cat([R.attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], 0.125) for b in range(B)])
    assert_close(o, ref.permute(0, 2, 1, 3).reshape(B, Sq, C), f"attention_vt overflow {mode}")


@pytest.mark.parametrize("M,N,K,act,vt", [
    (2048, 1280, 1280, 0, False), (8192, 640, 640, 0, False), (2048, 3840, 1280, 0, True),
    (8192, 1920, 640, 0, True), (2048, 10240, 1280, 4, False), (8192, 5120, 640, 4, False),
    (300, 96, 192, 0, False), (130, 160, 128, 4, False)])
def test_linear_layernorm_folded(gpu, M, N, K, act, vt):
    """LayerNorm folded into the consuming linear (the UNet's QKV, cross-Q and
    GEGLU shapes, plus ragged ones): gamma in the weight columns, per-row
    statistics accumulated inside the GEMM, against LayerNorm then linear in
    fp32 on the CPU.  Rows carry an offset (mean 0.5, std 2)."""
    act = ops.ACT_GEGLU if act == 4 else ops.ACT_NONE
    announce(f"linear_ln M={M} N={N} K={K} act={act} vt={vt}")
    x = randn((M, K), 140, std=2.0, mean=0.5)
    g, b = randn((K,), 141, std=0.3, mean=1.0), randn((K,), 142, std=0.3)
    w, bias = randn((N, K), 143, std=0.04), randn((N,), 144, std=0.1)
    ref = R.linear(R.layer_norm(x, g, b, 1e-5), w, bias)
    wg, bg = to_gpu(w), to_gpu(bias)
    if act == ops.ACT_GEGLU:
        wg, bg = ops.pack_geglu(wg, bg)
        ref = R.geglu(ref)
    wf, c1, c2 = ops.ln_fold(wg, to_gpu(g), to_gpu(b), bg)
    if vt:
        C = N // 3
        y, vtt = ops.linear_vt_ln(to_gpu(x), wf, c1, c2, 1e-5, 2 * C, 1024)
        assert_close(y, ref[:, :2 * C], "linear_vt_ln y")
        assert_close(vtt, ref[:, 2 * C:].reshape(M // 1024, 1024, C).transpose(1, 2), "linear_vt_ln vt")
    else:
        y = ops.linear_ln(to_gpu(x), wf, c1, c2, 1e-5, act=act)
        assert_close(y, ref, "linear_ln")


def test_linear_layernorm_folded_large_offset(gpu):
    """Rows with mean 40 and std 0.5: the one-pass fp32 statistics (as the
    reference's LayerNorm) stay accurate; residual and beta in the epilogue."""
    M, N, K = 1024, 640, 640
    announce("linear_ln mean 40 / std 0.5, residual")
    x = randn((M, K), 145, std=0.5, mean=40.0)
    g, b = randn((K,), 146, std=0.3, mean=1.0), randn((K,), 147, std=0.3)
    w, bias = randn((N, K), 148, std=0.04), randn((N,), 149, std=0.1)
    r = randn((M, N), 150)
    ref = R.linear(R.layer_norm(x.double(), g.double(), b.double(), 1e-5), w.double(), bias.double()).float() + 0.5 * r
    wf, c1, c2 = ops.ln_fold(to_gpu(w), to_gpu(g), to_gpu(b), to_gpu(bias))
    y = ops.linear_ln(to_gpu(x), wf, c1, c2, 1e-5, residual=to_gpu(r), beta=0.5)
    assert_close(y, ref, "linear_ln large offset")


@pytest.mark.parametrize("B,S,C,ld", [(2, 1024, 1280, 1024), (2, 64, 128, 64), (3, 40, 192, 40),
                                      (2, 77, 640, 80)])
def test_linear_vt(gpu, B, S, C, ld):
    """Fused QKV projection writing Q|K row-major and V transposed per sample,
    V^T rows padded to `ld` with zeros."""
    announce(f"linear_vt B={B} S={S} C={C} ld={ld}")
    x, w, b = randn((B * S, C), 130), randn((3 * C, C), 131, 0.05), randn((3 * C,), 132, 0.1)
    y, vt = ops.linear_vt(to_gpu(x), to_gpu(w), 2 * C, S, bias=to_gpu(b), vt_ld=ld)
    ref = R.linear(x, w, b)
    assert_close(y, ref[:, :2 * C], "linear_vt y")
    assert_close(vt[:, :, :S], ref[:, 2 * C:].reshape(B, S, C).transpose(1, 2), "linear_vt vt")
    assert bool((vt[:, :, S:] == 0).all())


# ------------------------------------------------------------ small ops ---
def test_elementwise_ops(gpu):
    announce("silu/gelu/add/upsample/bias/geglu")
    n = 10007
    a, b = randn((n,), 120, std=3.0), randn((n,), 121)
    out = torch.empty(n, dtype=torch.float16, device=gpu)
    ops.launch_silu(to_gpu(a), out, n)
    assert_close(out, R.silu(a), "silu")
    ops.launch_gelu(to_gpu(a), out, n)
    assert_close(out, R.gelu_erf(a), "gelu")
    ops.launch_gelu_tanh(to_gpu(a), out, n)
    assert_close(out, R.gelu_tanh(a), "gelu_tanh")
    inplace = to_gpu(a)
    ops.launch_gelu_tanh(inplace, inplace, n)
    assert torch.equal(inplace, out), "gelu_tanh in place"
    ops.launch_add(to_gpu(a), to_gpu(b), out, n)
    assert_close(out, a + b, "add")
    x = randn((2, 3, 5, 7), 122)
    up = torch.empty(2, 3, 10, 14, dtype=torch.float16, device=gpu)
    ops.launch_upsample_nearest2x(to_gpu(x), up, 2, 3, 5, 7)
    assert torch.equal(from_gpu(up), R.upsample_nearest2x(x))
    t, C = 33, 48
    x, bias = randn((t, C), 123), randn((C,), 124)
    o2 = torch.empty(t, C, dtype=torch.float16, device=gpu)
    ops.launch_bias_add_rowvec(to_gpu(x), to_gpu(bias), o2, t, C)
    assert_close(o2, x + bias, "bias rowvec")
    h = randn((t, 2 * C), 125)
    o3 = torch.empty(t, C, dtype=torch.float16, device=gpu)
    ops.launch_geglu(to_gpu(h), o3, t, C)
    assert_close(o3, R.geglu(h), "geglu standalone")
    x4, cb, tp, rs = randn((2, 8, 4, 4), 126), randn((8,), 127), randn((2, 8), 128), randn((2, 8, 4, 4), 129)
    o4 = torch.empty(2, 8, 4, 4, dtype=torch.float16, device=gpu)
    ops.launch_conv_bias_biasch(to_gpu(x4), to_gpu(cb), to_gpu(tp), o4, 2, 8, 4, 4)
    assert_close(o4, x4 + cb[None, :, None, None] + tp[:, :, None, None], "conv_bias_biasch")
    ops.launch_conv_bias_residual(to_gpu(x4), to_gpu(cb), to_gpu(rs), o4, 2, 8, 4, 4)
    assert_close(o4, x4 + cb[None, :, None, None] + rs, "conv_bias_residual")
    ops.launch_bias_add_channel(to_gpu(x4), to_gpu(cb), o4, 2, 8, 4, 4)
    assert_close(o4, x4 + cb[None, :, None, None], "bias channel")


def test_timestep_and_sdxl_embeddings(gpu):
    announce("timestep embedding / sdxl embed inputs")
    out = torch.empty(320, dtype=torch.float16, device=gpu)
    ops.launch_timestep_embedding(out, 999.0, 320)
    ref = R.timestep_embedding(torch.tensor([999.0]), 320)[0]
    assert (from_gpu(out) - ref).abs().max() < 2e-3
    B = 2
    ts = torch.full((B,), 999.0, dtype=torch.float32, device=gpu)
    text = randn((B, 1280), 130)
    ids = torch.tensor([1024, 1024, 0, 0, 1024, 1024], dtype=torch.float32)
    t_emb, add_in = ops.sdxl_embed_inputs(ts, to_gpu(text), to_gpu(ids))
    assert (from_gpu(t_emb) - R.timestep_embedding(torch.full((B,), 999.0), 320)).abs().max() < 2e-3
    assert (from_gpu(add_in) - R.add_embedding_input(text, ids)).abs().max() < 2e-3


@pytest.mark.parametrize("M", [1, 3, 5, 16])
def test_linear_small_row_bounds(gpu, M):
    """Every row bound of the skinny linear (rows padded to 2, 4, 8, 16 load
    the last real row, never stored), with a column count that leaves the
    last block's waves partly idle, and the accumulate form."""
    announce(f"linear_small M={M}")
    x, w, b = randn((M, 520), 150 + M), randn((37, 520), 151, std=0.05), randn((37,), 152, std=0.01)
    y = ops.linear_small(to_gpu(x), to_gpu(w), to_gpu(b))
    assert_close(y, R.linear(x, w, b), f"linear_small M={M}")
    base = randn((M, 37), 153)
    y2 = to_gpu(base)
    ops.linear_small(to_gpu(x), to_gpu(w), to_gpu(b), out=y2, accumulate=True)
    assert_close(y2, R.linear(x, w, b) + base.half().float(), f"linear_small M={M} accumulate")


def test_linear_small(gpu):
    announce("linear_small M=2")
    x, w, b = randn((2, 2816), 140), randn((1280, 2816), 141, std=0.02), randn((1280,), 142, std=0.01)
    y = ops.linear_small(to_gpu(x), to_gpu(w), to_gpu(b), act=ops.ACT_SILU)
    assert_close(y, R.silu(R.linear(x, w, b)), "linear_small silu")
    y = ops.linear_small(to_gpu(x[:, :1280]), to_gpu(w[:, :1280].contiguous()), to_gpu(b), silu_in=True)
    assert_close(y, R.linear(R.silu(x[:, :1280]), w[:, :1280], b), "linear_small silu_in")
