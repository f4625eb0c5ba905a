"""GroupNorm chunk statistics written by a convolution's epilogue
(dlm_conv_nhwc_args::gn_stats) and the GroupNorm that runs from them
(dlm_group_norm_nhwc_prestats_fp16).

The statistics must equal, bit for bit, what the statistics pass
(dlm_group_norm_chunk_stats_fp16) computes on the conv's output, whichever
kernel runs the conv: every DMA tile configuration, split-K, the register
kernels (which leave the statistics to the pass), and outputs whose pixel
count is not a multiple of the 64-pixel chunk.  The GroupNorm that runs from
them must equal the ordinary GroupNorm bit for bit and the float64 oracle
within the fp16 output rounding.
"""
import pytest
import torch

from dollama_amd import _lib, ops
from oracle import ref_ops as R
from tests._util import assert_close, randn, to_gpu

G = 32


def announce(msg):
    print(f"[case] {msg}", flush=True)


def _stats_region(ws, N, C, HW):
    chunks = (HW + 63) // 64
    return ws[: N * chunks * C * 8]


def _conv_case(N, Cin, H, W, Cout, stride, seed):
    x = randn((N, Cin, H, W), seed)
    w = randn((Cout, Cin, 3, 3), seed + 1, std=0.03)
    b = randn((Cout,), seed + 2, std=0.5)
    return ops.nchw_to_nhwc(to_gpu(x)), ops.pack_conv_weight(to_gpu(w)), to_gpu(b), (x, w, b)


@pytest.mark.gpu
@pytest.mark.parametrize("tile", [0] + list(range(1, 8)) + list(range(8, 45)))
def test_conv_gn_stats_equal_stats_pass(gpu, tile):
    """Forced tile `tile` (0: the heuristic; 1-7 register kernels; 8-44 DMA
    tiles), whole and split-K: the epilogue's statistics equal the statistics
    pass's on the same output, bit for bit, and the GroupNorm from them equals
    the ordinary one."""
    N, Cin, Cout = 2, 128, 160
    try:
        _lib.call("dlm_gemm_force_tile", tile)
        for (H, W, stride) in ((16, 16, 1), (32, 24, 2), (12, 10, 1)):
            for splits in (0, 3):
                announce(f"conv gn_stats tile {tile} splits {splits} {H}x{W} stride {stride}")
                _lib.call("dlm_gemm_force_split", splits)
                x, wp, b, _ = _conv_case(N, Cin, H, W, Cout, stride, 300 + H)
                Ho, Wo = (H - 1) // stride + 1, (W - 1) // stride + 1
                HW = Ho * Wo
                ws = ops.group_norm_workspace(N, Cout, HW, gpu)
                ws.zero_()
                y = ops.conv2d_nhwc(x, wp, KH=3, KW=3, stride=stride, bias=b, gn_stats=ws)
                ws2 = ops.group_norm_workspace(N, Cout, HW, gpu)
                ops.group_norm_chunk_stats(y, ws2)
                torch.cuda.synchronize()
                a, c = _stats_region(ws, N, Cout, HW), _stats_region(ws2, N, Cout, HW)
                assert torch.equal(a, c), f"tile {tile} splits {splits} {H}x{W}/{stride}: epilogue statistics differ"
                gm, bt = to_gpu(randn((Cout,), 7, std=0.3, mean=1.0)), to_gpu(randn((Cout,), 8, std=0.3))
                g1 = ops.group_norm_nhwc_prestats(y, gm, bt, G, 1e-5, True, ws)
                g2 = ops.group_norm_nhwc(y, gm, bt, G, 1e-5, True)
                assert torch.equal(g1, g2), f"tile {tile}: GroupNorm from producer statistics differs"
    finally:
        _lib.call("dlm_gemm_force_tile", 0)
        _lib.call("dlm_gemm_force_split", 0)


@pytest.mark.gpu
@pytest.mark.parametrize("tile", [0, 1, 2, 5] + list(range(8, 42)))
def test_linear_gn_stats_equal_stats_pass(gpu, tile):
    """dlm_linear_gn_stats_fp16 (the transformer's proj_out + residual,
    written in place): statistics equal to the pass's on Y, bit for bit, on
    every forced tile, whole and split-K, for 2 samples of 1024 tokens and of
    100 tokens (a partial chunk)."""
    K, Nc = 320, 320
    try:
        _lib.call("dlm_gemm_force_tile", tile)
        for tokens in (1024, 100):
            for splits in (0, 3):
                announce(f"linear gn_stats tile {tile} splits {splits} tokens {tokens}")
                _lib.call("dlm_gemm_force_split", splits)
                M = 2 * tokens
                x, w = to_gpu(randn((M, K), 600)), to_gpu(randn((Nc, K), 601, std=0.05))
                b, r = to_gpu(randn((Nc,), 602, std=0.3)), to_gpu(randn((M, Nc), 603))
                ws = ops.group_norm_workspace(2, Nc, tokens, gpu)
                ws.zero_()
                y = r.clone()
                ops.linear(x, w, bias=b, residual=y, out=y, gn_stats=ws, tokens=tokens)
                ws2 = ops.group_norm_chunk_stats(y.view(2, tokens, 1, Nc), ops.group_norm_workspace(2, Nc, tokens, gpu))
                torch.cuda.synchronize()
                a, c = _stats_region(ws, 2, Nc, tokens), _stats_region(ws2, 2, Nc, tokens)
                assert torch.equal(a, c), f"tile {tile} splits {splits} tokens {tokens}: statistics differ"
                assert_close(y, R.linear(x.float().cpu(), w.float().cpu(), b.float().cpu()) + r.float().cpu(),
                             f"linear in place tile {tile}")
    finally:
        _lib.call("dlm_gemm_force_tile", 0)
        _lib.call("dlm_gemm_force_split", 0)


@pytest.mark.gpu
@pytest.mark.parametrize("N,C,H,W,mean,std", [(2, 320, 128, 128, 0.0, 1.0), (2, 640, 64, 64, 40.0, 0.5),
                                              (1, 1280, 32, 32, -3.0, 2.0), (3, 64, 9, 7, 0.5, 1.5),
                                              (1, 1024, 128, 128, 0.0, 1.0), (1, 1280, 127, 121, 1.0, 1.0)])
def test_group_norm_chunk_statistics_vs_oracle(gpu, N, C, H, W, mean, std):
    """GroupNorm(+SiLU) over the chunk statistics (the path of every fp16
    GroupNorm of up to 16384 pixels) against the float64 oracle on the same
    fp16 values, at the UNet's three level shapes, a mean 80x the standard
    deviation, a pixel count that leaves a partial last chunk, groups of
    exactly as many entries as the merge holds in registers (256 chunks x 32
    channels) and of more (241 chunks x 40 channels); the prestats form from
    the statistics pass gives the same bits."""
    announce(f"group_norm chunk statistics N={N} C={C} {H}x{W} mean {mean} std {std}")
    x = randn((N, C, H, W), 90 + C, std=std, mean=mean)
    gm, bt = randn((C,), 91, std=0.3, mean=1.0), randn((C,), 92, std=0.3)
    xg = ops.nchw_to_nhwc(to_gpu(x))
    y = ops.group_norm_nhwc(xg, to_gpu(gm), to_gpu(bt), G, 1e-5, True)
    ws = ops.group_norm_chunk_stats(xg, ops.group_norm_workspace(N, C, H * W, gpu))
    y2 = ops.group_norm_nhwc_prestats(xg, to_gpu(gm), to_gpu(bt), G, 1e-5, True, ws)
    assert torch.equal(y, y2)
    ref = R.silu(R.group_norm(x.double(), G, gm.double(), bt.double(), 1e-5)).float()
    assert_close(ops.nhwc_to_nchw(y), ref, "group_norm chunk statistics", rel_tol=1e-3, cos_tol=0.999999)


@pytest.mark.gpu
@pytest.mark.parametrize("N,Ca,Cb,H,W,G", [(2, 640, 320, 16, 16, 32), (2, 1280, 640, 8, 8, 32),
                                          (1, 40, 24, 9, 7, 4), (3, 320, 320, 12, 10, 32)])
def test_group_norm_concat_from_two_sources_statistics(gpu, N, Ca, Cb, H, W, G):
    """GroupNorm(+SiLU) over concat(xa, xb) from each source's own chunk
    statistics (dlm_group_norm_nhwc_prestats2_fp16, the UNet's up-path norm1)
    equals the GroupNorm that computes the concatenation's statistics itself,
    bit for bit: UNet level shapes, a group that straddles the two sources
    (40 + 24 channels in groups of 16), and a partial last chunk."""
    announce(f"group_norm concat prestats N={N} Ca={Ca} Cb={Cb} {H}x{W} G={G}")
    xa = ops.nchw_to_nhwc(to_gpu(randn((N, Ca, H, W), 700 + Ca, std=1.5, mean=0.3)))
    xb = ops.nchw_to_nhwc(to_gpu(randn((N, Cb, H, W), 701 + Cb, std=0.7, mean=-2.0)))
    C = Ca + Cb
    gm, bt = to_gpu(randn((C,), 702, std=0.3, mean=1.0)), to_gpu(randn((C,), 703, std=0.3))
    wa = ops.group_norm_chunk_stats(xa, ops.group_norm_workspace(N, Ca, H * W, gpu))
    wb = ops.group_norm_chunk_stats(xb, ops.group_norm_workspace(N, Cb, H * W, gpu))
    for silu in (True, False):
        y1 = ops.group_norm_nhwc_prestats2(xa, xb, gm, bt, G, 1e-5, silu, wa, wb)
        y2 = ops.group_norm_nhwc(xa, gm, bt, G, 1e-5, silu, x_b=xb)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), f"silu={silu}: two-source statistics differ from the pass"


@pytest.mark.gpu
def test_conv_gn_stats_argument_checks(gpu):
    """gn_stats is refused with an NCHW or fp32 output."""
    x, wp, b, _ = _conv_case(1, 64, 8, 8, 64, 1, 500)
    ws = ops.group_norm_workspace(1, 64, 64, gpu)
    with pytest.raises(_lib.DlmError):
        ops.conv2d_nhwc(x, wp, KH=3, KW=3, bias=b, out_nchw=True, gn_stats=ws)
    with pytest.raises(_lib.DlmError):
        ops.conv2d_nhwc(x, wp, KH=3, KW=3, bias=b, out_f32=True, gn_stats=ws)
