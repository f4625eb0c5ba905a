"""Block-level parity at the SDXL widths (the ResnetBlock2D and
BasicTransformerBlock benchmark shapes), through
the prepared UNet's block runners (the same code the forward runs), against
the fp32 CPU oracle's resnet_block / transformer_block
(oracle/unet_ref.py, restating src/infer/unet.cu:537-797).

- ResnetBlock2D at CFG batch 2: 640 ch @ 64x64, 1280 ch @ 32x32, and
  320 -> 640 @ 64x64 with the 1x1 conv_shortcut; x ~ N(0,1), temb
  2 x 1280 ~ N(0,1) through SiLU and the block's time_emb_proj.
- BasicTransformerBlock on 2 x 4096 x 640 tokens with context 2 x 77 x 2048.
Weights ~ N(0, 0.02^2) (norm scales 1 + N(0, 0.02^2)), drawn on the GPU and
handed to the oracle as the same fp16 values.
"""
import pytest
import torch

from dollama_amd import ops
from dollama_amd import unet as U
from oracle import ref_ops as R
from oracle import unet_ref as OR
from tests._util import assert_close, randn

pytestmark = pytest.mark.gpu

# SDXL widths; one transformer block per Transformer2D keeps the model small
CFG = U.UNetConfig(depth1=1, depth2=1)


@pytest.fixture(scope="module")
def model(gpu):
    W = U.random_weights(CFG, 424242, device="cuda:0")
    net = U.UNet(CFG)
    net.set_weights(W)
    net.prepare()
    yield net, W
    net.close()


def _host(W, prefix):
    return {k: v.float().cpu() for k, v in W.items() if k.startswith(prefix)}


@pytest.mark.parametrize("prefix,Ci,Co,HW", [
    ("down_blocks.1.resnets.1.", 640, 640, 64),
    ("down_blocks.2.resnets.1.", 1280, 1280, 32),
    ("down_blocks.1.resnets.0.", 320, 640, 64),
])
def test_resnet_block_sdxl_shapes(model, prefix, Ci, Co, HW):
    net, W = model
    B = 2
    print(f"[case] ResnetBlock2D {prefix} {Ci}->{Co} @{HW}x{HW} B={B}", flush=True)
    x = randn((B, Ci, HW, HW), 61)
    temb = randn((B, 4 * CFG.C0), 62)
    xg = ops.nchw_to_nhwc(x.half().cuda())
    out = net.run_resnet(prefix, xg, temb.half().cuda())
    got = ops.nhwc_to_nchw(out).float().cpu()
    ref = OR.resnet_block(_host(W, prefix), prefix, x, R.silu(temb))
    assert_close(got, ref, f"resnet {prefix}")


def test_resnet_block_concat_input(model):
    """An up-path resnet: input = concat(current, skip) read from two tensors."""
    net, W = model
    prefix, Ca, Cb, Co, HW, B = "up_blocks.1.resnets.2.", 640, 320, 640, 64, 2
    print(f"[case] ResnetBlock2D {prefix} concat {Ca}+{Cb}->{Co} @{HW}x{HW}", flush=True)
    xa, xb = randn((B, Ca, HW, HW), 63), randn((B, Cb, HW, HW), 64)
    temb = randn((B, 4 * CFG.C0), 65)
    out = net.run_resnet(prefix, ops.nchw_to_nhwc(xa.half().cuda()), temb.half().cuda(),
                         x_b=ops.nchw_to_nhwc(xb.half().cuda()))
    got = ops.nhwc_to_nchw(out).float().cpu()
    ref = OR.resnet_block(_host(W, prefix), prefix, torch.cat([xa, xb], 1), R.silu(temb))
    assert_close(got, ref, f"resnet {prefix} concat")


def test_basic_transformer_block_sdxl_shape(model):
    net, W = model
    prefix = "down_blocks.1.attentions.0.transformer_blocks.0."
    B, S, C, L = 2, 4096, 640, 77
    print(f"[case] BasicTransformerBlock {prefix} [{B},{S},{C}] ctx [{B},{L},2048]", flush=True)
    x = randn((B, S, C), 66)
    ctx = randn((B, L, 2048), 67)
    xg = x.half().cuda().contiguous()
    net.run_transformer_block(prefix, xg, ctx.half().cuda())
    ref = OR.transformer_block(_host(W, prefix), prefix, x, ctx, C // 64)
    assert_close(xg.float().cpu(), ref, "basic transformer block")


def test_block_runner_rejects_unknown_prefix(model):
    net, _ = model
    x = torch.zeros(1, 8, 8, 640, dtype=torch.float16, device="cuda:0")
    with pytest.raises((KeyError, U._lib.DlmError)):
        net.run_resnet("down_blocks.9.resnets.0.", x, torch.zeros(1, 1280, dtype=torch.float16, device="cuda:0"))
    with pytest.raises(U._lib.DlmError):
        net.run_transformer_block("mid_block.attentions.0.transformer_blocks.5.",
                                  torch.zeros(1, 64, 1280, dtype=torch.float16, device="cuda:0"),
                                  torch.zeros(1, 77, 2048, dtype=torch.float16, device="cuda:0"))
