"""Pins the CPU oracle (CPU only, no GPU).

Each oracle function is checked three ways:
  1. the torch restatement (oracle/ref_ops.py) against the independent plain-C
     restatement of the reference's own CPU test references (oracle/naive.c);
  2. known answers: the reference tests' hand-computed cases
     (src/tests/test_groupnorm.cu:236-299, test_layernorm.cu:205-262,
     test_geglu.cu:130-160, test_activation.cu:183-260,
     test_timeembed.cu:99-124) and closed forms;
  3. invariants that a plausible mistake (a dropped term, a transposed
     operand, a wrong index or sign) would break: delta-kernel convolution,
     1x1 conv == GEMM, equal keys -> mean(V), key-permutation invariance,
     shift invariance of the normalisations.
The Euler schedule is also compared with the reference's own scheduler
header compiled by oracle/Makefile (oracle/_ref/sched_ref) when that binary
exists, and the UNet parameter list with the reference's published count
(docs/measurements-log.md:40, 2.57 B) and the product's own C++ list.
"""
import math
import os
import subprocess

import numpy as np
import pytest
import torch

from oracle import metrics, naive
from oracle import ref_ops as R
from oracle import unet_ref as OR

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return R.to_fp16_grid(torch.randn(*shape, generator=g) * scale)


def _close(a, b, tol=2e-5):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = max(np.abs(b).max(), 1e-6)
    err = np.abs(a - b).max() / den
    assert err <= tol, f"max rel err {err:.3e} > {tol}"


@pytest.fixture(scope="module", autouse=True)
def _built():
    if not os.path.exists(os.path.join(ROOT, "oracle", "libnaive.so")):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "libnaive.so"], check=True)


# ---------------------------------------------------------------- conv
@pytest.mark.parametrize("stride,pad,dil,k", [(1, 1, 1, 3), (2, 1, 1, 3), (1, 0, 1, 1), (1, 2, 2, 3),
                                             ((2, 1), (1, 0), (1, 3), 3), ((1, 2), (3, 2), (3, 2), 3)])
def test_conv_torch_vs_c(stride, pad, dil, k):
    x, w, b = _rand((2, 5, 9, 7), 1), _rand((6, 5, k, k), 2, 0.2), _rand((6,), 3, 0.1)
    ref = torch.nn.functional.conv2d(x, w, b, stride=stride, padding=pad, dilation=dil)
    got = naive.conv2d(x, w, b, stride=stride, pad=pad, dilation=dil)
    assert got.shape == tuple(ref.shape)  # output-size formula, src/kernels/conv2d.cu:275-278
    _close(got, ref)
    _close(R.conv2d(x, w, b, stride=stride, pad=pad, dilation=dil), ref)


@pytest.mark.parametrize("dh,dw", [(2, 2), (3, 1), (1, 2)])
def test_conv_dilation_is_zero_inserted_kernel(dh, dw):
    """A conv with dilation (dh, dw) equals the undilated conv whose kernel has
    (dh - 1, dw - 1) zero rows / columns inserted between taps
    (src/kernels/conv2d.cu:88-164 reads input row oh*sh - ph + kh*dh)."""
    x, w = _rand((2, 3, 11, 12), 4), _rand((4, 3, 3, 3), 5, 0.3)
    wz = torch.zeros(4, 3, 2 * dh + 1, 2 * dw + 1)
    wz[:, :, ::dh, ::dw] = w
    for pad in ((1, 1), (2, 3)):
        got = naive.conv2d(x, w, None, stride=1, pad=pad, dilation=(dh, dw))
        ref = naive.conv2d(x, wz, None, stride=1, pad=pad, dilation=1)
        _close(got, ref)


def test_conv_delta_kernel_is_shifted_copy():
    """A kernel with a single 1 at tap (kh, kw) copies the input shifted by
    (kh - 1, kw - 1) with zero fill (src/tests/test_conv2d.cu:599-724)."""
    x = _rand((1, 3, 6, 5), 4)
    for kh, kw in [(0, 0), (1, 2), (2, 1)]:
        w = torch.zeros(3, 3, 3, 3)
        for c in range(3):
            w[c, c, kh, kw] = 1.0
        got = torch.from_numpy(naive.conv2d(x, w, None))
        exp = torch.zeros_like(x)
        dy, dx = kh - 1, kw - 1
        for y in range(6):
            for xx in range(5):
                sy, sx = y + dy, xx + dx
                if 0 <= sy < 6 and 0 <= sx < 5:
                    exp[0, :, y, xx] = x[0, :, sy, sx]
        assert torch.equal(got, exp)


def test_conv_ones_counts_taps():
    """ones (*) ones with zero padding counts in-bounds taps: 4 at corners,
    6 on edges, 9 inside (times Cin)."""
    got = naive.conv2d(torch.ones(1, 2, 4, 4), torch.ones(1, 2, 3, 3), None)[0, 0]
    exp = np.array([[4, 6, 6, 4], [6, 9, 9, 6], [6, 9, 9, 6], [4, 6, 6, 4]], np.float32) * 2
    assert np.array_equal(got, exp)


def test_conv_1x1_is_gemm_and_bias_linear():
    x, w, b = _rand((2, 8, 3, 4), 5), _rand((5, 8, 1, 1), 6, 0.3), _rand((5,), 7)
    conv = naive.conv2d(x, w, b, pad=0)
    xm = x.permute(0, 2, 3, 1).reshape(-1, 8)
    gem = naive.gemm(xm, w.reshape(5, 8), trans_b=True) + b.numpy()
    _close(conv.transpose(0, 2, 3, 1).reshape(-1, 5), gem)
    # bias linearity: conv(x, w, b) - conv(x, w, 0) == b per channel
    diff = conv - naive.conv2d(x, w, None, pad=0)
    _close(diff, np.broadcast_to(b.numpy()[None, :, None, None], diff.shape))


def test_conv_batch_is_per_sample():
    x, w = _rand((2, 4, 5, 5), 8), _rand((3, 4, 3, 3), 9, 0.2)
    both = naive.conv2d(x, w)
    assert np.array_equal(both[0], naive.conv2d(x[:1], w)[0])
    assert np.array_equal(both[1], naive.conv2d(x[1:], w)[0])


# ---------------------------------------------------------------- gemm
def test_gemm_identity_alpha_beta():
    """src/tests/test_gemm.cu:155-240: identity, alpha/beta, transB."""
    a = _rand((7, 5), 10)
    eye = torch.eye(5)
    _close(naive.gemm(a, eye), a)
    _close(naive.gemm(a, eye, trans_b=True), a)
    b, c = _rand((5, 4), 11), _rand((7, 4), 12)
    _close(naive.gemm(a, b, c, alpha=0.5, beta=2.0), 0.5 * (a @ b) + 2.0 * c)
    _close(naive.gemm(a, b.t().contiguous(), trans_b=True), a @ b)
    _close(R.gemm(a, b, c, alpha=0.5, beta=2.0), 0.5 * (a @ b) + 2.0 * c)
    _close(R.linear(a, b.t().contiguous(), None), a @ b)


# ---------------------------------------------------------------- group norm
def test_group_norm_known_case():
    """src/tests/test_groupnorm.cu:236-299: N=1, C=4, 2x2, G=2, eps=1e-6,
    gamma=1, beta=0.  Group 0 holds 1..8 (mean 4.5, var 5.25), group 1 holds
    -1,-2,-3,-4,2,2,2,2 (mean -0.25, var 5.6875)."""
    x = torch.tensor([1, 2, 3, 4, 5, 6, 7, 8, -1, -2, -3, -4, 2, 2, 2, 2], dtype=torch.float32).reshape(1, 4, 2, 2)
    exp = torch.empty(16)
    exp[:8] = (x.reshape(-1)[:8] - 4.5) / math.sqrt(5.25 + 1e-6)
    exp[8:] = (x.reshape(-1)[8:] + 0.25) / math.sqrt(5.6875 + 1e-6)
    for got in (naive.group_norm(x, 2, torch.ones(4), torch.zeros(4), 1e-6),
                R.group_norm(x, 2, torch.ones(4), torch.zeros(4), 1e-6).numpy()):
        _close(got.reshape(-1), exp, 1e-5)


@pytest.mark.parametrize("silu", [False, True])
def test_group_norm_torch_vs_c(silu):
    x = _rand((2, 64, 6, 5), 13)
    g, b = 1 + _rand((64,), 14, 0.1), _rand((64,), 15, 0.1)
    ref = R.group_norm(x, 32, g, b, 1e-5)
    if silu:
        ref = R.silu(ref)
    _close(naive.group_norm(x, 32, g, b, 1e-5, silu=silu), ref, 1e-4)


def test_group_norm_invariants():
    """Per-group mean -> beta and variance -> gamma^2 for constant gamma/beta;
    adding a constant to a group leaves the output unchanged."""
    x = _rand((1, 8, 4, 4), 16, 3.0)
    y = naive.group_norm(x, 2, torch.full((8,), 2.0), torch.full((8,), 0.5), 1e-6).reshape(2, -1)
    assert np.allclose(y.mean(1), 0.5, atol=1e-5)
    assert np.allclose(y.var(1), 4.0, rtol=1e-4)
    ones, zeros = torch.ones(8), torch.zeros(8)
    _close(naive.group_norm(x + 7.0, 2, ones, zeros, 1e-6), naive.group_norm(x, 2, ones, zeros, 1e-6), 1e-4)


# ---------------------------------------------------------------- layer norm
def test_layer_norm_known_case():
    """src/tests/test_layernorm.cu:205-262: rows [1,2,3,4] and [-2,0,2,4]
    (means 2.5 and 1, variances 1.25 and 5), eps=1e-5, no affine."""
    x = torch.tensor([[1.0, 2, 3, 4], [-2.0, 0, 2, 4]])
    exp = torch.stack([(x[0] - 2.5) / math.sqrt(1.25 + 1e-5), (x[1] - 1.0) / math.sqrt(5.0 + 1e-5)])
    _close(naive.layer_norm(x), exp, 1e-6)
    _close(R.layer_norm(x, None, None), exp, 1e-6)


def test_layer_norm_torch_vs_c():
    x = _rand((9, 320), 17, 2.0)
    g, b = 1 + _rand((320,), 18, 0.1), _rand((320,), 19, 0.1)
    _close(naive.layer_norm(x, g, b), R.layer_norm(x, g, b), 1e-5)
    _close(naive.layer_norm(x + 5.0, g, b), naive.layer_norm(x, g, b), 2e-4)  # shift invariance


# ---------------------------------------------------------------- attention
def test_attention_torch_vs_c():
    q, k, v = _rand((2, 3, 9, 16), 20), _rand((2, 3, 13, 16), 21), _rand((2, 3, 13, 16), 22)
    _close(naive.attention(q, k, v, 0.25), R.attention(q, k, v, 0.25), 1e-5)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=0.25)
    _close(R.attention(q, k, v, 0.25), ref, 1e-5)


def test_attention_invariants():
    """src/tests/test_attention.cu:266-304 and closed forms: equal keys ->
    mean(V); one key -> V; scale 0 -> mean(V); key permutation invariance."""
    q, v = _rand((1, 2, 5, 8), 23), _rand((1, 2, 6, 8), 24)
    k_eq = _rand((1, 2, 1, 8), 25).expand(1, 2, 6, 8).contiguous()
    mean_v = v.mean(dim=2, keepdim=True).expand(1, 2, 5, 8).numpy()
    _close(naive.attention(q, k_eq, v, 0.125), mean_v, 1e-5)
    _close(naive.attention(q, _rand((1, 2, 6, 8), 26), v, 0.0), mean_v, 1e-5)
    one_k, one_v = _rand((1, 2, 1, 8), 27), _rand((1, 2, 1, 8), 28)
    _close(naive.attention(q, one_k, one_v, 0.125), one_v.expand(1, 2, 5, 8).numpy(), 1e-6)
    k = _rand((1, 2, 6, 8), 29)
    perm = torch.tensor([3, 0, 5, 1, 4, 2])
    _close(naive.attention(q, k[:, :, perm], v[:, :, perm], 0.3), naive.attention(q, k, v, 0.3), 1e-5)


# ---------------------------------------------------------------- activations
def test_activation_known_values():
    """src/tests/test_activation.cu:183-260: silu(0)=0, silu(+-20) ~ (20, 0);
    gelu(1) = Phi(1) = 0.8413447460685429, gelu(-1) = -0.15865525393145707."""
    assert naive.silu(np.array([0.0]))[0] == 0.0
    assert abs(naive.silu(np.array([20.0]))[0] - 20.0) < 1e-5
    assert abs(naive.silu(np.array([-20.0]))[0]) < 1e-6
    assert abs(naive.silu(np.array([1.0]))[0] - 1.0 / (1.0 + math.exp(-1.0))) < 1e-6
    assert abs(naive.gelu_erf(np.array([1.0]))[0] - 0.8413447460685429) < 1e-6
    assert abs(naive.gelu_erf(np.array([-1.0]))[0] + 0.15865525393145707) < 1e-6
    x = _rand((64,), 30, 3.0)
    _close(naive.silu(x.numpy()), R.silu(x), 1e-6)
    _close(naive.gelu_erf(x.numpy()), R.gelu_erf(x), 1e-6)


def test_gelu_tanh_oracle():
    """The tanh-approximate GELU (src/tests/test_activation.cu:127-131, 276-284)
    against torch's own approximate='tanh' GELU, its odd-part identity
    f(x) - f(-x) = x, f(0) = 0, and its departure from the erf form (a few
    1e-4 near |x| = 2.5, so a swapped formula is caught)."""
    x = _rand((257,), 31, 3.0)
    _close(R.gelu_tanh(x), torch.nn.functional.gelu(x, approximate="tanh"), 1e-6)
    _close(R.gelu_tanh(x) - R.gelu_tanh(-x), x, 1e-5)
    assert float(R.gelu_tanh(torch.tensor([0.0]))[0]) == 0.0
    d = float((R.gelu_tanh(torch.tensor([2.5], dtype=torch.float64))
               - R.gelu_erf(torch.tensor([2.5], dtype=torch.float64)))[0])
    assert 3e-4 < d < 6e-4


def test_geglu_known_and_random():
    """src/tests/test_geglu.cu:130-160: [1, -1, 1, 0] -> [gelu(1), -gelu(0)] = [0.8413, 0];
    value is the first half, gate the second."""
    got = naive.geglu(np.array([[1.0, -1.0, 1.0, 0.0]], np.float32))[0]
    assert abs(got[0] - 0.8413447) < 1e-6 and abs(got[1]) < 1e-7
    h = _rand((7, 40), 31, 2.0)
    _close(naive.geglu(h), R.geglu(h), 1e-6)


# ---------------------------------------------------------------- time embedding
def test_timestep_embedding_known():
    """src/tests/test_timeembed.cu:99-124: element 0 is cos(t), element dim/2
    is sin(t) (frequency exp(0) = 1); t=0 gives cos=1, sin=0."""
    t = 2.5
    e = naive.time_embedding(t, 320)
    assert abs(e[0] - math.cos(t)) < 1e-6 and abs(e[160] - math.sin(t)) < 1e-6
    z = naive.time_embedding(0.0, 320)
    assert np.all(z[:160] == 1.0) and np.all(z[160:] == 0.0)
    # last frequency: exp(-ln(10000) * 159/160)
    f = math.exp(-math.log(10000.0) * 159 / 160)
    assert abs(naive.time_embedding(999.0, 320)[159] - math.cos(999.0 * f)) < 1e-4
    # fp32 argument rounding at |t * f| ~ 1e3 rad differs between the two
    # restatements by ~3e-5
    for tt in (0.0, 1.0, 100.0, 500.0, 999.0):
        _close(naive.time_embedding(tt, 320), R.timestep_embedding(torch.tensor([tt]), 320)[0], 1e-4)
        _close(naive.time_embedding(tt, 256), R.timestep_embedding(torch.tensor([tt]), 256)[0], 1e-4)


# ---------------------------------------------------------------- scheduler
def test_euler_schedule_closed_form_and_reference():
    """Leading spacing, offset 1, 20 steps: timesteps 951, 901, ..., 1 and
    sigma_0 = 11.028 (src/infer/scheduler.hpp:20)."""
    sig, ts = naive.euler_schedule(20)
    assert list(ts) == [951 - 50 * i for i in range(20)]
    assert abs(sig[0] - 11.0283) < 1e-3 and sig[-1] == 0.0
    assert np.all(np.diff(sig) < 0)
    # sigma(t) = sqrt((1 - acp) / acp) at t=951 from the closed-form product
    acp = 1.0
    for i in range(952):
        sb = math.sqrt(0.00085) + (math.sqrt(0.012) - math.sqrt(0.00085)) * i / 999
        acp *= 1.0 - sb * sb
    assert abs(sig[0] - math.sqrt((1 - acp) / acp)) < 1e-5
    ref = os.path.join(ROOT, "oracle", "_ref", "sched_ref")
    if os.path.exists(ref):
        for steps in (1, 7, 20, 50):
            out = subprocess.run([ref, str(steps)], capture_output=True, text=True, check=True).stdout.split("\n")
            rs = np.array([list(map(float, l.split())) for l in out[:steps]])
            s, t = naive.euler_schedule(steps)
            assert np.array_equal(t, rs[:, 1].astype(np.float32))
            _close(s[:steps], rs[:, 0], 1e-7)
            assert float(out[steps]) == 0.0


def test_product_scheduler_matches_oracle():
    from dollama_amd import unet as U
    for steps in (1, 20, 30):
        s, t = U.euler_schedule(steps)
        ns, nt = naive.euler_schedule(steps)
        assert np.array_equal(np.asarray(t, np.float32), nt)
        _close(np.asarray(s), ns, 1e-7)


# ---------------------------------------------------------------- SSIM
def test_ssim_restatements_agree():
    a = _rand((2, 4, 23, 17), 32)
    b = a + _rand((2, 4, 23, 17), 33, 0.05)
    s_vec, s_loop, s_c = metrics.ssim_uniform(a, b), metrics.ssim_uniform_loops(a, b), naive.ssim_uniform(a, b)
    assert abs(s_vec - s_loop) < 1e-12 and abs(s_vec - s_c) < 1e-6
    assert metrics.ssim_uniform(a, a) == pytest.approx(1.0, abs=1e-12)
    assert metrics.ssim_uniform(a, a + _rand((2, 4, 23, 17), 34, 0.5)) < s_vec < 1.0


# ---------------------------------------------------------------- UNet structure
def test_unet_param_count_and_product_spec():
    """2,567,463,684 parameters (the reference measures 2.57 B,
    docs/measurements-log.md:40); the product's C++ weight list has the same
    names and shapes as the oracle's independently written list."""
    from dollama_amd import unet as U
    ps = OR.param_shapes(OR.SDXL)
    assert sum(math.prod(s) for s in ps.values()) == 2_567_463_684
    ws = U.weight_specs(U.SDXL_CONFIG)
    assert set(ws) == set(ps)
    assert all(tuple(ws[k]) == tuple(ps[k]) for k in ps)


def test_step_flop_count():
    """Per B=2 step at 128x128 latent: 13.522 TFLOP in total; the mid block
    (resnet, 10-deep Transformer2D, resnet at 32x32x1280) counted by hand."""
    from dollama_amd.flops import mid_block_flops, unet_step_flops
    f = unet_step_flops(B=2, H=128, W=128)
    assert abs(f["total"] / 1e12 - 13.5224) < 1e-3
    HW, C, B, ctx = 32 * 32, 1280, 2, 77
    conv = 4 * (2 * B * HW * C * 9 * C)  # two resnets, two 3x3 convs each
    lin_blk = 2 * B * HW * C * (3 * C + C + C + C + 8 * C + 4 * C) + 2 * B * ctx * 2048 * 2 * C
    attn_blk = 4 * B * HW * HW * C + 4 * B * HW * ctx * C
    proj = 2 * 2 * B * HW * C * C
    assert mid_block_flops(B=2) == pytest.approx(conv + 10 * (lin_blk + attn_blk) + proj, rel=1e-9)


def test_small_unet_forward_runs_and_is_deterministic():
    """The oracle forward on the small topology is finite, deterministic and
    its stage list covers the graph (time/add embedding to conv_out)."""
    W = OR.random_weights(OR.TINY, seed=3)
    g = torch.Generator().manual_seed(1)
    lat = torch.randn(1, 4, 16, 16, generator=g)
    ehs = torch.randn(1, 77, 96, generator=g)
    text = torch.randn(1, 64, generator=g)
    ids = torch.tensor([1024.0, 1024.0, 0.0, 0.0, 1024.0, 1024.0])
    stages = {}
    a = OR.unet_forward(W, OR.TINY, lat, torch.tensor([999.0]), ehs, text, ids, stages=stages)
    b = OR.unet_forward(W, OR.TINY, lat, torch.tensor([999.0]), ehs, text, ids)
    assert torch.isfinite(a).all() and torch.equal(a, b) and a.shape == (1, 4, 16, 16)
    assert len(stages) >= 10


# ------------------------------------------------------------------ VAE --
def test_vae_param_count_is_the_published_autoencoder_total():
    """Decoder + post_quant_conv list of the oracle plus the encoder +
    quant_conv of the same architecture (counted here from the diffusers
    AutoencoderKL layout) = 83,653,863, the published parameter count of the
    SD / SDXL AutoencoderKL."""
    from oracle import vae_ref as OV
    dec = sum(math.prod(s) for s in OV.param_shapes(OV.SDXL_VAE).values())

    def conv(o, i, k):
        return o * i * k * k + o

    def res(i, o):
        return 2 * i + conv(o, i, 3) + 2 * o + conv(o, o, 3) + (conv(o, i, 1) if i != o else 0)

    enc, cin = conv(128, 3, 3), 128
    for b, co in enumerate((128, 256, 512, 512)):
        enc += res(cin, co) + res(co, co) + (conv(co, co, 3) if b < 3 else 0)
        cin = co
    enc += 2 * res(512, 512) + 2 * 512 + 4 * (512 * 512 + 512)  # mid: 2 resnets + attention
    enc += 2 * 512 + conv(8, 512, 3) + conv(8, 8, 1)  # norm_out, conv_out, quant_conv
    assert dec == 49_490_199
    assert dec + enc == 83_653_863


def _vae_skeleton_weights(cfg, seed):
    """Weights under which every resnet and the attention are identities
    (conv2, to_out and their biases zero; shortcuts select the first Co
    channels) and every upsampler conv is the identity kernel."""
    from oracle import vae_ref as OV
    W = OV.random_weights(cfg, seed)
    for k, v in W.items():
        if ".conv2." in k or ".to_out.0." in k:
            W[k] = torch.zeros_like(v)
        elif ".conv_shortcut.weight" in k:
            o, i = v.shape[:2]
            W[k] = torch.eye(o, i)[:, :, None, None].contiguous()
        elif ".conv_shortcut.bias" in k:
            W[k] = torch.zeros_like(v)
        elif ".upsamplers.0.conv.weight" in k:
            o = v.shape[0]
            t = torch.zeros_like(v)
            t[:, :, 1, 1] = torch.eye(o)
            W[k] = t
        elif ".upsamplers.0.conv.bias" in k:
            W[k] = torch.zeros_like(v)
    return W


def test_vae_decoder_reduces_to_upsampled_head():
    """With identity resnets / attention / upsamplers the decoder must equal
    conv_out(silu(GN(nearest_8x(first C3 channels of conv_in(pqc(z)))))),
    computed here with library calls only; this fixes the number and order
    of the upsamples, the residual wiring and the channel flow."""
    import torch.nn.functional as F
    from oracle import vae_ref as OV
    cfg = OV.TINY_VAE
    W = _vae_skeleton_weights(cfg, 5)
    z = _rand((2, 4, 6, 5), 6)
    got = OV.vae_decode(W, cfg, z)
    c3 = OV.decoder_channels(cfg)[3]
    x = F.conv2d(z, W["post_quant_conv.weight"], W["post_quant_conv.bias"])
    x = F.conv2d(x, W["decoder.conv_in.weight"], W["decoder.conv_in.bias"], padding=1)
    x = F.interpolate(x[:, :c3], scale_factor=8, mode="nearest")
    x = F.silu(F.group_norm(x, 32, W["decoder.conv_norm_out.weight"], W["decoder.conv_norm_out.bias"], 1e-6))
    ref = F.conv2d(x, W["decoder.conv_out.weight"], W["decoder.conv_out.bias"], padding=1)
    assert got.shape == (2, 3, 48, 40)
    _close(got, ref, 1e-4)


def test_vae_attention_block_is_single_head_sdpa():
    """The mid-block attention equals torch's scaled_dot_product_attention
    (one head, default scale 1/sqrt(C)) between the same projections."""
    import torch.nn.functional as F
    from oracle import vae_ref as OV
    W = OV.random_weights(OV.TINY_VAE, 7)
    C = OV.decoder_channels(OV.TINY_VAE)[0]
    x = _rand((1, C, 6, 7), 8)
    p = "decoder.mid_block.attentions.0."
    got = OV.attn_block(W, p, x)
    h = F.group_norm(x, 32, W[p + "group_norm.weight"], W[p + "group_norm.bias"], 1e-6)
    h = h.flatten(2).transpose(1, 2)
    q, k, v = (F.linear(h, W[p + n + ".weight"], W[p + n + ".bias"]) for n in ("to_q", "to_k", "to_v"))
    o = F.scaled_dot_product_attention(q[:, None], k[:, None], v[:, None])[:, 0]
    o = F.linear(o, W[p + "to_out.0.weight"], W[p + "to_out.0.bias"])
    _close(got, x + o.transpose(1, 2).reshape(x.shape), 1e-4)


def test_rgb8_fixed_points():
    """-1 -> 0, 1 -> 255, 0 -> int(127.5 + 0.5) = 128, clamping beyond [-1, 1],
    HWC order (src/infer/diffusion.cu:146-165)."""
    from oracle import vae_ref as OV
    img = torch.tensor([-1.0, 1.0, 0.0, -3.0, 3.0, 0.5]).reshape(1, 3, 1, 2)
    q = OV.image_to_rgb8(img)
    assert q.shape == (1, 1, 2, 3)
    # channel planes [-1, 1], [0, -3], [3, 0.5] -> pixels (-1, 0, 3) and (1, -3, 0.5)
    assert q[0, 0, 0].tolist() == [0, 128, 255] and q[0, 0, 1].tolist() == [255, 0, 191]


# ------------------------------------------------------------------ noise --
def test_splitmix64_known_answer():
    """First SplitMix64 output for state 0: 0xE220A8397B1DCDAF
    (16294208416658607535), the published test value."""
    from oracle import noise_ref as NR
    assert NR.splitmix64(0) == 0xE220A8397B1DCDAF


def _berlekamp_massey(bits):
    """Shortest LFSR over GF(2): connection polynomial (bit i = x^i) and length."""
    C, B, L, m = 1, 1, 0, 1
    for i, s in enumerate(bits):
        d = s
        for j in range(1, L + 1):
            d ^= ((C >> j) & 1) & bits[i - j]
        if d == 0:
            m += 1
        elif 2 * L <= i:
            C, B, L, m = C ^ (B << m), C, i + 1 - L, 1
        else:
            C ^= B << m
            m += 1
    return C, L


def _pmulmod(a, b, p, deg):
    r = 0
    while b:
        if b & 1:
            r ^= a
        b >>= 1
        a <<= 1
        if (a >> deg) & 1:
            a ^= p
    return r


def _ppow_x(e, p, deg):
    r, base = 1, 2
    while e:
        if e & 1:
            r = _pmulmod(r, base, p, deg)
        base = _pmulmod(base, base, p, deg)
        e >>= 1
    return r


def test_xorshift128plus_transition_is_full_period():
    """The low output bit of xorshift128+ is a linear function of the state,
    so its minimal polynomial is the transition's characteristic polynomial.
    With the published shifts (23, 17, 26) that polynomial has degree 128 and
    is primitive (period 2^128 - 1); a mistyped shift or operand breaks this."""
    from oracle import noise_ref as NR
    g = NR.XorShift128Plus(NR.splitmix64(7), NR.splitmix64(8))
    bits = [g.step() & 1 for _ in range(600)]
    C, L = _berlekamp_massey(bits)
    assert L == 128
    P = 0
    for i in range(129):  # reciprocal polynomial x^128 C(1/x)
        if (C >> i) & 1:
            P |= 1 << (128 - i)
    primes = [3, 5, 17, 257, 641, 65537, 274177, 6700417, 67280421310721]
    order = (1 << 128) - 1
    assert math.prod(primes) == order
    assert _ppow_x(order, P, 128) == 1
    for q in primes:
        assert _ppow_x(order // q, P, 128) != 1


def test_box_muller_pairing_and_moments():
    """next() returns r cos(2 pi u2), then r sin(2 pi u2) with r^2 = -2 ln u1,
    u1, u2 the generator's consecutive uniforms; N(0, 1) moments."""
    from oracle import noise_ref as NR
    a, b = NR.Randn(123), NR.Randn(123)
    for _ in range(50):
        u1 = b.uniform()
        while u1 <= 1e-12:
            u1 = b.uniform()
        u2 = b.uniform()
        z0, z1 = a.next(), a.next()
        assert abs(z0 * z0 + z1 * z1 + 2.0 * math.log(u1)) < 1e-9
        assert abs(math.atan2(z1, z0) % (2 * math.pi) - 2 * math.pi * u2) < 1e-9
    z = NR.randn_latent(5, 1.0, 200000).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert abs((z ** 4).mean() - 3.0) < 0.05
