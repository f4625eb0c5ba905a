"""Runtime LoRA: loader mapping (host), merged weights, bit-exact revert,
stacking, and the forward with a LoRA applied.

Follows the reference's gates (src/tests/test_lora_runtime.cu:1-14, 285-590):
  [1] host mapping: module count, text-encoder keys skipped, incomplete
      modules skipped, scale = strength * alpha / rank (= strength without
      alpha), an unresolvable module raises;
  [2] resident weights after apply == fp32 W + scale * (B @ A) within
      atol 2e-3 + rtol 1e-2 (test_lora_runtime.cu:416-418);
  [3] after clear, every resident weight is bit-identical to the base;
  [4] two LoRAs stack additively; clear is bit-exact again.
The weights the reference test touches (to_q, the GEGLU projection, a 3x3
conv) are taken from the small UNet config, plus the packed forms this
library adds (1x1 shortcut sharing conv2's rows, conv_in's channel padding,
cross-attention K, time_emb_proj rows).  The fp32 merge is computed here in
torch from the file's own fp16 factors, independently of the loader.
"""
import os

import numpy as np
import pytest
import safetensors.numpy as stn
import torch

from dollama_amd import unet as U
from dollama_amd._lib import DlmError

TINY = U.UNetConfig(C0=64, C1=128, C2=192, depth1=1, depth2=2, cross_dim=96, text_dim=64, id_dim=16)

KEY_TOQ = "down_blocks.1.attentions.0.transformer_blocks.0.attn1.to_q.weight"
KEY_FF = "down_blocks.1.attentions.0.transformer_blocks.0.ff.net.0.proj.weight"
KEY_CONV = "down_blocks.0.resnets.0.conv1.weight"
KEY_UNTOUCHED = "mid_block.resnets.0.conv2.weight"
EXTRA = [  # packed forms beyond the reference test's three
    "down_blocks.1.resnets.0.conv_shortcut.weight",
    "down_blocks.1.resnets.0.conv2.weight",
    "conv_in.weight",
    "down_blocks.2.attentions.1.transformer_blocks.1.attn2.to_k.weight",
    "up_blocks.1.attentions.2.transformer_blocks.0.attn2.to_v.weight",
    "down_blocks.0.resnets.1.time_emb_proj.weight",
    "mid_block.attentions.0.proj_out.weight",
]


def _flat(key):
    return key[: -len(".weight")].replace(".", "_")


def _f16(shape, seed, scale):
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape).astype(np.float32) * scale).astype(np.float16)


def _module(tensors, key, rank, seed, alpha=None, dtype=np.float16, flat_names=False):
    """kohya down [rank, in(,kh,kw)] / up [out, rank(,1,1)] for a base key."""
    shape = U.weight_specs(TINY)[key]
    out, rest = shape[0], tuple(shape[1:])
    mod = "lora_unet_" + _flat(key)
    down = _f16((rank,) + rest, seed, 0.05).astype(dtype)
    up = _f16((out, rank) + ((1, 1) if len(shape) == 4 else ()), seed + 1, 0.05).astype(dtype)
    sep = "_" if flat_names else "."
    tensors[mod + sep + "lora_down" + sep + "weight"] = down
    tensors[mod + sep + "lora_up" + sep + "weight"] = up
    if alpha is not None:
        tensors[mod + sep + "alpha"] = np.array(alpha, dtype=np.float32)


def _write(path, tensors):
    stn.save_file(tensors, path)
    return path


def lora1(tmp):
    t = {}
    _module(t, KEY_TOQ, 4, 200, alpha=4.0)
    _module(t, KEY_FF, 8, 202, alpha=4.0)
    _module(t, KEY_CONV, 4, 204, alpha=2.0)
    te = "lora_te1_text_model_encoder_layers_0_self_attn_q_proj"
    t[te + ".lora_down.weight"] = _f16((4, 32), 206, 0.05)
    t[te + ".lora_up.weight"] = _f16((32, 4), 207, 0.05)
    t[te + ".alpha"] = np.array(4.0, dtype=np.float32)
    t["lora_unet_" + _flat(KEY_FF) + "_broken.lora_down.weight"] = _f16((4, 128), 208, 0.05)
    return _write(os.path.join(tmp, "lora1.safetensors"), t)


def lora2(tmp):
    t = {}
    _module(t, KEY_TOQ, 2, 300)  # no alpha: scale = strength
    _module(t, KEY_CONV, 4, 302, alpha=4.0)
    return _write(os.path.join(tmp, "lora2.safetensors"), t)


def lora_extra(tmp):
    """F32 factors, the flat key spelling, 1x1 / padded / shared-row convs."""
    t = {}
    for i, key in enumerate(EXTRA):
        _module(t, key, 3 + (i % 3), 500 + 2 * i, alpha=2.0,
                dtype=np.float32 if i % 2 else np.float16, flat_names=(i == 2))
    t["some_other_tensor"] = np.zeros(3, np.float16)
    return _write(os.path.join(tmp, "lora_extra.safetensors"), t)


# ------------------------------------------------------------- host mapping --
def test_lora_scan_counts_and_scales(tmp_path):
    counts, mods = U.lora_scan(lora1(str(tmp_path)), 0.8, TINY)
    assert counts == {"modules": 3, "te_skipped": 3, "other_keys": 0, "incomplete": 1}
    expect = {KEY_TOQ: (4, 128, 128, 0.8), KEY_FF: (8, 128, 1024, 0.4),
              KEY_CONV: (4, 64 * 9, 64, 0.4)}
    assert set(mods) == set(expect)
    for k, (r, i, o, s) in expect.items():
        assert mods[k][:3] == (r, i, o), k
        assert abs(mods[k][3] - s) <= 1e-6, (k, mods[k][3], s)


def test_lora_scan_without_alpha_uses_strength(tmp_path):
    counts, mods = U.lora_scan(lora2(str(tmp_path)), 0.5, TINY)
    assert counts["modules"] == 2
    assert abs(mods[KEY_TOQ][3] - 0.5) <= 1e-6
    assert mods[KEY_TOQ][0] == 2
    assert abs(mods[KEY_CONV][3] - 0.5) <= 1e-6


def test_lora_scan_extra_forms(tmp_path):
    counts, mods = U.lora_scan(lora_extra(str(tmp_path)), 1.0, TINY)
    assert counts == {"modules": len(EXTRA), "te_skipped": 0, "other_keys": 1, "incomplete": 0}
    assert set(mods) == set(EXTRA)


def test_lora_scan_unresolved_module_raises(tmp_path):
    t = {"lora_unet_nonexistent_module_xyz.lora_down.weight": _f16((4, 16), 400, 0.05),
         "lora_unet_nonexistent_module_xyz.lora_up.weight": _f16((16, 4), 401, 0.05)}
    with pytest.raises(DlmError, match="matches no UNet weight"):
        U.lora_scan(_write(str(tmp_path / "bad.safetensors"), t), 1.0, TINY)


def test_lora_scan_shape_mismatch_raises(tmp_path):
    t = {}
    mod = "lora_unet_" + _flat(KEY_TOQ)
    t[mod + ".lora_down.weight"] = _f16((4, 96), 1, 0.05)  # in 96 != 128
    t[mod + ".lora_up.weight"] = _f16((128, 4), 2, 0.05)
    with pytest.raises(DlmError, match="does not match the shape"):
        U.lora_scan(_write(str(tmp_path / "bad.safetensors"), t), 1.0, TINY)


def test_lora_scan_bad_alpha_dtype_raises(tmp_path):
    t = {}
    _module(t, KEY_TOQ, 4, 1)
    t["lora_unet_" + _flat(KEY_TOQ) + ".alpha"] = np.array([1, 2], dtype=np.int32)
    with pytest.raises(DlmError, match="alpha"):
        U.lora_scan(_write(str(tmp_path / "bad.safetensors"), t), 1.0, TINY)


def test_f32_to_f16_round_to_nearest_even():
    """Against numpy's IEEE conversion (round to nearest, ties to even):
    ties at every exponent, subnormals, overflow, infinities, NaN."""
    rng = np.random.default_rng(0)
    e = rng.uniform(-30, 17, 200000).astype(np.float32)
    x = (rng.choice([-1.0, 1.0], e.size) * np.exp2(e)).astype(np.float32)
    bits = x.view(np.uint32)
    ties = ((bits & ~np.uint32(0x1FFF)) | np.uint32(0x1000)).view(np.float32)  # exact halfway points
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e-8, 2.98e-8, 2.9802322e-8,
                        5.96e-8, 6.1e-5, 6.097555e-5, np.inf, -np.inf], dtype=np.float32)
    for a in (x, ties, special):
        got = U.f32_to_f16_bits(a)
        with np.errstate(over="ignore"):
            want = a.astype(np.float16).view(np.uint16)
        assert np.array_equal(got, want)
    nan = U.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert np.isnan(nan.view(np.float16)).all()


# ------------------------------------------------------------------ device --
def _base_net(seed=7):
    from oracle import unet_ref as OR
    Wc = OR.random_weights(OR.TINY, seed=seed)
    net = U.UNet(TINY)
    Wg = {k: v.half().cuda() for k, v in Wc.items()}
    net.set_weights(Wg)
    net.prepare()
    return net, Wc


def _factors(path):
    """{base_key: (A fp32 [rank, in_flat], B fp32 [out, rank])} from the file."""
    t = stn.load_file(path)
    out = {}
    for k, v in t.items():
        if not k.startswith("lora_unet_"):
            continue
        for suf, idx in ((".lora_down.weight", 0), ("_lora_down_weight", 0),
                         (".lora_up.weight", 1), ("_lora_up_weight", 1)):
            if k.endswith(suf):
                mod = k[len("lora_unet_"): -len(suf)]
                out.setdefault(mod, [None, None])[idx] = torch.from_numpy(
                    v.astype(np.float16).astype(np.float32))
    res = {}
    for key in U.weight_specs(TINY):
        f = out.get(_flat(key))
        if f and f[0] is not None and f[1] is not None:
            res[key] = (f[0].reshape(f[0].shape[0], -1), f[1].reshape(f[1].shape[0], -1))
    return res


def _expected(Wc, loras):
    """fp32 W + sum scale_i * (B_i @ A_i), per touched key."""
    exp = {}
    for path, strength in loras:
        _, mods = U.lora_scan(path, strength, TINY)
        fac = _factors(path)
        for key, (rank, in_flat, out_dim, scale) in mods.items():
            A, B = fac[key]
            assert A.shape == (rank, in_flat) and B.shape == (out_dim, rank)
            base = exp.get(key, Wc[key].float().reshape(out_dim, in_flat))
            exp[key] = base + scale * (B @ A)
    return exp


def _check_weights(net, exp):
    for key, ref in exp.items():
        got = net.read_weight(key).float().reshape(ref.shape)
        bad = ((got - ref).abs() > 2e-3 + 1e-2 * ref.abs()).sum().item()
        print(f"[lora] {key}: max_abs={(got - ref).abs().max().item():.3e} bad={bad}", flush=True)
        assert bad == 0, key


def _snapshot(net):
    """Every resident 2-D / 4-D weight (the ones a LoRA can patch)."""
    return {k: net.read_weight(k) for k, s in U.weight_specs(TINY).items() if len(s) in (2, 4)}


@pytest.mark.gpu
def test_lora_apply_parity_revert_stack(gpu, tmp_path):
    print("[case] tiny UNet LoRA apply / clear / stack", flush=True)
    p1, p2, p3 = lora1(str(tmp_path)), lora2(str(tmp_path)), lora_extra(str(tmp_path))
    net, Wc = _base_net()
    base = _snapshot(net)
    for k, v in base.items():  # the readback itself is exact
        assert torch.equal(v.float(), Wc[k]), k
    # [2] parity
    counts = net.load_lora(p1, 0.8)
    assert counts == {"modules": 3, "te_skipped": 3, "other_keys": 0, "incomplete": 1}
    _check_weights(net, _expected(Wc, [(p1, 0.8)]))
    assert torch.equal(net.read_weight(KEY_UNTOUCHED), base[KEY_UNTOUCHED])
    # [3] revert bit-exact
    net.clear_loras()
    for k, v in _snapshot(net).items():
        assert torch.equal(v, base[k]), f"{k} not restored bit-exactly"
    # [4] stack (the same LoRA twice on one key, and a second file)
    net.load_lora(p1, 0.8)
    net.load_lora(p2, 0.5)
    net.load_lora(p3, 1.0)
    _check_weights(net, _expected(Wc, [(p1, 0.8), (p2, 0.5), (p3, 1.0)]))
    net.clear_loras()
    for k, v in _snapshot(net).items():
        assert torch.equal(v, base[k]), f"{k} not restored bit-exactly after stacking"
    net.close()


@pytest.mark.gpu
def test_lora_apply_rejects_bad_input(gpu):
    net, _ = _base_net(seed=3)
    A = torch.zeros(4, 100, dtype=torch.float16, device="cuda:0")
    B = torch.zeros(128, 4, dtype=torch.float16, device="cuda:0")
    with pytest.raises(DlmError, match="does not match"):
        net.apply_lora(KEY_TOQ, A, B, 1.0)
    with pytest.raises(DlmError, match="not a UNet weight"):
        net.apply_lora("no.such.weight", A, B, 1.0)
    net.close()


@pytest.mark.gpu
def test_lora_forward_matches_merged_oracle(gpu, tmp_path):
    """The forward with a LoRA applied against the fp32 oracle run on
    fp16(W + scale * B @ A); after clear, bit-identical to the base forward."""
    from oracle import metrics
    from oracle import unet_ref as OR
    from tests._util import assert_close
    print("[case] tiny UNet forward with LoRA vs merged-weight oracle", flush=True)
    p1, p3 = lora1(str(tmp_path)), lora_extra(str(tmp_path))
    net, Wc = _base_net(seed=9)
    g = torch.Generator().manual_seed(10)
    B, H, W, L = 2, 32, 32, 77
    q = lambda t: t.half().float()
    lat = q(torch.randn(B, 4, H, W, generator=g))
    ehs = q(torch.randn(B, L, TINY.cross_dim, generator=g))
    text = q(torch.randn(B, TINY.text_dim, generator=g))
    ids = torch.tensor([1024.0, 1024.0, 0.0, 0.0, 1024.0, 1024.0])
    ts = torch.full((B,), 500.0)
    args = lambda: (lat.half().cuda(), ts.cuda(), ehs.half().cuda(), text.half().cuda(), ids.half().cuda())
    base_out = net.forward(*args()).clone()
    net.load_lora(p1, 1.0)
    net.load_lora(p3, 1.0)
    out = net.forward(*args()).float().cpu()
    merged = dict(Wc)
    for key, w in _expected(Wc, [(p1, 1.0), (p3, 1.0)]).items():
        merged[key] = w.reshape(Wc[key].shape).half().float()
    ref = OR.unet_forward(merged, OR.TINY, lat, ts, ehs, text, ids)
    assert_close(out, ref, "tiny noise_pred with LoRA")
    s = metrics.ssim_uniform(out, ref)
    print(f"[parity] LoRA noise_pred SSIM={s:.7f}", flush=True)
    assert s >= 0.99999
    assert not torch.equal(out.half(), base_out.cpu()), "LoRA changed nothing"
    net.clear_loras()
    again = net.forward(*args())
    torch.cuda.synchronize()
    assert torch.equal(again, base_out), "forward after clear differs from the base forward"
    net.close()
