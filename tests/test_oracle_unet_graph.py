"""Pins the wiring of the UNet oracle (oracle/unet_ref.py) to the reference's
graph text with skeleton weights that reduce each part to a closed form built
from torch.nn.functional calls (CPU only).

What each case pins (reference src/infer/unet.cu):
- up-path concat order [current, skip] and LIFO pop order (:1168-1266), the
  skip pushes of the down path (:1071-1140), stride-2 downsample and
  nearest-2x upsample placement (:863-881), conv_norm_out eps 1e-5 + SiLU +
  conv_out (:1270-1291);
- add-embedding input = text_embeds first, then 6 x sinusoid(id_dim) of
  time_ids, cos first (:995-1014, timeembed.cuh:14-24); time MLP
  sinusoid(C0) -> linear_1 -> SiLU -> linear_2 (:976-992);
- Transformer2D: GN eps 1e-6, NCHW -> tokens -> NCHW, residual (:810-858);
- resnet: GN eps 1e-5 + SiLU, conv1, + time_emb_proj(silu(temb)) after conv1,
  GN + SiLU, conv2, + shortcut (:537-664);
- transformer block: cross-attention K/V from the context (Sk=1 -> V),
  self-attention with equal keys -> mean of V, GEGLU value/gate halves
  (:677-797, geglu.cuh:13-19).

Every closed form is checked against a mutant of the oracle with the one
detail changed (source text edited in memory, on the CPU): the mutant must
fail the same comparison, so each case has teeth.
"""
import importlib.util
import math
import os
import sys

import pytest
import torch
import torch.nn.functional as F

from oracle import unet_ref as OR

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TINY = OR.TINY


class AnchorError(Exception):
    """A mutation's anchor text is absent or not unique (a test bug, never a
    caught mutant)."""


def _mutant(old, new):
    """oracle.unet_ref with `old` replaced by `new` (exactly one occurrence)."""
    path = os.path.join(ROOT, "oracle", "unet_ref.py")
    with open(path) as f:
        src = f.read()
    if src.count(old) != 1:
        raise AnchorError(f"mutation anchor not unique: {old!r}")
    src = src.replace(old, new)
    spec = importlib.util.spec_from_loader("oracle._unet_ref_mutant", loader=None)
    mod = importlib.util.module_from_spec(spec)
    mod.__package__ = "oracle"
    sys.modules[spec.name] = mod     # dataclasses look their module up by name
    try:
        exec(compile(src, "unet_ref_mutant.py", "exec"), mod.__dict__)
    finally:
        del sys.modules[spec.name]
    return mod


def _agree(a, b, tol=1e-5):
    scale = max(float(b.abs().max()), 1e-6)
    return a.shape == b.shape and float((a - b).abs().max()) <= tol * scale


def _fails(fn):
    """True when fn() raises or returns False (a planted mistake is caught)."""
    try:
        return not fn()
    except (RuntimeError, AssertionError, IndexError, ValueError, KeyError):
        return True


def _rand(shape, g, std=1.0):
    return torch.randn(shape, generator=g) * std


def _delta3(c, scale=1.0):
    """3x3 conv weight whose centre tap copies channel i to channel i."""
    w = torch.zeros(c, c, 3, 3)
    idx = torch.arange(c)
    w[idx, idx, 1, 1] = scale
    return w


def _pad_ch(x, c):
    """First c channels of x, zero-filled when x has fewer."""
    if x.shape[1] >= c:
        return x[:, :c]
    return torch.cat([x, x.new_zeros(x.shape[0], c - x.shape[1], *x.shape[2:])], 1)


# --------------------------------------------------------------- full graph --
def _skeleton(cfg, seed):
    """Weights under which every resnet is shortcut(x) + conv2.bias, every
    Transformer2D is the identity, down/up-samplers are centre-tap deltas plus
    their bias, and each up resnet's 1x1 shortcut weighs the current half by 1
    and the skip half by 1/2."""
    g = torch.Generator().manual_seed(seed)
    W = {}
    for name, shape in OR.param_shapes(cfg).items():
        W[name] = torch.zeros(shape)
    for name in W:
        if "norm" in name.split(".")[-2] and name.endswith(".weight"):
            W[name] = torch.ones(W[name].shape)
    W["conv_in.weight"] = _rand(W["conv_in.weight"].shape, g, 0.3)
    W["conv_in.bias"] = _rand(W["conv_in.bias"].shape, g, 0.1)
    W["conv_out.weight"] = _rand(W["conv_out.weight"].shape, g, 0.05)
    W["conv_out.bias"] = _rand(W["conv_out.bias"].shape, g, 0.1)
    W["conv_norm_out.weight"] = 1 + _rand(W["conv_norm_out.weight"].shape, g, 0.1)
    W["conv_norm_out.bias"] = _rand(W["conv_norm_out.bias"].shape, g, 0.1)
    for name in list(W):
        if name.endswith("conv2.bias"):
            W[name] = _rand(W[name].shape, g, 0.5)   # a distinct offset per resnet
        if "samplers.0.conv.weight" in name:
            W[name] = _delta3(W[name].shape[0])
        if "samplers.0.conv.bias" in name:
            W[name] = _rand(W[name].shape, g, 0.5)
    return W


def _set_shortcut(W, prefix, cur, sk, cout):
    w = torch.zeros(cout, cur + sk, 1, 1)
    n = min(cout, cur)
    w[torch.arange(n), torch.arange(n), 0, 0] = 1.0
    m = min(cout, sk)
    w[torch.arange(m), cur + torch.arange(m), 0, 0] = 0.5
    W[prefix + "conv_shortcut.weight"] = w


def _skeleton_full(cfg, seed):
    W = _skeleton(cfg, seed)
    C0, C1, C2 = cfg.C0, cfg.C1, cfg.C2
    # down path: channel-growing shortcuts copy x into the first channels
    for p, ci, co in (("down_blocks.1.resnets.0.", C0, C1), ("down_blocks.2.resnets.0.", C1, C2)):
        w = torch.zeros(co, ci, 1, 1)
        w[torch.arange(ci), torch.arange(ci), 0, 0] = 1.0
        W[p + "conv_shortcut.weight"] = w
    # up path: (current channels, popped skip channels, out channels) per resnet,
    # written from the reference's comments "1280,1280,640" / "640,640,320" /
    # "320,320,320" (unet.cu:1166,1209,1252)
    plan = {0: [(C2, C2, C2), (C2, C2, C2), (C2, C1, C2)],
            1: [(C2, C1, C1), (C1, C1, C1), (C1, C0, C1)],
            2: [(C1, C0, C0), (C0, C0, C0), (C0, C0, C0)]}
    for u, rows in plan.items():
        for r, (cur, sk, co) in enumerate(rows):
            _set_shortcut(W, f"up_blocks.{u}.resnets.{r}.", cur, sk, co)
    return W


def _closed_form_full(W, cfg, lat):
    """The skeleton UNet written out by hand: the pushes in down-path order, the
    pops in reverse, resnet = shortcut + conv2.bias."""
    C0, C1, C2 = cfg.C0, cfg.C1, cfg.C2

    def b(name):
        return W[name][None, :, None, None]

    def down(x, p):
        return x[:, :, ::2, ::2] + b(p + "downsamplers.0.conv.bias")

    def up(x, p):
        return F.interpolate(x, scale_factor=2.0, mode="nearest") + b(p + "upsamplers.0.conv.bias")

    def rb(x, p):
        return x + b(p + "conv2.bias")

    x0 = F.conv2d(lat, W["conv_in.weight"], W["conv_in.bias"], padding=1)
    d0r0 = rb(x0, "down_blocks.0.resnets.0.")
    d0r1 = rb(d0r0, "down_blocks.0.resnets.1.")
    ds0 = down(d0r1, "down_blocks.0.")
    d1r0 = rb(_pad_ch(ds0, C1), "down_blocks.1.resnets.0.")
    d1r1 = rb(d1r0, "down_blocks.1.resnets.1.")
    ds1 = down(d1r1, "down_blocks.1.")
    d2r0 = rb(_pad_ch(ds1, C2), "down_blocks.2.resnets.0.")
    d2r1 = rb(d2r0, "down_blocks.2.resnets.1.")
    mid = rb(rb(d2r1, "mid_block.resnets.0."), "mid_block.resnets.1.")

    def ur(cur, skip, p, co):
        return _pad_ch(cur, co) + 0.5 * _pad_ch(skip, co) + b(p + "conv2.bias")

    u = ur(mid, d2r1, "up_blocks.0.resnets.0.", C2)
    u = ur(u, d2r0, "up_blocks.0.resnets.1.", C2)
    u = ur(u, ds1, "up_blocks.0.resnets.2.", C2)
    u = up(u, "up_blocks.0.")
    u = ur(u, d1r1, "up_blocks.1.resnets.0.", C1)
    u = ur(u, d1r0, "up_blocks.1.resnets.1.", C1)
    u = ur(u, ds0, "up_blocks.1.resnets.2.", C1)
    u = up(u, "up_blocks.1.")
    u = ur(u, d0r1, "up_blocks.2.resnets.0.", C0)
    u = ur(u, d0r0, "up_blocks.2.resnets.1.", C0)
    u = ur(u, x0, "up_blocks.2.resnets.2.", C0)
    h = F.silu(F.group_norm(u, 32, W["conv_norm_out.weight"], W["conv_norm_out.bias"], 1e-5))
    return F.conv2d(h, W["conv_out.weight"], W["conv_out.bias"], padding=1)


def _full_inputs(cfg, seed, hw=16):
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(2, cfg.in_channels, hw, hw, generator=g)
    ts = torch.full((2,), 999.0)
    ehs = torch.randn(2, 7, cfg.cross_dim, generator=g)
    text = torch.randn(2, cfg.text_dim, generator=g)
    ids = torch.tensor([1024.0, 1024.0, 0.0, 0.0, 1024.0, 1024.0])
    return lat, ts, ehs, text, ids


def _full_case(mod, quiet=False):
    W = _skeleton_full(TINY, 11)
    if quiet:
        # small activations (group variance ~1e-5) so the head GroupNorm's eps
        # moves the result: no offsets, conv_in scaled down
        W["conv_in.weight"] *= 0.01
        for k in W:
            if k.endswith("conv2.bias") or "samplers.0.conv.bias" in k or k == "conv_in.bias":
                W[k] = torch.zeros_like(W[k])
    lat, ts, ehs, text, ids = _full_inputs(TINY, 12)
    got = mod.unet_forward(W, TINY, lat, ts, ehs, text, ids)
    return _agree(got, _closed_form_full(W, TINY, lat))


@pytest.mark.parametrize("quiet", [False, True])
def test_unet_skeleton_reduces_to_skip_sum(quiet):
    assert _full_case(OR, quiet)


@pytest.mark.parametrize("old,new", [
    ("torch.cat([x, skips.pop()], dim=1)", "torch.cat([skips.pop(), x], dim=1)"),   # concat order
    ("torch.cat([x, skips.pop()], dim=1)", "torch.cat([x, skips.pop(0)], dim=1)"),  # FIFO pops
    ("            skips.append(x)\n        if lv < 2:",
     "            pass\n        if lv < 2:"),                                         # resnet pushes
    ("w[\"conv_norm_out.bias\"], 1e-5)", "w[\"conv_norm_out.bias\"], 1e-6)"),         # head GN eps
    ("                         w[f\"down_blocks.{lv}.downsamplers.0.conv.bias\"], 2, 1)\n"
     "            skips.append(x)",
     "                         w[f\"down_blocks.{lv}.downsamplers.0.conv.bias\"], 2, 1)"),  # downsample push
])
def test_unet_skeleton_catches_wiring_mutants(old, new):
    m = _mutant(old, new)
    assert _fails(lambda: _full_case(m) and _full_case(m, quiet=True))


def test_unet_skeleton_distinguishes_concat_halves():
    """The reduction weighs the two halves differently, so swapping them changes
    the result even where both halves have the same width."""
    W = _skeleton_full(TINY, 11)
    lat = _full_inputs(TINY, 12)[0]
    a = _closed_form_full(W, TINY, lat)
    for u in range(3):
        for r in range(3):
            w = W[f"up_blocks.{u}.resnets.{r}.conv_shortcut.weight"]
            assert w.sum() > 0 and (w == 0.5).any() and (w == 1.0).any()
    assert float(a.abs().max()) > 0


# ------------------------------------------------------------- embeddings --
def _sinusoid(t, dim):
    """cos(t * f_k) for k < dim/2 then sin(t * f_k); f_k = 10000^(-k/(dim/2))."""
    half = dim // 2
    out = torch.empty(t.shape[0], dim, dtype=torch.float64)
    for k in range(half):
        f = 10000.0 ** (-k / half)
        out[:, k] = torch.cos(t.double() * f)
        out[:, half + k] = torch.sin(t.double() * f)
    return out.float()


def _embed_case(mod):
    cfg = TINY
    T = cfg.T
    n_add = cfg.text_dim + 6 * cfg.id_dim
    W = {k: torch.zeros(s) for k, s in OR.param_shapes(cfg).items()}
    # add embedding: linear_1 row r reads input column r; linear_2 = identity
    W["add_embedding.linear_1.weight"][torch.arange(n_add), torch.arange(n_add)] = 1.0
    W["add_embedding.linear_2.weight"] = torch.eye(T)
    g = torch.Generator().manual_seed(21)
    text = torch.randn(2, cfg.text_dim, generator=g)
    ids = torch.tensor([[1024.0, 896.0, 3.0, 17.0, 1024.0, 768.0],
                        [512.0, 640.0, 0.0, 5.0, 1152.0, 1024.0]])
    ts = torch.tensor([999.0, 999.0])
    got = mod.embeddings(W, cfg, ts, text, ids)
    # closed form: text first, then each time id's sinusoid in id order
    x = torch.cat([text] + [_sinusoid(ids[:, i], cfg.id_dim) for i in range(6)], 1)
    ref = torch.zeros(2, T)
    ref[:, :n_add] = F.silu(x)
    return _agree(got, ref, 1e-5)


def _time_mlp_case(mod):
    cfg = TINY
    T = cfg.T
    W = {k: torch.zeros(s) for k, s in OR.param_shapes(cfg).items()}
    g = torch.Generator().manual_seed(22)
    w1 = torch.randn(T, cfg.C0, generator=g) * 0.2
    b1 = torch.randn(T, generator=g) * 0.1
    w2 = torch.randn(T, T, generator=g) * 0.1
    b2 = torch.randn(T, generator=g) * 0.1
    W.update({"time_embedding.linear_1.weight": w1, "time_embedding.linear_1.bias": b1,
              "time_embedding.linear_2.weight": w2, "time_embedding.linear_2.bias": b2})
    ts = torch.tensor([999.0, 451.0])
    got = mod.embeddings(W, cfg, ts, torch.zeros(2, cfg.text_dim), torch.zeros(6))
    ref = F.linear(F.silu(F.linear(_sinusoid(ts, cfg.C0), w1, b1)), w2, b2)
    return _agree(got, ref, 1e-5)


def test_add_embedding_is_text_then_time_id_sinusoids():
    assert _embed_case(OR)


def test_time_embedding_mlp():
    assert _time_mlp_case(OR)


@pytest.mark.parametrize("old,new", [
    ("a = torch.cat([text, emb], dim=1)", "a = torch.cat([emb, text], dim=1)"),
    ("emb = R.timestep_embedding(ids.reshape(-1), cfg.id_dim).reshape(B, 6 * cfg.id_dim)",
     "emb = R.timestep_embedding(ids.t().reshape(-1), cfg.id_dim).reshape(B, 6 * cfg.id_dim)"),
])
def test_add_embedding_catches_mutants(old, new):
    assert _fails(lambda: _embed_case(_mutant(old, new)))


def test_time_mlp_catches_mutant():
    m = _mutant("h = R.silu(R.linear(t_emb, w[\"time_embedding.linear_1.weight\"], "
                "w[\"time_embedding.linear_1.bias\"]))",
                "h = R.linear(t_emb, w[\"time_embedding.linear_1.weight\"], "
                "w[\"time_embedding.linear_1.bias\"])")
    assert _fails(lambda: _time_mlp_case(m))


# ---------------------------------------------------------- Transformer2D --
def _t2d_identity_blocks(c, depth, g):
    W = {}
    p = "t."
    W[p + "norm.weight"] = 1 + torch.randn(c, generator=g) * 0.2
    W[p + "norm.bias"] = torch.randn(c, generator=g) * 0.2
    W[p + "proj_in.weight"] = torch.eye(c)
    W[p + "proj_in.bias"] = torch.zeros(c)
    W[p + "proj_out.weight"] = torch.eye(c)
    W[p + "proj_out.bias"] = torch.zeros(c)
    for l in range(depth):
        b = f"{p}transformer_blocks.{l}."
        for n in ("norm1", "norm2", "norm3"):
            W[b + n + ".weight"] = torch.ones(c)
            W[b + n + ".bias"] = torch.zeros(c)
        for n in ("attn1.to_q", "attn1.to_k", "attn1.to_v", "attn2.to_q"):
            W[b + n + ".weight"] = torch.randn(c, c, generator=g) * 0.1
        for n in ("attn2.to_k", "attn2.to_v"):
            W[b + n + ".weight"] = torch.randn(c, 24, generator=g) * 0.1
        for n in ("attn1.to_out.0", "attn2.to_out.0"):
            W[b + n + ".weight"] = torch.zeros(c, c)
            W[b + n + ".bias"] = torch.zeros(c)
        W[b + "ff.net.0.proj.weight"] = torch.randn(8 * c, c, generator=g) * 0.1
        W[b + "ff.net.0.proj.bias"] = torch.zeros(8 * c)
        W[b + "ff.net.2.weight"] = torch.zeros(c, 4 * c)
        W[b + "ff.net.2.bias"] = torch.zeros(c)
    return W


def _t2d_case(mod):
    g = torch.Generator().manual_seed(31)
    c, depth = 64, 2
    W = _t2d_identity_blocks(c, depth, g)
    # low-variance groups (std 1e-3 around a per-group mean): eps 1e-6 and 1e-5
    # give normalised outputs that differ by a factor of about 3
    mean = torch.randn(2, 32, 1, 1, generator=g).repeat_interleave(c // 32, 1)
    x = mean + torch.randn(2, c, 6, 5, generator=g) * 1e-3
    ctx = torch.randn(2, 4, 24, generator=g)
    got = mod.transformer2d(W, "t.", x, ctx, depth)
    ref = x + F.group_norm(x, 32, W["t.norm.weight"], W["t.norm.bias"], 1e-6)
    return _agree(got, ref, 1e-4)


def test_transformer2d_identity_blocks_is_gn_residual():
    assert _t2d_case(OR)


@pytest.mark.parametrize("old,new", [
    ("w[p + \"norm.bias\"], 1e-6)", "w[p + \"norm.bias\"], 1e-5)"),
    ("h = h.permute(0, 2, 3, 1).reshape(B, H * W, C)", "h = h.permute(0, 3, 2, 1).reshape(B, H * W, C)"),
])
def test_transformer2d_catches_mutants(old, new):
    assert _fails(lambda: _t2d_case(_mutant(old, new)))


# ----------------------------------------------------------------- resnet --
def _resnet_case(mod):
    g = torch.Generator().manual_seed(41)
    c, T = 64, 48
    p = "r."
    W = {p + "norm1.weight": 1 + torch.randn(c, generator=g) * 0.2,
         p + "norm1.bias": torch.randn(c, generator=g) * 0.2,
         p + "conv1.weight": _delta3(c, 1.5),
         p + "conv1.bias": torch.randn(c, generator=g) * 0.2,
         p + "time_emb_proj.weight": torch.randn(c, T, generator=g) * 0.3,
         p + "time_emb_proj.bias": torch.randn(c, generator=g) * 0.2,
         p + "norm2.weight": 1 + torch.randn(c, generator=g) * 0.2,
         p + "norm2.bias": torch.randn(c, generator=g) * 0.2,
         p + "conv2.weight": _delta3(c, 0.75),
         p + "conv2.bias": torch.randn(c, generator=g) * 0.2}
    mean = torch.randn(2, 32, 1, 1, generator=g).repeat_interleave(2, 1)
    x = mean + torch.randn(2, c, 5, 6, generator=g) * 2e-3      # low variance: pins eps
    ts = F.silu(torch.randn(2, T, generator=g))
    got = mod.resnet_block(W, p, x, ts)
    h = F.silu(F.group_norm(x, 32, W[p + "norm1.weight"], W[p + "norm1.bias"], 1e-5))
    h = 1.5 * h + W[p + "conv1.bias"][None, :, None, None]
    h = h + F.linear(ts, W[p + "time_emb_proj.weight"], W[p + "time_emb_proj.bias"])[:, :, None, None]
    h = F.silu(F.group_norm(h, 32, W[p + "norm2.weight"], W[p + "norm2.bias"], 1e-5))
    ref = x + 0.75 * h + W[p + "conv2.bias"][None, :, None, None]
    return _agree(got, ref, 1e-4)


def test_resnet_block_closed_form():
    assert _resnet_case(OR)


@pytest.mark.parametrize("old,new", [
    ("w[p + \"norm1.bias\"], 1e-5))", "w[p + \"norm1.bias\"], 1e-6))"),
    ("    h = h + tp[:, :, None, None]\n    h = R.silu(R.group_norm(h, 32, w[p + \"norm2.weight\"], "
     "w[p + \"norm2.bias\"], 1e-5))",
     "    h = R.silu(R.group_norm(h, 32, w[p + \"norm2.weight\"], w[p + \"norm2.bias\"], 1e-5))\n"
     "    h = h + tp[:, :, None, None]"),
])
def test_resnet_block_catches_mutants(old, new):
    assert _fails(lambda: _resnet_case(_mutant(old, new)))


# ------------------------------------------------------ transformer block --
def _block_weights(c, ctx_dim, g, keep):
    """Weights of one transformer block; the three residual branches not in
    `keep` are switched off by zeroing their output projection."""
    p = "b."
    W = {}
    for n in ("norm1", "norm2", "norm3"):
        W[p + n + ".weight"] = 1 + torch.randn(c, generator=g) * 0.2
        W[p + n + ".bias"] = torch.randn(c, generator=g) * 0.2
    for n in ("attn1.to_q", "attn1.to_k", "attn1.to_v", "attn2.to_q"):
        W[p + n + ".weight"] = torch.randn(c, c, generator=g) * 0.2
    for n in ("attn2.to_k", "attn2.to_v"):
        W[p + n + ".weight"] = torch.randn(c, ctx_dim, generator=g) * 0.2
    for n in ("attn1.to_out.0", "attn2.to_out.0"):
        W[p + n + ".weight"] = torch.randn(c, c, generator=g) * 0.2
        W[p + n + ".bias"] = torch.randn(c, generator=g) * 0.2
    W[p + "ff.net.0.proj.weight"] = torch.randn(8 * c, c, generator=g) * 0.2
    W[p + "ff.net.0.proj.bias"] = torch.randn(8 * c, generator=g) * 0.2
    W[p + "ff.net.2.weight"] = torch.randn(c, 4 * c, generator=g) * 0.1
    W[p + "ff.net.2.bias"] = torch.randn(c, generator=g) * 0.2
    off = {"attn1": "attn1.to_out.0", "attn2": "attn2.to_out.0", "ff": "ff.net.2"}
    for k, n in off.items():
        if k not in keep:
            W[p + n + ".weight"].zero_()
            W[p + n + ".bias"].zero_()
    return W


def _cross_case(mod):
    """Only cross-attention on, one context token: attention returns V, so the
    block adds to_out(to_v(ctx)) to every token whatever the queries."""
    g = torch.Generator().manual_seed(51)
    c, cd = 128, 24
    W = _block_weights(c, cd, g, keep=("attn2",))
    x = torch.randn(2, 10, c, generator=g)
    ctx = torch.randn(2, 1, cd, generator=g)
    got = mod.transformer_block(W, "b.", x, ctx, c // 64)
    v = F.linear(ctx, W["b.attn2.to_v.weight"])
    ref = x + F.linear(v, W["b.attn2.to_out.0.weight"], W["b.attn2.to_out.0.bias"])
    return _agree(got, ref, 1e-5)


def _self_case(mod):
    """Only self-attention on, to_k = 0: equal keys, so each head returns the
    mean of V over tokens."""
    g = torch.Generator().manual_seed(52)
    c, cd = 128, 24
    W = _block_weights(c, cd, g, keep=("attn1",))
    W["b.attn1.to_k.weight"].zero_()
    x = torch.randn(2, 10, c, generator=g)
    ctx = torch.randn(2, 3, cd, generator=g)
    got = mod.transformer_block(W, "b.", x, ctx, c // 64)
    n = F.layer_norm(x, (c,), W["b.norm1.weight"], W["b.norm1.bias"], 1e-5)
    v = F.linear(n, W["b.attn1.to_v.weight"]).mean(dim=1, keepdim=True)
    ref = x + F.linear(v, W["b.attn1.to_out.0.weight"], W["b.attn1.to_out.0.bias"])
    return _agree(got, ref, 1e-5)


def _ff_case(mod):
    """Only the feed-forward on: value = first half of ff.net.0, gate = second
    half through erf-GELU."""
    g = torch.Generator().manual_seed(53)
    c, cd = 64, 24
    W = _block_weights(c, cd, g, keep=("ff",))
    x = torch.randn(2, 10, c, generator=g)
    ctx = torch.randn(2, 3, cd, generator=g)
    got = mod.transformer_block(W, "b.", x, ctx, c // 64)
    n = F.layer_norm(x, (c,), W["b.norm3.weight"], W["b.norm3.bias"], 1e-5)
    h = F.linear(n, W["b.ff.net.0.proj.weight"], W["b.ff.net.0.proj.bias"])
    val, gate = h[..., :4 * c], h[..., 4 * c:]
    gelu = 0.5 * gate * (1 + torch.erf(gate / math.sqrt(2.0)))
    ref = x + F.linear(val * gelu, W["b.ff.net.2.weight"], W["b.ff.net.2.bias"])
    return _agree(got, ref, 1e-5)


@pytest.mark.parametrize("case", [_cross_case, _self_case, _ff_case])
def test_transformer_block_branches(case):
    assert case(OR)


@pytest.mark.parametrize("case,old,new", [
    (_cross_case, "v = R.linear(ctx, w[p + \"attn2.to_v.weight\"])",
     "v = R.linear(n, w[p + \"attn2.to_v.weight\"])"),
    (_self_case, "n = R.layer_norm(x, w[p + \"norm1.weight\"], w[p + \"norm1.bias\"], 1e-5)",
     "n = R.layer_norm(x, w[p + \"norm2.weight\"], w[p + \"norm2.bias\"], 1e-5)"),
    (_ff_case, "n = R.layer_norm(x, w[p + \"norm3.weight\"], w[p + \"norm3.bias\"], 1e-5)",
     "n = R.layer_norm(x, w[p + \"norm2.weight\"], w[p + \"norm2.bias\"], 1e-5)"),
])
def test_transformer_block_catches_mutants(case, old, new):
    assert _fails(lambda: case(_mutant(old, new)))


def test_geglu_order_mutant_in_ref_ops_is_caught():
    """The GEGLU half order lives in ref_ops.geglu; a swapped copy must fail
    the feed-forward reduction."""
    from oracle import ref_ops

    class _Swapped:
        def __getattr__(self, k):
            if k == "geglu":
                return lambda h: ref_ops.geglu(torch.cat([h[..., h.shape[-1] // 2:],
                                                          h[..., :h.shape[-1] // 2]], -1))
            return getattr(ref_ops, k)

    m = _mutant("from . import ref_ops as R", "from . import ref_ops as R_")
    m.R = _Swapped()
    assert _fails(lambda: _ff_case(m))
