"""Pins the sampling-loop arithmetic of the pipeline oracle
(oracle/pipeline_ref.py) and the ResnetBlock2D of the VAE oracle
(oracle/vae_ref.py), CPU only.

- scale_model_input and the Euler step are compared with the reference's own
  scheduler header (src/infer/scheduler.hpp:112-143), compiled on the CPU by
  oracle/Makefile into oracle/_ref/sched_ref, on a fixed vector at every step
  index of several schedules; closed forms (sigma = 0 and sqrt(3), the x0
  prediction at sigma_next = 0) pin them where the binary is absent.
- Classifier-free guidance: a stub noise predictor whose output depends on
  which conditioning a batch slot carries fixes slot 0 = cond, slot 1 =
  uncond (src/infer/diffusion.cu:878-883, 928-931) and eps = u + g (c - u)
  (:968-973) through the special cases g = 1 (the cond prediction alone) and
  g = 0 (the uncond prediction alone), and a whole two-step loop against the
  scheduler driver.
- VAE ResnetBlock2D (src/kernels/vae_decode.cu:608-652): delta-kernel convs
  reduce the block to x + s2 * SiLU(GN2(s1 * SiLU(GN1(x)) + b1)) + b2 built
  from torch.nn.functional, with a low-variance group that separates eps
  1e-6 from 1e-5, and the 1x1 shortcut case.

Every case is run against a mutant of the oracle with exactly that detail
changed (source edited in memory): each mutant must fail the case.
"""
import importlib.util
import math
import os
import subprocess
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import naive
from oracle import pipeline_ref as PR
from oracle import vae_ref as OV

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCHED_REF = os.path.join(ROOT, "oracle", "_ref", "sched_ref")


class AnchorError(Exception):
    """A mutation's anchor text is absent or not unique (a test bug)."""


def _mutant(module_file, old, new):
    """The oracle module in oracle/<module_file> with `old` replaced by `new`
    (exactly one occurrence)."""
    path = os.path.join(ROOT, "oracle", module_file)
    with open(path) as f:
        src = f.read()
    if src.count(old) != 1:
        raise AnchorError(f"mutation anchor not unique in {module_file}: {old!r}")
    src = src.replace(old, new)
    name = "oracle._mutant_" + module_file.replace(".py", "")
    spec = importlib.util.spec_from_loader(name, loader=None)
    mod = importlib.util.module_from_spec(spec)
    mod.__package__ = "oracle"
    sys.modules[name] = mod  # dataclasses look their module up by name
    try:
        exec(compile(src, module_file + "_mutant", "exec"), mod.__dict__)
    finally:
        del sys.modules[name]
    return mod


def _fails(fn):
    try:
        return not fn()
    except (RuntimeError, AssertionError, IndexError, ValueError, KeyError):
        return True


def _agree(a, b, tol=1e-6):
    a = torch.as_tensor(a, dtype=torch.float64)
    b = torch.as_tensor(b, dtype=torch.float64)
    scale = max(float(b.abs().max()), 1e-6)
    return a.shape == b.shape and float((a - b).abs().max()) <= tol * scale


# ------------------------------------------------------------ scheduler ----
def _sched_apply(steps, sample, model):
    """Run the reference scheduler's scale_model_input / step at every step
    index: -> (scaled [steps, n], stepped [steps, n]) as float32."""
    n = sample.size
    text = f"{n}\n" + " ".join(f"{v:.9g}" for v in sample) + "\n" + " ".join(f"{v:.9g}" for v in model) + "\n"
    out = subprocess.run([SCHED_REF, str(steps), "apply"], input=text, capture_output=True, text=True,
                         check=True).stdout.strip().split("\n")
    rows = np.array([list(map(float, l.split())) for l in out], dtype=np.float32)
    return rows[0::2], rows[1::2]


def _vectors(seed, n=257):
    g = np.random.default_rng(seed)
    sample = (g.standard_normal(n) * 9.0).astype(np.float32)
    model = (g.standard_normal(n) * 1.5).astype(np.float32)
    return sample, model


def _check_scale_step(mod, steps, sample, model, scaled_ref, stepped_ref):
    sig, _ = naive.euler_schedule(steps)
    x = torch.from_numpy(sample)
    e = torch.from_numpy(model)
    for i in range(steps):
        if not _agree(mod.scale_model_input(x, sig[i]), scaled_ref[i], 3e-7):
            return False
        if not _agree(mod.euler_step(x, e, sig[i], sig[i + 1]), stepped_ref[i], 3e-7):
            return False
    return True


@pytest.mark.skipif(not os.path.exists(SCHED_REF), reason="reference scheduler driver not built")
@pytest.mark.parametrize("steps", [1, 7, 20])
def test_scale_and_step_match_reference_scheduler(steps):
    sample, model = _vectors(steps)
    scaled_ref, stepped_ref = _sched_apply(steps, sample, model)
    assert _check_scale_step(PR, steps, sample, model, scaled_ref, stepped_ref)
    for old, new in [("float(sigma) ** 2 + 1.0", "float(sigma) ** 2"),
                     ("(float(sigma_next) - float(sigma))", "(float(sigma) - float(sigma_next))"),
                     ("return sample + eps *", "return sample - eps *")]:
        m = _mutant("pipeline_ref.py", old, new)
        assert _fails(lambda: _check_scale_step(m, steps, sample, model, scaled_ref, stepped_ref)), old


def _scale_step_closed_forms(mod):
    x = torch.tensor([3.0, -1.5, 0.25])
    e = torch.tensor([0.5, 2.0, -4.0])
    ok = _agree(mod.scale_model_input(x, 0.0), x, 0)                # sigma 0: identity
    ok &= _agree(mod.scale_model_input(x, math.sqrt(3.0)), x / 2, 1e-7)
    # to sigma_next = 0 the step returns the x0 prediction sample - sigma * eps
    ok &= _agree(mod.euler_step(x, e, 2.0, 0.0), x - 2.0 * e, 1e-7)
    ok &= _agree(mod.euler_step(x, e, 2.0, 2.0), x, 0)
    return ok


def test_scale_and_step_closed_forms():
    assert _scale_step_closed_forms(PR)
    for old, new in [("float(sigma) ** 2 + 1.0", "float(sigma) ** 2 + 2.0"),
                     ("(float(sigma_next) - float(sigma))", "(float(sigma) - float(sigma_next))")]:
        assert _fails(lambda: _scale_step_closed_forms(_mutant("pipeline_ref.py", old, new))), old


# -------------------------------------------------------------- CFG --------
A_COND, A_UNCOND, K_X = 0.75, -0.5, 0.125


def _stub_unet(x, t, ehs, txt, ids):
    """Noise prediction of a batch slot: the conditioning's marker value
    (ehs[b, 0, 0]) + K_X * x + 1e-3 * t; cond rows carry A_COND, uncond rows
    A_UNCOND."""
    B = x.shape[0]
    a = ehs[:, 0, 0].reshape(B, 1, 1, 1)
    return a + K_X * x + 1e-3 * t.reshape(B, 1, 1, 1)


def _cfg_inputs(cfg=True):
    ehs = torch.zeros(2 if cfg else 1, 3, 4)
    ehs[0, 0, 0] = A_COND
    if cfg:
        ehs[1, 0, 0] = A_UNCOND
    txt = torch.zeros(ehs.shape[0], 5)
    ids = torch.zeros(6)
    lat = torch.from_numpy(np.random.default_rng(7).standard_normal((1, 4, 3, 5)).astype(np.float32)) * 11.0
    return lat, ehs, txt, ids


def _one_step(mod, guidance, cfg=True):
    sig, ts = naive.euler_schedule(1)
    lat, ehs, txt, ids = _cfg_inputs(cfg)
    got = mod.denoise(_stub_unet, sig, ts, lat, ehs, txt, ids, guidance=guidance, cfg=cfg)
    return got, lat, float(sig[0]), float(sig[1]), float(ts[0])


def _cfg_special_cases(mod):
    """g = 1 takes the cond slot's prediction, g = 0 the uncond slot's, and a
    single-slot loop (no guidance) equals g = 1."""
    ok = True
    for g, a in ((1.0, A_COND), (0.0, A_UNCOND)):
        got, lat, s0, s1, t0 = _one_step(mod, g)
        x = lat / math.sqrt(s0 * s0 + 1.0)
        eps = a + K_X * x + 1e-3 * t0
        ok &= _agree(got, lat + eps * (s1 - s0), 1e-6)
    got1, *_ = _one_step(mod, 1.0)
    got_nocfg, *_ = _one_step(mod, 7.5, cfg=False)
    ok &= _agree(got_nocfg, got1, 1e-6)
    return ok


def test_cfg_slot_order_and_guidance_special_cases():
    assert _cfg_special_cases(PR)
    for old, new in [("c, u = noise[0:1], noise[1:2]", "c, u = noise[1:2], noise[0:1]"),
                     ("return u + guidance * (c - u)", "return c + guidance * (c - u)"),
                     ("float(sigma) ** 2 + 1.0", "float(sigma) ** 2")]:
        assert _fails(lambda: _cfg_special_cases(_mutant("pipeline_ref.py", old, new))), old


def _loop_vs_scheduler(mod, steps=2, guidance=7.5):
    """A two-step CFG loop over the stub against the reference scheduler's
    own scale / step (the guidance combine done here, u + g (c - u))."""
    sig, ts = naive.euler_schedule(steps)
    lat, ehs, txt, ids = _cfg_inputs()
    got = mod.denoise(_stub_unet, sig, ts, lat, ehs, txt, ids, guidance=guidance, cfg=True)
    x = lat.reshape(-1).numpy().astype(np.float32)
    for i in range(steps):
        # eps = u + g (c - u) with c, u the stub at the scaled input
        scaled, _ = _sched_apply(steps, x, np.zeros_like(x))
        xs = scaled[i].astype(np.float64)
        c = A_COND + K_X * xs + 1e-3 * ts[i]
        u = A_UNCOND + K_X * xs + 1e-3 * ts[i]
        eps = (u + guidance * (c - u)).astype(np.float32)
        _, stepped = _sched_apply(steps, x, eps)
        x = stepped[i]
    return _agree(got.reshape(-1), torch.from_numpy(x), 2e-6)


@pytest.mark.skipif(not os.path.exists(SCHED_REF), reason="reference scheduler driver not built")
def test_cfg_loop_matches_reference_scheduler():
    assert _loop_vs_scheduler(PR)
    for old, new in [("c, u = noise[0:1], noise[1:2]", "c, u = noise[1:2], noise[0:1]"),
                     ("float(sigma) ** 2 + 1.0", "float(sigma) ** 2"),
                     ("x = scale_model_input(lat, sig[i])", "x = scale_model_input(lat, sig[i + 1])")]:
        assert _fails(lambda: _loop_vs_scheduler(_mutant("pipeline_ref.py", old, new))), old


# -------------------------------------------------------- VAE resnet -------
def _delta(cout, cin, scale):
    """3x3 conv weight whose centre tap copies channel i to channel i
    (i < min(cout, cin)), times scale."""
    w = torch.zeros(cout, cin, 3, 3)
    idx = torch.arange(min(cout, cin))
    w[idx, idx, 1, 1] = scale
    return w


def _resnet_case(mod, cin, cout, seed):
    """Delta-kernel convs: the block reduces to
    shortcut(x) + s2 * SiLU(GN2(pad(s1 * SiLU(GN1(x))) + b1)) + b2."""
    g = torch.Generator().manual_seed(seed)
    p = "decoder.mid_block.resnets.0."
    s1, s2 = 1.5, 2.0
    w = {
        p + "norm1.weight": 1 + 0.2 * torch.randn(cin, generator=g),
        p + "norm1.bias": 0.3 * torch.randn(cin, generator=g),
        p + "conv1.weight": _delta(cout, cin, s1),
        p + "conv1.bias": 0.4 * torch.randn(cout, generator=g),
        p + "norm2.weight": 1 + 0.2 * torch.randn(cout, generator=g),
        p + "norm2.bias": 0.3 * torch.randn(cout, generator=g),
        p + "conv2.weight": _delta(cout, cout, s2),
        p + "conv2.bias": 0.4 * torch.randn(cout, generator=g),
    }
    if cin != cout:
        w[p + "conv_shortcut.weight"] = 0.3 * torch.randn(cout, cin, 1, 1, generator=g)
        w[p + "conv_shortcut.bias"] = 0.1 * torch.randn(cout, generator=g)
    x = torch.randn(2, cin, 6, 5, generator=g) * 2.0 + 0.5
    # group 3 of the input: 1e-3 spread, so GN1's variance (~1e-6) is of the
    # order of eps and eps = 1e-5 would change its output several-fold
    gs = cin // 32
    x[:, 3 * gs:4 * gs] = 0.7 + 1e-3 * torch.randn(2, gs, 6, 5, generator=g)
    eps = 1e-6
    h = F.silu(F.group_norm(x, 32, w[p + "norm1.weight"], w[p + "norm1.bias"], eps))
    h = s1 * h
    if cout > cin:
        h = torch.cat([h, h.new_zeros(2, cout - cin, 6, 5)], 1)
    h = h + w[p + "conv1.bias"].reshape(1, -1, 1, 1)
    h = s2 * F.silu(F.group_norm(h, 32, w[p + "norm2.weight"], w[p + "norm2.bias"], eps))
    h = h + w[p + "conv2.bias"].reshape(1, -1, 1, 1)
    sc = x if cin == cout else F.conv2d(x, w[p + "conv_shortcut.weight"], w[p + "conv_shortcut.bias"])
    return _agree(mod.resnet_block(w, p, x), sc + h, 2e-5)


def _resnet_cases(mod):
    return _resnet_case(mod, 64, 64, 1) and _resnet_case(mod, 64, 128, 2)


def test_vae_resnet_block_closed_form():
    assert _resnet_cases(OV)
    mutations = [
        ('h = R.silu(R.group_norm(h, GROUPS, w[p + "norm2.weight"], w[p + "norm2.bias"], EPS))',
         'h = R.group_norm(h, GROUPS, w[p + "norm2.weight"], w[p + "norm2.bias"], EPS)'),
        ('h = R.silu(R.group_norm(x, GROUPS, w[p + "norm1.weight"], w[p + "norm1.bias"], EPS))',
         'h = R.group_norm(x, GROUPS, w[p + "norm1.weight"], w[p + "norm1.bias"], EPS)'),
        ("EPS = 1e-6", "EPS = 1e-5"),
        ("    return x + h\n\n\ndef attn_block", "    return h\n\n\ndef attn_block"),
        ('x = R.conv2d(x, w[p + "conv_shortcut.weight"], w[p + "conv_shortcut.bias"], 1, 0)',
         'x = x[:, :1].expand(-1, h.shape[1], -1, -1)'),
    ]
    for old, new in mutations:
        assert _fails(lambda: _resnet_cases(_mutant("vae_ref.py", old, new))), old
