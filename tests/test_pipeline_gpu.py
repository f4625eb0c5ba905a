"""Device Euler / CFG kernels against the pinned pipeline oracle (GPU).

dlm_euler_cfg_step fuses the reference's host-side loop body
(src/infer/diffusion.cu:968-973: eps = u + g (c - u) over the cond / uncond
halves of the batch-2 prediction; src/infer/scheduler.hpp:122-143: latent +=
eps * (sigma_next - sigma)) with the next step's scale_model_input
(scheduler.hpp:112-120) and fp16 rounding of the model input
(diffusion.cu:899-905).  The expected values come from
oracle/pipeline_ref.py's cfg_combine / euler_step / scale_model_input
(pinned against the reference scheduler compiled on the CPU and a stub
predictor, tests/test_oracle_pipeline.py), computed in float64, on the
4x128x128 latent of a 1024x1024 image.

Bars: the fp32 latent within a few fp32 ulps of the float64 value (the
device may contract u + g (c - u) and latent + eps dt into fused
multiply-adds; the reference forms dt and the update in double); the fp16
model input equal to the rounded float64 value except where the fp32
latent's last-bit difference crosses an fp16 rounding midpoint (at most 1
fp16 ulp, on at most 0.1% of the elements).
"""
import math

import numpy as np
import pytest
import torch

from oracle import naive
from oracle import pipeline_ref as PR

pytestmark = pytest.mark.gpu

N = 4 * 128 * 128


def _inputs(seed, copies):
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(N, generator=g) * 11.0
    noise = (torch.randn(copies, N, generator=g) * 1.2).half()
    return lat, noise


def _check_latent(got, ref, scale_terms, what):
    tol = 4 * 2.0 ** -24 * scale_terms + 1e-30
    bad = (got.double() - ref).abs() > tol
    print(f"[parity] {what}: max |d| {float((got.double() - ref).abs().max()):.3e}", flush=True)
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} elements beyond a few fp32 ulps"


def _check_model_in(got, ref64, what):
    ref = ref64.to(torch.float16)
    diff = got.view(torch.int16).int() - ref.view(torch.int16).int()
    n_off = int((diff != 0).sum())
    print(f"[parity] {what}: fp16 mismatches {n_off} of {got.numel()}", flush=True)
    assert int(diff.abs().max()) <= 1, f"{what}: a model input differs by more than 1 fp16 ulp"
    assert n_off <= got.numel() // 1000, f"{what}: {n_off} fp16 mismatches"


@pytest.mark.parametrize("step", [0, 9, 19])
def test_euler_cfg_step_matches_oracle(gpu, step):
    sig, _ = naive.euler_schedule(20)
    s, sn = float(sig[step]), float(sig[step + 1])
    in_scale = 1.0 / math.sqrt(sn * sn + 1.0) if step + 1 < 20 else 1.0
    g = 7.5
    lat, noise = _inputs(100 + step, 2)
    d_lat = lat.to(gpu)
    d_noise = noise.to(gpu)
    d_in = torch.empty(2, N, dtype=torch.float16, device=gpu)
    from dollama_amd import ops
    ops.euler_cfg_step(d_lat, d_noise, d_in, g, s, sn, in_scale)
    torch.cuda.synchronize()

    nz = noise.double()
    eps = PR.cfg_combine(nz, g)[0]
    ref = PR.euler_step(lat.double(), eps, s, sn)
    terms = lat.double().abs() + g * (nz[0].abs() + nz[1].abs()) * abs(sn - s) + nz[1].abs() * abs(sn - s)
    _check_latent(d_lat.cpu(), ref, terms, f"euler_cfg_step latent (step {step})")
    mi = d_in.cpu()
    assert torch.equal(mi[0], mi[1]), "both batch slots get the same model input"
    ref_in = PR.scale_model_input(ref, sn) if step + 1 < 20 else ref
    _check_model_in(mi[0], ref_in, f"euler_cfg_step model input (step {step})")


def test_euler_step_no_guidance_matches_oracle(gpu):
    sig, _ = naive.euler_schedule(20)
    s, sn = float(sig[4]), float(sig[5])
    in_scale = 1.0 / math.sqrt(sn * sn + 1.0)
    lat, noise = _inputs(7, 1)
    d_lat = lat.to(gpu)
    d_in = torch.empty(N, dtype=torch.float16, device=gpu)
    from dollama_amd import ops
    ops.euler_step(d_lat, noise[0].to(gpu).contiguous(), d_in, s, sn, in_scale)
    torch.cuda.synchronize()
    ref = PR.euler_step(lat.double(), noise[0].double(), s, sn)
    _check_latent(d_lat.cpu(), ref, lat.double().abs() + noise[0].double().abs() * abs(sn - s),
                  "euler_step latent")
    _check_model_in(d_in.cpu(), PR.scale_model_input(ref, sn), "euler_step model input")


def test_scale_latent_first_step(gpu):
    sig, _ = naive.euler_schedule(20)
    lat, _ = _inputs(3, 1)
    d_in = torch.empty(2, N, dtype=torch.float16, device=gpu)
    from dollama_amd import ops
    ops.scale_latent(lat.to(gpu), d_in, 1.0 / math.sqrt(float(sig[0]) ** 2 + 1.0), 2)
    torch.cuda.synchronize()
    mi = d_in.cpu()
    assert torch.equal(mi[0], mi[1])
    _check_model_in(mi[0], PR.scale_model_input(lat.double(), float(sig[0])), "scale_latent")


def test_twenty_step_chain_matches_oracle(gpu):
    """The whole 20-step schedule of fused steps over fixed per-step noise
    predictions, against the oracle's chain in float64."""
    sig, _ = naive.euler_schedule(20)
    g = 7.5
    lat, _ = _inputs(11, 1)
    gen = torch.Generator().manual_seed(12)
    noises = [(torch.randn(2, N, generator=gen)).half() for _ in range(20)]
    d_lat = lat.to(gpu)
    d_in = torch.empty(2, N, dtype=torch.float16, device=gpu)
    from dollama_amd import ops
    ref = lat.double()
    for i in range(20):
        s, sn = float(sig[i]), float(sig[i + 1])
        ops.euler_cfg_step(d_lat, noises[i].to(gpu), d_in, g, s, sn,
                           1.0 / math.sqrt(sn * sn + 1.0) if i + 1 < 20 else 1.0)
        ref = PR.euler_step(ref, PR.cfg_combine(noises[i].double(), g)[0], s, sn)
    torch.cuda.synchronize()
    got = d_lat.cpu().double()
    rel = float((got - ref).abs().max() / ref.abs().max())
    print(f"[parity] 20-step Euler/CFG chain: rel {rel:.3e}", flush=True)
    assert rel <= 1e-5
    assert np.isfinite(got.numpy()).all()
