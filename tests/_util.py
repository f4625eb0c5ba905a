"""Seeded inputs and parity assertions shared by the tests."""
import torch

from oracle import metrics

REL_TOL = 1e-2
COS_TOL = 0.9999


def randn(shape, seed, std=1.0, mean=0.0):
    """fp32 normal on the CPU from a seeded generator, rounded to the fp16 grid."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g, dtype=torch.float32) * std + mean
    return x.to(torch.float16).to(torch.float32)


def to_gpu(x, dev="cuda:0"):
    return x.to(torch.float16).to(dev).contiguous()


def from_gpu(x):
    return x.detach().to("cpu", torch.float32)


def assert_close(got, ref, what, rel_tol=REL_TOL, cos_tol=COS_TOL):
    got = from_gpu(got) if isinstance(got, torch.Tensor) else got
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    r = metrics.rel_err(got, ref)
    c = metrics.cosine(got, ref)
    print(f"[parity] {what}: rel_err={r:.3e} cos={c:.7f}", flush=True)
    assert r <= rel_tol, f"{what}: rel_err {r:.3e} > {rel_tol}"
    assert c >= cos_tol, f"{what}: cosine {c:.7f} < {cos_tol}"
