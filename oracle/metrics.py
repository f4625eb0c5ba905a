"""Parity metrics (test oracle only).

Tolerances follow the per-op gates of this path: relative error
max|g - r| / max|r| <= 1e-2 and cosine similarity >= 0.9999; the full UNet
uses the reference's SSIM (src/tests/test_unet.cu:161-201).
"""
from __future__ import annotations

import numpy as np
import torch


def _np64(x):
    if isinstance(x, torch.Tensor):
        x = x.detach().to("cpu", torch.float64).numpy()
    return np.asarray(x, dtype=np.float64)


def rel_err(got, ref) -> float:
    """max|g - r| / max|r| (0 when both are all-zero)."""
    g, r = _np64(got).ravel(), _np64(ref).ravel()
    den = np.max(np.abs(r)) if r.size else 0.0
    num = np.max(np.abs(g - r)) if r.size else 0.0
    if den == 0.0:
        return float(num)
    return float(num / den)


def cosine(got, ref) -> float:
    g, r = _np64(got).ravel(), _np64(ref).ravel()
    ng, nr = np.linalg.norm(g), np.linalg.norm(r)
    if ng == 0.0 and nr == 0.0:
        return 1.0
    if ng == 0.0 or nr == 0.0:
        return 0.0
    return float(np.dot(g, r) / (ng * nr))


def p99_elem_rel(got, ref, floor=1e-3) -> float:
    g, r = _np64(got).ravel(), _np64(ref).ravel()
    return float(np.percentile(np.abs(g - r) / (np.abs(r) + floor), 99)) if r.size else 0.0


def ssim_uniform(a, b) -> float:
    """SSIM as the reference computes it for noise_pred
    (src/tests/test_unet.cu:161-201): L = joint range of both arrays,
    C1 = (0.01 L)^2, C2 = (0.03 L)^2, 7x7 uniform window, centres stepped by 3
    on each channel plane, biased window variances, mean over windows.
    a, b: arrays of shape [C, H, W] (or [B, C, H, W], planes concatenated)."""
    A, Bv = _np64(a), _np64(b)
    if A.ndim == 4:
        A = A.reshape(-1, A.shape[-2], A.shape[-1])
        Bv = Bv.reshape(-1, Bv.shape[-2], Bv.shape[-1])
    lo = min(A.min(), Bv.min())
    hi = max(A.max(), Bv.max())
    L = hi - lo
    C1 = (0.01 * L) ** 2
    C2 = (0.03 * L) ** 2
    win, half = 7, 3
    C, H, W = A.shape
    ys = np.arange(half, H - half, half)
    xs = np.arange(half, W - half, half)
    # box sums via 2-D cumulative sums
    def box(x):
        s = np.zeros((C, H + 1, W + 1))
        s[:, 1:, 1:] = x.cumsum(1).cumsum(2)
        y0, x0 = ys - half, xs - half
        y1, x1 = ys + half + 1, xs + half + 1
        return (s[:, y1][:, :, x1] - s[:, y0][:, :, x1] - s[:, y1][:, :, x0] + s[:, y0][:, :, x0])
    inv = 1.0 / (win * win)
    sa, sb = box(A) * inv, box(Bv) * inv
    saa, sbb, sab = box(A * A) * inv, box(Bv * Bv) * inv, box(A * Bv) * inv
    va = saa - sa * sa
    vb = sbb - sb * sb
    cov = sab - sa * sb
    ssim = ((2 * sa * sb + C1) * (2 * cov + C2)) / ((sa * sa + sb * sb + C1) * (va + vb + C2))
    return float(ssim.mean()) if ssim.size else 0.0


def ssim_uniform_loops(a, b) -> float:
    """Direct loop form of ``ssim_uniform`` (small inputs only), kept as an
    independent restatement to pin the vectorised one."""
    A, Bv = _np64(a), _np64(b)
    if A.ndim == 4:
        A = A.reshape(-1, A.shape[-2], A.shape[-1])
        Bv = Bv.reshape(-1, Bv.shape[-2], Bv.shape[-1])
    lo = min(A.min(), Bv.min())
    hi = max(A.max(), Bv.max())
    L = hi - lo
    C1, C2 = (0.01 * L) ** 2, (0.03 * L) ** 2
    half = 3
    inv = 1.0 / 49.0
    total, cnt = 0.0, 0
    C, H, W = A.shape
    for c in range(C):
        for y in range(half, H - half, half):
            for x in range(half, W - half, half):
                sa = sb = saa = sbb = sab = 0.0
                for dy in range(-half, half + 1):
                    for dx in range(-half, half + 1):
                        va, vb = A[c, y + dy, x + dx], Bv[c, y + dy, x + dx]
                        sa += va; sb += vb; saa += va * va; sbb += vb * vb; sab += va * vb
                mu_a, mu_b = sa * inv, sb * inv
                var_a = saa * inv - mu_a * mu_a
                var_b = sbb * inv - mu_b * mu_b
                cov = sab * inv - mu_a * mu_b
                total += ((2 * mu_a * mu_b + C1) * (2 * cov + C2)) / (
                    (mu_a * mu_a + mu_b * mu_b + C1) * (var_a + var_b + C2))
                cnt += 1
    return total / cnt if cnt else 0.0
