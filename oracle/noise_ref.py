"""Restatement of the reference's initial-noise generator (test oracle only).

src/infer/diffusion.cu:80-136 (class Randn) and :828-835 (initial latent):
  - state s0 = splitmix64(seed), s1 = splitmix64(seed + 0x9E3779B97F4A7C15),
    splitmix64 being the output function of Steele, Lea and Flood's
    SplitMix64 (add the golden gamma, two xor-shift-multiply rounds, a final
    xor-shift);
  - uniform(): one xorshift128+ step (Vigna 2014, shifts 23, 17, 26) whose
    output s1_new + s1_old keeps its top 53 bits as k / 2^53 in [0, 1);
  - next(): Box-Muller on (u1, u2), u1 redrawn while <= 1e-12, returning
    r cos(2 pi u2) first and r sin(2 pi u2) on the following call;
  - latent[k] = float(next() * double(sigma_0)).

Pins (tests/test_oracle.py): the splitmix64 known answer for seed 0, the
primitivity of the xorshift128+ transition's characteristic polynomial
(the full-period property of the published shift triple), the Box-Muller
pairing and moments, and agreement with the product's C++ generator.
"""
from __future__ import annotations

import math

import numpy as np

M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def splitmix64(x: int) -> int:
    x = (x + GOLDEN) & M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


class XorShift128Plus:
    def __init__(self, s0: int, s1: int):
        self.s0, self.s1 = s0 & M64, s1 & M64

    def step(self) -> int:
        """Advance once; return the 64-bit output s1_new + s1_old."""
        a, b = self.s0, self.s1
        self.s0 = b
        a = (a ^ (a << 23)) & M64
        self.s1 = a ^ b ^ (a >> 17) ^ (b >> 26)
        return (self.s1 + b) & M64


class Randn:
    def __init__(self, seed: int):
        self.g = XorShift128Plus(splitmix64(seed), splitmix64((seed + GOLDEN) & M64))
        self.spare = None

    def uniform(self) -> float:
        return (self.g.step() >> 11) * (1.0 / 9007199254740992.0)

    def next(self) -> float:
        if self.spare is not None:
            z, self.spare = self.spare, None
            return z
        u1 = self.uniform()
        while u1 <= 1e-12:
            u1 = self.uniform()
        u2 = self.uniform()
        r = math.sqrt(-2.0 * math.log(u1))
        th = 2.0 * math.pi * u2
        self.spare = r * math.sin(th)
        return r * math.cos(th)


def randn_latent(seed: int, sigma0: float, n: int) -> np.ndarray:
    g = Randn(seed)
    return np.array([g.next() * sigma0 for _ in range(n)], dtype=np.float64).astype(np.float32)
