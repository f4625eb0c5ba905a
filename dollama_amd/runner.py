"""Python mirror of the reference's diffusion runner and backend plugin API.

``DiffusionRunner`` wraps ``make_diffusion_runner`` / ``IDiffusionRunner``
(src/server/diffusion_runner.hpp:33-79): ``run_txt2img`` (CFG with caller
conditioning), ``generate`` (guidance 1, conditioning from the embeddings
file), ``apply_loras`` / ``clear_loras``.  ``Backend`` wraps ``make_backend``
/ ``IDiffusionBackend`` (src/server/diffusion_backend.hpp:40-126) for the
"sdxl" backend over precomputed conditioning.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_size_t, c_uint64, c_void_p
from typing import Optional, Sequence, Tuple

import numpy as np

from . import _lib
from .unet import SDXL_CONFIG, UNetConfig, UNetConfigC, host_lib
from .vae import SDXL_VAE_CONFIG, SCALING_FACTOR, VaeConfig, VaeConfigC

P, I = c_void_p, c_int


class BackendConfigC(ctypes.Structure):
    _fields_ = [("backend_name", c_char_p), ("preset", c_char_p), ("unet_weights", c_char_p),
                ("vae_weights", c_char_p), ("embeds", c_char_p), ("vae_scaling_factor", c_float),
                ("unet_cfg", POINTER(UNetConfigC)), ("vae_cfg", POINTER(VaeConfigC)),
                ("latent_size", c_int)]


RUNNER_SIGNATURES = {
    "dlm_runner_create": (I, [c_char_p, c_char_p, c_char_p, c_float, POINTER(UNetConfigC),
                              POINTER(VaeConfigC), I, I, POINTER(c_void_p)]),
    "dlm_runner_destroy": (I, [P]),
    "dlm_runner_txt2img": (I, [P, I, c_uint64, c_float, P, P, P, P, P, P, c_size_t, POINTER(c_int),
                               POINTER(c_int)]),
    "dlm_runner_generate": (I, [P, I, c_uint64, P, c_size_t, POINTER(c_int), POINTER(c_int)]),
    "dlm_runner_apply_loras": (I, [P, POINTER(c_char_p), POINTER(c_float), I]),
    "dlm_runner_clear_loras": (I, [P]),
    "dlm_backend_create": (I, [POINTER(BackendConfigC), POINTER(c_void_p)]),
    "dlm_backend_destroy": (I, [P]),
    "dlm_backend_generate": (I, [P, c_char_p, c_char_p, I, c_uint64, c_float, I, I, P, c_size_t,
                                 POINTER(c_int), POINTER(c_int)]),
    "dlm_backend_info": (I, [P, c_char_p, I, POINTER(c_int), POINTER(c_int), POINTER(c_int)]),
    "dlm_backend_model_id": (I, [P, c_char_p, I]),
    "dlm_backend_apply_loras": (I, [P, POINTER(c_char_p), POINTER(c_float), I]),
    "dlm_backend_clear_loras": (I, [P]),
    "dlm_randn_latent": (I, [c_uint64, c_double, P, c_size_t]),
}

_bound = False


def _rlib():
    global _bound
    lib = host_lib()
    if not _bound:
        _lib._bind(lib, RUNNER_SIGNATURES)
        _bound = True
    return lib


def _rcall(name, *args):
    _lib.check(getattr(_rlib(), name)(*args))


def randn_latent(seed: int, sigma0: float, n: int) -> np.ndarray:
    """float32 [n] = z * sigma0 from the reference's seeded normal stream (host)."""
    out = np.empty(n, dtype=np.float32)
    _rcall("dlm_randn_latent", c_uint64(seed), float(sigma0), c_void_p(out.ctypes.data), n)
    return out


def _f32(a, n, name):
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32).reshape(-1))
    if a.size != n:
        raise ValueError(f"{name}: {a.size} elements, expected {n}")
    return a


def _strs(items):
    arr = (c_char_p * len(items))(*[s.encode() for s in items])
    return arr


class DiffusionRunner:
    """make_diffusion_runner(...) -> IDiffusionRunner."""

    def __init__(self, unet_weights: str, vae_weights: str, embeds: str,
                 vae_scaling_factor: float = SCALING_FACTOR, unet_cfg: UNetConfig = SDXL_CONFIG,
                 vae_cfg: VaeConfig = SDXL_VAE_CONFIG, latent_size: Tuple[int, int] = (128, 128)):
        self.unet_cfg, self.vae_cfg = unet_cfg, vae_cfg
        self.latent_size = latent_size
        self._uc, self._vc = unet_cfg.to_c(), vae_cfg.to_c()
        h = c_void_p()
        _rcall("dlm_runner_create", unet_weights.encode(), vae_weights.encode(), embeds.encode(),
               float(vae_scaling_factor), ctypes.byref(self._uc), ctypes.byref(self._vc),
               latent_size[0], latent_size[1], ctypes.byref(h))
        self._h = h

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            _rlib().dlm_runner_destroy(self._h)
            self._h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _rgb_buf(self):
        lh, lw = self.latent_size
        return np.empty((8 * lh, 8 * lw, 3), dtype=np.uint8)

    def run_txt2img(self, steps: int, seed: int, guidance: float, cond_ehs, cond_text, uncond_ehs,
                    uncond_text, time_ids) -> np.ndarray:
        """RGB8 [h, w, 3] (reference run_txt2img); conditioning as host arrays."""
        ne = cond_ehs.size if hasattr(cond_ehs, "size") else len(cond_ehs)
        nt = self.unet_cfg.text_dim
        ce, ue = _f32(cond_ehs, ne, "cond_ehs"), _f32(uncond_ehs, ne, "uncond_ehs")
        ct, ut = _f32(cond_text, nt, "cond_text"), _f32(uncond_text, nt, "uncond_text")
        ids = _f32(time_ids, 6, "time_ids")
        out = self._rgb_buf()
        w, h = c_int(), c_int()
        _rcall("dlm_runner_txt2img", self._h, steps, c_uint64(seed), float(guidance),
               *[c_void_p(a.ctypes.data) for a in (ce, ct, ue, ut, ids)], c_void_p(out.ctypes.data),
               out.size, ctypes.byref(w), ctypes.byref(h))
        return out[: h.value, : w.value]

    def generate(self, steps: int, seed: int) -> np.ndarray:
        """RGB8 [h, w, 3] without guidance, conditioning from the embeddings file."""
        out = self._rgb_buf()
        w, h = c_int(), c_int()
        _rcall("dlm_runner_generate", self._h, steps, c_uint64(seed), c_void_p(out.ctypes.data),
               out.size, ctypes.byref(w), ctypes.byref(h))
        return out[: h.value, : w.value]

    def apply_loras(self, reqs: Sequence[Tuple[str, float]]):
        paths = _strs([p for p, _ in reqs])
        st = (c_float * len(reqs))(*[s for _, s in reqs])
        _rcall("dlm_runner_apply_loras", self._h, paths, st, len(reqs))

    def clear_loras(self):
        _rcall("dlm_runner_clear_loras", self._h)


class Backend:
    """make_backend(BackendConfig) -> IDiffusionBackend ("sdxl")."""

    def __init__(self, backend_name: str, unet_weights: str, vae_weights: str, embeds: str,
                 preset: str = "", vae_scaling_factor: float = SCALING_FACTOR,
                 unet_cfg: UNetConfig = SDXL_CONFIG, vae_cfg: VaeConfig = SDXL_VAE_CONFIG,
                 latent_size: int = 128):
        self._uc, self._vc = unet_cfg.to_c(), vae_cfg.to_c()
        self._cfg = BackendConfigC(backend_name.encode(), preset.encode(), unet_weights.encode(),
                                   vae_weights.encode(), embeds.encode(), float(vae_scaling_factor),
                                   ctypes.pointer(self._uc), ctypes.pointer(self._vc), latent_size)
        self.latent_size = latent_size
        h = c_void_p()
        _rcall("dlm_backend_create", ctypes.byref(self._cfg), ctypes.byref(h))
        self._h = h

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            _rlib().dlm_backend_destroy(self._h)
            self._h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def generate(self, prompt: str = "", negative: str = "", steps: int = 0, seed: int = 0,
                 cfg: float = 0.0, w: int = 0, h: int = 0) -> np.ndarray:
        out = np.empty((8 * self.latent_size, 8 * self.latent_size, 3), dtype=np.uint8)
        wo, ho = c_int(), c_int()
        _rcall("dlm_backend_generate", self._h, prompt.encode(), negative.encode(), steps, c_uint64(seed),
               float(cfg), w, h, c_void_p(out.ctypes.data), out.size, ctypes.byref(wo), ctypes.byref(ho))
        return out[: ho.value, : wo.value]

    def info(self) -> dict:
        name = ctypes.create_string_buffer(64)
        lc, nr, t5 = c_int(), c_int(), c_int()
        _rcall("dlm_backend_info", self._h, name, 64, ctypes.byref(lc), ctypes.byref(nr), ctypes.byref(t5))
        return {"name": name.value.decode(), "latent_channels": lc.value,
                "native_resolution": nr.value, "needs_t5": bool(t5.value)}

    def model_id(self) -> str:
        buf = ctypes.create_string_buffer(256)
        _rcall("dlm_backend_model_id", self._h, buf, 256)
        return buf.value.decode()

    def apply_loras(self, reqs: Sequence[Tuple[str, float]]):
        names = _strs([n for n, _ in reqs])
        st = (c_float * len(reqs))(*[s for _, s in reqs])
        _rcall("dlm_backend_apply_loras", self._h, names, st, len(reqs))

    def clear_loras(self):
        _rcall("dlm_backend_clear_loras", self._h)
