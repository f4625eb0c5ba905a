"""Python mirror of the reference's VAE decoder host API over libdollama.so.

Keeps the reference's shape (src/kernels/vae_decode.cuh:50-75): a resident
weight handle (``vae_weights_create`` -> ``VAE(...)`` + ``set_weights`` +
``prepare``) and ``launch_vae_decode`` -> ``decode``, plus the stage hook the
golden tests read intermediate stages through.
"""
from __future__ import annotations

import ctypes
from ctypes import CFUNCTYPE, POINTER, c_char_p, c_int, c_int64, c_size_t, c_void_p
from dataclasses import dataclass
from typing import Callable, Dict, Optional, Tuple

import torch

from . import _lib
from .unet import _call, _stream, host_lib

P, I = c_void_p, c_int

SCALING_FACTOR = 0.13025  # SDXL VAE latent scaling factor


class VaeConfigC(ctypes.Structure):
    _fields_ = [("ch", c_int * 4), ("latent_channels", c_int), ("out_channels", c_int),
                ("layers", c_int), ("groups", c_int), ("fp32_from", c_int)]


@dataclass(frozen=True)
class VaeConfig:
    ch: Tuple[int, int, int, int] = (128, 256, 512, 512)
    latent_channels: int = 4
    out_channels: int = 3
    layers: int = 3
    groups: int = 32
    fp32_from: int = 2

    def to_c(self) -> VaeConfigC:
        return VaeConfigC((c_int * 4)(*self.ch), self.latent_channels, self.out_channels,
                          self.layers, self.groups, self.fp32_from)


SDXL_VAE_CONFIG = VaeConfig()

VAE_STAGE_HOOK = CFUNCTYPE(None, c_char_p, c_void_p, c_size_t, c_int, c_int, c_void_p)

VAE_SIGNATURES = {
    "dlm_vae_config_sdxl": (I, [POINTER(VaeConfigC)]),
    "dlm_vae_weight_count": (I, [POINTER(VaeConfigC), POINTER(c_int)]),
    "dlm_vae_weight_spec": (I, [POINTER(VaeConfigC), I, c_char_p, I, POINTER(c_int), POINTER(c_int64)]),
    "dlm_vae_create": (I, [POINTER(VaeConfigC), POINTER(c_void_p)]),
    "dlm_vae_destroy": (I, [P]),
    "dlm_vae_set_weight": (I, [P, c_char_p, P, I, POINTER(c_int64)]),
    "dlm_vae_load_safetensors": (I, [P, c_char_p, P]),
    "dlm_vae_prepare": (I, [P, P]),
    "dlm_vae_packed_bytes": (I, [P, POINTER(c_size_t)]),
    "dlm_vae_decode": (I, [P, I, I, I, P, P, P]),
    "dlm_vae_set_stage_hook": (I, [P, VAE_STAGE_HOOK, P]),
    "dlm_vae_set_profiling": (I, [P, I]),
    "dlm_vae_profile_report": (I, [P, POINTER(ctypes.c_double), P]),
}

_bound = False


def _vlib():
    global _bound
    lib = host_lib()
    if not _bound:
        _lib._bind(lib, VAE_SIGNATURES)
        _bound = True
    return lib


def _vcall(name, *args):
    _lib.check(getattr(_vlib(), name)(*args))


def weight_specs(cfg: VaeConfig = SDXL_VAE_CONFIG) -> Dict[str, tuple]:
    """name -> shape of every parameter the decoder reads (diffusers names)."""
    c = cfg.to_c()
    n = c_int()
    _vcall("dlm_vae_weight_count", ctypes.byref(c), ctypes.byref(n))
    out = {}
    buf = ctypes.create_string_buffer(256)
    nd = c_int()
    shp = (c_int64 * 4)()
    for i in range(n.value):
        _vcall("dlm_vae_weight_spec", ctypes.byref(c), i, buf, 256, ctypes.byref(nd), shp)
        out[buf.value.decode()] = tuple(shp[j] for j in range(nd.value))
    return out


def latent_to_vae(latent: torch.Tensor, scaling_factor: float = SCALING_FACTOR) -> torch.Tensor:
    """fp16(latent / scaling_factor) on the device (fp32 latent in)."""
    if not latent.is_cuda or latent.dtype != torch.float32 or not latent.is_contiguous():
        raise ValueError("latent must be a contiguous fp32 GPU tensor")
    out = torch.empty(latent.shape, dtype=torch.float16, device=latent.device)
    _lib.call("dlm_latent_to_vae_fp16", c_void_p(latent.data_ptr()), c_void_p(out.data_ptr()),
              latent.numel(), float(scaling_factor), _stream())
    return out


def image_to_rgb8(image: torch.Tensor) -> torch.Tensor:
    """[N, 3, H, W] fp16 in [-1, 1] -> [N, H, W, 3] uint8 on the device."""
    if not image.is_cuda or image.dtype != torch.float16 or not image.is_contiguous() or image.dim() != 4 \
            or image.shape[1] != 3:
        raise ValueError("image must be a contiguous fp16 GPU tensor [N, 3, H, W]")
    N, _, H, W = image.shape
    out = torch.empty(N, H, W, 3, dtype=torch.uint8, device=image.device)
    _lib.call("dlm_image_to_rgb8", c_void_p(image.data_ptr()), c_void_p(out.data_ptr()), N, H, W,
              _stream())
    return out


class VAE:
    """Resident-weight SDXL VAE decoder (reference vae_weights_create + launch_vae_decode)."""

    KERNEL_CLASSES = ("conv", "linear", "attention", "groupnorm", "other")

    def __init__(self, cfg: VaeConfig = SDXL_VAE_CONFIG):
        self.cfg = cfg
        self._c = cfg.to_c()
        h = c_void_p()
        _vcall("dlm_vae_create", ctypes.byref(self._c), ctypes.byref(h))
        self._h = h
        self._hook = None
        self._specs = weight_specs(cfg)

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            _vlib().dlm_vae_destroy(self._h)
            self._h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_weights(self, weights: Dict[str, torch.Tensor]):
        """Register fp16 GPU tensors by diffusers name (borrowed until prepare)."""
        for name, shape in self._specs.items():
            t = weights.get(name)
            if t is None:
                raise KeyError(f"missing weight {name}")
            if t.numel() != int(torch.tensor(shape).prod()):
                raise ValueError(f"{name}: shape {tuple(t.shape)} != {shape}")
            if not t.is_cuda or t.dtype != torch.float16 or not t.is_contiguous():
                raise ValueError(f"{name}: must be a contiguous fp16 GPU tensor")
            dims = (c_int64 * t.dim())(*t.shape)
            _vcall("dlm_vae_set_weight", self._h, name.encode(), c_void_p(t.data_ptr()), t.dim(), dims)

    def prepare(self):
        _vcall("dlm_vae_prepare", self._h, _stream())

    def load_safetensors(self, path: str):
        _vcall("dlm_vae_load_safetensors", self._h, path.encode(), _stream())

    @property
    def packed_bytes(self) -> int:
        v = c_size_t()
        _vcall("dlm_vae_packed_bytes", self._h, ctypes.byref(v))
        return v.value

    def decode(self, latent: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """latent [N, 4, h, w] fp16 (already / scaling_factor) -> image [N, 3, 8h, 8w] fp16."""
        if not latent.is_cuda or latent.dtype != torch.float16 or not latent.is_contiguous() \
                or latent.dim() != 4 or latent.shape[1] != self.cfg.latent_channels:
            raise ValueError("latent must be a contiguous fp16 GPU tensor [N, latent_channels, h, w]")
        N, _, h, w = latent.shape
        shape = (N, self.cfg.out_channels, 8 * h, 8 * w)
        if out is None:
            out = torch.empty(shape, dtype=torch.float16, device=latent.device)
        if not out.is_contiguous() or tuple(out.shape) != shape or out.dtype != torch.float16:
            raise ValueError("bad out tensor")
        _vcall("dlm_vae_decode", self._h, N, h, w, c_void_p(latent.data_ptr()), c_void_p(out.data_ptr()),
               _stream())
        return out

    def set_profiling(self, on: bool):
        _vcall("dlm_vae_set_profiling", self._h, int(bool(on)))

    def profile_report(self) -> dict:
        v = (ctypes.c_double * 20)()
        _vcall("dlm_vae_profile_report", self._h, v, _stream())
        return {c: {"launches": int(v[4 * i]), "ms": v[4 * i + 1], "flops": v[4 * i + 2],
                    "bytes": v[4 * i + 3]} for i, c in enumerate(self.KERNEL_CLASSES)}

    def set_stage_hook(self, fn: Optional[Callable[[str, int, int, int, bool], None]]):
        """fn(name, device_ptr, n_elements, channels, is_f32) after each stage."""
        if fn is None:
            self._hook = None
            _vcall("dlm_vae_set_stage_hook", self._h, VAE_STAGE_HOOK(), None)
            return

        def _cb(name, ptr, n, C, is_f32, user):
            fn(name.decode(), ptr, n, C, bool(is_f32))

        self._hook = VAE_STAGE_HOOK(_cb)
        _vcall("dlm_vae_set_stage_hook", self._h, self._hook, None)


def random_weights(cfg: VaeConfig, seed: int, device="cuda:0") -> Dict[str, torch.Tensor]:
    """Random-init fp16 GPU weights of the architecture: conv / linear weights
    ~N(0, 1/fan_in), biases ~N(0, 0.02^2), norm scales 1 + N(0, 0.02^2),
    norm shifts N(0, 0.02^2)."""
    g = torch.Generator(device=device).manual_seed(seed)
    W = {}
    for name, shape in weight_specs(cfg).items():
        t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
        if len(shape) >= 2:
            fan_in = 1
            for d in shape[1:]:
                fan_in *= d
            t /= fan_in ** 0.5
        else:
            t *= 0.02
            parts = name.split(".")
            if "norm" in parts[-2] and parts[-1] == "weight":
                t += 1.0
        W[name] = t.to(torch.float16)
    return W
