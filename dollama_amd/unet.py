"""Python mirror of the reference's UNet host API over libdollama.so.

Keeps the reference's shape (src/infer/unet.cuh:53-146): a resident weight
handle (``unet_weights_create`` -> ``UNet(...)`` + ``set_weights`` +
``prepare``), a batched forward (``launch_unet_batched`` -> ``forward``),
and the stage hook used by the golden tests (``set_stage_hook``).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import CFUNCTYPE, POINTER, c_char_p, c_int, c_int64, c_size_t, c_uint64, c_void_p
from dataclasses import dataclass, fields
from typing import Callable, Dict, Optional

import torch

from . import _lib
from ._lib import DlmError

P, I = c_void_p, c_int


class UNetConfigC(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("C0", "C1", "C2", "depth1", "depth2", "head_dim", "cross_dim",
                                    "text_dim", "id_dim", "in_channels", "out_channels", "groups")]


@dataclass(frozen=True)
class UNetConfig:
    C0: int = 320
    C1: int = 640
    C2: int = 1280
    depth1: int = 2
    depth2: int = 10
    head_dim: int = 64
    cross_dim: int = 2048
    text_dim: int = 1280
    id_dim: int = 256
    in_channels: int = 4
    out_channels: int = 4
    groups: int = 32

    def to_c(self) -> UNetConfigC:
        return UNetConfigC(*[getattr(self, f.name) for f in fields(self)])


SDXL_CONFIG = UNetConfig()

STAGE_HOOK = CFUNCTYPE(None, c_char_p, c_void_p, c_size_t, c_int, c_void_p)

HOST_SIGNATURES = {
    "dlm_unet_config_sdxl": (I, [POINTER(UNetConfigC)]),
    "dlm_unet_weight_count": (I, [POINTER(UNetConfigC), POINTER(c_int)]),
    "dlm_unet_weight_spec": (I, [POINTER(UNetConfigC), I, c_char_p, I, POINTER(c_int), POINTER(c_int64)]),
    "dlm_unet_create": (I, [POINTER(UNetConfigC), POINTER(c_void_p)]),
    "dlm_unet_destroy": (I, [P]),
    "dlm_unet_set_weight": (I, [P, c_char_p, P, I, POINTER(c_int64)]),
    "dlm_unet_load_safetensors": (I, [P, c_char_p, P]),
    "dlm_unet_prepare": (I, [P, P]),
    "dlm_unet_packed_bytes": (I, [P, POINTER(c_size_t)]),
    "dlm_unet_forward": (I, [P, I, I, I, P, P, P, I, P, P, I, P, P]),
    "dlm_unet_set_stage_hook": (I, [P, STAGE_HOOK, P]),
    "dlm_unet_set_profiling": (I, [P, I]),
    "dlm_unet_set_graphs": (I, [P, I]),
    "dlm_unet_set_ln_fold": (I, [P, I]),
    "dlm_unet_set_gn_fold": (I, [P, I]),
    "dlm_unet_graphs_captured": (I, [P, POINTER(c_size_t)]),
    "dlm_unet_profile_report": (I, [P, POINTER(ctypes.c_double), P]),
    "dlm_euler_schedule": (I, [I, POINTER(ctypes.c_float), POINTER(ctypes.c_float)]),
    "dlm_pipeline_denoise": (I, [P, I, ctypes.c_float, I, I, P, P, I, P, P, P]),
    "dlm_unet_apply_lora": (I, [P, ctypes.c_char_p, P, P, I, I, I, ctypes.c_float, P]),
    "dlm_unet_load_lora": (I, [P, ctypes.c_char_p, ctypes.c_float, POINTER(c_int), P]),
    "dlm_unet_clear_loras": (I, [P, P]),
    "dlm_lora_scan": (I, [P, ctypes.c_char_p, ctypes.c_float, POINTER(c_int), P, P]),
    "dlm_unet_read_weight": (I, [P, ctypes.c_char_p, P, c_size_t, P]),
    "dlm_f32_to_f16": (I, [P, P, c_size_t]),
    "dlm_arena_stats": (I, [I, POINTER(c_uint64)]),
    "dlm_arena_fill": (I, [I, I]),
    "dlm_unet_run_resnet": (I, [P, ctypes.c_char_p, P, I, P, I, P, I, I, I, P, P]),
    "dlm_unet_profile_kernels": (I, [P, ctypes.c_char_p, c_size_t, POINTER(c_size_t), P]),
    "dlm_unet_run_transformer_block": (I, [P, ctypes.c_char_p, P, I, I, P, I, P]),
    "dlm_arena_release": (I, [I]),
    "dlm_arena_reserve": (I, [I, c_size_t]),
}

_host = None


def host_lib():
    """Load libdollama.so (which links libdlm_hip.so); raises if missing."""
    global _host
    if _host is None:
        _lib.hip_lib()
        if not os.path.exists(_lib.HOST_LIB_PATH):
            raise OSError(f"{_lib.HOST_LIB_PATH} is missing: run __graft_entry__.build()")
        lib = ctypes.CDLL(_lib.HOST_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        _lib._bind(lib, HOST_SIGNATURES)
        _host = lib
    return _host


def _call(name, *args):
    _lib.check(getattr(host_lib(), name)(*args))


def weight_specs(cfg: UNetConfig = SDXL_CONFIG) -> Dict[str, tuple]:
    """name -> shape of every parameter the GPU forward reads."""
    c = cfg.to_c()
    n = c_int()
    _call("dlm_unet_weight_count", ctypes.byref(c), ctypes.byref(n))
    out = {}
    buf = ctypes.create_string_buffer(256)
    nd = c_int()
    shp = (c_int64 * 4)()
    for i in range(n.value):
        _call("dlm_unet_weight_spec", ctypes.byref(c), i, buf, 256, ctypes.byref(nd), shp)
        out[buf.value.decode()] = tuple(shp[j] for j in range(nd.value))
    return out


ARENA_STAT_FIELDS = ("cuda_malloc_calls", "cuda_free_calls", "chunk_alloc_calls", "alloc_calls",
                     "total_capacity", "live_chunks", "bytes_in_use", "peak_bytes_in_use",
                     "live_request_bytes", "peak_request_bytes", "reserved_bytes")
ARENA_UNET, ARENA_VAE, ARENA_UNET_PERSIST = 0, 1, 2


LORA_COUNT_FIELDS = ("modules", "te_skipped", "other_keys", "incomplete")


LORA_MODULE_FN = CFUNCTYPE(None, c_char_p, c_int, c_int, c_int, ctypes.c_float, c_void_p)


def lora_scan(path: str, strength: float = 1.0, cfg: UNetConfig = SDXL_CONFIG):
    """Resolve a kohya-named LoRA file against the UNet weight names of cfg
    (host only; reference load_lora_modules, src/infer/lora.hpp:265-445).
    Returns (counts, modules) with modules = {base_key: (rank, in_flat,
    out_dim, scale)}.  Raises on a module that matches no weight or has
    mismatched shapes."""
    c = cfg.to_c()
    v = (c_int * 4)()
    mods = {}

    def _cb(key, rank, in_flat, out_dim, scale, user):
        mods[key.decode()] = (rank, in_flat, out_dim, scale)

    fn = LORA_MODULE_FN(_cb)
    _call("dlm_lora_scan", ctypes.byref(c), path.encode(), float(strength), v,
          ctypes.cast(fn, c_void_p), None)
    return dict(zip(LORA_COUNT_FIELDS, list(v))), mods


def f32_to_f16_bits(x) -> "numpy.ndarray":
    """fp32 -> fp16 bit patterns with round-to-nearest-even, as the LoRA
    loader converts F32 tensors."""
    import numpy as np
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    _call("dlm_f32_to_f16", c_void_p(a.ctypes.data), c_void_p(out.ctypes.data), a.size)
    return out


def arena_stats(arena_id: int) -> dict:
    v = (c_uint64 * 11)()
    _call("dlm_arena_stats", arena_id, v)
    return dict(zip(ARENA_STAT_FIELDS, list(v)))


def arena_fill(arena_id: int, pattern: int) -> None:
    """Fill every byte the (quiescent) arena holds with `pattern`."""
    _call("dlm_arena_fill", arena_id, pattern)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class UNet:
    """Resident-weight SDXL UNet (reference unet_weights_create + launch_unet_batched)."""

    def __init__(self, cfg: UNetConfig = SDXL_CONFIG):
        self.cfg = cfg
        self._c = cfg.to_c()
        h = c_void_p()
        _call("dlm_unet_create", ctypes.byref(self._c), ctypes.byref(h))
        self._h = h
        self._hook = None
        self._specs = weight_specs(cfg)

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            host_lib().dlm_unet_destroy(self._h)
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
            if tuple(t.shape) != tuple(shape):
                raise ValueError(f"{name}: shape {tuple(t.shape)} != {shape}")
            if not t.is_cuda or t.dtype != torch.float16 or not t.is_contiguous():
                raise ValueError(f"{name}: must be a contiguous fp16 GPU tensor")
            dims = (c_int64 * len(shape))(*shape)
            _call("dlm_unet_set_weight", self._h, name.encode(), c_void_p(t.data_ptr()), len(shape), dims)

    def prepare(self):
        _call("dlm_unet_prepare", self._h, _stream())

    def load_safetensors(self, path: str):
        _call("dlm_unet_load_safetensors", self._h, path.encode(), _stream())

    @property
    def packed_bytes(self) -> int:
        v = c_size_t()
        _call("dlm_unet_packed_bytes", self._h, ctypes.byref(v))
        return v.value

    def forward(self, latent: torch.Tensor, timesteps: torch.Tensor, ehs: torch.Tensor,
                text: torch.Tensor, time_ids: torch.Tensor, out: Optional[torch.Tensor] = None):
        """latent [B,in,H,W] fp16, timesteps [B] fp32, ehs [B,L,cross] fp16,
        text [B,text_dim] fp16, time_ids [6] or [B,6] fp16 -> noise [B,out,H,W] fp16."""
        B, cin, H, W = latent.shape
        cfg = self.cfg
        if cin != cfg.in_channels:
            raise ValueError("latent channel count mismatch")
        L = ehs.shape[1]
        checks = [(latent, torch.float16, (B, cin, H, W)), (timesteps, torch.float32, (B,)),
                  (ehs, torch.float16, (B, L, cfg.cross_dim)), (text, torch.float16, (B, cfg.text_dim))]
        for t, dt, shp in checks:
            if not t.is_cuda or t.dtype != dt or not t.is_contiguous() or tuple(t.shape) != shp:
                raise ValueError(f"bad input: expected contiguous {dt} GPU tensor of shape {shp}, "
                                 f"got {t.dtype} {tuple(t.shape)}")
        if time_ids.dtype != torch.float16 or not time_ids.is_cuda or not time_ids.is_contiguous():
            raise ValueError("time_ids must be a contiguous fp16 GPU tensor")
        if time_ids.numel() == 6:
            ids_stride = 0
        elif tuple(time_ids.shape) == (B, 6):
            ids_stride = 6
        else:
            raise ValueError("time_ids must be [6] or [B, 6]")
        if out is None:
            out = torch.empty(B, cfg.out_channels, H, W, dtype=torch.float16, device=latent.device)
        if not out.is_contiguous() or tuple(out.shape) != (B, cfg.out_channels, H, W):
            raise ValueError("bad out tensor")
        _call("dlm_unet_forward", self._h, B, H, W, c_void_p(latent.data_ptr()),
              c_void_p(timesteps.data_ptr()), c_void_p(ehs.data_ptr()), L, c_void_p(text.data_ptr()),
              c_void_p(time_ids.data_ptr()), ids_stride, c_void_p(out.data_ptr()), _stream())
        return out

    def run_resnet(self, prefix: str, x: torch.Tensor, temb: torch.Tensor,
                   x_b: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
        """One ResnetBlock2D of the prepared model: x [B,H,W,Ca] (+ x_b [B,H,W,Cb]
        concatenated) channels-last fp16, temb [B, time_dim] fp16 (the time MLP
        output, before SiLU) -> [B,H,W,Co]."""
        B, H, W, Ca = x.shape
        Cb = 0 if x_b is None else x_b.shape[3]
        T = 4 * self.cfg.C0
        ts = [(x, (B, H, W, Ca)), (temb, (B, T))] + ([] if x_b is None else [(x_b, (B, H, W, Cb))])
        for t, shp in ts:
            if not t.is_cuda or t.dtype != torch.float16 or not t.is_contiguous() or tuple(t.shape) != shp:
                raise ValueError(f"expected a contiguous fp16 GPU tensor of shape {shp}")
        co = self._resnet_out_channels(prefix)
        if out is None:
            out = torch.empty(B, H, W, co, dtype=torch.float16, device=x.device)
        if not out.is_contiguous() or tuple(out.shape) != (B, H, W, co):
            raise ValueError("bad out tensor")
        _call("dlm_unet_run_resnet", self._h, prefix.encode(), c_void_p(x.data_ptr()), Ca,
              c_void_p(0 if x_b is None else x_b.data_ptr()), Cb, c_void_p(out.data_ptr()), B, H, W,
              c_void_p(temb.data_ptr()), _stream())
        return out

    def _resnet_out_channels(self, prefix: str) -> int:
        if getattr(self, "_specs", None) is None:
            self._specs = weight_specs(self.cfg)
        shape = self._specs.get(prefix.rstrip(".") + ".conv1.weight")
        if shape is None:
            raise KeyError(f"no resnet '{prefix}'")
        return shape[0]

    def run_transformer_block(self, prefix: str, x: torch.Tensor, ehs: torch.Tensor) -> torch.Tensor:
        """One BasicTransformerBlock of the prepared model on x [B, S, C] fp16
        (updated in place and returned); ehs [B, L, cross_dim] fp16."""
        B, S, C = x.shape
        L = ehs.shape[1]
        for t, shp in ((x, (B, S, C)), (ehs, (B, L, self.cfg.cross_dim))):
            if not t.is_cuda or t.dtype != torch.float16 or not t.is_contiguous() or tuple(t.shape) != shp:
                raise ValueError(f"expected a contiguous fp16 GPU tensor of shape {shp}")
        _call("dlm_unet_run_transformer_block", self._h, prefix.encode(), c_void_p(x.data_ptr()), B, S,
              c_void_p(ehs.data_ptr()), L, _stream())
        return x

    def apply_lora(self, key: str, A: torch.Tensor, B: torch.Tensor, scale: float):
        """W += scale * (B @ A) on the resident weight `key` (diffusers name);
        A [rank, in(,kh,kw)] and B [out, rank(,1,1)] fp16 GPU tensors
        (reference src/infer/unet.cuh:97-114)."""
        for t in (A, B):
            if not t.is_cuda or t.dtype != torch.float16 or not t.is_contiguous():
                raise ValueError("LoRA factors must be contiguous fp16 GPU tensors")
        rank = A.shape[0]
        in_flat = A.numel() // max(rank, 1)
        out_dim = B.shape[0]
        if B.numel() != out_dim * rank:
            raise ValueError("B does not match the rank of A")
        _call("dlm_unet_apply_lora", self._h, key.encode(), c_void_p(A.data_ptr()),
              c_void_p(B.data_ptr()), rank, in_flat, out_dim, float(scale), _stream())

    def load_lora(self, path: str, strength: float = 1.0) -> dict:
        """Apply every UNet module of a kohya-named LoRA safetensors file with
        scale = strength * alpha / rank; returns the loader's counts."""
        v = (c_int * 4)()
        _call("dlm_unet_load_lora", self._h, path.encode(), float(strength), v, _stream())
        return dict(zip(LORA_COUNT_FIELDS, list(v)))

    def clear_loras(self):
        """Restore every weight patched by apply_lora / load_lora bit-exactly."""
        _call("dlm_unet_clear_loras", self._h, _stream())

    def read_weight(self, name: str) -> torch.Tensor:
        """The resident fp16 weight `name` as a CPU tensor in diffusers layout."""
        shape = self._specs[name]
        out = torch.empty(shape, dtype=torch.float16)
        _call("dlm_unet_read_weight", self._h, name.encode(), c_void_p(out.data_ptr()),
              out.numel() * 2, _stream())
        return out

    def set_ln_fold(self, mask: int):
        """Bit mask (0-3) of the LayerNorms folded into their consuming linears:
        bit 0 norm1 -> QKV, bit 1 norm2 -> cross-attention Q (default 3)."""
        _call("dlm_unet_set_ln_fold", self._h, int(mask))

    def set_gn_fold(self, on: bool):
        """GroupNorm statistics written by the producing convs (default on);
        off, every GroupNorm runs its own statistics pass (same bits)."""
        _call("dlm_unet_set_gn_fold", self._h, int(bool(on)))

    def set_graphs(self, on: bool):
        """HIP-graph replay of repeated forwards (needs a non-default torch stream)."""
        _call("dlm_unet_set_graphs", self._h, int(bool(on)))

    @property
    def graphs_captured(self) -> int:
        v = c_size_t()
        _call("dlm_unet_graphs_captured", self._h, ctypes.byref(v))
        return v.value

    KERNEL_CLASSES = ("conv", "linear", "attention", "groupnorm", "layernorm", "other")

    def set_profiling(self, on: bool):
        _call("dlm_unet_set_profiling", self._h, int(bool(on)))

    def profile_report(self) -> dict:
        """Per kernel class: launches, kernel ms, algorithmic FLOPs / bytes of the
        last forward run with profiling on."""
        v = (ctypes.c_double * 24)()
        _call("dlm_unet_profile_report", self._h, v, _stream())
        return {c: {"launches": int(v[4 * i]), "ms": v[4 * i + 1], "flops": v[4 * i + 2],
                    "bytes": v[4 * i + 3]} for i, c in enumerate(self.KERNEL_CLASSES)}

    def profile_kernels(self) -> dict:
        """The last profiled forward by kernel instantiation: name -> {class,
        launches, ms, flops, bytes}."""
        need = c_size_t()
        _call("dlm_unet_profile_kernels", self._h, None, 0, ctypes.byref(need), _stream())
        buf = ctypes.create_string_buffer(need.value)
        _call("dlm_unet_profile_kernels", self._h, buf, need.value, ctypes.byref(need), _stream())
        out = {}
        for line in buf.value.decode().splitlines():
            name, cls, n, ms, fl, by, dims = line.split("\t")
            problems = {}
            for item in filter(None, dims.split(";")):
                key, cnt = item.split(":")
                problems[tuple(int(v) for v in key.split(","))] = int(cnt)
            out[name] = {"class": self.KERNEL_CLASSES[int(cls)], "launches": int(n), "ms": float(ms),
                         "flops": float(fl), "bytes": float(by), "problems": problems}
        return out

    def set_stage_hook(self, fn: Optional[Callable[[str, int, int, int], None]]):
        """fn(name, device_ptr, n_elements, channels) after each stage."""
        if fn is None:
            self._hook = None
            _call("dlm_unet_set_stage_hook", self._h, STAGE_HOOK(), None)
            return

        def _cb(name, ptr, n, C, user):
            fn(name.decode(), ptr, n, C)

        self._hook = STAGE_HOOK(_cb)
        _call("dlm_unet_set_stage_hook", self._h, self._hook, None)


def random_weights(cfg: UNetConfig, seed: int, device="cuda:0", std: float = 0.02):
    """Random-init fp16 GPU weights of the architecture: matrices, kernels and
    biases ~N(0, std^2); norm scales 1 + N(0, std^2), norm shifts N(0, std^2)."""
    g = torch.Generator(device=device).manual_seed(seed)
    W = {}
    for name, shape in weight_specs(cfg).items():
        t = torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std
        parts = name.split(".")
        if "norm" in parts[-2] and parts[-1] == "weight" and len(shape) == 1:
            t += 1.0
        W[name] = t.to(torch.float16)
    return W


def euler_schedule(steps: int):
    """(sigmas[steps+1], timesteps[steps]) of the SDXL Euler discrete scheduler."""
    s = (ctypes.c_float * (steps + 1))()
    t = (ctypes.c_float * steps)()
    _call("dlm_euler_schedule", steps, s, t)
    return list(s), list(t)


def denoise(net: "UNet", latent: torch.Tensor, ehs: torch.Tensor, text: torch.Tensor,
            time_ids: torch.Tensor, steps: int = 20, guidance: float = 7.5) -> torch.Tensor:
    """Run the CFG Euler loop on the device.  latent: fp32 [C,H,W] = randn * sigma_0
    (updated in place and returned); ehs [2,L,cross] / text [2,text_dim] fp16 with the
    cond row first; time_ids [6] fp16."""
    C, H, W = latent.shape
    if latent.dtype != torch.float32 or not latent.is_cuda or not latent.is_contiguous():
        raise ValueError("latent must be a contiguous fp32 GPU tensor [C,H,W]")
    cfg = net.cfg
    if tuple(ehs.shape[::2]) != (2, cfg.cross_dim) or tuple(text.shape) != (2, cfg.text_dim):
        raise ValueError("ehs must be [2,L,cross_dim] and text [2,text_dim]")
    for t in (ehs, text, time_ids):
        if t.dtype != torch.float16 or not t.is_cuda or not t.is_contiguous():
            raise ValueError("ehs, text and time_ids must be contiguous fp16 GPU tensors")
    if time_ids.numel() != 6:
        raise ValueError("time_ids must hold 6 values")
    _call("dlm_pipeline_denoise", net._h, steps, float(guidance), H, W, c_void_p(latent.data_ptr()),
          c_void_p(ehs.data_ptr()), ehs.shape[1], c_void_p(text.data_ptr()),
          c_void_p(time_ids.data_ptr()), _stream())
    return latent
