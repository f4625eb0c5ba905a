"""ctypes binding of oracle/libnaive.so (the plain-C restatement in naive.c).

Test infrastructure only.  Every wrapper takes float32 numpy arrays (or torch
CPU tensors) in the reference's layouts and returns float32 numpy arrays.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_fp = C.POINTER(C.c_float)
_SIGS = {
    "naive_conv2d": [_fp, _fp, _fp, _fp] + [C.c_int] * 13,
    "naive_gemm": [_fp, _fp, _fp, _fp, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, C.c_int],
    "naive_group_norm": [_fp, _fp, _fp, _fp] + [C.c_int] * 5 + [C.c_float, C.c_int],
    "naive_layer_norm": [_fp, _fp, _fp, _fp, C.c_int, C.c_int, C.c_float],
    "naive_attention": [_fp, _fp, _fp, _fp] + [C.c_int] * 5 + [C.c_float],
    "naive_gelu_erf": [C.c_float],
    "naive_silu": [C.c_float],
    "naive_geglu": [_fp, _fp, C.c_int, C.c_int],
    "naive_time_embedding": [C.c_float, C.c_int, C.c_float, _fp],
    "naive_euler_schedule": [C.c_int, C.c_int, C.c_double, C.c_double, _fp, _fp],
    "naive_ssim_uniform": [_fp, _fp, C.c_int, C.c_int, C.c_int],
}
_RES = {"naive_gelu_erf": C.c_float, "naive_silu": C.c_float, "naive_euler_schedule": C.c_int,
        "naive_ssim_uniform": C.c_double}


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libnaive.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = C.CDLL(path)
        for name, args in _SIGS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = _RES.get(name, None)
        _LIB = L
    return _LIB


def _f32(x):
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(x, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data_as(_fp)


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def conv2d(x, w, b=None, stride=1, pad=1, dilation=1):
    """stride / pad / dilation: an int or an (h, w) pair."""
    x, w, b = _f32(x), _f32(w), _f32(b)
    N, Cin, H, W = x.shape
    Cout, _, KH, KW = w.shape
    (sh, sw), (ph, pw), (dh, dw) = _pair(stride), _pair(pad), _pair(dilation)
    Ho = (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1
    Wo = (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1
    out = np.empty((N, Cout, Ho, Wo), np.float32)
    lib().naive_conv2d(_p(x), _p(w), _p(b), _p(out), N, Cin, H, W, Cout, KH, KW, sh, sw,
                       ph, pw, dh, dw)
    return out


def gemm(a, b, c=None, alpha=1.0, beta=0.0, trans_b=False):
    a, b, c = _f32(a), _f32(b), _f32(c)
    M, K = a.shape
    N = b.shape[0] if trans_b else b.shape[1]
    out = np.empty((M, N), np.float32)
    lib().naive_gemm(_p(a), _p(b), _p(c), _p(out), M, N, K, alpha, beta, int(trans_b))
    return out


def group_norm(x, groups, gamma, beta, eps, silu=False):
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    N, Cc, H, W = x.shape
    out = np.empty_like(x)
    lib().naive_group_norm(_p(x), _p(gamma), _p(beta), _p(out), N, Cc, H, W, groups, eps, int(silu))
    return out


def layer_norm(x, gamma=None, beta=None, eps=1e-5):
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    Cc = x.shape[-1]
    rows = x.size // Cc
    out = np.empty_like(x)
    lib().naive_layer_norm(_p(x), _p(gamma), _p(beta), _p(out), rows, Cc, eps)
    return out


def attention(q, k, v, scale):
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, Sq, Dh = q.shape
    Sk = k.shape[2]
    out = np.empty_like(q)
    lib().naive_attention(_p(q), _p(k), _p(v), _p(out), B, H, Sq, Sk, Dh, scale)
    return out


def gelu_erf(x):
    return np.array([lib().naive_gelu_erf(float(v)) for v in np.ravel(x)], np.float32).reshape(np.shape(x))


def silu(x):
    return np.array([lib().naive_silu(float(v)) for v in np.ravel(x)], np.float32).reshape(np.shape(x))


def geglu(h):
    h = _f32(h)
    d = h.shape[-1] // 2
    tokens = h.size // (2 * d)
    out = np.empty(h.shape[:-1] + (d,), np.float32)
    lib().naive_geglu(_p(h), _p(out), tokens, d)
    return out


def time_embedding(t, dim, max_period=10000.0):
    out = np.empty(dim, np.float32)
    lib().naive_time_embedding(float(t), dim, max_period, _p(out))
    return out


def euler_schedule(steps, T=1000, beta_start=0.00085, beta_end=0.012):
    sig = np.empty(steps + 1, np.float32)
    ts = np.empty(steps, np.float32)
    rc = lib().naive_euler_schedule(steps, T, beta_start, beta_end, _p(sig), _p(ts))
    if rc:
        raise ValueError("steps and T must be positive")
    return sig, ts


def ssim_uniform(a, b):
    a, b = _f32(a), _f32(b)
    a = a.reshape(-1, a.shape[-2], a.shape[-1])
    b = b.reshape(-1, b.shape[-2], b.shape[-1])
    Cc, H, W = a.shape
    return lib().naive_ssim_uniform(_p(a), _p(b), Cc, H, W)
