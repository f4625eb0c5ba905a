"""ctypes binding of the C ABI declared in include/dlm.h.

The shared libraries are built in place by ``__graft_entry__.build()``
(``dollama_amd/csrc/Makefile``).  There is no fallback: if ``libdlm_hip.so``
is missing, loading raises, so no GPU path can silently run on the CPU.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_longlong, c_size_t, c_void_p

_HERE = os.path.dirname(os.path.abspath(__file__))
HIP_LIB_PATH = os.path.join(_HERE, "libdlm_hip.so")
HOST_LIB_PATH = os.path.join(_HERE, "libdollama.so")

DLM_OK = 0
DLM_ERR_INVALID_ARG = 1
DLM_ERR_HIP = 2
DLM_ERR_OUT_OF_MEMORY = 3
DLM_ERR_UNSUPPORTED = 4
DLM_ERR_NOT_FOUND = 5
DLM_ERR_STATE = 6

ACT_NONE, ACT_SILU, ACT_GEGLU, ACT_GELU = 0, 1, 2, 3

P = c_void_p
I = c_int
F = c_float
LL = c_longlong


class ConvNhwcArgs(ctypes.Structure):
    _fields_ = [
        ("src0a", P), ("src0b", P), ("C0a", I), ("C0b", I), ("ld0a", I), ("ld0b", I),
        ("src1a", P), ("src1b", P), ("C1a", I), ("C1b", I), ("ld1a", I), ("ld1b", I),
        ("N", I), ("H", I), ("W", I), ("KH", I), ("KW", I), ("stride", I), ("pad", I),
        ("upsample", I),
        ("weight", P), ("ldw", I), ("Cout", I),
        ("bias", P), ("tbias", P), ("tbias_ld", I),
        ("residual", P), ("res_ld", I),
        ("out", P), ("ldy", I), ("out_nchw", I), ("act", I),
        ("out_f32", I), ("res_f32", I),
        ("gn_stats", P),
    ]


class AttentionArgs(ctypes.Structure):
    _fields_ = [
        ("q", P), ("q_sb", LL), ("q_ss", LL), ("q_sh", LL),
        ("k", P), ("k_sb", LL), ("k_ss", LL), ("k_sh", LL),
        ("v", P), ("v_sb", LL), ("v_ss", LL), ("v_sh", LL),
        ("o", P), ("o_sb", LL), ("o_ss", LL), ("o_sh", LL),
        ("B", I), ("H", I), ("Sq", I), ("Sk", I), ("Dh", I), ("scale", F),
    ]


class AttentionVtArgs(ctypes.Structure):
    _fields_ = [
        ("q", P), ("k", P), ("vt", P), ("o", P),
        ("q_sb", LL), ("q_ss", LL), ("q_sh", LL),
        ("k_sb", LL), ("k_ss", LL), ("k_sh", LL),
        ("vt_sb", LL), ("vt_sh", LL),
        ("o_sb", LL), ("o_ss", LL), ("o_sh", LL),
        ("vt_ld", I), ("B", I), ("H", I), ("Sq", I), ("Sk", I), ("scale", F),
        ("k_bytes", ctypes.c_ulonglong), ("vt_bytes", ctypes.c_ulonglong),
    ]


# name -> (restype, argtypes); every int-returning entry point is a status.
HIP_SIGNATURES = {
    "dlm_last_error": (c_char_p, []),
    "dlm_get_device_count": (I, [POINTER(c_int)]),
    "dlm_set_device": (I, [I]),
    "dlm_device_arch": (I, [ctypes.c_char_p, I]),
    "dlm_malloc": (I, [POINTER(c_void_p), c_size_t]),
    "dlm_free": (I, [P]),
    "dlm_host_malloc_pinned": (I, [POINTER(c_void_p), c_size_t]),
    "dlm_host_free_pinned": (I, [P]),
    "dlm_memcpy": (I, [P, P, c_size_t, I]),
    "dlm_memcpy_async": (I, [P, P, c_size_t, I, P]),
    "dlm_memset_async": (I, [P, I, c_size_t, P]),
    "dlm_device_synchronize": (I, []),
    "dlm_mem_get_info": (I, [POINTER(c_size_t), POINTER(c_size_t)]),
    "dlm_stream_create": (I, [POINTER(c_void_p)]),
    "dlm_stream_destroy": (I, [P]),
    "dlm_stream_synchronize": (I, [P]),
    "dlm_event_create": (I, [POINTER(c_void_p)]),
    "dlm_event_destroy": (I, [P]),
    "dlm_event_record": (I, [P, P]),
    "dlm_event_synchronize": (I, [P]),
    "dlm_event_elapsed_ms": (I, [POINTER(c_float), P, P]),
    "dlm_prof_arm": (I, [P, P]),
    "dlm_prof_disarm": (I, []),
    "dlm_conv2d_fp16": (I, [P, P, P, P] + [I] * 13 + [P]),
    "dlm_gemm_fp16": (I, [P, P, P, I, I, I, F, F, I, I, P]),
    "dlm_group_norm_fp16": (I, [P, P, P, P, I, I, I, I, I, F, I, P]),
    "dlm_layer_norm_fp16": (I, [P, P, P, P, I, I, F, P]),
    "dlm_attention_fp16": (I, [P, P, P, P, I, I, I, I, I, F, P]),
    "dlm_geglu_fp16": (I, [P, P, I, I, P]),
    "dlm_silu_fp16": (I, [P, P, I, P]),
    "dlm_gelu_fp16": (I, [P, P, I, P]),
    "dlm_gelu_tanh_fp16": (I, [P, P, I, P]),
    "dlm_add_fp16": (I, [P, P, P, I, P]),
    "dlm_upsample_nearest2x_fp16": (I, [P, P, I, I, I, I, P]),
    "dlm_bias_add_rowvec_fp16": (I, [P, P, P, I, I, P]),
    "dlm_bias_add_channel_fp16": (I, [P, P, P, I, I, I, I, P]),
    "dlm_conv_bias_biasch_fp16": (I, [P, P, P, P, I, I, I, I, P]),
    "dlm_conv_bias_residual_fp16": (I, [P, P, P, P, I, I, I, I, P]),
    "dlm_timestep_embedding_fp16": (I, [P, F, I, F, P]),
    "dlm_linear_fp16": (I, [P, I, P, I, P, P, I, P, I, I, I, I, F, F, I, P]),
    "dlm_linear_gn_stats_fp16": (I, [P, I, P, I, P, P, I, P, I, I, I, I, F, F, I, I, P, P]),
    "dlm_geglu_pack_fp16": (I, [P, P, P, P, I, I, P]),
    "dlm_conv_weight_pack_fp16": (I, [P, P, I, I, I, I, I, I, I, P]),
    "dlm_nchw_to_nhwc_fp16": (I, [P, P, I, I, I, I, P]),
    "dlm_nhwc_to_nchw_fp16": (I, [P, P, I, I, I, I, P]),
    "dlm_conv2d_nhwc_fp16": (I, [POINTER(ConvNhwcArgs), P]),
    "dlm_group_norm_nhwc_workspace_bytes": (c_size_t, [I, I, I]),
    "dlm_group_norm_nhwc_fp16": (I, [P, I, I, P, I, P, P, P, I, I, I, I, I, F, I, P, P]),
    "dlm_attention_strided_fp16": (I, [POINTER(AttentionArgs), P]),
    "dlm_attention_vt_fp16": (I, [POINTER(AttentionVtArgs), P]),
    "dlm_linear_vt_fp16": (I, [P, I, P, I, P, P, I, P, I, I, I, I, I, I, P]),
    "dlm_linear_ln_fp16": (I, [P, I, P, I, P, P, F, P, I, P, I, I, I, I, F, I, P]),
    "dlm_linear_vt_ln_fp16": (I, [P, I, P, I, P, P, F, P, I, P, I, I, I, I, I, I, P]),
    "dlm_ln_fold_fp16": (I, [P, I, I, I, P, P, P, P, I, P, P, P]),
    "dlm_sdxl_embed_inputs_fp16": (I, [P, P, I, P, I, I, P, I, P, I, P]),
    "dlm_linear_small_fp16": (I, [P, I, P, P, P, I, I, I, I, I, I, I, P]),
    "dlm_euler_cfg_step": (I, [P, P, P, I, F, F, F, F, P]),
    "dlm_euler_step": (I, [P, P, P, I, F, F, F, P]),
    "dlm_scale_latent_fp16": (I, [P, P, I, F, I, P]),
    "dlm_linear_f32out_fp16": (I, [P, I, P, I, P, P, I, P, I, I, I, I, F, F, I, P]),
    "dlm_group_norm_nhwc_f32in": (I, [P, I, P, P, P, I, I, I, I, I, F, I, P, P]),
    "dlm_group_norm_nhwc_prestats_fp16": (I, [P, I, P, P, P, I, I, I, I, I, F, I, P, P]),
    "dlm_group_norm_nhwc_prestats2_fp16": (I, [P, I, I, P, I, P, P, P, P, P, I, I, I, I, I, F, I, P, P]),
    "dlm_group_norm_chunk_stats_fp16": (I, [P, I, I, I, I, P, P]),
    "dlm_cast_f32_to_f16": (I, [P, P, LL, F, P]),
    "dlm_scale_fp16": (I, [P, LL, F, P]),
    "dlm_latent_to_vae_fp16": (I, [P, P, LL, F, P]),
    "dlm_image_to_rgb8": (I, [P, P, I, I, I, P]),
    "dlm_softmax_rows_f32_fp16": (I, [P, LL, P, LL, I, I, P]),
    "dlm_gemm_force_tile": (I, [I]),
    "dlm_gemm_override_shape": (I, [I, I, I, I, I]),
    "dlm_gemm_force_split": (I, [I]),
    "dlm_gemm_set_variant": (I, [I]),
    "dlm_mfma_probe": (I, [I, I, P, P]),
    "dlm_scratch_release": (I, [P]),
    "dlm_scratch_bytes": (I, [POINTER(c_size_t)]),
}


class DlmError(RuntimeError):
    """A C-ABI call returned a non-zero status (the reference throws
    std::runtime_error from its launch_* wrappers, src/kernels/utils.cuh:17-45)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[dlm status {code}] {msg}")
        self.code = code


_hip = None


def _bind(lib, table):
    for name, (res, args) in table.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def hip_lib():
    """Load libdlm_hip.so (raises OSError if it has not been built)."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_LIB_PATH):
            raise OSError(
                f"{HIP_LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        lib = ctypes.CDLL(HIP_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        _bind(lib, HIP_SIGNATURES)
        _hip = lib
    return _hip


def last_error() -> str:
    return hip_lib().dlm_last_error().decode(errors="replace")


def check(status: int) -> None:
    if status != DLM_OK:
        raise DlmError(status, last_error())


def call(name: str, *args) -> None:
    check(getattr(hip_lib(), name)(*args))
