"""The C-ABI libraries load without a GPU and export every function their
headers declare (CPU only: nothing here launches a kernel).  Also checks the
host-side error behaviour that needs no device: invalid arguments are
rejected with a status code and a message, and the host library's pure-host
entry points (config, weight list, scheduler) work."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBS = {
    "dlm.h": os.path.join(ROOT, "dollama_amd", "libdlm_hip.so"),
    "dollama.h": os.path.join(ROOT, "dollama_amd", "libdollama.so"),
}


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(dlm_\w+)\s*\(", text)))


@pytest.mark.parametrize("header", sorted(LIBS))
def test_library_exports_every_declared_symbol(header):
    path = LIBS[header]
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    names = _declared(header)
    assert len(names) > 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{os.path.basename(path)} lacks {missing}"


def test_invalid_arguments_are_rejected_without_a_device():
    lib = ctypes.CDLL(LIBS["dlm.h"])
    lib.dlm_last_error.restype = ctypes.c_char_p
    lib.dlm_linear_fp16.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    # non-positive dims are a silent no-op (the reference's convention,
    # src/kernels/conv2d.cu:762-769)
    assert lib.dlm_linear_fp16(None, 8, None, 8, None, None, 0, None, 8, 4, 4, -1, 1.0, 0.0, 0, None) == 0
    # a NULL operand with positive dims is rejected before the device is used
    rc = lib.dlm_linear_fp16(None, 8, None, 8, None, None, 0, None, 8, 4, 4, 8, 1.0, 0.0, 0, None)
    assert rc == 1  # DLM_ERR_INVALID_ARG
    assert b"NULL" in lib.dlm_last_error()


def test_groupnorm_statistics_entries_reject_bad_arguments_without_a_device():
    """The GroupNorm chunk-statistics entries check their arguments before any
    device call: NULL operands, more pixels than the chunk statistics cover,
    and a concatenation split outside (0, C)."""
    lib = ctypes.CDLL(LIBS["dlm.h"])
    lib.dlm_last_error.restype = ctypes.c_char_p
    P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    lib.dlm_group_norm_chunk_stats_fp16.argtypes = [P, I, I, I, I, P, P]
    lib.dlm_group_norm_nhwc_prestats_fp16.argtypes = [P, I, P, P, P, I, I, I, I, I, F, I, P, P]
    lib.dlm_group_norm_nhwc_prestats2_fp16.argtypes = [P, I, I, P, I, P, P, P, P, P, I, I, I, I, I, F, I, P, P]
    fake = 1 << 20  # aligned, never dereferenced: every case fails its checks first
    assert lib.dlm_group_norm_chunk_stats_fp16(None, 64, 2, 64, 64, fake, None) == 1
    assert lib.dlm_group_norm_chunk_stats_fp16(fake, 64, 2, 16385, 64, fake, None) == 1
    assert b"16384" in lib.dlm_last_error()
    assert lib.dlm_group_norm_nhwc_prestats_fp16(None, 64, None, None, fake, 64, 2, 64, 64, 32, 1e-5, 1,
                                                 fake, None) == 1
    # concat: NULL second source, then C_a outside (0, C)
    assert lib.dlm_group_norm_nhwc_prestats2_fp16(fake, 32, 32, None, 32, fake, fake, None, None, fake, 64,
                                                  2, 64, 64, 32, 1e-5, 1, fake, None) == 1
    assert b"NULL" in lib.dlm_last_error()
    assert lib.dlm_group_norm_nhwc_prestats2_fp16(fake, 64, 64, fake, 8, fake, fake, None, None, fake, 64,
                                                  2, 64, 64, 32, 1e-5, 1, fake, None) == 1
    assert b"C_a" in lib.dlm_last_error()
    # non-positive dims stay a silent no-op
    assert lib.dlm_group_norm_nhwc_prestats2_fp16(None, 32, 32, None, 32, None, None, None, None, None, 64,
                                                  0, 64, 64, 32, 1e-5, 1, None, None) == 0


def test_host_library_pure_host_entry_points():
    from dollama_amd import unet as U
    specs = U.weight_specs(U.SDXL_CONFIG)
    assert len(specs) == 1680
    assert specs["conv_in.weight"] == (320, 4, 3, 3)
    sig, ts = U.euler_schedule(20)
    assert len(sig) == 21 and ts[0] == 951.0 and ts[-1] == 1.0


def test_dispatch_timing_arm_contract_without_a_device():
    lib = ctypes.CDLL(LIBS["dlm.h"])
    lib.dlm_prof_arm.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    # both events are required
    assert lib.dlm_prof_arm(None, None) == 1  # DLM_ERR_INVALID_ARG
    # disarming when nothing is armed, or after an arm with no launch, reports 0 kernels
    assert lib.dlm_prof_disarm() == 0
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: no kernel is launched while armed
    assert lib.dlm_prof_arm(fake, fake) == 0
    assert lib.dlm_prof_disarm() == 0
    assert lib.dlm_prof_disarm() == 0
