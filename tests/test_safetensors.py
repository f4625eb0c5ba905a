"""The host safetensors reader (weight loading for the UNet, VAE and runner)
against the reference's own format fixture and known answers
(src/tests/data/golden.safetensors, copied as
tests/golden/reference_format_golden.safetensors, and the expectations of
src/tests/test_safetensors.cpp: names, dtypes, shapes, values, fp16/bf16 bit
patterns, missing file, oversized header length, unknown tensor)."""
import ctypes
import os
import struct

import numpy as np
import pytest

from dollama_amd import _lib
from dollama_amd.unet import host_lib

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_format_golden.safetensors")
F32, F16, BF16, I64, I8 = 1, 2, 3, 4, 7

P = ctypes.c_void_p
SIGS = {
    "dlm_st_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(P)]),
    "dlm_st_close": (ctypes.c_int, [P]),
    "dlm_st_count": (ctypes.c_int, [P, ctypes.POINTER(ctypes.c_int)]),
    "dlm_st_name": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_char_p, ctypes.c_int]),
    "dlm_st_info": (ctypes.c_int, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                   ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_size_t)]),
    "dlm_st_read": (ctypes.c_int, [P, ctypes.c_char_p, P, ctypes.c_size_t]),
}


@pytest.fixture(scope="module")
def lib():
    L = host_lib()
    _lib._bind(L, SIGS)
    return L


def _open(lib, path):
    h = P()
    _lib.check(lib.dlm_st_open(path.encode(), ctypes.byref(h)))
    return h


def _info(lib, h, name):
    dt, nd = ctypes.c_int(), ctypes.c_int()
    shp = (ctypes.c_int64 * 8)()
    nb = ctypes.c_size_t()
    _lib.check(lib.dlm_st_info(h, name.encode(), ctypes.byref(dt), ctypes.byref(nd), shp, ctypes.byref(nb)))
    return dt.value, tuple(shp[i] for i in range(nd.value)), nb.value


def _read(lib, h, name, dtype):
    _, shape, nb = _info(lib, h, name)
    out = np.empty(nb // np.dtype(dtype).itemsize, dtype=dtype)
    _lib.check(lib.dlm_st_read(h, name.encode(), P(out.ctypes.data), nb))
    return out


def test_names_dtypes_shapes(lib):
    h = _open(lib, GOLDEN)
    n = ctypes.c_int()
    _lib.check(lib.dlm_st_count(h, ctypes.byref(n)))
    names = []
    buf = ctypes.create_string_buffer(64)
    for i in range(n.value):
        _lib.check(lib.dlm_st_name(h, i, buf, 64))
        names.append(buf.value.decode())
    assert sorted(names) == ["t_bf16", "t_f16", "t_f32", "t_i64", "t_i8"]
    assert "__metadata__" not in names
    assert _info(lib, h, "t_f32")[:2] == (F32, (2, 3))
    assert _info(lib, h, "t_f16")[:2] == (F16, (4,))
    assert _info(lib, h, "t_i64")[:2] == (I64, (2, 2))
    assert _info(lib, h, "t_i8")[:2] == (I8, (3,))
    assert _info(lib, h, "t_bf16")[:2] == (BF16, (2,))
    _lib.check(lib.dlm_st_close(h))


def test_values_and_bit_patterns(lib):
    h = _open(lib, GOLDEN)
    assert _read(lib, h, "t_f32", np.float32).tolist() == [0.0, 1.0, 2.0, 3.0, 4.0, 5.0]
    assert _read(lib, h, "t_i64", np.int64).tolist() == [1, 2, 3, 4]
    assert _read(lib, h, "t_i8", np.int8).tolist() == [-128, 0, 127]
    assert _read(lib, h, "t_f16", np.uint16).tolist() == [0x3E00, 0xC000, 0x0000, 0x7BFF]
    assert _read(lib, h, "t_bf16", np.uint16).tolist() == [0x3F80, 0xC020]
    _lib.check(lib.dlm_st_close(h))


def test_errors(lib, tmp_path):
    h = P()
    assert lib.dlm_st_open(str(tmp_path / "missing.safetensors").encode(), ctypes.byref(h)) != 0
    raw = bytearray(open(GOLDEN, "rb").read())
    raw[:8] = struct.pack("<Q", 0xFFFFFFFFFFFFFFFF)
    bad = tmp_path / "corrupt.safetensors"
    bad.write_bytes(bytes(raw))
    assert lib.dlm_st_open(str(bad).encode(), ctypes.byref(h)) != 0
    h = _open(lib, GOLDEN)
    dt, nd = ctypes.c_int(), ctypes.c_int()
    shp = (ctypes.c_int64 * 8)()
    nb = ctypes.c_size_t()
    assert lib.dlm_st_info(h, b"__nope__", ctypes.byref(dt), ctypes.byref(nd), shp, ctypes.byref(nb)) == 5
    _lib.check(lib.dlm_st_close(h))


def test_shape_whose_byte_size_wraps_is_rejected(lib, tmp_path):
    """A header whose element count times the element size wraps around 2^64
    to the stored byte range must be refused, not reported as that shape."""
    import json
    d2 = (2 ** 63 + 4) // 3            # 3 * d2 = 2^63 + 4; * 2 bytes = 2^64 + 8 -> 8 mod 2^64
    assert 3 * d2 == 2 ** 63 + 4
    hdr = json.dumps({"t": {"dtype": "F16", "shape": [3, d2], "data_offsets": [0, 8]}}).encode()
    path = tmp_path / "wrap.safetensors"
    path.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 8)
    h = P()
    assert lib.dlm_st_open(str(path).encode(), ctypes.byref(h)) != 0
    assert "overflow" in _lib.last_error()
    # the same file with an honest shape opens
    hdr = json.dumps({"t": {"dtype": "F16", "shape": [2, 2], "data_offsets": [0, 8]}}).encode()
    path.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 8)
    h = _open(lib, str(path))
    assert _info(lib, h, "t")[:2] == (F16, (2, 2))
    _lib.check(lib.dlm_st_close(h))
