"""The allocation-free reference-layout conv (dlm_conv2d_fp16_noalloc) against
the allocating entry point it varies (dlm_conv2d_fp16), through the C ABI.

Both run the same kernels (NCHW -> channels-last staging, weight repack,
implicit-GEMM conv, NCHW epilogue); the variant stages in the library's fixed
device array instead of grow-only library buffers, so its output must equal
the allocating entry point's bit for bit.  Two calls in a row, the second
smaller, check that stale contents of the shared array from the first call
never leak into the second.  A call whose staging exceeds the fixed maximum is
refused with DLM_ERR_INVALID_ARG before anything is launched.
"""
import ctypes
import math

import pytest
import torch

from dollama_amd import _lib
from oracle import ref_ops as R
from tests._util import assert_close, randn, to_gpu

pytestmark = pytest.mark.gpu


def _conv(name, x, w, b, out, geom):
    N, Cin, H, W = x.shape
    Cout, _, KH, KW = w.shape
    sh, sw, ph, pw, dh, dw = geom
    fn = getattr(_lib.hip_lib(), name)
    fn.restype = ctypes.c_int
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
            ctypes.c_void_p(b.data_ptr()), ctypes.c_void_p(out.data_ptr())]
    args += [ctypes.c_int(v) for v in (N, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, dh, dw)]
    return fn(*args, stream)


def _case(gpu, shape, geom, seed):
    N, Cin, H, W, Cout, KH, KW = shape
    sh, sw, ph, pw, dh, dw = geom
    Ho = (H + 2 * ph - dh * (KH - 1) - 1) // sh + 1
    Wo = (W + 2 * pw - dw * (KW - 1) - 1) // sw + 1
    x = randn((N, Cin, H, W), seed)
    w = randn((Cout, Cin, KH, KW), seed + 1, std=0.02)
    b = randn((Cout,), seed + 2, std=0.01)
    xg, wg, bg = to_gpu(x), to_gpu(w), to_gpu(b)
    y_ref = torch.empty(N, Cout, Ho, Wo, dtype=torch.float16, device=gpu)
    y_na = torch.full_like(y_ref, float("nan"))
    assert _conv("dlm_conv2d_fp16", xg, wg, bg, y_ref, geom) == 0, _lib.last_error()
    assert _conv("dlm_conv2d_fp16_noalloc", xg, wg, bg, y_na, geom) == 0, _lib.last_error()
    torch.cuda.synchronize()
    return x, w, b, y_ref, y_na


def test_noalloc_conv_matches_allocating_entry_point(gpu):
    print("[case] noalloc conv: 1x320x128x128 -> 320 3x3, then 2x64x17x23 -> 96 dilated",
          flush=True)
    x, w, b, y_ref, y_na = _case(gpu, (1, 320, 128, 128, 320, 3, 3), (1, 1, 1, 1, 1, 1), 40)
    assert torch.equal(y_na, y_ref), "noalloc conv differs from dlm_conv2d_fp16 (call 1)"
    assert_close(y_na, R.conv2d(x, w, b, 1, 1), "noalloc conv call 1 vs oracle")
    x, w, b, y_ref, y_na = _case(gpu, (2, 64, 17, 23, 96, 3, 3), (1, 2, 2, 1, 2, 2), 50)
    assert torch.equal(y_na, y_ref), "noalloc conv differs from dlm_conv2d_fp16 (call 2)"
    assert_close(y_na, R.conv2d(x, w, b, (1, 2), (2, 1), (2, 2)), "noalloc conv call 2 vs oracle")
    # the strided / dilated call allocates nothing either
    xg, wg, bg = to_gpu(x), to_gpu(w), to_gpu(b)
    torch.cuda.synchronize()
    before = torch.cuda.mem_get_info()[0]
    assert _conv("dlm_conv2d_fp16_noalloc", xg, wg, bg, y_na, (1, 2, 2, 1, 2, 2)) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == before
    assert torch.equal(y_na, y_ref)
    # a third call, again of the first shape, after the smaller one
    x, w, b, y_ref, y_na = _case(gpu, (1, 320, 128, 128, 320, 3, 3), (1, 1, 1, 1, 1, 1), 60)
    assert torch.equal(y_na, y_ref), "noalloc conv differs from dlm_conv2d_fp16 (call 3)"
    # a further call must leave the device's free memory where it was (its
    # operands are allocated before the reading is taken)
    xg, wg, bg = to_gpu(x), to_gpu(w), to_gpu(b)
    torch.cuda.synchronize()
    before = torch.cuda.mem_get_info()[0]
    assert _conv("dlm_conv2d_fp16_noalloc", xg, wg, bg, y_na, (1, 1, 1, 1, 1, 1)) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == before
    assert torch.equal(y_na, y_ref)


def test_noalloc_conv_under_graph_capture(gpu):
    """Captured into a HIP graph (the callers it is for), the conv replays
    bit-identical to its eager call, also after eager calls of another shape
    have overwritten the shared staging array between replays."""
    print("[case] noalloc conv captured: 2x320x64x64 -> 320 3x3, replays between eager calls",
          flush=True)
    x = to_gpu(randn((2, 320, 64, 64), 70))
    w = to_gpu(randn((320, 320, 3, 3), 71, std=0.02))
    b = to_gpu(randn((320,), 72, std=0.01))
    geom = (1, 1, 1, 1, 1, 1)
    y_eager = torch.empty(2, 320, 64, 64, dtype=torch.float16, device=gpu)
    y_graph = torch.full_like(y_eager, float("nan"))
    assert _conv("dlm_conv2d_fp16_noalloc", x, w, b, y_eager, geom) == 0, _lib.last_error()
    torch.cuda.synchronize()
    # another shape, run eagerly between replays to clobber the staging array
    xo = to_gpu(randn((2, 64, 17, 23), 73))
    wo = to_gpu(randn((96, 64, 3, 3), 74, std=0.02))
    bo = to_gpu(randn((96,), 75, std=0.01))
    yo = torch.empty(2, 96, 17, 23, dtype=torch.float16, device=gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        assert _conv("dlm_conv2d_fp16_noalloc", x, w, b, y_graph, geom) == 0, _lib.last_error()
    torch.cuda.synchronize()
    for rep in range(3):
        y_graph.fill_(float("nan"))
        assert _conv("dlm_conv2d_fp16_noalloc", xo, wo, bo, yo, geom) == 0, _lib.last_error()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_eager), f"graph replay {rep} differs from the eager call"
    del graph


def test_noalloc_conv_rejects_staging_beyond_the_fixed_maximum(gpu):
    N, Cin, H, W, Cout = 4, 640, 128, 128, 8     # staged input 80 MiB > 64 MiB
    print(f"[case] noalloc conv refusal N={N} Cin={Cin} {H}x{W}", flush=True)
    x = torch.zeros(N, Cin, H, W, dtype=torch.float16, device=gpu)
    w = torch.zeros(Cout, Cin, 1, 1, dtype=torch.float16, device=gpu)
    b = torch.zeros(Cout, dtype=torch.float16, device=gpu)
    out = torch.full((N, Cout, H, W), 7.0, dtype=torch.float16, device=gpu)
    st = _conv("dlm_conv2d_fp16_noalloc", x, w, b, out, (1, 1, 0, 0, 1, 1))
    assert st == _lib.DLM_ERR_INVALID_ARG
    assert "fixed maximum" in _lib.last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a refused call must launch nothing"
    assert math.isfinite(float(out[0, 0, 0, 0]))
