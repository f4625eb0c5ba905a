"""Per-stream library staging of the reference-layout entry points is
released with its stream (dlm_scratch_release) and does not accumulate a
set per stream (GPU).

The reference's launch_* wrappers cudaMalloc / cudaFree their temporaries
per call (src/kernels/conv2d.cu:362-448, attention.cu); this library keeps
grow-only staging per (device, stream) instead.  A caller that cycles through
streams (a stream per request, a stream pool) gets every byte back by
releasing each stream before destroying it, and results do not depend on
whether a stream's staging was freed and re-created in between.
"""
import ctypes

import pytest
import torch

from dollama_amd import _lib, ops
from tests._util import randn, to_gpu

pytestmark = pytest.mark.gpu


def _held():
    n = ctypes.c_size_t(0)
    fn = _lib.hip_lib().dlm_scratch_bytes
    fn.restype = ctypes.c_int
    assert fn(ctypes.byref(n)) == 0
    return n.value


def _release(stream):
    fn = _lib.hip_lib().dlm_scratch_release
    fn.restype = ctypes.c_int
    assert fn(ctypes.c_void_p(stream.cuda_stream)) == 0, _lib.last_error()


def test_streams_cycled_through_reference_entries_give_memory_back(gpu):
    print("[case] 6 streams x (NCHW conv 320@64x64, [B,H,S,Dh] attention 2x10x1024x64)", flush=True)
    x = to_gpu(randn((1, 320, 64, 64), 1))
    w = to_gpu(randn((320, 320, 3, 3), 2, std=0.02))
    b = to_gpu(randn((320,), 3, std=0.01))
    q, k, v = (to_gpu(randn((2, 10, 1024, 64), s)) for s in (4, 5, 6))
    torch.cuda.synchronize()
    _release(torch.cuda.current_stream())
    base = _held()  # what earlier tests' streams still hold
    outs = []
    streams = [torch.cuda.Stream() for _ in range(6)]
    for st in streams:
        with torch.cuda.stream(st):
            y = torch.empty(1, 320, 64, 64, dtype=torch.float16, device=gpu)
            o = torch.empty(2, 10, 1024, 64, dtype=torch.float16, device=gpu)
            ops.launch_conv2d(x, w, b, y, 1, 320, 64, 64, 320, 3, 3, 1, 1, 1, 1)
            ops.launch_attention(q, k, v, o, 2, 10, 1024, 1024, 64, 0.125)
            outs.append((y, o))
    torch.cuda.synchronize()
    grown = _held()
    assert grown > base, "the calls staged nothing per stream"
    per_stream = (grown - base) / len(streams)
    for st in streams:
        _release(st)
    # (<=: staging of other, older streams may have been dropped at the cap)
    assert _held() <= base, "released streams left staging behind"
    # results are the same on every stream, and again after release
    for y, o in outs[1:]:
        assert torch.equal(y, outs[0][0]) and torch.equal(o, outs[0][1])
    with torch.cuda.stream(streams[0]):
        y = torch.empty_like(outs[0][0])
        ops.launch_conv2d(x, w, b, y, 1, 320, 64, 64, 320, 3, 3, 1, 1, 1, 1)
    torch.cuda.synchronize()
    assert torch.equal(y, outs[0][0])
    _release(streams[0])
    assert _held() <= base
    print(f"[scratch] {per_stream / 2**20:.1f} MiB per stream, all returned", flush=True)
