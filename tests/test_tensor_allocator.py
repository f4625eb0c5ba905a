"""dollama::Tensor / PinnedAllocator / CudaAllocator / UniqueBuffer contracts
(the reference's src/core/tensor.hpp and allocator.hpp API, its tests
src/tests/test_tensor.cpp and test_allocator.cpp), compiled with g++ against
the headers in dollama_amd/csrc/host and run as a program."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _build(tmp_path):
    exe = tmp_path / "test_tensor_allocator"
    lib = os.path.join(ROOT, "dollama_amd")
    if not os.path.exists(os.path.join(lib, "libdlm_hip.so")):
        pytest.fail("libdlm_hip.so is not built")
    cmd = ["g++", "-std=c++20", "-O1", "-Wall", "-Wextra",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "dollama_amd", "csrc", "host"),
           os.path.join(ROOT, "tests", "cpp", "test_tensor_allocator.cpp"),
           "-L", lib, "-ldlm_hip", f"-Wl,-rpath,{lib}", "-o", str(exe)]
    subprocess.run(cmd, check=True)
    return exe


def _run(exe, mode, env=None):
    r = subprocess.run([str(exe), mode], capture_output=True, text=True, timeout=120, env=env)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr


def test_tensor_and_allocators_without_gpu(tmp_path):
    """Host tensors, the no-GPU pinned fallback and the refused device
    allocation; the GPU is hidden from the child process."""
    exe = _build(tmp_path)
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    _run(exe, "cpu", env)


@pytest.mark.gpu
def test_tensor_and_allocators_on_gpu(tmp_path, gpu):
    """Pinned and device buffers with a host -> device -> host round trip."""
    exe = _build(tmp_path)
    _run(exe, "gpu")
