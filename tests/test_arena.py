"""Device arena contracts (the reference's src/tests/test_device_arena.cu and
the poisoned-arena gate of src/tests/test_unet_fast.cu:136-172).

- The arena API cases run as a C++ program against libdollama.so, once with
  the pool on and once in a process started with DOLLAMA_POOL=0
  (src/meson.build:732 runs the reference's test that way too).
- UNet forwards stay bit-identical when the UNet arenas are filled with 0xFF,
  0x00 and 0xA5 between forwards, eager and as graph replays: no kernel reads
  scratch it has not written.
- A forward in a DOLLAMA_POOL=0 process (every scratch buffer its own
  allocation, freed at rewind) equals the pooled forward bit for bit.
"""
import os
import subprocess
import sys

import pytest
import torch

from dollama_amd import unet as U
from oracle import unet_ref as OR

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TINY = U.UNetConfig(C0=64, C1=128, C2=192, depth1=1, depth2=2, cross_dim=96, text_dim=64, id_dim=16)


def _build(tmp_path):
    exe = tmp_path / "test_device_arena"
    lib = os.path.join(ROOT, "dollama_amd")
    cmd = ["g++", "-std=c++20", "-O1", "-Wall", "-pthread",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "dollama_amd", "csrc", "host"),
           os.path.join(ROOT, "tests", "cpp", "test_device_arena.cpp"),
           "-L", lib, "-ldollama", "-ldlm_hip", f"-Wl,-rpath,{lib}", "-o", str(exe)]
    subprocess.run(cmd, check=True)
    return exe


@pytest.mark.parametrize("pool", ["1", "0"])
def test_device_arena_contract(gpu, tmp_path, pool):
    print(f"[case] device arena contract DOLLAMA_POOL={pool}", flush=True)
    exe = _build(tmp_path)
    env = dict(os.environ, DOLLAMA_POOL=pool)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"pool={pool}: 0 failure(s)" in r.stdout


def _tiny_inputs(seed=31):
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(2, 4, 32, 32, generator=g).half()
    ehs = torch.randn(2, 77, 96, generator=g).half()
    text = torch.randn(2, 64, generator=g).half()
    ts = torch.full((2,), 999.0)
    ids = torch.tensor([1024.0, 1024.0, 0.0, 0.0, 1024.0, 1024.0]).half()
    return lat, ts, ehs, text, ids


def _tiny_net(seed=30):
    W = OR.random_weights(OR.TINY, seed=seed)
    net = U.UNet(TINY)
    net.set_weights({k: v.half().cuda() for k, v in W.items()})
    net.prepare()
    return net


def test_unet_forward_bit_exact_over_poisoned_arenas(gpu):
    print("[case] tiny UNet B=2 32x32 forwards over arenas filled 0xFF / 0x00 / 0xA5", flush=True)
    net = _tiny_net()
    args = [t.cuda() for t in _tiny_inputs()]
    for graphs in (False, True):
        net.set_graphs(graphs)
        ref = net.forward(*args).clone()
        torch.cuda.synchronize()
        for pattern in (0xFF, 0x00, 0xA5):
            for arena in (U.ARENA_UNET, U.ARENA_UNET_PERSIST):
                U.arena_fill(arena, pattern)
            out = net.forward(*args)
            torch.cuda.synchronize()
            assert torch.isfinite(out.float()).all()
            assert torch.equal(out, ref), f"graphs={graphs}: output changed after filling with {pattern:#x}"
    net.set_graphs(False)
    net.close()


_CHILD = r'''
import sys, torch
sys.path.insert(0, sys.argv[1])
from dollama_amd import unet as U
from tests.test_arena import _tiny_net, _tiny_inputs
net = _tiny_net()
args = [t.cuda() for t in _tiny_inputs()]
out = net.forward(*args); net.forward(*args)
torch.cuda.synchronize()
st = U.arena_stats(U.ARENA_UNET)
assert st["cuda_malloc_calls"] > 0 and st["cuda_malloc_calls"] == st["cuda_free_calls"], st
assert st["chunk_alloc_calls"] == 0 and st["total_capacity"] == 0, st
torch.save(out.cpu(), sys.argv[2])
net.close()
print("child ok", st["cuda_malloc_calls"])
'''


def test_unet_forward_pool_off_process_matches(gpu, tmp_path):
    """DOLLAMA_POOL=0 is read once per process, so the pool-off forward runs in a
    child started with the variable set (before it touches the GPU)."""
    print("[case] tiny UNet forward, DOLLAMA_POOL=0 child vs pooled", flush=True)
    path = str(tmp_path / "pool_off.pt")
    env = dict(os.environ, DOLLAMA_POOL="0")
    r = subprocess.run([sys.executable, "-c", _CHILD, ROOT, path], capture_output=True, text=True,
                       timeout=300, env=env, cwd=ROOT)
    print(r.stdout, r.stderr[-2000:])
    assert r.returncode == 0, r.stderr[-2000:]
    net = _tiny_net()
    out = net.forward(*[t.cuda() for t in _tiny_inputs()]).cpu()
    net.close()
    assert torch.equal(out, torch.load(path, weights_only=True))
