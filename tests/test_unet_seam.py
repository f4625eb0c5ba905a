"""The reference-signature UNet seam (dollama_amd/csrc/host/unet_api.hpp):
unet_weights_create(const SafeTensors&), launch_unet, launch_unet_batched,
unet_apply_loras / unet_clear_loras and the global stage hook with the
reference's signatures (src/infer/unet.cuh:53-146), over the C ABI.

The seam runs as a C++ program (tests/cpp/test_unet_seam.cpp) against
libdollama.so.  On a small SDXL-topology UNet (channels 64/128/192, depths
1/2, SDXL's 6 x 256 time-id sinusoids) written to a safetensors file, it
checks: the configuration read from the tensor shapes; launch_unet_batched
(B=2) and launch_unet (B=1) equal dlm_unet_forward on the same file bit for
bit; with graphs on, replays with a different host timestep per call equal
the eager native forwards at those timesteps; a LoRA module applied through
the seam equals the native LoRA path and clears bit-exactly; the stage hook
receives the block-boundary stages with noise_pred equal to the output;
errors throw.  The build of the program also runs on the CPU.
"""
import os
import subprocess

import numpy as np
import pytest

from dollama_amd import unet as U

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CFG = U.UNetConfig(C0=64, C1=128, C2=192, depth1=1, depth2=2, cross_dim=96, text_dim=64, id_dim=256)


def _build(tmp_path):
    exe = tmp_path / "test_unet_seam"
    lib = os.path.join(ROOT, "dollama_amd")
    cmd = ["g++", "-std=c++20", "-O1", "-Wall", "-pthread",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "dollama_amd", "csrc", "host"),
           os.path.join(ROOT, "tests", "cpp", "test_unet_seam.cpp"),
           "-L", lib, "-ldollama", "-ldlm_hip", f"-Wl,-rpath,{lib}", "-o", str(exe)]
    subprocess.run(cmd, check=True)
    return exe


def _write_weights(path, seed=5):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(seed)
    tensors = {}
    for name, shape in U.weight_specs(CFG).items():
        x = rng.standard_normal(shape).astype(np.float32) * 0.02
        if len(shape) == 1 and name.endswith(".weight") and "norm" in name.split(".")[-2]:
            x = x + 1.0
        tensors[name] = x.astype(np.float16)
    save_file(tensors, str(path))


def test_seam_program_builds(tmp_path):
    _build(tmp_path)


@pytest.mark.gpu
def test_reference_signature_seam_matches_native_forward(gpu, tmp_path):
    print("[case] UNet seam: tiny SDXL-topology UNet, latent 32x32, ctx 77", flush=True)
    exe = _build(tmp_path)
    st = tmp_path / "unet.safetensors"
    _write_weights(st)
    r = subprocess.run([str(exe), str(st), "32", "77"], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "seam: 0 failure(s)" in r.stdout
    assert "config C=64/128/192 depth=1/2 cross=96 text=64 id=256 in=4 out=4" in r.stdout
