"""Text-to-image runner and "sdxl" backend plugin (reference
src/server/diffusion_runner.hpp, diffusion_backend.hpp, sdxl_backend.hpp,
src/infer/diffusion.cu generate / generate_txt2img).

CPU: the product's seeded noise equals the oracle's restatement of the
reference generator bit for bit; missing files and unknown backends fail
the way the reference's factories do (no runner / no backend).
GPU (small UNet and VAE of the SDXL topology, written to safetensors files
with diffusers names): the RGB8 image of run_txt2img (CFG) and generate
(no guidance) against the fp32 oracle pipeline; the backend's generate ==
run_txt2img with the embeddings file's conditioning and zero uncond, info /
model_id, seed determinism, and LoRA apply / clear through the backend
(bit-exact restore).
"""
import math
import os

import numpy as np
import pytest
import torch

from dollama_amd import _lib
from dollama_amd import runner as RN
from dollama_amd import unet as U
from dollama_amd import vae as V
from oracle import naive
from oracle import noise_ref as NR
from oracle import pipeline_ref as PR
from oracle import unet_ref as OR
from oracle import vae_ref as OV

UCFG = U.UNetConfig(C0=64, C1=128, C2=192, depth1=1, depth2=2, cross_dim=96, text_dim=64, id_dim=16)
VCFG = V.VaeConfig(ch=(64, 128, 192, 192))
LAT = 16
CTX = 77


@pytest.mark.parametrize("seed", [0, 1, 42, 2 ** 63 + 5, 2 ** 64 - 1])
def test_product_noise_matches_oracle(seed):
    sig, _ = naive.euler_schedule(20)
    n = 4 * 32 * 32
    got = RN.randn_latent(seed, float(sig[0]), n)
    ref = NR.randn_latent(seed, float(sig[0]), n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_runner_and_backend_factories_refuse(tmp_path):
    with pytest.raises(_lib.DlmError):
        RN.DiffusionRunner(str(tmp_path / "no_unet.safetensors"), str(tmp_path / "no_vae.safetensors"),
                           str(tmp_path / "no_embeds.safetensors"))
    with pytest.raises(_lib.DlmError) as e:
        RN.Backend("sd-unknown", "", "", "")
    assert e.value.code == 5  # DLM_ERR_NOT_FOUND: make_backend's nullptr


def _files(tmp_path, seed=3, with_uncond=False):
    from safetensors.torch import save_file
    Wu = OR.random_weights(OR.TINY, seed=seed)
    Wv = OV.random_weights(OV.TINY_VAE, seed=seed + 1)
    g = torch.Generator().manual_seed(seed + 2)
    ehs = (torch.randn(CTX * UCFG.cross_dim, generator=g)).half()
    txt = (torch.randn(UCFG.text_dim, generator=g)).half()
    ids = torch.tensor([1024.0, 1024.0, 0.0, 0.0, 1024.0, 1024.0]).half()
    up = str(tmp_path / "unet.safetensors")
    vp = str(tmp_path / "vae.safetensors")
    ep = str(tmp_path / "embeds.safetensors")
    save_file({k: v.half().contiguous() for k, v in Wu.items()}, up)
    save_file({k: v.half().contiguous() for k, v in Wv.items()}, vp)
    emb = {"input_encoder_hidden_states_f16": ehs, "input_text_embeds_f16": txt, "input_time_ids_f16": ids}
    if with_uncond:
        emb["uncond_encoder_hidden_states_f16"] = (torch.randn(CTX * UCFG.cross_dim, generator=g) * 0.5).half()
        emb["uncond_text_embeds_f16"] = (torch.randn(UCFG.text_dim, generator=g) * 0.5).half()
    save_file(emb, ep)
    return up, vp, ep, Wu, Wv, {k: v.float() for k, v in emb.items()}


def _compare_rgb(got, ref, what):
    d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    mse = float((d.astype(np.float64) ** 2).mean())
    psnr = 10 * math.log10(255.0 ** 2 / max(mse, 1e-12))
    print(f"[parity] {what}: max|d|={d.max()} mean|d|={d.mean():.4f} PSNR={psnr:.2f} dB", flush=True)
    assert d.mean() <= 0.5 and psnr >= 40.0, what


@pytest.mark.gpu
def test_runner_txt2img_matches_oracle(gpu, tmp_path):
    up, vp, ep, Wu, Wv, emb = _files(tmp_path)
    r = RN.DiffusionRunner(up, vp, ep, unet_cfg=UCFG, vae_cfg=VCFG, latent_size=(LAT, LAT))
    g = torch.Generator().manual_seed(9)
    ce = torch.randn(CTX * UCFG.cross_dim, generator=g)
    ct = torch.randn(UCFG.text_dim, generator=g)
    ue = torch.randn(CTX * UCFG.cross_dim, generator=g) * 0.3
    ut = torch.randn(UCFG.text_dim, generator=g) * 0.3
    ids = torch.tensor([512.0, 512.0, 0.0, 0.0, 512.0, 512.0])
    got = r.run_txt2img(4, 1234, 5.0, ce.numpy(), ct.numpy(), ue.numpy(), ut.numpy(), ids.numpy())
    assert got.shape == (8 * LAT, 8 * LAT, 3)
    q = lambda t: t.half().float()  # the runner rounds the conditioning to fp16
    ref, _ = PR.txt2img(Wu, OR.TINY, Wv, OV.TINY_VAE, seed=1234, steps=4, lh=LAT, lw=LAT, cond_ehs=q(ce),
                        cond_text=q(ct), uncond_ehs=q(ue), uncond_text=q(ut), time_ids=q(ids), guidance=5.0)
    _compare_rgb(got, ref[0].numpy(), "run_txt2img 4 steps g=5 vs oracle")
    again = r.run_txt2img(4, 1234, 5.0, ce.numpy(), ct.numpy(), ue.numpy(), ut.numpy(), ids.numpy())
    assert np.array_equal(got, again), "same seed, different image"
    other = r.run_txt2img(4, 1235, 5.0, ce.numpy(), ct.numpy(), ue.numpy(), ut.numpy(), ids.numpy())
    assert not np.array_equal(got, other)
    r.close()


@pytest.mark.gpu
def test_runner_generate_without_guidance_matches_oracle(gpu, tmp_path):
    up, vp, ep, Wu, Wv, emb = _files(tmp_path, seed=5)
    r = RN.DiffusionRunner(up, vp, ep, unet_cfg=UCFG, vae_cfg=VCFG, latent_size=(LAT, LAT))
    got = r.generate(3, 77)
    ref, _ = PR.txt2img(Wu, OR.TINY, Wv, OV.TINY_VAE, seed=77, steps=3, lh=LAT, lw=LAT,
                        cond_ehs=emb["input_encoder_hidden_states_f16"], cond_text=emb["input_text_embeds_f16"],
                        time_ids=emb["input_time_ids_f16"], cfg=False)
    _compare_rgb(got, ref[0].numpy(), "generate (no guidance) 3 steps vs oracle")
    r.close()


@pytest.mark.gpu
@pytest.mark.parametrize("with_uncond", [False, True])
def test_backend_sdxl_generate_info_and_loras(gpu, tmp_path, monkeypatch, with_uncond):
    up, vp, ep, Wu, Wv, emb = _files(tmp_path, seed=7, with_uncond=with_uncond)
    be = RN.Backend("sdxl", up, vp, ep, preset="tiny", unet_cfg=UCFG, vae_cfg=VCFG, latent_size=LAT)
    assert be.info() == {"name": "sdxl", "latent_channels": 4, "native_resolution": 8 * LAT,
                         "needs_t5": False}
    assert be.model_id() == "sdxl-1.0/tiny"
    img = be.generate("a prompt the backend does not read", "", steps=3, seed=11, cfg=6.0)
    # == the runner with the file's cond and (file or zero) uncond
    r = RN.DiffusionRunner(up, vp, ep, unet_cfg=UCFG, vae_cfg=VCFG, latent_size=(LAT, LAT))
    ue = emb.get("uncond_encoder_hidden_states_f16", torch.zeros(CTX * UCFG.cross_dim))
    ut = emb.get("uncond_text_embeds_f16", torch.zeros(UCFG.text_dim))
    ref = r.run_txt2img(3, 11, 6.0, emb["input_encoder_hidden_states_f16"].numpy(),
                        emb["input_text_embeds_f16"].numpy(), ue.numpy(), ut.numpy(),
                        emb["input_time_ids_f16"].numpy())
    assert np.array_equal(img, ref)
    r.close()
    # LoRA by name from DOLLAMA_LORA_DIR; clear restores the image bit for bit
    from safetensors.torch import save_file
    lora_dir = tmp_path / "loras"
    lora_dir.mkdir()
    key = "down_blocks.1.attentions.0.transformer_blocks.0.attn1.to_q"
    C = UCFG.C1
    g = torch.Generator().manual_seed(13)
    flat = "lora_unet_" + key.replace(".", "_")
    save_file({flat + ".lora_down.weight": (torch.randn(4, C, generator=g) * 0.5).half(),
               flat + ".lora_up.weight": (torch.randn(C, 4, generator=g) * 0.5).half(),
               flat + ".alpha": torch.tensor(4.0).half()}, str(lora_dir / "style_a.safetensors"))
    monkeypatch.setenv("DOLLAMA_LORA_DIR", str(lora_dir))
    be.apply_loras([("style_a", 1.0)])
    with_lora = be.generate(steps=3, seed=11, cfg=6.0)
    assert not np.array_equal(with_lora, img)
    be.clear_loras()
    assert np.array_equal(be.generate(steps=3, seed=11, cfg=6.0), img)
    with pytest.raises(_lib.DlmError):
        be.apply_loras([("missing_lora", 1.0)])
    with pytest.raises(_lib.DlmError):
        be.apply_loras([("../escape", 1.0)])
    be.close()
