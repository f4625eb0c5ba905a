#!/usr/bin/env python3
"""Benchmark: SDXL UNet denoise step at 1024x1024 (latent 128x128), CFG batch
B=2, fp16 with fp32 accumulation, random-init weights of the SDXL
architecture (N(0, 0.02^2)), synthetic inputs, on one MI355X.

Prints one JSON line.  ``value`` is the mean wall time of one full UNet step
(ms, lower is better) over ``--steps`` timed forwards with all inputs
resident in HBM.  Extra fields report, from device events around every
launch of a separately profiled forward, each kernel class's time and
algorithmic TFLOP/s, the conv+attention fraction of the fp16 MFMA peak, the
roofline of the dominant kernel class, a 20-step CFG Euler denoise loop
timed on the device, and the fp32 CPU oracle timed on this host's cores
over a bounded sample (the mid block), scaled to one step by FLOPs.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_FP16_PEAK = 2.5166e15  # dense fp16 MFMA, MI355X spec
HBM_PEAK = 8.0e12


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--loop-steps", type=int, default=20, help="Euler loop length (0 = skip)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-runs", type=int, default=3)
    ap.add_argument("--eager", action="store_true",
                    help="time eager forwards only (default: HIP-graph replay, eager timed beside it)")
    ap.add_argument("--workload", choices=("unet", "vae"), default="unet",
                    help="unet: the UNet step (default); vae: the VAE decode of one 1024x1024 image")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain device copy of 256 MiB (5 times), to scale the "
                         "FETCH_SIZE / WRITE_SIZE counters of a PMC run")
    return ap.parse_args()


def calibrate_copy():
    """A plain device-to-device copy of known size for counter calibration:
    each of the 5 dispatches reads and writes exactly 256 MiB."""
    import torch
    n = 128 << 20  # fp16 elements = 256 MiB
    a = torch.ones(n, dtype=torch.float16, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes_per_dispatch": 2 * n}), flush=True)


def measured_traffic():
    """HBM bytes per launch of the dominant kernel class, as measured by
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on this bench and scaled by the
    same counters on a plain copy (profiles/hbm_traffic.json)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def cpu_baseline(seed):
    """fp32 torch-CPU oracle over the mid block (resnet, Transformer2D depth 10,
    resnet at 32x32x1280, B=2), scaled to a full step by algorithmic FLOPs."""
    import torch
    from oracle import unet_ref as OR
    cores = min(16, os.cpu_count() or 1)
    torch.set_num_threads(cores)
    cfg = OR.SDXL
    shapes = {k: v for k, v in OR.param_shapes(cfg).items() if k.startswith("mid_block.")}
    g = torch.Generator().manual_seed(seed)
    W = {}
    for k, shp in shapes.items():
        t = torch.randn(shp, generator=g) * 0.02
        if "norm" in k.split(".")[-2] and k.endswith(".weight") and len(shp) == 1:
            t += 1.0
        W[k] = t
    B, C, Hh = 2, cfg.C2, 32
    x = torch.randn(B, C, Hh, Hh, generator=g)
    ctx = torch.randn(B, 77, cfg.cross_dim, generator=g)
    temb = torch.randn(B, cfg.T, generator=g)
    ts = OR.R.silu(temb)

    def run():
        with torch.no_grad():
            y = OR.resnet_block(W, "mid_block.resnets.0.", x, ts)
            y = OR.transformer2d(W, "mid_block.attentions.0.", y, ctx, cfg.depth2)
            return OR.resnet_block(W, "mid_block.resnets.1.", y, ts)

    run()  # warm
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    sec = sorted(times)[1]
    from dollama_amd.flops import unet_step_flops, mid_block_flops
    full = unet_step_flops(B=2, H=128, W=128)["total"]
    mid = mid_block_flops(B=2)
    return {
        "value": sec * (full / mid) * 1e3,
        "unit": "ms/step (scaled)",
        "cores": cores,
        "kind": "port",
        "sample": f"oracle mid_block (resnet + Transformer2D depth 10 + resnet, B=2, 32x32x1280, "
                  f"{mid / 1e12:.3f} TFLOP) median of 3 = {sec * 1e3:.0f} ms, scaled by "
                  f"{full / 1e12:.3f}/{mid / 1e12:.3f} TFLOP",
    }


def main():
    args = parse()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the UNet step "
              "is not sharded across GPUs in this build.", file=sys.stderr)
        sys.exit(2)
    if args.workload == "vae":
        vae_main(args)
        return
    import torch
    from dollama_amd import unet as U
    from dollama_amd.flops import unet_step_flops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = U.SDXL_CONFIG
    B, H, W, L = 2, 128, 128, 77
    t_setup = time.time()
    net = U.UNet(cfg)
    weights = U.random_weights(cfg, args.seed, device=dev)
    net.set_weights(weights)
    net.prepare()
    del weights
    torch.cuda.empty_cache()
    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    latent = torch.randn(B, 4, H, W, generator=g, device=dev).half()
    ehs = torch.randn(B, L, cfg.cross_dim, generator=g, device=dev).half()
    text = torch.randn(B, cfg.text_dim, generator=g, device=dev).half()
    ts = torch.full((B,), 999.0, device=dev)
    ids = torch.tensor([1024, 1024, 0, 0, 1024, 1024], dtype=torch.float16, device=dev)
    out = torch.empty(B, 4, H, W, dtype=torch.float16, device=dev)
    setup_s = time.time() - t_setup

    # all work on one created stream (HIP graphs cannot capture the null stream)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)

    def timed(graphs):
        net.set_graphs(graphs)
        for _ in range(max(args.warmup, 3 if graphs else 0)):  # graphs: eager, capture, replay
            net.forward(latent, ts, ehs, text, ids, out=out)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            net.forward(latent, ts, ehs, text, ids, out=out)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps, (time.perf_counter() - w0) / args.steps * 1e3

    eager_ms, eager_wall = timed(False)
    eager_out = out.clone()
    if args.eager:
        ms, wall = eager_ms, eager_wall
    else:
        ms, wall = timed(True)
        if not torch.equal(out, eager_out):
            raise RuntimeError("graph replay differs from the eager forward")
        net.set_graphs(False)
    if not torch.isfinite(out.float()).all():
        raise RuntimeError("non-finite noise_pred")

    # per-class kernel time from device events around every launch
    net.set_profiling(True)
    reports = []
    for _ in range(max(1, args.profile_runs)):
        net.forward(latent, ts, ehs, text, ids, out=out)
        reports.append(net.profile_report())
    net.set_profiling(False)
    classes = {}
    for c in U.UNet.KERNEL_CLASSES:
        ms_c = sorted(r[c]["ms"] for r in reports)[len(reports) // 2]
        r0 = reports[-1][c]
        classes[c] = {"launches": r0["launches"], "ms": round(ms_c, 4),
                      "tflops": round(r0["flops"] / (ms_c * 1e-3) / 1e12, 1) if r0["flops"] and ms_c else None,
                      "gbps": round(r0["bytes"] / (ms_c * 1e-3) / 1e9, 1) if r0["bytes"] and ms_c else None}
    fl = unet_step_flops(B=B, H=H, W=W)
    conv_attn_flops = fl["conv"] + fl["attention"]
    conv_attn_ms = classes["conv"]["ms"] + classes["attention"]["ms"]
    kernel_ms = sum(v["ms"] for v in classes.values())
    dom = max(("conv", "linear", "attention"), key=lambda c: classes[c]["ms"])
    dom_flops = reports[-1][dom]["flops"]
    dom_ms = classes[dom]["ms"]
    dom_launches = classes[dom]["launches"]
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12

    # 20-step CFG Euler denoise loop on the device
    loop = None
    if args.loop_steps > 0:
        sig, _ = U.euler_schedule(args.loop_steps)
        lat32 = torch.randn(4, H, W, generator=g, device=dev) * sig[0]
        net.set_graphs(not args.eager)
        lt = lat32.clone()
        U.denoise(net, lt, ehs, text, ids, steps=args.loop_steps, guidance=7.5)  # warm
        lt = lat32.clone()
        torch.cuda.synchronize()
        l0 = time.perf_counter()
        U.denoise(net, lt, ehs, text, ids, steps=args.loop_steps, guidance=7.5)
        torch.cuda.synchronize()
        loop = {"steps": args.loop_steps, "guidance": 7.5, "s": round(time.perf_counter() - l0, 4),
                "finite": bool(torch.isfinite(lt).all()), "graphs": not args.eager}
        net.set_graphs(False)

    cpu = None if args.no_cpu_baseline else cpu_baseline(args.seed)

    line = {
        "metric": "SDXL UNet step ms @1024^2 CFG B=2; conv/attn TFLOPS & % fp16 MFMA peak",
        "value": round(ms, 3),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (fp32 accumulate)",
        "data": "synthetic: random-init SDXL UNet weights N(0,0.02^2), latent/ehs/text N(0,1), t=999",
        "config": {"workload": "sdxl_unet_step_1024px_cfg_b2", "batch": B, "latent": [4, H, W],
                   "ctx": [L, cfg.cross_dim], "params": 2567463684},
        "wall_ms_per_step": round(wall, 3),
        "timing": "eager forwards" if args.eager else "HIP-graph replay of the forward (one hipGraphLaunch per step)",
        "eager_ms_per_step": round(eager_ms, 3),
        "step_tflop": round(fl["total"] / 1e12, 4),
        "whole_step_tflops": round(fl["total"] / (ms * 1e-3) / 1e12, 1),
        "whole_step_frac_mfma": round(fl["total"] / (ms * 1e-3) / MFMA_FP16_PEAK, 4),
        "conv_attn_tflop": round(conv_attn_flops / 1e12, 4),
        "conv_attn_kernel_ms": round(conv_attn_ms, 3),
        "conv_attn_tflops": round(conv_attn_flops / (conv_attn_ms * 1e-3) / 1e12, 1),
        "conv_attn_frac_mfma": round(conv_attn_flops / (conv_attn_ms * 1e-3) / MFMA_FP16_PEAK, 4),
        "kernel_ms_sum": round(kernel_ms, 3),
        "classes": classes,
        "roofline": {
            "bound": "mfma",
            "kernel": {"conv": "dma_gemm_kernel<ConvDesc> (implicit-GEMM conv, LDS-DMA)",
                       "linear": "dma_gemm_kernel<RowDesc> (linears, LDS-DMA)",
                       "attention": "flash_vt_pipe_kernel (self and cross attention)"}[dom],
            "achieved": round(achieved, 1),
            "peak": MFMA_FP16_PEAK / 1e12,
            "unit": "TFLOP/s",
            "frac": round(achieved * 1e12 / MFMA_FP16_PEAK, 4),
            "traffic": measured_traffic().get(dom, {}).get("hbm_bytes_per_launch"),
            "launches_per_step": dom_launches,
            "avg_launch_us": round(dom_ms / max(1, dom_launches) * 1e3, 2),
            "flop_per_step": dom_flops,
        },
        "euler_loop": loop,
        "cpu_baseline": cpu,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line), flush=True)


def vae_main(args):
    """SDXL VAE decode of one 128x128 latent into a 1024x1024 image (the
    reference's only VAE shape), random-init weights ~N(0, 1/fan_in)."""
    import torch
    from dollama_amd import vae as V

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = V.SDXL_VAE_CONFIG
    net = V.VAE(cfg)
    w = V.random_weights(cfg, args.seed, device=dev)
    net.set_weights(w)
    net.prepare()
    del w
    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    lat = torch.randn(1, 4, 128, 128, generator=g, device=dev).half()
    img = torch.empty(1, 3, 1024, 1024, dtype=torch.float16, device=dev)
    for _ in range(args.warmup):
        net.decode(lat, out=img)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        net.decode(lat, out=img)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    if not torch.isfinite(img.float()).all():
        raise RuntimeError("non-finite image")
    net.set_profiling(True)
    reports = []
    for _ in range(max(1, args.profile_runs)):
        net.decode(lat, out=img)
        reports.append(net.profile_report())
    net.set_profiling(False)
    classes = {}
    flops = 0.0
    for c in V.VAE.KERNEL_CLASSES:
        ms_c = sorted(r[c]["ms"] for r in reports)[len(reports) // 2]
        r0 = reports[-1][c]
        flops += r0["flops"]
        classes[c] = {"launches": r0["launches"], "ms": round(ms_c, 4),
                      "tflops": round(r0["flops"] / (ms_c * 1e-3) / 1e12, 1) if r0["flops"] and ms_c else None,
                      "gbps": round(r0["bytes"] / (ms_c * 1e-3) / 1e9, 1) if r0["bytes"] and ms_c else None}
    line = {
        "metric": "SDXL VAE decode ms @1024^2 (latent 128x128)",
        "value": round(ms, 3), "unit": "ms/image", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16 operands, fp32 accumulate; fp32 up blocks 2-3",
        "data": "synthetic: random-init SDXL VAE decoder weights N(0,1/fan_in), latent N(0,1)",
        "config": {"workload": "sdxl_vae_decode_1024px", "batch": 1, "latent": [4, 128, 128],
                   "params": 49490199},
        "decode_tflop": round(flops / 1e12, 4),
        "decode_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "frac_mfma": round(flops / (ms * 1e-3) / MFMA_FP16_PEAK, 4),
        "classes": classes,
        "reference_rtx5080_ms": 1000.9,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
