#!/usr/bin/env python3
"""Benchmark: SDXL UNet denoise step at 1024x1024 (latent 128x128), CFG batch
B=2, fp16 with fp32 accumulation, random-init weights of the SDXL
architecture (N(0, 0.02^2)), synthetic inputs, on one MI355X.

Prints one JSON line.  ``value`` is the mean device time of one full UNet step
(ms, lower is better) over ``--steps`` timed forwards (HIP-graph replays)
with all inputs resident in HBM.  Extra fields:
- per kernel class and per kernel instantiation, time and algorithmic
  TFLOP/s from separately profiled forwards in which every launch carries a
  device event pair in its own dispatch (hipExtLaunchKernel, on the stream
  the kernel runs on), so the intervals are the kernels' execution without
  marker packets between them;
- ``roofline``: the single kernel instantiation with the most time, its
  algorithmic FLOPs per launch over its average launch duration against the
  fp16 MFMA peak, and its HBM bytes per launch from rocprofv3 PMC counters
  (profiles/hbm_traffic.json);
- ``configs``: the other benchmark configurations timed on their own (single
  3x3 conv, three ResnetBlock2D shapes, the two self-attention shapes, one
  BasicTransformerBlock);
- a 20-step CFG Euler loop on the device;
- ``cpu_baseline``: the fp32 CPU oracle running full steps of the same
  workload (same weights and inputs) on this host, median of 3, with its
  noise_pred compared against the GPU's; each ``configs`` entry carries the
  oracle's time for that configuration (``cpu_ms``, median of 5).
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
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config timings")
    ap.add_argument("--eager", action="store_true",
                    help="time eager forwards only (default: HIP-graph replay, eager timed beside it)")
    ap.add_argument("--workload", choices=("unet", "vae"), default="unet",
                    help="unet: the UNet step (default); vae: the VAE decode of one 1024x1024 image")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain device copy of 256 MiB (5 times), to scale the "
                         "FETCH_SIZE / WRITE_SIZE counters of a PMC run")
    ap.add_argument("--calibrate-mfma", action="store_true",
                    help="only run the MFMA calibration kernel (register-only fp16 MFMA "
                         "stream of known FLOPs, 5 launches) and print its measured rate, to "
                         "read the MFMA counters of a PMC run against")
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


def calibrate_mfma():
    """The library's MFMA calibration kernel (dlm_mfma_probe): 1024
    workgroups of 4 waves (4 waves per SIMD), each wave 4000 rounds of eight
    32x32x16 fp16 MFMAs on registers.  Prints FLOPs per launch and the rate of
    each of 5 launches timed with device events on the launch stream."""
    import ctypes
    import torch
    from dollama_amd import _lib
    blocks, iters = 1024, 4000
    flop = blocks * 4 * iters * 8 * 32768
    out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda:0")
    st = torch.cuda.current_stream()
    rates = []
    for _ in range(6):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        _lib.call("dlm_mfma_probe", blocks, iters, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(st.cuda_stream))
        e1.record(st)
        torch.cuda.synchronize()
        rates.append(flop / (e0.elapsed_time(e1) * 1e-3))
    rates = rates[1:]  # the first launch warms the clocks
    print(json.dumps({"calibrate_mfma_flop_per_dispatch": flop,
                      "tflops": [round(r / 1e12, 1) for r in rates],
                      "frac_of_peak": [round(r / MFMA_FP16_PEAK, 4) for r in rates],
                      "finite": bool(torch.isfinite(out).all())}), flush=True)


def measured_traffic():
    """HBM bytes per launch by kernel instantiation, from rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE runs on this bench scaled by the same counters on a
    plain copy (profiles/hbm_traffic.json)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f).get("kernels", {})


def _progress(msg):
    """One progress line on stderr per phase (the JSON line stays alone on
    stdout)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads():
    import torch
    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    return threads


def _median_s(fn, runs, warmup=1):
    """Median wall time (s) of fn() over `runs` calls after `warmup` calls."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2], ts


def cpu_baseline(w_cpu, inputs, gpu_out, runs=3):
    """Full UNet steps of the same workload (same weights, same fp16 inputs)
    through the fp32 torch-CPU oracle on this host's CPU share: one warm-up
    forward on a 32x32 latent, then `runs` full steps, median reported.  The
    oracle's noise_pred is compared with the GPU's (SSIM of the reference's
    definition, relative error, cosine)."""
    import torch
    from oracle import metrics
    from oracle import unet_ref as OR
    threads = _cpu_threads()
    lat, ts, ehs, text, ids = inputs
    OR.unet_forward(w_cpu, OR.SDXL, lat[:, :, :32, :32].contiguous(), ts, ehs, text, ids)
    box = {}

    def step():
        t0 = time.perf_counter()
        box["ref"] = OR.unet_forward(w_cpu, OR.SDXL, lat, ts, ehs, text, ids)
        _progress(f"CPU oracle step {time.perf_counter() - t0:.1f} s")

    med, all_s = _median_s(step, runs, warmup=0)
    ref = box["ref"]
    got = gpu_out.float().cpu()
    return {
        "value": round(med * 1e3, 1),
        "unit": "ms/step",
        "cores": threads,
        "kind": "port",
        "runs": runs,
        "runs_ms": [round(t * 1e3, 1) for t in all_s],
        "sample": f"median of {runs} full SDXL UNet steps (B=2, latent 128x128, ctx 77x2048) through the "
                  "fp32 torch-CPU oracle with the GPU run's weights and inputs, after a 32x32 warm-up",
        "cpu_model": cpu_model(),
        "host_logical_cpus": os.cpu_count(),
        "gpu_vs_cpu": {"ssim": round(metrics.ssim_uniform(got, ref), 7),
                       "rel_err": float(f"{metrics.rel_err(got, ref):.3e}"),
                       "cosine": round(metrics.cosine(got, ref), 7)},
    }


def cpu_config_timings(w_cpu, seed, runs=5):
    """The benchmark's configurations 1-4 on the fp32 torch-CPU oracle (one
    warm-up, median of `runs`), same shapes as config_timings: ms per call,
    keyed like its entries."""
    import torch
    from oracle import ref_ops as R
    from oracle import unet_ref as OR
    _cpu_threads()
    g = torch.Generator().manual_seed(seed)

    def rn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g) * std).half().float()

    out = {}
    x = rn(1, 320, 128, 128)
    w, b = rn(320, 320, 3, 3, std=0.02), rn(320, std=0.01)
    out["conv3x3_320_128px_n1_bias_silu"] = _median_s(lambda: R.silu(R.conv2d(x, w, b, 1, 1)), runs)[0]
    temb = R.silu(rn(2, 1280))
    for name, prefix, ci, hw in (("resnet_640ch_64px", "down_blocks.1.resnets.1.", 640, 64),
                                 ("resnet_1280ch_32px", "mid_block.resnets.0.", 1280, 32),
                                 ("resnet_320to640_64px_1x1skip", "down_blocks.1.resnets.0.", 320, 64)):
        xr = rn(2, ci, hw, hw)
        out[name] = _median_s(lambda: OR.resnet_block(w_cpu, prefix, xr, temb), runs)[0]
    for name, B, H, S in (("attention_b2_h10_s4096", 2, 10, 4096), ("attention_b2_h20_s1024", 2, 20, 1024)):
        q, k, v = rn(B, H, S, 64), rn(B, H, S, 64), rn(B, H, S, 64)
        out[name] = _median_s(lambda: R.attention(q, k, v, 0.125), runs)[0]
    xt, ctx = rn(2, 4096, 640), rn(2, 77, 2048)
    out["basic_transformer_block_2x4096x640"] = _median_s(
        lambda: OR.transformer_block(w_cpu, "down_blocks.1.attentions.0.transformer_blocks.0.", xt, ctx, 10),
        runs)[0]
    # the reference-layout entries compute the same functions on the same shapes
    out["reference_layout_conv2d_nchw_320_128px_n1_bias"] = out["conv3x3_320_128px_n1_bias_silu"]
    out["reference_layout_attention_b2_h10_s4096"] = out["attention_b2_h10_s4096"]
    return {k: round(v * 1e3, 2) for k, v in out.items()}


def queue_ahead(seconds=0.01):
    """Hold the current stream with a spin kernel of about `seconds` so that the
    work enqueued next runs back to back on the device: event pairs then time
    the kernels, not the host's launch gaps (the host must finish enqueueing
    before the spin ends)."""
    import torch
    torch.cuda._sleep(int(2.5e9 * seconds))


def time_calls(fn, reps=20, warmup=3):
    """Mean device time (ms) of fn() over reps back-to-back calls between one
    event pair on the current stream, queued behind a spin kernel."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    queue_ahead(max(0.01, reps * 2e-4))  # 200 us of host time per call at most
    e0.record(st)
    for _ in range(reps):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def time_graph(fn, reps=20):
    """Device time (ms) per call of fn() when reps calls are captured into one
    HIP graph and the graph is replayed between an event pair: back-to-back
    kernels with the inter-node gap of a graph, as in the graph-replayed step."""
    import torch
    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    graph.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def replay_kernel(name, problems, dev, seed):
    """Average launch duration (us) and FLOPs of one GEMM kernel instantiation
    over the problems it ran in the step: each problem's launches are captured
    into a HIP graph and replayed between one event pair (time_graph), and the
    per-problem times are weighted by the problem's launches per step.  The
    kernel each launch ran is checked against `name`.  None for convs and
    LayerNorm-folded linears."""
    import ctypes
    import torch
    from dollama_amd import _lib, ops
    lib = _lib.hip_lib()
    lib.dlm_last_kernel.restype = ctypes.c_char_p
    lib.dlm_last_kernel.argtypes = [ctypes.c_int]
    g = torch.Generator(device=dev).manual_seed(seed)

    def rn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * std).half()

    tot_us = tot_flop = 0.0
    tot_n = 0
    for (M, N, K, flags), cnt in problems.items():
        if flags & (256 | 512):  # convs, LayerNorm-folded linears
            return None
        act, res = (flags >> 4) & 15, flags & 1
        ncols = N // 2 if act == ops.ACT_GEGLU else N
        x, w, b = rn(M, K), rn(N, K, std=0.02), rn(N, std=0.01)
        r = rn(M, ncols) if res else None
        y = torch.empty(M, ncols, dtype=torch.float16, device=dev)
        fn = lambda: ops.linear(x, w, bias=b, residual=r, act=act, out=y)
        fn()
        ran = lib.dlm_last_kernel(1).decode()
        if ran != name:
            raise RuntimeError(f"replay of {M}x{N}x{K} ran {ran}, not {name}")
        ms = time_graph(fn, reps=max(20, cnt))
        tot_us += ms * 1e3 * cnt
        tot_flop += 2.0 * M * N * K * cnt
        tot_n += cnt
    return tot_us / tot_n, tot_flop / tot_n


def config_timings(net, U, dev, seed):
    """The benchmark's other configurations, each timed on its own."""
    import torch
    from dollama_amd import ops
    g = torch.Generator(device=dev).manual_seed(seed)

    def rn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * std).half()

    def entry(ms, flop):
        return {"ms": round(ms, 4), "tflop": round(flop / 1e12, 4),
                "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
                "frac_mfma": round(flop / (ms * 1e-3) / MFMA_FP16_PEAK, 4)}

    out = {}
    # 1: conv 3x3 320->320 @128x128, N=1, bias + SiLU epilogue
    x = rn(1, 128, 128, 320)
    wp = ops.pack_conv_weight(rn(320, 320, 3, 3, std=0.02))
    b = rn(320, std=0.01)
    y = torch.empty(1, 128, 128, 320, dtype=torch.float16, device=dev)
    ms = time_calls(lambda: ops.conv2d_nhwc(x, wp, KH=3, KW=3, bias=b, act=ops.ACT_SILU, out=y))
    out["conv3x3_320_128px_n1_bias_silu"] = entry(ms, 2.0 * 16384 * 320 * 2880)
    # 2: ResnetBlock2D at B=2 (FLOPs of the convs, as the configuration counts them)
    temb = rn(2, 1280)
    for name, prefix, ci, co, hw in (("resnet_640ch_64px", "down_blocks.1.resnets.1.", 640, 640, 64),
                                     ("resnet_1280ch_32px", "mid_block.resnets.0.", 1280, 1280, 32),
                                     ("resnet_320to640_64px_1x1skip", "down_blocks.1.resnets.0.", 320, 640, 64)):
        xr = rn(2, hw, hw, ci)
        yr = torch.empty(2, hw, hw, co, dtype=torch.float16, device=dev)
        ms = time_calls(lambda: net.run_resnet(prefix, xr, temb, out=yr))
        flop = 2.0 * 2 * hw * hw * co * (9 * ci + 9 * co + (ci if ci != co else 0))
        out[name] = entry(ms, flop)
    # 3: flash self-attention, fp16 with fp32 softmax (V^T form of the UNet)
    for name, B, H, S in (("attention_b2_h10_s4096", 2, 10, 4096), ("attention_b2_h20_s1024", 2, 20, 1024)):
        C = H * 64
        qk = rn(B, S, 2 * C)
        vt = rn(B, H, 64, S)
        o = torch.empty(B, S, C, dtype=torch.float16, device=dev)
        ms = time_calls(lambda: ops.attention_vt(qk, qk[:, :, C:], vt, o, B=B, H=H, Sq=S, Sk=S,
                                                 q_strides=(S * 2 * C, 2 * C, 64), k_strides=(S * 2 * C, 2 * C, 64),
                                                 vt_strides=(H * 64 * S, 64 * S), vt_ld=S,
                                                 o_strides=(S * C, C, 64), scale=0.125))
        out[name] = entry(ms, 4.0 * B * H * S * S * 64)
    # the reference-layout entry points a reference caller binds (NCHW conv with
    # bias, [B, H, S, Dh] attention): layout conversions included
    xn = rn(1, 320, 128, 128)
    wn = rn(320, 320, 3, 3, std=0.02)
    yn = torch.empty(1, 320, 128, 128, dtype=torch.float16, device=dev)
    ms = time_calls(lambda: ops.launch_conv2d(xn, wn, b, yn, 1, 320, 128, 128, 320, 3, 3, 1, 1, 1, 1))
    out["reference_layout_conv2d_nchw_320_128px_n1_bias"] = entry(ms, 2.0 * 16384 * 320 * 2880)
    B, H, S = 2, 10, 4096
    qa, ka, va = rn(B, H, S, 64), rn(B, H, S, 64), rn(B, H, S, 64)
    oa = torch.empty(B, H, S, 64, dtype=torch.float16, device=dev)
    ms = time_calls(lambda: ops.launch_attention(qa, ka, va, oa, B, H, S, S, 64, 0.125))
    out["reference_layout_attention_b2_h10_s4096"] = entry(ms, 4.0 * B * H * S * S * 64)
    # 4: BasicTransformerBlock on 2x4096x640, context 2x77x2048 (incl. its K/V projections)
    xt = rn(2, 4096, 640)  # the block updates it in place on every call
    ctx = rn(2, 77, 2048)
    ms = time_calls(lambda: net.run_transformer_block("down_blocks.1.attentions.0.transformer_blocks.0.", xt, ctx))
    M, C = 8192, 640
    flop = 2.0 * M * C * C * 18 + 2 * 2.0 * 154 * 2048 * C + 4.0 * 2 * 10 * 4096 * 4096 * 64 + 4.0 * 2 * 10 * 4096 * 77 * 64
    out["basic_transformer_block_2x4096x640"] = entry(ms, flop)
    return out


def main():
    args = parse()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.calibrate_mfma:
        calibrate_mfma()
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
    # the CPU leg runs the same model: an fp32 host copy of the fp16 weights
    w_cpu = None if args.no_cpu_baseline else {k: v.float().cpu() for k, v in weights.items()}
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

    _progress("setup done, timing eager forwards")
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

    _progress(f"step {ms:.3f} ms (eager {eager_ms:.3f} ms); profiling forwards")
    # per-class and per-kernel time from device events attached to every launch's own dispatch
    net.set_profiling(True)
    reports, kreports = [], []
    for _ in range(max(1, args.profile_runs)):
        queue_ahead(0.03)
        net.forward(latent, ts, ehs, text, ids, out=out)
        reports.append(net.profile_report())
        kreports.append(net.profile_kernels())
    net.set_profiling(False)
    kernels = {}
    for name, k0 in kreports[-1].items():
        ms_k = sorted(r[name]["ms"] for r in kreports)[len(kreports) // 2]
        kernels[name] = {"class": k0["class"], "launches": k0["launches"], "ms": round(ms_k, 4),
                         "flops": k0["flops"], "bytes": k0["bytes"],
                         "tflops": round(k0["flops"] / (ms_k * 1e-3) / 1e12, 1) if k0["flops"] and ms_k else None}
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
    # the dominant kernel: the one instantiation with the most time among the
    # MFMA-bound classes
    dom = max((n for n, k in kernels.items() if k["class"] in ("conv", "linear", "attention")),
              key=lambda n: kernels[n]["ms"])
    dk = kernels[dom]
    # its average launch duration inside the step: the dispatch-attached event
    # pairs of its launches in the profiled forwards
    dom_avg_us, dom_flop = dk["ms"] / dk["launches"] * 1e3, dk["flops"] / dk["launches"]
    dom_timing = ("this kernel's launches in the profiled forwards, each carrying a device event pair in "
                  "its own dispatch (hipExtLaunchKernel) on the stream it runs on")
    # cross-check: the step's problems of this kernel replayed in isolation
    rp = replay_kernel(dom, kreports[-1][dom]["problems"], dev, args.seed + 3)
    achieved = dom_flop / (dom_avg_us * 1e-6) / 1e12
    traffic = measured_traffic().get(dom, {})

    _progress("profiled; Euler loop")
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

    _progress("per-config timings")
    configs = None if args.no_configs else config_timings(net, U, dev, args.seed + 2)

    cpu = None
    if w_cpu is not None:
        if configs is not None:
            _progress("CPU oracle legs of configurations 1-4 (median of 5 each)")
            cpu_ms = cpu_config_timings(w_cpu, args.seed + 4)
            for name, c in configs.items():
                c["cpu_ms"] = cpu_ms.get(name)
                c["gpu_vs_cpu"] = round(cpu_ms[name] / c["ms"], 1) if name in cpu_ms else None
        inputs = (latent.float().cpu(), ts.cpu(), ehs.float().cpu(), text.float().cpu(), ids.float().cpu())
        _progress("CPU oracle full steps (median of 3)")
        cpu = cpu_baseline(w_cpu, inputs, eager_out)
        cpu["configs_runs"] = 5 if configs is not None else None
        del w_cpu

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
            "kernel": dom,
            "class": dk["class"],
            "achieved": round(achieved, 1),
            "peak": MFMA_FP16_PEAK / 1e12,
            "unit": "TFLOP/s",
            "frac": round(achieved * 1e12 / MFMA_FP16_PEAK, 4),
            "traffic": traffic.get("hbm_bytes_per_launch"),
            "algorithmic_bytes_per_launch": round(dk["bytes"] / dk["launches"]),
            "launches_per_step": dk["launches"],
            "avg_launch_us": round(dom_avg_us, 2),
            "flop_per_launch": dom_flop,
            "timing": dom_timing,
            "replay_avg_launch_us": round(rp[0], 2) if rp is not None else None,
        },
        "kernels": {n: {kk: v for kk, v in k.items() if kk not in ("bytes", "problems")}
                    for n, k in sorted(kernels.items(), key=lambda kv: -kv[1]["ms"])[:12]},
        "configs": configs,
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
