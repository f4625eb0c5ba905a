"""CPU oracle for the SDXL UNet dense-contraction path — TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package, and only as the checker (or as the CPU baseline
that is timed beside the GPU).  The product path (``dollama_amd``) never
imports it and has no CPU fallback.

Contents
  ref_ops.py   fp32 torch-CPU restatement of each kernel's arithmetic
  naive.c      plain C loops restating the reference's own CPU test
               references (independent of torch); built to libnaive.so
  naive.py     ctypes binding of libnaive.so
  unet_ref.py  fp32 torch-CPU restatement of the SDXL UNet graph
  metrics.py   tolerance metrics: relative error, cosine, the reference SSIM
  sched_ref.cpp  driver of the reference's own header-only Euler scheduler
               (src/infer/scheduler.hpp), compiled by the Makefile from the
               reference tree into _ref/sched_ref when that tree is present

How each function is pinned (besides these two independent restatements
agreeing with each other) is listed in tests/test_oracle.py.
"""
