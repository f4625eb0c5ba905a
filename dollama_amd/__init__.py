"""dollama_amd — MI355X (gfx950) SDXL UNet dense-contraction hot path.

Hand-written HIP kernels behind the C ABI of include/dlm.h (libdlm_hip.so),
a C++20 host layer (libdollama.so) that keeps the reference's UNet /
VRAM-arena / backend-plugin surface, and a thin Python mirror used by the
tests and the benchmark.  Nothing here falls back to the CPU: if the HIP
library is missing, importing ``dollama_amd.ops`` still works but the first
call raises.
"""
__version__ = "0.1.0"
