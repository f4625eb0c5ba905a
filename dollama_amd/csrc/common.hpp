// Shared device types and host helpers for the gfx950 kernels.
//
// Device code is written for CDNA4 (gfx950) only: wave64, MFMA
// v_mfma_f32_32x32x16_f16, 160 KiB LDS per CU.  fp16 values are _Float16;
// accumulation is always fp32.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include <string>
#include <tuple>
#include <type_traits>
#include <utility>

#include "../../include/dlm.h"

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace dlm {

// ---------------------------------------------------------------------------
// MFMA 32x32x16 f16 -> f32 (gfx950).  Operand layouts (wave64):
//   A (32 rows x 16 k): lane l holds row (l & 31), k = 8*(l >> 5) + [0..7]
//   B (16 k x 32 cols): lane l holds col (l & 31), k = 8*(l >> 5) + [0..7]
//   C/D (32 x 32):      lane l holds col (l & 31); element e is
//                       row 8*(e >> 2) + 4*(l >> 5) + (e & 3)
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x16 mfma32x32x16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// MFMA 16x16x32 f16 -> f32 (gfx950):
//   A (16 rows x 32 k): lane l holds row (l & 15), k = 8*(l >> 4) + [0..7]
//   B (32 k x 16 cols): lane l holds col (l & 15), k = 8*(l >> 4) + [0..7]
//   C/D (16 x 16):      lane l holds col (l & 15), rows 4*(l >> 4) + [0..3]
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int mfma_row(int e, int lane) {
  return 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}

// x * sigmoid(x) with the hardware exp2 and reciprocal (about 1 ulp each, far
// below the fp16 rounding every caller applies): five VALU instructions
// against ten more for an IEEE division.  Large negative x gives -0 through
// 1 / inf, as the quotient form does.
__device__ __forceinline__ float silu_f(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

__device__ __forceinline__ float gelu_erf_f(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
}

// erf by Abramowitz & Stegun, Handbook of Mathematical Functions, 7.1.26:
// erf(z) = 1 - (a1 t + ... + a5 t^5) exp(-z^2), t = 1 / (1 + p z), z >= 0,
// |error| <= 1.5e-7 (far below the fp16 output step).  Branch-free: one
// reciprocal, one exp2, six FMAs; erf(-z) = -erf(z).
__device__ __forceinline__ float erf_as(float x) {
  const float z = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, z, 1.0f));
  float poly = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  poly = __builtin_fmaf(poly, t, 1.421413741f);
  poly = __builtin_fmaf(poly, t, -0.284496736f);
  poly = __builtin_fmaf(poly, t, 0.254829592f);
  poly *= t;
  const float e = __builtin_amdgcn_exp2f(-z * z * 1.4426950408889634f);
  const float r = __builtin_fmaf(-poly, e, 1.0f);
  return __builtin_copysignf(r, x);
}
__device__ __forceinline__ float gelu_erf_fast(float x) {
  return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752f));
}

// Wave-wide reductions (wave64) without LDS round trips: two DPP quad
// permutations (lane ^ 1, lane ^ 2), the half-row and row mirrors (lane i with
// 7 - i, then 15 - i: the other quad, then the other half-row), then the
// row-pair and half-wave swaps of gfx950 (v_permlane16_swap,
// v_permlane32_swap).  Each step adds the same two operands on both partners,
// so every lane ends with the same value.  Needs all 64 lanes active.
template <int CTRL>
__device__ __forceinline__ unsigned dpp_u32(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
  constexpr int W = sizeof(T) / 4;
  auto step_dpp = [&](auto ctrl) {
    unsigned w[W];
    __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = dpp_u32<decltype(ctrl)::value>(w[i]);
    T o;
    __builtin_memcpy(&o, w, sizeof(T));
    v = op(v, o);
  };
  step_dpp(std::integral_constant<int, kDppXor1>{});
  step_dpp(std::integral_constant<int, kDppXor2>{});
  step_dpp(std::integral_constant<int, kDppHalfMirror>{});
  step_dpp(std::integral_constant<int, kDppMirror>{});
  auto step_swap = [&](auto sw) {
    unsigned w[W], a[W], b[W];
    __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const auto s = sw(w[i]);
      a[i] = s[0];
      b[i] = s[1];
    }
    T x, y;
    __builtin_memcpy(&x, a, sizeof(T));
    __builtin_memcpy(&y, b, sizeof(T));
    v = op(x, y);
  };
  step_swap([](unsigned u) { return __builtin_amdgcn_permlane16_swap(u, u, false, false); });
  step_swap([](unsigned u) { return __builtin_amdgcn_permlane32_swap(u, u, false, false); });
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  return wave_reduce(v, [](double a, double b) { return a + b; });
}

// GroupNorm chunk statistics, one definition for every producer (the
// statistics pass over a tensor, and GEMM / conv epilogues that write them
// for their own output), so they agree bit for bit and a sample's statistics
// never depend on the batch or on the kernel that computed them.
// Chunk k of a sample is its pixel rows [64k, min(64k + 64, HW)).  Per
// channel, over the chunk's rows in ascending order, with shift = the
// chunk's first value:
//   d = x - shift;  s1 = s1 + d;  s2 = fma(d, d, s2)
// and then (mean, M2) = (shift + s1 / cnt, max(s2 - s1 (s1 / cnt), 0)).
// Stored as float2 [N][chunks][C].
constexpr int kGnChunk = 64;
__device__ __forceinline__ void gn_stat_add(float x, float shift, float& s1, float& s2) {
  const float d = x - shift;
  s1 = s1 + d;
  s2 = __builtin_fmaf(d, d, s2);
}
__device__ __forceinline__ float2 gn_stat_finish(float s1, float s2, float shift, int cnt) {
  // a whole chunk divides by 64 exactly as a multiply, whatever the division lowering
  const float md = cnt == kGnChunk ? s1 * (1.0f / kGnChunk) : s1 / (float)cnt;
  return make_float2(shift + md, fmaxf(__builtin_fmaf(-s1, md, s2), 0.0f));
}

// Grid of a grid-stride elementwise launch over n items.
static inline int grid_for(long long n, int threads = 256, int cap = 8192) {
  return (int)std::max<long long>(1, std::min<long long>((n + threads - 1) / threads, cap));
}

#define GRID_STRIDE(i, n)                                                          \
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < (n); \
       i += (long long)gridDim.x * blockDim.x)

}  // namespace dlm

// ---------------------------------------------------------------------------
// Host-side error state shared by every C entry point.
// ---------------------------------------------------------------------------
namespace dlm {
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what, const char* file, int line);
// Grow-only staging buffer `slot` of the current device for `stream`, used by
// the reference-layout entry points.  Growing it synchronises the device and
// frees the old block, so those entry points are not capturable into a graph
// until their slots have reached size.
void* scratch_slot(size_t bytes, int slot, hipStream_t stream, int* status);
int scratch_release(hipStream_t stream);
size_t scratch_bytes();
int split_workspace_release(hipStream_t stream);
size_t split_workspace_bytes();
// GroupNorm chunk statistics (kGnChunk) of fp16 channels-last x [N, HW, C]
// (row stride ld) into stats [N][chunks][C] (norm.hip).
int gn_chunk_stats(const void* x, int ld, int N, int HW, int C, float2* stats, hipStream_t s);
// Name of the kernel an entry point launches last (per thread), for
// per-kernel timing attribution (dlm_last_kernel).
void note_kernel(const char* name);
// GEMM / conv launches also note their problem: rows M, output columns N,
// reduction length K, flags (bit 0 residual, bits 4.. epilogue activation,
// bit 8 implicit-GEMM conv).
void note_dims(int M, int N, int K, int flags);
// Events armed by dlm_prof_arm on this thread (stop == nullptr: disarmed) and
// the number of kernels launched since arming.
struct ProfArm {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
  int launched = 0;
};
ProfArm& prof_arm();

// Every kernel launch of the library.  The arguments are converted to the
// kernel's parameter types and passed by address, as hipLaunchKernelGGL does;
// while dispatch timing is armed the launch goes through hipExtLaunchKernel
// with the armed events attached to this dispatch.
template <typename... F, typename... A>
inline void launch(void (*kernel)(F...), const dim3& grid, const dim3& block, uint32_t shmem,
                   hipStream_t s, A&&... a) {
  static_assert(sizeof...(F) == sizeof...(A), "kernel argument count mismatch");
  std::tuple<F...> args{std::forward<A>(a)...};
  std::apply(
      [&](auto&... e) {
        void* ptrs[] = {static_cast<void*>(&e)..., nullptr};
        ProfArm& p = prof_arm();
        if (p.stop) {
          (void)hipExtLaunchKernel(reinterpret_cast<void*>(kernel), grid, block, ptrs, shmem, s,
                                   p.launched == 0 ? p.start : nullptr, p.stop, 0);
          ++p.launched;
        } else {
          (void)hipLaunchKernel(reinterpret_cast<void*>(kernel), grid, block, ptrs, shmem, s);
        }
      },
      args);
}
}  // namespace dlm

#define DLM_LAUNCH(name, ...)          \
  do {                                 \
    ::dlm::note_kernel(name);          \
    ::dlm::launch(__VA_ARGS__);        \
  } while (0)

#define DLM_HIP(expr)                                                          \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess) return dlm::hip_fail(e_, #expr, __FILE__, __LINE__); \
  } while (0)

#define DLM_LAUNCH_CHECK()                                                     \
  do {                                                                         \
    hipError_t e_ = hipGetLastError();                                         \
    if (e_ != hipSuccess) return dlm::hip_fail(e_, "kernel launch", __FILE__, __LINE__); \
  } while (0)

#define DLM_REQUIRE(cond, msg)                                                 \
  do {                                                                         \
    if (!(cond)) return dlm::fail(DLM_ERR_INVALID_ARG, std::string(__func__) + ": " + (msg)); \
  } while (0)

static inline bool dlm_aligned16(const void* p) { return (((uintptr_t)p) & 15) == 0; }
