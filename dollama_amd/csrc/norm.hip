// GroupNorm(+SiLU) and LayerNorm for gfx950.  Both are HBM-bound: every
// kernel moves 16-byte vectors and keeps statistics in fp32 (merged in fp64).
//
// GroupNorm replaces launch_group_norm / _mb / _silu
// (reference src/kernels/groupnorm.cu:91-148, :246-353, :428-461), which
// accumulate sum / sum-of-squares per (n, group) in fp32 and clamp the
// variance at 0.  Here activations are channels-last [N, HW, C], so a pixel
// row holds every group; the statistics are computed per channel over pixel
// chunks with a per-chunk shift (first pixel of the chunk), which keeps the
// fp32 partial sums well conditioned, and merged per group with Chan's
// pairwise formula in fp64.  Three launches: partial statistics over
// (chunk, n), a per-(n, group) merge producing per-channel scale/shift, and a
// vectorised apply (+SiLU) pass.  Deterministic: fixed reduction order.
//
// LayerNorm replaces launch_layer_norm (src/kernels/layernorm.cu:78-126):
// one wave per row, the row held in registers, exact two-pass mean/variance.
#include <algorithm>

#include "common.hpp"

namespace dlm {

struct GnPlan {
  int S;        // 16-byte vectors per pixel row (C / 8)
  int R;        // pixel rows in flight per block
  int threads;  // S * R
  int chunk;    // pixels per chunk
  int chunks;   // chunks per sample
};

static GnPlan gn_plan(int N, int C, int HW) {
  GnPlan p;
  p.S = C / 8;
  p.R = std::max(1, 256 / p.S);
  while (p.S * p.R > 1024 && p.R > 1) --p.R;
  p.threads = p.S * p.R;
  const int target = std::max(1, 512 / std::max(1, N));
  p.chunk = std::max(p.R * 4, (HW + target - 1) / target);
  p.chunks = (HW + p.chunk - 1) / p.chunk;
  return p;
}

static size_t gn_workspace_bytes(int N, int C, int HW) {
  const GnPlan p = gn_plan(N, C, HW);
  return (size_t)N * p.chunks * C * sizeof(float2) + (size_t)N * C * sizeof(float2) + 256;
}

__device__ __forceinline__ void load8(const f16* p, float (&v)[8]) {
  const f16x8 x = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)x[i];
}

// partial[n][chunk][c] = (mean_c, M2_c) over the chunk's pixels
__global__ void gn_partial_kernel(const f16* __restrict__ a, int Ca, int lda,
                                  const f16* __restrict__ b, int ldb, int HW, int C, int chunk,
                                  int chunks, int S, int R, float2* __restrict__ partial) {
  extern __shared__ float2 red[];  // [R][C]
  const int n = blockIdx.y, ch = blockIdx.x;
  const int tid = threadIdx.x;
  const int s = tid % S, r = tid / S;
  const int c = s * 8;
  const f16* src;
  int ld;
  if (c < Ca) {
    src = a + (size_t)n * HW * lda + c;
    ld = lda;
  } else {
    src = b + (size_t)n * HW * ldb + (c - Ca);
    ld = ldb;
  }
  const int p0 = ch * chunk;
  const int p1 = min(HW, p0 + chunk);
  float shift[8], s1[8], s2[8];
  load8(src + (size_t)p0 * ld, shift);
#pragma unroll
  for (int i = 0; i < 8; ++i) s1[i] = s2[i] = 0.0f;
  for (int p = p0 + r; p < p1; p += R) {
    float v[8];
    load8(src + (size_t)p * ld, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float d = v[i] - shift[i];
      s1[i] += d;
      s2[i] += d * d;
    }
  }
  if (r < R) {
#pragma unroll
    for (int i = 0; i < 8; ++i) red[r * C + c + i] = make_float2(s1[i], s2[i]);
  }
  __syncthreads();
  if (r == 0) {
    const float cnt = (float)(p1 - p0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float t1 = 0.0f, t2 = 0.0f;
      for (int rr = 0; rr < R; ++rr) {
        const float2 q = red[rr * C + c + i];
        t1 += q.x;
        t2 += q.y;
      }
      const float mean_d = t1 / cnt;
      const float m2 = fmaxf(t2 - t1 * mean_d, 0.0f);
      partial[((size_t)n * chunks + ch) * C + c + i] = make_float2(shift[i] + mean_d, m2);
    }
  }
}

// One block (64 threads) per (n, group): merge (chunk, channel) partials with
// Chan's formula in fp64, then emit per-channel scale/shift.
__global__ void gn_finalize_kernel(const float2* __restrict__ partial, int HW, int C, int G,
                                   int chunk, int chunks, const f16* __restrict__ gamma,
                                   const f16* __restrict__ beta, float eps,
                                   float2* __restrict__ ss) {
  const int n = blockIdx.x / G, g = blockIdx.x % G;
  const int cpg = C / G;
  const int tid = threadIdx.x;
  double cnt = 0.0, mean = 0.0, m2 = 0.0;
  const int entries = chunks * cpg;
  for (int e = tid; e < entries; e += blockDim.x) {
    const int chn = e / cpg, ci = e % cpg;
    const float2 q = partial[((size_t)n * chunks + chn) * C + g * cpg + ci];
    const double nb = (double)(min(HW, (chn + 1) * chunk) - chn * chunk);
    const double delta = (double)q.x - mean;
    const double tot = cnt + nb;
    mean += delta * nb / tot;
    m2 += (double)q.y + delta * delta * cnt * nb / tot;
    cnt = tot;
  }
  __shared__ double sc[64], sm[64], sq[64];
  sc[tid] = cnt;
  sm[tid] = mean;
  sq[tid] = m2;
  __syncthreads();
  if (tid == 0) {
    double c0 = 0.0, mu = 0.0, q2 = 0.0;
    for (int t = 0; t < (int)blockDim.x; ++t) {
      const double nb = sc[t];
      if (nb == 0.0) continue;
      const double delta = sm[t] - mu;
      const double tot = c0 + nb;
      mu += delta * nb / tot;
      q2 += sq[t] + delta * delta * c0 * nb / tot;
      c0 = tot;
    }
    sm[0] = mu;
    sq[0] = q2 / c0;
  }
  __syncthreads();
  const double mu = sm[0];
  const double var = sq[0] > 0.0 ? sq[0] : 0.0;
  const float rstd = (float)(1.0 / sqrt(var + (double)eps));
  for (int ci = tid; ci < cpg; ci += blockDim.x) {
    const int c = g * cpg + ci;
    const float gm = gamma ? (float)gamma[c] : 1.0f;
    const float bt = beta ? (float)beta[c] : 0.0f;
    const float scale = gm * rstd;
    ss[(size_t)n * C + c] = make_float2(scale, bt - (float)mu * scale);
  }
}

__global__ void gn_apply_kernel(const f16* __restrict__ a, int Ca, int lda,
                                const f16* __restrict__ b, int ldb, f16* __restrict__ out,
                                int ldo, int HW, int C, long long total_vec,
                                const float2* __restrict__ ss, int silu) {
  const int S = C / 8;
  for (long long v = blockIdx.x * (long long)blockDim.x + threadIdx.x; v < total_vec;
       v += (long long)gridDim.x * blockDim.x) {
    const long long row = v / S;  // n*HW + p
    const int s = (int)(v - row * S);
    const int n = (int)(row / HW);
    const int c = s * 8;
    const f16* src = c < Ca ? a + (size_t)row * lda + c : b + (size_t)row * ldb + (c - Ca);
    float x[8];
    load8(src, x);
    const float4* ssv = reinterpret_cast<const float4*>(ss + (size_t)n * C + c);
    f16x8 y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 q = ssv[i];
      float y0 = x[2 * i] * q.x + q.y;
      float y1 = x[2 * i + 1] * q.z + q.w;
      if (silu) {
        y0 = silu_f(y0);
        y1 = silu_f(y1);
      }
      y[2 * i] = (f16)y0;
      y[2 * i + 1] = (f16)y1;
    }
    *reinterpret_cast<f16x8*>(out + (size_t)row * ldo + c) = y;
  }
}

int group_norm_nhwc(const void* in_a, int C_a, int ld_a, const void* in_b, int ld_b,
                    const void* gamma, const void* beta, void* out, int ld_out, int N, int HW,
                    int C, int G, float eps, int silu, void* ws, hipStream_t s) {
  const GnPlan p = gn_plan(N, C, HW);
  float2* partial = (float2*)ws;
  float2* ss = partial + (size_t)N * p.chunks * C;
  ss = (float2*)(((uintptr_t)ss + 15) & ~(uintptr_t)15);
  const f16* a = (const f16*)in_a;
  const f16* b = in_b ? (const f16*)in_b : a;
  const size_t red_bytes = (size_t)p.R * C * sizeof(float2);
  if (red_bytes > 160 * 1024)
    return fail(DLM_ERR_UNSUPPORTED, "group_norm: channel count too large for one block");
  hipLaunchKernelGGL(gn_partial_kernel, dim3(p.chunks, N), dim3(p.threads), red_bytes, s, a, C_a,
                     ld_a, b, ld_b, HW, C, p.chunk, p.chunks, p.S, p.R, partial);
  DLM_LAUNCH_CHECK();
  hipLaunchKernelGGL(gn_finalize_kernel, dim3(N * G), dim3(64), 0, s, partial, HW, C, G, p.chunk,
                     p.chunks, (const f16*)gamma, (const f16*)beta, eps, ss);
  DLM_LAUNCH_CHECK();
  const long long total_vec = (long long)N * HW * (C / 8);
  const int blocks = (int)std::min<long long>((total_vec + 255) / 256, 4096);
  hipLaunchKernelGGL(gn_apply_kernel, dim3(blocks), dim3(256), 0, s, a, C_a, ld_a, b, ld_b,
                     (f16*)out, ld_out, HW, C, total_vec, ss, silu);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

// ---------------------------------------------------------------------------
// LayerNorm: one wave per row, up to 8 vectors (64 channels) per lane.
// ---------------------------------------------------------------------------
template <int VPL>
__global__ void __launch_bounds__(256)
layer_norm_kernel(const f16* __restrict__ in, const f16* __restrict__ gamma,
                  const f16* __restrict__ beta, f16* __restrict__ out, int rows, int C,
                  float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int S = C / 8;
  const f16* x = in + (size_t)row * C;
  float v[VPL][8];
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int s = lane + 64 * j;
    if (s < S) {
      load8(x + s * 8, v[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) sum += v[j][i];
    }
  }
  const float mean = wave_sum(sum) / (float)C;
  float sq = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int s = lane + 64 * j;
    if (s < S) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = v[j][i] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = rsqrtf(wave_sum(sq) / (float)C + eps);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int s = lane + 64 * j;
    if (s < S) {
      float g[8], bb[8];
      if (gamma) load8(gamma + s * 8, g);
      else
#pragma unroll
        for (int i = 0; i < 8; ++i) g[i] = 1.0f;
      if (beta) load8(beta + s * 8, bb);
      else
#pragma unroll
        for (int i = 0; i < 8; ++i) bb[i] = 0.0f;
      f16x8 y;
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = (f16)((v[j][i] - mean) * rstd * g[i] + bb[i]);
      *reinterpret_cast<f16x8*>(out + (size_t)row * C + s * 8) = y;
    }
  }
}

// Scalar fallback for C not a multiple of 8 (reference API generality).
__global__ void layer_norm_scalar_kernel(const f16* __restrict__ in, const f16* __restrict__ gamma,
                                         const f16* __restrict__ beta, f16* __restrict__ out,
                                         int rows, int C, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const f16* x = in + (size_t)row * C;
  float sum = 0.0f;
  for (int c = lane; c < C; c += 64) sum += (float)x[c];
  const float mean = wave_sum(sum) / (float)C;
  float sq = 0.0f;
  for (int c = lane; c < C; c += 64) {
    const float d = (float)x[c] - mean;
    sq += d * d;
  }
  const float rstd = rsqrtf(wave_sum(sq) / (float)C + eps);
  for (int c = lane; c < C; c += 64) {
    const float g = gamma ? (float)gamma[c] : 1.0f;
    const float b = beta ? (float)beta[c] : 0.0f;
    out[(size_t)row * C + c] = (f16)(((float)x[c] - mean) * rstd * g + b);
  }
}

int layer_norm(const void* in, const void* gamma, const void* beta, void* out, int rows, int C,
               float eps, hipStream_t s) {
  const dim3 grid((rows + 3) / 4), block(256);
  const bool vec = C % 8 == 0 && dlm_aligned16(in) && dlm_aligned16(out) &&
                   (!gamma || dlm_aligned16(gamma)) && (!beta || dlm_aligned16(beta));
  const f16* x = (const f16*)in;
  const f16* g = (const f16*)gamma;
  const f16* b = (const f16*)beta;
  f16* y = (f16*)out;
  if (vec && C <= 64 * 8 * 1)
    hipLaunchKernelGGL(layer_norm_kernel<1>, grid, block, 0, s, x, g, b, y, rows, C, eps);
  else if (vec && C <= 64 * 8 * 2)
    hipLaunchKernelGGL(layer_norm_kernel<2>, grid, block, 0, s, x, g, b, y, rows, C, eps);
  else if (vec && C <= 64 * 8 * 3)
    hipLaunchKernelGGL(layer_norm_kernel<3>, grid, block, 0, s, x, g, b, y, rows, C, eps);
  else if (vec && C <= 64 * 8 * 8)
    hipLaunchKernelGGL(layer_norm_kernel<8>, grid, block, 0, s, x, g, b, y, rows, C, eps);
  else
    hipLaunchKernelGGL(layer_norm_scalar_kernel, grid, block, 0, s, x, g, b, y, rows, C, eps);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int nchw_to_nhwc(const void* in, void* out, int N, int C, int HW, int C_pad, hipStream_t s);
int nhwc_to_nchw(const void* in, void* out, int N, int C, int HW, int C_pad, hipStream_t s);

}  // namespace dlm

using namespace dlm;

extern "C" {

size_t dlm_group_norm_nhwc_workspace_bytes(int N, int C, int HW) {
  if (N <= 0 || C <= 0 || HW <= 0) return 0;
  return gn_workspace_bytes(N, C, HW);
}

int dlm_group_norm_nhwc_fp16(const void* in_a, int C_a, int ld_a, const void* in_b, int ld_b,
                             const void* gamma, const void* beta, void* out, int ld_out, int N,
                             int HW, int C, int num_groups, float eps, int fuse_silu,
                             void* workspace, void* stream) {
  if (N <= 0 || HW <= 0 || C <= 0 || num_groups <= 0) return DLM_OK;
  DLM_REQUIRE(in_a && out && workspace, "NULL pointer");
  DLM_REQUIRE(C % num_groups == 0, "C must be divisible by num_groups");
  DLM_REQUIRE(C % 8 == 0 && C_a % 8 == 0 && C_a > 0 && C_a <= C, "channel counts must be multiples of 8");
  DLM_REQUIRE(C_a == C || in_b != nullptr, "in_b NULL with C_a < C");
  DLM_REQUIRE(ld_a % 8 == 0 && ld_a >= C_a && ld_out % 8 == 0 && ld_out >= C, "bad row strides");
  DLM_REQUIRE(C_a == C || (ld_b % 8 == 0 && ld_b >= C - C_a), "bad ld_b");
  DLM_REQUIRE(dlm_aligned16(in_a) && dlm_aligned16(out) && (!in_b || dlm_aligned16(in_b)),
              "buffers must be 16-byte aligned");
  DLM_REQUIRE(dlm_aligned16(workspace), "workspace must be 16-byte aligned");
  return group_norm_nhwc(in_a, C_a, ld_a, in_b, ld_b, gamma, beta, out, ld_out, N, HW, C,
                         num_groups, eps, fuse_silu, workspace, (hipStream_t)stream);
}

int dlm_group_norm_fp16(const void* in, const void* gamma, const void* beta, void* out, int N,
                        int C, int H, int W, int num_groups, float eps, int fuse_silu,
                        void* stream) {
  if (N <= 0 || C <= 0 || H <= 0 || W <= 0 || num_groups <= 0) return DLM_OK;
  DLM_REQUIRE(in && out, "NULL pointer");
  DLM_REQUIRE(C % num_groups == 0, "C must be divisible by num_groups");
  hipStream_t s = (hipStream_t)stream;
  const int HW = H * W;
  const int Cp = (C + 7) & ~7;
  if (Cp != C)
    return fail(DLM_ERR_UNSUPPORTED, "dlm_group_norm_fp16: C must be a multiple of 8");
  int st = DLM_OK;
  f16* x = (f16*)scratch((size_t)N * HW * Cp * 2, 4, s, &st);
  if (!x) return st;
  void* ws = scratch(gn_workspace_bytes(N, Cp, HW), 5, s, &st);
  if (!ws) return st;
  if ((st = nchw_to_nhwc(in, x, N, C, HW, Cp, s)) != DLM_OK) return st;
  if ((st = group_norm_nhwc(x, Cp, Cp, nullptr, 0, gamma, beta, x, Cp, N, HW, Cp, num_groups, eps,
                            fuse_silu, ws, s)) != DLM_OK)
    return st;
  return nhwc_to_nchw(x, out, N, C, HW, Cp, s);
}

int dlm_layer_norm_fp16(const void* in, const void* gamma, const void* beta, void* out, int rows,
                        int C, float eps, void* stream) {
  if (rows <= 0 || C <= 0) return DLM_OK;
  DLM_REQUIRE(in && out, "NULL pointer");
  return layer_norm(in, gamma, beta, out, rows, C, eps, (hipStream_t)stream);
}

}  // extern "C"
