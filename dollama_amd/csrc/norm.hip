// GroupNorm(+SiLU) and LayerNorm for gfx950.  Both are HBM-bound: every
// kernel moves 16-byte vectors and keeps statistics in fp32 (merged in fp64).
//
// GroupNorm replaces launch_group_norm / _mb / _silu
// (reference src/kernels/groupnorm.cu:91-148, :246-353, :428-461), which
// accumulate sum / sum-of-squares per (n, group) in fp32 and clamp the
// variance at 0.  Here activations are channels-last [N, HW, C], so a pixel
// row holds every group; the statistics are computed per channel over pixel
// chunks with a per-chunk shift (first pixel of the chunk), which keeps the
// fp32 partial sums well conditioned; each block combines its channels into
// per-group (mean, M2) with the equal-count form of Chan's formula, and the
// chunks of one (n, group) are merged in fp64 by the two-pass decomposition
// (mean first, then sum of M2_b + n_b (m_b - mean)^2).  Three launches:
// partial statistics over (chunk, n), the per-(n, group) merge producing
// per-channel scale/shift, and a vectorised apply (+SiLU) pass.
// Deterministic: fixed reduction order.
//
// fp16 inputs of up to 16384 pixels per sample (every UNet GroupNorm at 1024²) use the
// per-channel chunk statistics of common.hpp (64-pixel chunks, [N][chunks][C])
// instead of the per-group partials: a GEMM / conv epilogue can write those
// for its own output (dlm_conv_nhwc_args::gn_stats), and then the GroupNorm
// runs from them (dlm_group_norm_nhwc_prestats_fp16) with no statistics pass.
// The statistics pass computes the same values bit for bit.
//
// LayerNorm replaces launch_layer_norm (src/kernels/layernorm.cu:78-126):
// one wave per row, the row held in registers, exact two-pass mean/variance.
#include <algorithm>
#include <type_traits>

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
  // chunking depends on HW only, so each sample's statistics are computed
  // identically whatever the batch size (B=2 == 2 x B=1, bit for bit).
  // About 1024 chunks per sample: a streaming pass needs several waves per
  // CU in flight (256 chunks measured 3.4 TB/s on 1024x1024x128 fp32).
  (void)N;
  const int target = 1024;
  p.chunk = std::max(p.R * 4, (HW + target - 1) / target);
  p.chunks = (HW + p.chunk - 1) / p.chunk;
  return p;
}

// Per-channel chunk statistics (the form a producer's epilogue can write):
// fp16 inputs with at most this many pixels per sample.
constexpr int kGnChanMaxHW = 16384;
static inline int gn_chan_chunks(int HW) { return (HW + kGnChunk - 1) / kGnChunk; }

static size_t gn_workspace_bytes(int N, int C, int HW) {
  const GnPlan p = gn_plan(N, C, HW);
  const size_t legacy = (size_t)N * p.chunks * C * sizeof(float2);
  const size_t chan = HW <= kGnChanMaxHW ? (size_t)N * gn_chan_chunks(HW) * C * sizeof(float2) : 0;
  return std::max(legacy, chan) + (size_t)N * C * sizeof(float2) + 256;
}
// scale/shift follow the statistics, 16-byte aligned
static float2* gn_ss_of(void* ws, int N, int C, int HW) {
  const GnPlan p = gn_plan(N, C, HW);
  const size_t legacy = (size_t)N * p.chunks * C * sizeof(float2);
  const size_t chan = HW <= kGnChanMaxHW ? (size_t)N * gn_chan_chunks(HW) * C * sizeof(float2) : 0;
  return (float2*)(((uintptr_t)ws + std::max(legacy, chan) + 15) & ~(uintptr_t)15);
}

__device__ __forceinline__ void load8(const f16* p, float (&v)[8]) {
  const f16x8 x = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)x[i];
}
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
  const float4 x0 = reinterpret_cast<const float4*>(p)[0];
  const float4 x1 = reinterpret_cast<const float4*>(p)[1];
  v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
  v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
}

// partial[n][g][chunk] = (mean, M2) of group g over the chunk's pixels (a
// group's chunks contiguous, so the merge's lanes read consecutive partials).
// Per-channel sums are shifted by the chunk's first pixel, reduced over the R
// rows in LDS, turned into per-channel (mean, M2) and combined per group with
// the equal-count form of Chan's formula.
// T is the activation type: fp16, or fp32 for the VAE decoder's wide-range
// stages (reference k_group_norm_f32, src/kernels/vae_decode.cu:466-545).
template <typename T>
__global__ void gn_partial_kernel(const T* __restrict__ a, int Ca, int lda,
                                  const T* __restrict__ b, int ldb, int HW, int C, int G,
                                  int chunk, int chunks, int S, int R,
                                  float2* __restrict__ partial) {
  extern __shared__ float2 red[];  // [R][C], reused as [C] per-channel (mean, M2)
  const int n = blockIdx.y, ch = blockIdx.x;
  const int tid = threadIdx.x;
  const int s = tid % S, r = tid / S;
  const int c = s * 8;
  const T* src;
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
  int p = p0 + r;
  // four rows per iteration: four independent loads in flight per thread
  for (; p + 3 * R < p1; p += 4 * R) {
    float v[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) load8(src + (size_t)(p + u * R) * ld, v[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = v[u][i] - shift[i];
        s1[i] += d;
        s2[i] += d * d;
      }
  }
  for (; p < p1; p += R) {
    float v[8];
    load8(src + (size_t)p * ld, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float d = v[i] - shift[i];
      s1[i] += d;
      s2[i] += d * d;
    }
  }
  // LDS entries channel-interleaved (channel s*8+i at i*S+s), so the lanes of
  // one store or load touch consecutive 8-byte words
#pragma unroll
  for (int i = 0; i < 8; ++i) red[r * C + i * S + s] = make_float2(s1[i], s2[i]);
  __syncthreads();
  const float cnt = (float)(p1 - p0);
  float2 mc[8];
  if (r == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float t1 = 0.0f, t2 = 0.0f;
      for (int rr = 0; rr < R; ++rr) {
        const float2 q = red[rr * C + i * S + s];
        t1 += q.x;
        t2 += q.y;
      }
      const float md = t1 / cnt;
      mc[i] = make_float2(shift[i] + md, fmaxf(t2 - t1 * md, 0.0f));
    }
  }
  __syncthreads();
  if (r == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) red[i * S + s] = mc[i];
  }
  __syncthreads();
  const int cpg = C / G;
  auto chan = [&](int ch) { return red[(ch & 7) * S + (ch >> 3)]; };
  for (int g = tid; g < G; g += blockDim.x) {
    float mean = 0.0f;
    for (int ci = 0; ci < cpg; ++ci) mean += chan(g * cpg + ci).x;
    mean /= (float)cpg;
    float m2 = 0.0f;
    for (int ci = 0; ci < cpg; ++ci) {
      const float2 q = chan(g * cpg + ci);
      const float d = q.x - mean;
      m2 += q.y + cnt * d * d;
    }
    partial[((size_t)n * G + g) * chunks + ch] = make_float2(mean, m2);
  }
}

__device__ __forceinline__ void chan_merge(double& n, double& mean, double& m2, double nb,
                                           double mb, double m2b) {
  if (nb == 0.0) return;
  const double tot = n + nb;
  const double delta = mb - mean;
  mean += delta * nb / tot;
  m2 += m2b + delta * delta * n * nb / tot;
  n = tot;
}

// One wave per (n, group): combine the chunk partials (count n_b, mean m_b,
// M2_b) in fp64 by the two-pass decomposition
//   mean = sum(n_b m_b) / sum(n_b),  M2 = sum(M2_b + n_b (m_b - mean)^2),
// which needs no division per chunk (a pairwise Chan merge needs one), then
// emit per-channel scale = gamma*rstd and shift = beta - mean*scale.  Each
// lane sums its chunks in order and the wave reduction adds identical operand
// pairs on both partners, so every lane ends with the same, launch-invariant
// result.
__global__ void gn_finalize_kernel(const float2* __restrict__ partial, int HW, int C, int G,
                                   int chunk, int chunks, const f16* __restrict__ gamma,
                                   const f16* __restrict__ beta, float eps,
                                   float2* __restrict__ ss) {
  const int n = blockIdx.x / G, g = blockIdx.x % G;
  const int lane = threadIdx.x;
  const int cpg = C / G;
  const float2* pg = partial + ((size_t)n * G + g) * chunks;
  double cnt = 0.0, s1 = 0.0;
  for (int chn = lane; chn < chunks; chn += 64) {
    const float2 q = pg[chn];
    const double nb = (double)(min(HW, (chn + 1) * chunk) - chn * chunk) * cpg;
    cnt += nb;
    s1 = fma(nb, (double)q.x, s1);
  }
  cnt = wave_sum_f64(cnt);
  s1 = wave_sum_f64(s1);
  const double mean = cnt > 0.0 ? s1 / cnt : 0.0;
  double m2 = 0.0;
  for (int chn = lane; chn < chunks; chn += 64) {
    const float2 q = pg[chn];
    const double nb = (double)(min(HW, (chn + 1) * chunk) - chn * chunk) * cpg;
    const double d = (double)q.x - mean;
    m2 += (double)q.y + nb * d * d;
  }
  m2 = wave_sum_f64(m2);
  const double var = cnt > 0.0 ? fmax(m2 / cnt, 0.0) : 0.0;
  const float rstd = (float)(1.0 / sqrt(var + (double)eps));
  for (int ci = lane; ci < cpg; ci += 64) {
    const int c = g * cpg + ci;
    const float gm = gamma ? (float)gamma[c] : 1.0f;
    const float bt = beta ? (float)beta[c] : 0.0f;
    const float scale = gm * rstd;
    ss[(size_t)n * C + c] = make_float2(scale, bt - (float)mean * scale);
  }
}

// Per-channel chunk statistics of fp16 [N, HW, C] (+ concatenated second
// source): one thread per (chunk, 8-channel vector), the chunk's rows in
// ascending order, eight rows' loads in flight.
__global__ void __launch_bounds__(256)
gn_chan_stats_kernel(const f16* __restrict__ a, int Ca, int lda, const f16* __restrict__ b, int ldb,
                     int HW, int C, int S, int chunks, float2* __restrict__ stats) {
  const int n = blockIdx.y;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  const int k = idx / S, s = idx - k * S;
  if (k >= chunks) return;
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
  const int p0 = k * kGnChunk, p1 = min(HW, p0 + kGnChunk);
  float shift[8], s1[8], s2[8];
  load8(src + (size_t)p0 * ld, shift);
#pragma unroll
  for (int i = 0; i < 8; ++i) s1[i] = s2[i] = 0.0f;
  int p = p0;
  for (; p + 8 <= p1; p += 8) {
    float v[8][8];
#pragma unroll
    for (int u = 0; u < 8; ++u) load8(src + (size_t)(p + u) * ld, v[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) gn_stat_add(v[u][i], shift[i], s1[i], s2[i]);
  }
  for (; p < p1; ++p) {
    float v[8];
    load8(src + (size_t)p * ld, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) gn_stat_add(v[i], shift[i], s1[i], s2[i]);
  }
  float4* dst = reinterpret_cast<float4*>(stats + ((size_t)n * chunks + k) * C + c);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float2 e0 = gn_stat_finish(s1[2 * i], s2[2 * i], shift[2 * i], p1 - p0);
    const float2 e1 = gn_stat_finish(s1[2 * i + 1], s2[2 * i + 1], shift[2 * i + 1], p1 - p0);
    dst[i] = make_float4(e0.x, e0.y, e1.x, e1.y);
  }
}

// Merge of the per-channel chunk statistics of one (n, group), one block of
// kGnFinT threads each, in fp64 by the same two-pass decomposition as
// gn_finalize_kernel; entry j = (chunk j / cpg, channel j % cpg) of the
// group.  Per-thread sums in order, then the wave reduction (the same value
// in every lane) and the waves' results added in a fixed tree, so every
// thread holds the same, launch-invariant result.
constexpr int kGnFinT = 512;
constexpr int kGnFinW = kGnFinT / 64;
static_assert(kGnFinW >= 2 && (kGnFinW & (kGnFinW - 1)) == 0, "the tree adds a power of two of wave sums");
__device__ __forceinline__ double gn_block_sum(double v, double* red) {
  v = wave_sum_f64(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red free (an earlier sum's readers are done)
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  double t[kGnFinW / 2];
#pragma unroll
  for (int i = 0; i < kGnFinW / 2; ++i) t[i] = red[2 * i] + red[2 * i + 1];
#pragma unroll
  for (int w = kGnFinW / 4; w >= 1; w /= 2)
#pragma unroll
    for (int i = 0; i < w; ++i) t[i] = t[2 * i] + t[2 * i + 1];
  return t[0];
}

// A (sample, group) of up to kGnFinT * kGnFinE entries (every UNet GroupNorm:
// at most 256 chunks x 30 channels) is loaded once into registers, every
// load in flight together, and both passes run over the registers: one
// global round trip per launch.  Larger groups read global memory in both
// passes, in the same per-thread order.
constexpr int kGnFinE = 16;
// The statistics of channels [0, Ca) are read from sa ([N][chunks][Ca]), those
// of [Ca, C) from sb ([N][chunks][C - Ca]): a channel concatenation's two
// sources, each with its own producer's statistics.  One source: Ca = C.
__global__ void __launch_bounds__(kGnFinT)
gn_chan_finalize_kernel(const float2* __restrict__ sa, int Ca, const float2* __restrict__ sb, int HW,
                        int C, int G, int chunks, const f16* __restrict__ gamma,
                        const f16* __restrict__ beta, float eps, float2* __restrict__ ss) {
  __shared__ double red[kGnFinW];
  const int n = blockIdx.x / G, g = blockIdx.x % G;
  const int cpg = C / G;
  const int Cb = C - Ca;
  const int total = chunks * cpg;
  auto load = [&](int j) -> float2 {
    const int k = j / cpg;
    const int c = g * cpg + (j - k * cpg);
    const size_t row = (size_t)n * chunks + k;
    return c < Ca ? sa[row * Ca + c] : sb[row * Cb + (c - Ca)];
  };
  // pixels in entry j's chunk: 64, except in a partial last chunk
  const int last0 = (chunks - 1) * cpg;
  const double nlast = (double)(HW - (chunks - 1) * kGnChunk);
  auto count = [&](int j) { return j >= last0 ? nlast : (double)kGnChunk; };
  const double cnt = (double)HW * cpg;
  const int tid = threadIdx.x;
  double s1 = 0.0, m2 = 0.0, mean;
  if (total <= kGnFinT * kGnFinE) {
    float2 q[kGnFinE];
#pragma unroll
    for (int i = 0; i < kGnFinE; ++i) {
      const int j = tid + i * kGnFinT;
      q[i] = j < total ? load(j) : make_float2(0.0f, 0.0f);
    }
#pragma unroll
    for (int i = 0; i < kGnFinE; ++i) {
      const int j = tid + i * kGnFinT;
      if (j < total) s1 = fma(count(j), (double)q[i].x, s1);
    }
    s1 = gn_block_sum(s1, red);
    mean = s1 / cnt;
#pragma unroll
    for (int i = 0; i < kGnFinE; ++i) {
      const int j = tid + i * kGnFinT;
      if (j < total) {
        const double d = (double)q[i].x - mean;
        m2 += (double)q[i].y + count(j) * d * d;
      }
    }
  } else {
    for (int j = tid; j < total; j += kGnFinT) s1 = fma(count(j), (double)load(j).x, s1);
    s1 = gn_block_sum(s1, red);
    mean = s1 / cnt;
    for (int j = tid; j < total; j += kGnFinT) {
      const float2 q = load(j);
      const double d = (double)q.x - mean;
      m2 += (double)q.y + count(j) * d * d;
    }
  }
  m2 = gn_block_sum(m2, red);
  const double var = fmax(m2 / cnt, 0.0);
  const float rstd = (float)(1.0 / sqrt(var + (double)eps));
  for (int ci = tid; ci < cpg; ci += kGnFinT) {
    const int c = g * cpg + ci;
    const float gm = gamma ? (float)gamma[c] : 1.0f;
    const float bt = beta ? (float)beta[c] : 0.0f;
    const float scale = gm * rstd;
    ss[(size_t)n * C + c] = make_float2(scale, bt - (float)mean * scale);
  }
}

// Apply: one chunk of one sample's pixels per block, S * R threads.  A
// thread owns one 8-channel vector for the whole chunk: its source (concat
// half), scale and shift are fixed, so they are resolved once and stay in
// registers, and the loop keeps U pixel rows in flight per thread.
template <typename T, bool SILU, int U>
__global__ void gn_apply_kernel(const T* __restrict__ a, int Ca, int lda,
                                const T* __restrict__ b, int ldb, f16* __restrict__ out,
                                int ldo, int HW, int C, int S, int R, int chunk,
                                const float2* __restrict__ ss) {
  const int n = blockIdx.y;
  const int r = threadIdx.x / S, s = threadIdx.x - r * S;
  const int c = s * 8;
  const int p0 = blockIdx.x * chunk;
  const int p1 = min(HW, p0 + chunk);
  const T* src;
  int ld;
  if (c < Ca) {
    src = a + c;
    ld = lda;
  } else {
    src = b + (c - Ca);
    ld = ldb;
  }
  src += (size_t)n * HW * ld;
  f16* dst = out + (size_t)n * HW * ldo + c;
  const float4* ssv = reinterpret_cast<const float4*>(ss + (size_t)n * C + c);
  int p = p0 + r;
  if (p >= p1) return;
  // The first trip's rows, then the scale / shift, all issued before any is
  // waited for: rows past the chunk re-read its last row (never stored)
  // instead of skipping the load, since a load under a lane branch is copied,
  // and waited for, inside it; and a scale / shift loaded ahead of the loop
  // would be waited for at its head, before the rows are requested.
  float x[U][8];
#pragma unroll
  for (int u = 0; u < U; ++u) load8(src + (size_t)min(p + u * R, p1 - 1) * ld, x[u]);
  float sc[8], sh[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 q = ssv[i];
    sc[2 * i] = q.x;
    sh[2 * i] = q.y;
    sc[2 * i + 1] = q.z;
    sh[2 * i + 1] = q.w;
  }
  while (true) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (p + u * R < p1) {
        f16x8 y;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float t = x[u][i] * sc[i] + sh[i];
          if constexpr (SILU) t = silu_f(t);
          y[i] = (f16)t;
        }
        *reinterpret_cast<f16x8*>(dst + (size_t)(p + u * R) * ldo) = y;
      }
    }
    p += U * R;
    if (p >= p1) break;
#pragma unroll
    for (int u = 0; u < U; ++u) load8(src + (size_t)min(p + u * R, p1 - 1) * ld, x[u]);
  }
}

static int gn_chan_stats_launch(const f16* a, int C_a, int ld_a, const f16* b, int ld_b, int N,
                                int HW, int C, float2* stats, hipStream_t s) {
  const int S = C / 8, chunks = gn_chan_chunks(HW);
  DLM_LAUNCH("gn_chan_stats_kernel", gn_chan_stats_kernel, dim3((chunks * S + 255) / 256, N), dim3(256), 0, s, a,
             C_a, ld_a, b, ld_b, HW, C, S, chunks, stats);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int gn_chunk_stats(const void* x, int ld, int N, int HW, int C, float2* stats, hipStream_t s) {
  return gn_chan_stats_launch((const f16*)x, C, ld, (const f16*)x, ld, N, HW, C, stats, s);
}

// prestats: the per-channel chunk statistics are already at the start of ws
template <typename T>
static int group_norm_nhwc_t(const void* in_a, int C_a, int ld_a, const void* in_b, int ld_b,
                             const void* gamma, const void* beta, void* out, int ld_out, int N,
                             int HW, int C, int G, float eps, int silu, void* ws, hipStream_t s,
                             bool prestats = false, const float2* stats_a = nullptr,
                             const float2* stats_b = nullptr) {
  const GnPlan p = gn_plan(N, C, HW);
  float2* partial = (float2*)ws;
  float2* ss = gn_ss_of(ws, N, C, HW);
  const T* a = (const T*)in_a;
  const T* b = in_b ? (const T*)in_b : a;
  const long long total_vec = (long long)N * HW * (C / 8);
  if (total_vec >= (1LL << 31) || (long long)N * HW * std::max(ld_a, ld_out) >= (1LL << 31))
    return fail(DLM_ERR_UNSUPPORTED, "group_norm: tensor too large for 32-bit indexing");
  if (std::is_same<T, f16>::value && HW <= kGnChanMaxHW) {
    if (!prestats) {
      const int st = gn_chan_stats_launch((const f16*)a, C_a, ld_a, (const f16*)b, ld_b, N, HW, C, partial, s);
      if (st != DLM_OK) return st;
    }
    // producer statistics of two sources (stats_b), or of one source, or the
    // statistics pass's, in the workspace
    const float2* sa = stats_b ? stats_a : partial;
    const int Ca = stats_b ? C_a : C;
    DLM_LAUNCH("gn_chan_finalize_kernel", gn_chan_finalize_kernel, dim3(N * G), dim3(kGnFinT), 0, s, sa, Ca, stats_b,
               HW, C, G, gn_chan_chunks(HW), (const f16*)gamma, (const f16*)beta, eps, ss);
    DLM_LAUNCH_CHECK();
  } else {
    if (prestats) return fail(DLM_ERR_UNSUPPORTED, "group_norm: chunk statistics need fp16 input of <= 16384 pixels");
    const size_t red_bytes = (size_t)p.R * C * sizeof(float2);
    if (red_bytes > 160 * 1024)
      return fail(DLM_ERR_UNSUPPORTED, "group_norm: channel count too large for one block");
    DLM_LAUNCH("gn_partial_kernel", gn_partial_kernel<T>, dim3(p.chunks, N), dim3(p.threads), red_bytes, s, a, C_a,
               ld_a, b, ld_b, HW, C, G, p.chunk, p.chunks, p.S, p.R, partial);
    DLM_LAUNCH_CHECK();
    DLM_LAUNCH("gn_finalize_kernel", gn_finalize_kernel, dim3(N * G), dim3(64), 0, s, partial, HW, C, G, p.chunk,
               p.chunks, (const f16*)gamma, (const f16*)beta, eps, ss);
    DLM_LAUNCH_CHECK();
  }
  // the entry's label: the kernels of the whole GroupNorm
  const char* label = !(std::is_same<T, f16>::value && HW <= kGnChanMaxHW)
                          ? "gn_partial_kernel+gn_finalize_kernel+gn_apply_kernel"
                          : (prestats ? "gn_chan_finalize_kernel+gn_apply_kernel"
                                      : "gn_chan_stats_kernel+gn_chan_finalize_kernel+gn_apply_kernel");
  // Apply blocks: the statistics pass's (four rows in flight per thread)
  // where that pass ran; after chunk statistics, whose 64-pixel chunks do
  // not constrain it, two rows per thread and twice the blocks (GN + SiLU from
  // producer statistics: 2x128^2x320 14.8 -> 13.7 us, 2x64^2x1920 18.1 ->
  // 17.2 us; 2x64^2x640 10.0 -> 10.2 us).
  if (std::is_same<T, f16>::value && HW <= kGnChanMaxHW) {
    const int chunk = std::max(p.R * 2, (HW + 1023) / 1024), chunks = (HW + chunk - 1) / chunk;
    if (silu)
      DLM_LAUNCH(label, (gn_apply_kernel<T, true, 2>), dim3(chunks, N), dim3(p.threads), 0, s, a, C_a, ld_a, b,
                 ld_b, (f16*)out, ld_out, HW, C, p.S, p.R, chunk, ss);
    else
      DLM_LAUNCH(label, (gn_apply_kernel<T, false, 2>), dim3(chunks, N), dim3(p.threads), 0, s, a, C_a, ld_a, b,
                 ld_b, (f16*)out, ld_out, HW, C, p.S, p.R, chunk, ss);
  } else if (silu) {
    DLM_LAUNCH(label, (gn_apply_kernel<T, true, 4>), dim3(p.chunks, N), dim3(p.threads), 0, s, a, C_a, ld_a, b,
               ld_b, (f16*)out, ld_out, HW, C, p.S, p.R, p.chunk, ss);
  } else {
    DLM_LAUNCH(label, (gn_apply_kernel<T, false, 4>), dim3(p.chunks, N), dim3(p.threads), 0, s, a, C_a, ld_a, b,
               ld_b, (f16*)out, ld_out, HW, C, p.S, p.R, p.chunk, ss);
  }
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int group_norm_nhwc(const void* in_a, int C_a, int ld_a, const void* in_b, int ld_b,
                    const void* gamma, const void* beta, void* out, int ld_out, int N, int HW,
                    int C, int G, float eps, int silu, void* ws, hipStream_t s, bool in_f32 = false,
                    bool prestats = false, const float2* stats_a = nullptr, const float2* stats_b = nullptr) {
  return in_f32 ? group_norm_nhwc_t<float>(in_a, C_a, ld_a, in_b, ld_b, gamma, beta, out, ld_out, N,
                                           HW, C, G, eps, silu, ws, s, prestats)
                : group_norm_nhwc_t<f16>(in_a, C_a, ld_a, in_b, ld_b, gamma, beta, out, ld_out, N,
                                         HW, C, G, eps, silu, ws, s, prestats, stats_a, stats_b);
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
  // Rows over 1024 channels request gamma / beta together with the row, so
  // the affine operands arrive while the two reductions run (2048 x 1280:
  // 6.2 -> 5.5 us); narrower rows load them after the statistics (8192 x 640
  // measured 5% slower with the early loads).
  constexpr bool kEarly = VPL >= 3;
  // Every load of the row is issued before any is waited for: lanes past
  // the row's end re-read its last vector (never used) instead of skipping
  // the load, since a load under a lane branch has its result copied, and
  // waited for, inside the branch, one memory round trip per vector.
  f16x8 xh[VPL], gh[VPL], bh[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int s = min(lane + 64 * j, S - 1);
    xh[j] = *reinterpret_cast<const f16x8*>(x + s * 8);
    if (kEarly && gamma) gh[j] = *reinterpret_cast<const f16x8*>(gamma + s * 8);
    if (kEarly && beta) bh[j] = *reinterpret_cast<const f16x8*>(beta + s * 8);
  }
  float v[VPL][8];
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const bool in = lane + 64 * j < S;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[j][i] = in ? (float)xh[j][i] : 0.0f;
      sum += v[j][i];
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
  if constexpr (!kEarly) {
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int s = min(lane + 64 * j, S - 1);
      if (gamma) gh[j] = *reinterpret_cast<const f16x8*>(gamma + s * 8);
      if (beta) bh[j] = *reinterpret_cast<const f16x8*>(beta + s * 8);
    }
  }
  const float rstd = rsqrtf(wave_sum(sq) / (float)C + eps);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int s = lane + 64 * j;
    if (s < S) {
      f16x8 y;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float gi = gamma ? (float)gh[j][i] : 1.0f;
        const float bi = beta ? (float)bh[j][i] : 0.0f;
        y[i] = (f16)((v[j][i] - mean) * rstd * gi + bi);
      }
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
    DLM_LAUNCH("layer_norm_kernel<1>", layer_norm_kernel<1>, grid, block, 0, s, x, g, b, y, rows, C, eps);
  else if (vec && C <= 64 * 8 * 2)
    DLM_LAUNCH("layer_norm_kernel<2>", layer_norm_kernel<2>, grid, block, 0, s, x, g, b, y, rows, C, eps);
  else if (vec && C <= 64 * 8 * 3)
    DLM_LAUNCH("layer_norm_kernel<3>", layer_norm_kernel<3>, grid, block, 0, s, x, g, b, y, rows, C, eps);
  else if (vec && C <= 64 * 8 * 8)
    DLM_LAUNCH("layer_norm_kernel<8>", layer_norm_kernel<8>, grid, block, 0, s, x, g, b, y, rows, C, eps);
  else
    DLM_LAUNCH("layer_norm_scalar_kernel", layer_norm_scalar_kernel, grid, block, 0, s, x, g, b, y, rows, C, eps);
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

int dlm_group_norm_nhwc_prestats_fp16(const void* in, int ld_in, const void* gamma, const void* beta,
                                      void* out, int ld_out, int N, int HW, int C, int num_groups,
                                      float eps, int fuse_silu, void* workspace, void* stream) {
  if (N <= 0 || HW <= 0 || C <= 0 || num_groups <= 0) return DLM_OK;
  DLM_REQUIRE(in && out && workspace, "NULL pointer");
  DLM_REQUIRE(C % num_groups == 0, "C must be divisible by num_groups");
  DLM_REQUIRE(C % 8 == 0, "C must be a multiple of 8");
  DLM_REQUIRE(HW <= kGnChanMaxHW, "chunk statistics cover at most 16384 pixels per sample");
  DLM_REQUIRE(ld_in % 8 == 0 && ld_in >= C && ld_out % 8 == 0 && ld_out >= C, "bad row strides");
  DLM_REQUIRE(dlm_aligned16(in) && dlm_aligned16(out) && dlm_aligned16(workspace),
              "buffers must be 16-byte aligned");
  return group_norm_nhwc(in, C, ld_in, nullptr, 0, gamma, beta, out, ld_out, N, HW, C, num_groups, eps,
                         fuse_silu, workspace, (hipStream_t)stream, false, true);
}

int dlm_group_norm_nhwc_prestats2_fp16(const void* in_a, int C_a, int ld_a, const void* in_b, int ld_b,
                                       const void* stats_a, const void* stats_b, const void* gamma,
                                       const void* beta, void* out, int ld_out, int N, int HW, int C,
                                       int num_groups, float eps, int fuse_silu, void* workspace,
                                       void* stream) {
  if (N <= 0 || HW <= 0 || C <= 0 || num_groups <= 0) return DLM_OK;
  DLM_REQUIRE(in_a && in_b && stats_a && stats_b && out && workspace, "NULL pointer");
  DLM_REQUIRE(C % num_groups == 0, "C must be divisible by num_groups");
  DLM_REQUIRE(C % 8 == 0 && C_a % 8 == 0 && C_a > 0 && C_a < C, "C and C_a must be multiples of 8, 0 < C_a < C");
  DLM_REQUIRE(HW <= kGnChanMaxHW, "chunk statistics cover at most 16384 pixels per sample");
  DLM_REQUIRE(ld_a % 8 == 0 && ld_a >= C_a && ld_b % 8 == 0 && ld_b >= C - C_a && ld_out % 8 == 0 &&
                  ld_out >= C,
              "bad row strides");
  DLM_REQUIRE(dlm_aligned16(in_a) && dlm_aligned16(in_b) && dlm_aligned16(out) && dlm_aligned16(workspace) &&
                  ((uintptr_t)stats_a & 7) == 0 && ((uintptr_t)stats_b & 7) == 0,
              "buffers must be 16-byte aligned (statistics 8-byte)");
  return group_norm_nhwc(in_a, C_a, ld_a, in_b, ld_b, gamma, beta, out, ld_out, N, HW, C, num_groups, eps,
                         fuse_silu, workspace, (hipStream_t)stream, false, true, (const float2*)stats_a,
                         (const float2*)stats_b);
}

int dlm_group_norm_chunk_stats_fp16(const void* in, int ld_in, int N, int HW, int C, void* workspace,
                                    void* stream) {
  if (N <= 0 || HW <= 0 || C <= 0) return DLM_OK;
  DLM_REQUIRE(in && workspace, "NULL pointer");
  DLM_REQUIRE(C % 8 == 0 && ld_in % 8 == 0 && ld_in >= C, "C and ld_in must be multiples of 8, ld_in >= C");
  DLM_REQUIRE(HW <= kGnChanMaxHW, "chunk statistics cover at most 16384 pixels per sample");
  DLM_REQUIRE(dlm_aligned16(in) && dlm_aligned16(workspace), "buffers must be 16-byte aligned");
  return gn_chunk_stats(in, ld_in, N, HW, C, (float2*)workspace, (hipStream_t)stream);
}

int dlm_group_norm_nhwc_f32in(const float* in, int ld_in, const void* gamma, const void* beta,
                              void* out, int ld_out, int N, int HW, int C, int num_groups,
                              float eps, int fuse_silu, void* workspace, void* stream) {
  if (N <= 0 || HW <= 0 || C <= 0 || num_groups <= 0) return DLM_OK;
  DLM_REQUIRE(in && out && workspace, "NULL pointer");
  DLM_REQUIRE(C % num_groups == 0, "C must be divisible by num_groups");
  DLM_REQUIRE(C % 8 == 0, "C must be a multiple of 8");
  DLM_REQUIRE(ld_in % 8 == 0 && ld_in >= C && ld_out % 8 == 0 && ld_out >= C, "bad row strides");
  DLM_REQUIRE(dlm_aligned16(in) && dlm_aligned16(out) && dlm_aligned16(workspace),
              "buffers must be 16-byte aligned");
  return group_norm_nhwc(in, C, ld_in, nullptr, 0, gamma, beta, out, ld_out, N, HW, C, num_groups,
                         eps, fuse_silu, workspace, (hipStream_t)stream, true);
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
  f16* x = (f16*)scratch_slot((size_t)N * HW * Cp * 2, 4, s, &st);
  if (!x) return st;
  void* ws = scratch_slot(gn_workspace_bytes(N, Cp, HW), 5, s, &st);
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
