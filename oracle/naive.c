/* Plain-C restatement of the reference's own CPU test references for the
 * SDXL UNet dense-contraction path.  TEST INFRASTRUCTURE ONLY: built into
 * oracle/libnaive.so and called from tests/ (through oracle/naive.py) as an
 * independent second oracle beside the torch one in ref_ops.py.  Nothing in
 * the product links or loads it.
 *
 * All tensors are float32, row-major, in the reference's layouts (NCHW for
 * conv / GroupNorm, [B,H,S,Dh] for attention).  Loop order and accumulation
 * type follow the cited reference functions (fp32 accumulation, one-pass
 * sum / sum-of-squares normalisation statistics with the variance clamped at
 * zero), so these functions reproduce the reference's CPU numerics, not
 * torch's.
 */
#include <math.h>
#include <stdlib.h>

/* Output extent of a convolution (src/kernels/conv2d.cu:275-278). */
static int out_dim(int in, int pad, int dil, int k, int stride) {
  return (in + 2 * pad - dil * (k - 1) - 1) / stride + 1;
}

/* Direct convolution, fp32 accumulate, bias optional
 * (src/tests/test_conv2d.cu:134-196). */
void naive_conv2d(const float* in, const float* w, const float* bias, float* out, int N, int Cin,
                  int H, int W, int Cout, int KH, int KW, int sh, int sw, int ph, int pw, int dh,
                  int dw) {
  const int Ho = out_dim(H, ph, dh, KH, sh), Wo = out_dim(W, pw, dw, KW, sw);
  for (int n = 0; n < N; ++n)
    for (int co = 0; co < Cout; ++co)
      for (int ho = 0; ho < Ho; ++ho)
        for (int wo = 0; wo < Wo; ++wo) {
          float acc = 0.0f;
          for (int ci = 0; ci < Cin; ++ci)
            for (int kh = 0; kh < KH; ++kh) {
              const int hi = ho * sh - ph + kh * dh;
              if (hi < 0 || hi >= H) continue;
              for (int kw = 0; kw < KW; ++kw) {
                const int wi = wo * sw - pw + kw * dw;
                if (wi < 0 || wi >= W) continue;
                acc += in[(((long)n * Cin + ci) * H + hi) * W + wi] *
                       w[(((long)co * Cin + ci) * KH + kh) * KW + kw];
              }
            }
          if (bias) acc += bias[co];
          out[(((long)n * Cout + co) * Ho + ho) * Wo + wo] = acc;
        }
}

/* C = alpha * A op(B) + beta * C_in, fp32 accumulate, A [M,K] row-major,
 * B [K,N] or (transB) [N,K] (src/tests/test_gemm.cu:54-80). */
void naive_gemm(const float* A, const float* B, const float* C_in, float* out, int M, int N, int K,
                float alpha, float beta, int transB) {
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) {
      float acc = 0.0f;
      for (int k = 0; k < K; ++k)
        acc += A[(long)i * K + k] * (transB ? B[(long)j * K + k] : B[(long)k * N + j]);
      float v = alpha * acc;
      if (C_in && beta != 0.0f) v += beta * C_in[(long)i * N + j];
      out[(long)i * N + j] = v;
    }
}

/* GroupNorm over NCHW, one-pass fp32 statistics, var clamped at 0
 * (src/tests/test_groupnorm.cu:103-148; kernel formula
 * src/kernels/groupnorm.cu:91-148).  fuse_silu applies x*sigmoid(x) after the
 * affine step (src/kernels/groupnorm.cu:467, launch_group_norm_silu). */
void naive_group_norm(const float* in, const float* gamma, const float* beta, float* out, int N,
                      int C, int H, int W, int G, float eps, int fuse_silu) {
  const int HW = H * W, cpg = C / G, K = cpg * HW;
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < G; ++g) {
      const long base = ((long)n * C + (long)g * cpg) * HW;
      float sum = 0.0f, sq = 0.0f;
      for (int i = 0; i < K; ++i) {
        sum += in[base + i];
        sq += in[base + i] * in[base + i];
      }
      const float mean = sum / (float)K;
      float var = sq / (float)K - mean * mean;
      if (var < 0.0f) var = 0.0f;
      const float inv_std = 1.0f / sqrtf(var + eps);
      for (int i = 0; i < K; ++i) {
        const int c = g * cpg + i / HW;
        float y = (in[base + i] - mean) * inv_std * gamma[c] + beta[c];
        if (fuse_silu) y = y / (1.0f + expf(-y));
        out[base + i] = y;
      }
    }
}

/* LayerNorm over the last dim, one-pass fp32 statistics, affine optional
 * (src/tests/test_layernorm.cu:92-130). */
void naive_layer_norm(const float* in, const float* gamma, const float* beta, float* out, int rows,
                      int C, float eps) {
  for (int r = 0; r < rows; ++r) {
    const long base = (long)r * C;
    float sum = 0.0f, sq = 0.0f;
    for (int c = 0; c < C; ++c) {
      sum += in[base + c];
      sq += in[base + c] * in[base + c];
    }
    const float mean = sum / (float)C;
    float var = sq / (float)C - mean * mean;
    if (var < 0.0f) var = 0.0f;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int c = 0; c < C; ++c) {
      const float gm = gamma ? gamma[c] : 1.0f, bt = beta ? beta[c] : 0.0f;
      out[base + c] = (in[base + c] - mean) * inv_std * gm + bt;
    }
  }
}

/* O = softmax(scale Q K^T) V with a two-pass max-subtracted softmax,
 * Q/O [B,H,Sq,Dh], K/V [B,H,Sk,Dh] (src/tests/test_attention.cu:99-161). */
void naive_attention(const float* q, const float* k, const float* v, float* out, int B, int H,
                     int Sq, int Sk, int Dh, float scale) {
  float* p = (float*)malloc(sizeof(float) * (size_t)(Sk > 0 ? Sk : 1));
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const long qh = ((long)b * H + h) * Sq * Dh, kh = ((long)b * H + h) * Sk * Dh;
      for (int i = 0; i < Sq; ++i) {
        float mx = -INFINITY;
        for (int j = 0; j < Sk; ++j) {
          float dot = 0.0f;
          for (int d = 0; d < Dh; ++d) dot += q[qh + (long)i * Dh + d] * k[kh + (long)j * Dh + d];
          p[j] = scale * dot;
          if (p[j] > mx) mx = p[j];
        }
        float sum = 0.0f;
        for (int j = 0; j < Sk; ++j) {
          p[j] = expf(p[j] - mx);
          sum += p[j];
        }
        const float inv = 1.0f / sum;
        for (int d = 0; d < Dh; ++d) {
          float acc = 0.0f;
          for (int j = 0; j < Sk; ++j) acc += p[j] * inv * v[kh + (long)j * Dh + d];
          out[qh + (long)i * Dh + d] = acc;
        }
      }
    }
  free(p);
}

/* 0.5 x (1 + erf(x / sqrt 2)) (src/tests/test_activation.cu:122-125). */
float naive_gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678f)); }

/* x * sigmoid(x) (src/tests/test_activation.cu:117-120). */
float naive_silu(float x) { return x / (1.0f + expf(-x)); }

/* [tokens, 2d] -> [tokens, d] = x1 * gelu_erf(x2), value = first half
 * (src/tests/test_geglu.cu:56-72). */
void naive_geglu(const float* in, float* out, int tokens, int d) {
  for (int t = 0; t < tokens; ++t)
    for (int c = 0; c < d; ++c)
      out[(long)t * d + c] = in[(long)t * 2 * d + c] * naive_gelu_erf(in[(long)t * 2 * d + d + c]);
}

/* Sinusoidal embedding, cos first (src/tests/test_timeembed.cu:32-46). */
void naive_time_embedding(float t, int dim, float max_period, float* out) {
  const int half = dim / 2;
  const float lmp = logf(max_period);
  for (int i = 0; i < dim; ++i) out[i] = 0.0f;
  for (int i = 0; i < half; ++i) {
    const float arg = t * expf(-lmp * (float)i / (float)half);
    out[i] = cosf(arg);
    out[half + i] = sinf(arg);
  }
}

/* Euler discrete schedule: scaled_linear betas (sqrt-space linear between
 * beta_start and beta_end), sigma = sqrt((1 - acp) / acp), "leading" spacing
 * with step_ratio = T / steps and offset 1, timesteps descending, sigma by
 * linear interpolation of the training sigmas, final sigma 0
 * (src/infer/scheduler.hpp:45-143).  sigmas has steps + 1 entries. */
int naive_euler_schedule(int steps, int T, double beta_start, double beta_end, float* sigmas,
                         float* timesteps) {
  if (steps <= 0 || T <= 0) return 1;
  double* train = (double*)malloc(sizeof(double) * (size_t)T);
  const double s0 = sqrt(beta_start), s1 = sqrt(beta_end);
  double acp = 1.0;
  for (int i = 0; i < T; ++i) {
    const double f = T == 1 ? 0.0 : (double)i / (T - 1);
    const double sb = s0 + (s1 - s0) * f;
    acp *= 1.0 - sb * sb;
    train[i] = sqrt((1.0 - acp) / acp);
  }
  const int ratio = T / steps;
  for (int i = 0; i < steps; ++i) {
    const double t = round((double)(steps - 1 - i) * ratio) + 1.0;
    double s;
    if (t <= 0.0)
      s = train[0];
    else if (t >= (double)(T - 1))
      s = train[T - 1];
    else {
      const int lo = (int)floor(t);
      s = train[lo] + (train[lo + 1] - train[lo]) * (t - lo);
    }
    timesteps[i] = (float)t;
    sigmas[i] = (float)s;
  }
  sigmas[steps] = 0.0f;
  free(train);
  return 0;
}

/* Uniform-window SSIM over C planes of HxW (src/tests/test_unet.cu:161-201):
 * L = joint value range, C1 = (0.01 L)^2, C2 = (0.03 L)^2, 7x7 windows whose
 * centres step by 3, biased window variances, mean over windows. */
double naive_ssim_uniform(const float* a, const float* b, int C, int H, int W) {
  const long n = (long)C * H * W;
  float lo = a[0], hi = a[0];
  for (long i = 0; i < n; ++i) {
    if (a[i] < lo) lo = a[i];
    if (a[i] > hi) hi = a[i];
    if (b[i] < lo) lo = b[i];
    if (b[i] > hi) hi = b[i];
  }
  const double L = (double)(hi - lo), C1 = (0.01 * L) * (0.01 * L), C2 = (0.03 * L) * (0.03 * L);
  const int half = 3;
  const double inv = 1.0 / 49.0;
  double total = 0.0;
  long cnt = 0;
  for (int c = 0; c < C; ++c)
    for (int y = half; y < H - half; y += half)
      for (int x = half; x < W - half; x += half) {
        double sa = 0, sb = 0, saa = 0, sbb = 0, sab = 0;
        for (int dy = -half; dy <= half; ++dy)
          for (int dx = -half; dx <= half; ++dx) {
            const long i = ((long)c * H + y + dy) * W + x + dx;
            const double va = a[i], vb = b[i];
            sa += va;
            sb += vb;
            saa += va * va;
            sbb += vb * vb;
            sab += va * vb;
          }
        const double ma = sa * inv, mb = sb * inv;
        const double va = saa * inv - ma * ma, vb = sbb * inv - mb * mb, cov = sab * inv - ma * mb;
        total += ((2 * ma * mb + C1) * (2 * cov + C2)) / ((ma * ma + mb * mb + C1) * (va + vb + C2));
        ++cnt;
      }
  return cnt ? total / (double)cnt : 0.0;
}
