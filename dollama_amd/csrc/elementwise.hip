// Small kernels around the dense path: activations, bias / residual adds,
// nearest-2x upsampling (reference layout), sinusoidal embeddings, the skinny
// linears of the time / add embedding MLPs, and the fused CFG + Euler step.
//
// Reference behaviour followed:
//   silu / gelu_erf            src/kernels/activation.cu:25-69
//   add / upsample_nearest2x   src/kernels/elementwise.cu:24-73
//   bias adds and conv bias epilogues  src/kernels/bias_add.cu:26-159
//     (here the fp32 sum is rounded once, not twice)
//   geglu                      src/kernels/geglu.cu:26-48 (value = first half)
//   timestep_embedding         src/kernels/timeembed.cu:30-49 (cos first)
//   add-embedding input        src/infer/unet.cu:995-1024 (text_embeds first,
//                              then 6 x sinusoid_256(time_ids))
//   CFG combine + Euler step   src/infer/diffusion.cu:968-973,
//                              src/infer/scheduler.hpp:112-143
#include <algorithm>

#include "common.hpp"

namespace dlm {

__global__ void silu_kernel(const f16* in, f16* out, long long n) {
  GRID_STRIDE(i, n) out[i] = (f16)silu_f((float)in[i]);
}

__global__ void gelu_kernel(const f16* in, f16* out, long long n) {
  GRID_STRIDE(i, n) out[i] = (f16)gelu_erf_f((float)in[i]);
}

// GELU, tanh approximation: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
// in fp32 (reference gelu_tanh_fp16, src/kernels/activation.cu:54-70)
__global__ void gelu_tanh_kernel(const f16* in, f16* out, long long n) {
  GRID_STRIDE(i, n) {
    const float x = (float)in[i];
    const float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    out[i] = (f16)(0.5f * x * (1.0f + tanhf(inner)));
  }
}

__global__ void add_kernel(const f16* a, const f16* b, f16* out, long long n) {
  GRID_STRIDE(i, n) out[i] = (f16)((float)a[i] + (float)b[i]);
}

__global__ void upsample2x_nchw_kernel(const f16* in, f16* out, int H, int W, long long n) {
  const int W2 = 2 * W, H2 = 2 * H;
  GRID_STRIDE(i, n) {
    const int x = (int)(i % W2);
    const long long r = i / W2;
    const int y = (int)(r % H2);
    const long long nc = r / H2;
    out[i] = in[(nc * H + (y >> 1)) * W + (x >> 1)];
  }
}

__global__ void bias_rowvec_kernel(const f16* in, const f16* bias, f16* out, int C, long long n) {
  GRID_STRIDE(i, n) out[i] = (f16)((float)in[i] + (float)bias[i % C]);
}

// out[n][c][p] = in + bias[c] (+ tproj[n][c]) (+ residual)
__global__ void bias_channel_kernel(const f16* in, const f16* bias, const f16* tproj,
                                    const f16* residual, f16* out, int C, int HW, long long n) {
  GRID_STRIDE(i, n) {
    const long long nc = i / HW;
    const int c = (int)(nc % C);
    float v = (float)in[i];
    if (bias) v += (float)bias[c];
    if (tproj) v += (float)tproj[nc];
    if (residual) v += (float)residual[i];
    out[i] = (f16)v;
  }
}

__global__ void geglu_kernel(const f16* in, f16* out, int d, long long n) {
  GRID_STRIDE(i, n) {
    const long long t = i / d;
    const int j = (int)(i - t * d);
    const float x = (float)in[t * 2 * d + j];
    const float gte = (float)in[t * 2 * d + d + j];
    out[i] = (f16)(x * gelu_erf_f(gte));
  }
}

// Sinusoid of one scalar: out[j] = cos(t*f_j), out[half+j] = sin(t*f_j),
// f_j = exp(-ln(max_period) * j / half) evaluated in fp32.
__device__ __forceinline__ void sinusoid_one(f16* out, float t, int dim, float log_max_period,
                                             int j) {
  const int half = dim / 2;
  if (j < half) {
    const float expo = -log_max_period * (float)j / (float)half;
    const float arg = t * expf(expo);
    out[j] = (f16)cosf(arg);
    out[half + j] = (f16)sinf(arg);
  }
}

__global__ void timestep_embedding_kernel(f16* out, float t, int dim, float log_mp) {
  sinusoid_one(out, t, dim, log_mp, blockIdx.x * blockDim.x + threadIdx.x);
}

// One block per batch row: t_emb[b, 0:t_dim] = sinusoid(t_b), and
// add_in[b] = text[b, 0:text_dim] ++ sinusoid_{id_dim}(ids[b*stride + i]), i < 6.
__global__ void sdxl_embed_kernel(const float* timesteps, const f16* text, int text_dim,
                                  const f16* ids, int ids_bstride, int id_dim, f16* t_emb,
                                  int t_dim, f16* add_in) {
  const int b = blockIdx.x;
  const float log_mp = 9.210340371976184f;  // ln(10000)
  const int tid = threadIdx.x;
  for (int j = tid; j < t_dim / 2; j += blockDim.x)
    sinusoid_one(t_emb + (size_t)b * t_dim, timesteps[b], t_dim, log_mp, j);
  const int add_dim = text_dim + 6 * id_dim;
  f16* a = add_in + (size_t)b * add_dim;
  for (int i = tid; i < text_dim; i += blockDim.x) a[i] = text[(size_t)b * text_dim + i];
  const int hd = id_dim / 2;
  for (int i = tid; i < 6 * hd; i += blockDim.x) {
    const int k = i / hd, j = i % hd;
    sinusoid_one(a + text_dim + k * id_dim, (float)ids[b * ids_bstride + k], id_dim, log_mp, j);
  }
}

// Skinny linear (M <= MB <= 16): one wave per output column, W row streamed
// once.  The MB rows' loads are unconditional (rows past M re-read row
// M - 1, never stored), so each k-step issues all its loads before waiting:
// a load under a lane branch is copied, and waited for, inside it.
template <int MB>
__global__ void __launch_bounds__(256)
linear_small_kernel(const f16* __restrict__ X, int ldx, const f16* __restrict__ W,
                    const f16* __restrict__ bias, f16* __restrict__ Y, int ldy, int M, int N,
                    int K, int silu_in, int act, int accumulate) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  float acc[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) acc[m] = 0.0f;
  const f16* w = W + (size_t)n * K;
  for (int k = lane * 8; k < K; k += 512) {
    const f16x8 wv = *reinterpret_cast<const f16x8*>(w + k);
    f16x8 xv[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) xv[m] = *reinterpret_cast<const f16x8*>(X + (size_t)min(m, M - 1) * ldx + k);
#pragma unroll
    for (int m = 0; m < MB; ++m) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float xf = (float)xv[m][i];
        if (silu_in) xf = silu_f(xf);
        acc[m] += xf * (float)wv[i];
      }
    }
  }
  const float bn = bias ? (float)bias[n] : 0.0f;
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    if (m < M) {
      float v = wave_sum(acc[m]) + bn;
      if (act == DLM_ACT_SILU) v = silu_f(v);
      if (lane == 0) {
        f16* dst = Y + (size_t)m * ldy + n;
        if (accumulate) v += (float)*dst;
        *dst = (f16)v;
      }
    }
  }
}

__global__ void euler_cfg_kernel(float* latent, const f16* noise, f16* model_in, int n, float g,
                                 float dt, float in_scale) {
  GRID_STRIDE(i, n) {
    const float c = (float)noise[i];
    const float u = (float)noise[n + i];
    const float eps = u + g * (c - u);
    const float x = latent[i] + eps * dt;
    latent[i] = x;
    const f16 mi = (f16)(x * in_scale);
    model_in[i] = mi;
    model_in[n + i] = mi;
  }
}

// Euler step without guidance (one noise prediction, the reference's
// generate() path, src/infer/diffusion.cu:650-660 + scheduler.hpp step).
__global__ void euler_kernel(float* latent, const f16* noise, f16* model_in, int n, float dt,
                             float in_scale) {
  GRID_STRIDE(i, n) {
    const float x = latent[i] + (float)noise[i] * dt;
    latent[i] = x;
    model_in[i] = (f16)(x * in_scale);
  }
}

__global__ void scale_latent_kernel(const float* latent, f16* model_in, int n, float scale,
                                    int copies) {
  GRID_STRIDE(i, n) {
    const f16 v = (f16)(latent[i] * scale);
    for (int c = 0; c < copies; ++c) model_in[(size_t)c * n + i] = v;
  }
}

// out = fp16(in * scale); eight elements per vector step, scalar tail.
__global__ void cast_f32_f16_kernel(const float* __restrict__ in, f16* __restrict__ out,
                                    long long n, float scale) {
  const long long n8 = n >> 3;
  GRID_STRIDE(i, n8) {
    const float4 a = reinterpret_cast<const float4*>(in)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(in)[2 * i + 1];
    const f16x8 o = {(f16)(a.x * scale), (f16)(a.y * scale), (f16)(a.z * scale), (f16)(a.w * scale),
                     (f16)(b.x * scale), (f16)(b.y * scale), (f16)(b.z * scale), (f16)(b.w * scale)};
    reinterpret_cast<f16x8*>(out)[i] = o;
  }
  GRID_STRIDE(j, n - (n8 << 3)) out[(n8 << 3) + j] = (f16)(in[(n8 << 3) + j] * scale);
}

__global__ void scale_f16_kernel(f16* x, long long n, float scale) {
  GRID_STRIDE(i, n) x[i] = (f16)((float)x[i] * scale);
}

// VAE input: fp16(latent / scaling_factor) (reference src/infer/diffusion.cu:980-984).
__global__ void latent_to_vae_kernel(const float* latent, f16* out, long long n, float sf) {
  GRID_STRIDE(i, n) out[i] = (f16)(latent[i] / sf);
}

// Decoded image [N, 3, H, W] fp16 in [-1, 1] -> RGB8 [N, H, W, 3]:
// q = int(clamp(v * 0.5 + 0.5, 0, 1) * 255 + 0.5) (reference image_f16_to_rgb_u8,
// src/infer/diffusion.cu:146-165); a NaN maps to 0.
__global__ void image_to_rgb8_kernel(const f16* img, uint8_t* rgb, long long HW, long long n) {
  GRID_STRIDE(i, n) {  // i = (b * HW + p) * 3 + c
    const long long c = i % 3, bp = i / 3;
    const long long b = bp / HW, p = bp - b * HW;
    const float v = (float)img[(b * 3 + c) * HW + p];
    // separately rounded multiply and add, as the reference's host code
    // computes them (no fused multiply-add)
    float n01 = __fadd_rn(__fmul_rn(v, 0.5f), 0.5f);
    n01 = n01 < 0.0f ? 0.0f : n01;
    n01 = n01 > 1.0f ? 1.0f : n01;
    const int q = n01 == n01 ? (int)__fadd_rn(__fmul_rn(n01, 255.0f), 0.5f) : 0;
    rgb[i] = (uint8_t)(q < 0 ? 0 : (q > 255 ? 255 : q));
  }
}

}  // namespace dlm

using namespace dlm;

#define EW_PRE(n)                     \
  if ((n) <= 0) return DLM_OK;        \
  hipStream_t s_ = (hipStream_t)stream

extern "C" {

int dlm_silu_fp16(const void* in, void* out, int n, void* stream) {
  EW_PRE(n);
  DLM_REQUIRE(in && out, "NULL pointer");
  DLM_LAUNCH("silu_kernel", silu_kernel, dim3(grid_for(n)), dim3(256), 0, s_, (const f16*)in, (f16*)out,
                     (long long)n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_gelu_fp16(const void* in, void* out, int n, void* stream) {
  EW_PRE(n);
  DLM_REQUIRE(in && out, "NULL pointer");
  DLM_LAUNCH("gelu_kernel", gelu_kernel, dim3(grid_for(n)), dim3(256), 0, s_, (const f16*)in, (f16*)out,
                     (long long)n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_gelu_tanh_fp16(const void* in, void* out, int n, void* stream) {
  EW_PRE(n);
  DLM_REQUIRE(in && out, "NULL pointer");
  DLM_LAUNCH("gelu_tanh_kernel", gelu_tanh_kernel, dim3(grid_for(n)), dim3(256), 0, s_, (const f16*)in,
             (f16*)out, (long long)n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_add_fp16(const void* a, const void* b, void* out, int n, void* stream) {
  EW_PRE(n);
  DLM_REQUIRE(a && b && out, "NULL pointer");
  DLM_LAUNCH("add_kernel", add_kernel, dim3(grid_for(n)), dim3(256), 0, s_, (const f16*)a, (const f16*)b,
                     (f16*)out, (long long)n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_upsample_nearest2x_fp16(const void* in, void* out, int N, int C, int H, int W,
                                void* stream) {
  if (N <= 0 || C <= 0 || H <= 0 || W <= 0) return DLM_OK;
  DLM_REQUIRE(in && out, "NULL pointer");
  const long long n = (long long)N * C * 4 * H * W;
  DLM_LAUNCH("upsample2x_nchw_kernel", upsample2x_nchw_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)in, (f16*)out, H, W, n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_bias_add_rowvec_fp16(const void* in, const void* bias, void* out, int tokens, int C,
                             void* stream) {
  if (tokens <= 0 || C <= 0) return DLM_OK;
  DLM_REQUIRE(in && bias && out, "NULL pointer");
  const long long n = (long long)tokens * C;
  DLM_LAUNCH("bias_rowvec_kernel", bias_rowvec_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)in, (const f16*)bias, (f16*)out, C, n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

static int bias_channel(const void* in, const void* bias, const void* tproj, const void* res,
                        void* out, int N, int C, int HW, void* stream) {
  const long long n = (long long)N * C * HW;
  DLM_LAUNCH("bias_channel_kernel", bias_channel_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)in, (const f16*)bias, (const f16*)tproj, (const f16*)res,
                     (f16*)out, C, HW, n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_bias_add_channel_fp16(const void* in, const void* bias, void* out, int N, int C, int H,
                              int W, void* stream) {
  if (N <= 0 || C <= 0 || H <= 0 || W <= 0) return DLM_OK;
  DLM_REQUIRE(in && bias && out, "NULL pointer");
  return bias_channel(in, bias, nullptr, nullptr, out, N, C, H * W, stream);
}

int dlm_conv_bias_biasch_fp16(const void* conv, const void* convbias, const void* tproj,
                              void* out, int B, int Cout, int H, int W, void* stream) {
  if (B <= 0 || Cout <= 0 || H <= 0 || W <= 0) return DLM_OK;
  DLM_REQUIRE(conv && convbias && tproj && out, "NULL pointer");
  return bias_channel(conv, convbias, tproj, nullptr, out, B, Cout, H * W, stream);
}

int dlm_conv_bias_residual_fp16(const void* conv, const void* convbias, const void* residual,
                                void* out, int B, int Cout, int H, int W, void* stream) {
  if (B <= 0 || Cout <= 0 || H <= 0 || W <= 0) return DLM_OK;
  DLM_REQUIRE(conv && convbias && residual && out, "NULL pointer");
  return bias_channel(conv, convbias, nullptr, residual, out, B, Cout, H * W, stream);
}

int dlm_geglu_fp16(const void* in, void* out, int tokens, int d, void* stream) {
  if (tokens <= 0 || d <= 0) return DLM_OK;
  DLM_REQUIRE(in && out, "NULL pointer");
  DLM_REQUIRE(in != out, "geglu cannot run in place");
  const long long n = (long long)tokens * d;
  DLM_LAUNCH("geglu_kernel", geglu_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)in, (f16*)out, d, n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_timestep_embedding_fp16(void* out, float timestep, int dim, float max_period,
                                void* stream) {
  if (dim <= 1) return DLM_OK;
  DLM_REQUIRE(out != nullptr, "NULL pointer");
  DLM_REQUIRE(max_period > 0.0f, "max_period must be positive");
  const int half = dim / 2;
  DLM_LAUNCH("timestep_embedding_kernel", timestep_embedding_kernel, dim3((half + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, (f16*)out, timestep, dim, logf(max_period));
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_sdxl_embed_inputs_fp16(const float* timesteps, const void* text_embeds, int text_dim,
                               const void* time_ids, int ids_bstride, int id_dim, void* t_emb,
                               int t_dim, void* add_in, int B, void* stream) {
  if (B <= 0) return DLM_OK;
  DLM_REQUIRE(timesteps && text_embeds && time_ids && t_emb && add_in, "NULL pointer");
  DLM_REQUIRE(ids_bstride >= 0 && text_dim > 0 && id_dim > 0 && t_dim > 0, "bad dims");
  DLM_REQUIRE(t_dim % 2 == 0 && id_dim % 2 == 0, "embedding dims must be even");
  DLM_LAUNCH("sdxl_embed_kernel", sdxl_embed_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, timesteps,
                     (const f16*)text_embeds, text_dim, (const f16*)time_ids, ids_bstride, id_dim,
                     (f16*)t_emb, t_dim, (f16*)add_in);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_linear_small_fp16(const void* X, int ldx, const void* W, const void* bias, void* Y,
                          int ldy, int M, int N, int K, int silu_in, int act, int accumulate,
                          void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(X && W && Y, "NULL pointer");
  DLM_REQUIRE(M <= 16, "linear_small supports M <= 16");
  DLM_REQUIRE(K % 8 == 0 && ldx % 8 == 0 && ldx >= K && ldy >= N, "bad K / strides");
  DLM_REQUIRE(dlm_aligned16(X) && dlm_aligned16(W), "X and W must be 16-byte aligned");
  DLM_REQUIRE(act == DLM_ACT_NONE || act == DLM_ACT_SILU, "act must be none or silu");
#define DLM_LINEAR_SMALL(MB)                                                                               \
  DLM_LAUNCH("linear_small_kernel", linear_small_kernel<MB>, dim3((N + 3) / 4), dim3(256), 0,                  \
             (hipStream_t)stream, (const f16*)X, ldx, (const f16*)W, (const f16*)bias, (f16*)Y, ldy, M, N, K, \
             silu_in, act, accumulate)
  if (M <= 2)
    DLM_LINEAR_SMALL(2);
  else if (M <= 4)
    DLM_LINEAR_SMALL(4);
  else if (M <= 8)
    DLM_LINEAR_SMALL(8);
  else
    DLM_LINEAR_SMALL(16);
#undef DLM_LINEAR_SMALL
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_euler_cfg_step(float* latent, const void* noise, void* model_in, int n, float guidance,
                       float sigma, float sigma_next, float in_scale, void* stream) {
  if (n <= 0) return DLM_OK;
  DLM_REQUIRE(latent && noise && model_in, "NULL pointer");
  DLM_LAUNCH("euler_cfg_kernel", euler_cfg_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     latent, (const f16*)noise, (f16*)model_in, n, guidance, sigma_next - sigma,
                     in_scale);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_euler_step(float* latent, const void* noise, void* model_in, int n, float sigma,
                   float sigma_next, float in_scale, void* stream) {
  if (n <= 0) return DLM_OK;
  DLM_REQUIRE(latent && noise && model_in, "NULL pointer");
  DLM_LAUNCH("euler_kernel", euler_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, latent,
                     (const f16*)noise, (f16*)model_in, n, sigma_next - sigma, in_scale);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_cast_f32_to_f16(const float* in, void* out, long long n, float scale, void* stream) {
  if (n <= 0) return DLM_OK;
  DLM_REQUIRE(in && out, "NULL pointer");
  DLM_REQUIRE(dlm_aligned16(in) && dlm_aligned16(out), "buffers must be 16-byte aligned");
  DLM_LAUNCH("cast_f32_f16_kernel", cast_f32_f16_kernel, dim3(grid_for(std::max(n >> 3, 1LL))), dim3(256), 0,
                     (hipStream_t)stream, in, (f16*)out, n, scale);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_scale_fp16(void* x, long long n, float scale, void* stream) {
  if (n <= 0) return DLM_OK;
  DLM_REQUIRE(x, "NULL pointer");
  DLM_LAUNCH("scale_f16_kernel", scale_f16_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     (f16*)x, n, scale);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_latent_to_vae_fp16(const float* latent, void* out, long long n, float scaling_factor,
                           void* stream) {
  if (n <= 0) return DLM_OK;
  DLM_REQUIRE(latent && out, "NULL pointer");
  DLM_REQUIRE(scaling_factor != 0.0f, "scaling_factor must be non-zero");
  DLM_LAUNCH("latent_to_vae_kernel", latent_to_vae_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     latent, (f16*)out, n, scaling_factor);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_image_to_rgb8(const void* image, uint8_t* rgb, int N, int H, int W, void* stream) {
  if (N <= 0 || H <= 0 || W <= 0) return DLM_OK;
  DLM_REQUIRE(image && rgb, "NULL pointer");
  const long long HW = (long long)H * W, n = (long long)N * HW * 3;
  DLM_LAUNCH("image_to_rgb8_kernel", image_to_rgb8_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)image, rgb, HW, n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_scale_latent_fp16(const float* latent, void* model_in, int n, float scale, int copies,
                          void* stream) {
  if (n <= 0 || copies <= 0) return DLM_OK;
  DLM_REQUIRE(latent && model_in, "NULL pointer");
  DLM_LAUNCH("scale_latent_kernel", scale_latent_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     latent, (f16*)model_in, n, scale, copies);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

}  // extern "C"
