/*
 * dlm.h — C ABI of the MI355X (gfx950) SDXL UNet dense-contraction hot path.
 *
 * Every entry point takes plain device pointers (fp16 = IEEE binary16 bit
 * patterns, passed as void*), int dimensions, float scalars and an opaque
 * stream handle (a hipStream_t passed as void*; NULL = the default stream).
 * Every entry point returns an int status (DLM_OK == 0); on failure
 * dlm_last_error() returns a thread-local description.  Work is enqueued on
 * the stream and is stream-ordered; nothing synchronises unless its name says
 * so.  The caller owns every buffer; no pointer is retained past a call.
 *
 * Dimension convention (reference src/kernels/conv2d.cu:762-771): a call with
 * a non-positive dimension is a silent no-op that returns DLM_OK.
 *
 * Two layouts appear:
 *   - reference layout entry points (dlm_conv2d_fp16, dlm_group_norm_fp16,
 *     dlm_attention_fp16, ...) take exactly the reference kernel host API's
 *     arguments and layouts (NCHW activations, [B,H,S,Dh] attention);
 *   - channels-last entry points (*_nhwc_*, dlm_linear_fp16,
 *     dlm_attention_strided_fp16) are the fused native forms that the UNet
 *     driver uses: activations are [N,H,W,C] == [tokens,C], so the
 *     transformer's sequence layout needs no transposes.
 */
#ifndef DLM_H
#define DLM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DLM_OK 0
#define DLM_ERR_INVALID_ARG 1
#define DLM_ERR_HIP 2
#define DLM_ERR_OUT_OF_MEMORY 3
#define DLM_ERR_UNSUPPORTED 4
#define DLM_ERR_NOT_FOUND 5
#define DLM_ERR_STATE 6

/* ------------------------------------------------------------------ */
/* Status, device, memory, streams, events                             */
/* ------------------------------------------------------------------ */

/* Replaces the CUDA_CHECK / std::runtime_error reporting of the reference
 * (src/kernels/utils.cuh:17-45): returns the last error text of this thread. */
const char* dlm_last_error(void);
/* Set this thread's error text (lets the C++ host layer report through the
 * same channel). */
void dlm_set_last_error(const char* msg);
/* Name of the kernel (template instantiation, as a profiler lists it) that
 * the last entry point called on this thread launched last; "" if none since
 * the last reset.  reset = 1 clears it after reading.  Lets a caller that
 * times each call attribute the time to a kernel. */
const char* dlm_last_kernel(int reset);
/* Problem of that launch when it was a GEMM or implicit-GEMM conv: dims[0..3]
 * = rows M, output columns N, reduction length K, flags (bit 0: residual
 * epilogue; bits 4-7: activation code; bit 8: conv; bit 9: LayerNorm folded
 * in, dlm_linear_ln_fp16); zeros otherwise. */
int dlm_last_kernel_dims(int* dims);
/* Dispatch timing, for a caller that times each entry-point call (no
 * reference counterpart: the reference times its kernels with an external
 * profiler).  While armed on this thread, every kernel the library launches
 * carries the two events in its own dispatch (hipExtLaunchKernel): `start`
 * takes the start of the first launch after arming, `stop` the end of each
 * launch.  The pair then spans the kernels of the calls made while armed with
 * no marker packets between them, i.e. the kernels' own execution as a
 * profiler's kernel trace reports it.  dlm_prof_disarm returns how many
 * kernels were launched while armed (0: the events were not touched).  Not
 * for work being captured into a graph. */
int dlm_prof_arm(void* start, void* stop);
int dlm_prof_disarm(void);
int dlm_get_device_count(int* count);
int dlm_set_device(int device);
/* Name of the GPU architecture of the current device (e.g. "gfx950"). */
int dlm_device_arch(char* buf, int buflen);

/* Device memory for the VRAM arena and allocators (reference
 * src/core/allocator.hpp:16-130 CudaAllocator, src/kernels/device_arena.cu
 * cudaMalloc/cudaFree call sites). */
int dlm_malloc(void** ptr, size_t bytes);
int dlm_free(void* ptr);
int dlm_host_malloc_pinned(void** ptr, size_t bytes);
int dlm_host_free_pinned(void* ptr);
/* kind: 0 host->device, 1 device->host, 2 device->device, 3 default (UVA). */
int dlm_memcpy(void* dst, const void* src, size_t bytes, int kind);
int dlm_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream);
int dlm_memset_async(void* dst, int value, size_t bytes, void* stream);
int dlm_device_synchronize(void);
int dlm_mem_get_info(size_t* free_bytes, size_t* total_bytes);
/* Library staging of the reference-layout entry points (dlm_conv2d_fp16,
 * dlm_gemm_fp16, dlm_attention_fp16) and the split-K workspace of the
 * channels-last GEMMs are kept per (device, stream) and grow on first use;
 * staging of other streams is dropped when a device's total would pass
 * 2 GiB.  dlm_scratch_release synchronises `stream` and frees everything
 * the library holds for it: call it before destroying a stream that ran
 * library entry points (a new stream may reuse the handle).  Graphs captured
 * on that stream must not be replayed afterwards.  No reference counterpart
 * (the reference's launch_* wrappers cudaMalloc / cudaFree per call).
 * dlm_scratch_bytes reports the device bytes the library holds for all
 * streams. */
int dlm_scratch_release(void* stream);
int dlm_scratch_bytes(size_t* bytes);

int dlm_stream_create(void** stream);
int dlm_stream_destroy(void* stream);
int dlm_stream_synchronize(void* stream);
/* HIP graphs: capture the work enqueued on a created stream (thread-local
 * capture mode), instantiate it, replay it.  end_capture returns the
 * executable graph; the captured work itself does not run until launched.
 * Replaces the reference's CUDA-graph switch (FastConfig::graphs,
 * src/server/fast_config.hpp). */
int dlm_graph_begin_capture(void* stream);
int dlm_graph_end_capture(void* stream, void** exec);
int dlm_graph_launch(void* exec, void* stream);
int dlm_graph_destroy(void* exec);
int dlm_event_create(void** event);
int dlm_event_destroy(void* event);
int dlm_event_record(void* event, void* stream);
int dlm_event_synchronize(void* event);
int dlm_event_elapsed_ms(float* ms, void* start, void* stop);

/* ------------------------------------------------------------------ */
/* Reference-layout kernel host API (1:1 with src/kernels/ *.cuh)       */
/* ------------------------------------------------------------------ */

/* conv2d, NCHW fp16, fp32 accumulate, optional bias (NULL = none), any
 * per-axis stride, zero padding and dilation; output size
 * (H + 2 pad - dilation (KH - 1) - 1) / stride + 1 per axis.
 * Replaces dollama::launch_conv2d (src/kernels/conv2d.cuh:38-40).  Stages the
 * input channels-last and the packed weight in library buffers kept per
 * (device, stream); they grow on first use (hipMalloc after a device
 * synchronisation).  Not for graph capture: a later call may re-allocate
 * the staging a captured launch reads (dlm_conv2d_fp16_noalloc is the
 * capturable form). */
int dlm_conv2d_fp16(const void* in, const void* weight, const void* bias, void* out,
                    int N, int Cin, int H, int W, int Cout, int KH, int KW,
                    int stride_h, int stride_w, int pad_h, int pad_w,
                    int dilation_h, int dilation_w, void* stream);

/* Allocation-free variant of dlm_conv2d_fp16 (same arguments, same kernels,
 * bit-identical output).  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The staging (channels-
 * last input padded to a multiple of 8 channels, then the packed weight at
 * the next 256-byte boundary: 2*N*H*W*Cin8 + 2*Cout*KH*KW*Cin8 bytes) lives
 * in one fixed array of DLM_CONV2D_NOALLOC_MAX_BYTES per GPU, held from the
 * library's first use of that GPU until the process ends; a call needing
 * more returns DLM_ERR_INVALID_ARG before launching anything.  Split-K is
 * not used.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, two threads) race and must be ordered by
 * the caller. */
#define DLM_CONV2D_NOALLOC_MAX_BYTES ((size_t)64 << 20)
int dlm_conv2d_fp16_noalloc(const void* in, const void* weight, const void* bias, void* out,
                            int N, int Cin, int H, int W, int Cout, int KH, int KW,
                            int stride_h, int stride_w, int pad_h, int pad_w,
                            int dilation_h, int dilation_w, void* stream);

/* C = alpha * op(A) op(B) + beta * C, row-major, fp16 in/out, fp32 accumulate.
 * op(A) = [M,K], op(B) = [K,N].  Operands that are not [M,K] / [N,K] with
 * 16-byte aligned rows are first copied (transposed, K padded to a multiple
 * of 8) into per-stream library staging, so like dlm_conv2d_fp16 this entry
 * is not for graph capture.
 * Replaces dollama::launch_gemm_fp16 (src/kernels/gemm.cuh:44-53). */
int dlm_gemm_fp16(const void* A, const void* B, void* C, int M, int N, int K,
                  float alpha, float beta, int transA, int transB, void* stream);

/* GroupNorm over NCHW, fp32 statistics; fuse_silu = 1 applies x*sigmoid(x).
 * Replaces launch_group_norm / launch_group_norm_mb / launch_group_norm_silu
 * (src/kernels/groupnorm.cuh:51-108). */
int dlm_group_norm_fp16(const void* in, const void* gamma, const void* beta, void* out,
                        int N, int C, int H, int W, int num_groups, float eps,
                        int fuse_silu, void* stream);

/* LayerNorm over the last dim C of [rows, C]; gamma/beta may be NULL.
 * Replaces launch_layer_norm (src/kernels/layernorm.cuh:51-57). */
int dlm_layer_norm_fp16(const void* in, const void* gamma, const void* beta, void* out,
                        int rows, int C, float eps, void* stream);

/* O = softmax(scale * Q K^T) V, Q/O [B,H,Sq,Dh], K/V [B,H,Sk,Dh], fp32 softmax,
 * any head size (as launch_attention picks a path by Dh,
 * src/kernels/attention.cu:18-21): Dh = 64 runs the flash kernel over a
 * transposed-V copy, other head sizes an fp32 scores GEMM, a row softmax and
 * a P V^T GEMM in row chunks whose scores stay within 256 MiB.  The copies
 * live in per-stream library staging: not for graph capture.  Replaces
 * launch_attention / launch_attention_fast (src/kernels/attention.cuh:53-73). */
int dlm_attention_fp16(const void* q, const void* k, const void* v, void* out,
                       int B, int H, int Sq, int Sk, int Dh, float scale, void* stream);

/* out[t, j] = in[t, j] * gelu_erf(in[t, d + j]); in [tokens, 2d], out [tokens, d].
 * Replaces launch_geglu (src/kernels/geglu.cuh:42). */
int dlm_geglu_fp16(const void* in, void* out, int tokens, int d, void* stream);

/* Replace launch_silu / launch_gelu / launch_gelu_tanh
 * (src/kernels/activation.cuh:33-41): x sigmoid(x), 0.5 x (1 + erf(x/sqrt 2)),
 * 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))); fp32 math, in place
 * allowed. */
int dlm_silu_fp16(const void* in, void* out, int n, void* stream);
int dlm_gelu_fp16(const void* in, void* out, int n, void* stream);
int dlm_gelu_tanh_fp16(const void* in, void* out, int n, void* stream);
/* Replace launch_add / launch_upsample_nearest2x (src/kernels/elementwise.cuh:26-37). */
int dlm_add_fp16(const void* a, const void* b, void* out, int n, void* stream);
int dlm_upsample_nearest2x_fp16(const void* in, void* out, int N, int C, int H, int W,
                                void* stream);
/* Replace launch_bias_add_rowvec / launch_bias_add_channel /
 * launch_conv_bias_biasch / launch_conv_bias_residual
 * (src/kernels/bias_add.cuh:32-103).  Single rounding of the fp32 sum. */
int dlm_bias_add_rowvec_fp16(const void* in, const void* bias, void* out, int tokens, int C,
                             void* stream);
int dlm_bias_add_channel_fp16(const void* in, const void* bias, void* out,
                              int N, int C, int H, int W, void* stream);
int dlm_conv_bias_biasch_fp16(const void* conv, const void* convbias, const void* tproj,
                              void* out, int B, int Cout, int H, int W, void* stream);
int dlm_conv_bias_residual_fp16(const void* conv, const void* convbias, const void* residual,
                                void* out, int B, int Cout, int H, int W, void* stream);
/* Sinusoidal embedding, cos first (flip_sin_to_cos), shift 0.
 * Replaces launch_timestep_embedding (src/kernels/timeembed.cuh:44-47). */
int dlm_timestep_embedding_fp16(void* out, float timestep, int dim, float max_period,
                                void* stream);

/* ------------------------------------------------------------------ */
/* Channels-last fused entry points (native forms used by the UNet)     */
/* ------------------------------------------------------------------ */

/* Epilogue activation codes. */
#define DLM_ACT_NONE 0
#define DLM_ACT_SILU 1
/* GEGLU: the weight rows (and bias) are interleaved in groups of 4
 * (4 value rows, then the 4 matching gate rows, see dlm_geglu_pack_fp16);
 * the output has N/2 columns: out = value * gelu_erf(gate).  N % 16 == 0. */
#define DLM_ACT_GEGLU 2
#define DLM_ACT_GELU 3

/* Y[M, N] = act(alpha * X[M,K] W[N,K]^T + bias[N]) + beta * R[M, N]
 * X row stride lda, W row stride ldw, Y row stride ldy, R row stride ldr
 * (all in elements; all multiples of 8; K multiple of 8).
 * bias and R may be NULL.  act = DLM_ACT_*.  For GEGLU, ldy counts output
 * columns (N/2).  Replaces linear() = launch_gemm_fp16(transB) +
 * launch_bias_add_rowvec (src/infer/unet.cu:517-525), with the residual add
 * (launch_add, unet.cu:739) and launch_geglu (unet.cu:793) fused. */
int dlm_linear_fp16(const void* X, int lda, const void* W, int ldw, const void* bias,
                    const void* R, int ldr, void* Y, int ldy, int M, int N, int K,
                    float alpha, float beta, int act, void* stream);

/* dlm_linear_fp16 (act none/silu/gelu) that also writes the GroupNorm chunk
 * statistics of Y, as dlm_conv_nhwc_args::gn_stats does: Y holds
 * M / tokens samples of tokens rows (tokens <= 16384); gn_stats is a
 * GroupNorm workspace of dlm_group_norm_nhwc_workspace_bytes(M / tokens, N,
 * tokens) bytes for dlm_group_norm_nhwc_prestats_fp16.  N and ldy multiples
 * of 8.  No counterpart in the reference (the transformer's proj_out feeding
 * the next ResnetBlock2D's GroupNorm). */
int dlm_linear_gn_stats_fp16(const void* X, int lda, const void* W, int ldw, const void* bias,
                             const void* R, int ldr, void* Y, int ldy, int M, int N, int K, float alpha,
                             float beta, int act, int tokens, void* gn_stats, void* stream);

/* Linear with a transposed tail: Y = X W^T for columns [0, vt_col0) (row
 * stride ldy) and, for columns n >= vt_col0, the transpose per sample:
 * VT[(m / tokens) * (N - vt_col0) + n - vt_col0][m % tokens] with row stride
 * vt_ld >= tokens; entries [tokens, vt_ld) of every V^T row are set to 0.
 * Fed with the fused QKV weight [3C, C] and vt_col0 = 2C it writes Q|K as
 * [M, 2C] and V^T as [B, C, vt_ld] = [B, H, 64, vt_ld], the layout
 * dlm_attention_vt_fp16 reads.  No counterpart in the reference, which
 * splits heads with separate kernels (k_split_heads,
 * src/infer/unet.cu:153-278). */
int dlm_linear_vt_fp16(const void* X, int lda, const void* W, int ldw, const void* bias, void* Y,
                       int ldy, void* VT, int vt_col0, int tokens, int vt_ld, int M, int N, int K,
                       void* stream);

/* dlm_linear_fp16 with an fp32 output Y and an fp32 residual R (fp16 X, W,
 * bias; act none/silu/gelu): Y = act(alpha * X W^T + bias) + beta * R.  Used
 * where a result leaves the fp16 range or feeds a softmax: the VAE mid-block
 * attention scores (the reference computes them inside launch_attention,
 * src/kernels/vae_decode.cu:682-683) and the decoder's fp32 stages
 * (src/kernels/vae_decode.cu:317-327). */
int dlm_linear_f32out_fp16(const void* X, int lda, const void* W, int ldw, const void* bias,
                           const float* R, int ldr, float* Y, int ldy, int M, int N, int K,
                           float alpha, float beta, int act, void* stream);

/* LayerNorm folded into the linear that consumes it (no LayerNorm launch,
 * no normalised copy of X):
 *   Y = act(LN(X) W0^T + b) + beta * R,  LN(X) = (X - mean) * rstd * gamma + lnbeta
 * with per-row mean and variance over X's K columns (one pass in fp32:
 * var = max(E[x^2] - mean^2, 0), rstd = 1 / sqrt(var + eps), as
 * launch_layer_norm computes them, src/kernels/layernorm.cu:78-126),
 * computed inside the GEMM from the X operand it multiplies.  W, c1, c2 come
 * from dlm_ln_fold_fp16(W0, gamma, lnbeta, b); W may be GEGLU-packed (fold
 * after dlm_geglu_pack_fp16, with the packed bias).  K % 64 == 0; c1, c2
 * 16-byte aligned.  Same epilogue options as dlm_linear_fp16 / _vt_fp16
 * (no bias argument: it is inside c2).  No counterpart entry in the
 * reference, whose LayerNorm is a separate launch. */
int dlm_linear_ln_fp16(const void* X, int lda, const void* W, int ldw, const float* c1,
                       const float* c2, float eps, const void* R, int ldr, void* Y, int ldy, int M,
                       int N, int K, float beta, int act, void* stream);
int dlm_linear_vt_ln_fp16(const void* X, int lda, const void* W, int ldw, const float* c1,
                          const float* c2, float eps, void* Y, int ldy, void* VT, int vt_col0,
                          int tokens, int vt_ld, int M, int N, int K, void* stream);
/* Weight side of the fold: W_out[n] = fp16(W[n] * gamma) (a copy when gamma
 * is NULL), c1[n] = sum_k W_out[n][k], c2[n] = sum_k lnbeta[k] W[n][k] + b[n]
 * (fp32; lnbeta / b may be NULL).  W_out may be W itself (in place, with
 * ldo == ldw); any other overlap of the two is DLM_ERR_INVALID_ARG. */
int dlm_ln_fold_fp16(const void* W, int ldw, int N, int K, const void* gamma, const void* lnbeta,
                     const void* b, void* W_out, int ldo, float* c1, float* c2, void* stream);

/* Repack GEGLU projection weight [2d, K] and bias [2d] (value rows first, as
 * diffusers stores them) into the 4-row value/gate interleave DLM_ACT_GEGLU
 * expects: packed row 8q+s holds value row 4q+s (s < 4) or gate row
 * d+4q+s-4 (d % 4 == 0). */
int dlm_geglu_pack_fp16(const void* w, const void* bias, void* w_out, void* bias_out,
                        int d, int K, void* stream);

/* Repack a conv weight [Cout, Cin, KH, KW] into the channels-last GEMM form
 * (Cin_pad >= Cin, zero filled), written at row stride ld_out elements
 * (ld_out >= KH*KW*Cin_pad) starting at column col0.  Column order: when
 * Cin_pad is a multiple of 64, [Cin_pad/64][KH][KW][64] (channel blocks
 * outermost, the K order the implicit-GEMM conv walks); otherwise
 * [KH][KW][Cin_pad].  A 1x1 weight is [Cin_pad] either way. */
int dlm_conv_weight_pack_fp16(const void* w, void* out, int Cout, int Cin, int KH, int KW,
                              int Cin_pad, int ld_out, int col0, void* stream);

/* Same layout as dlm_conv_weight_pack_fp16, accumulating instead of
 * overwriting: out[...] = fp16(out[...] + w[...]) for ci < Cin; the padding
 * channels are left unchanged.  Used to merge a LoRA delta into a packed
 * conv weight (no counterpart in the reference, whose weights stay NCHW). */
int dlm_conv_weight_pack_add_fp16(const void* w, void* out, int Cout, int Cin, int KH, int KW,
                                  int Cin_pad, int ld_out, int col0, void* stream);

/* Layout transposes: NCHW <-> NHWC (C_pad >= C channels in the NHWC side,
 * extra channels zero filled on the way in). */
int dlm_nchw_to_nhwc_fp16(const void* in, void* out, int N, int C, int HW, int C_pad,
                          void* stream);
int dlm_nhwc_to_nchw_fp16(const void* in, void* out, int N, int C, int HW, int C_pad,
                          void* stream);

/* Implicit-GEMM convolution on channels-last activations.
 * Output pixel m = (n, oh, ow), output channel co:
 *   y[m, co] = act( sum_seg sum_taps sum_ci x_seg[...] * w[co, k] + bias[co]
 *                   + tbias[n * tbias_ld + co] ) + residual[m * res_ld + co]
 * Segment 0 is a KHxKW conv (stride, pad) over the channel concatenation of
 * src0 (C0a channels, row stride ld0a) and src0b (C0b channels, may be NULL)
 * of spatial size H x W (or 2H x 2W nearest-upsampled when upsample = 1).
 * Segment 1 (optional, C1a > 0) is a 1x1 stride-1 conv over the concatenation
 * of src1a/src1b at the output resolution, accumulated into the same sum
 * (the fused ResnetBlock2D conv_shortcut).  Weight rows are [Cout, Ktot] with
 * Ktot = KH*KW*(C0a+C0b) + (C1a+C1b), segment 0 in the column order of
 * dlm_conv_weight_pack_fp16 with Cin_pad = C0a+C0b, then segment 1, row
 * stride ldw.  Output channels-last with row
 * stride ldy, or NCHW when out_nchw = 1; fp32 output elements when
 * out_f32 = 1 and an fp32 residual when res_f32 = 1 (the VAE decoder's fp32
 * stages, src/kernels/vae_decode.cu:317-327; operands stay fp16).
 * gn_stats (may be NULL): the GroupNorm chunk statistics of the output are
 * also written there, as the first bytes of a GroupNorm workspace
 * (dlm_group_norm_nhwc_workspace_bytes(N, Cout, Ho*Wo)) that
 * dlm_group_norm_nhwc_prestats_fp16 then normalises the output with, with no
 * statistics pass; fp16 channels-last output, Cout and ldy multiples of 8,
 * Ho*Wo <= 16384.  The values equal dlm_group_norm_chunk_stats_fp16's on the
 * output bit for bit, whichever kernel the convolution runs. */
typedef struct dlm_conv_nhwc_args {
  const void* src0a; const void* src0b; int C0a; int C0b; int ld0a; int ld0b;
  const void* src1a; const void* src1b; int C1a; int C1b; int ld1a; int ld1b;
  int N; int H; int W; int KH; int KW; int stride; int pad; int upsample;
  const void* weight; int ldw; int Cout;
  const void* bias; const void* tbias; int tbias_ld;
  const void* residual; int res_ld;
  void* out; int ldy; int out_nchw; int act;
  int out_f32;  /* 1: out holds fp32 elements */
  int res_f32;  /* 1: residual holds fp32 elements */
  void* gn_stats; /* GroupNorm chunk statistics of the output, or NULL */
} dlm_conv_nhwc_args;
int dlm_conv2d_nhwc_fp16(const dlm_conv_nhwc_args* args, void* stream);

/* GroupNorm on channels-last [N, HW, C] (row stride ld_in / ld_out), C split
 * into num_groups contiguous groups; optional second source (concatenation
 * along channels: the first C_a channels from in_a, the rest from in_b).
 * fuse_silu = 1 applies x*sigmoid(x).  workspace must hold
 * dlm_group_norm_nhwc_workspace_bytes(N, C, HW) bytes. */
size_t dlm_group_norm_nhwc_workspace_bytes(int N, int C, int HW);
int dlm_group_norm_nhwc_fp16(const void* in_a, int C_a, int ld_a, const void* in_b, int ld_b,
                             const void* gamma, const void* beta, void* out, int ld_out,
                             int N, int HW, int C, int num_groups, float eps, int fuse_silu,
                             void* workspace, void* stream);
/* GroupNorm chunk statistics: per channel c of sample n, over the pixel rows
 * [64k, min(64k + 64, HW)) of chunk k, shift = the chunk's first value,
 * s1 = sum (x - shift), s2 = sum (x - shift)^2 (fp32, rows in order), stored
 * as float2 (shift + s1/cnt, max(s2 - s1 * s1/cnt, 0)) at [n][k][c] from the
 * start of a GroupNorm workspace.  fp16 input, HW <= 16384.  No counterpart
 * in the reference: the statistics half of the GroupNorm, which producers
 * write from their epilogues (dlm_conv_nhwc_args::gn_stats). */
int dlm_group_norm_chunk_stats_fp16(const void* in, int ld_in, int N, int HW, int C, void* workspace,
                                    void* stream);
/* dlm_group_norm_nhwc_fp16 (one source, fp16, HW <= 16384) whose workspace
 * already holds the input's chunk statistics (written by a producer with
 * gn_stats, or by dlm_group_norm_chunk_stats_fp16): the merge and the apply
 * pass only.  Same result as dlm_group_norm_nhwc_fp16 on that input, bit for
 * bit.  No counterpart in the reference (its GroupNorm computes the
 * statistics itself, src/kernels/groupnorm.cu:91-148). */
int dlm_group_norm_nhwc_prestats_fp16(const void* in, int ld_in, const void* gamma, const void* beta,
                                      void* out, int ld_out, int N, int HW, int C, int num_groups,
                                      float eps, int fuse_silu, void* workspace, void* stream);
/* The same over the channel concatenation of two fp16 sources (in_a's C_a
 * channels, then in_b's C - C_a), each with its own chunk statistics:
 * stats_a [N][chunks][C_a] and stats_b [N][chunks][C - C_a], as their
 * producers wrote them (the first bytes of a GroupNorm workspace for that
 * source's channel count).  workspace (dlm_group_norm_nhwc_workspace_bytes(N,
 * C, HW)) receives the scale / shift only.  Same result as
 * dlm_group_norm_nhwc_fp16 over the two sources, bit for bit.  The UNet's
 * up-path ResnetBlock2D norm1 over concat(h, skip); the reference
 * concatenates first and normalises the copy (src/infer/unet.cu:1168-1181,
 * k_concat_chw at :247-277). */
int dlm_group_norm_nhwc_prestats2_fp16(const void* in_a, int C_a, int ld_a, const void* in_b, int ld_b,
                                       const void* stats_a, const void* stats_b, const void* gamma,
                                       const void* beta, void* out, int ld_out, int N, int HW, int C,
                                       int num_groups, float eps, int fuse_silu, void* workspace,
                                       void* stream);
/* Same GroupNorm(+SiLU) over fp32 channels-last input (one source), fp16
 * output: the VAE decoder's fp32 stages (reference launch_group_norm_f32,
 * src/kernels/vae_decode.cu:466-545). */
int dlm_group_norm_nhwc_f32in(const float* in, int ld_in, const void* gamma, const void* beta,
                              void* out, int ld_out, int N, int HW, int C, int num_groups,
                              float eps, int fuse_silu, void* workspace, void* stream);

/* Strided flash attention: element (b, s, h, d) of Q is at
 * q[b*q_sb + s*q_ss + h*q_sh + d] (likewise K, V, O); Dh = 64. */
typedef struct dlm_attention_args {
  const void* q; long long q_sb; long long q_ss; long long q_sh;
  const void* k; long long k_sb; long long k_ss; long long k_sh;
  const void* v; long long v_sb; long long v_ss; long long v_sh;
  void* o; long long o_sb; long long o_ss; long long o_sh;
  int B; int H; int Sq; int Sk; int Dh; float scale;
} dlm_attention_args;
int dlm_attention_strided_fp16(const dlm_attention_args* args, void* stream);

/* Flash attention with V supplied transposed: element (b, h, d, key) of V^T
 * is at vt[b*vt_sb + h*vt_sh + d*vt_ld + key] (vt_ld a multiple of 8 and at
 * least Sk rounded up to 8; keys [Sk, that) must hold finite values, e.g.
 * the zeros dlm_linear_vt_fp16 writes).  Q, K, O as in dlm_attention_args;
 * Dh = 64.  k_bytes and
 * vt_bytes bound the K and V^T allocations (each < 2 GiB): reads past them
 * return zero.  The UNet's QKV projection writes V^T directly (see
 * dlm_linear_vt_fp16), so self-attention needs no LDS transpose.
 * Same arithmetic as dlm_attention_fp16 (launch_attention,
 * src/kernels/attention.cuh:53-73). */
typedef struct dlm_attention_vt_args {
  const void* q;
  const void* k;
  const void* vt;
  void* o;
  long long q_sb, q_ss, q_sh;
  long long k_sb, k_ss, k_sh;
  long long vt_sb, vt_sh;
  long long o_sb, o_ss, o_sh;
  int vt_ld;
  int B, H, Sq, Sk;
  float scale;
  unsigned long long k_bytes, vt_bytes;
} dlm_attention_vt_args;
int dlm_attention_vt_fp16(const dlm_attention_vt_args* args, void* stream);

/* SDXL conditioning inputs on the device (no host round trip, unlike the
 * reference's D2H of time_ids, src/infer/unet.cu:999-1000):
 * t_emb[b, 0:t_dim] = sinusoid(timesteps[b]) and
 * add_in[b] = text_embeds[b, 0:text_dim] ++ sinusoid_{id_dim}(time_ids[b*ids_bstride + i]), i < 6
 * (SDXL: t_dim 320, text_dim 1280, id_dim 256, add_in width 2816; ids_bstride 0 shares
 * one time_ids vector across the batch). */
int dlm_sdxl_embed_inputs_fp16(const float* timesteps, const void* text_embeds, int text_dim,
                               const void* time_ids, int ids_bstride, int id_dim, void* t_emb,
                               int t_dim, void* add_in, int B, void* stream);

/* Skinny linear for M <= 16 rows (the time / add embedding MLPs and the
 * per-resnet time_emb_proj): Y[m, n] = act(X'[m,:] . W[n,:] + bias[n]) where
 * X' = silu(X) when silu_in = 1.  act: DLM_ACT_NONE or DLM_ACT_SILU.
 * Y rows may accumulate: Y = Y + result when accumulate = 1. */
int dlm_linear_small_fp16(const void* X, int ldx, const void* W, const void* bias, void* Y,
                          int ldy, int M, int N, int K, int silu_in, int act, int accumulate,
                          void* stream);

/* Euler step fused with classifier-free guidance (reference
 * src/infer/diffusion.cu:968-973 and src/infer/scheduler.hpp:112-143):
 * eps = u + g (c - u) from noise [2, n] (cond slice first, uncond second),
 * latent += eps * (sigma_next - sigma) in fp32, then the next model input
 * model_in[0:n] = model_in[n:2n] = fp16(latent * in_scale), where in_scale =
 * 1/sqrt(sigma_next^2 + 1) (scale_model_input of the next step). */
int dlm_euler_cfg_step(float* latent, const void* noise, void* model_in, int n,
                       float guidance, float sigma, float sigma_next, float in_scale,
                       void* stream);

/* Euler step without guidance (one noise prediction [n]): latent +=
 * noise * (sigma_next - sigma) in fp32, model_in[0:n] = fp16(latent *
 * in_scale) (reference generate(), src/infer/diffusion.cu:551-680). */
int dlm_euler_step(float* latent, const void* noise, void* model_in, int n, float sigma,
                   float sigma_next, float in_scale, void* stream);

/* model_in[c*n + i] = fp16(latent[i] * scale) for c < copies (the first
 * step's scale_model_input, reference src/infer/scheduler.hpp:112-120). */
int dlm_scale_latent_fp16(const float* latent, void* model_in, int n, float scale, int copies,
                          void* stream);

/* ------------------------------------------------------------------ */
/* VAE decoder helpers                                                 */
/* ------------------------------------------------------------------ */

/* out[i] = fp16(in[i] * scale) (reference k_f2h, src/kernels/vae_decode.cu:
 * 340-347, with a power-of-two scale that keeps an fp32 activation inside
 * the fp16 range when it becomes a conv operand). */
int dlm_cast_f32_to_f16(const float* in, void* out, long long n, float scale, void* stream);
/* x[i] = fp16(x[i] * scale) in place. */
int dlm_scale_fp16(void* x, long long n, float scale, void* stream);
/* out[i] = fp16(latent[i] / scaling_factor): the VAE input (reference
 * src/infer/diffusion.cu:980-984; SDXL scaling_factor 0.13025). */
int dlm_latent_to_vae_fp16(const float* latent, void* out, long long n, float scaling_factor,
                           void* stream);
/* Decoded image [N, 3, H, W] fp16 in [-1, 1] -> device RGB8 [N, H, W, 3]
 * with q = int(clamp(v/2 + 1/2, 0, 1) * 255 + 0.5) (reference
 * image_f16_to_rgb_u8, src/infer/diffusion.cu:146-165); NaN -> 0. */
int dlm_image_to_rgb8(const void* image, uint8_t* rgb, int N, int H, int W, void* stream);
/* P[r, :] = softmax(S[r, :]) for fp32 scores S [rows, cols] (row stride
 * lds) into fp16 P (row stride ldp); cols, lds, ldp multiples of 4.  The
 * softmax step of the VAE mid-block attention (reference launch_attention
 * with Dh = 512, src/kernels/vae_decode.cu:682-683). */
int dlm_softmax_rows_f32_fp16(const float* S, long long lds, void* P, long long ldp, int rows,
                              int cols, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DLM_H */
