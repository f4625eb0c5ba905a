// MFMA GEMM core for gfx950 and everything built on it: linears with fused
// bias / residual / GEGLU epilogues, and implicit-GEMM convolution on
// channels-last activations (no im2col buffer).
//
// Replaces, by behaviour (not by code):
//   - launch_gemm_fp16 -> cublasGemmEx (reference src/kernels/gemm.cu:425-434)
//   - linear() = gemm + launch_bias_add_rowvec (src/infer/unet.cu:517-525)
//   - launch_conv2d's im2col + GEMM + conv_bias_add_rows
//     (src/kernels/conv2d.cu:362-448, :219-270, :171-182)
//   - launch_geglu (src/kernels/geglu.cu:26-48) as a GEMM epilogue
//   - launch_conv_bias_biasch / launch_conv_bias_residual
//     (src/kernels/bias_add.cu:106-159) as conv epilogues.
//
// Design: C[M,N] = A[M,K] * W[N,K]^T with both operands K-contiguous, the
// form MFMA consumes directly.  Two kernels:
//   - dma_gemm_kernel (every aligned UNet / VAE shape): a BM x BN tile per
//     workgroup of 8 waves, each wave a WM x WN block of
//     v_mfma_f32_16x16x32_f16 tiles in transposed form (W fragment x A
//     fragment), so a lane holds one output row and 4 consecutive columns.
//     K advances in 64-wide slices copied global -> LDS by DMA
//     (buffer_load ... lds) into a ring of NS stages (one or two slices
//     each, one barrier per stage); LDS rows are 128 B with their 16-byte
//     chunks XOR-swizzled by (row >> 1) & 7, so every ds_read_b128 fragment
//     phase is conflict-free; the next k-step's fragments are read before
//     the current k-step's MFMAs.  Optional split-K with a last-arriver
//     reduction in split order, and an XCD-aware tile order.
//   - mfma_gemm_kernel (small channel counts, small grids, unaligned
//     operands): 4 waves of 32x32x16 MFMA blocks with VGPR-staged,
//     double-buffered LDS slices (row stride 72 halfs).
// The A operand is produced by a loader: plain rows for linears, or the
// implicit im2col gather (zero padding, channel concatenation of two
// sources, nearest-2x upsampling, a second 1x1 segment) for convolutions.
#include <algorithm>
#include <map>
#include <vector>
#include <mutex>
#include <type_traits>
#include <utility>

#include "common.hpp"
#include "dlm_tuning.h"

namespace dlm {

constexpr int BK = 64;
constexpr int LS = BK + 8;  // LDS row stride in halfs

struct EpiArgs {
  f16* y;
  int ldy;
  const f16* bias;
  const f16* res;
  int ldr;
  float alpha;
  float beta;
  int act;
  const f16* tbias;
  int tbias_ld;
  int rows_per_sample;  // output pixels per sample (conv), for tbias / NCHW out
  int out_nchw;
  int M;
  int N;
  // transposed-V output (DMA core only): columns >= vt_col0 of row m go to
  // vt[((m / vt_tokens) * (N - vt_col0) + col - vt_col0) * vt_ld + m % vt_tokens];
  // positions [vt_tokens, vt_ld) of every V^T row are written with zeros
  f16* vt;
  int vt_col0;
  int vt_tokens;
  int vt_ld;
  // fp32 output (y holds floats) / fp32 residual (res holds floats): the
  // wide-range paths (VAE decoder stages whose pre-residual sums leave the
  // fp16 range, attention scores ahead of a softmax)
  int y_f32;
  int res_f32;
  // LayerNorm folded into the GEMM (LNS kernels): A holds the raw rows x, W
  // the weight with gamma folded into its K columns; the epilogue forms
  // rstd * acc - rstd * mean * ln_c1[col] + ln_c2[col] with the row's
  // statistics accumulated in the K loop (mean = sum x / K,
  // var = max(sum x^2 / K - mean^2, 0), rstd = 1 / sqrt(var + ln_eps))
  const float* ln_c1;
  const float* ln_c2;
  float ln_invk;
  float ln_eps;
  // GroupNorm chunk statistics of the fp16 output (common.hpp): written to
  // gn_stats[n][chunk][col] when non-null, gn_hw output rows per sample (a
  // multiple of 64), gn_chunks = gn_hw / 64
  float2* gn_stats;
  int gn_hw;
  int gn_chunks;
};

// ---------------------------------------------------------------------------
// A/B operand loaders.  Each thread owns V 16-byte vectors of a 64-wide K
// slice: vector i covers row (tid/8 + i*NT/8), halfs [8*(tid%8), +8).
// Loads are raw buffer loads: a masked-off vector (tail row, tail K, zero
// padding of the conv) gets an offset past the buffer end and reads zeros,
// so the loaders have no branches and the compiler can keep several slices'
// loads in flight with exact wait counts.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kOOB = (int)0x80000000;  // any offset >= the buffer size reads 0

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Branch-free choice between two wave-uniform values.  Written as
// arithmetic: a select between two fields of one struct is otherwise turned
// into an indexed load, which forces the struct into scratch memory.
__device__ __forceinline__ int pick(bool c, int a, int b) { return b + (int)c * (a - b); }
__device__ __forceinline__ unsigned pick(bool c, unsigned a, unsigned b) {
  return b + (unsigned)c * (a - b);
}
__device__ __forceinline__ const f16* pick(bool c, const f16* a, const f16* b) {
  const uint64_t ua = (uint64_t)a, ub = (uint64_t)b;
  return (const f16*)(ub + (uint64_t)c * (ua - ub));
}

__device__ __forceinline__ u32x4 buffer_load16(rsrc_t r, int byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}

struct RowDesc {
  const f16* p;
  int ld;
  int rows;
  int K;
  unsigned bytes;  // rows * ld * 2

  template <int BM, int NT>
  struct Loader {
    static constexpr int V = BM * BK / 8 / NT;
    rsrc_t rs;
    int ld, rows, K, row0, cv;
    __device__ Loader(const RowDesc& d, int r0, int tid)
        : rs(make_rsrc(d.p, d.bytes)), ld(d.ld), rows(d.rows), K(d.K), row0(r0 + tid / 8),
          cv(tid % 8) {}
    __device__ __forceinline__ void load(int kt, u32x4 (&r)[V]) const {
      const int k = kt * BK + cv * 8;
      const bool kin = k < K;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int row = row0 + i * (NT / 8);
        const int off = (row < rows && kin) ? (row * ld + k) * 2 : kOOB;
        r[i] = buffer_load16(rs, off);
      }
    }
  };
};

struct ConvParams {
  // segment 0: KHxKW conv over concat(src0a[:C0a], src0b[:C0-C0a])
  const f16* s0a;
  const f16* s0b;
  int C0a, C0, ld0a, ld0b;
  int H, W;    // stored source resolution
  int Hv, Wv;  // resolution the taps index (2H x 2W when upsampling)
  int KH, KW, stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, up;  // up: stride 1, dil 1 only
  int K0;      // KH*KW*C0
  // segment 1: 1x1 conv over concat(src1a[:C1a], src1b[:C1-C1a]) at output res
  const f16* s1a;
  const f16* s1b;
  int C1a, C1, ld1a, ld1b;
  int HoWo, Wo, M;
  int generic;  // 1 when C0 is not a multiple of 64 (per-vector tap decode, no concat)
  unsigned bytes0a, bytes0b, bytes1a, bytes1b;
};

struct ConvDesc : ConvParams {
  template <int BM, int NT>
  struct Loader {
    static constexpr int V = BM * BK / 8 / NT;
    ConvParams d;
    int pbase[V], ihb[V], iwb[V];
    int row0, cv;
    __device__ Loader(const ConvDesc& desc, int m0, int tid) : d(desc) {
      cv = tid % 8;
      row0 = m0 + tid / 8;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const int m = row0 + i * (NT / 8);
        if (m < d.M) {
          const int n = m / d.HoWo;
          const int p = m - n * d.HoWo;
          const int oh = p / d.Wo;
          const int ow = p - oh * d.Wo;
          pbase[i] = n * d.H * d.W;
          ihb[i] = oh * d.stride_h - d.pad_h;
          iwb[i] = ow * d.stride_w - d.pad_w;
        } else {
          pbase[i] = -1;
          ihb[i] = 0;
          iwb[i] = 0;
        }
      }
    }
    __device__ __forceinline__ void load(int kt, u32x4 (&r)[V]) const {
      const int k0 = kt * BK;
      int off[V];
      rsrc_t rs;
      if (k0 < d.K0) {
        int kh, kw, ld, cc;
        bool kin = true;
        if (!d.generic) {
          // one tap per K slice (C0 % 64 == 0), channel blocks outermost:
          // tap and channel are wave-uniform
          const int taps = d.KH * d.KW;
          const int cb = kt / taps;
          const int tap = kt - cb * taps;
          const int c = cb * BK;
          kh = tap / d.KW;
          kw = tap - kh * d.KW;
          const bool isa = c < d.C0a;
          // select pointer and size, then build the descriptor (a select on
          // descriptor values is lowered through scratch memory)
          rs = make_rsrc(pick(isa, d.s0a, d.s0b), pick(isa, d.bytes0a, d.bytes0b));
          ld = pick(isa, d.ld0a, d.ld0b);
          cc = pick(isa, c, c - d.C0a) + cv * 8;
        } else {
          // small-channel convs (conv_in): decode the tap per 8-channel vector
          const int k = k0 + cv * 8;
          kin = k < d.K0;
          const int tap = kin ? k / d.C0 : 0;
          cc = k - tap * d.C0;
          kh = tap / d.KW;
          kw = tap - kh * d.KW;
          rs = make_rsrc(d.s0a, d.bytes0a);
          ld = d.ld0a;
        }
#pragma unroll
        for (int i = 0; i < V; ++i) {
          int ih = ihb[i] + kh * d.dil_h, iw = iwb[i] + kw * d.dil_w;
          const bool ok = kin && pbase[i] >= 0 && (unsigned)ih < (unsigned)d.Hv &&
                          (unsigned)iw < (unsigned)d.Wv;
          if (d.up) {
            ih >>= 1;
            iw >>= 1;
          }
          off[i] = ok ? ((pbase[i] + ih * d.W + iw) * ld + cc) * 2 : kOOB;
        }
      } else {
        // segment 1 (1x1 over the block input at output resolution); the
        // a/b split is 64-aligned so the source is wave-uniform
        const int cs = k0 - d.K0;
        const bool isa = cs < d.C1a;
        rs = make_rsrc(pick(isa, d.s1a, d.s1b), pick(isa, d.bytes1a, d.bytes1b));
        const int ld = pick(isa, d.ld1a, d.ld1b);
        const int c = pick(isa, cs, cs - d.C1a) + cv * 8;
        const bool cin = cs + cv * 8 < d.C1;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const int m = row0 + i * (NT / 8);
          off[i] = (cin && m < d.M) ? (m * ld + c) * 2 : kOOB;
        }
      }
#pragma unroll
      for (int i = 0; i < V; ++i) r[i] = buffer_load16(rs, off[i]);
    }
  };
};

// ---------------------------------------------------------------------------
// Tile scheduling: spread consecutive logical tiles over one XCD (the
// hardware deals workgroup i to XCD i % 8, each XCD has its own L2), then
// walk logical tiles in groups of 8 M-tiles so co-resident tiles share both
// operand panels.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int q = total >> 3, r = total & 7;
  const int x = bid & 7, slot = bid >> 3;
  const int logical = x * q + (x < r ? x : r) + slot;
  constexpr int GM = 8;
  const int per_group = GM * tiles_n;
  const int g = logical / per_group;
  const int first_m = g * GM;
  const int gsz = min(tiles_m - first_m, GM);
  const int rem = logical - g * per_group;
  tm = first_m + rem % gsz;
  tn = rem / gsz;
}

// Epilogue of one 32x32 accumulator block: lane owns column `col`, element
// e is row row0 + mfma_row(e, lane).  Kept as a separate inlined function
// whose 16-element loop always unrolls, so the accumulators stay in registers.
__device__ __forceinline__ void epilogue_tile(const f32x16& a, int row0, int col, int lane,
                                              const EpiArgs& ep) {
  const bool col_ok = col < ep.N;
  const float bcol = (ep.bias && col_ok) ? (float)ep.bias[col] : 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int row = row0 + mfma_row(e, lane);
    if (col_ok && row < ep.M) {
      float v = a[e] * ep.alpha + bcol;
      int n = 0, p = row;
      if (ep.rows_per_sample > 0) {
        n = row / ep.rows_per_sample;
        p = row - n * ep.rows_per_sample;
      }
      if (ep.tbias) v += (float)ep.tbias[(size_t)n * ep.tbias_ld + col];
      if (ep.act == DLM_ACT_SILU) v = silu_f(v);
      else if (ep.act == DLM_ACT_GELU) v = gelu_erf_f(v);
      if (ep.res) {
        const size_t ri = (size_t)row * ep.ldr + col;
        v += ep.beta * (ep.res_f32 ? reinterpret_cast<const float*>(ep.res)[ri] : (float)ep.res[ri]);
      }
      const size_t yi = ep.out_nchw ? ((size_t)n * ep.N + col) * ep.rows_per_sample + p
                                    : (size_t)row * ep.ldy + col;
      if (ep.y_f32)
        reinterpret_cast<float*>(ep.y)[yi] = v;
      else
        ep.y[yi] = (f16)v;
    }
  }
}

// GEGLU epilogue of one 32x32 accumulator block.  The packed weight
// interleaves value and gate rows in groups of 4 (see geglu_pack_kernel), so
// packed column c is a value when (c & 4) == 0 and its gate is column c ^ 4,
// held by lane ^ 4 in this layout (lane owns column `col`).  Every lane takes
// part in the exchange; value lanes write output column (c / 8) * 4 + c % 4.
__device__ __forceinline__ void epilogue_geglu_tile(const f32x16& a, int row0, int col, int lane,
                                                    const EpiArgs& ep) {
  float partner[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) partner[e] = __shfl_xor(a[e], 4, 64);
  if ((col & 4) || col >= ep.N) return;
  const int ocol = (col >> 3) * 4 + (col & 3);
  const float bv = ep.bias ? (float)ep.bias[col] : 0.0f;
  const float bg = ep.bias ? (float)ep.bias[col + 4] : 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int row = row0 + mfma_row(e, lane);
    if (row < ep.M) {
      float v = (a[e] * ep.alpha + bv) * gelu_erf_f(partner[e] * ep.alpha + bg);
      if (ep.res) v += ep.beta * (float)ep.res[(size_t)row * ep.ldr + ocol];
      ep.y[(size_t)row * ep.ldy + ocol] = (f16)v;
    }
  }
}

template <int BM, int BN, int WM, int WN, bool DEEP, class Desc>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
mfma_gemm_kernel(Desc ad, RowDesc bd, EpiArgs ep, int tiles_m, int tiles_n) {
  constexpr int WAVES_N = BN / WN;
  constexpr int NT = (BM / WM) * WAVES_N * 64;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int AV = BM * BK / 8 / NT;
  constexpr int BV = BN * BK / 8 / NT;
  static_assert(AV * NT * 8 == BM * BK && BV * NT * 8 == BN * BK, "tile/thread mismatch");
  // DEEP: two slices in flight in registers (one otherwise)
  constexpr bool kDeep = DEEP;
  constexpr int STAGE = (BM + BN) * LS;
  __shared__ __attribute__((aligned(16))) f16 smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  int tmi, tni;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;

  typename Desc::template Loader<BM, NT> al(ad, m0, tid);
  RowDesc::Loader<BN, NT> bl(bd, n0, tid);
  const int K = bd.K;
  const int nk = (K + BK - 1) / BK;
  const int last = nk - 1;

  // Pipeline: LDS holds slice kt (double-buffered); two register sets hold
  // slices kt+1 and kt+2 in flight, so each global load has two slices of
  // MFMA work to land.  Loads past the end re-read the last slice (clamped)
  // so every load and wait count stays unconditional.
  u32x4 ra0[AV], rb0[BV];
  u32x4 ra1[kDeep ? AV : 1], rb1[kDeep ? BV : 1];
  auto stage_lds = [&](int buf, const u32x4(&ra)[AV], const u32x4(&rb)[BV]) {
    f16* As = smem + buf * STAGE;
    f16* Bs = As + BM * LS;
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int v = tid + i * NT;
      *reinterpret_cast<u32x4*>(As + (v >> 3) * LS + (v & 7) * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int v = tid + i * NT;
      *reinterpret_cast<u32x4*>(Bs + (v >> 3) * LS + (v & 7) * 8) = rb[i];
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int a_row = wm * WM + (lane & 31);
  const int b_row = wn * WN + (lane & 31);
  const int k_off = (lane >> 5) * 8;
  // Fragment registers are double-buffered across the four 16-wide k-steps of
  // a slice: the ds_reads of step s+1 are issued before the MFMAs of step s,
  // and the staging of the next slice into the other LDS buffer is spread
  // over the first two steps, so LDS traffic overlaps the MFMA pipe instead
  // of alternating with it.
  f16x8 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
  auto rd = [&](int buf, int ks, f16x8 (&fa)[TM], f16x8 (&fb)[TN]) {
    const f16* As = smem + buf * STAGE;
    const f16* Bs = As + BM * LS;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      fa[i] = *reinterpret_cast<const f16x8*>(As + (a_row + i * 32) * LS + ks * 16 + k_off);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      fb[j] = *reinterpret_cast<const f16x8*>(Bs + (b_row + j * 32) * LS + ks * 16 + k_off);
  };
  auto mm = [&](const f16x8 (&fa)[TM], const f16x8 (&fb)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16(fa[i], fb[j], acc[i][j]);
  };
  // write half `part` of the staged registers into LDS buffer `buf`
  auto stage_half = [&](int buf, const u32x4(&ra)[AV], const u32x4(&rb)[BV], int part) {
    f16* As = smem + buf * STAGE;
    f16* Bs = As + BM * LS;
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      if ((i * 2 < AV) == (part == 0)) {
        const int v = tid + i * NT;
        *reinterpret_cast<u32x4*>(As + (v >> 3) * LS + (v & 7) * 8) = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      if ((i * 2 < BV) == (part == 0)) {
        const int v = tid + i * NT;
        *reinterpret_cast<u32x4*>(Bs + (v >> 3) * LS + (v & 7) * 8) = rb[i];
      }
    }
  };
  // one K slice from LDS buffer `buf` (step-0 fragments already in fa0/fb0),
  // staging ra/rb into buffer `nbuf`; leaves step 0 of nothing in flight
  auto slice = [&](int buf, int nbuf, const u32x4(&ra)[AV], const u32x4(&rb)[BV], bool stage) {
    rd(buf, 1, fa1, fb1);
    mm(fa0, fb0);
    if (stage) stage_half(nbuf, ra, rb, 0);
    rd(buf, 2, fa0, fb0);
    mm(fa1, fb1);
    if (stage) stage_half(nbuf, ra, rb, 1);
    rd(buf, 3, fa1, fb1);
    mm(fa0, fb0);
    mm(fa1, fb1);
  };

  al.load(0, ra0);
  bl.load(0, rb0);
  stage_lds(0, ra0, rb0);
  if constexpr (!kDeep) {
    // one slice in flight: enough when a slice carries >= 32 MFMAs per wave
    al.load(min(1, last), ra0);
    bl.load(min(1, last), rb0);
    __syncthreads();
    rd(0, 0, fa0, fb0);
    int kt = 0;
    for (; kt < last; ++kt) {
      const int cur = kt & 1;
      slice(cur, cur ^ 1, ra0, rb0, true);
      __syncthreads();
      rd(cur ^ 1, 0, fa0, fb0);
      al.load(min(kt + 2, last), ra0);
      bl.load(min(kt + 2, last), rb0);
      __builtin_amdgcn_sched_barrier(0);
    }
    slice(kt & 1, 0, ra0, rb0, false);
  } else {
  al.load(min(1, last), ra1);
  bl.load(min(1, last), rb1);
  al.load(min(2, last), ra0);
  bl.load(min(2, last), rb0);
  __syncthreads();
  rd(0, 0, fa0, fb0);

  // Slices are consumed in pairs by a loop with a single exit (a second exit
  // sharing the latch makes the wait-count analysis treat the newer register
  // set as the older one and drain every load); sched_barrier keeps each
  // load group where it is written instead of letting it sink below the
  // LDS stores of the other set.
  int kt = 0;
  for (; kt + 1 <= last; kt += 2) {
    // even slice: LDS buffer 0 holds kt, ra1 holds kt+1, ra0 holds kt+2
    slice(0, 1, ra1, rb1, true);
    __syncthreads();
    rd(1, 0, fa0, fb0);
    al.load(min(kt + 3, last), ra1);
    bl.load(min(kt + 3, last), rb1);
    __builtin_amdgcn_sched_barrier(0);
    // odd slice: LDS buffer 1 holds kt+1, ra0 holds kt+2, ra1 holds kt+3
    slice(1, 0, ra0, rb0, true);
    __syncthreads();
    rd(0, 0, fa0, fb0);
    al.load(min(kt + 4, last), ra0);
    bl.load(min(kt + 4, last), rb0);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (kt == last) slice(0, 1, ra1, rb1, false);  // odd slice count: buffer 0 holds the last slice
  }

  // ------------------------------ epilogue ------------------------------
  const int row_base = m0 + wm * WM;
  if (ep.act == DLM_ACT_GEGLU) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i)
        epilogue_geglu_tile(acc[i][j], row_base + i * 32, n0 + wn * WN + j * 32 + (lane & 31), lane, ep);
    return;
  }
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i)
      epilogue_tile(acc[i][j], row_base + i * 32, n0 + wn * WN + j * 32 + (lane & 31), lane, ep);
}

// ===========================================================================
// LDS-DMA GEMM core.  Used for every linear whose operands and output are
// suitably aligned and for convolutions whose channel counts are multiples of
// 64 (all of the UNet except conv_in); the kernel above remains the general
// fallback.
//
// Operand staging: global -> LDS directly (buffer_load ... lds), no VGPR
// staging and no ds_write; on gfx950 ds_write_b128 moves ~72 B/clk/CU, half
// of what a tile needs, while the direct path leaves the LDS write port to
// the DMA.  Each 64-wide K slice of a row is 128 contiguous bytes, so every
// L2 request is a full line.  LDS rows are 128 B (no padding) with the
// 16-byte chunks XOR-swizzled by (row >> 1) & 7: the 16 rows one ds_read_b128
// phase touches then cover all 64 banks exactly once.
//
// Pipeline: an NS-slice ring in LDS; slice kt+NS-1 is requested while slice
// kt is consumed; one s_waitcnt vmcnt + s_barrier per slice.  Fragment reads
// of k-step s+1 are issued before the MFMAs of step s.
//
// MFMA: v_mfma_f32_16x16x32_f16.  Measured on 8192^3 with N(0,1) data, the
// 16x16x32 form sustains ~12% more than 32x32x16 in the same loop (the
// 32x32 form's rate drops with data entropy; the 16x16 form's barely does).
// acc = W-fragment x X-fragment, i.e. the transposed product, so a lane
// holds one output row and four consecutive output columns per block: the
// epilogue stores 8 bytes per instruction and reads bias and residual as
// 8-byte vectors.
// ===========================================================================
typedef int i32x4 __attribute__((ext_vector_type(4)));
#define DLM_LDS __attribute__((address_space(3)))

// 128-bit raw-buffer descriptor in SGPRs: base, no stride, byte size
// (offsets at or past it read 0).
__device__ __forceinline__ i32x4 dma_rsrc(const void* p, unsigned bytes) {
  const uint64_t a = (uint64_t)p;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// One wave-wide global -> LDS copy: lane l reads 16 bytes at byte offset voff
// of the buffer and the hardware writes them to LDS at dst + 16 l (dst goes
// through M0).  Issued as inline asm so the compiler neither tracks nor
// drains it: the kernel orders it with explicit vmcnt waits and barriers.
// Nothing else in this file uses M0, so clobbering it is safe although the
// compiler warns that it treats M0 as reserved.
__device__ __forceinline__ void dma16(const i32x4& r, const unsigned char DLM_LDS* dst, int voff) {
  const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)dst);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds),
               "v"(voff), "s"(r)
               : "memory", "m0");
}

// s_waitcnt vmcnt(n), other counters untouched (gfx9 encoding: vmcnt in bits
// [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
#define DLM_WAIT_VM(n) \
  __builtin_amdgcn_s_waitcnt((((n)&15) | (((n) >> 4) << 14)) | (0x7 << 4) | (0xF << 8))

// Lane -> (row, chunk) map of DMA instruction i of wave w (NW waves): row
// group g = i*NW + w of 8 rows x 128 B; lane l covers row 8g + l/8, physical
// chunk l%8, which holds the logical K chunk (l%8) ^ ((row >> 1) & 7).  A
// tile whose row-group count is not a multiple of NW leaves the last
// instruction to the first (groups % NW) waves.
__device__ __forceinline__ int dma_row(int nw, int i, int wave, int lane) {
  return (i * nw + wave) * 8 + (lane >> 3);
}
__device__ __forceinline__ int dma_chunk(int row, int lane) { return (lane & 7) ^ ((row >> 1) & 7); }

template <int I>
struct RowDma {
  i32x4 rs;
  int base[I];  // byte offset of the lane's chunk in K-slice 0, -1 past the last row
  int kc[I];    // K index of that chunk within a slice
  int K;
  __device__ RowDma(const RowDesc& d, int r0, int nw, int wave, int lane)
      : rs(dma_rsrc(d.p, d.bytes)), K(d.K) {
#pragma unroll
    for (int i = 0; i < I; ++i) {
      const int row = dma_row(nw, i, wave, lane);
      const int c = dma_chunk(row, lane);
      kc[i] = c * 8;
      base[i] = r0 + row < d.rows ? ((r0 + row) * d.ld + c * 8) * 2 : -1;
    }
  }
  __device__ __forceinline__ void seek(int) {}
  __device__ __forceinline__ void prepare(int) {}
  __device__ __forceinline__ int off(int i, int kt) const {
    return (base[i] >= 0 && kt * BK + kc[i] < K) ? base[i] + kt * (BK * 2) : kOOB;
  }
};

// Implicit-im2col rows for the DMA path (C0, C0a, C1, C1a multiples of 64:
// one tap and one source per K slice, both wave-uniform).  Every parameter is
// copied into registers (the DMA asm clobbers memory, which would otherwise
// force kernel-argument reloads inside the loop) and the per-lane offset is
// computed with selects only.
__device__ __forceinline__ int rfl(int v) { return __builtin_amdgcn_readfirstlane(v); }

template <int I>
struct ConvDma {
  int pbase[I], ihb[I], iwb[I], mrow[I], cch[I];
  // uniform parameters
  const f16 *s0a, *s0b, *s1a, *s1b;
  unsigned bytes0a, bytes0b, bytes1a, bytes1b;
  int C0, C0a, ld0a, ld0b, C1, C1a, ld1a, ld1b, K0, KH, KW, Hv, Wv, W, up, M, dil_h, dil_w;
  // per-slice state
  i32x4 rs;
  int seg, kh, kw, ld, cbase;
  __device__ ConvDma(const ConvParams& d, int m0, int nw, int wave, int lane)
      : s0a(d.s0a), s0b(d.s0b), s1a(d.s1a), s1b(d.s1b), bytes0a(d.bytes0a), bytes0b(d.bytes0b),
        bytes1a(d.bytes1a), bytes1b(d.bytes1b), C0(d.C0), C0a(d.C0a), ld0a(d.ld0a), ld0b(d.ld0b),
        C1(d.C1), C1a(d.C1a), ld1a(d.ld1a), ld1b(d.ld1b), K0(d.K0), KH(d.KH), KW(d.KW), Hv(d.Hv), Wv(d.Wv),
        W(d.W), up(d.up), M(d.M), dil_h(d.dil_h), dil_w(d.dil_w) {
#pragma unroll
    for (int i = 0; i < I; ++i) {
      const int row = dma_row(nw, i, wave, lane);
      cch[i] = dma_chunk(row, lane) * 8;
      const int m = m0 + row;
      mrow[i] = m;
      const int mm = m < d.M ? m : 0;
      const int n = mm / d.HoWo;
      const int q = mm - n * d.HoWo;
      const int oh = q / d.Wo;
      const int ow = q - oh * d.Wo;
      pbase[i] = m < d.M ? n * d.H * d.W : -1;
      ihb[i] = oh * d.stride_h - d.pad_h;
      iwb[i] = ow * d.stride_w - d.pad_w;
    }
  }
  // Segment-0 K order: 64-channel blocks outermost, then the taps (kh, kw),
  // so the KH*KW slices that re-read one block of a pixel's channels run
  // back to back and find its lines still in the L2.  Slices are requested
  // in order (kb, kb+1, ..., then the last one repeated), so the tap /
  // channel position advances by one slice at a time: no integer division
  // and no branch in the loop (all selects).
  int cur_kt = 0, cur_c = 0, cur_kh = 0, cur_kw = 0;
  // position the tap state at slice kt (start of a split-K range)
  __device__ __forceinline__ void seek(int kt) {
    const int taps = KH * KW;
    const bool s0 = kt * BK < K0;
    const int cb = s0 ? kt / taps : 0;
    const int tap = s0 ? kt - cb * taps : 0;
    cur_kt = kt;
    cur_c = rfl(cb * BK);
    cur_kh = rfl(tap / KW);
    cur_kw = rfl(tap - (tap / KW) * KW);
  }
  __device__ __forceinline__ void prepare(int kt) {
    const bool adv = kt != cur_kt;  // kt == cur_kt + 1
    int kw1 = cur_kw + 1;
    const bool wrapw = kw1 == KW;
    kw1 = wrapw ? 0 : kw1;
    int kh1 = cur_kh + (wrapw ? 1 : 0);
    const bool wraph = kh1 == KH;
    kh1 = wraph ? 0 : kh1;
    const int c1 = cur_c + (wraph ? BK : 0);
    cur_c = rfl(adv ? c1 : cur_c);
    cur_kw = rfl(adv ? kw1 : cur_kw);
    cur_kh = rfl(adv ? kh1 : cur_kh);
    cur_kt = kt;
    const int k0 = kt * BK;
    const bool s1 = k0 >= K0;
    const int cs = k0 - K0;  // segment-1 K index of the slice
    const bool isa0 = cur_c < C0a, isa1 = cs < C1a;
    // arithmetic selects throughout: a ternary between members lets the
    // compiler select their addresses instead, which moves them to scratch
    const f16* src = pick(s1, pick(isa1, s1a, s1b), pick(isa0, s0a, s0b));
    const unsigned bytes = pick(s1, pick(isa1, bytes1a, bytes1b), pick(isa0, bytes0a, bytes0b));
    rs = dma_rsrc(src, bytes);
    ld = rfl(pick(s1, pick(isa1, ld1a, ld1b), pick(isa0, ld0a, ld0b)));
    cbase = rfl(pick(s1, pick(isa1, cs, cs - C1a), pick(isa0, cur_c, cur_c - C0a)));
    kh = rfl(pick(s1, cs, cur_kh * dil_h));  // segment 0: tap offset in input rows
    kw = rfl(pick(s1, 0, cur_kw * dil_w));
    seg = rfl(s1 ? 1 : 0);
  }
  // Both segment offsets are always computed and chosen with arithmetic
  // selects, so the DMA sequence stays free of divergent branches.
  __device__ __forceinline__ int off(int i, int) const {
    int ih = ihb[i] + kh, iw = iwb[i] + kw;
    const bool ok0 = (pbase[i] >= 0) & ((unsigned)ih < (unsigned)Hv) & ((unsigned)iw < (unsigned)Wv);
    ih >>= up;
    iw >>= up;
    const int o0 = ((pbase[i] + ih * W + iw) * ld + cbase + cch[i]) * 2;
    const bool ok1 = (mrow[i] < M) & (kh + cch[i] < C1);
    const int o1 = (mrow[i] * ld + cbase + cch[i]) * 2;
    return pick(seg == 0, pick(ok0, o0, kOOB), pick(ok1, o1, kOOB));
  }
};

template <class Desc>
struct DmaOf;
template <>
struct DmaOf<RowDesc> {
  template <int I>
  using T = RowDma<I>;
};
template <>
struct DmaOf<ConvDesc> {
  template <int I>
  using T = ConvDma<I>;
};

__device__ __forceinline__ f16x4 ld4h(const f16* p) { return *reinterpret_cast<const f16x4*>(p); }

// LayerNorm fold of four accumulators of columns [col, col+4): r = rstd,
// rm = rstd * mean of the row, c1 / c2 the columns' ln_c1 / ln_c2.
__device__ __forceinline__ f32x4 ln_fold4(const f32x4& a, const f32x4& c1, const f32x4& c2, float r,
                                         float rm) {
  f32x4 o;
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = __builtin_fmaf(a[t], r, __builtin_fmaf(-rm, c1[t], c2[t]));
  return o;
}

// Epilogue of four consecutive output columns [col, col+4) of one row.
__device__ __forceinline__ void epi4(const f32x4& a, int row, int col, const EpiArgs& ep) {
  if (row >= ep.M || col >= ep.N) return;
  float v[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) v[t] = a[t] * ep.alpha;
  if (ep.bias) {
    const f16x4 b = ld4h(ep.bias + col);
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] += (float)b[t];
  }
  int n = 0, p = row;
  if (ep.rows_per_sample > 0) {
    n = row / ep.rows_per_sample;
    p = row - n * ep.rows_per_sample;
  }
  if (ep.tbias) {
    const f16x4 b = ld4h(ep.tbias + (size_t)n * ep.tbias_ld + col);
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] += (float)b[t];
  }
  if (ep.act == DLM_ACT_SILU) {
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] = silu_f(v[t]);
  } else if (ep.act == DLM_ACT_GELU) {
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] = gelu_erf_f(v[t]);
  }
  if (ep.res) {
    if (ep.res_f32) {
      const float4 r =
          *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(ep.res) + (size_t)row * ep.ldr + col);
      v[0] += ep.beta * r.x;
      v[1] += ep.beta * r.y;
      v[2] += ep.beta * r.z;
      v[3] += ep.beta * r.w;
    } else {
      const f16x4 r = ld4h(ep.res + (size_t)row * ep.ldr + col);
#pragma unroll
      for (int t = 0; t < 4; ++t) v[t] += ep.beta * (float)r[t];
    }
  }
  if (ep.y_f32) {
    float* y = reinterpret_cast<float*>(ep.y);
    if (ep.out_nchw) {
#pragma unroll
      for (int t = 0; t < 4; ++t) y[((size_t)n * ep.N + col + t) * ep.rows_per_sample + p] = v[t];
    } else {
      *reinterpret_cast<float4*>(y + (size_t)row * ep.ldy + col) = make_float4(v[0], v[1], v[2], v[3]);
    }
  } else if (ep.vt && col >= ep.vt_col0) {
    const int smp = row / ep.vt_tokens;
    const int tok = row - smp * ep.vt_tokens;
    f16* dst = ep.vt + ((size_t)smp * (ep.N - ep.vt_col0) + (col - ep.vt_col0)) * ep.vt_ld + tok;
#pragma unroll
    for (int t = 0; t < 4; ++t) dst[(size_t)t * ep.vt_ld] = (f16)v[t];
    if (tok == ep.vt_tokens - 1)  // the last token also clears the row's padding
      for (int t = 0; t < 4; ++t)
        for (int q = 1; q < ep.vt_ld - tok; ++q) dst[(size_t)t * ep.vt_ld + q] = (f16)0.0f;
  } else if (ep.out_nchw) {
#pragma unroll
    for (int t = 0; t < 4; ++t) ep.y[((size_t)n * ep.N + col + t) * ep.rows_per_sample + p] = (f16)v[t];
  } else {
    const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
    *reinterpret_cast<f16x4*>(ep.y + (size_t)row * ep.ldy + col) = o;
  }
}

// GEGLU epilogue of one 16x16 block.  Value and gate rows of the packed
// weight alternate in groups of 4 (geglu_pack_kernel), so the lane's 4
// packed columns col..col+3 are values when (col & 4) == 0 and the matching
// gates are held by lane ^ 16.  The pair splits the group: the value lane
// computes output columns 0-1 of the group, the gate lane columns 2-3, each
// after one exchange of two values (no lane idles).
__device__ __forceinline__ void epi4_geglu(const f32x4& a, int row, int col, const EpiArgs& ep) {
  const bool is_gate = (col & 4) != 0;
  // value lane sends values 2-3, gate lane sends gates 0-1
  const float r0 = __shfl_xor(is_gate ? a[0] : a[2], 16, 64);
  const float r1 = __shfl_xor(is_gate ? a[1] : a[3], 16, 64);
  const int vcol = col & ~4;            // packed column of value 0 of the group
  const int t0 = is_gate ? 2 : 0;       // group columns this lane computes
  if (row >= ep.M || vcol >= ep.N) return;
  float v[2], g[2];
  v[0] = (is_gate ? r0 : a[0]) * ep.alpha;
  v[1] = (is_gate ? r1 : a[1]) * ep.alpha;
  g[0] = (is_gate ? a[2] : r0) * ep.alpha;
  g[1] = (is_gate ? a[3] : r1) * ep.alpha;
  if (ep.bias) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      v[t] += (float)ep.bias[vcol + t0 + t];
      g[t] += (float)ep.bias[vcol + 4 + t0 + t];
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) v[t] *= gelu_erf_fast(g[t]);  // A&S erf: -0.25 ms per UNet step
  const int ocol = (vcol >> 1) + t0;
  if (ep.res) {
#pragma unroll
    for (int t = 0; t < 2; ++t) v[t] += ep.beta * (float)ep.res[(size_t)row * ep.ldr + ocol + t];
  }
  f16 o2[2] = {(f16)v[0], (f16)v[1]};
  *reinterpret_cast<uint32_t*>(ep.y + (size_t)row * ep.ldy + ocol) = *reinterpret_cast<uint32_t*>(o2);
}

// Whole-tile epilogues of a wave's TM x TN blocks (lane: row (lane & 15) of
// block i, columns 4 (lane >> 4) + [0, 4) of block j) for fp16 row-major
// output.  Every bias / time-bias / residual load is issued before the first
// use, at addresses clamped into the tensors, so the wave waits on memory
// once; per block, the loads, guards and stores of epi4 (one round trip per
// operand and block) made the epilogue several times longer.  The arithmetic
// is epi4's, in the same order.
__host__ __device__ __forceinline__ bool epi_tile_fast(const EpiArgs& ep) {
  return !ep.y_f32 && !ep.res_f32 && !ep.out_nchw && !ep.vt;
}

// Bias and residual of the wave tile, loaded unconditionally (a missing
// operand reads the output tile instead, never used): exactly TN + TM TN
// loads, so a K loop that issues them before its last waits can count them.
template <int TM, int TN>
__device__ __forceinline__ void epi_tile_early(int row0, int col0, const EpiArgs& ep, f16x4 (&bv)[TN],
                                               f16x4 (&rv)[TM][TN]) {
  const f16* bp = ep.bias ? ep.bias : ep.y;
#pragma unroll
  for (int j = 0; j < TN; ++j) bv[j] = ld4h(bp + min(col0 + j * 16, ep.N - 4));
  const f16* rp = ep.res ? ep.res : ep.y;
  const int ld = ep.res ? ep.ldr : ep.ldy;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int r = min(row0 + i * 16, ep.M - 1);
#pragma unroll
    for (int j = 0; j < TN; ++j) rv[i][j] = ld4h(rp + (size_t)r * ld + min(col0 + j * 16, ep.N - 4));
  }
}

// EARLY: bias and residual already in bv / rv (epi_tile_early).
// to_lds: stl is this lane's position in an LDS copy of the workgroup's
// output tile (row stride sld halfs), which receives the stored fp16 values
// (a flag, not a null test: LDS address 0 is a valid position).
template <int TM, int TN, bool EARLY = false>
__device__ __forceinline__ void epi_tile(const f32x4 (&acc)[TM][TN], int row0, int col0, const EpiArgs& ep,
                                         f16x4 (&bv)[TN], f16x4 (&rv)[TM][TN], bool to_lds = false,
                                         f16 DLM_LDS* stl = nullptr, int sld = 0) {
  f16x4 tv[TM][TN];
  if (!EARLY && ep.bias) {
#pragma unroll
    for (int j = 0; j < TN; ++j) bv[j] = ld4h(ep.bias + min(col0 + j * 16, ep.N - 4));
  }
  if (ep.tbias) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = min(row0 + i * 16, ep.M - 1);
      const int n = ep.rows_per_sample > 0 ? r / ep.rows_per_sample : 0;
#pragma unroll
      for (int j = 0; j < TN; ++j) tv[i][j] = ld4h(ep.tbias + (size_t)n * ep.tbias_ld + min(col0 + j * 16, ep.N - 4));
    }
  }
  if (!EARLY && ep.res) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = min(row0 + i * 16, ep.M - 1);
#pragma unroll
      for (int j = 0; j < TN; ++j) rv[i][j] = ld4h(ep.res + (size_t)r * ep.ldr + min(col0 + j * 16, ep.N - 4));
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = row0 + i * 16;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = col0 + j * 16;
      float v[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) v[t] = acc[i][j][t] * ep.alpha;
      if (ep.bias) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] += (float)bv[j][t];
      }
      if (ep.tbias) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] += (float)tv[i][j][t];
      }
      if (ep.act == DLM_ACT_SILU) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = silu_f(v[t]);
      } else if (ep.act == DLM_ACT_GELU) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = gelu_erf_f(v[t]);
      }
      if (ep.res) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] += ep.beta * (float)rv[i][j][t];
      }
      const f16x4 o = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
      if (row < ep.M && col < ep.N) *reinterpret_cast<f16x4*>(ep.y + (size_t)row * ep.ldy + col) = o;
      if (to_lds) *reinterpret_cast<f16x4 DLM_LDS*>(stl + i * 16 * sld + j * 16) = o;
    }
  }
}

// GroupNorm chunk statistics (common.hpp) of a BM x BN output tile held in
// LDS (row stride BN): one thread per (64-row chunk, column), the chunk's
// rows in ascending order.  Needs ep.gn_hw % 64 == 0, so a chunk that starts
// inside M lies inside it.
template <int BM, int BN>
__device__ __forceinline__ void gn_tile_stats(const f16 DLM_LDS* st, int m0, int n0, const EpiArgs& ep,
                                              int tid, int nt) {
  constexpr int PAIRS = (BM / kGnChunk) * BN;
  for (int p = tid; p < PAIRS; p += nt) {
    const int kk = p / BN, c = p - kk * BN;
    const int grow = m0 + kk * kGnChunk, gcol = n0 + c;
    if (grow >= ep.M || gcol >= ep.N) continue;
    const f16 DLM_LDS* col = st + kk * kGnChunk * BN + c;
    const float shift = (float)col[0];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll 16
    for (int r = 0; r < kGnChunk; ++r) gn_stat_add((float)col[r * BN], shift, s1, s2);
    const int n = grow / ep.gn_hw, k = (grow - n * ep.gn_hw) / kGnChunk;
    ep.gn_stats[((size_t)n * ep.gn_chunks + k) * ep.N + gcol] = gn_stat_finish(s1, s2, shift, kGnChunk);
  }
}

// GEGLU form of epi_tile.  The value lanes of a pair (see epi4_geglu) are
// the even 16-lane rows of the wave (packed column 4 (lane >> 4) of a block
// is a value column when lane >> 4 is even, since tile and block origins are
// multiples of 16), the gate lanes the odd rows; one v_permlane16_swap per
// accumulator pair (0, 2) and (1, 3) leaves every lane holding the values and
// gates of its own two output columns, with no select and no LDS traffic.
// FULL: the wave tile lies inside M x N, so no store needs a guard and the
// blocks' independent GELU chains can interleave.
template <int TM, int TN, bool FULL>
__device__ __forceinline__ void epi_tile_geglu(const f32x4 (&acc)[TM][TN], int row0, int col0,
                                               const EpiArgs& ep) {
  const bool is_gate = (col0 & 4) != 0;
  const int t0 = is_gate ? 2 : 0;
  f16x2 bvv[TN], bgg[TN], rv[TM][TN];
  if (ep.bias) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int vc = min((col0 + j * 16) & ~4, ep.N - 8);
      bvv[j] = *reinterpret_cast<const f16x2*>(ep.bias + vc + t0);
      bgg[j] = *reinterpret_cast<const f16x2*>(ep.bias + vc + 4 + t0);
    }
  }
  if (ep.res) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = min(row0 + i * 16, ep.M - 1);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int oc = (min((col0 + j * 16) & ~4, ep.N - 8) >> 1) + t0;
        rv[i][j] = *reinterpret_cast<const f16x2*>(ep.res + (size_t)r * ep.ldr + oc);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = row0 + i * 16;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const f32x4& a = acc[i][j];
      const auto s02 = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[0]), __float_as_uint(a[2]), false, false);
      const auto s13 = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[1]), __float_as_uint(a[3]), false, false);
      const int vcol = (col0 + j * 16) & ~4;
      float v[2], g[2];
      v[0] = __uint_as_float(s02[0]) * ep.alpha;
      v[1] = __uint_as_float(s13[0]) * ep.alpha;
      g[0] = __uint_as_float(s02[1]) * ep.alpha;
      g[1] = __uint_as_float(s13[1]) * ep.alpha;
      if (ep.bias) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          v[t] += (float)bvv[j][t];
          g[t] += (float)bgg[j][t];
        }
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) v[t] *= gelu_erf_fast(g[t]);
      if (ep.res) {
#pragma unroll
        for (int t = 0; t < 2; ++t) v[t] += ep.beta * (float)rv[i][j][t];
      }
      f16 o2[2] = {(f16)v[0], (f16)v[1]};
      uint32_t* dst = reinterpret_cast<uint32_t*>(ep.y + (size_t)row * ep.ldy + (vcol >> 1) + t0);
      if (FULL || (row < ep.M && vcol < ep.N)) *dst = *reinterpret_cast<uint32_t*>(o2);
    }
  }
}

// Split-K: the K slices of a tile are divided into S ranges of kps slices,
// one workgroup each.  Every split stores its fp32 accumulators (agent-scope
// stores, so the data is visible device-wide once the store is counted
// complete), then bumps the tile's counter; the split that sees S-1 is the
// last: it adds the partials in split order 0..S-1 (its own from registers),
// so the result does not depend on arrival order, resets the counter for
// the next launch and runs the epilogue.  No workgroup ever waits on another.
struct SplitArgs {
  int S;      // splits per tile (1 = no split)
  int kps;    // K slices per split
  float* ws;  // partials: [tile][split][BM*BN] in accumulator-register order
  int* cnt;   // per-tile arrival counters, zero between launches
};

// blockIdx -> (tile, split) for S > 1: every split of a tile on one XCD
// (workgroup b runs on XCD b % 8), XCDs own contiguous logical tile ranges,
// logical tiles walk groups of 8 M-tiles as in tile_coords.  tm < 0 marks a
// padding workgroup.
__device__ __forceinline__ void split_coords(int bid, int tiles_m, int tiles_n, int S, int& tm,
                                             int& tn, int& sidx) {
  const int total = tiles_m * tiles_n;
  const int q = (total + 7) >> 3;
  const int x = bid & 7, slot = bid >> 3;
  const int local = slot / S;
  sidx = slot - local * S;
  const int logical = x * q + local;
  if (local >= q || logical >= total) {
    tm = -1;
    tn = 0;
    return;
  }
  constexpr int GM = 8;
  const int per_group = GM * tiles_n;
  const int g = logical / per_group;
  const int first_m = g * GM;
  const int gsz = min(tiles_m - first_m, GM);
  const int rem = logical - g * per_group;
  tm = first_m + rem % gsz;
  tn = rem / gsz;
}

// PF: the first k-step's fragments of slice kt+1 are read from LDS right
// after the barrier that publishes it, while the second k-step of slice kt
// (already in registers) runs on the MFMA pipe; the whole ring is filled
// before the loop and slot kt is refilled (with slice kt+NS) as soon as that
// barrier proves every wave has read it.
// SPS > 1: a ring stage holds SPS consecutive K slices published by one
// barrier (fewer barriers and exposed first reads per slice); slices past the
// range end are loaded clamped and skipped by the MFMAs.
// LNS: LayerNorm folded in (EpiArgs::ln_*): every wave sums x and x^2 of its
// rows from the A fragments it multiplies (two v_dot2 per 4 halves, fp32
// accumulation of exact fp16 products); the four lanes that hold one row's
// K chunks combine their sums after the loop.  No split-K.
template <int BM, int BN, int WM, int WN, int NS, bool PF, int SPS, bool LNS, class Desc>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
dma_gemm_kernel(Desc ad, RowDesc bd, EpiArgs ep, int tiles_m, int tiles_n, SplitArgs sp) {
  constexpr int WAVES_N = BN / WN;
  constexpr int NW = (BM / WM) * WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;  // 16x16 MFMA blocks per wave
  constexpr int KS = BK / 32;                // 32-deep k-steps per slice
  constexpr int SA = BM * BK * 2;
  constexpr int SLICE = (BM + BN) * BK * 2;  // one K slice of both operands
  constexpr int STAGE = SLICE * SPS;
  constexpr int GA = BM / 8, GB = BN / 8;    // 8-row DMA groups per operand tile
  constexpr int IA = (GA + NW - 1) / NW, IB = (GB + NW - 1) / NW;  // DMA instructions per wave
  static_assert(BM % 8 == 0 && BN % 8 == 0 && WM % 16 == 0 && WN % 16 == 0, "tile shape");
  static_assert(NS >= 2, "at least two slices");
  static_assert(SPS == 1 || !PF, "multi-slice stages use the plain loop");
  __shared__ __attribute__((aligned(1024))) unsigned char smem_generic[NS * STAGE];
  unsigned char DLM_LDS* smem = (unsigned char DLM_LDS*)smem_generic;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  int tmi, tni, sidx = 0;
  if (sp.S > 1) {
    split_coords(blockIdx.x, tiles_m, tiles_n, sp.S, tmi, tni, sidx);
    if (tmi < 0) return;
  } else {
    tile_coords(blockIdx.x, tiles_m, tiles_n, tmi, tni);
  }
  const int m0 = tmi * BM, n0 = tni * BN;

  typename DmaOf<Desc>::template T<IA> al(ad, m0, NW, wave, lane);
  RowDma<IB> bl(bd, n0, NW, wave, lane);
  const int nk_all = (bd.K + BK - 1) / BK;
  const int kb = sidx * sp.kps;
  const int ke = min(nk_all, kb + sp.kps);
  al.seek(kb);

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float ln_s1[LNS ? TM : 1], ln_s2[LNS ? TM : 1];
#pragma unroll
  for (int i = 0; i < (LNS ? TM : 1); ++i) ln_s1[i] = ln_s2[i] = 0.0f;
  // row sums of x and x^2 over one k-step's A fragments
  auto ln_acc = [&](const f16x8* fa) {
    if constexpr (LNS) {
      const f16x2 one2 = f16x2{(f16)1.0f, (f16)1.0f};
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const f16x2 x2 = f16x2{fa[i][2 * h], fa[i][2 * h + 1]};
          ln_s1[i] = __builtin_amdgcn_fdot2(x2, one2, ln_s1[i], false);
          ln_s2[i] = __builtin_amdgcn_fdot2(x2, x2, ln_s2[i], false);
        }
    }
  };

  // 16-row operand fragment of k-step ks: lane holds row (lane & 15), k
  // chunk 4 ks + (lane >> 4) (the 16x16x32 MFMA operand layout).
  auto frag = [&](const unsigned char DLM_LDS* st, int row, int ks) -> f16x8 {
    const int c = (4 * ks + (lane >> 4)) ^ ((row >> 1) & 7);
    return *reinterpret_cast<const f16x8 DLM_LDS*>(st + row * 128 + c * 16);
  };
  // DMA instruction i of this wave for the A / B tile (skipped by the waves
  // past the last row group)
  auto dma_a = [&](unsigned char DLM_LDS* st, int i, int kt) {
    if (IA * NW == GA || i + 1 < IA || wave < GA - (IA - 1) * NW)
      dma16(al.rs, st + (i * NW + wave) * 1024, al.off(i, kt));
  };
  auto dma_b = [&](unsigned char DLM_LDS* st, int i, int kt) {
    if (IB * NW == GB || i + 1 < IB || wave < GB - (IB - 1) * NW)
      dma16(bl.rs, st + SA + (i * NW + wave) * 1024, bl.off(i, kt));
  };
  auto issue_all = [&](int buf, int kt) {
    unsigned char DLM_LDS* st = smem + buf * STAGE;
    al.prepare(kt);
#pragma unroll
    for (int i = 0; i < IA; ++i) dma_a(st, i, kt);
#pragma unroll
    for (int i = 0; i < IB; ++i) dma_b(st, i, kt);
  };

  // Early epilogue loads (two-slice-stage loop, residual linears): the bias
  // and residual of the wave tile are requested once the last real refill
  // is issued, so their latency passes under the last stages' MFMAs; the
  // refills past the end are then skipped and the tail's waits count them.
  const int erow0 = m0 + wm * WM + (lane & 15);
  const int ecol0 = n0 + wn * WN + 4 * (lane >> 4);
  f16x4 ebv[TN], erv[TM][TN];
  bool early = false;

  constexpr int PRE = SPS > 1 ? 0 : (PF ? NS : NS - 1);  // slices in flight before the loop
#pragma unroll
  for (int s = 0; s < PRE; ++s) issue_all(s, min(kb + s, ke - 1));

  // DMA instructions this wave skips per slice (0..2): the vmcnt wait for
  // "slice kt landed" allows P later slices of this wave's own requests
  const int skips = ((IA * NW == GA || wave < GA - (IA - 1) * NW) ? 0 : 1) +
                    ((IB * NW == GB || wave < GB - (IB - 1) * NW) ? 0 : 1);
#define DLM_WAIT_SLICES(P)                   \
  do {                                       \
    if (skips == 0) {                        \
      DLM_WAIT_VM((P) * (IA + IB));          \
    } else if (skips == 1) {                 \
      DLM_WAIT_VM((P) * (IA + IB - 1));      \
    } else {                                 \
      DLM_WAIT_VM((P) * (IA + IB - 2));      \
    }                                        \
  } while (0)
  // P slices of DMA plus E other loads may still be outstanding
#define DLM_WAIT_SLICES_PLUS(P, E)                \
  do {                                            \
    if (skips == 0) {                             \
      DLM_WAIT_VM((P) * (IA + IB) + (E));         \
    } else if (skips == 1) {                      \
      DLM_WAIT_VM((P) * (IA + IB - 1) + (E));     \
    } else {                                      \
      DLM_WAIT_VM((P) * (IA + IB - 2) + (E));     \
    }                                             \
  } while (0)
  if constexpr (SPS > 1) {
    static_assert(KS == 2, "multi-slice stages assume two k-steps per slice");
    const int nsteps = (ke - kb + SPS - 1) / SPS;
    auto slice_kt = [&](int t, int j) { return min(kb + t * SPS + j, ke - 1); };
#pragma unroll
    for (int t = 0; t < NS - 1; ++t)
#pragma unroll
      for (int j = 0; j < SPS; ++j) {
        unsigned char DLM_LDS* dst = smem + t * STAGE + j * SLICE;
        const int kt = slice_kt(t, j);
        al.prepare(kt);
#pragma unroll
        for (int i = 0; i < IA; ++i) dma_a(dst, i, kt);
#pragma unroll
        for (int i = 0; i < IB; ++i) dma_b(dst, i, kt);
      }
    // t_e: first stage whose refill would lie past the end (every real
    // stage's DMA is issued before it)
    const int t_e = nsteps - (NS - 1);
    if constexpr (TM * TN <= 20)
      early = sp.S == 1 && t_e >= 1 && ep.res && !ep.tbias && ep.act != DLM_ACT_GEGLU && epi_tile_fast(ep);
    int slot = 0, nslot = NS - 1;  // stage being read, stage being refilled
    for (int t = 0; t < nsteps; ++t) {
      if (early && t > t_e) {
        // newer than stage t: the DMA of stages t+1 .. nsteps-1 and the
        // TN + TM TN early loads
        static_assert(NS <= 4, "tail waits written out for rings of up to four stages");
        if (nsteps - 1 - t == 0) {
          DLM_WAIT_SLICES_PLUS(0, TN + TM * TN);
        } else {
          DLM_WAIT_SLICES_PLUS(SPS, TN + TM * TN);
        }
      } else {
        DLM_WAIT_SLICES((NS - 2) * SPS);  // stage t landed (this wave's part)
      }
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if (early && t == t_e) epi_tile_early<TM, TN>(erow0, ecol0, ep, ebv, erv);
      const bool refill = !early || t < t_e;
      const unsigned char DLM_LDS* st = smem + slot * STAGE;
      unsigned char DLM_LDS* nst = smem + nslot * STAGE;
      f16x8 fa[2][TM], fb[2][TN];
      auto rd = [&](int q) {  // k-step q of the stage: slice q / KS, step q % KS
        const unsigned char DLM_LDS* sl = st + (q / KS) * SLICE;
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[q & 1][i] = frag(sl, wm * WM + i * 16 + (lane & 15), q % KS);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[q & 1][j] = frag(sl + SA, wn * WN + j * 16 + (lane & 15), q % KS);
      };
      rd(0);
#pragma unroll
      for (int q = 0; q < SPS * KS; ++q) {
        __builtin_amdgcn_sched_barrier(0);
        if (q + 1 < SPS * KS) rd(q + 1);
        // refill of stage t+NS-1: slice r's A rows at k-step 2r, its B rows at 2r+1
        if (!refill) {
        } else if ((q & 1) == 0) {
          const int r = q >> 1;
          const int kt = slice_kt(t + NS - 1, r);
          al.prepare(kt);
#pragma unroll
          for (int i = 0; i < IA; ++i) dma_a(nst + r * SLICE, i, kt);
        } else {
          const int r = q >> 1;
          const int kt = slice_kt(t + NS - 1, r);
#pragma unroll
          for (int i = 0; i < IB; ++i) dma_b(nst + r * SLICE, i, kt);
        }
        if (kb + t * SPS + q / KS < ke) {  // uniform: the last stage may end early
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(fb[q & 1][j], fa[q & 1][i], acc[i][j]);
          ln_acc(fa[q & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      slot = slot + 1 == NS ? 0 : slot + 1;
      nslot = nslot + 1 == NS ? 0 : nslot + 1;
    }
  } else if constexpr (PF) {
    static_assert(KS == 2, "prefetch form assumes two k-steps per slice");
    f16x8 f0a[TM], f0b[TN], f1a[TM], f1b[TN];
    auto rd = [&](const unsigned char DLM_LDS* st, int ks, f16x8 (&fa)[TM], f16x8 (&fb)[TN]) {
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = frag(st, wm * WM + i * 16 + (lane & 15), ks);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = frag(st + SA, wn * WN + j * 16 + (lane & 15), ks);
    };
    auto mma = [&](const f16x8 (&fa)[TM], const f16x8 (&fb)[TN]) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(fb[j], fa[i], acc[i][j]);
      ln_acc(fa);
    };
    DLM_WAIT_SLICES(NS - 1);  // slice kb
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    rd(smem, 0, f0a, f0b);
    for (int kt = kb; kt < ke; ++kt) {
      const int rel = kt - kb;
      const int slot = rel % NS;
      __builtin_amdgcn_sched_barrier(0);
      rd(smem + slot * STAGE, 1, f1a, f1b);
      mma(f0a, f0b);
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 1 < ke) {
        // this wave's reads of the slot are complete before the barrier
        // after which another wave may refill it
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        DLM_WAIT_SLICES(NS - 2);             // slice kt+1
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        rd(smem + ((rel + 1) % NS) * STAGE, 0, f0a, f0b);
        issue_all(slot, min(kt + NS, ke - 1));
      }
      __builtin_amdgcn_sched_barrier(0);
      mma(f1a, f1b);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
  int pslot = 0, pnslot = NS - 1;  // slot read this slice, slot refilled this slice
  for (int kt = kb; kt < ke; ++kt) {
    if (skips == 0) {
      DLM_WAIT_VM((NS - 2) * (IA + IB));
    } else if (skips == 1) {
      DLM_WAIT_VM((NS - 2) * (IA + IB - 1));
    } else {
      DLM_WAIT_VM((NS - 2) * (IA + IB - 2));
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const unsigned char DLM_LDS* st = smem + pslot * STAGE;
    unsigned char DLM_LDS* nst = smem + pnslot * STAGE;
    const int nkt = min(kt + NS - 1, ke - 1);
    al.prepare(nkt);
    f16x8 fa[2][TM], fb[2][TN];
    auto rd = [&](int ks) {
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[ks & 1][i] = frag(st, wm * WM + i * 16 + (lane & 15), ks);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[ks & 1][j] = frag(st + SA, wn * WN + j * 16 + (lane & 15), ks);
    };
    rd(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 1 < KS) rd(ks + 1);
      // the next slice's DMA, spread over the k-steps
#pragma unroll
      for (int i = 0; i < IA; ++i)
        if (i % KS == ks) dma_a(nst, i, nkt);
#pragma unroll
      for (int i = 0; i < IB; ++i)
        if ((IA + i) % KS == ks) dma_b(nst, i, nkt);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(fb[ks & 1][j], fa[ks & 1][i], acc[i][j]);
      ln_acc(fa[ks & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    pslot = pslot + 1 == NS ? 0 : pslot + 1;
    pnslot = pnslot + 1 == NS ? 0 : pnslot + 1;
  }
  }
#undef DLM_WAIT_SLICES
#undef DLM_WAIT_SLICES_PLUS
  DLM_WAIT_VM(0);  // no DMA may still be writing this workgroup's LDS at exit

  if (!LNS && sp.S > 1) {
    // ---- split-K reduction (last arriver) ----
    const int tile = tmi * tiles_n + tni;
    constexpr int PER = BM * BN;  // floats per partial
    float* mine = sp.ws + ((size_t)tile * sp.S + sidx) * PER;
    const int base = (wave * TM * TN) * 256 + lane * 4;  // float index of block (0,0)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        unsigned long long* p = reinterpret_cast<unsigned long long*>(mine + base + (i * TN + j) * 256);
        const unsigned long long lo = ((unsigned long long)__float_as_uint(acc[i][j][1]) << 32) |
                                      __float_as_uint(acc[i][j][0]);
        const unsigned long long hi = ((unsigned long long)__float_as_uint(acc[i][j][3]) << 32) |
                                      __float_as_uint(acc[i][j][2]);
        __hip_atomic_store(p, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    DLM_WAIT_VM(0);  // this wave's partial is complete at agent scope
    __syncthreads();  // every wave's partial complete, every fragment read done
    int* flag = reinterpret_cast<int*>(smem_generic);  // the operand ring is free now
    // acquire-release at agent scope: this split's partial (and every earlier
    // split's, through the counter) happens-before the last split's reads
    if (tid == 0)
      *flag = __hip_atomic_fetch_add(sp.cnt + tile, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*flag != sp.S - 1) return;
    f32x4 tot[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) tot[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < sp.S; ++s) {
      if (s == sidx) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) tot[i][j] += acc[i][j];
      } else {
        const float* other = sp.ws + ((size_t)tile * sp.S + s) * PER;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const unsigned long long* p =
                reinterpret_cast<const unsigned long long*>(other + base + (i * TN + j) * 256);
            const unsigned long long lo = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned long long hi = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            tot[i][j] += f32x4{__uint_as_float((unsigned)lo), __uint_as_float((unsigned)(lo >> 32)),
                               __uint_as_float((unsigned)hi), __uint_as_float((unsigned)(hi >> 32))};
          }
      }
    }
    if (tid == 0) __hip_atomic_store(sp.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = tot[i][j];
  }

  // ------------------------------ epilogue ------------------------------
  // acc[i][j] = W-fragment x X-fragment: lane holds output row (lane & 15) of
  // block i and output columns 4 (lane >> 4) + [0, 4) of block j.
  const int row0 = m0 + wm * WM + (lane & 15);
  const int col0 = n0 + wn * WN + 4 * (lane >> 4);
  if constexpr (LNS) {
    // LayerNorm fold: rstd and rstd * mean of each row from the x and x^2
    // sums (lanes l, l^16, l^32, l^48 hold the four K chunks of row l & 15),
    // the columns' ln_c1 / ln_c2 loaded together (clamped into N), then
    // acc <- rstd acc - rstd mean c1 + c2 and the ordinary epilogue
    f32x4 c1v[TN], c2v[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = min(col0 + j * 16, ep.N - 4);
      c1v[j] = *reinterpret_cast<const f32x4*>(ep.ln_c1 + col);
      c2v[j] = *reinterpret_cast<const f32x4*>(ep.ln_c2 + col);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float a = ln_s1[i], b = ln_s2[i];
      a += __shfl_xor(a, 16, 64);
      b += __shfl_xor(b, 16, 64);
      a += __shfl_xor(a, 32, 64);
      b += __shfl_xor(b, 32, 64);
      const float mean = a * ep.ln_invk;
      const float var = fmaxf(b * ep.ln_invk - mean * mean, 0.0f);
      const float r = rsqrtf(var + ep.ln_eps), rm = r * mean;
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = ln_fold4(acc[i][j], c1v[j], c2v[j], r, rm);
    }
  }
  // the batched forms hold every loaded operand in registers: wave tiles of
  // up to 20 blocks (the largest wave tile, 128x64, keeps the per-block form)
  if constexpr (TM * TN <= 20) {
    if (ep.act == DLM_ACT_GEGLU) {
      if (m0 + BM <= ep.M && n0 + BN <= ep.N) {
        epi_tile_geglu<TM, TN, true>(acc, row0, col0, ep);
      } else {
        epi_tile_geglu<TM, TN, false>(acc, row0, col0, ep);
      }
      return;
    }
    if (epi_tile_fast(ep)) {
      // GroupNorm statistics of the output: the tile's fp16 values are copied
      // into the (now free) operand ring and reduced from there
      static_assert(BM * BN * 2 <= NS * STAGE, "output tile larger than the LDS ring");
      f16 DLM_LDS* stile = (f16 DLM_LDS*)smem;
      f16 DLM_LDS* stl = stile + (wm * WM + (lane & 15)) * BN + wn * WN + 4 * (lane >> 4);
      const bool gn = ep.gn_stats != nullptr;
      if (gn) __syncthreads();  // every wave is done with the ring
      if (early) {
        epi_tile<TM, TN, true>(acc, row0, col0, ep, ebv, erv, gn, stl, BN);
      } else {
        f16x4 bv[TN], rv[TM][TN];
        epi_tile<TM, TN>(acc, row0, col0, ep, bv, rv, gn, stl, BN);
      }
      if (ep.gn_stats) {
        __syncthreads();
        gn_tile_stats<BM, BN>(stile, m0, n0, ep, tid, NW * 64);
      }
      return;
    }
  }
  if (ep.act == DLM_ACT_GEGLU) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) epi4_geglu(acc[i][j], row0 + i * 16, col0 + j * 16, ep);
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) epi4(acc[i][j], row0 + i * 16, col0 + j * 16, ep);
}

// ---------------------------------------------------------------------------
// Host-side tile configuration choice and launch.
// ---------------------------------------------------------------------------
// Split-K workspace per (device, stream): launches on one stream run in
// order and share it; another stream gets its own.  Sized once; a launch
// that would need more falls back to one split.
struct SplitWorkspace {
  float* ws = nullptr;
  int* cnt = nullptr;
};
constexpr size_t kSplitWsFloats = size_t(24) << 20;  // 96 MiB of fp32 partials
constexpr int kSplitCounters = 1 << 16;
static std::mutex g_split_mu;
static std::map<std::pair<int, hipStream_t>, SplitWorkspace> g_split_ws;

// A stream under graph capture gets no new workspace (the allocation and its
// synchronous clear would invalidate the capture): its launches run unsplit
// until the stream has made one outside capture.
static const SplitWorkspace* split_workspace(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lk(g_split_mu);
  auto it = g_split_ws.find({dev, s});
  if (it != g_split_ws.end() && it->second.ws) return &it->second;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
  SplitWorkspace& w = g_split_ws[{dev, s}];
  if (!w.ws) {
    float* ws = nullptr;
    int* cnt = nullptr;
    if (hipMalloc(&ws, kSplitWsFloats * sizeof(float)) != hipSuccess) return nullptr;
    if (hipMalloc(&cnt, kSplitCounters * sizeof(int)) != hipSuccess ||
        hipMemset(cnt, 0, kSplitCounters * sizeof(int)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
      (void)hipFree(ws);
      if (cnt) (void)hipFree(cnt);
      return nullptr;
    }
    w.ws = ws;
    w.cnt = cnt;
  }
  return &w;
}

// Frees the split-K workspace of `s` on every device (after synchronising
// the stream).  Explicit only: a graph captured on a stream holds its
// workspace's address, so nothing frees it behind the caller's back.
int split_workspace_release(hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_split_mu);
  bool any = false;
  for (const auto& kv : g_split_ws) any |= kv.first.second == s;
  if (!any) return DLM_OK;
  if (hipStreamSynchronize(s) != hipSuccess) return fail(DLM_ERR_HIP, "split workspace: stream synchronisation failed");
  for (auto it = g_split_ws.begin(); it != g_split_ws.end();) {
    if (it->first.second == s) {
      if ((it->second.ws && hipFree(it->second.ws) != hipSuccess) ||
          (it->second.cnt && hipFree(it->second.cnt) != hipSuccess))
        return fail(DLM_ERR_HIP, "split workspace: hipFree failed");
      it = g_split_ws.erase(it);
    } else {
      ++it;
    }
  }
  return DLM_OK;
}

size_t split_workspace_bytes() {
  std::lock_guard<std::mutex> lk(g_split_mu);
  size_t t = 0;
  for (const auto& kv : g_split_ws)
    if (kv.second.ws) t += kSplitWsFloats * sizeof(float) + kSplitCounters * sizeof(int);
  return t;
}

// Tuning aids (dlm_gemm_force_split / _set_variant / _force_tile /
// _override_shape): thread-local, so they steer only launches made by the
// thread that set them.
static thread_local int g_forced_split = 0;
static thread_local int g_variant = 0;  // bits select alternative heuristics
// Set while an allocation-free entry point runs: split-K stays off, since its
// workspace is allocated on first use.
static thread_local bool t_no_split = false;
struct NoSplitScope {
  bool prev;
  NoSplitScope() : prev(t_no_split) { t_no_split = true; }
  ~NoSplitScope() { t_no_split = prev; }
};

// "dma_gemm_kernel<BM, BN, WM, WN, NS, PF, SPS, LNS, RowDesc|ConvDesc>", as
// the profiler prints the instantiation
template <int BM, int BN, int WM, int WN, int NS, bool PF, int SPS, bool LNS, class Desc>
static const char* dma_kernel_name() {
  static const std::string n = "dma_gemm_kernel<" + std::to_string(BM) + ", " + std::to_string(BN) +
                               ", " + std::to_string(WM) + ", " + std::to_string(WN) + ", " +
                               std::to_string(NS) + ", " + (PF ? "true" : "false") + ", " +
                               std::to_string(SPS) + ", " + (LNS ? "true" : "false") + ", " +
                               (std::is_same<Desc, RowDesc>::value ? "RowDesc" : "ConvDesc") + ">";
  return n.c_str();
}

// Tile configurations with a LayerNorm-folding instantiation: the ones the
// LayerNorm-consuming linears of the UNet take (2048- and 8192-row QKV, cross
// Q and GEGLU shapes), plus their non-prefetch variants.
template <int BM, int BN, int WM, int WN, int NS, bool PF, int SPS>
constexpr bool ln_tile() {
  return (BM == 128 && BN == 80 && WM == 16 && WN == 80 && NS == 3 && !PF && SPS == 2) ||
         (BM == 128 && BN == 128 && WM == 64 && WN == 32 && NS == 2 && SPS == 1) ||
         (BM == 128 && BN == 128 && WM == 32 && WN == 64 && NS == 2 && SPS == 1) ||
         (BM == 256 && BN == 160 && WM == 64 && WN == 80 && NS == 3 && SPS == 1) ||
         (BM == 256 && BN == 160 && WM == 32 && WN == 160 && NS == 3 && SPS == 1) ||
         (BM == 128 && BN == 160 && WM == 32 && WN == 80 && SPS == 1);
}
template <int BM, int BN, int WM, int WN, bool DEEP, class Desc>
static const char* mfma_kernel_name() {
  static const std::string n = "mfma_gemm_kernel<" + std::to_string(BM) + ", " + std::to_string(BN) +
                               ", " + std::to_string(WM) + ", " + std::to_string(WN) + ", " +
                               (DEEP ? "true" : "false") + ", " +
                               (std::is_same<Desc, RowDesc>::value ? "RowDesc" : "ConvDesc") + ">";
  return n.c_str();
}

// Set by a launch whose epilogue writes the requested GroupNorm statistics
// (EpiArgs::gn_stats); a launch that cannot leaves it false and the entry
// point runs the statistics pass instead.
static thread_local bool t_gn_written = false;

template <int BM, int BN, int WM, int WN, int NS, bool PF = false, int SPS = 1, class Desc>
static int launch_dma(const Desc& ad, const RowDesc& bd, const EpiArgs& ep_in, int M, int N,
                      hipStream_t s, int S = 1) {
  static_assert(NS * SPS * (BM + BN) * BK * 2 <= 160 * 1024, "LDS ring larger than 160 KiB");
  // the batched epilogue (wave tiles of at most 20 blocks) is the one that
  // writes GroupNorm statistics
  EpiArgs ep = ep_in;
  const bool gn = ep.gn_stats && (WM / 16) * (WN / 16) <= 20 && epi_tile_fast(ep) &&
                  ep.act != DLM_ACT_GEGLU && ep.gn_hw > 0 && ep.gn_hw % kGnChunk == 0;
  if (!gn) ep.gn_stats = nullptr;
  t_gn_written = gn;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  const int nk = (bd.K + BK - 1) / BK;
  if (g_forced_split > 0) S = g_forced_split;
  if (t_no_split) S = 1;
  SplitArgs sp{1, nk, nullptr, nullptr};
  if (S > 1 && nk > 1) {
    const int kps = (nk + S - 1) / S;
    S = (nk + kps - 1) / kps;  // no empty split
    const SplitWorkspace* w = S > 1 ? split_workspace(s) : nullptr;
    if (w && (size_t)tiles * S * BM * BN <= kSplitWsFloats && tiles <= kSplitCounters)
      sp = SplitArgs{S, kps, w->ws, w->cnt};
  }
  constexpr int NT = (BM / WM) * (BN / WN) * 64;
  // the problem's dims (after note_kernel, which clears them)
  const int dims_flags = (ep.res ? 1 : 0) | (ep.act << 4) | (std::is_same<Desc, ConvDesc>::value ? 256 : 0) |
                         (ep.ln_c1 ? 512 : 0);
  if (ep.ln_c1) {
    if constexpr (std::is_same<Desc, RowDesc>::value && ln_tile<BM, BN, WM, WN, NS, PF, SPS>()) {
      sp = SplitArgs{1, nk, nullptr, nullptr};
      note_kernel(dma_kernel_name<BM, BN, WM, WN, NS, PF, SPS, true, Desc>());
      note_dims(M, N, bd.K, dims_flags);
      launch((dma_gemm_kernel<BM, BN, WM, WN, NS, PF, SPS, true, Desc>), dim3(tiles), dim3(NT),
                         0, s, ad, bd, ep, tiles_m, tiles_n, sp);
      DLM_LAUNCH_CHECK();
      return DLM_OK;
    } else {
      return fail(DLM_ERR_UNSUPPORTED, "LayerNorm-folding GEMM: tile without a folding kernel");
    }
  }
  const int grid = sp.S > 1 ? 8 * ((tiles + 7) / 8) * sp.S : tiles;
  note_kernel(dma_kernel_name<BM, BN, WM, WN, NS, PF, SPS, false, Desc>());
  note_dims(M, N, bd.K, dims_flags);
  launch((dma_gemm_kernel<BM, BN, WM, WN, NS, PF, SPS, false, Desc>), dim3(grid), dim3(NT), 0,
                     s, ad, bd, ep, tiles_m, tiles_n, sp);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

template <int BM, int BN, int WM, int WN, bool DEEP = true, class Desc>
static int launch_cfg(const Desc& ad, const RowDesc& bd, const EpiArgs& ep, int M, int N,
                      hipStream_t s) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  constexpr int NT = (BM / WM) * (BN / WN) * 64;
  note_kernel(mfma_kernel_name<BM, BN, WM, WN, DEEP, Desc>());
  note_dims(M, N, bd.K, (ep.res ? 1 : 0) | (ep.act << 4) | (std::is_same<Desc, ConvDesc>::value ? 256 : 0));
  launch((mfma_gemm_kernel<BM, BN, WM, WN, DEEP, Desc>), dim3(tiles_m * tiles_n),
                     dim3(NT), 0, s, ad, bd, ep, tiles_m, tiles_n);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

static inline long long ceil_div(long long a, long long b) { return (a + b - 1) / b; }

// Tile-shape override for tuning sweeps (0 = automatic choice).
static thread_local int g_forced_tile = 0;

static bool al8(const void* p) { return ((uintptr_t)p & 7) == 0; }

// The DMA core needs 16-byte aligned operands (true of every RowDesc/ConvDesc
// the entry points accept), whole 4-column output groups and 8-byte aligned
// epilogue vectors.
static bool dma_epilogue_ok(const EpiArgs& ep) {
  if (ep.N % 4 != 0 || !al8(ep.y) || (ep.bias && !al8(ep.bias))) return false;
  if (!ep.out_nchw && ep.ldy % 4 != 0) return false;
  if (ep.y_f32 && !ep.out_nchw && !dlm_aligned16(ep.y)) return false;
  if (ep.res && (ep.ldr % 4 != 0 || !al8(ep.res))) return false;
  if (ep.res && ep.res_f32 && !dlm_aligned16(ep.res)) return false;
  if (ep.tbias && (ep.tbias_ld % 4 != 0 || !al8(ep.tbias))) return false;
  return true;
}
static bool dma_operand_ok(const RowDesc& a) { return dlm_aligned16(a.p) && a.ld % 8 == 0; }
static bool dma_operand_ok(const ConvDesc& d) {
  return !d.generic && d.C1 % BK == 0 && d.C1a % BK == 0;
}

template <class Desc>
static int launch_gemm_impl(const Desc& ad, const RowDesc& bd, const EpiArgs& ep, int M, int N,
                            hipStream_t s);

// Tuning aid: per-shape tile / split overrides (dlm_gemm_override_shape),
// matched on (M, N, K); per thread, like the other tuning aids.
struct ShapeOverride {
  int M, N, K, tile, split;
};
static thread_local std::vector<ShapeOverride> g_overrides;

template <class Desc>
static int launch_gemm(const Desc& ad, const RowDesc& bd, const EpiArgs& ep, int M, int N,
                       hipStream_t s) {
  if (!g_overrides.empty()) {
    for (const ShapeOverride& o : g_overrides)
      if (o.M == M && o.N == N && o.K == bd.K) {
        const int t = g_forced_tile, sp = g_forced_split;
        g_forced_tile = o.tile;
        g_forced_split = o.split;
        const int st = launch_gemm_impl(ad, bd, ep, M, N, s);
        g_forced_tile = t;
        g_forced_split = sp;
        return st;
      }
  }
  return launch_gemm_impl(ad, bd, ep, M, N, s);
}

template <class Desc>
static int launch_gemm_impl(const Desc& ad, const RowDesc& bd, const EpiArgs& ep, int M, int N,
                            hipStream_t s) {
  constexpr int kCUs = 256;
  if ((ep.y_f32 || ep.res_f32) && (ep.vt || ep.act == DLM_ACT_GEGLU))
    return fail(DLM_ERR_UNSUPPORTED, "fp32 output/residual with a GEGLU or V^T epilogue");
  const bool dma = dma_epilogue_ok(ep) && dma_operand_ok(ad) && dma_operand_ok(bd);
  if (ep.ln_c1) {
    // LayerNorm-folding linears: the tiles of the plain heuristic below for the
    // UNet's shapes, 128x128 prefetch tiles for any other
    if constexpr (!std::is_same<Desc, RowDesc>::value) {
      return fail(DLM_ERR_UNSUPPORTED, "LayerNorm folding applies to linears only");
    } else {
      if (!dma) return fail(DLM_ERR_UNSUPPORTED, "LayerNorm-folding GEMM needs aligned operands");
      switch (g_forced_tile) {  // tuning aid: the tiles with a folding kernel
        case 24: return launch_dma<128, 160, 32, 80, 4>(ad, bd, ep, M, N, s);
        case 28: return launch_dma<256, 160, 64, 80, 3, true>(ad, bd, ep, M, N, s);
        case 29: return launch_dma<128, 128, 64, 32, 2, true>(ad, bd, ep, M, N, s);
        case 31: return launch_dma<128, 160, 32, 80, 3, true>(ad, bd, ep, M, N, s);
        case 35: return launch_dma<128, 80, 16, 80, 3, false, 2>(ad, bd, ep, M, N, s);
        case 40: return launch_dma<128, 128, 32, 64, 2, true>(ad, bd, ep, M, N, s);
        case 41: return launch_dma<256, 160, 32, 160, 3, true>(ad, bd, ep, M, N, s);
        case 0: break;
        default: return fail(DLM_ERR_UNSUPPORTED, "forced tile has no LayerNorm-folding kernel");
      }
      // Every wave accumulates the statistics of its own rows, so waves that
      // hold fewer row blocks (and fewer waves sharing rows) spend less VALU
      // on them.  Measured against LayerNorm + linear, graph-replayed (us):
      // QKV 2048x3840x1280 128x128 (32x64 waves) 35.4 vs 43.5; cross Q
      // 2048x1280x1280 128x80 15.7 vs 23.5; GEGLU 2048x10240x1280 256x160
      // (32x160 waves) 79.9 vs 86.7; 8192 rows: QKV 41.3 vs 45.7, Q 18.0 vs
      // 26.4, GEGLU 99.4 vs 100.3.
      const long long t256 = ceil_div(M, 256) * (N / 160), t80 = ceil_div(M, 128) * (N / 80);
      const long long t160 = ceil_div(M, 128) * (N / 160);
      const int nk = (int)ceil_div(bd.K, BK);
      if (ep.act == DLM_ACT_GEGLU && N % 160 == 0 && t256 >= kCUs)
        return launch_dma<256, 160, 32, 160, 3, true>(ad, bd, ep, M, N, s);
      if (!ep.vt && ep.act != DLM_ACT_GEGLU && N % 80 == 0 && t80 >= kCUs * 3 / 4 && t80 <= kCUs)
        return launch_dma<128, 80, 16, 80, 3, false, 2>(ad, bd, ep, M, N, s);
      if (!ep.vt && ep.act != DLM_ACT_GEGLU && N % 160 == 0 && N <= 1280 && t160 >= kCUs && nk <= 100)
        return launch_dma<128, 160, 32, 80, 4>(ad, bd, ep, M, N, s);
      return launch_dma<128, 128, 32, 64, 2, true>(ad, bd, ep, M, N, s);
    }
  }
  if (dma) {
    switch (g_forced_tile) {
      case 8: return launch_dma<128, 128, 64, 64, 2>(ad, bd, ep, M, N, s);
      case 9: return launch_dma<128, 64, 64, 32, 2>(ad, bd, ep, M, N, s);
      case 10: return launch_dma<128, 128, 64, 64, 4>(ad, bd, ep, M, N, s);
      case 11: return launch_dma<128, 64, 64, 32, 4>(ad, bd, ep, M, N, s);
      case 12: return launch_dma<64, 128, 32, 64, 2>(ad, bd, ep, M, N, s);
      case 13: return launch_dma<256, 128, 128, 64, 2>(ad, bd, ep, M, N, s);
      case 14: return launch_dma<128, 128, 64, 32, 4>(ad, bd, ep, M, N, s);
      case 15: return launch_dma<128, 128, 64, 32, 2>(ad, bd, ep, M, N, s);
      case 16: return launch_dma<256, 128, 64, 64, 2>(ad, bd, ep, M, N, s);
      case 17: return launch_dma<128, 128, 32, 64, 4>(ad, bd, ep, M, N, s);
      case 18: return launch_dma<128, 128, 64, 32, 5>(ad, bd, ep, M, N, s);
      case 19: return launch_dma<256, 128, 64, 64, 3>(ad, bd, ep, M, N, s);
      case 20: return launch_dma<128, 64, 64, 32, 6>(ad, bd, ep, M, N, s);
      case 21: return launch_dma<256, 160, 64, 80, 3>(ad, bd, ep, M, N, s);
      case 22: return launch_dma<128, 160, 32, 80, 3>(ad, bd, ep, M, N, s);
      case 23: return launch_dma<128, 160, 64, 80, 2>(ad, bd, ep, M, N, s);
      case 24: return launch_dma<128, 160, 32, 80, 4>(ad, bd, ep, M, N, s);
      case 25: return launch_dma<64, 160, 32, 80, 2>(ad, bd, ep, M, N, s);
      case 26: return launch_dma<128, 80, 16, 80, 5>(ad, bd, ep, M, N, s);
      case 27: return launch_dma<128, 80, 16, 80, 5, true>(ad, bd, ep, M, N, s);
      case 28: return launch_dma<256, 160, 64, 80, 3, true>(ad, bd, ep, M, N, s);
      case 29: return launch_dma<128, 128, 64, 32, 2, true>(ad, bd, ep, M, N, s);
      case 30: return launch_dma<128, 160, 32, 80, 4, true>(ad, bd, ep, M, N, s);
      case 31: return launch_dma<128, 160, 32, 80, 3, true>(ad, bd, ep, M, N, s);
      case 32: return launch_dma<256, 128, 64, 64, 3, true>(ad, bd, ep, M, N, s);
      case 33: return launch_dma<128, 128, 64, 32, 4, true>(ad, bd, ep, M, N, s);
      case 34: return launch_dma<128, 64, 64, 32, 2, true>(ad, bd, ep, M, N, s);
      case 35: return launch_dma<128, 80, 16, 80, 3, false, 2>(ad, bd, ep, M, N, s);
      case 36: return launch_dma<128, 80, 16, 80, 2, false, 2>(ad, bd, ep, M, N, s);
      case 37: return launch_dma<128, 160, 32, 80, 2, false, 2>(ad, bd, ep, M, N, s);
      case 38: return launch_dma<128, 128, 64, 32, 2, false, 2>(ad, bd, ep, M, N, s);
      case 39: return launch_dma<128, 64, 64, 32, 3, false, 2>(ad, bd, ep, M, N, s);
      case 40: return launch_dma<128, 128, 32, 64, 2, true>(ad, bd, ep, M, N, s);
      case 41: return launch_dma<256, 160, 32, 160, 3, true>(ad, bd, ep, M, N, s);
      case 42: return launch_dma<128, 16, 16, 16, 3>(ad, bd, ep, M, N, s);
      case 43: return launch_dma<64, 16, 16, 16, 3>(ad, bd, ep, M, N, s);
      case 44: return launch_dma<192, 160, 48, 80, 3>(ad, bd, ep, M, N, s);
      default: break;
    }
    if (g_forced_tile == 0) {
      // at most 16 output columns (the UNet's conv_out, 4 channels): one
      // 16-column block per wave, 8 waves of 16 rows, instead of a 64-column
      // tile that is mostly padding
      if (N <= 16 && !ep.vt && ep.act != DLM_ACT_GEGLU && ceil_div(M, 128) >= kCUs / 2)
        return launch_dma<128, 16, 16, 16, 3>(ad, bd, ep, M, N, s);
      // Measured on the UNet's shapes (warmed-up clocks, N(0,1) data):
      // 8-wave tiles (two waves per SIMD) everywhere.  128x128 tiles: two
      // slices in flight when two workgroups share a CU, four when the grid
      // leaves CUs with one.  GEGLU can take any tile (its value/gate pairs
      // sit in lanes 16 apart, so any 16-column-multiple wave works).
      const long long t128 = ceil_div(M, 128) * ceil_div(N, 128);
      const bool pf = !(g_variant & 2);
      // GEGLU FF1 at 2048x10240x1280: 256x160 tiles, three-slice ring, with
      // fragment prefetch, measured in the whole UNet step in one process
      // (25.3 ms against 26.0 with 128x128 and 26.7 with 256x128 for both FF1
      // shapes).  Grids of four or more 256x160 tiles per CU (8192x5120x640)
      // take the 128x128 prefetch tiles below: 0.11 ms less per step.
      if (ep.act == DLM_ACT_GEGLU && N % 160 == 0 && ceil_div(M, 256) * (N / 160) >= kCUs &&
          ceil_div(M, 256) * (N / 160) < 4 * kCUs)
        return pf ? launch_dma<256, 160, 64, 80, 3, true>(ad, bd, ep, M, N, s)
                  : launch_dma<256, 160, 64, 80, 3>(ad, bd, ep, M, N, s);
      // Output widths that are multiples of 160 (SDXL's 320 / 640 / 1280
      // channels): 160-column tiles give whole waves of tiles on 256 CUs
      // where 128-column tiles leave a partial wave; few tiles with a long K
      // are split-K so every CU gets work.  Choices measured per UNet level
      // (B=2): 32768x320 convs 256x160 (four splits from 80 slices on measured
      // the same as none; 8192x1280x11520 is ~130 us faster unsplit), 8192
      // rows 128x160 up to 100 slices and 256x160 x2 splits beyond, 2048 rows
      // 128x160 x2 splits from 44 slices, 256x160 x4 from 300.  Two splits of
      // a grid that already fills the chip measured slower than one or four.
      const int nk = (int)ceil_div(bd.K, BK);
      // 2048-row outputs 1280 wide (one 1024-token level at B=2) and the
      // 8192x320 stride-2 conv: 128x80 tiles, 8 waves of 16x80 -> exactly
      // 256 tiles.  Ring of three two-slice stages (one barrier per 128 of
      // K): 15.5 / 40.3 us at K = 1280 / 5120 against 16.4 / 42.6 for a
      // five-slice ring and 16.2 / 43.9 for 128x128; the conv 39.1 us
      // against 47.3 for 128x160 x2 splits.  Convolutions with a long K
      // (2048x1280x11520) stay on split 128x160 tiles.
      if ((std::is_same<Desc, RowDesc>::value || nk <= 100) && !ep.vt && N % 80 == 0 &&
          ceil_div(M, 128) * (N / 80) >= kCUs * 3 / 4 &&
          ceil_div(M, 128) * (N / 80) <= kCUs && !(g_variant & 1))
        return launch_dma<128, 80, 16, 80, 3, false, 2>(ad, bd, ep, M, N, s);
      if (!ep.vt && N % 160 == 0 && N <= 1280 && !(g_variant & 1)) {
        const long long t256 = ceil_div(M, 256) * (N / 160), t160 = ceil_div(M, 128) * (N / 160);
        if (t256 >= kCUs)
          return launch_dma<256, 160, 64, 80, 3>(ad, bd, ep, M, N, s, !pf && nk >= 80 ? 4 : 1);
        if (t160 >= kCUs) {
          if (nk <= 100) return launch_dma<128, 160, 32, 80, 4>(ad, bd, ep, M, N, s);
          return launch_dma<256, 160, 64, 80, 3>(ad, bd, ep, M, N, s, 2);
        } else if (nk >= 300 && t256 * 4 >= kCUs) {
          return launch_dma<256, 160, 64, 80, 3>(ad, bd, ep, M, N, s, 4);
        } else if (nk >= 44 && t160 * 4 >= kCUs) {
          return launch_dma<128, 160, 32, 80, 3>(ad, bd, ep, M, N, s, t160 * 2 >= kCUs ? 2 : 4);
        }
      }
      // Outputs of 129-192 rows with at least one 160-column tile per CU (the
      // text tokens' K/V projection of every transformer block at CFG batch
      // 2, 154 x 166400 x 2048): 192x160 tiles (8 waves of 48x80) compute the
      // rows as 192 instead of 256, 235-251 -> 206-212 us per launch,
      // bit-identical.
      if (std::is_same<Desc, RowDesc>::value && M > 128 && M <= 192 && N % 160 == 0 && N / 160 >= kCUs &&
          ep.act != DLM_ACT_GEGLU)
        return launch_dma<192, 160, 48, 80, 3>(ad, bd, ep, M, N, s);
      if (t128 >= kCUs / 2) {
        if (N % 128 != 0)
          return ceil_div(M, 128) * ceil_div(N, 64) >= kCUs
                     ? launch_dma<128, 64, 64, 32, 2>(ad, bd, ep, M, N, s)
                     : launch_dma<128, 64, 64, 32, 4>(ad, bd, ep, M, N, s);
        // convolutions with one to four 128x128 tiles per CU: 256x128 tiles
        // (fewer operand bytes per MFMA; the im2col loader is the costlier one)
        if (std::is_same<Desc, ConvDesc>::value && t128 >= kCUs && t128 < 4 * kCUs)
          return launch_dma<256, 128, 64, 64, 3>(ad, bd, ep, M, N, s);
        // one workgroup's ring of two slices: the prefetch form (2048x3840x1280
        // QKV ~2 us faster per launch, 8192x1920x640 the same)
        if (t128 >= kCUs)
          return pf ? launch_dma<128, 128, 64, 32, 2, true>(ad, bd, ep, M, N, s)
                    : launch_dma<128, 128, 64, 32, 2>(ad, bd, ep, M, N, s);
        return launch_dma<128, 128, 64, 32, 4>(ad, bd, ep, M, N, s);
      }
      if (ep.vt)  // the transposed-V epilogue exists only in the DMA core
        return launch_dma<128, 128, 64, 32, 4>(ad, bd, ep, M, N, s);
      // fewer than 128 tiles of 128x128: the small-tile kernel below
    }
  }
  if (ep.vt) return fail(DLM_ERR_UNSUPPORTED, "transposed-V output needs aligned operands");
  if (ep.act == DLM_ACT_GEGLU) return launch_cfg<128, 128, 64, 64>(ad, bd, ep, M, N, s);
  switch (g_forced_tile) {
    case 1: return launch_cfg<128, 128, 64, 64>(ad, bd, ep, M, N, s);
    case 2: return launch_cfg<128, 64, 64, 32>(ad, bd, ep, M, N, s);
    case 3: return launch_cfg<64, 64, 32, 32>(ad, bd, ep, M, N, s);
    case 4: return launch_cfg<128, 32, 32, 32>(ad, bd, ep, M, N, s);
    case 5: return launch_cfg<256, 128, 128, 64>(ad, bd, ep, M, N, s);
    case 6: return launch_cfg<128, 256, 64, 128>(ad, bd, ep, M, N, s);
    case 7: return launch_cfg<256, 256, 128, 128>(ad, bd, ep, M, N, s);
    default: break;
  }
  if (N <= 32) return launch_cfg<128, 32, 32, 32>(ad, bd, ep, M, N, s);
  if (N <= 64) return launch_cfg<128, 64, 64, 32>(ad, bd, ep, M, N, s);
  if (ceil_div(M, 128) * ceil_div(N, 128) >= kCUs)
    return launch_cfg<128, 128, 64, 64>(ad, bd, ep, M, N, s);
  if (ceil_div(M, 128) * ceil_div(N, 64) >= kCUs)
    return launch_cfg<128, 64, 64, 32>(ad, bd, ep, M, N, s);
  return launch_cfg<64, 64, 32, 32>(ad, bd, ep, M, N, s);
}

static EpiArgs make_epi(void* Y, int ldy, const void* bias, const void* R, int ldr, int M, int N,
                        float alpha, float beta, int act) {
  EpiArgs ep{};
  ep.y = (f16*)Y;
  ep.ldy = ldy;
  ep.bias = (const f16*)bias;
  ep.res = (const f16*)R;
  ep.ldr = ldr;
  ep.alpha = alpha;
  ep.beta = beta;
  ep.act = act;
  ep.tbias = nullptr;
  ep.tbias_ld = 0;
  ep.rows_per_sample = 0;
  ep.out_nchw = 0;
  ep.M = M;
  ep.N = N;
  ep.vt = nullptr;
  ep.vt_col0 = 0;
  ep.vt_tokens = 0;
  ep.vt_ld = 0;
  ep.y_f32 = 0;
  ep.res_f32 = 0;
  return ep;
}

int linear_impl(const void* X, int lda, const void* W, int ldw, const void* bias, const void* R,
                int ldr, void* Y, int ldy, int M, int N, int K, float alpha, float beta, int act,
                hipStream_t s) {
  RowDesc ad{(const f16*)X, lda, M, K, (unsigned)((size_t)M * lda * 2)};
  RowDesc bd{(const f16*)W, ldw, N, K, (unsigned)((size_t)N * ldw * 2)};
  EpiArgs ep = make_epi(Y, ldy, bias, R, ldr, M, N, alpha, beta, act);
  return launch_gemm(ad, bd, ep, M, N, s);
}

// ---------------------------------------------------------------------------
// Small helper kernels: layout transposes and weight repacking.
// ---------------------------------------------------------------------------
// out[n][p][c] (row stride C_pad) = in[n][c][p]; channels >= C are zero.
__global__ void nchw_to_nhwc_kernel(const f16* __restrict__ in, f16* __restrict__ out, int C,
                                    int HW, int C_pad) {
  __shared__ f16 tile[32][33];
  const int n = blockIdx.z;
  const int c0 = blockIdx.y * 32, p0 = blockIdx.x * 32;
  const int tx = threadIdx.x, ty = threadIdx.y;  // 32 x 8
  const f16* src = in + (size_t)n * C * HW;
  for (int r = ty; r < 32; r += 8) {
    const int c = c0 + r, p = p0 + tx;
    tile[r][tx] = (c < C && p < HW) ? src[(size_t)c * HW + p] : (f16)0.0f;
  }
  __syncthreads();
  f16* dst = out + (size_t)n * HW * C_pad;
  for (int r = ty; r < 32; r += 8) {
    const int p = p0 + r, c = c0 + tx;
    if (p < HW && c < C_pad) dst[(size_t)p * C_pad + c] = tile[tx][r];
  }
}

// out[n][c][p] = in[n][p][c] (row stride C_pad), c < C.
__global__ void nhwc_to_nchw_kernel(const f16* __restrict__ in, f16* __restrict__ out, int C,
                                    int HW, int C_pad) {
  __shared__ f16 tile[32][33];
  const int n = blockIdx.z;
  const int c0 = blockIdx.y * 32, p0 = blockIdx.x * 32;
  const int tx = threadIdx.x, ty = threadIdx.y;
  const f16* src = in + (size_t)n * HW * C_pad;
  for (int r = ty; r < 32; r += 8) {
    const int p = p0 + r, c = c0 + tx;
    tile[r][tx] = (p < HW && c < C) ? src[(size_t)p * C_pad + c] : (f16)0.0f;
  }
  __syncthreads();
  f16* dst = out + (size_t)n * C * HW;
  for (int r = ty; r < 32; r += 8) {
    const int c = c0 + r, p = p0 + tx;
    if (c < C && p < HW) dst[(size_t)c * HW + p] = tile[tx][r];
  }
}

// out[co*ld + col0 + tap*Cin_pad + ci] = w[co][ci][tap] (zero for ci >= Cin)
// Column of weight (tap, ci) within a packed conv segment of `taps` taps over
// Cin_pad channels.  Cin_pad a multiple of 64 (the implicit-GEMM loaders'
// one-tap-per-K-slice form): 64-channel blocks outermost, then taps, then
// the block's channels, the K order those loaders walk; otherwise (the
// small-channel form that decodes a tap per 8-channel vector) tap-major.
__device__ __forceinline__ long long conv_wcol(int tap, int ci, int taps, int Cin_pad) {
  if (Cin_pad % BK == 0) return ((long long)(ci / BK) * taps + tap) * BK + ci % BK;
  return (long long)tap * Cin_pad + ci;
}

__global__ void conv_weight_pack_kernel(const f16* __restrict__ w, f16* __restrict__ out, int Cout,
                                        int Cin, int taps, int Cin_pad, int ld, int col0) {
  const long long total = (long long)Cout * taps * Cin_pad;
  for (long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int ci = (int)(idx % Cin_pad);
    const long long r = idx / Cin_pad;
    const int tap = (int)(r % taps);
    const int co = (int)(r / taps);
    const f16 v = ci < Cin ? w[((size_t)co * Cin + ci) * taps + tap] : (f16)0.0f;
    out[(size_t)co * ld + col0 + conv_wcol(tap, ci, taps, Cin_pad)] = v;
  }
}

// out[co*ld + col0 + conv_wcol(tap, ci)] += w[co][ci][tap] for ci < Cin
// (fp32 add, fp16 round); the zero padding ci >= Cin is left untouched.
__global__ void conv_weight_pack_add_kernel(const f16* __restrict__ w, f16* __restrict__ out,
                                            int Cout, int Cin, int taps, int Cin_pad, int ld,
                                            int col0) {
  const long long total = (long long)Cout * taps * Cin;
  for (long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int ci = (int)(idx % Cin);
    const long long r = idx / Cin;
    const int tap = (int)(r % taps);
    const int co = (int)(r / taps);
    f16* o = out + (size_t)co * ld + col0 + conv_wcol(tap, ci, taps, Cin_pad);
    *o = (f16)((float)*o + (float)w[((size_t)co * Cin + ci) * taps + tap]);
  }
}

// GEGLU interleave in groups of 4: packed row 8q+s <- value row 4q+s (s<4)
// or gate row d+4q+s-4 (s>=4).  A 16-column MFMA block then holds two
// (value, gate) groups whose halves sit in lanes that differ by 16 (16x16
// form) or 4 (32x32 form), so any tile width that is a multiple of 16 can
// pair them.
__global__ void geglu_pack_kernel(const f16* __restrict__ w, const f16* __restrict__ b,
                                  f16* __restrict__ wo, f16* __restrict__ bo, int d, int K) {
  const int r = blockIdx.x;  // packed row
  const int q = r >> 3, s = r & 7;
  const int src = s < 4 ? 4 * q + s : d + 4 * q + (s - 4);
  for (int k = threadIdx.x; k < K; k += blockDim.x) wo[(size_t)r * K + k] = w[(size_t)src * K + k];
  if (threadIdx.x == 0 && b && bo) bo[r] = b[src];
}

// [rows, cols] -> [cols, rows_pad] transpose used to bring operands of
// dlm_gemm_fp16 into K-contiguous form: out[c * ld_out + r] = in[r][c] for
// r < rows and 0 for rows <= r < rows_pad (the K padding), so the whole
// destination is written by the kernel and no clearing pass is needed.
__global__ void transpose_kernel(const f16* __restrict__ in, f16* __restrict__ out, int rows,
                                 int cols, int ld_out, int rows_pad) {
  __shared__ f16 tile[32][33];
  const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
  const int tx = threadIdx.x, ty = threadIdx.y;
  for (int r = ty; r < 32; r += 8) {
    const int rr = r0 + r, cc = c0 + tx;
    tile[r][tx] = (rr < rows && cc < cols) ? in[(size_t)rr * cols + cc] : (f16)0.0f;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int cc = c0 + r, rr = r0 + tx;
    if (cc < cols && rr < rows_pad) out[(size_t)cc * ld_out + rr] = tile[tx][r];
  }
}

// out[r * ld_out + k] = in[r * ld_in + k] for k < K, 0 for K <= k < ld_out
// (rows of an operand copied to an aligned, zero-padded row stride).
__global__ void pad_k_kernel(const f16* __restrict__ in, int ld_in, f16* __restrict__ out,
                                int ld_out, int rows, int K) {
  const long long n = (long long)rows * ld_out;
  GRID_STRIDE(i, n) {
    const long long r = i / ld_out;
    const int k = (int)(i - r * ld_out);
    out[i] = k < K ? in[r * ld_in + k] : (f16)0.0f;
  }
}

int nchw_to_nhwc(const void* in, void* out, int N, int C, int HW, int C_pad, hipStream_t s) {
  dim3 grid((HW + 31) / 32, (std::max(C, C_pad) + 31) / 32, N);
  DLM_LAUNCH("nchw_to_nhwc_kernel", nchw_to_nhwc_kernel, grid, dim3(32, 8), 0, s, (const f16*)in, (f16*)out, C,
                     HW, C_pad);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int nhwc_to_nchw(const void* in, void* out, int N, int C, int HW, int C_pad, hipStream_t s) {
  dim3 grid((HW + 31) / 32, (C + 31) / 32, N);
  DLM_LAUNCH("nhwc_to_nchw_kernel", nhwc_to_nchw_kernel, grid, dim3(32, 8), 0, s, (const f16*)in, (f16*)out, C,
                     HW, C_pad);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int conv_weight_pack_add(const void* w, void* out, int Cout, int Cin, int KH, int KW, int Cin_pad,
                         int ld, int col0, hipStream_t s) {
  const long long total = (long long)Cout * KH * KW * Cin;
  const int blocks = (int)std::min<long long>((total + 255) / 256, 65536);
  DLM_LAUNCH("conv_weight_pack_add_kernel", conv_weight_pack_add_kernel, dim3(blocks), dim3(256), 0, s, (const f16*)w,
                     (f16*)out, Cout, Cin, KH * KW, Cin_pad, ld, col0);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int conv_weight_pack(const void* w, void* out, int Cout, int Cin, int KH, int KW, int Cin_pad,
                     int ld, int col0, hipStream_t s) {
  const long long total = (long long)Cout * KH * KW * Cin_pad;
  const int blocks = (int)std::min<long long>((total + 255) / 256, 65536);
  DLM_LAUNCH("conv_weight_pack_kernel", conv_weight_pack_kernel, dim3(blocks), dim3(256), 0, s, (const f16*)w,
                     (f16*)out, Cout, Cin, KH * KW, Cin_pad, ld, col0);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

// LayerNorm folded into a following linear, weight side: row n of W_out is
// fp16(W[n] * gamma) (gamma absent: a copy), c1[n] = sum_k W_out[n][k] (of the
// rounded values), c2[n] = sum_k beta[k] W[n][k] + bias[n], both in fp32.
// One 256-thread block per row; fixed-order reduction (deterministic).
// w and wo may be the same rows (in-place fold, ldo == ldw): each element is
// read and then written by the same thread, so they carry no __restrict__.
__global__ void ln_fold_kernel(const f16* w, int ldw, int K,
                               const f16* __restrict__ gamma, const f16* __restrict__ beta,
                               const f16* __restrict__ bias, f16* wo, int ldo,
                               float* __restrict__ c1, float* __restrict__ c2) {
  const int n = blockIdx.x, tid = threadIdx.x;
  const f16* wr = w + (size_t)n * ldw;
  f16* orow = wo + (size_t)n * ldo;
  float a = 0.0f, b = 0.0f;
  for (int k = tid; k < K; k += blockDim.x) {
    const float x = (float)wr[k];
    const f16 f = (f16)(gamma ? x * (float)gamma[k] : x);
    orow[k] = f;
    a += (float)f;
    if (beta) b = __builtin_fmaf((float)beta[k], x, b);
  }
  __shared__ float ra[256], rb[256];
  ra[tid] = a;
  rb[tid] = b;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) {
      ra[tid] += ra[tid + o];
      rb[tid] += rb[tid + o];
    }
    __syncthreads();
  }
  if (tid == 0) {
    c1[n] = ra[0];
    c2[n] = rb[0] + (bias ? (float)bias[n] : 0.0f);
  }
}

int ln_fold(const void* w, int ldw, int N, int K, const void* gamma, const void* beta,
            const void* bias, void* wo, int ldo, float* c1, float* c2, hipStream_t s) {
  DLM_LAUNCH("ln_fold_kernel", ln_fold_kernel, dim3(N), dim3(256), 0, s, (const f16*)w, ldw, K,
             (const f16*)gamma, (const f16*)beta, (const f16*)bias, (f16*)wo, ldo, c1, c2);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

// ---------------------------------------------------------------------------
// Convolution (channels-last) host entry.
// ---------------------------------------------------------------------------
// Geometry of one convolution: per-axis stride, zero padding and dilation.
struct ConvGeom {
  int sh, sw, ph, pw, dh, dw;
};
static inline int conv_out_size(int in, int pad, int dil, int k, int stride) {
  return (in + 2 * pad - dil * (k - 1) - 1) / stride + 1;
}

int conv_nhwc_impl(const dlm_conv_nhwc_args* a, const ConvGeom& g, hipStream_t s) {
  const int Hv = a->upsample ? 2 * a->H : a->H;
  const int Wv = a->upsample ? 2 * a->W : a->W;
  const int Ho = conv_out_size(Hv, g.ph, g.dh, a->KH, g.sh);
  const int Wo = conv_out_size(Wv, g.pw, g.dw, a->KW, g.sw);
  const int C0 = a->C0a + a->C0b;
  const int C1 = a->C1a + a->C1b;
  ConvDesc d{};
  d.s0a = (const f16*)a->src0a;
  d.s0b = (const f16*)a->src0b;
  d.C0a = a->C0a;
  d.C0 = C0;
  d.ld0a = a->ld0a;
  d.ld0b = a->ld0b;
  d.H = a->H;
  d.W = a->W;
  d.Hv = Hv;
  d.Wv = Wv;
  d.KH = a->KH;
  d.KW = a->KW;
  d.stride_h = g.sh;
  d.stride_w = g.sw;
  d.pad_h = g.ph;
  d.pad_w = g.pw;
  d.dil_h = g.dh;
  d.dil_w = g.dw;
  d.up = a->upsample;
  d.K0 = a->KH * a->KW * C0;
  d.s1a = (const f16*)a->src1a;
  d.s1b = (const f16*)a->src1b;
  d.C1a = a->C1a;
  d.C1 = C1;
  d.ld1a = a->ld1a;
  d.ld1b = a->ld1b;
  d.HoWo = Ho * Wo;
  d.Wo = Wo;
  d.M = a->N * Ho * Wo;
  d.generic = (C0 % BK != 0 || a->C0a % BK != 0) ? 1 : 0;
  const size_t in_pix = (size_t)a->N * a->H * a->W;
  d.bytes0a = (unsigned)(in_pix * a->ld0a * 2);
  d.bytes0b = (unsigned)(in_pix * a->ld0b * 2);
  d.bytes1a = (unsigned)((size_t)d.M * a->ld1a * 2);
  d.bytes1b = (unsigned)((size_t)d.M * a->ld1b * 2);
  const int K = d.K0 + C1;
  RowDesc bd{(const f16*)a->weight, a->ldw, a->Cout, K, (unsigned)((size_t)a->Cout * a->ldw * 2)};
  EpiArgs ep = make_epi(a->out, a->ldy, a->bias, a->residual, a->res_ld, d.M, a->Cout, 1.0f, 1.0f,
                        a->act);
  ep.tbias = (const f16*)a->tbias;
  ep.tbias_ld = a->tbias_ld;
  ep.rows_per_sample = d.HoWo;
  ep.out_nchw = a->out_nchw;
  ep.y_f32 = a->out_f32 ? 1 : 0;
  ep.res_f32 = a->res_f32 ? 1 : 0;
  ep.gn_stats = (float2*)a->gn_stats;
  ep.gn_hw = d.HoWo;
  ep.gn_chunks = (d.HoWo + kGnChunk - 1) / kGnChunk;
  t_gn_written = false;
  const int st = launch_gemm(d, bd, ep, d.M, a->Cout, s);
  if (st != DLM_OK || !a->gn_stats || t_gn_written) return st;
  return gn_chunk_stats(a->out, a->ldy, a->N, d.HoWo, a->Cout, (float2*)a->gn_stats, s);
}

}  // namespace dlm

// ===========================================================================
// C ABI
// ===========================================================================
using namespace dlm;

extern "C" {

int dlm_linear_fp16(const void* X, int lda, const void* W, int ldw, const void* bias,
                    const void* R, int ldr, void* Y, int ldy, int M, int N, int K, float alpha,
                    float beta, int act, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(X && W && Y, "NULL operand");
  DLM_REQUIRE(K % 8 == 0 && lda % 8 == 0 && ldw % 8 == 0, "K, lda and ldw must be multiples of 8");
  DLM_REQUIRE(lda >= K && ldw >= K, "lda/ldw smaller than K");
  DLM_REQUIRE(dlm_aligned16(X) && dlm_aligned16(W), "X and W must be 16-byte aligned");
  DLM_REQUIRE(2LL * M * lda < (1LL << 31) && 2LL * N * ldw < (1LL << 31),
              "X or W larger than 2 GiB");
  DLM_REQUIRE(act >= DLM_ACT_NONE && act <= DLM_ACT_GELU, "unknown act");
  if (act == DLM_ACT_GEGLU) {
    DLM_REQUIRE(N % 16 == 0, "GEGLU needs N (interleaved value+gate columns) % 16 == 0");
    DLM_REQUIRE(ldy >= N / 2, "ldy smaller than N/2");
    DLM_REQUIRE(!R || ldr >= N / 2, "ldr smaller than N/2");
  } else {
    DLM_REQUIRE(ldy >= N, "ldy smaller than N");
    DLM_REQUIRE(!R || ldr >= N, "ldr smaller than N");
  }
  return linear_impl(X, lda, W, ldw, bias, R, ldr, Y, ldy, M, N, K, alpha, beta, act,
                     (hipStream_t)stream);
}

int dlm_linear_gn_stats_fp16(const void* X, int lda, const void* W, int ldw, const void* bias,
                             const void* R, int ldr, void* Y, int ldy, int M, int N, int K, float alpha,
                             float beta, int act, int tokens, void* gn_stats, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(gn_stats, "gn_stats is NULL (use dlm_linear_fp16)");
  DLM_REQUIRE(act != DLM_ACT_GEGLU, "gn_stats with a GEGLU output");
  DLM_REQUIRE(tokens > 0 && M % tokens == 0 && tokens <= 16384, "M must be samples x tokens, tokens <= 16384");
  DLM_REQUIRE(N % 8 == 0 && ldy % 8 == 0 && dlm_aligned16(Y) && dlm_aligned16(gn_stats),
              "gn_stats needs N and ldy multiples of 8 and 16-byte aligned Y / gn_stats");
  DLM_REQUIRE(X && W && Y, "NULL operand");
  DLM_REQUIRE(K % 8 == 0 && lda % 8 == 0 && ldw % 8 == 0, "K, lda and ldw must be multiples of 8");
  DLM_REQUIRE(lda >= K && ldw >= K, "lda/ldw smaller than K");
  DLM_REQUIRE(dlm_aligned16(X) && dlm_aligned16(W), "X and W must be 16-byte aligned");
  DLM_REQUIRE(2LL * M * lda < (1LL << 31) && 2LL * N * ldw < (1LL << 31), "X or W larger than 2 GiB");
  DLM_REQUIRE(act >= DLM_ACT_NONE && act <= DLM_ACT_GELU, "unknown act");
  DLM_REQUIRE(ldy >= N && (!R || ldr >= N), "ldy / ldr smaller than N");
  hipStream_t s = (hipStream_t)stream;
  RowDesc ad{(const f16*)X, lda, M, K, (unsigned)((size_t)M * lda * 2)};
  RowDesc bd{(const f16*)W, ldw, N, K, (unsigned)((size_t)N * ldw * 2)};
  EpiArgs ep = make_epi(Y, ldy, bias, R, ldr, M, N, alpha, beta, act);
  ep.gn_stats = (float2*)gn_stats;
  ep.gn_hw = tokens;
  ep.gn_chunks = (tokens + kGnChunk - 1) / kGnChunk;
  t_gn_written = false;
  const int st = launch_gemm(ad, bd, ep, M, N, s);
  if (st != DLM_OK || t_gn_written) return st;
  return gn_chunk_stats(Y, ldy, M / tokens, tokens, N, (float2*)gn_stats, s);
}

int dlm_linear_vt_fp16(const void* X, int lda, const void* W, int ldw, const void* bias, void* Y,
                       int ldy, void* VT, int vt_col0, int tokens, int vt_ld, int M, int N, int K,
                       void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(X && W && Y && VT, "NULL operand");
  DLM_REQUIRE(K % 8 == 0 && lda % 8 == 0 && ldw % 8 == 0, "K, lda and ldw must be multiples of 8");
  DLM_REQUIRE(lda >= K && ldw >= K, "lda/ldw smaller than K");
  DLM_REQUIRE(dlm_aligned16(X) && dlm_aligned16(W), "X and W must be 16-byte aligned");
  DLM_REQUIRE(2LL * M * lda < (1LL << 31) && 2LL * N * ldw < (1LL << 31),
              "X or W larger than 2 GiB");
  DLM_REQUIRE(vt_col0 >= 0 && vt_col0 < N && vt_col0 % 4 == 0 && N % 4 == 0,
              "vt_col0 must be a multiple of 4 inside [0, N), N % 4 == 0");
  DLM_REQUIRE(tokens > 0 && M % tokens == 0, "M must be a whole number of samples of `tokens` rows");
  DLM_REQUIRE(vt_ld >= tokens, "vt_ld smaller than tokens");
  DLM_REQUIRE(ldy >= vt_col0 && ldy % 4 == 0, "ldy must cover the columns before vt_col0");
  DLM_REQUIRE(((uintptr_t)Y & 7) == 0 && (!bias || ((uintptr_t)bias & 7) == 0),
              "Y and bias must be 8-byte aligned");
  RowDesc ad{(const f16*)X, lda, M, K, (unsigned)((size_t)M * lda * 2)};
  RowDesc bd{(const f16*)W, ldw, N, K, (unsigned)((size_t)N * ldw * 2)};
  EpiArgs ep = make_epi(Y, ldy, bias, nullptr, 0, M, N, 1.0f, 0.0f, DLM_ACT_NONE);
  ep.vt = (f16*)VT;
  ep.vt_col0 = vt_col0;
  ep.vt_tokens = tokens;
  ep.vt_ld = vt_ld;
  return launch_gemm(ad, bd, ep, M, N, (hipStream_t)stream);
}

int dlm_linear_f32out_fp16(const void* X, int lda, const void* W, int ldw, const void* bias,
                           const float* R, int ldr, float* Y, int ldy, int M, int N, int K,
                           float alpha, float beta, int act, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(X && W && Y, "NULL operand");
  DLM_REQUIRE(K % 8 == 0 && lda % 8 == 0 && ldw % 8 == 0, "K, lda and ldw must be multiples of 8");
  DLM_REQUIRE(lda >= K && ldw >= K, "lda/ldw smaller than K");
  DLM_REQUIRE(dlm_aligned16(X) && dlm_aligned16(W), "X and W must be 16-byte aligned");
  DLM_REQUIRE(2LL * M * lda < (1LL << 31) && 2LL * N * ldw < (1LL << 31),
              "X or W larger than 2 GiB");
  DLM_REQUIRE(act == DLM_ACT_NONE || act == DLM_ACT_SILU || act == DLM_ACT_GELU,
              "act must be none/silu/gelu");
  DLM_REQUIRE(ldy >= N && (!R || ldr >= N), "ldy/ldr smaller than N");
  RowDesc ad{(const f16*)X, lda, M, K, (unsigned)((size_t)M * lda * 2)};
  RowDesc bd{(const f16*)W, ldw, N, K, (unsigned)((size_t)N * ldw * 2)};
  EpiArgs ep = make_epi(Y, ldy, bias, R, ldr, M, N, alpha, beta, act);
  ep.y_f32 = 1;
  ep.res_f32 = 1;
  return launch_gemm(ad, bd, ep, M, N, (hipStream_t)stream);
}

int dlm_linear_ln_fp16(const void* X, int lda, const void* W, int ldw, const float* c1,
                       const float* c2, float eps, const void* R, int ldr, void* Y, int ldy, int M,
                       int N, int K, float beta, int act, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(X && W && Y && c1 && c2, "NULL operand");
  DLM_REQUIRE(K % 64 == 0 && lda % 8 == 0 && ldw % 8 == 0, "K must be a multiple of 64, lda and ldw of 8");
  DLM_REQUIRE(lda >= K && ldw >= K, "lda/ldw smaller than K");
  DLM_REQUIRE(dlm_aligned16(X) && dlm_aligned16(W) && dlm_aligned16(c1) && dlm_aligned16(c2),
              "X, W, c1 and c2 must be 16-byte aligned");
  DLM_REQUIRE(2LL * M * lda < (1LL << 31) && 2LL * N * ldw < (1LL << 31), "X or W larger than 2 GiB");
  DLM_REQUIRE(act == DLM_ACT_NONE || act == DLM_ACT_SILU || act == DLM_ACT_GELU || act == DLM_ACT_GEGLU,
              "unknown act");
  DLM_REQUIRE(eps >= 0.0f, "eps must be non-negative");
  if (act == DLM_ACT_GEGLU) {
    DLM_REQUIRE(N % 16 == 0, "GEGLU needs N (interleaved value+gate columns) % 16 == 0");
    DLM_REQUIRE(ldy >= N / 2 && (!R || ldr >= N / 2), "ldy/ldr smaller than N/2");
  } else {
    DLM_REQUIRE(N % 4 == 0, "N must be a multiple of 4");
    DLM_REQUIRE(ldy >= N && (!R || ldr >= N), "ldy/ldr smaller than N");
  }
  RowDesc ad{(const f16*)X, lda, M, K, (unsigned)((size_t)M * lda * 2)};
  RowDesc bd{(const f16*)W, ldw, N, K, (unsigned)((size_t)N * ldw * 2)};
  EpiArgs ep = make_epi(Y, ldy, nullptr, R, ldr, M, N, 1.0f, beta, act);
  ep.ln_c1 = c1;
  ep.ln_c2 = c2;
  ep.ln_invk = 1.0f / (float)K;
  ep.ln_eps = eps;
  return launch_gemm(ad, bd, ep, M, N, (hipStream_t)stream);
}

int dlm_linear_vt_ln_fp16(const void* X, int lda, const void* W, int ldw, const float* c1,
                          const float* c2, float eps, void* Y, int ldy, void* VT, int vt_col0,
                          int tokens, int vt_ld, int M, int N, int K, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(X && W && Y && VT && c1 && c2, "NULL operand");
  DLM_REQUIRE(K % 64 == 0 && lda % 8 == 0 && ldw % 8 == 0, "K must be a multiple of 64, lda and ldw of 8");
  DLM_REQUIRE(lda >= K && ldw >= K, "lda/ldw smaller than K");
  DLM_REQUIRE(dlm_aligned16(X) && dlm_aligned16(W) && dlm_aligned16(c1) && dlm_aligned16(c2),
              "X, W, c1 and c2 must be 16-byte aligned");
  DLM_REQUIRE(2LL * M * lda < (1LL << 31) && 2LL * N * ldw < (1LL << 31), "X or W larger than 2 GiB");
  DLM_REQUIRE(vt_col0 >= 0 && vt_col0 < N && vt_col0 % 4 == 0 && N % 4 == 0,
              "vt_col0 must be a multiple of 4 inside [0, N), N % 4 == 0");
  DLM_REQUIRE(tokens > 0 && M % tokens == 0, "M must be a whole number of samples of `tokens` rows");
  DLM_REQUIRE(vt_ld >= tokens, "vt_ld smaller than tokens");
  DLM_REQUIRE(ldy >= vt_col0 && ldy % 4 == 0, "ldy must cover the columns before vt_col0");
  DLM_REQUIRE(((uintptr_t)Y & 7) == 0, "Y must be 8-byte aligned");
  DLM_REQUIRE(eps >= 0.0f, "eps must be non-negative");
  RowDesc ad{(const f16*)X, lda, M, K, (unsigned)((size_t)M * lda * 2)};
  RowDesc bd{(const f16*)W, ldw, N, K, (unsigned)((size_t)N * ldw * 2)};
  EpiArgs ep = make_epi(Y, ldy, nullptr, nullptr, 0, M, N, 1.0f, 0.0f, DLM_ACT_NONE);
  ep.vt = (f16*)VT;
  ep.vt_col0 = vt_col0;
  ep.vt_tokens = tokens;
  ep.vt_ld = vt_ld;
  ep.ln_c1 = c1;
  ep.ln_c2 = c2;
  ep.ln_invk = 1.0f / (float)K;
  ep.ln_eps = eps;
  return launch_gemm(ad, bd, ep, M, N, (hipStream_t)stream);
}

int dlm_ln_fold_fp16(const void* W, int ldw, int N, int K, const void* gamma, const void* beta,
                     const void* bias, void* W_out, int ldo, float* c1, float* c2, void* stream) {
  if (N <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(W && W_out && c1 && c2, "NULL operand");
  DLM_REQUIRE(ldw >= K && ldo >= K, "ldw/ldo smaller than K");
  // in place only row for row: any other overlap of W and W_out would let one
  // block overwrite rows another block still reads
  const char* w0 = (const char*)W;
  const char* w1 = w0 + ((size_t)(N - 1) * ldw + K) * 2;
  const char* o0 = (const char*)W_out;
  const char* o1 = o0 + ((size_t)(N - 1) * ldo + K) * 2;
  if (o0 < w1 && w0 < o1)
    DLM_REQUIRE(W_out == W && ldo == ldw, "W_out overlaps W: only the exact in-place fold (W_out == W, ldo == ldw) is allowed");
  return ln_fold(W, ldw, N, K, gamma, beta, bias, W_out, ldo, c1, c2, (hipStream_t)stream);
}

int dlm_gemm_fp16(const void* A, const void* B, void* C, int M, int N, int K, float alpha,
                  float beta, int transA, int transB, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(A && B && C, "NULL operand");
  hipStream_t s = (hipStream_t)stream;
  // The MFMA core consumes A as [M,K] and B as [N,K] (both K-contiguous).
  // Other orientations are transposed once into scratch.
  const int Kp = (K + 7) & ~7;
  const f16* a_ptr = (const f16*)A;
  const f16* b_ptr = (const f16*)B;
  int lda = K, ldb = K;
  int st = DLM_OK;
  // The scratch copy is written whole by one kernel (values, then the zero K
  // padding): no clearing pass.
  if (transA || Kp != K || !dlm_aligned16(A)) {
    f16* t = (f16*)scratch_slot((size_t)M * Kp * 2, 0, s, &st);
    if (!t) return st;
    if (transA) {  // A stored [K, M]
      DLM_LAUNCH("transpose_kernel", transpose_kernel, dim3((M + 31) / 32, (Kp + 31) / 32), dim3(32, 8), 0, s,
                 (const f16*)A, t, K, M, Kp, Kp);
    } else {
      DLM_LAUNCH("pad_k_kernel", pad_k_kernel, dim3(grid_for((long long)M * Kp)), dim3(256), 0, s,
                 (const f16*)A, K, t, Kp, M, K);
    }
    DLM_LAUNCH_CHECK();
    a_ptr = t;
    lda = Kp;
  }
  if (!transB || Kp != K || !dlm_aligned16(B)) {
    f16* t = (f16*)scratch_slot((size_t)N * Kp * 2, 1, s, &st);
    if (!t) return st;
    if (!transB) {  // B stored [K, N]
      DLM_LAUNCH("transpose_kernel", transpose_kernel, dim3((N + 31) / 32, (Kp + 31) / 32), dim3(32, 8), 0, s,
                 (const f16*)B, t, K, N, Kp, Kp);
    } else {
      DLM_LAUNCH("pad_k_kernel", pad_k_kernel, dim3(grid_for((long long)N * Kp)), dim3(256), 0, s,
                 (const f16*)B, K, t, Kp, N, K);
    }
    DLM_LAUNCH_CHECK();
    b_ptr = t;
    ldb = Kp;
  }
  return linear_impl(a_ptr, lda, b_ptr, ldb, nullptr, beta != 0.0f ? C : nullptr, N, C, N, M, N,
                     Kp, alpha, beta, DLM_ACT_NONE, s);
}

int dlm_geglu_pack_fp16(const void* w, const void* bias, void* w_out, void* bias_out, int d, int K,
                        void* stream) {
  if (d <= 0 || K <= 0) return DLM_OK;
  DLM_REQUIRE(w && w_out, "NULL pointer");
  DLM_REQUIRE(d % 4 == 0, "d must be a multiple of 4");
  DLM_LAUNCH("geglu_pack_kernel", geglu_pack_kernel, dim3(2 * d), dim3(256), 0, (hipStream_t)stream,
                     (const f16*)w, (const f16*)bias, (f16*)w_out, (f16*)bias_out, d, K);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

int dlm_conv_weight_pack_fp16(const void* w, void* out, int Cout, int Cin, int KH, int KW,
                              int Cin_pad, int ld_out, int col0, void* stream) {
  if (Cout <= 0 || Cin <= 0 || KH <= 0 || KW <= 0) return DLM_OK;
  DLM_REQUIRE(w && out, "NULL pointer");
  DLM_REQUIRE(Cin_pad >= Cin, "Cin_pad < Cin");
  DLM_REQUIRE(ld_out >= col0 + KH * KW * Cin_pad, "ld_out too small");
  return conv_weight_pack(w, out, Cout, Cin, KH, KW, Cin_pad, ld_out, col0, (hipStream_t)stream);
}

int dlm_conv_weight_pack_add_fp16(const void* w, void* out, int Cout, int Cin, int KH, int KW,
                                  int Cin_pad, int ld_out, int col0, void* stream) {
  if (Cout <= 0 || Cin <= 0 || KH <= 0 || KW <= 0) return DLM_OK;
  DLM_REQUIRE(w && out, "NULL pointer");
  DLM_REQUIRE(Cin_pad >= Cin, "Cin_pad < Cin");
  DLM_REQUIRE(ld_out >= col0 + KH * KW * Cin_pad, "ld_out too small");
  return conv_weight_pack_add(w, out, Cout, Cin, KH, KW, Cin_pad, ld_out, col0,
                              (hipStream_t)stream);
}

int dlm_nchw_to_nhwc_fp16(const void* in, void* out, int N, int C, int HW, int C_pad,
                          void* stream) {
  if (N <= 0 || C <= 0 || HW <= 0) return DLM_OK;
  DLM_REQUIRE(in && out, "NULL pointer");
  DLM_REQUIRE(C_pad >= C, "C_pad < C");
  return nchw_to_nhwc(in, out, N, C, HW, C_pad, (hipStream_t)stream);
}

int dlm_nhwc_to_nchw_fp16(const void* in, void* out, int N, int C, int HW, int C_pad,
                          void* stream) {
  if (N <= 0 || C <= 0 || HW <= 0) return DLM_OK;
  DLM_REQUIRE(in && out, "NULL pointer");
  DLM_REQUIRE(C_pad >= C, "C_pad < C");
  return nhwc_to_nchw(in, out, N, C, HW, C_pad, (hipStream_t)stream);
}

int dlm_conv2d_nhwc_fp16(const dlm_conv_nhwc_args* a, void* stream) {
  DLM_REQUIRE(a != nullptr, "args is NULL");
  if (a->N <= 0 || a->H <= 0 || a->W <= 0 || a->Cout <= 0 || a->KH <= 0 || a->KW <= 0 ||
      a->C0a <= 0)
    return DLM_OK;
  DLM_REQUIRE(a->src0a && a->weight && a->out, "NULL operand");
  DLM_REQUIRE(a->stride >= 1 && a->pad >= 0, "bad stride/pad");
  DLM_REQUIRE(!a->upsample || a->stride == 1, "upsample requires stride 1");
  DLM_REQUIRE(a->C0b == 0 || a->src0b, "src0b NULL with C0b > 0");
  DLM_REQUIRE(a->C1a == 0 || a->src1a, "src1a NULL with C1a > 0");
  DLM_REQUIRE(a->C1b == 0 || a->src1b, "src1b NULL with C1b > 0");
  const int C0 = a->C0a + a->C0b;
  DLM_REQUIRE(a->C0a % 8 == 0 && a->C0b % 8 == 0 && a->C1a % 8 == 0 && a->C1b % 8 == 0,
              "channel counts must be multiples of 8 (pad the input)");
  DLM_REQUIRE(a->ld0a % 8 == 0 && a->ld0a >= a->C0a, "bad ld0a");
  DLM_REQUIRE(a->C0b == 0 || (a->ld0b % 8 == 0 && a->ld0b >= a->C0b), "bad ld0b");
  DLM_REQUIRE(a->C1a == 0 || (a->ld1a % 8 == 0 && a->ld1a >= a->C1a), "bad ld1a");
  DLM_REQUIRE(a->C1b == 0 || (a->ld1b % 8 == 0 && a->ld1b >= a->C1b), "bad ld1b");
  DLM_REQUIRE(a->C1a + a->C1b == 0 || (C0 % BK == 0 && a->C0a % BK == 0),
              "the 1x1 segment needs 64-aligned segment-0 channels");
  DLM_REQUIRE(a->C1b == 0 || a->C1a % BK == 0, "segment-1 split must be 64-aligned");
  const int K = a->KH * a->KW * C0 + a->C1a + a->C1b;
  DLM_REQUIRE(a->ldw % 8 == 0 && a->ldw >= K, "bad ldw");
  DLM_REQUIRE(dlm_aligned16(a->src0a) && dlm_aligned16(a->weight) &&
                  (!a->src0b || dlm_aligned16(a->src0b)) && (!a->src1a || dlm_aligned16(a->src1a)) &&
                  (!a->src1b || dlm_aligned16(a->src1b)),
              "operands must be 16-byte aligned");
  const int Hv = a->upsample ? 2 * a->H : a->H;
  const int Wv = a->upsample ? 2 * a->W : a->W;
  const int Ho = (Hv + 2 * a->pad - a->KH) / a->stride + 1;
  const int Wo = (Wv + 2 * a->pad - a->KW) / a->stride + 1;
  if (Ho <= 0 || Wo <= 0) return DLM_OK;
  DLM_REQUIRE(a->C1a + a->C1b == 0 || (Ho == a->H && Wo == a->W && !a->upsample),
              "the 1x1 segment needs output resolution == input resolution");
  DLM_REQUIRE(a->out_nchw || a->ldy >= a->Cout, "ldy < Cout");
  DLM_REQUIRE(!a->residual || a->res_ld >= a->Cout, "res_ld < Cout");
  DLM_REQUIRE(!a->tbias || a->tbias_ld >= a->Cout, "tbias_ld < Cout");
  DLM_REQUIRE(a->act == DLM_ACT_NONE || a->act == DLM_ACT_SILU || a->act == DLM_ACT_GELU,
              "conv act must be none/silu/gelu");
  // every operand is addressed through a buffer resource with 32-bit byte
  // offsets; masked vectors use offset 2^31, so each operand stays below that
  const long long in_pix = (long long)a->N * a->H * a->W;
  const long long out_pix = (long long)a->N * Ho * Wo;
  DLM_REQUIRE(2 * in_pix * std::max(a->ld0a, a->ld0b) < (1LL << 31) &&
                  2 * out_pix * std::max(a->ld1a, a->ld1b) < (1LL << 31) &&
                  2LL * a->Cout * a->ldw < (1LL << 31),
              "operand larger than 2 GiB");
  DLM_REQUIRE((C0 % BK == 0 && a->C0a % BK == 0) || a->C0b == 0,
              "channel concatenation needs 64-aligned channel counts");
  if (a->gn_stats) {
    DLM_REQUIRE(!a->out_nchw && !a->out_f32, "gn_stats needs fp16 channels-last output");
    DLM_REQUIRE(a->Cout % 8 == 0 && a->ldy % 8 == 0, "gn_stats needs Cout and ldy multiples of 8");
    DLM_REQUIRE(dlm_aligned16(a->out) && dlm_aligned16(a->gn_stats), "gn_stats: out and gn_stats 16-byte aligned");
    DLM_REQUIRE((long long)Ho * Wo <= 16384, "gn_stats covers at most 16384 output pixels per sample");
  }
  return conv_nhwc_impl(a, ConvGeom{a->stride, a->stride, a->pad, a->pad, 1, 1}, (hipStream_t)stream);
}

}  // extern "C"

namespace dlm {

// Reference-layout conv (NCHW), launch_conv2d (src/kernels/conv2d.cuh:38-40):
// stage the input channels-last (padded to a multiple of 8 channels) in `x`,
// repack the weight into `wp`, run the implicit-GEMM kernel and write NCHW
// straight from the epilogue.  `x` and `wp` are caller-chosen staging
// buffers of conv2d_nchw_staging() bytes each (every byte that the kernels
// read is written first).
static void conv2d_nchw_staging(int N, int Cin, int H, int W, int Cout, int KH, int KW,
                                size_t* x_bytes, size_t* w_bytes) {
  const int Cp = (Cin + 7) & ~7;
  *x_bytes = (size_t)N * H * W * Cp * 2;
  *w_bytes = (size_t)Cout * (size_t)KH * KW * Cp * 2;
}

static int conv2d_nchw_run(const void* in, const void* weight, const void* bias, void* out, int N,
                           int Cin, int H, int W, int Cout, int KH, int KW, const ConvGeom& g,
                           f16* x, f16* wp, hipStream_t s) {
  const int Cp = (Cin + 7) & ~7;
  const int ldw = KH * KW * Cp;  // a multiple of 8
  int st = DLM_OK;
  if ((st = nchw_to_nhwc(in, x, N, Cin, H * W, Cp, s)) != DLM_OK) return st;
  if ((st = conv_weight_pack(weight, wp, Cout, Cin, KH, KW, Cp, ldw, 0, s)) != DLM_OK) return st;
  dlm_conv_nhwc_args a{};
  a.src0a = x;
  a.C0a = Cp;
  a.ld0a = Cp;
  a.N = N;
  a.H = H;
  a.W = W;
  a.KH = KH;
  a.KW = KW;
  a.stride = g.sh;
  a.pad = g.ph;
  a.weight = wp;
  a.ldw = ldw;
  a.Cout = Cout;
  a.bias = bias;
  a.out = out;
  a.ldy = Cout;
  a.out_nchw = 1;
  a.act = DLM_ACT_NONE;
  return conv_nhwc_impl(&a, g, s);
}

// Argument checks shared by both reference-layout conv entry points.  Returns
// DLM_OK with *noop set for the reference's silent no-op cases.
static int conv2d_nchw_check(const void* in, const void* weight, void* out, int N, int Cin, int H,
                             int W, int Cout, int KH, int KW, const ConvGeom& g, bool* noop) {
  *noop = true;
  if (N <= 0 || Cin <= 0 || H <= 0 || W <= 0 || Cout <= 0 || KH <= 0 || KW <= 0) return DLM_OK;
  if (g.sh <= 0 || g.sw <= 0 || g.dh <= 0 || g.dw <= 0) return DLM_OK;
  DLM_REQUIRE(in && weight && out, "NULL operand");
  DLM_REQUIRE(g.ph >= 0 && g.pw >= 0, "negative padding");
  const int Ho = conv_out_size(H, g.ph, g.dh, KH, g.sh);
  const int Wo = conv_out_size(W, g.pw, g.dw, KW, g.sw);
  if (Ho <= 0 || Wo <= 0) return DLM_OK;
  const int Cp = (Cin + 7) & ~7;
  DLM_REQUIRE(2LL * N * H * W * Cp < (1LL << 31) && 2LL * Cout * KH * KW * Cp < (1LL << 31),
              "input or weight larger than 2 GiB");
  *noop = false;
  return DLM_OK;
}

}  // namespace dlm

// The allocation-free conv's staging memory: one array per GPU, resolved to
// a device address with hipGetSymbolAddress once per device (the array's
// name is only a host-side stand-in in host code).
constexpr size_t kNoAllocScratchBytes = DLM_CONV2D_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace dlm {
namespace {
std::mutex g_noalloc_mu;
std::vector<void*> g_noalloc_ptr;  // [device] -> device address of `scratch`

int noalloc_scratch(void** out) {
  int dev = 0;
  DLM_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if ((int)g_noalloc_ptr.size() <= dev) g_noalloc_ptr.resize(dev + 1, nullptr);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    DLM_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(DLM_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch array");
    g_noalloc_ptr[dev] = p;
  }
  *out = g_noalloc_ptr[dev];
  return DLM_OK;
}
}  // namespace
}  // namespace dlm

extern "C" {

int dlm_conv2d_fp16(const void* in, const void* weight, const void* bias, void* out, int N,
                    int Cin, int H, int W, int Cout, int KH, int KW, int stride_h, int stride_w,
                    int pad_h, int pad_w, int dilation_h, int dilation_w, void* stream) {
  const ConvGeom g{stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w};
  bool noop = true;
  int st = conv2d_nchw_check(in, weight, out, N, Cin, H, W, Cout, KH, KW, g, &noop);
  if (st != DLM_OK || noop) return st;
  hipStream_t s = (hipStream_t)stream;
  size_t xb = 0, wb = 0;
  conv2d_nchw_staging(N, Cin, H, W, Cout, KH, KW, &xb, &wb);
  f16* x = (f16*)scratch_slot(xb, 2, s, &st);
  if (!x) return st;
  f16* wp = (f16*)scratch_slot(wb, 3, s, &st);
  if (!wp) return st;
  return conv2d_nchw_run(in, weight, bias, out, N, Cin, H, W, Cout, KH, KW, g, x, wp, s);
}

int dlm_conv2d_fp16_noalloc(const void* in, const void* weight, const void* bias, void* out,
                            int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride_h,
                            int stride_w, int pad_h, int pad_w, int dilation_h, int dilation_w,
                            void* stream) {
  const ConvGeom g{stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w};
  bool noop = true;
  int st = conv2d_nchw_check(in, weight, out, N, Cin, H, W, Cout, KH, KW, g, &noop);
  if (st != DLM_OK || noop) return st;
  size_t xb = 0, wb = 0;
  conv2d_nchw_staging(N, Cin, H, W, Cout, KH, KW, &xb, &wb);
  const size_t x_off = 0, w_off = (xb + 255) & ~size_t(255);
  if (w_off + wb > kNoAllocScratchBytes)
    return fail(DLM_ERR_INVALID_ARG,
                "dlm_conv2d_fp16_noalloc: staging needs " + std::to_string(w_off + wb) +
                    " bytes, above the fixed maximum of " + std::to_string(kNoAllocScratchBytes));
  void* base = nullptr;
  if ((st = noalloc_scratch(&base)) != DLM_OK) return st;
  unsigned char* b = (unsigned char*)base;
  NoSplitScope no_split;  // split-K would need the lazily allocated workspace
  return conv2d_nchw_run(in, weight, bias, out, N, Cin, H, W, Cout, KH, KW, g, (f16*)(b + x_off),
                         (f16*)(b + w_off), (hipStream_t)stream);
}

}  // extern "C"

extern "C" int dlm_gemm_set_variant(int variant) {
  DLM_REQUIRE(variant >= 0, "variant must be >= 0");
  dlm::g_variant = variant;
  return DLM_OK;
}

extern "C" int dlm_gemm_force_split(int splits) {
  DLM_REQUIRE(splits >= 0 && splits <= 64, "splits must be in [0, 64]");
  dlm::g_forced_split = splits;
  return DLM_OK;
}

extern "C" int dlm_gemm_override_shape(int M, int N, int K, int tile_id, int splits) {
  DLM_REQUIRE(tile_id >= 0 && tile_id <= 44 && splits >= 0 && splits <= 64, "bad tile / split");
  if (M == 0 && N == 0 && K == 0) {
    dlm::g_overrides.clear();
    return DLM_OK;
  }
  auto& v = dlm::g_overrides;
  for (size_t i = 0; i < v.size(); ++i)
    if (v[i].M == M && v[i].N == N && v[i].K == K) {
      v.erase(v.begin() + i);
      break;
    }
  if (tile_id != 0 || splits != 0) v.push_back({M, N, K, tile_id, splits});
  return DLM_OK;
}

extern "C" int dlm_gemm_force_tile(int tile_id) {
  DLM_REQUIRE(tile_id >= 0 && tile_id <= 44, "tile_id must be in [0, 44]");
  dlm::g_forced_tile = tile_id;
  return DLM_OK;
}
