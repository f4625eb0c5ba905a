// Flash attention (non-causal, Dh = 64) for gfx950 with fp16 MFMA and an
// fp32 online softmax.
//
// Replaces launch_attention / launch_attention_fast
// (reference src/kernels/attention.cu:393-597, attention_fast.cu:58-286),
// which compute O = softmax(scale * Q K^T) V with fp32 softmax over 16-row
// warp tiles.
//
// Layout of the computation (wave64, v_mfma_f32_32x32x16_f16):
//   * each wave owns 32 queries, a workgroup 4 waves (128 queries) of one
//     (batch, head); K/V tiles of 64 keys are double-buffered in LDS, K as
//     [key][d], V transposed to [d][key] while staging;
//   * scores are computed transposed, S^T = K Q^T (A = K from LDS, B = Q held
//     in registers), so a lane owns one query and 16 of its keys: the row
//     max needs one exchange with the lane 32 apart, not a 32-lane reduction;
//   * the exponentiated scores stay in registers and feed O^T = V^T P^T
//     directly as the B operand (the key order inside a 16-key step is a
//     fixed permutation shared by both operands), so the output accumulator
//     is also lane-per-query and the online-softmax rescale is per lane.
// Q, K, V and O are addressed with independent batch / token / head strides,
// so the fused QKV projection output [B, S, 3C] is read in place.
#include "common.hpp"

namespace dlm {

struct AttnParams {
  const f16* q;
  const f16* k;
  const f16* v;
  f16* o;
  long long q_sb, q_ss, q_sh;
  long long k_sb, k_ss, k_sh;
  long long v_sb, v_ss, v_sh;
  long long o_sb, o_ss, o_sh;
  int Sq, Sk;
  float scale_log2;
};

constexpr int AQ_WAVE = 32;
constexpr int AQ_BLOCK = 128;
constexpr int AKT = 64;      // keys per tile
constexpr int AKS = 64 + 8;  // K tile row stride (halfs)
constexpr int AVS = AKT + 4; // V^T tile row stride (halfs)

__global__ void __launch_bounds__(256) flash_attn_d64_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) f16 ks[2][AKT * AKS];
  __shared__ __attribute__((aligned(16))) f16 vt[2][64 * AVS];

  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5;
  const int qi = blockIdx.x * AQ_BLOCK + wave * AQ_WAVE + (lane & 31);

  const f16* qbase = p.q + b * p.q_sb + h * p.q_sh;
  const f16* kbase = p.k + b * p.k_sb + h * p.k_sh;
  const f16* vbase = p.v + b * p.v_sb + h * p.v_sh;

  f16x8 qf[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    if (qi < p.Sq)
      qf[ds] = *reinterpret_cast<const f16x8*>(qbase + (long long)qi * p.q_ss + ds * 16 + g * 8);
    else
      qf[ds] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }

  // staging: 64 keys x 8 vectors of 8 halfs = 512 vectors, 2 per thread
  u32x4 rk[2], rv[2];
  auto fetch = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int vidx = tid + 256 * i;
      const int key = kt * AKT + (vidx >> 3);
      const int dv = (vidx & 7) * 8;
      if (key < p.Sk) {
        rk[i] = *reinterpret_cast<const u32x4*>(kbase + (long long)key * p.k_ss + dv);
        rv[i] = *reinterpret_cast<const u32x4*>(vbase + (long long)key * p.v_ss + dv);
      } else {
        rk[i] = u32x4{0u, 0u, 0u, 0u};
        rv[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int vidx = tid + 256 * i;
      const int key = vidx >> 3;
      const int dv = (vidx & 7) * 8;
      *reinterpret_cast<u32x4*>(&ks[buf][key * AKS + dv]) = rk[i];
      const f16x8 vv = __builtin_bit_cast(f16x8, rv[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) vt[buf][(dv + e) * AVS + key] = vv[e];
    }
  };

  const int nkt = (p.Sk + AKT - 1) / AKT;
  fetch(0);
  stage(0);
  __syncthreads();

  float m_run = -INFINITY, l_run = 0.0f;
  f32x16 o[2];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    o[0][e] = 0.0f;
    o[1][e] = 0.0f;
  }

  for (int kt = 0; kt < nkt; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nkt;
    if (more) fetch(kt + 1);

    // S^T = K Q^T for keys [kt*64, kt*64+64)
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.0f;
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const f16x8 kf =
            *reinterpret_cast<const f16x8*>(&ks[cur][(kb * 32 + (lane & 31)) * AKS + ds * 16 + g * 8]);
        s[kb] = mfma32x32x16(kf, qf[ds], s[kb]);
      }
    }

    // scale (log2 domain), mask, tile max
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = kt * AKT + kb * 32 + mfma_row(e, lane);
        const float x = key < p.Sk ? s[kb][e] * p.scale_log2 : -INFINITY;
        s[kb][e] = x;
        mt = fmaxf(mt, x);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = exp2f(m_run - m_new);
    float lsum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = exp2f(s[kb][e] - m_new);
        s[kb][e] = pe;
        lsum += pe;
      }
    }
    l_run = l_run * alpha + lsum;
    m_run = m_new;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      o[0][e] *= alpha;
      o[1][e] *= alpha;
    }

    // O^T += V^T P^T, four 16-key steps
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kb = j >> 1;
      const int eb = (j & 1) * 8;
      f16x8 pf;
#pragma unroll
      for (int t = 0; t < 8; ++t) pf[t] = (f16)s[kb][eb + t];
      const int kcol = kb * 32 + (j & 1) * 16 + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const f16* row = &vt[cur][(dt * 32 + (lane & 31)) * AVS];
        const f16x4 lo = *reinterpret_cast<const f16x4*>(row + kcol);
        const f16x4 hi = *reinterpret_cast<const f16x4*>(row + kcol + 8);
        const f16x8 vf = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[dt] = mfma32x32x16(vf, pf, o[dt]);
      }
    }

    if (more) stage(cur ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / l_tot;
  if (qi < p.Sq) {
    f16* obase = p.o + b * p.o_sb + h * p.o_sh + (long long)qi * p.o_ss;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        f16x4 r;
#pragma unroll
        for (int t = 0; t < 4; ++t) r[t] = (f16)(o[dt][4 * gq + t] * inv);
        *reinterpret_cast<f16x4*>(obase + dt * 32 + 8 * gq + 4 * g) = r;
      }
    }
  }
}

int attention_strided(const dlm_attention_args* a, hipStream_t s) {
  AttnParams p;
  p.q = (const f16*)a->q;
  p.k = (const f16*)a->k;
  p.v = (const f16*)a->v;
  p.o = (f16*)a->o;
  p.q_sb = a->q_sb; p.q_ss = a->q_ss; p.q_sh = a->q_sh;
  p.k_sb = a->k_sb; p.k_ss = a->k_ss; p.k_sh = a->k_sh;
  p.v_sb = a->v_sb; p.v_ss = a->v_ss; p.v_sh = a->v_sh;
  p.o_sb = a->o_sb; p.o_ss = a->o_ss; p.o_sh = a->o_sh;
  p.Sq = a->Sq;
  p.Sk = a->Sk;
  p.scale_log2 = a->scale * 1.4426950408889634f;
  const dim3 grid((a->Sq + AQ_BLOCK - 1) / AQ_BLOCK, a->H, a->B);
  hipLaunchKernelGGL(flash_attn_d64_kernel, grid, dim3(256), 0, s, p);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

static bool stride_ok(long long x) { return x % 8 == 0; }

}  // namespace dlm

using namespace dlm;

extern "C" {

int dlm_attention_strided_fp16(const dlm_attention_args* a, void* stream) {
  DLM_REQUIRE(a != nullptr, "args is NULL");
  if (a->B <= 0 || a->H <= 0 || a->Sq <= 0 || a->Sk <= 0 || a->Dh <= 0) return DLM_OK;
  DLM_REQUIRE(a->q && a->k && a->v && a->o, "NULL operand");
  if (a->Dh != 64) return fail(DLM_ERR_UNSUPPORTED, "attention: only Dh == 64 is implemented");
  DLM_REQUIRE(dlm_aligned16(a->q) && dlm_aligned16(a->k) && dlm_aligned16(a->v) &&
                  ((uintptr_t)a->o & 7) == 0,
              "Q/K/V must be 16-byte aligned, O 8-byte aligned");
  DLM_REQUIRE(stride_ok(a->q_sb) && stride_ok(a->q_ss) && stride_ok(a->q_sh) &&
                  stride_ok(a->k_sb) && stride_ok(a->k_ss) && stride_ok(a->k_sh) &&
                  stride_ok(a->v_sb) && stride_ok(a->v_ss) && stride_ok(a->v_sh) &&
                  a->o_sb % 4 == 0 && a->o_ss % 4 == 0 && a->o_sh % 4 == 0,
              "strides must keep 16-byte (Q/K/V) and 8-byte (O) alignment");
  return attention_strided(a, (hipStream_t)stream);
}

int dlm_attention_fp16(const void* q, const void* k, const void* v, void* out, int B, int H,
                       int Sq, int Sk, int Dh, float scale, void* stream) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || Dh <= 0) return DLM_OK;
  dlm_attention_args a{};
  a.q = q; a.k = k; a.v = v; a.o = out;
  a.q_sh = (long long)Sq * Dh; a.q_sb = a.q_sh * H; a.q_ss = Dh;
  a.k_sh = (long long)Sk * Dh; a.k_sb = a.k_sh * H; a.k_ss = Dh;
  a.v_sh = (long long)Sk * Dh; a.v_sb = a.v_sh * H; a.v_ss = Dh;
  a.o_sh = (long long)Sq * Dh; a.o_sb = a.o_sh * H; a.o_ss = Dh;
  a.B = B; a.H = H; a.Sq = Sq; a.Sk = Sk; a.Dh = Dh; a.scale = scale;
  return dlm_attention_strided_fp16(&a, stream);
}

}  // extern "C"
