// Flash attention (non-causal, Dh = 64) for gfx950 with fp16 MFMA and an
// fp32 online softmax.
//
// Replaces launch_attention / launch_attention_fast
// (reference src/kernels/attention.cu:393-597, attention_fast.cu:58-286),
// which compute O = softmax(scale * Q K^T) V with fp32 softmax over 16-row
// warp tiles.
//
// Two kernels share one formulation (wave64, v_mfma_f32_32x32x16_f16):
//   * scores are computed transposed, S^T = K Q^T (A = K from LDS, B = Q held
//     in registers), so a lane owns one query and 16 of its keys per 32-key
//     block: the row max needs one exchange with the lane 32 apart, not a
//     32-lane reduction;
//   * the exponentiated scores stay in registers and feed O^T = V^T P^T
//     directly as the B operand (the key order inside a 16-key step is a
//     fixed permutation shared by both operands), so the output accumulator
//     is also lane-per-query and the online-softmax rescale is per lane.
// flash_vt_pipe_kernel (the UNet's self and cross attention) reads a
// transposed V, DMAs K and V^T tiles into a three-tile LDS ring and
// software-pipelines each tile's scores under the previous tile's softmax;
// it is described at its definition.  flash_attn_d64_kernel (the strided
// entry dlm_attention_strided_fp16, V as [key][d]) uses 4 waves of 32 queries per
// workgroup and double-buffered K / V tiles staged through VGPRs, V
// transposed to [d][key] while staging.
// Q, K, V and O are addressed with independent batch / token / head strides,
// so the fused QKV projection output [B, S, 3C] is read in place.
#include <algorithm>
#include <type_traits>

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

// ===========================================================================
// Flash attention over a transposed V (V^T[b][h][d][key]).
//
// Same lane-per-query formulation as above (S^T = K Q^T, O^T = V^T P^T), but
//   * K and V^T tiles of 64 keys are copied global -> LDS by DMA
//     (buffer_load ... lds) into a three-tile ring, rows of 128 B with the
//     16-byte chunks XOR-swizzled by (row >> 1) & 7, so every fragment is one
//     conflict-free ds_read_b128 and no VGPR staging or LDS transpose exists;
//   * K rows are placed in LDS in a fixed permutation (rows 4..7 and 8..11 of
//     every 16 swapped), chosen so that the eight exponentiated scores a lane
//     feeds to one P^T fragment belong to eight consecutive keys: the matching
//     V^T fragment is then 16 contiguous bytes of a V^T row;
//   * each wave owns one block of 32 queries;
//   * Q is multiplied by c = scale * log2 e once, and every score chain starts
//     its MFMA accumulator at -m (the lane's base), so p = 2^s is one
//     v_exp_f32; the base moves only when a tile's P would overflow fp16 (a
//     rare branch, see the softmax), so there is no per-tile max; masking
//     runs only on a partial last key tile.
// ===========================================================================
typedef int i32x4 __attribute__((ext_vector_type(4)));
#define DLM_LDS __attribute__((address_space(3)))

struct FlashVtParams {
  const f16* q;
  const f16* k;
  const f16* vt;
  f16* o;
  long long q_sb, q_ss, q_sh;
  long long k_sb, k_ss, k_sh;
  long long vt_sb, vt_sh;  // element offset of head (b, h) in V^T; row d at + d * vt_ld
  long long o_sb, o_ss, o_sh;
  int vt_ld;
  int Sq, Sk;
  float c;                  // scale * log2(e)
  unsigned k_bytes, vt_bytes;
  int nqb, H, B;            // query blocks per head, heads, batch: the 1-D grid's shape
};

__device__ __forceinline__ i32x4 fa_rsrc(const void* p, unsigned bytes) {
  const uint64_t a = (uint64_t)p;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// M0 carries the LDS destination; nothing else in this file uses M0 (the
// compiler's own code never reads it here), so the clobber is safe even
// though the compiler treats M0 as reserved.
__device__ __forceinline__ void fa_dma16(const i32x4& r, const unsigned char DLM_LDS* dst, int voff) {
  const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)dst);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds),
               "v"(voff), "s"(r)
               : "memory", "m0");
}

#define FA_WAIT_VM(n) \
  __builtin_amdgcn_s_waitcnt((((n)&15) | (((n) >> 4) << 14)) | (0x7 << 4) | (0xF << 8))

// LDS row r of a K tile holds key fa_perm(r) of the tile.
__device__ __forceinline__ int fa_perm(int r) {
  const int q = r & 12;
  return (q == 4 || q == 8) ? (r ^ 12) : r;
}

constexpr int FA_TK = 64;             // keys per tile
constexpr int FA_TILE = FA_TK * 128;  // bytes of one K (or V^T) tile
constexpr int FA_STAGE = 2 * FA_TILE;
constexpr int FA_NS = 3;
constexpr int kFaOOB = (int)0x80000000;

// x of this lane and of lane ^ 32, as the pair (s[0], s[1]) in some order:
// v_permlane32_swap exchanges the upper half of its first operand with the
// lower half of its second, so with x in both every lane ends holding its
// own value and its partner's (a VALU op; a shuffle is an LDS round trip).
// max and + over the pair are symmetric, so the results equal the shuffle's.
__device__ __forceinline__ float fa_max_halves(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float fa_sum_halves(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Software pipeline, one 32-query block per wave (more waves beat sharing
// K/V fragments between two blocks: the softmax is VALU work that other
// waves' MFMAs hide): the scores of tile kt+1 (MFMA) are issued before the
// softmax of tile kt (VALU), so each wave's own MFMAs run in the shadow of
// its exp / convert / row-sum work.  The barrier that publishes tile kt+1 also
// proves every wave is done with tile kt-1, whose buffer then receives tile
// kt+2: one tile of DMA latency hidden, three buffers.  Full tiles carry no
// masking code; the rescale is a real (rare) branch; the row sum is taken
// over the fp16 P the MFMA consumes, two terms per dot2.
// NWV waves per workgroup (4: 128 queries; 2: 64 queries for grids that
// would otherwise leave SIMDs with a single wave).  Each wave issues 8 / NWV
// of the 8-row DMA groups of every K and V^T tile.
template <int NWV>
__global__ void __launch_bounds__(NWV * 64) __attribute__((amdgpu_waves_per_eu(2)))
flash_vt_pipe_kernel(FlashVtParams p) {
  constexpr int DI = 8 / NWV;  // DMA instructions per wave per operand tile
  __shared__ __attribute__((aligned(1024))) unsigned char smem_g[FA_NS * FA_STAGE];
  unsigned char DLM_LDS* smem = (unsigned char DLM_LDS*)smem_g;
  // XCD-aware placement: the hardware deals workgroup i to XCD i % 8 and each
  // XCD has its own L2, so consecutive logical blocks (the query blocks of one
  // head, then the next head) are given to one XCD; each L2 then fetches the
  // K / V^T of its own heads only.
  int b, h, qb;
  {
    const int total = p.nqb * p.H * p.B;
    const int q8 = total >> 3, r8 = total & 7;
    const int x = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int logical = x * q8 + (x < r8 ? x : r8) + slot;
    qb = logical % p.nqb;
    const int bh = logical / p.nqb;
    h = bh % p.H;
    b = bh / p.H;
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int q0 = qb * (NWV * 32) + wave * 32;

  f16x8 qf[4];  // this wave's 32 queries, loaded below
  const i32x4 rk = fa_rsrc(p.k, p.k_bytes);
  const i32x4 rv = fa_rsrc(p.vt, p.vt_bytes);
  // DMA instruction i of this wave: LDS row r of the tile, 16-byte chunk c of
  // it; the K row holds key fa_perm(r), the V^T row's chunk keys 8c .. 8c+7
  auto dma_row = [&](int i) { return (wave * DI + i) * 8 + (lane >> 3); };
  auto dma_chunk = [&](int r) { return (lane & 7) ^ ((r >> 1) & 7); };
  int koff[DI], voff[DI];
#pragma unroll
  for (int i = 0; i < DI; ++i) {
    const int r = dma_row(i), c = dma_chunk(r);
    koff[i] = (int)((b * p.k_sb + h * p.k_sh + (long long)fa_perm(r) * p.k_ss + c * 8) * 2);
    voff[i] = (int)((b * p.vt_sb + h * p.vt_sh + (long long)r * p.vt_ld + c * 8) * 2);
  }
  const int kstep = (int)(FA_TK * p.k_ss * 2);
  // keys past Sk exist only in a partial last tile; their rows and chunks are
  // recomputed there rather than held in registers for the whole loop
  auto issue = [&](int buf, int kt) {
    unsigned char DLM_LDS* st = smem + buf * FA_STAGE;
    const int k0 = kt * FA_TK;
    if (k0 + FA_TK <= p.Sk) {  // a full tile (all but a partial last one): no masking
#pragma unroll
      for (int i = 0; i < DI; ++i) fa_dma16(rk, st + (wave * DI + i) * 1024, koff[i] + kt * kstep);
#pragma unroll
      for (int i = 0; i < DI; ++i)
        fa_dma16(rv, st + FA_TILE + (wave * DI + i) * 1024, voff[i] + kt * (FA_TK * 2));
      return;
    }
#pragma unroll
    for (int i = 0; i < DI; ++i) {
      const bool in = k0 + fa_perm(dma_row(i)) < p.Sk;
      fa_dma16(rk, st + (wave * DI + i) * 1024, in ? koff[i] + kt * kstep : kFaOOB);
    }
#pragma unroll
    for (int i = 0; i < DI; ++i) {
      const bool in = k0 + dma_chunk(dma_row(i)) * 8 < p.Sk;
      fa_dma16(rv, st + FA_TILE + (wave * DI + i) * 1024, in ? voff[i] + kt * (FA_TK * 2) : kFaOOB);
    }
  };
  auto frag = [&](const unsigned char DLM_LDS* st, int row, int chunk) -> f16x8 {
    const int c = chunk ^ ((row >> 1) & 7);
    return *reinterpret_cast<const f16x8 DLM_LDS*>(st + row * 128 + c * 16);
  };
  // S^T = init + K (c Q)^T of the tile in st: lane = query, element e of
  // block kb = LDS key row kb*32 + 8*(e>>2) + 4g + (e&3).  init is the
  // accumulator's start: -m (the lane's running max, broadcast), so the
  // scores leave the MFMA already shifted and p = 2^s needs no VALU
  // subtraction.
  // The two key blocks' chains alternate, so consecutive MFMAs are
  // independent and VALU work can issue between dependent ones.
  auto scores = [&](const unsigned char DLM_LDS* st, f32x16 (&sv)[2], const f32x16& init) {
    f16x8 kf[2][4];
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) kf[kb][ds] = frag(st, kb * 32 + (lane & 31), 2 * ds + g);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) sv[kb] = mfma32x32x16(kf[kb][0], qf[0], init);
#pragma unroll
    for (int ds = 1; ds < 4; ++ds)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) sv[kb] = mfma32x32x16(kf[kb][ds], qf[ds], sv[kb]);
  };

  const int nkt = (p.Sk + FA_TK - 1) / FA_TK;
  issue(0, 0);
  if (nkt > 1) issue(1, 1);

  // Q scaled by c = scale * log2(e) once (one fp16 rounding of q * c), so the
  // scores come out of the MFMA in the exponent's units.  Loaded after the
  // first tiles' DMA is issued, so the two latencies overlap (loaded first,
  // the scaling's wait held the DMA back by one memory round trip).
  // Rows past Sq load row Sq - 1 and scale it by 0: no branch around the
  // loads (the compiler copies, and waits for, a load's result inside one).
  // A padded row's scores stay in its own lane and its output is never
  // stored.
  {
    const int qi = q0 + (lane & 31);
    const bool qin = qi < p.Sq;
    const f16* qp = p.q + b * p.q_sb + h * p.q_sh + (long long)(qin ? qi : p.Sq - 1) * p.q_ss + g * 8;
    f16x8 v[4];
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) v[ds] = *reinterpret_cast<const f16x8*>(qp + ds * 16);
    const float cq = qin ? p.c : 0.0f;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
      for (int t = 0; t < 8; ++t) v[ds][t] = (f16)((float)v[ds][t] * cq);
      qf[ds] = v[ds];
    }
  }


  // Running state, in log2 units: the scores of a tile arrive as s - m with m
  // the lane's current base (negm = -m broadcast is every score chain's
  // accumulator start).  The base moves only when a tile's P would overflow
  // fp16 (a rare, wave-uniform branch; see softmax below).  The next tile's
  // scores are issued before this tile's softmax; when that softmax moves the
  // base it re-bases them too.
  float l_run = 0.0f;
  f32x16 negm;
  f32x16 o[2];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    o[0][e] = 0.0f;
    o[1][e] = 0.0f;
  }

  // p = 2^s of the 16 scores of one key block into two P fragments
  auto exp_block = [&](const f32x16& sk, f16x8& p0, f16x8& p1) {
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const f16x2 hr = f16x2{(f16)__builtin_amdgcn_exp2f(sk[e]), (f16)__builtin_amdgcn_exp2f(sk[e + 1])};
      f16x8& d8 = e < 8 ? p0 : p1;
      d8[e & 7] = hr[0];
      d8[(e & 7) + 1] = hr[1];
    }
  };
  // the lane's sum of its 32 fp16 P values (two terms per dot2, fp32
  // accumulate), in four chains so the check below waits on four dot2
  auto row_sum = [&](const f16x8 (&pf)[4]) {
    float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < 8; t += 2)
        l[j] = __builtin_amdgcn_fdot2(f16x2{pf[j][t], pf[j][t + 1]}, f16x2{(f16)1.0f, (f16)1.0f}, l[j], false);
    return (l[0] + l[1]) + (l[2] + l[3]);
  };
  // softmax of one tile's (shifted) scores sv into fp16 P; sn, when given,
  // holds the next tile's scores, already issued against the current base.
  // No per-tile max: p = 2^s is exact to fp16 precision up to 65504, so the
  // base has to move only when some p of the tile overflowed, which the row
  // sum the denominator needs anyway shows (it is then not finite; 32 finite
  // fp16 values sum to at most 2.1e6).  The first tile (base 0) also moves it
  // down when its row sum is below 2^-8, so the row's largest p is a normal
  // fp16 number and a row whose scores all lie far below 0 cannot underflow
  // every p.  The rare branch takes the tile's max, re-bases the running
  // state, this tile and the already issued next tile, and redoes the
  // exponentials.
  auto softmax = [&](f32x16 (&sv)[2], f16x8 (&pf)[4], f32x16* sn, bool first) {
    exp_block(sv[0], pf[0], pf[1]);
    exp_block(sv[1], pf[2], pf[3]);
    float lsum = row_sum(pf);
    const bool low = first && fa_sum_halves(lsum) < (1.0f / 256.0f);
    if (__builtin_amdgcn_ballot_w64(!(lsum <= 3.0e6f) || low) != 0) {
      asm volatile("" ::: "memory");  // a real branch: never evaluated speculatively
      float mt = sv[0][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) mt = fmaxf(mt, sv[kb][e]);
      mt = fa_max_halves(mt);
      const float d = first ? mt : fmaxf(mt, 0.0f);
      const float alpha = __builtin_amdgcn_exp2f(-d);
      l_run *= alpha;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        o[0][e] *= alpha;
        o[1][e] *= alpha;
        negm[e] -= d;
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) sv[kb][e] -= d;
      if (sn) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) sn[kb][e] -= d;
      }
      exp_block(sv[0], pf[0], pf[1]);
      exp_block(sv[1], pf[2], pf[3]);
      lsum = row_sum(pf);
    }
    l_run += lsum;
  };
  // O^T += V^T P^T over four 16-key steps (step j: tile keys 16j + 8g + [0, 8))
  auto pv = [&](const f16x8 (&vf)[8], const f16x8 (&pf)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) o[dt] = mfma32x32x16(vf[j * 2 + dt], pf[j], o[dt]);
  };
  auto vread = [&](const unsigned char DLM_LDS* st, f16x8 (&vf)[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) vf[j * 2 + dt] = frag(st + FA_TILE, dt * 32 + (lane & 31), 2 * j + g);
  };

  // prologue: tile 0 published, its scores issued
  if (nkt > 1) {
    FA_WAIT_VM(2 * DI);  // tile 1's requests may still be in flight
  } else {
    FA_WAIT_VM(0);
  }
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);

  // one tile at ring position c: sc holds its scores, the next tile's
  // scores go to sn
  auto body = [&](int kt, int c, f32x16 (&sc)[2], f32x16 (&sn)[2]) {
    const int nxt = c == FA_NS - 1 ? 0 : c + 1;
    const int nn = nxt == FA_NS - 1 ? 0 : nxt + 1;
    FA_WAIT_VM(0);  // tile kt+1 (this wave's part)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 2 < nkt) issue(nn, kt + 2);
    const unsigned char DLM_LDS* st = smem + c * FA_STAGE;
    scores(smem + nxt * FA_STAGE, sn, negm);  // tile kt+1, in the shadow of the softmax below
    f16x8 vf[8];
    vread(st, vf);
    f16x8 pf[4];
    // the instruction mix of the block up to the growth branch, interleaved:
    // the K fragments of the first k-step, then per score MFMA one more
    // fragment read and five VALU (max, exponentials, converts)
    softmax(sc, pf, sn, kt == 0);  // tiles before the last are full: no mask
    pv(vf, pf);
  };
  int cur = 0;  // ring position of the current tile
  auto step = [&](int kt, f32x16 (&sc)[2], f32x16 (&sn)[2]) {
    body(kt, cur, sc, sn);
    cur = cur == FA_NS - 1 ? 0 : cur + 1;
  };
  // last tile: its keys may end inside the tile
  auto last = [&](f32x16 (&sc)[2]) {
    const int kt = nkt - 1;
    if (kt * FA_TK + FA_TK > p.Sk) {
      // element e of key block kb holds tile key fa_perm(kb*32 + mfma_row(e, lane))
      // = 8g + kb*32 + 16*(e>>3) + 4*((e>>2)&1) + (e&3): one lane-dependent
      // limit against per-element constants
      const int lim = p.Sk - kt * FA_TK - 8 * g;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (kb * 32 + 16 * (e >> 3) + 4 * ((e >> 2) & 1) + (e & 3) >= lim) sc[kb][e] = -INFINITY;
    }
    f16x8 vf[8];
    vread(smem + cur * FA_STAGE, vf);
    f16x8 pf[4];
    softmax(sc, pf, nullptr, kt == 0);
    pv(vf, pf);
  };
  // two tiles per iteration with the score buffers swapping roles, so no
  // loop-carried copy of the next tile's 32 scores is needed
  f32x16 sa[2], sb[2];
  // the base starts at 0: tile 0's softmax moves it to that tile's max when
  // a p overflows or the row's sum is below 2^-8
#pragma unroll
  for (int e = 0; e < 16; ++e) negm[e] = 0.0f;
  scores(smem, sa, negm);
  int kt = 0;
  // six tiles per iteration: the ring position and the score buffers both
  // come back to where they started, so every LDS address in the body is a
  // constant offset from one base
  for (; kt + 6 < nkt; kt += 6) {
    body(kt, 0, sa, sb);
    body(kt + 1, 1, sb, sa);
    body(kt + 2, 2, sa, sb);
    body(kt + 3, 0, sb, sa);
    body(kt + 4, 1, sa, sb);
    body(kt + 5, 2, sb, sa);
  }
  for (; kt + 2 < nkt; kt += 2) {
    step(kt, sa, sb);
    step(kt + 1, sb, sa);
  }
  if (kt + 1 < nkt) {
    step(kt, sa, sb);
    last(sb);
  } else {
    last(sa);
  }
  FA_WAIT_VM(0);

  // O leaves through LDS: a lane holds 8-byte pieces of one query row, so
  // direct stores would write 32 rows in 16-byte fragments per instruction;
  // staged, every store instruction writes four whole 128-byte head rows.
  // When every workgroup ends together (two-tile cross attention) the
  // fragment stores took several microseconds of the launch.
  const int ql = lane & 31;
  const float l_tot = fa_sum_halves(l_run);
  const float inv = 1.0f / l_tot;
  __syncthreads();  // every wave is done reading the K / V^T ring
  unsigned char DLM_LDS* ob = smem + wave * 4096;  // this wave's 32 rows x 128 B, chunks swizzled
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      f16x4 r;
#pragma unroll
      for (int t = 0; t < 4; ++t) r[t] = (f16)(o[dt][4 * gq + t] * inv);
      const int chunk = dt * 4 + gq;
      *reinterpret_cast<f16x4 DLM_LDS*>(ob + ql * 128 + ((chunk ^ (ql & 7)) * 16) + g * 8) = r;
    }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = i * 4 + (lane >> 4), piece = lane & 15;
    const f16x4 r = *reinterpret_cast<const f16x4 DLM_LDS*>(ob + row * 128 + (((piece >> 1) ^ (row & 7)) * 16) +
                                                             (piece & 1) * 8);
    const int qi = q0 + row;
    if (qi < p.Sq)
      *reinterpret_cast<f16x4*>(p.o + b * p.o_sb + h * p.o_sh + (long long)qi * p.o_ss + piece * 4) = r;
  }
}

int attention_vt(const dlm_attention_vt_args* a, hipStream_t s) {
  FlashVtParams p;
  p.q = (const f16*)a->q;
  p.k = (const f16*)a->k;
  p.vt = (const f16*)a->vt;
  p.o = (f16*)a->o;
  p.q_sb = a->q_sb; p.q_ss = a->q_ss; p.q_sh = a->q_sh;
  p.k_sb = a->k_sb; p.k_ss = a->k_ss; p.k_sh = a->k_sh;
  p.vt_sb = a->vt_sb; p.vt_sh = a->vt_sh; p.vt_ld = a->vt_ld;
  p.o_sb = a->o_sb; p.o_ss = a->o_ss; p.o_sh = a->o_sh;
  p.Sq = a->Sq;
  p.Sk = a->Sk;
  p.c = a->scale * 1.4426950408889634f;
  p.k_bytes = (unsigned)a->k_bytes;
  p.vt_bytes = (unsigned)a->vt_bytes;
  // One 32-query block per wave: the softmax is VALU work that only other
  // waves' MFMAs can hide, so more waves beat sharing K/V fragments between
  // two query blocks (2x4096^2 x10 heads: 144 us vs 170 us).  Grids of fewer
  // than two 128-query workgroups per CU (1024 tokens x 20 heads x 2) take
  // 64-query workgroups: twice the K/V staging, but waves spread evenly.
  // Cross attention (every key in at most two tiles): always 128-query
  // workgroups, whose one K/V staging serves twice the queries.
  p.H = a->H;
  p.B = a->B;
  // the 1-D grid counts query blocks x heads x batch in int (host and kernel)
  if ((long long)((a->Sq + 63) / 64) * a->H * a->B >= (1LL << 31))
    return fail(DLM_ERR_UNSUPPORTED, "attention: more than 2^31 query blocks x heads x batch");
  if (a->Sk > 2 * FA_TK && (long long)((a->Sq + 127) / 128) * a->H * a->B < 512) {
    p.nqb = (a->Sq + 63) / 64;
    DLM_LAUNCH("flash_vt_pipe_kernel<2>", flash_vt_pipe_kernel<2>, dim3(p.nqb * p.H * p.B), dim3(128), 0, s, p);
  } else {
    p.nqb = (a->Sq + 127) / 128;
    DLM_LAUNCH("flash_vt_pipe_kernel<4>", flash_vt_pipe_kernel<4>, dim3(p.nqb * p.H * p.B), dim3(256), 0, s, p);
  }
  DLM_LAUNCH_CHECK();
  return DLM_OK;
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
  DLM_LAUNCH("flash_attn_d64_kernel", flash_attn_d64_kernel, grid, dim3(256), 0, s, p);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

static bool stride_ok(long long x) { return x % 8 == 0; }

// ---------------------------------------------------------------------------
// Row softmax of fp32 scores into fp16 probabilities: the middle step of the
// VAE mid-block attention (one head, Dh = 512, S = h*w of the latent), which
// runs as scores GEMM -> softmax -> P V GEMM instead of a flash kernel (the
// reference's generic attention kernel, src/kernels/attention.cu:137-219,
// likewise keeps a whole score row and takes a two-pass softmax).
// One 256-thread block per row.  Rows up to 256 * 4 * VPT columns are held in
// registers (one read of S); longer rows take a second read.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void block_max_sum(float& m, float& l, float* red) {
  // merge (max, sum-of-exp) pairs: wave level, then across the 4 waves
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float mo = __shfl_xor(m, o, 64), lo = __shfl_xor(l, o, 64);
    const float mn = fmaxf(m, mo);
    l = (mn == -INFINITY) ? 0.0f : l * __expf(m - mn) + lo * __expf(mo - mn);
    m = mn;
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[2 * w] = m;
    red[2 * w + 1] = l;
  }
  __syncthreads();
  m = -INFINITY;
  l = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float mo = red[2 * i], lo = red[2 * i + 1];
    const float mn = fmaxf(m, mo);
    l = (mn == -INFINITY) ? 0.0f : l * __expf(m - mn) + lo * __expf(mo - mn);
    m = mn;
  }
}

// Row softmax of `cols` scores (any count; lds a multiple of 4 and at least
// cols rounded up to 4) into fp16 P, writing colw (a multiple of 4, >= cols)
// columns: probabilities for [0, cols), zeros for [cols, colw).
__device__ __forceinline__ float4 mask4(float4 x, int v, int cols) {
  const int c = 4 * v;
  if (c + 0 >= cols) x.x = -INFINITY;
  if (c + 1 >= cols) x.y = -INFINITY;
  if (c + 2 >= cols) x.z = -INFINITY;
  if (c + 3 >= cols) x.w = -INFINITY;
  return x;
}

template <int VPT>
__global__ void __launch_bounds__(256)
softmax_rows_kernel(const float* __restrict__ S, long long lds, f16* __restrict__ P, long long ldp,
                    int cols, int colw) {
  __shared__ float red[8];
  const float* row = S + (size_t)blockIdx.x * lds;
  f16* prow = P + (size_t)blockIdx.x * ldp;
  const int nv = (cols + 3) >> 2;  // vectors holding scores
  const int nw = colw >> 2;        // vectors written
  const float4 ninf = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
  const int t = threadIdx.x;
  float m = -INFINITY, l = 0.0f;
  if (VPT > 0) {
    float4 x[VPT > 0 ? VPT : 1];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = t + i * 256;
      x[i] = v < nv ? mask4(reinterpret_cast<const float4*>(row)[v], v, cols) : ninf;
      m = fmaxf(m, fmaxf(fmaxf(x[i].x, x[i].y), fmaxf(x[i].z, x[i].w)));
    }
    if (m != -INFINITY) {
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        l += __expf(x[i].x - m) + __expf(x[i].y - m) + __expf(x[i].z - m) + __expf(x[i].w - m);
    }
    block_max_sum(m, l, red);
    const float inv = 1.0f / l;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int v = t + i * 256;
      if (v < nw) {
        const f16x4 o = {(f16)(__expf(x[i].x - m) * inv), (f16)(__expf(x[i].y - m) * inv),
                         (f16)(__expf(x[i].z - m) * inv), (f16)(__expf(x[i].w - m) * inv)};
        *reinterpret_cast<f16x4*>(prow + 4 * v) = o;
      }
    }
  } else {
    for (int v = t; v < nv; v += 256) {
      const float4 x = mask4(reinterpret_cast<const float4*>(row)[v], v, cols);
      const float mx = fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w));
      const float mn = fmaxf(m, mx);
      l = (mn == -INFINITY) ? 0.0f
                            : l * __expf(m - mn) + __expf(x.x - mn) + __expf(x.y - mn) +
                                  __expf(x.z - mn) + __expf(x.w - mn);
      m = mn;
    }
    block_max_sum(m, l, red);
    const float inv = 1.0f / l;
    for (int v = t; v < nw; v += 256) {
      const float4 x = v < nv ? mask4(reinterpret_cast<const float4*>(row)[v], v, cols) : ninf;
      const f16x4 o = {(f16)(__expf(x.x - m) * inv), (f16)(__expf(x.y - m) * inv),
                       (f16)(__expf(x.z - m) * inv), (f16)(__expf(x.w - m) * inv)};
      *reinterpret_cast<f16x4*>(prow + 4 * v) = o;
    }
  }
}

int softmax_rows(const float* S, long long lds, f16* P, long long ldp, int rows, int cols, int colw,
                 hipStream_t s) {
  if (colw <= 256 * 4 * 4)
    DLM_LAUNCH("softmax_rows_kernel<4>", softmax_rows_kernel<4>, dim3(rows), dim3(256), 0, s, S, lds, P, ldp, cols, colw);
  else if (colw <= 256 * 4 * 16)
    DLM_LAUNCH("softmax_rows_kernel<16>", softmax_rows_kernel<16>, dim3(rows), dim3(256), 0, s, S, lds, P, ldp, cols, colw);
  else
    DLM_LAUNCH("softmax_rows_kernel<0>", softmax_rows_kernel<0>, dim3(rows), dim3(256), 0, s, S, lds, P, ldp, cols, colw);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

// ---------------------------------------------------------------------------
// Reference-layout attention ([B, H, S, Dh] Q / K / V / O, any Dh), the
// counterpart of the reference's launch_attention dispatch
// (src/kernels/attention.cu:602-700: flash kernels up to its shared-memory
// limit, a one-row-per-block kernel beyond).
//   Dh == 64: V is transposed per head (zero-padded to a multiple of 8 keys)
//   and the pipelined flash kernel runs;
//   any other Dh: per head, fp32 scores = scale Q K^T (MFMA GEMM), row
//   softmax to fp16 P, O = P V (MFMA GEMM over V^T), query rows in chunks so
//   the scores of one chunk stay within 256 MiB.  Q / K rows are copied to a
//   pitch padded to a multiple of 8 (zeros) when Dh is not one or the bases
//   are not 16-byte aligned.
// ---------------------------------------------------------------------------
// out[r * ld + c] = c < cols ? in[r * cols + c] : 0
__global__ void pad_rows_kernel(const f16* __restrict__ in, f16* __restrict__ out, long long rows,
                                int cols, int ld) {
  const long long total = rows * ld;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long r = i / ld;
    const int c = (int)(i - r * ld);
    out[i] = c < cols ? in[r * cols + c] : (f16)0.0f;
  }
}

// Per head z: out[z][d][key] = v[z][key][d] for key < Sk, 0 for key in [Sk, ld).
__global__ void vt_pad_kernel(const f16* __restrict__ v, f16* __restrict__ out, int Sk, int Dh,
                              int ld) {
  __shared__ f16 tile[32][33];
  const long long z = blockIdx.z;
  const int k0 = blockIdx.x * 32, d0 = blockIdx.y * 32;
  const int tx = threadIdx.x, ty = threadIdx.y;  // 32 x 8
  const f16* src = v + z * Sk * (long long)Dh;
  for (int r = ty; r < 32; r += 8) {
    const int key = k0 + r, d = d0 + tx;
    tile[r][tx] = (key < Sk && d < Dh) ? src[(long long)key * Dh + d] : (f16)0.0f;
  }
  __syncthreads();
  f16* dst = out + z * Dh * (long long)ld;
  for (int r = ty; r < 32; r += 8) {
    const int d = d0 + r, key = k0 + tx;
    if (d < Dh && key < ld) dst[(long long)d * ld + key] = tile[tx][r];
  }
}

static int vt_pad(const f16* v, f16* out, long long BH, int Sk, int Dh, int ld, hipStream_t s) {
  const dim3 grid((ld + 31) / 32, (Dh + 31) / 32, (unsigned)BH);
  DLM_LAUNCH("vt_pad_kernel", vt_pad_kernel, grid, dim3(32, 8), 0, s, v, out, Sk, Dh, ld);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

static int pad_rows(const f16* in, f16* out, long long rows, int cols, int ld, hipStream_t s) {
  const long long total = rows * ld;
  const int blocks = (int)std::min<long long>((total + 255) / 256, 65536);
  DLM_LAUNCH("pad_rows_kernel", pad_rows_kernel, dim3(blocks), dim3(256), 0, s, in, out, rows, cols, ld);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

static int attention_reference_layout(const f16* q, const f16* k, const f16* v, f16* o, int B,
                                      int H, int Sq, int Sk, int Dh, float scale, hipStream_t s) {
  const long long BH = (long long)B * H;
  const int K8 = (Sk + 7) & ~7;
  int st = DLM_OK;
  if (Dh == 64 && dlm_aligned16(q) && dlm_aligned16(k) && ((uintptr_t)o & 7) == 0) {
    f16* vt = (f16*)scratch_slot((size_t)BH * 64 * K8 * 2, 6, s, &st);
    if (!vt) return st;
    if ((st = vt_pad(v, vt, BH, Sk, 64, K8, s)) != DLM_OK) return st;
    dlm_attention_vt_args a{};
    a.q = q; a.k = k; a.vt = vt; a.o = o;
    a.q_sh = (long long)Sq * 64; a.q_sb = a.q_sh * H; a.q_ss = 64;
    a.k_sh = (long long)Sk * 64; a.k_sb = a.k_sh * H; a.k_ss = 64;
    a.vt_sh = 64LL * K8; a.vt_sb = a.vt_sh * H; a.vt_ld = K8;
    a.o_sh = (long long)Sq * 64; a.o_sb = a.o_sh * H; a.o_ss = 64;
    a.B = B; a.H = H; a.Sq = Sq; a.Sk = Sk; a.scale = scale;
    a.k_bytes = (unsigned long long)BH * Sk * 64 * 2;
    a.vt_bytes = (unsigned long long)BH * 64 * K8 * 2;
    if (a.k_bytes >= (1ull << 31) || a.vt_bytes >= (1ull << 31))
      return fail(DLM_ERR_UNSUPPORTED, "attention: K or V larger than 2 GiB");
    return attention_vt(&a, s);
  }
  const int D8 = (Dh + 7) & ~7;
  const int K4 = (Sk + 3) & ~3;
  const f16* qp = q;
  const f16* kp = k;
  int ld = Dh;
  if (Dh % 8 != 0 || !dlm_aligned16(q) || !dlm_aligned16(k)) {
    f16* qb = (f16*)scratch_slot((size_t)BH * Sq * D8 * 2, 7, s, &st);
    if (!qb) return st;
    f16* kb = (f16*)scratch_slot((size_t)BH * Sk * D8 * 2, 8, s, &st);
    if (!kb) return st;
    if ((st = pad_rows(q, qb, BH * Sq, Dh, D8, s)) != DLM_OK) return st;
    if ((st = pad_rows(k, kb, BH * Sk, Dh, D8, s)) != DLM_OK) return st;
    qp = qb;
    kp = kb;
    ld = D8;
  }
  f16* vt = (f16*)scratch_slot((size_t)BH * Dh * K8 * 2, 6, s, &st);
  if (!vt) return st;
  if ((st = vt_pad(v, vt, BH, Sk, Dh, K8, s)) != DLM_OK) return st;
  const long long rows_cap = std::max<long long>(1, (256LL << 20) / (4LL * K4));
  const int rows = (int)std::min<long long>(Sq, rows_cap);
  float* S = (float*)scratch_slot((size_t)rows * K4 * 4, 9, s, &st);
  if (!S) return st;
  f16* P = (f16*)scratch_slot((size_t)rows * K8 * 2, 10, s, &st);
  if (!P) return st;
  for (long long z = 0; z < BH; ++z) {
    for (int r0 = 0; r0 < Sq; r0 += rows) {
      const int n = std::min(rows, Sq - r0);
      st = dlm_linear_f32out_fp16(qp + (z * Sq + r0) * ld, ld, kp + z * Sk * ld, ld, nullptr,
                                  nullptr, 0, S, K4, n, Sk, ld, scale, 0.0f, DLM_ACT_NONE, s);
      if (st != DLM_OK) return st;
      if ((st = softmax_rows(S, K4, P, K8, n, Sk, K8, s)) != DLM_OK) return st;
      st = dlm_linear_fp16(P, K8, vt + z * Dh * (long long)K8, K8, nullptr, nullptr, 0,
                           o + (z * Sq + r0) * Dh, Dh, n, Dh, K8, 1.0f, 0.0f, DLM_ACT_NONE, s);
      if (st != DLM_OK) return st;
    }
  }
  return DLM_OK;
}

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

int dlm_attention_vt_fp16(const dlm_attention_vt_args* a, void* stream) {
  DLM_REQUIRE(a != nullptr, "args is NULL");
  if (a->B <= 0 || a->H <= 0 || a->Sq <= 0 || a->Sk <= 0) return DLM_OK;
  DLM_REQUIRE(a->q && a->k && a->vt && a->o, "NULL operand");
  DLM_REQUIRE(dlm_aligned16(a->q) && dlm_aligned16(a->k) && dlm_aligned16(a->vt) &&
                  ((uintptr_t)a->o & 7) == 0,
              "Q/K/V^T must be 16-byte aligned, O 8-byte aligned");
  DLM_REQUIRE(stride_ok(a->q_sb) && stride_ok(a->q_ss) && stride_ok(a->q_sh) &&
                  stride_ok(a->k_sb) && stride_ok(a->k_ss) && stride_ok(a->k_sh) &&
                  stride_ok(a->vt_sb) && stride_ok(a->vt_sh) && a->vt_ld % 8 == 0 &&
                  a->o_sb % 4 == 0 && a->o_ss % 4 == 0 && a->o_sh % 4 == 0,
              "strides must keep 16-byte (Q/K/V^T) and 8-byte (O) alignment");
  const int sk8 = (a->Sk + 7) & ~7;
  DLM_REQUIRE(a->vt_ld >= sk8, "vt_ld must cover Sk rounded up to a multiple of 8");
  DLM_REQUIRE(a->k_bytes > 0 && a->k_bytes < (1ull << 31) && a->vt_bytes > 0 &&
                  a->vt_bytes < (1ull << 31),
              "K and V^T buffers must be non-empty and smaller than 2 GiB");
  // every DMA offset must stay below 2^31: the last head's last key row
  const long long klast =
      ((a->B - 1) * a->k_sb + (a->H - 1) * a->k_sh + (long long)(a->Sk - 1) * a->k_ss + 64) * 2;
  const long long vlast = ((a->B - 1) * a->vt_sb + (a->H - 1) * a->vt_sh + 63LL * a->vt_ld + sk8) * 2;
  DLM_REQUIRE(klast <= (long long)a->k_bytes && vlast <= (long long)a->vt_bytes,
              "K or V^T extends past its buffer size");
  return attention_vt(a, (hipStream_t)stream);
}

int dlm_softmax_rows_f32_fp16(const float* S, long long lds, void* P, long long ldp, int rows,
                              int cols, void* stream) {
  if (rows <= 0 || cols <= 0) return DLM_OK;
  DLM_REQUIRE(S && P, "NULL pointer");
  DLM_REQUIRE(cols % 4 == 0 && lds % 4 == 0 && ldp % 4 == 0 && lds >= cols && ldp >= cols,
              "cols, lds and ldp must be multiples of 4 with lds, ldp >= cols");
  DLM_REQUIRE(dlm_aligned16(S) && ((uintptr_t)P & 7) == 0, "S must be 16-byte, P 8-byte aligned");
  return softmax_rows(S, lds, (f16*)P, ldp, rows, cols, cols, (hipStream_t)stream);
}

int dlm_attention_fp16(const void* q, const void* k, const void* v, void* out, int B, int H,
                       int Sq, int Sk, int Dh, float scale, void* stream) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || Dh <= 0) return DLM_OK;
  DLM_REQUIRE(q && k && v && out, "NULL operand");
  const long long BH = (long long)B * H;
  DLM_REQUIRE(BH * std::max(Sq, Sk) * (long long)((Dh + 7) & ~7) * 2 < (1LL << 31),
              "Q, K or V larger than 2 GiB");
  return attention_reference_layout((const f16*)q, (const f16*)k, (const f16*)v, (f16*)out, B, H,
                                    Sq, Sk, Dh, scale, (hipStream_t)stream);
}

}  // extern "C"
