// SDXL UNet2DConditionModel forward on channels-last activations.
//
// Graph and weight names follow the reference's UNet driver
// (src/infer/unet.cu:537-1309, diffusers key names) and its public API
// (src/infer/unet.cuh:53-146): resident weight handle, B-major batched
// forward with time_ids shared across the batch, stage hook for tests.
//
// What differs by design (MI355X-first, same arithmetic up to rounding):
//   - activations are [B, H, W, C] (== [tokens, C]), so the Transformer2D
//     chw<->sc transposes and the head split/merge kernels disappear;
//   - every conv is one implicit-GEMM launch with its epilogue fused (bias,
//     time-embedding bias, residual, or the 1x1 conv_shortcut accumulated as
//     a second K segment); channel concatenation and nearest-2x upsampling
//     happen in the conv operand loader, never in memory;
//   - q/k/v are one GEMM, the GEGLU gate runs in the FF1 GEMM epilogue, and
//     residual adds run in the out-projection epilogues;
//   - all resnets' time_emb_proj are one skinny GEMM, and the cross-attention
//     K/V projections of every transformer block are one GEMM over the
//     encoder hidden states (they depend only on the context);
//   - nothing crosses to the host during a forward (time_ids stay on device).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <set>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "dlm.h"

namespace dollama {

struct UNetConfig {
  int C0 = 320, C1 = 640, C2 = 1280;  // block_out_channels
  int depth1 = 2, depth2 = 10;        // transformer depth at levels 1 and 2 (and mid)
  int head_dim = 64;
  int cross_dim = 2048;
  int text_dim = 1280;  // pooled text embedding width
  int id_dim = 256;     // sinusoid width per time id (6 ids)
  int in_channels = 4, out_channels = 4;
  int groups = 32;
  int time_dim() const { return 4 * C0; }
  int add_dim() const { return text_dim + 6 * id_dim; }
};

struct WeightSpec {
  std::string name;
  std::vector<int64_t> shape;
};

// All parameters the forward reads, with diffusers names and shapes.
std::vector<WeightSpec> unet_weight_specs(const UNetConfig& cfg);

using UnetStageHook = void (*)(const char* name, const void* dptr, size_t n, int C, void* user);

class UNet {
 public:
  explicit UNet(const UNetConfig& cfg);
  ~UNet();
  UNet(const UNet&) = delete;
  UNet& operator=(const UNet&) = delete;

  const UNetConfig& config() const { return cfg_; }

  // Register a device fp16 weight (borrowed until prepare()).
  void set_weight(const std::string& name, const void* dptr, const std::vector<int64_t>& shape);
  // Pack every registered weight into the handle's own device memory; the
  // registered buffers may be freed afterwards.  Throws if a weight is
  // missing or mis-shaped.
  void prepare(void* stream);
  bool prepared() const { return packed_ != nullptr; }
  size_t packed_bytes() const { return packed_bytes_; }

  // noise_pred[B, out, H, W] (NCHW) for latent[B, in, H, W] (NCHW), per-batch
  // timesteps (device fp32 [B]), ehs [B, ctx_len, cross_dim], text [B, text_dim],
  // time_ids [6] shared (ids_bstride 0) or [B, 6] (ids_bstride 6).
  void forward(int B, int H, int W, const void* latent, const float* d_timesteps, const void* ehs,
               int ctx_len, const void* text, const void* time_ids, int ids_bstride, void* out,
               void* stream);

  // Runtime LoRA merge on the resident weights: W += scale * (B @ A) with
  // device fp16 A [rank, in_flat] and B [out_dim, rank]; clear_loras() restores
  // every patched weight bit-exactly.  Synchronises the stream.
  void apply_lora(const std::string& key, const void* dA, const void* dB, int rank, int in_flat,
                  int out_dim, float scale, void* stream);
  void clear_loras(void* stream);
  size_t lora_patched() const { return patched_.size(); }
  // Copy the resident fp16 weight `key` back to host memory in its diffusers
  // layout (undoing the GEGLU interleave and the per-tap conv packing);
  // bytes must equal 2 * its element count.  Synchronises the stream.
  void read_weight(const std::string& key, void* host, size_t bytes, void* stream) const;

  // One block of the prepared model on its own (block-level tests and
  // timing; the forward does not use these):
  //   run_resnet: prefix "down_blocks.1.resnets.0" style; x = concat(xa[:, :Ca],
  //   xb[:, :Cb]) channels-last [B, H, W, Ca + Cb]; temb [B, time_dim] fp16 as
  //   the time MLP outputs it (SiLU and this block's time_emb_proj applied
  //   here); out [B, H, W, Co].
  //   run_transformer_block: prefix "...attentions.a.transformer_blocks.l";
  //   x [B * HW, C] updated in place; ehs [B, ctx_len, cross_dim] (the block's
  //   cross-attention K / V projections are computed here).
  void run_resnet(const std::string& prefix, const void* xa, int Ca, const void* xb, int Cb,
                  void* out, int B, int H, int W, const void* temb, void* stream);
  void run_transformer_block(const std::string& prefix, void* x, int B, int HW, const void* ehs,
                             int ctx_len, void* stream);

  void set_stage_hook(UnetStageHook hook, void* user) {
    hook_ = hook;
    hook_user_ = user;
  }

  // HIP-graph replay of forward().  With graphs on, a forward whose
  // arguments, stream and arena state (mark and chunk epoch of the UNet and
  // UNetPersist arenas) equal those of an earlier forward replays that
  // forward's captured graph.  The first such forward runs eagerly (it
  // allocates every arena chunk and split-K workspace), the second is
  // captured and launched, later ones launch the graph.  Needs a created
  // stream (not the null stream); inactive while a stage hook or profiling
  // is on.  Replays are stream-ordered like the eager forward they replace.
  void set_graphs(bool on);
  // LayerNorm of the transformer blocks folded into the QKV, cross-attention
  // Q and GEGLU linears (on by default) or run as separate launches
  void set_ln_fold(int mask);
  int ln_fold() const { return ln_fold_; }
  // GroupNorm statistics written by the producing conv's epilogue (on by
  // default); off, every GroupNorm runs its own statistics pass.  Same bits
  // either way.
  void set_gn_fold(bool on);
  bool gn_fold() const { return gn_fold_; }
  size_t graphs_captured() const { return graphs_.size(); }

  // Per-launch timing with device events, grouped by kernel class.  While
  // enabled, every launch of a forward is bracketed by two events; the
  // report (after the stream is synchronised) gives per class the launch
  // count, summed kernel milliseconds, algorithmic FLOPs and algorithmic
  // bytes of the last profiled forward.
  enum KernelClass { kConv = 0, kLinear, kAttention, kGroupNorm, kLayerNorm, kOther, kClassCount };
  void set_profiling(bool on);
  struct ClassStats {
    int count = 0;
    double ms = 0.0, flops = 0.0, bytes = 0.0;
  };
  std::vector<ClassStats> profile_report(void* stream);
  // Same launches grouped by the kernel each one ran last (dlm_last_kernel):
  // name -> class, launch count, kernel ms, algorithmic FLOPs and bytes.
  struct KernelStats {
    std::string name;
    int cls = 0;
    int count = 0;
    double ms = 0.0, flops = 0.0, bytes = 0.0;
    std::map<std::vector<int>, int> dims;  // GEMM problems (M, N, K, flags) -> launches
  };
  std::vector<KernelStats> profile_kernels(void* stream);

 private:
  struct Resnet {
    int Ci = 0, Co = 0;
    bool shortcut = false;
    const void *n1g, *n1b, *c1w, *c1b, *n2g, *n2b, *c2w, *c2b;
    int c2_ldw = 0;
    int tproj_off = 0;
  };
  // A linear that consumes a LayerNorm, with the LayerNorm folded in:
  // w_f = w * gamma (per K column), c1 = row sums of w_f, c2 = w beta + b
  // (dlm_ln_fold_fp16).  w stays the master copy (LoRA patches, weight
  // reads); the fold is redone from it after every change.
  struct LnFold {
    const void *w = nullptr, *g = nullptr, *b = nullptr, *bias = nullptr;
    void* wf = nullptr;
    float *c1 = nullptr, *c2 = nullptr;
    int N = 0, K = 0;
  };
  struct Block {
    const void *ln1g, *ln1b, *wqkv, *wo1, *bo1, *ln2g, *ln2b, *wq2, *wo2, *bo2, *ln3g, *ln3b;
    const void *wff1, *bff1, *wff2, *bff2;
    int kv_off = 0;
    LnFold fqkv, fq2;  // norm1 -> to_q/k/v, norm2 -> attn2.to_q
  };
  struct T2D {
    int C = 0;
    const void *ng, *nb, *pin_w, *pin_b, *pout_w, *pout_b;
    std::vector<Block> blocks;
  };
  struct Conv {
    const void *w = nullptr, *b = nullptr;
    int ldw = 0;
  };

  struct Src {
    const void* ptr;
    std::vector<int64_t> shape;
  };

  // where each named weight lives in the packed storage (for LoRA)
  struct Placement {
    enum Kind { kCopy, kConv, kGeglu } kind = kCopy;
    char* dst = nullptr;
    size_t elems = 0;
    int Co = 0, Ci = 0, k = 0, cin_pad = 0, ld = 0, col0 = 0;
  };
  struct Backup {
    char* dst;
    void* copy;
    size_t bytes;
  };
  std::unordered_map<std::string, Placement> placed_;
  std::vector<Backup> backups_;
  std::unordered_set<std::string> patched_;
  void place_copy(const std::string& name, void* dst, size_t n);
  void place_conv(const std::string& name, void* dst, int Co, int Ci, int k, int cin_pad, int ld,
                  int col0);

  // packing helpers (two passes: sizing, then filling)
  const Src& src(const std::string& name, const std::vector<int64_t>& shape) const;
  void* take(size_t elems);
  const void* copy_of(const std::string& name, const std::vector<int64_t>& shape, void* stream);
  Resnet pack_resnet(const std::string& p, int Ci, int Co, void* stream);
  T2D pack_t2d(const std::string& p, int C, int depth, void* stream);
  Conv pack_conv(const std::string& p, int Co, int Ci, int k, int cin_pad, void* stream);
  void pack_all(void* stream);

  void forward_impl(int B, int H, int W, const void* latent, const float* d_timesteps,
                    const void* ehs, int ctx_len, const void* text, const void* time_ids,
                    int ids_bstride, void* out, void* stream);
  void clear_graphs();
  bool graphs_on_ = false;
  // LayerNorms folded into their consuming linears: bit 0 norm1 -> QKV,
  // bit 1 norm2 -> cross-attention Q (both by default: step 23.07 -> 22.76 ms)
  int ln_fold_ = 3;
  bool gn_fold_ = true;
  LnFold make_fold(const void* w, const void* g, const void* b, const void* bias, int N, int K,
                   const std::vector<std::string>& deps, void* stream);
  void refold(const LnFold& f, void* stream);
  // folds that depend on each named weight (LoRA refolds them)
  std::unordered_map<std::string, std::vector<LnFold>> fold_deps_;
  std::map<std::vector<uint64_t>, void*> graphs_;
  std::set<std::vector<uint64_t>> seen_;

  // forward pieces
  // in_stats: GroupNorm chunk statistics of xa (no xb) already written by
  // its producer, or null; out_stats: where conv2 writes those of out, or null
  void resnet(const Resnet& r, const void* xa, int Ca, const void* xb, int Cb, void* out, int B,
              int H, int W, const void* tproj, void* stream, const void* in_stats = nullptr,
              void* out_stats = nullptr, const void* in_stats_b = nullptr);
  // every block's cross-attention K ([B*ctx, sumC]) and V^T ([B, sumC, ld])
  struct CrossKV {
    void* k;
    void* vt;
    int ld;
  };
  void t2d(const T2D& t, void* x, int B, int HW, const CrossKV& kv, int ctx_len, void* stream,
           const void* in_stats = nullptr, void* out_stats = nullptr);
  // one BasicTransformerBlock over the residual stream h [B*HW, C]; this
  // block's context K rows start at row kv_off of kv.k (row stride kv_stride)
  // and its V^T rows at row kv_off of kv.vt (kv_stride rows per sample)
  struct TScratch {
    void *n, *qkv, *vt;
    int vt_ld;
    void *o, *f;
  };
  void tblock(const Block& k, int C, void* h, const TScratch& ts, int B, int HW, const CrossKV& kv,
              int kv_off, int kv_stride, int ctx_len, void* stream);
  // prestats: a GroupNorm workspace whose chunk statistics of xa (no xb)
  // its producer wrote (dlm_conv_nhwc_args::gn_stats), or null
  void gn(const void* xa, int Ca, const void* xb, int Cb, const void* g, const void* b, void* out,
          int B, int HW, float eps, bool silu, void* stream, const void* prestats = nullptr,
          const void* prestats_b = nullptr);
  void conv3(const Conv& c, const void* x, int C, const void* xb, int Cb, void* out, int Co, int B,
             int H, int W, int stride, bool up, void* stream, int flop_cin = -1,
             void* gn_stats = nullptr);
  void stage(const char* name, const void* p, size_t n, int C, void* stream);

  UNetConfig cfg_;
  std::unordered_map<std::string, Src> srcs_;
  // packed weights
  bool sizing_ = false;
  char* packed_ = nullptr;
  size_t packed_bytes_ = 0;
  size_t cursor_ = 0;
  Conv conv_in_, conv_out_, down0_, down1_, up0_, up1_;
  const void *te1w_, *te1b_, *te2w_, *te2b_, *ae1w_, *ae1b_, *ae2w_, *ae2b_;
  const void *tproj_w_, *tproj_b_, *kv_w_;
  const void *norm_out_g_, *norm_out_b_;
  int tproj_total_ = 0, kv_total_ = 0;
  std::vector<Resnet> res_;  // in forward order
  std::vector<T2D> t2d_;     // in forward order
  std::vector<std::string> res_names_, t2d_names_;  // their weight-name prefixes
  UnetStageHook hook_ = nullptr;
  void* hook_user_ = nullptr;

  // profiling state
  struct ProfRec {
    int cls;
    double flops, bytes;
    std::string kernel;
    int dims[4];
  };
  bool prof_on_ = false;
  std::vector<void*> prof_events_;
  std::vector<ProfRec> prof_recs_;
  size_t prof_next_ = 0;
  void prof_begin(int cls, double flops, double bytes, void* stream);
  void prof_end(void* stream);
};

}  // namespace dollama
