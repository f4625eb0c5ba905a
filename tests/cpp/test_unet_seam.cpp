// The reference-signature UNet seam (dollama_amd/csrc/host/unet_api.hpp:
// unet_weights_create(const SafeTensors&), launch_unet, launch_unet_batched,
// unet_apply_loras / unet_clear_loras, unet_set_stage_hook; reference
// src/infer/unet.cuh:53-146) against the native C ABI (dlm_unet_forward) on
// the same safetensors file: bit-identical outputs, eager and under graphs.
// Usage: test_unet_seam <unet.safetensors> <latent size> <ctx_len>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "dollama.h"
#include "safetensors.hpp"
#include "unet_api.hpp"

using namespace dollama;

static int g_fail = 0;
#define CHECK(cond, what)                                                  \
  do {                                                                     \
    if (cond) {                                                            \
      std::printf("ok   %s\n", what);                                      \
    } else {                                                               \
      std::printf("FAIL %s (%s:%d)\n", what, __FILE__, __LINE__);          \
      ++g_fail;                                                            \
    }                                                                      \
    std::fflush(stdout);                                                   \
  } while (0)

#define OKC(expr)                                                                  \
  do {                                                                             \
    const int st_ = (expr);                                                        \
    if (st_ != DLM_OK) {                                                           \
      std::printf("FAIL %s -> %d: %s\n", #expr, st_, dlm_last_error());            \
      std::exit(2);                                                                \
    }                                                                              \
  } while (0)

// N(0, 1)-ish fp16 values (sum of 12 uniforms - 6) from a fixed LCG
static std::vector<uint16_t> randn_f16(size_t n, uint64_t seed, float scale = 1.0f) {
  std::vector<float> f(n);
  uint64_t s = seed * 6364136223846793005ULL + 1442695040888963407ULL;
  for (size_t i = 0; i < n; ++i) {
    float acc = -6.0f;
    for (int k = 0; k < 12; ++k) {
      s = s * 6364136223846793005ULL + 1442695040888963407ULL;
      acc += (float)((s >> 40) & 0xFFFFFF) / 16777216.0f;
    }
    f[i] = acc * scale;
  }
  std::vector<uint16_t> h(n);
  OKC(dlm_f32_to_f16(f.data(), h.data(), n));
  return h;
}

static void* to_dev(const void* host, size_t bytes) {
  void* d = nullptr;
  OKC(dlm_malloc(&d, bytes));
  OKC(dlm_memcpy(d, host, bytes, 0));
  return d;
}

static std::vector<uint16_t> from_dev(const void* d, size_t n) {
  std::vector<uint16_t> h(n);
  OKC(dlm_memcpy(h.data(), d, n * 2, 1));
  return h;
}

struct Half {  // a caller's own fp16 type, as the reference's __half
  uint16_t bits;
};
static std::vector<std::string> g_stages;
static std::vector<uint16_t> g_hook_noise;
static void ref_hook(const char* name, const Half* d_buf, size_t n) {
  g_stages.push_back(name);
  if (std::string(name) == "noise_pred") g_hook_noise = from_dev(d_buf, n);
}

int main(int argc, char** argv) {
  if (argc < 4) {
    std::printf("usage: %s unet.safetensors latent ctx_len\n", argv[0]);
    return 2;
  }
  const std::string path = argv[1];
  const int L = std::atoi(argv[2]), ctx = std::atoi(argv[3]);
  SafeTensors st(path);

  // configuration read from the shapes
  const UNetConfig c = unet_config_from_weights(st);
  std::printf("config C=%d/%d/%d depth=%d/%d cross=%d text=%d id=%d in=%d out=%d\n", c.C0, c.C1, c.C2,
              c.depth1, c.depth2, c.cross_dim, c.text_dim, c.id_dim, c.in_channels, c.out_channels);
  CHECK(st.contains("conv_in.weight") && !st.contains("no.such.tensor"), "SafeTensors::contains");
  CHECK(st.shape("conv_in.weight") == (std::vector<size_t>{(size_t)c.C0, 4, 3, 3}),
        "SafeTensors::shape as std::vector<size_t>");

  UnetWeightsHandle h = unet_weights_create(st);
  unet_set_geometry(h, L, L, ctx);

  // the native handle on the same file
  dlm_unet_config cc{c.C0, c.C1, c.C2, c.depth1, c.depth2, c.head_dim, c.cross_dim, c.text_dim,
                     c.id_dim, c.in_channels, c.out_channels, c.groups};
  void* nh = nullptr;
  OKC(dlm_unet_create(&cc, &nh));
  OKC(dlm_unet_load_safetensors(nh, path.c_str(), nullptr));
  void* ns = nullptr;
  OKC(dlm_stream_create(&ns));

  const int B = 2;
  const size_t n_lat = (size_t)4 * L * L, n_ehs = (size_t)ctx * c.cross_dim, n_txt = c.text_dim;
  const auto lat = randn_f16(B * n_lat, 1), ehs = randn_f16(B * n_ehs, 2), txt = randn_f16(B * n_txt, 3);
  std::vector<float> idsf = {1024, 1024, 0, 0, 1024, 1024};
  std::vector<uint16_t> ids(6);
  OKC(dlm_f32_to_f16(idsf.data(), ids.data(), 6));
  void* d_lat = to_dev(lat.data(), lat.size() * 2);
  void* d_ehs = to_dev(ehs.data(), ehs.size() * 2);
  void* d_txt = to_dev(txt.data(), txt.size() * 2);
  void* d_ids = to_dev(ids.data(), 12);
  void *d_out = nullptr, *d_ref = nullptr;
  OKC(dlm_malloc(&d_out, B * n_lat * 2));
  OKC(dlm_malloc(&d_ref, B * n_lat * 2));
  float* d_t = nullptr;
  OKC(dlm_malloc((void**)&d_t, 16 * sizeof(float)));

  auto native = [&](int b, float t) {
    std::vector<float> ts(b, t);
    OKC(dlm_memcpy(d_t, ts.data(), b * sizeof(float), 0));
    OKC(dlm_unet_forward(nh, b, L, L, d_lat, d_t, d_ehs, ctx, d_txt, d_ids, 0, d_ref, ns));
    OKC(dlm_stream_synchronize(ns));
    return from_dev(d_ref, b * n_lat);
  };

  // launch_unet_batched (B = 2) and launch_unet (B = 1), eager
  launch_unet_batched(h, B, d_lat, 999.0f, d_ehs, d_txt, d_ids, d_out);
  const auto ref2 = native(B, 999.0f);
  CHECK(from_dev(d_out, B * n_lat) == ref2, "launch_unet_batched(B=2) == dlm_unet_forward, bit for bit");
  launch_unet(h, d_lat, 999.0f, d_ehs, d_txt, d_ids, d_out);
  const auto ref1 = native(1, 999.0f);
  CHECK(from_dev(d_out, n_lat) == ref1, "launch_unet(B=1) == dlm_unet_forward, bit for bit");
  bool finite = true;
  for (uint16_t v : ref2) finite &= (v & 0x7C00) != 0x7C00;
  CHECK(finite, "noise_pred finite");

  // graphs: one captured graph, the host timestep refreshed before each replay
  unet_set_graphs(h, true);
  const float steps[] = {999.0f, 500.0f, 999.0f, 1.0f, 500.0f};
  bool same = true;
  for (float t : steps) {
    launch_unet_batched(h, B, d_lat, t, d_ehs, d_txt, d_ids, d_out);
    same &= from_dev(d_out, B * n_lat) == native(B, t);
  }
  size_t ng = 0;
  OKC(dlm_unet_graphs_captured(&unet_model(h), &ng));
  std::printf("graphs captured: %zu\n", ng);
  CHECK(same && ng >= 1, "graph replays with per-call timesteps == eager native forwards");
  CHECK(native(B, 500.0f) != native(B, 999.0f), "the timestep changes the output");
  unet_set_graphs(h, false);

  // LoRA: the same module through the seam and through the native C ABI
  LoraModule m;
  m.base_key = "down_blocks.1.attentions.0.transformer_blocks.0.attn1.to_q.weight";
  m.rank = 4;
  m.in_flat = c.C1;
  m.out_dim = c.C1;
  m.scale = 0.75f;
  m.a_fp16 = randn_f16((size_t)m.rank * m.in_flat, 7, 0.1f);
  m.b_fp16 = randn_f16((size_t)m.out_dim * m.rank, 8, 0.1f);
  const auto w0 = unet_read_weight(h, m.base_key);
  unet_apply_loras(h, &m, 1);
  void* dA = to_dev(m.a_fp16.data(), m.a_fp16.size() * 2);
  void* dB = to_dev(m.b_fp16.data(), m.b_fp16.size() * 2);
  OKC(dlm_unet_apply_lora(nh, m.base_key.c_str(), dA, dB, m.rank, m.in_flat, m.out_dim, m.scale, ns));
  CHECK(unet_read_weight(h, m.base_key) != w0, "unet_apply_loras patches the weight");
  launch_unet_batched(h, B, d_lat, 999.0f, d_ehs, d_txt, d_ids, d_out);
  const auto refl = native(B, 999.0f);
  CHECK(from_dev(d_out, B * n_lat) == refl && refl != ref2, "LoRA-patched forward == native LoRA forward");
  unet_clear_loras(h);
  OKC(dlm_unet_clear_loras(nh, ns));
  CHECK(unet_read_weight(h, m.base_key) == w0, "unet_clear_loras restores the weight bit for bit");
  launch_unet_batched(h, B, d_lat, 999.0f, d_ehs, d_txt, d_ids, d_out);
  CHECK(from_dev(d_out, B * n_lat) == ref2, "forward after clear == the unpatched forward");

  // stage hook with the reference's signature (global), NCHW stage copies
  unet_set_stage_hook(ref_hook);
  launch_unet_batched(h, B, d_lat, 999.0f, d_ehs, d_txt, d_ids, d_out);
  unet_set_stage_hook(static_cast<UnetStageHookFn>(nullptr));
  std::string names;
  for (const auto& s : g_stages) names += s + " ";
  std::printf("stages: %s\n", names.c_str());
  CHECK(g_stages.size() == 10 && g_stages.front() == "temb_final" && g_stages.back() == "noise_pred",
        "stage hook called at the block boundaries, temb_final first, noise_pred last");
  CHECK(g_hook_noise == ref2, "hooked noise_pred == the forward's output");
  g_stages.clear();
  launch_unet_batched(h, B, d_lat, 999.0f, d_ehs, d_txt, d_ids, d_out);
  CHECK(g_stages.empty(), "a removed hook is not called");

  // the per-call form (uploads the file for one B = 1 forward)
  {
    UnetWeightsHandle h2 = unet_weights_create(st);
    unet_set_geometry(h2, L, L, ctx);
    launch_unet(h2, d_lat, 999.0f, d_ehs, d_txt, d_ids, d_out);
    CHECK(from_dev(d_out, n_lat) == ref1, "a second handle from the same file gives the same bits");
    unet_weights_destroy(h2);
  }
  // errors throw, as the reference's CUDA_CHECK does
  bool threw = false;
  try {
    launch_unet_batched(h, 0, d_lat, 999.0f, d_ehs, d_txt, d_ids, d_out);
  } catch (const std::exception&) {
    threw = true;
  }
  CHECK(threw, "B = 0 throws");
  threw = false;
  try {
    launch_unet(nullptr, d_lat, 999.0f, d_ehs, d_txt, d_ids, d_out);
  } catch (const std::exception&) {
    threw = true;
  }
  CHECK(threw, "a null handle throws");
  unet_weights_destroy(nullptr);  // ignored

  unet_weights_destroy(h);
  OKC(dlm_unet_destroy(nh));
  OKC(dlm_stream_destroy(ns));
  for (void* p : {d_lat, d_ehs, d_txt, d_ids, d_out, d_ref, (void*)d_t, dA, dB}) OKC(dlm_free(p));
  std::printf("seam: %d failure(s)\n", g_fail);
  return g_fail ? 1 : 0;
}
