// Device-resident CFG denoise loop (see pipeline.hpp).
#include "pipeline.hpp"

#include <stdexcept>
#include <vector>

#include "check.hpp"
#include "device_arena.hpp"
#include "scheduler.hpp"

namespace dollama {

void denoise(UNet& unet, const DenoiseArgs& a, void* stream) {
  if (a.steps <= 0) throw std::invalid_argument("denoise: steps must be positive");
  if (!a.latent || !a.ehs || !a.text || !a.time_ids) throw std::invalid_argument("denoise: NULL input");
  const UNetConfig& c = unet.config();
  const int n = c.in_channels * a.H * a.W;
  if (c.in_channels != c.out_channels) throw std::invalid_argument("denoise: in/out channels differ");

  EulerDiscreteScheduler sched;
  sched.set_timesteps(a.steps);
  const auto& ts = sched.timesteps();
  const auto& sg = sched.sigmas();

  DeviceArenaScope scope(DeviceArenaId::UNetPersist);
  // per-step timestep pairs [steps][2] (cond and uncond share t)
  std::vector<float> host_t(2 * (size_t)a.steps);
  for (int i = 0; i < a.steps; ++i) host_t[2 * i] = host_t[2 * i + 1] = ts[i];
  float* d_t = scope.alloc<float>(host_t.size());
  DLM_CALL(dlm_memcpy(d_t, host_t.data(), host_t.size() * sizeof(float), 0));
  void* model_in = scope.alloc<uint16_t>(2 * (size_t)n);
  void* noise = scope.alloc<uint16_t>(2 * (size_t)n);

  DLM_CALL(dlm_scale_latent_fp16(a.latent, model_in, n, (float)sched.input_scale(0), 2, stream));
  for (int i = 0; i < a.steps; ++i) {
    unet.forward(2, a.H, a.W, model_in, d_t + 2 * i, a.ehs, a.ctx_len, a.text, a.time_ids, 0, noise,
                 stream);
    const float next_scale = i + 1 < a.steps ? (float)sched.input_scale(i + 1) : 1.0f;
    DLM_CALL(dlm_euler_cfg_step(a.latent, noise, model_in, n, a.guidance, sg[i], sg[i + 1], next_scale,
                                stream));
  }
}

}  // namespace dollama
