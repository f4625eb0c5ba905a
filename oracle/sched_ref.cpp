// Driver of the reference's header-only Euler scheduler
// (src/infer/scheduler.hpp), compiled by oracle/Makefile into
// oracle/_ref/sched_ref.  Test infrastructure only.
// Usage:
//   sched_ref STEPS        prints "sigma timestep" per line (STEPS lines),
//                          then the final sigma on its own line;
//   sched_ref STEPS apply  reads n, then n sample values and n model-output
//                          values from stdin, and for every step index i
//                          prints one line of scale_model_input(sample, i)
//                          and one line of step(model_output, i, sample)
//                          (scheduler.hpp:112-143), n values each.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "scheduler.hpp"

int main(int argc, char** argv) {
  const int steps = argc > 1 ? std::atoi(argv[1]) : 20;
  dollama::EulerDiscreteScheduler s;
  s.set_timesteps(steps);
  if (argc > 2 && std::strcmp(argv[2], "apply") == 0) {
    size_t n = 0;
    if (std::scanf("%zu", &n) != 1) return 2;
    std::vector<float> sample(n), model(n), out(n);
    for (auto& v : sample)
      if (std::scanf("%f", &v) != 1) return 2;
    for (auto& v : model)
      if (std::scanf("%f", &v) != 1) return 2;
    for (int i = 0; i < steps; ++i) {
      out = sample;
      s.scale_model_input(out.data(), n, i);
      for (size_t k = 0; k < n; ++k) std::printf("%.9g%c", out[k], k + 1 < n ? ' ' : '\n');
      s.step(model.data(), i, sample.data(), out.data(), n);
      for (size_t k = 0; k < n; ++k) std::printf("%.9g%c", out[k], k + 1 < n ? ' ' : '\n');
    }
    return 0;
  }
  for (int i = 0; i < steps; ++i) std::printf("%.9g %.9g\n", s.sigmas()[i], s.timesteps()[i]);
  std::printf("%.9g\n", s.sigmas()[steps]);
  return 0;
}
