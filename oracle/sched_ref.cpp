// Driver of the reference's header-only Euler scheduler
// (src/infer/scheduler.hpp), compiled by oracle/Makefile into
// oracle/_ref/sched_ref.  Test infrastructure only.
// Usage: sched_ref STEPS  ->  prints "sigma timestep" per line (STEPS lines),
// then the final sigma on its own line.
#include <cstdio>
#include <cstdlib>

#include "scheduler.hpp"

int main(int argc, char** argv) {
  const int steps = argc > 1 ? std::atoi(argv[1]) : 20;
  dollama::EulerDiscreteScheduler s;
  s.set_timesteps(steps);
  for (int i = 0; i < steps; ++i) std::printf("%.9g %.9g\n", s.sigmas()[i], s.timesteps()[i]);
  std::printf("%.9g\n", s.sigmas()[steps]);
  return 0;
}
