// Euler discrete scheduler for SDXL (host, double precision).
//
// Same configuration and arithmetic as the reference's scheduler
// (src/infer/scheduler.hpp:31-197): num_train_timesteps 1000, betas
// scaled_linear from 0.00085 to 0.012, "leading" timestep spacing with
// steps_offset 1, sigmas interpolated linearly on the training sigma table,
// a trailing 0 appended; epsilon prediction.
//   scale_model_input: x / sqrt(sigma_i^2 + 1)
//   step:              x + eps * (sigma_{i+1} - sigma_i)
//   initial latent:    randn * sigma_0
#pragma once

#include <cmath>
#include <stdexcept>
#include <vector>

namespace dollama {

class EulerDiscreteScheduler {
 public:
  explicit EulerDiscreteScheduler(int num_train_timesteps = 1000, double beta_start = 0.00085,
                                  double beta_end = 0.012)
      : n_train_(num_train_timesteps) {
    if (n_train_ <= 1) throw std::invalid_argument("EulerDiscreteScheduler: need >= 2 train timesteps");
    train_sigmas_.resize(n_train_);
    const double a = std::sqrt(beta_start), b = std::sqrt(beta_end);
    double alpha_bar = 1.0;
    for (int i = 0; i < n_train_; ++i) {
      const double s = a + (b - a) * (double)i / (double)(n_train_ - 1);
      alpha_bar *= 1.0 - s * s;
      train_sigmas_[i] = std::sqrt((1.0 - alpha_bar) / alpha_bar);
    }
  }

  void set_timesteps(int steps) {
    if (steps <= 0 || steps > n_train_) throw std::invalid_argument("EulerDiscreteScheduler: bad step count");
    steps_ = steps;
    const int ratio = n_train_ / steps;
    timesteps_.assign(steps, 0.0f);
    sigmas_.assign(steps + 1, 0.0f);
    for (int i = 0; i < steps; ++i) {
      // descending: the i-th step uses the (steps-1-i)-th leading timestep
      const double t = std::round((double)(steps - 1 - i) * ratio) + 1.0;
      timesteps_[i] = (float)t;
      sigmas_[i] = (float)sigma_at(t);
    }
    sigmas_[steps] = 0.0f;
  }

  int steps() const { return steps_; }
  const std::vector<float>& timesteps() const { return timesteps_; }
  const std::vector<float>& sigmas() const { return sigmas_; }
  float init_noise_sigma() const { return sigmas_.empty() ? 1.0f : sigmas_[0]; }
  double input_scale(int i) const {
    const double s = sigmas_.at(i);
    return 1.0 / std::sqrt(s * s + 1.0);
  }

 private:
  double sigma_at(double t) const {
    if (t <= 0.0) return train_sigmas_.front();
    if (t >= n_train_ - 1) return train_sigmas_.back();
    const int lo = (int)std::floor(t);
    const double f = t - lo;
    return train_sigmas_[lo] + (train_sigmas_[lo + 1] - train_sigmas_[lo]) * f;
  }

  int n_train_;
  int steps_ = 0;
  std::vector<double> train_sigmas_;
  std::vector<float> timesteps_, sigmas_;
};

}  // namespace dollama
