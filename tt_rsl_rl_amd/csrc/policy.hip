// Rollout-side Gaussian head (rsl_rl/algorithms/ppo.py:124-135 act(); rsl_rl/modules/distribution.py:183-232):
// std = clamp/exp of the std parameter, actions = noise * std + mean (torch.normal(mean, std) draws a standard
// normal and scales it), log_prob of the actions summed over the action dimension, and the per-row std copy the
// rollout storage keeps as distribution_params[1].  The standard-normal noise is drawn by the caller (torch's
// device generator), so the rollout stays on torch's RNG stream.
#include "common.hpp"

#pragma clang fp contract(off)

namespace ppo {
namespace {

constexpr double kLogSqrt2Pi = 0.91893853320467274178;

struct SampleArgs {
  const float* mean; int64_t ld_mean;
  const float* std_param; int32_t std_type; float std_lo, std_hi;
  const float* noise; int64_t ld_noise;     // NULL: actions are given in `actions` (log-prob only)
  float* actions; int64_t ld_actions;
  float* logp;                              // [rows] or NULL
  float* std_out; int64_t ld_std;           // [rows, A] or NULL
  int64_t rows; int32_t A;
};

__global__ __launch_bounds__(256) void gauss_sample_kernel(const SampleArgs a) {
  __shared__ float s_std[PPO_MAX_ACTIONS], s_var[PPO_MAX_ACTIONS], s_log[PPO_MAX_ACTIONS];
  for (int j = threadIdx.x; j < a.A; j += blockDim.x) {
    float sd, lg;
    std_from_param(a.std_param[j], a.std_type, a.std_lo, a.std_hi, sd, lg);
    s_std[j] = sd;
    s_var[j] = sd * sd;
    s_log[j] = lg;
  }
  __syncthreads();
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= a.rows) return;
  const float* mu = a.mean + r * a.ld_mean;
  float* act = a.actions + r * a.ld_actions;
  const float c_lp = static_cast<float>(kLogSqrt2Pi);
  double lp = 0.0;
  for (int j = 0; j < a.A; ++j) {
    float x;
    if (a.noise != nullptr) {
      x = a.noise[r * a.ld_noise + j] * s_std[j] + mu[j];
      act[j] = x;
    } else {
      x = act[j];
    }
    const float d = x - mu[j];
    float t = -(d * d) / (2.0f * s_var[j]);
    t = t - s_log[j];
    t = t - c_lp;
    lp += static_cast<double>(t);
    if (a.std_out != nullptr) a.std_out[r * a.ld_std + j] = s_std[j];
  }
  if (a.logp != nullptr) a.logp[r] = static_cast<float>(lp);
}

}  // namespace
}  // namespace ppo

using namespace ppo;

extern "C" int ppo_gauss_sample(const float* mean, int64_t ld_mean, const float* std_param, int32_t std_type,
                                double std_lo, double std_hi, const float* noise, int64_t ld_noise, float* actions,
                                int64_t ld_actions, float* logp, float* std_out, int64_t ld_std, int64_t rows,
                                int32_t num_actions, ppo_stream_t stream) {
  PPO_REQUIRE(mean && std_param && actions, "ppo_gauss_sample: null pointer");
  PPO_REQUIRE(rows > 0 && num_actions > 0 && num_actions <= PPO_MAX_ACTIONS, "ppo_gauss_sample: rows=%lld A=%d",
              (long long)rows, num_actions);
  PPO_REQUIRE(std_type == PPO_STD_LOG || std_type == PPO_STD_SCALAR, "ppo_gauss_sample: std_type=%d", std_type);
  PPO_REQUIRE(ld_mean >= num_actions && ld_actions >= num_actions && (noise == nullptr || ld_noise >= num_actions) &&
                  (std_out == nullptr || ld_std >= num_actions),
              "ppo_gauss_sample: bad leading dimension");
  SampleArgs a{mean, ld_mean, std_param, std_type, static_cast<float>(std_lo), static_cast<float>(std_hi), noise,
               ld_noise, actions, ld_actions, logp, std_out, ld_std, rows, num_actions};
  const int64_t blocks = ceil_div(rows, 256);
  PPO_REQUIRE(blocks <= INT32_MAX, "ppo_gauss_sample: too many rows");
  hipLaunchKernelGGL(gauss_sample_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("gauss_sample_kernel");
}
