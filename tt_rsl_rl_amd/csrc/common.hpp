// Shared plumbing for the PPO HIP library: status codes, the thread-local error message, argument checks.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/ppo_hip.h"

namespace ppo {

void set_error(const char* fmt, ...);
void clear_error();

// Records the message and returns the status code, so call sites can `return fail(PPO_EINVAL, "...")`.
int fail(int code, const char* fmt, ...);

// Checks the launch that was just enqueued (does not synchronise).
int check_launch(const char* what);

// Compute units and XCDs (accelerator complex dies, each with its own L2) of the current device, queried once per
// device; {0, 0} when no device is current.  A partitioned MI355X shows fewer of both than the whole chip's 256 / 8.
struct DeviceInfo {
  int cus;
  int xcds;
};
DeviceInfo device_info();
constexpr int kMaxDevices = 64;

constexpr int kWave = 64;

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The distribution's std from its parameter (rsl_rl/modules/distribution.py:186-190): clamp in the parameter's
// space, exp for the log parameterisation; log_sd = log(std) as Normal.log_prob / entropy take it.  exp and log
// are evaluated in fp64 and rounded once, i.e. correctly rounded fp32 results, so a std computed here equals the
// std of any implementation that rounds correctly (a 1-ulp difference would leave KL(p||p) a few 1e-15 above 0).
__device__ inline void std_from_param(float q, int std_type, float lo, float hi, float& sd, float& log_sd) {
  const float c = fminf(fmaxf(q, lo), hi);
  sd = (std_type == PPO_STD_LOG) ? static_cast<float>(exp(static_cast<double>(c))) : c;
  log_sd = static_cast<float>(log(static_cast<double>(sd)));
}

}  // namespace ppo

#define PPO_REQUIRE(cond, ...)                          \
  do {                                                  \
    if (!(cond)) return ::ppo::fail(PPO_EINVAL, __VA_ARGS__); \
  } while (0)

#define PPO_HIP_CHECK(expr)                                                                      \
  do {                                                                                           \
    hipError_t _e = (expr);                                                                      \
    if (_e != hipSuccess) return ::ppo::fail(PPO_EHIP, "%s: %s", #expr, hipGetErrorString(_e)); \
  } while (0)
