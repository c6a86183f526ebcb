// A1 GAE reverse-time scan and A2 advantage normalisation (rsl_rl/algorithms/ppo.py:166-191, :213-216).
//
// GAE: one lane per environment walks t = T-1..0; the [T, N] layout makes every time step one coalesced row
// read across the wavefront (64-lane blocks spread small env counts over many CUs).  HBM-bound: per element 4 B reward + 4 B value + 1 B done in, 4 B return + 4 B
// advantage out.  Contraction is disabled so the fp32 results are bit-identical to torch's op-by-op evaluation.
//
// Advantage normalisation: fp64 block partial sums, a fixed-order second stage (deterministic), then the
// normalising pass.  Three launches over n floats.
#include "common.hpp"

#pragma clang fp contract(off)

namespace ppo {
namespace {

// One lane per environment.  All loads of a chunk of CHUNK steps are issued before its scan (they do not depend on
// the recurrence) in straight-line code, so a lane waits for memory once per chunk instead of once per step: steps
// past the first `cnt` of a chunk re-read a step inside it (discarded), and the done flags stay bytes until the
// scan (a load whose result is converted at once, or a load under a branch, compiles to a wait of its own).
// The arithmetic is unchanged: the same fp32 operations in the same order as upstream's loop.
constexpr int kGaeThreads = 64;

template <int CHUNK>
__global__ __launch_bounds__(kGaeThreads) void gae_kernel(const float* __restrict__ rewards,
                                                          const float* __restrict__ values,
                                                          const uint8_t* __restrict__ dones,
                                                          const float* __restrict__ last_values,
                                                          float* __restrict__ returns,
                                                          float* __restrict__ advantages, int64_t T, int64_t N,
                                                          float gamma, float lam) {
  // 32-bit element indices (T * N < 2^31, checked on the host)
  const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= static_cast<uint32_t>(N)) return;
  const uint32_t NN = static_cast<uint32_t>(N);
  float next_value = last_values[n];
  float adv = 0.0f;
  for (int t0 = static_cast<int>(T) - 1; t0 >= 0; t0 -= CHUNK) {
    const int cnt = t0 + 1 < CHUNK ? t0 + 1 : CHUNK;
    float r[CHUNK], v[CHUNK];
    uint32_t d[CHUNK];
#pragma unroll
    for (int j = 0; j < CHUNK; ++j) {
      const uint32_t i = static_cast<uint32_t>(t0 - (j < cnt ? j : cnt - 1)) * NN + n;
      r[j] = rewards[i];
      v[j] = values[i];
      d[j] = dones[i];
    }
    auto step = [&](int j) {
      const uint32_t i = static_cast<uint32_t>(t0 - j) * NN + n;
      const float not_terminal = 1.0f - static_cast<float>(d[j]);
      const float ng = not_terminal * gamma;
      const float delta = (r[j] + ng * next_value) - v[j];
      adv = delta + (ng * lam) * adv;
      const float ret = adv + v[j];
      returns[i] = ret;
      advantages[i] = ret - v[j];
      next_value = v[j];
    };
    if (cnt == CHUNK) {  // a full chunk (every chunk of a rollout of CHUNK steps): no branch the loads could sink into
#pragma unroll
      for (int j = 0; j < CHUNK; ++j) step(j);
    } else {
#pragma unroll
      for (int j = 0; j < CHUNK; ++j)
        if (j < cnt) step(j);
    }
  }
}

constexpr int kNormThreads = 256;
constexpr int kNormMaxBlocks = 1024;

__device__ inline double block_sum(double x, double* red) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_down(x, off, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = x;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0) {
    for (int w = 0; w < kNormThreads / 64; ++w) s += red[w];
  }
  __syncthreads();
  return s;  // valid in thread 0
}

// Pass 1 (mode 0): partial sums of x.  Pass 2 (mode 1): partial sums of (x - mean)^2 with mean from stats[0].
__global__ __launch_bounds__(kNormThreads) void adv_partials_kernel(const float* __restrict__ x, int64_t stride,
                                                                    int64_t n, int mode,
                                                                    const double* __restrict__ stats,
                                                                    double* __restrict__ partials) {
  __shared__ double red[kNormThreads / 64];
  const double mean = mode ? stats[0] : 0.0;
  double acc = 0.0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kNormThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kNormThreads) {
    const double v = static_cast<double>(x[i * stride]);
    if (mode == 0) {
      acc += v;
    } else {
      const double d = v - mean;
      acc += d * d;
    }
  }
  const double s = block_sum(acc, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = s;
}

// Fixed-order reduction of the partials.  mode 0 -> stats[0] = mean (rounded through fp32 like torch's mean());
// mode 1 -> stats[1] = unbiased std rounded to fp32.
// One wavefront: lane l sums partials l, l + 64, ... in order (all of its loads issued before the first add), then
// a fixed butterfly combines the lanes.
__global__ __launch_bounds__(64) void adv_stats_kernel(const double* __restrict__ partials, int nparts, int64_t n,
                                                       int mode, double* __restrict__ stats) {
  constexpr int kPer = (kNormMaxBlocks + 63) / 64;
  double v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) v[j] = partials[min(static_cast<int>(threadIdx.x) + 64 * j, nparts - 1)];
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    if (static_cast<int>(threadIdx.x) + 64 * j < nparts) s += v[j];
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (threadIdx.x != 0) return;
  if (mode == 0) {
    stats[0] = static_cast<double>(static_cast<float>(s / static_cast<double>(n)));
  } else {
    const double var = s / static_cast<double>(n - 1);
    stats[1] = static_cast<double>(static_cast<float>(sqrt(var)));
  }
}

__global__ __launch_bounds__(kNormThreads) void adv_apply_kernel(const float* __restrict__ x, int64_t in_stride,
                                                                 float* __restrict__ out, int64_t out_stride,
                                                                 int64_t n, float eps,
                                                                 const double* __restrict__ stats) {
  const float mean = static_cast<float>(stats[0]);
  const float denom = static_cast<float>(stats[1]) + eps;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kNormThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kNormThreads) {
    out[i * out_stride] = (x[i * in_stride] - mean) / denom;
  }
}

__global__ void copy_strided_kernel(const float* __restrict__ x, int64_t in_stride, float* __restrict__ out,
                                    int64_t out_stride, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i * out_stride] = x[i * in_stride];
}

int norm_blocks(int64_t n) {
  return static_cast<int>(std::min<int64_t>(kNormMaxBlocks, std::max<int64_t>(1, ceil_div(n, kNormThreads * 4))));
}

}  // namespace
}  // namespace ppo

using namespace ppo;

extern "C" int ppo_gae(const float* rewards, const float* values, const uint8_t* dones, const float* last_values,
                       float* returns, float* advantages, int64_t num_steps, int64_t num_envs, float gamma,
                       float lam, ppo_stream_t stream) {
  PPO_REQUIRE(rewards && values && dones && last_values && returns && advantages, "ppo_gae: null pointer");
  PPO_REQUIRE(num_steps > 0 && num_envs > 0, "ppo_gae: num_steps=%lld num_envs=%lld must be positive",
              (long long)num_steps, (long long)num_envs);
  PPO_REQUIRE(num_steps * num_envs < (int64_t(1) << 31), "ppo_gae: %lld x %lld elements (at most 2^31 - 1)",
              (long long)num_steps, (long long)num_envs);
  const int64_t blocks = ceil_div(num_envs, kGaeThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 block(kGaeThreads);
  // the chunk: all of a rollout of up to 32 steps at once (the smallest of 8, 16, 24, 32 that holds it)
  const dim3 grid(static_cast<unsigned>(blocks));
  if (num_steps <= 8) {
    hipLaunchKernelGGL(gae_kernel<8>, grid, block, 0, s, rewards, values, dones, last_values, returns, advantages,
                       num_steps, num_envs, gamma, lam);
  } else if (num_steps <= 16) {
    hipLaunchKernelGGL(gae_kernel<16>, grid, block, 0, s, rewards, values, dones, last_values, returns, advantages,
                       num_steps, num_envs, gamma, lam);
  } else if (num_steps <= 24) {
    hipLaunchKernelGGL(gae_kernel<24>, grid, block, 0, s, rewards, values, dones, last_values, returns, advantages,
                       num_steps, num_envs, gamma, lam);
  } else {
    hipLaunchKernelGGL(gae_kernel<32>, grid, block, 0, s, rewards, values, dones, last_values, returns, advantages,
                       num_steps, num_envs, gamma, lam);
  }
  return check_launch("gae_kernel");
}

extern "C" size_t ppo_adv_normalize_workspace_bytes(int64_t n) {
  return sizeof(double) * (2 + static_cast<size_t>(n > 0 ? norm_blocks(n) : 1));
}

extern "C" int ppo_adv_normalize(const float* x, int64_t in_stride, float* out, int64_t out_stride, int64_t n,
                                 float eps, void* workspace, size_t workspace_bytes, ppo_stream_t stream) {
  PPO_REQUIRE(x && out, "ppo_adv_normalize: null pointer");
  PPO_REQUIRE(n > 0 && in_stride > 0 && out_stride > 0, "ppo_adv_normalize: bad size/stride");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n == 1) {
    if (x != out) {
      hipLaunchKernelGGL(copy_strided_kernel, dim3(1), dim3(64), 0, s, x, in_stride, out, out_stride, n);
      return check_launch("copy_strided_kernel");
    }
    return PPO_OK;
  }
  PPO_REQUIRE(workspace && workspace_bytes >= ppo_adv_normalize_workspace_bytes(n),
              "ppo_adv_normalize: workspace too small (%zu < %zu)", workspace_bytes,
              ppo_adv_normalize_workspace_bytes(n));
  double* stats = static_cast<double*>(workspace);
  double* partials = stats + 2;
  const int blocks = norm_blocks(n);
  hipLaunchKernelGGL(adv_partials_kernel, dim3(blocks), dim3(kNormThreads), 0, s, x, in_stride, n, 0, stats,
                     partials);
  hipLaunchKernelGGL(adv_stats_kernel, dim3(1), dim3(64), 0, s, partials, blocks, n, 0, stats);
  hipLaunchKernelGGL(adv_partials_kernel, dim3(blocks), dim3(kNormThreads), 0, s, x, in_stride, n, 1, stats,
                     partials);
  hipLaunchKernelGGL(adv_stats_kernel, dim3(1), dim3(64), 0, s, partials, blocks, n, 1, stats);
  hipLaunchKernelGGL(adv_apply_kernel, dim3(blocks), dim3(kNormThreads), 0, s, x, in_stride, out, out_stride, n,
                     eps, stats);
  return check_launch("adv_normalize");
}
