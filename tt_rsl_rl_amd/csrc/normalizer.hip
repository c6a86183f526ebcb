// A7: EmpiricalNormalization.update (rsl_rl/modules/normalization.py:51-78, single process) over the rollout's
// stored observations, once per update after the epochs (rsl_rl/algorithms/ppo.py:327-330).
//
// Batch moments are reduced in fp64 and two passes (mean, then the biased variance around it), column-parallel:
// each block owns a slab of rows, each thread a column, so every row is one coalesced read.  Partials are summed
// in a fixed order.  The running-statistics update then replays torch's fp32 operation order on [dim] vectors.
#include "common.hpp"

#pragma clang fp contract(off)

namespace ppo {
namespace {

constexpr int kNormThreads = 256;
constexpr int kRowsPerSlab = 128;
constexpr int kMaxBlocks = PPO_MAX_GATHER_SEGMENTS;

struct Blocks {
  ppo_column_block b[kMaxBlocks];
  int32_t col_begin[kMaxBlocks + 1];
  int32_t count;
  int32_t dim;
};

__device__ inline float load_col(const Blocks& bl, int64_t r, int c) {
  int i = 0;
  for (int k = 1; k < kMaxBlocks; ++k)
    if (k < bl.count && c >= bl.col_begin[k]) i = k;
  return bl.b[i].src[r * bl.b[i].stride + (c - bl.col_begin[i])];
}

// pass 0: partial column sums; pass 1: partial sums of (x - mean)^2 (mean from stats[0..dim)).
__global__ __launch_bounds__(kNormThreads) void moments_kernel(const Blocks bl, int64_t rows, int pass,
                                                               const double* __restrict__ stats,
                                                               double* __restrict__ partials) {
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRowsPerSlab;
  const int64_t r1 = min(rows, r0 + kRowsPerSlab);
  for (int c = threadIdx.x; c < bl.dim; c += kNormThreads) {
    const double mu = pass ? stats[c] : 0.0;
    double acc = 0.0;
    for (int64_t r = r0; r < r1; ++r) {
      const double v = load_col(bl, r, c);
      if (pass == 0) {
        acc += v;
      } else {
        const double d = v - mu;
        acc += d * d;
      }
    }
    partials[static_cast<int64_t>(blockIdx.x) * bl.dim + c] = acc;
  }
}

// Fixed-order column reduction of the slab partials: stats[c] = sum / rows (pass 0 -> mean, pass 1 -> var).
__global__ __launch_bounds__(kNormThreads) void moments_reduce_kernel(const double* __restrict__ partials, int slabs,
                                                                      int dim, int64_t rows, double* __restrict__ out) {
  for (int c = blockIdx.x * kNormThreads + threadIdx.x; c < dim; c += gridDim.x * kNormThreads) {
    double s = 0.0;
    for (int k = 0; k < slabs; ++k) s += partials[static_cast<int64_t>(k) * dim + c];
    out[c] = s / static_cast<double>(rows);
  }
}

// normalization.py:73-78 in fp32: count += n; rate = n / count; delta = mean_x - mean; mean += rate * delta;
// var += rate * (var_x - var + delta * (mean_x - mean)); std = sqrt(var).
__global__ __launch_bounds__(kNormThreads) void running_update_kernel(const double* __restrict__ batch_mean,
                                                                      const double* __restrict__ batch_var, int dim,
                                                                      int64_t n, float* __restrict__ mean,
                                                                      float* __restrict__ var,
                                                                      float* __restrict__ std,
                                                                      int64_t* __restrict__ count) {
  const int64_t total = *count + n;
  const float rate = static_cast<float>(n) / static_cast<float>(total);
  for (int c = threadIdx.x; c < dim; c += kNormThreads) {
    const float mx = static_cast<float>(batch_mean[c]);
    const float vx = static_cast<float>(batch_var[c]);
    const float m0 = mean[c];
    const float delta = mx - m0;
    const float m1 = m0 + rate * delta;
    const float v0 = var[c];
    const float v1 = v0 + rate * ((vx - v0) + delta * (mx - m1));
    mean[c] = m1;
    var[c] = v1;
    std[c] = sqrtf(v1);
  }
  __syncthreads();
  if (threadIdx.x == 0) *count = total;
}

struct NormPlan {
  int64_t slabs;
  size_t partial_off, mean_off, var_off, total;  // doubles
};

NormPlan plan_norm(int64_t rows, int dim) {
  NormPlan p;
  p.slabs = ceil_div(rows, kRowsPerSlab);
  p.partial_off = 0;
  p.mean_off = static_cast<size_t>(p.slabs) * dim;
  p.var_off = p.mean_off + dim;
  p.total = p.var_off + dim;
  return p;
}

}  // namespace
}  // namespace ppo

using namespace ppo;

extern "C" size_t ppo_normalizer_update_workspace_bytes(int64_t rows, int32_t dim) {
  if (rows <= 0 || dim <= 0) return 0;
  return plan_norm(rows, dim).total * sizeof(double);
}

extern "C" int ppo_normalizer_update(const ppo_column_block* blocks, int32_t num_blocks, int64_t rows,
                                     float* state_mean, float* state_var, float* state_std, int64_t* count,
                                     void* workspace, size_t workspace_bytes, ppo_stream_t stream) {
  PPO_REQUIRE(blocks && state_mean && state_var && state_std && count, "ppo_normalizer_update: null pointer");
  PPO_REQUIRE(num_blocks >= 1 && num_blocks <= kMaxBlocks, "ppo_normalizer_update: num_blocks=%d", num_blocks);
  PPO_REQUIRE(rows > 0, "ppo_normalizer_update: rows=%lld", (long long)rows);
  Blocks bl{};
  int dim = 0;
  for (int i = 0; i < num_blocks; ++i) {
    PPO_REQUIRE(blocks[i].src && blocks[i].width > 0 && blocks[i].stride >= blocks[i].width,
                "ppo_normalizer_update: block %d malformed", i);
    bl.b[i] = blocks[i];
    bl.col_begin[i] = dim;
    dim += blocks[i].width;
  }
  for (int i = num_blocks; i <= kMaxBlocks; ++i) bl.col_begin[i] = INT32_MAX;
  bl.count = num_blocks;
  bl.dim = dim;
  const NormPlan plan = plan_norm(rows, dim);
  PPO_REQUIRE(plan.slabs <= INT32_MAX, "ppo_normalizer_update: too many rows");
  PPO_REQUIRE(workspace && workspace_bytes >= plan.total * sizeof(double),
              "ppo_normalizer_update: workspace too small");
  double* ws = static_cast<double*>(workspace);
  double* partials = ws + plan.partial_off;
  double* bmean = ws + plan.mean_off;
  double* bvar = ws + plan.var_off;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int slabs = static_cast<int>(plan.slabs);
  const int rblocks = static_cast<int>(ceil_div(dim, kNormThreads));
  hipLaunchKernelGGL(moments_kernel, dim3(slabs), dim3(kNormThreads), 0, s, bl, rows, 0, bmean, partials);
  hipLaunchKernelGGL(moments_reduce_kernel, dim3(rblocks), dim3(kNormThreads), 0, s, partials, slabs, dim, rows,
                     bmean);
  hipLaunchKernelGGL(moments_kernel, dim3(slabs), dim3(kNormThreads), 0, s, bl, rows, 1, bmean, partials);
  hipLaunchKernelGGL(moments_reduce_kernel, dim3(rblocks), dim3(kNormThreads), 0, s, partials, slabs, dim, rows,
                     bvar);
  hipLaunchKernelGGL(running_update_kernel, dim3(1), dim3(kNormThreads), 0, s, bmean, bvar, dim, rows, state_mean,
                     state_var, state_std, count);
  return check_launch("normalizer_update");
}
