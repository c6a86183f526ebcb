// A7: EmpiricalNormalization.update (rsl_rl/modules/normalization.py:51-78, single process) over the rollout's
// stored observations, once per update after the epochs (rsl_rl/algorithms/ppo.py:327-330).
//
// Batch moments are reduced in fp64 and two passes (mean, then the biased variance around it): blocks own
// (64-column tile, row slab) pairs, a wavefront reads 64 consecutive columns of a row (one coalesced 256 B access),
// and the slab partials are summed by one block per column in a fixed order (deterministic).  The
// running-statistics update then replays torch's fp32 operation order on [dim] vectors.
#include "common.hpp"

#pragma clang fp contract(off)

namespace ppo {
namespace {

constexpr int kNormThreads = 256;
constexpr int kColTile = 64;     // one wavefront covers 64 consecutive columns
constexpr int kMaxSlabs = 256;   // row slabs (blocks along the rows)
constexpr int kMaxBlocks = PPO_MAX_GATHER_SEGMENTS;
constexpr int kUnroll = 16;   // rows per wave whose loads are in flight together

struct Blocks {
  ppo_column_block b[kMaxBlocks];
  int32_t col_begin[kMaxBlocks + 1];
  int32_t count;
  int32_t dim;
};

// pass 0: per-slab column sums; pass 1: per-slab sums of (x - mean)^2 (mean from stats[0..dim)).
// grid = (column tiles, slabs); lane = column inside the tile, wave w takes rows r0 + w, r0 + w + 4, ... (each row's
// value added in that order)
__global__ __launch_bounds__(kNormThreads) void moments_kernel(const Blocks bl, int64_t rows, int64_t slab_rows,
                                                               int pass, const double* __restrict__ stats,
                                                               double* __restrict__ partials) {
  __shared__ double red[kNormThreads / 64][kColTile];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * kColTile + lane;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * slab_rows;
  const int64_t r1 = min(rows, r0 + slab_rows);
  double acc = 0.0;
  if (c < bl.dim) {
    int i = 0;
    for (int k = 1; k < kMaxBlocks; ++k)
      if (k < bl.count && c >= bl.col_begin[k]) i = k;
    const float* src = bl.b[i].src + (c - bl.col_begin[i]);
    const int64_t stride = bl.b[i].stride;
    const double mu = pass ? stats[c] : 0.0;
    // kUnroll rows' loads in flight before they are added, in the same order as one row at a time (rows past the
    // slab re-read row r0 and are not added)
    constexpr int kStep = kNormThreads / 64;
    for (int64_t rb = r0 + wave; rb < r1; rb += kStep * kUnroll) {
      float x[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t r = rb + u * kStep;
        x[u] = src[(r < r1 ? r : r0) * stride];
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (rb + u * kStep < r1) {
          const double v = x[u];
          if (pass == 0) {
            acc += v;
          } else {
            const double d = v - mu;
            acc += d * d;
          }
        }
      }
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && c < bl.dim) {
    double s = 0.0;
    for (int w = 0; w < kNormThreads / 64; ++w) s += red[w][lane];
    partials[static_cast<int64_t>(blockIdx.y) * bl.dim + c] = s;
  }
}

// One block per column: fixed-order strided sums over the slab partials, then a fixed tree -> sum / rows.
__global__ __launch_bounds__(kNormThreads) void moments_reduce_kernel(const double* __restrict__ partials, int slabs,
                                                                      int dim, int64_t rows, double* __restrict__ out) {
  __shared__ double red[kNormThreads / 64];
  const int c = blockIdx.x;
  double acc = 0.0;
  for (int k = threadIdx.x; k < slabs; k += kNormThreads) acc += partials[static_cast<int64_t>(k) * dim + c];
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_down(acc, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int w = 0; w < kNormThreads / 64; ++w) s += red[w];
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
  int64_t slabs, slab_rows;
  size_t partial_off, mean_off, var_off, total;  // doubles
};

NormPlan plan_norm(int64_t rows, int dim) {
  NormPlan p;
  p.slabs = std::min<int64_t>(kMaxSlabs, ceil_div(rows, 64));
  p.slab_rows = ceil_div(rows, p.slabs);
  p.slabs = ceil_div(rows, p.slab_rows);
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
  const dim3 grid(static_cast<unsigned>(ceil_div(dim, kColTile)), static_cast<unsigned>(slabs));
  hipLaunchKernelGGL(moments_kernel, grid, dim3(kNormThreads), 0, s, bl, rows, plan.slab_rows, 0, bmean, partials);
  hipLaunchKernelGGL(moments_reduce_kernel, dim3(dim), dim3(kNormThreads), 0, s, partials, slabs, dim, rows, bmean);
  hipLaunchKernelGGL(moments_kernel, grid, dim3(kNormThreads), 0, s, bl, rows, plan.slab_rows, 1, bmean, partials);
  hipLaunchKernelGGL(moments_reduce_kernel, dim3(dim), dim3(kNormThreads), 0, s, partials, slabs, dim, rows, bvar);
  hipLaunchKernelGGL(running_update_kernel, dim3(1), dim3(kNormThreads), 0, s, bmean, bvar, dim, rows, state_mean,
                     state_var, state_std, count);
  return check_launch("normalizer_update");
}
