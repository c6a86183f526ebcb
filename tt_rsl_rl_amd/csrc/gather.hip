// A5 permutation gather (rsl_rl/storage/rollout_storage.py:232-259) and the observation-normaliser forward
// (rsl_rl/modules/normalization.py:46-48), fused: one pass over the rollout per update writes the packed,
// permuted, normalised row table that every mini-batch of every epoch then reads contiguously.
//
// One wavefront per destination row: each segment of the source row is read as a contiguous run of floats
// across the lanes (coalesced), so the kernel streams HBM at ~2 x 4 B per copied float plus the 8 B index.
#include "common.hpp"

#pragma clang fp contract(off)

namespace ppo {
namespace {

struct GatherArgs {
  ppo_gather_segment seg[PPO_MAX_GATHER_SEGMENTS];
  int32_t num_segments;
};

constexpr int kGatherThreads = 256;
constexpr int kRowsPerBlock = kGatherThreads / kWave;

__global__ __launch_bounds__(kGatherThreads) void gather_rows_kernel(const int64_t* __restrict__ perm, int64_t rows,
                                                                     int64_t src_rows, GatherArgs args, float* __restrict__ dst,
                                                                     int64_t dst_stride) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave_id = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  const int64_t wave_count = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
  for (int64_t j = wave_id; j < rows; j += wave_count) {
    const int64_t src_row = perm[j];
    if (src_row < 0 || src_row >= src_rows) continue;  // never read outside the source (the host checks perm)
    float* out = dst + j * dst_stride;
    for (int s = 0; s < args.num_segments; ++s) {
      const ppo_gather_segment& g = args.seg[s];
      const float* in = g.src + src_row * g.src_stride;
      float* o = out + g.dst_col;
      if (g.norm_mean != nullptr) {
        for (int c = lane; c < g.width; c += kWave) o[c] = (in[c] - g.norm_mean[c]) / (g.norm_std[c] + g.norm_eps);
      } else {
        for (int c = lane; c < g.width; c += kWave) o[c] = in[c];
      }
    }
  }
}

__global__ __launch_bounds__(256) void obs_normalize_kernel(const float* __restrict__ x, int64_t ldx,
                                                            float* __restrict__ y, int64_t ldy, int64_t rows,
                                                            int32_t width, const float* __restrict__ mean,
                                                            const float* __restrict__ std, float eps) {
  const int64_t total = rows * width;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / width;
    const int c = static_cast<int>(i - r * width);
    y[r * ldy + c] = (x[r * ldx + c] - mean[c]) / (std[c] + eps);
  }
}

}  // namespace
}  // namespace ppo

using namespace ppo;

extern "C" int ppo_gather_rows(const int64_t* perm, int64_t rows, int64_t src_rows,
                               const ppo_gather_segment* segments, int32_t num_segments, float* dst,
                               int64_t dst_stride, ppo_stream_t stream) {
  PPO_REQUIRE(perm && segments && dst, "ppo_gather_rows: null pointer");
  PPO_REQUIRE(rows > 0 && src_rows > 0, "ppo_gather_rows: rows=%lld src_rows=%lld", (long long)rows,
              (long long)src_rows);
  PPO_REQUIRE(num_segments > 0 && num_segments <= PPO_MAX_GATHER_SEGMENTS,
              "ppo_gather_rows: num_segments=%d outside [1, %d]", num_segments, PPO_MAX_GATHER_SEGMENTS);
  GatherArgs args{};
  args.num_segments = num_segments;
  for (int s = 0; s < num_segments; ++s) {
    const ppo_gather_segment& g = segments[s];
    PPO_REQUIRE(g.src != nullptr && g.width > 0 && g.src_stride >= g.width && g.dst_col >= 0,
                "ppo_gather_rows: segment %d malformed (width=%d stride=%lld col=%d)", s, g.width,
                (long long)g.src_stride, g.dst_col);
    PPO_REQUIRE(static_cast<int64_t>(g.dst_col) + g.width <= dst_stride,
                "ppo_gather_rows: segment %d ends at column %lld beyond dst_stride %lld", s,
                (long long)(g.dst_col + g.width), (long long)dst_stride);
    PPO_REQUIRE(g.norm_mean == nullptr || g.norm_std != nullptr, "ppo_gather_rows: segment %d has mean but no std",
                s);
    args.seg[s] = g;
  }
  const int64_t blocks = std::min<int64_t>(ceil_div(rows, kRowsPerBlock), 65536);
  hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kGatherThreads), 0,
                     static_cast<hipStream_t>(stream), perm, rows, src_rows, args, dst, dst_stride);
  return check_launch("gather_rows_kernel");
}

extern "C" int ppo_obs_normalize(const float* x, int64_t ldx, float* y, int64_t ldy, int64_t rows, int32_t width,
                                 const float* mean, const float* std, float eps, ppo_stream_t stream) {
  PPO_REQUIRE(x && y && mean && std, "ppo_obs_normalize: null pointer");
  PPO_REQUIRE(rows > 0 && width > 0 && ldx >= width && ldy >= width, "ppo_obs_normalize: bad shape");
  const int64_t blocks = std::min<int64_t>(ceil_div(rows * width, 256), 16384);
  hipLaunchKernelGGL(obs_normalize_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, ldx, y, ldy, rows, width, mean, std, eps);
  return check_launch("obs_normalize_kernel");
}
