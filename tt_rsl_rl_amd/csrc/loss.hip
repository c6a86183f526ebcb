// A8-A11: Gaussian policy head, clipped surrogate, clipped value loss, entropy bonus and the KL of the adaptive
// learning-rate rule, forward and backward in one pass over the mini-batch
// (rsl_rl/algorithms/ppo.py:226-285, rsl_rl/modules/distribution.py:183-238, torch's Normal / kl_divergence).
//
// The loss kernel writes dloss/dmu [R, A] and dloss/dV [R] and per-block fp64 partial sums (surrogate, value loss,
// KL, and the per-action dlogp/dlog(std) sums for the std-parameter gradient).  The partials are reduced in a
// fixed order by a single-block finalize kernel, which also applies the adaptive-KL learning-rate rule on the
// device, so the update loop never waits on the host.  HBM-bound: per row 5 A-wide fp32 runs (mean, actions,
// old mean, old std in; dloss/dmu out) and 6 scalars.
//
// Gradients follow torch autograd's conventions: max() sends the gradient to the larger operand and splits it
// 50/50 on a tie; clamp() passes it on the closed interval [lo, hi].
#include <cstdlib>

#include "common.hpp"

#pragma clang fp contract(off)

namespace ppo {
namespace {

constexpr int kLossThreads = 256;
constexpr int kFixedCols = 3;     // surrogate, value loss, kl

// log(sqrt(2*pi)) and 0.5 + 0.5*log(2*pi) as the fp32 values torch subtracts / adds (Python doubles cast once).
constexpr double kLogSqrt2Pi = 0.91893853320467274178;
constexpr double kEntropyConst = 1.41893853320467274178;

struct LossParams {
  ppo_loss_args a;
  float ratio_lo, ratio_hi, vclip_lo, vclip_hi;
  float c_v, inv_rows_surr, inv_rows_value;
  float std_lo, std_hi;
};

__device__ inline double wave_sum(double x) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_down(x, off, 64);
  return x;
}

// std and its log exactly as torch builds them: clamp in the parameter's space, exp for the log form, then
// Normal.log_prob / entropy take log(scale) of that std.
__device__ inline void std_of(const LossParams& p, int a, float& sd, float& log_sd) {
  std_from_param(p.a.std_param[a], p.a.std_type, p.std_lo, p.std_hi, sd, log_sd);
}

// Each group of L lanes (L = 32 for A <= 32, else 64) owns one row at a time, lane a <-> action a, so the A-wide
// row segments are read as one coalesced run.  The per-row log-prob is a butterfly sum over the group in fp64; the
// row scalars (advantage, returns, ...) are broadcast loads.  Every lane keeps fp64 running sums of its own action's
// std-gradient and KL terms across the rows it visits, so no per-action reduction is needed until the block ends.
template <int L>
__global__ __launch_bounds__(kLossThreads) void ppo_loss_kernel(const LossParams p, double* __restrict__ partials) {
  constexpr int kGroups = kLossThreads / L;  // rows in flight per block
  const ppo_loss_args& a = p.a;
  const int A = a.num_actions;
  const int cols = kFixedCols + A;
  const int lane = threadIdx.x & 63;
  const int j = threadIdx.x % L;             // action of this lane
  const int grp = threadIdx.x / L;           // row slot of this lane
  const bool act_lane = j < A;

  __shared__ float s_std[PPO_MAX_ACTIONS], s_var[PPO_MAX_ACTIONS], s_log[PPO_MAX_ACTIONS];
  __shared__ double s_red[kLossThreads / 64][kFixedCols + PPO_MAX_ACTIONS];
  for (int q = threadIdx.x; q < A; q += kLossThreads) {
    float sd, lg;
    std_of(p, q, sd, lg);
    s_std[q] = sd;
    s_var[q] = sd * sd;
    s_log[q] = lg;
  }
  __syncthreads();
  const float sd = act_lane ? s_std[j] : 1.0f;
  const float var = act_lane ? s_var[j] : 1.0f;
  const float lg = act_lane ? s_log[j] : 0.0f;
  const float c_lp = static_cast<float>(kLogSqrt2Pi);

  double acc_surr = 0.0, acc_val = 0.0, acc_kl = 0.0, acc_dstd = 0.0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kGroups;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kGroups + grp; r < a.rows; r += stride) {
    float d = 0.0f;
    double t_acc = 0.0;
    if (act_lane) {
      const float mu = a.mean[r * a.ld_mean + j];
      d = a.actions[r * a.ld_batch + j] - mu;
      float t = -(d * d) / (2.0f * var);
      t = t - lg;
      t = t - c_lp;
      t_acc = static_cast<double>(t);
      // torch kl_divergence(Normal(old), Normal(new)) = 0.5 * (var_ratio + t1 - 1 - log(var_ratio))
      const float q = a.old_std[r * a.ld_batch + j] / sd;
      const float vr = q * q;
      const float e = (a.old_mean[r * a.ld_batch + j] - mu) / sd;
      const float t1 = e * e;
      acc_kl += static_cast<double>(0.5f * (((vr + t1) - 1.0f) - logf(vr)));
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) t_acc += __shfl_xor(t_acc, off, 64);
    const float logp = static_cast<float>(t_acc);
    const float old_logp = a.old_logp[r * a.ld_batch];
    const float adv = a.advantages[r * a.ld_batch];
    const float ratio = expf(logp - old_logp);
    const float nadv = -adv;
    const float s1 = nadv * ratio;
    const float rc = fminf(fmaxf(ratio, p.ratio_lo), p.ratio_hi);
    const float s2 = nadv * rc;
    // d surrogate_loss / d ratio with torch's max / clamp conventions
    const float gs = p.inv_rows_surr;
    const float ga = s1 > s2 ? gs : (s1 == s2 ? gs * 0.5f : 0.0f);
    const float gb = s2 > s1 ? gs : (s1 == s2 ? gs * 0.5f : 0.0f);
    const bool in_clip = (ratio >= p.ratio_lo) && (ratio <= p.ratio_hi);
    const float g_ratio = ga * nadv + (in_clip ? gb * nadv : 0.0f);
    const float g_logp = g_ratio * ratio;
    if (act_lane) {
      a.d_mean[r * a.ld_dmean + j] = (g_logp * d) / var;
      // d logp / d log(std_j) = d^2 / var_j - 1
      acc_dstd += static_cast<double>(g_logp) * (static_cast<double>(d) * d / var - 1.0);
    }
    if (j == 0) {
      const float v = a.value[r * a.ld_value];
      const float v_old = a.old_values[r * a.ld_batch];
      const float ret = a.returns[r * a.ld_batch];
      const float gv = p.inv_rows_value;  // c_v / R
      float dv, vloss;
      if (a.use_clipped_value_loss) {
        const float dvo = v - v_old;
        const float dvc = fminf(fmaxf(dvo, p.vclip_lo), p.vclip_hi);
        const float vc = v_old + dvc;
        const float e1 = v - ret, e2 = vc - ret;
        const float l1 = e1 * e1, l2 = e2 * e2;
        vloss = fmaxf(l1, l2);
        const float g1 = l1 > l2 ? gv : (l1 == l2 ? gv * 0.5f : 0.0f);
        const float g2 = l2 > l1 ? gv : (l1 == l2 ? gv * 0.5f : 0.0f);
        const bool in_vclip = (dvo >= p.vclip_lo) && (dvo <= p.vclip_hi);
        dv = (g1 * 2.0f) * e1 + (in_vclip ? (g2 * 2.0f) * e2 : 0.0f);
      } else {
        const float e = ret - v;
        vloss = e * e;
        dv = -((gv * 2.0f) * e);
      }
      a.d_value[r * a.ld_dvalue] = dv;
      acc_surr += static_cast<double>(fmaxf(s1, s2));
      acc_val += static_cast<double>(vloss);
    }
  }

  // block partials in a fixed order: fold the row groups of each wavefront, then the wavefronts through LDS
  const int wave = threadIdx.x >> 6;
  acc_kl = wave_sum(acc_kl);                   // lane 0 holds the wave's KL sum
  if (L == 32) {
    acc_dstd += __shfl_xor(acc_dstd, 32, 64);  // lanes j and j + 32 hold the same action
    acc_surr += __shfl_xor(acc_surr, 32, 64);
    acc_val += __shfl_xor(acc_val, 32, 64);
  }
  if (lane == 0) {
    s_red[wave][0] = acc_surr;
    s_red[wave][1] = acc_val;
    s_red[wave][2] = acc_kl;
  }
  if (lane < A && lane < L) s_red[wave][kFixedCols + lane] = acc_dstd;
  __syncthreads();
  // column-major partials [cols][blocks]: the finalize reads each column as one contiguous run
  for (int c = threadIdx.x; c < cols; c += kLossThreads) {
    double sum = 0.0;
    for (int w = 0; w < kLossThreads / 64; ++w) sum += s_red[w][c];
    partials[static_cast<int64_t>(c) * gridDim.x + blockIdx.x] = sum;
  }
}

constexpr int kFinThreads = 1024;
constexpr int kFinUnroll = 8;

// One block: 16 wavefronts own the columns (wave w: columns w, w + 16, ...).  Each lane keeps kFinUnroll
// independent fp64 partial sums over the block partials (b = lane + 64 u + 512 i), so a column costs one or two
// load round trips; the partial sums are combined in a fixed order, then across the wave by a fixed butterfly, so
// the result is the same on every run.  The per-action std values are computed once, in parallel.
__global__ __launch_bounds__(kFinThreads) void ppo_loss_finalize_kernel(
    const LossParams p, const double* __restrict__ partials, int nblocks, float* __restrict__ d_std_param,
    ppo_device_state* __restrict__ state, int adaptive, float kl_hi, float kl_lo, double* __restrict__ trace) {
  const int A = p.a.num_actions;
  const int cols = kFixedCols + A;
  __shared__ double s_col[kFixedCols + PPO_MAX_ACTIONS];
  __shared__ float s_sd[PPO_MAX_ACTIONS], s_lg[PPO_MAX_ACTIONS];
  __shared__ double s_entropy;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int c = wave; c < cols; c += kFinThreads / 64) {
    const double* col = partials + static_cast<int64_t>(c) * nblocks;
    double acc[kFinUnroll];
#pragma unroll
    for (int u = 0; u < kFinUnroll; ++u) acc[u] = 0.0;
    for (int b0 = lane; b0 < nblocks; b0 += 64 * kFinUnroll) {
#pragma unroll
      for (int u = 0; u < kFinUnroll; ++u) {
        const int b = b0 + 64 * u;
        if (b < nblocks) acc[u] += col[b];
      }
    }
    double sum = 0.0;
#pragma unroll
    for (int u = 0; u < kFinUnroll; ++u) sum += acc[u];
    sum = wave_sum(sum);
    if (lane == 0) s_col[c] = sum;
  }
  if (threadIdx.x < A) {
    float sd, lg;
    std_of(p, threadIdx.x, sd, lg);
    s_sd[threadIdx.x] = sd;
    s_lg[threadIdx.x] = lg;
  }
  __syncthreads();
  if (wave == 0) {  // every row's entropy is the same sum over actions: fp64, fixed-order butterfly
    const float ec = static_cast<float>(kEntropyConst);
    double e = 0.0;
    for (int j = lane; j < A; j += 64) e += static_cast<double>(ec + s_lg[j]);
    e = wave_sum(e);
    if (lane == 0) s_entropy = e;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const double R = static_cast<double>(p.a.rows);
    const float surrogate = static_cast<float>(s_col[0] / R);
    const float value = static_cast<float>(s_col[1] / R);
    const float kl_mean = static_cast<float>(s_col[2] / R);
    const float entropy = static_cast<float>(s_entropy);
    double lr = state->learning_rate;
    if (adaptive) {
      if (kl_mean > kl_hi) {
        lr = fmax(1e-5, lr / 1.5);
      } else if (kl_mean < kl_lo && kl_mean > 0.0f) {
        lr = fmin(1e-2, lr * 1.5);
      }
      state->learning_rate = lr;
    }
    state->sum_surrogate_loss += static_cast<double>(surrogate);
    state->sum_value_loss += static_cast<double>(value);
    state->sum_entropy += static_cast<double>(entropy);
    state->last_kl_mean = kl_mean;
    state->last_surrogate_loss = surrogate;
    state->last_value_loss = value;
    state->last_entropy = entropy;
    if (trace != nullptr) {
      double* t = trace + 5 * static_cast<int64_t>(state->num_minibatches);
      t[0] = kl_mean;
      t[1] = lr;
      t[2] = surrogate;
      t[3] = value;
      t[4] = entropy;
    }
    state->num_minibatches += 1;
  }
  // std-parameter gradient: d/dlog(std) = sum_r g_logp (d^2/var - 1) - c_e (entropy), then the clamp mask and
  // the chain rule of the parameterisation.
  const float c_e = static_cast<float>(p.a.entropy_coef);
  for (int j = threadIdx.x; j < A; j += kFinThreads) {
    const float q = p.a.std_param[j];
    const bool inside = (q >= p.std_lo) && (q <= p.std_hi);
    const double dlog = s_col[kFixedCols + j] - static_cast<double>(c_e);
    const double g = (p.a.std_type == PPO_STD_LOG) ? dlog : dlog / static_cast<double>(s_sd[j]);
    d_std_param[j] = inside ? static_cast<float>(g) : 0.0f;
  }
}

int lanes_per_row(int num_actions) { return num_actions <= 32 ? 32 : 64; }

// Blocks of the loss kernel (= block partials the finalize reduces), at most 512 (measured: 26.5 us for loss +
// finalize at 512, 28.0 at 1024, 32.2 at 256 on 24,576 rows); "PPO_HIP_LOSS_BLOCKS" overrides the cap
// (tuning aid).  Host arithmetic only: the workspace query must agree with the launch.
int64_t loss_blocks(int64_t rows, int num_actions) {
  const int groups = kLossThreads / lanes_per_row(num_actions);
  const char* e = std::getenv("PPO_HIP_LOSS_BLOCKS");
  const int64_t cap = e ? std::max(1, std::min(1024, std::atoi(e))) : 512;
  return std::max<int64_t>(1, std::min<int64_t>(cap, ceil_div(rows, groups)));
}

int make_params(const ppo_loss_args* args, LossParams& p, const char* who) {
  PPO_REQUIRE(args != nullptr, "%s: null args", who);
  const ppo_loss_args& a = *args;
  PPO_REQUIRE(a.rows > 0 && a.rows <= (int64_t)INT32_MAX * kLossThreads, "%s: rows=%lld", who, (long long)a.rows);
  PPO_REQUIRE(a.num_actions > 0 && a.num_actions <= PPO_MAX_ACTIONS, "%s: num_actions=%d outside [1, %d]", who,
              a.num_actions, PPO_MAX_ACTIONS);
  PPO_REQUIRE(a.std_type == PPO_STD_LOG || a.std_type == PPO_STD_SCALAR, "%s: std_type=%d", who, a.std_type);
  PPO_REQUIRE(a.mean && a.value && a.actions && a.old_mean && a.old_std && a.old_logp && a.advantages &&
                  a.old_values && a.returns && a.std_param && a.d_mean && a.d_value,
              "%s: null pointer in args", who);
  PPO_REQUIRE(a.ld_mean >= a.num_actions && a.ld_dmean >= a.num_actions && a.ld_batch >= 1 && a.ld_value >= 1 &&
                  a.ld_dvalue >= 1,
              "%s: bad leading dimension", who);
  p.a = a;
  p.ratio_lo = static_cast<float>(1.0 - a.clip_param);
  p.ratio_hi = static_cast<float>(1.0 + a.clip_param);
  p.vclip_lo = static_cast<float>(-a.clip_param);
  p.vclip_hi = static_cast<float>(a.clip_param);
  p.c_v = static_cast<float>(a.value_loss_coef);
  const float rows_f = static_cast<float>(a.rows);
  p.inv_rows_surr = 1.0f / rows_f;
  p.inv_rows_value = p.c_v / rows_f;
  p.std_lo = static_cast<float>(a.std_lo);
  p.std_hi = static_cast<float>(a.std_hi);
  return PPO_OK;
}

}  // namespace
}  // namespace ppo

using namespace ppo;

extern "C" size_t ppo_loss_workspace_bytes(int64_t rows, int32_t num_actions) {
  if (rows <= 0 || num_actions <= 0 || num_actions > PPO_MAX_ACTIONS) return 0;
  return sizeof(double) * static_cast<size_t>(loss_blocks(rows, num_actions)) * (kFixedCols + num_actions);
}

extern "C" int ppo_gauss_ppo_loss(const ppo_loss_args* args, void* workspace, size_t workspace_bytes,
                                  ppo_stream_t stream) {
  LossParams p{};
  int rc = make_params(args, p, "ppo_gauss_ppo_loss");
  if (rc != PPO_OK) return rc;
  const size_t need = ppo_loss_workspace_bytes(args->rows, args->num_actions);
  PPO_REQUIRE(workspace != nullptr && workspace_bytes >= need, "ppo_gauss_ppo_loss: workspace too small (%zu < %zu)",
              workspace_bytes, need);
  const int64_t blocks = loss_blocks(args->rows, args->num_actions);
  if (lanes_per_row(args->num_actions) == 32) {
    hipLaunchKernelGGL(ppo_loss_kernel<32>, dim3(static_cast<unsigned>(blocks)), dim3(kLossThreads), 0,
                       static_cast<hipStream_t>(stream), p, static_cast<double*>(workspace));
  } else {
    hipLaunchKernelGGL(ppo_loss_kernel<64>, dim3(static_cast<unsigned>(blocks)), dim3(kLossThreads), 0,
                       static_cast<hipStream_t>(stream), p, static_cast<double*>(workspace));
  }
  return check_launch("ppo_loss_kernel");
}

extern "C" int ppo_loss_finalize(const ppo_loss_args* args, const void* workspace, size_t workspace_bytes,
                                 float* d_std_param, ppo_device_state* state, int32_t adaptive, double desired_kl,
                                 double* trace, ppo_stream_t stream) {
  LossParams p{};
  int rc = make_params(args, p, "ppo_loss_finalize");
  if (rc != PPO_OK) return rc;
  const size_t need = ppo_loss_workspace_bytes(args->rows, args->num_actions);
  PPO_REQUIRE(workspace != nullptr && workspace_bytes >= need, "ppo_loss_finalize: workspace too small");
  PPO_REQUIRE(d_std_param != nullptr && state != nullptr, "ppo_loss_finalize: null pointer");
  const int64_t blocks = loss_blocks(args->rows, args->num_actions);
  // upstream compares the fp32 kl_mean with the Python floats desired_kl*2 and desired_kl/2, which torch rounds
  // to fp32 before comparing.
  const float kl_hi = static_cast<float>(desired_kl * 2.0);
  const float kl_lo = static_cast<float>(desired_kl / 2.0);
  hipLaunchKernelGGL(ppo_loss_finalize_kernel, dim3(1), dim3(kFinThreads), 0, static_cast<hipStream_t>(stream), p,
                     static_cast<const double*>(workspace), static_cast<int>(blocks), d_std_param, state,
                     adaptive ? 1 : 0, kl_hi, kl_lo, trace);
  return check_launch("ppo_loss_finalize_kernel");
}
