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

// The loss terms of row r.  Lane j of the row's group holds action j (act_lane: j < A) and its mean mu; every lane
// holds the row's value v.  Returns dloss/dmu_j in dmu and dloss/dV in dv (on every lane); adds the row's KL term and
// the lane's std-gradient term to acc_kl / acc_dstd on action lanes, and the surrogate / value loss to acc_surr /
// acc_val on lane 0 of the group.  The log-prob is a butterfly sum over the group in fp64.
template <int L>
__device__ __forceinline__ void row_terms(const LossParams& p, int64_t r, int j, bool act_lane, float mu, float v,
                                          float sd, float var, float lg, float& dmu, float& dv, double& acc_kl,
                                          double& acc_dstd, double& acc_surr, double& acc_val) {
  const ppo_loss_args& a = p.a;
  const float c_lp = static_cast<float>(kLogSqrt2Pi);
  float d = 0.0f;
  double t_acc = 0.0;
  if (act_lane) {
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
  dmu = 0.0f;
  if (act_lane) {
    dmu = (g_logp * d) / var;
    // d logp / d log(std_j) = d^2 / var_j - 1
    acc_dstd += static_cast<double>(g_logp) * (static_cast<double>(d) * d / var - 1.0);
  }
  const float v_old = a.old_values[r * a.ld_batch];
  const float ret = a.returns[r * a.ld_batch];
  const float gv = p.inv_rows_value;  // c_v / R
  float vloss;
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
  if (j == 0) {
    acc_surr += static_cast<double>(fmaxf(s1, s2));
    acc_val += static_cast<double>(vloss);
  }
}

// Block partials in a fixed order: fold the row groups of each wavefront, then the wavefronts through LDS; written
// column-major [cols][blocks], so the finalize reads each column as one contiguous run.
template <int L>
__device__ __forceinline__ void write_partials(int A, double acc_surr, double acc_val, double acc_kl, double acc_dstd,
                                               double (*s_red)[kFixedCols + PPO_MAX_ACTIONS],
                                               double* __restrict__ partials) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cols = kFixedCols + A;
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
  for (int c = threadIdx.x; c < cols; c += kLossThreads) {
    double sum = 0.0;
    for (int w = 0; w < kLossThreads / 64; ++w) sum += s_red[w][c];
    partials[static_cast<int64_t>(c) * gridDim.x + blockIdx.x] = sum;
  }
}

// Each group of L lanes (L = 32 for A <= 32, else 64) owns one row at a time, lane a <-> action a, so the A-wide
// row segments are read as one coalesced run.  The row scalars (advantage, returns, ...) are broadcast loads.  Every
// lane keeps fp64 running sums of its own action's std-gradient and KL terms across the rows it visits, so no
// per-action reduction is needed until the block ends.
template <int L>
__global__ __launch_bounds__(kLossThreads) void ppo_loss_kernel(const LossParams p, double* __restrict__ partials) {
  constexpr int kGroups = kLossThreads / L;  // rows in flight per block
  const ppo_loss_args& a = p.a;
  const int A = a.num_actions;
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

  double acc_surr = 0.0, acc_val = 0.0, acc_kl = 0.0, acc_dstd = 0.0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kGroups;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kGroups + grp; r < a.rows; r += stride) {
    const float mu = act_lane ? a.mean[r * a.ld_mean + j] : 0.0f;
    const float v = a.value[r * a.ld_value];
    float dmu, dv;
    row_terms<L>(p, r, j, act_lane, mu, v, sd, var, lg, dmu, dv, acc_kl, acc_dstd, acc_surr, acc_val);
    if (act_lane) a.d_mean[r * a.ld_dmean + j] = dmu;
    if (j == 0) a.d_value[r * a.ld_dvalue] = dv;
  }
  write_partials<L>(A, acc_surr, acc_val, acc_kl, acc_dstd, s_red, partials);
}

constexpr int kFinThreads = 1024;
constexpr int kFinWaves = kFinThreads / 64;
constexpr int kFinUnroll = 8;  // partials per lane and pass

// One block: 16 wavefronts own the columns (wave w: columns w + 16 it, it < CI = ceil(columns / 16)).  Each lane
// sums the block partials b = lane + 64 u (+ 512 per pass) in a fixed order, then the wave combines its lanes by a
// fixed butterfly, so the result is the same on every run.  The kernel is a chain of dependent steps, so every global
// load it needs (all its columns' partials for up to 512 blocks, the std parameter, the device state) is issued
// before the first wait: unconditional loads from clamped addresses, the out-of-range ones discarded afterwards.
template <int CI>
__global__ __launch_bounds__(kFinThreads) void ppo_loss_finalize_kernel(
    const LossParams p, const double* __restrict__ partials, int nblocks, float* __restrict__ d_std_param,
    ppo_device_state* __restrict__ state, int adaptive, float kl_hi, float kl_lo, double* __restrict__ trace,
    int trace_rows) {
  const int A = p.a.num_actions;
  const int cols = kFixedCols + A;
  __shared__ double s_col[kFixedCols + PPO_MAX_ACTIONS];
  __shared__ float s_sd[PPO_MAX_ACTIONS], s_lg[PPO_MAX_ACTIONS];
  __shared__ double s_entropy;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float q_param = p.a.std_param[threadIdx.x < A ? threadIdx.x : 0];
  // the state is written by this kernel's thread 0 only, at the end: read it now
  const double lr0 = state->learning_rate;
  const double sum_sur0 = state->sum_surrogate_loss, sum_val0 = state->sum_value_loss, sum_ent0 = state->sum_entropy;
  const int nmb = state->num_minibatches;
  double acc[CI];
#pragma unroll
  for (int it = 0; it < CI; ++it) acc[it] = 0.0;
  for (int b0 = lane; b0 < nblocks; b0 += 64 * kFinUnroll) {
    double x[CI][kFinUnroll];
#pragma unroll
    for (int it = 0; it < CI; ++it) {
      const double* col = partials + static_cast<int64_t>(min(wave + kFinWaves * it, cols - 1)) * nblocks;
#pragma unroll
      for (int u = 0; u < kFinUnroll; ++u) x[it][u] = col[min(b0 + 64 * u, nblocks - 1)];
    }
#pragma unroll
    for (int it = 0; it < CI; ++it)
#pragma unroll
      for (int u = 0; u < kFinUnroll; ++u) acc[it] += b0 + 64 * u < nblocks ? x[it][u] : 0.0;
  }
#pragma unroll
  for (int it = 0; it < CI; ++it) {
    const int c = wave + kFinWaves * it;
    const double sum = wave_sum(acc[it]);
    if (lane == 0 && c < cols) s_col[c] = sum;
  }
  if (threadIdx.x < A) {
    float sd, lg;
    std_from_param(q_param, p.a.std_type, p.std_lo, p.std_hi, sd, lg);
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
    double lr = lr0;
    if (adaptive) {
      if (kl_mean > kl_hi) {
        lr = fmax(1e-5, lr / 1.5);
      } else if (kl_mean < kl_lo && kl_mean > 0.0f) {
        lr = fmin(1e-2, lr * 1.5);
      }
      state->learning_rate = lr;
    }
    state->sum_surrogate_loss = sum_sur0 + static_cast<double>(surrogate);
    state->sum_value_loss = sum_val0 + static_cast<double>(value);
    state->sum_entropy = sum_ent0 + static_cast<double>(entropy);
    state->last_kl_mean = kl_mean;
    state->last_surrogate_loss = surrogate;
    state->last_value_loss = value;
    state->last_entropy = entropy;
    if (trace != nullptr && nmb < trace_rows) {  // rows past the caller's buffer are not written
      double* t = trace + 5 * static_cast<int64_t>(nmb);
      t[0] = kl_mean;
      t[1] = lr;
      t[2] = surrogate;
      t[3] = value;
      t[4] = entropy;
    }
    state->num_minibatches = nmb + 1;
  }
  // std-parameter gradient: d/dlog(std) = sum_r g_logp (d^2/var - 1) - c_e (entropy), then the clamp mask and
  // the chain rule of the parameterisation.
  const float c_e = static_cast<float>(p.a.entropy_coef);
  if (threadIdx.x < A) {
    const int j = threadIdx.x;
    const bool inside = (q_param >= p.std_lo) && (q_param <= p.std_hi);
    const double dlog = s_col[kFixedCols + j] - static_cast<double>(c_e);
    const double g = (p.a.std_type == PPO_STD_LOG) ? dlog : dlog / static_cast<double>(s_sd[j]);
    d_std_param[j] = inside ? static_cast<float>(g) : 0.0f;
  }
}

// ------------------------------------------------------------------------------------------------------------------
// The output layers fused with the loss: per 16-row tile one wavefront computes
//   mean = h_a W_a^T + b_a (v_mfma_f32_16x16x4f32), value = h_c . w_c + b_c (VALU),
//   the loss terms and dloss/dmean, dloss/dV of row_terms' mathematics,
//   dz_a = (dloss/dmean W_a) * ELU'(h_a) (MFMA) and dz_c = dloss/dV w_c * ELU'(h_c),
// so the rows' last hidden activations are read once and the three launches of the unfused path (output-layer
// forward, loss, output-layer input-grad with its weight transpose) become one.  ELU' is taken from the output:
// h > 0 ? 1 : h + 1.
//
// Register layout.  Lane l (row m = l % 16 of the tile, quarter q = l / 16) loads its row's activations as float4
// chunks 16g + 4q .. +3 (g = 0 .. K/16-1), which are exactly the MFMA operand values it supplies at the 4 steps of
// k-group g (any bijection of k is a valid order if both operands agree).  With the weights as the MFMA's first
// operand, accumulator element r of lane l holds row m and output column 4q + r of the 16-wide tile, so the lane
// owns the actions 16t + 4q + r (tile t = 0, 1; r = 0 .. 3): two float4 chunks of the row, and the four quarters of a
// row meet in two cross-lane shuffles.  The input-grad product uses the same roles: W^T (from LDS) first,
// dloss/dmean second (a = 16t + 4q + r is the lane's own element), so its accumulator holds row m, hidden units
// 16kt + 4q + r, which is the lane's own activation chunk kt: ELU' needs no reload.
// ------------------------------------------------------------------------------------------------------------------
constexpr int kHeadRows = 16;     // rows per wavefront tile
constexpr int kHeadWavesDefault = 4;
constexpr int kHeadMaxK = 128;    // hidden width of either model's last hidden layer
constexpr int kHeadMaxA = 32;     // two 16-wide MFMA tiles of actions
constexpr int kHeadG = kHeadMaxK / 16;
constexpr int kHeadWs = kHeadMaxK + 4;  // LDS row stride of W [a][k]: rows 16 bytes apart modulo 256 -> no conflicts
constexpr int kHeadWts = kHeadMaxA + 4; // LDS row stride of W^T [k][a]: 144 bytes -> conflict-free 16-lane reads

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct HeadParams {
  LossParams lp;
  ppo_policy_head h;
};

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void st4(float* p, const f32x4& v) { *reinterpret_cast<f32x4*>(p) = v; }

// Stores columns c .. c+3 of a row, only those < n (the chunk's first column is < n).
__device__ __forceinline__ void st4_masked(float* row, int c, int n, const f32x4& v) {
  if (c + 3 < n) {
    *reinterpret_cast<f32x4*>(row + c) = v;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c + e < n) row[c + e] = v[e];
  }
}

// One tile's operands in registers: the lane's chunks of its row's activations and batch columns.
struct HeadTileIn {
  f32x4 ha[kHeadG], hc[kHeadG];
  f32x4 act[2], om[2], os[2];
  float old_logp, adv, v_old, ret;
};

__device__ __forceinline__ void head_load_tile(const HeadParams& P, int64_t tile, int lane, HeadTileIn& in) {
  const ppo_loss_args& a = P.lp.a;
  const ppo_policy_head& H = P.h;
  const int m = lane & 15, q = lane >> 4;
  const int64_t row = tile * kHeadRows + m;
  const int64_t rr = row < a.rows ? row : a.rows - 1;  // the tail tile's lanes past R read the last row
  const int GA = H.k_actor / 16, GC = H.k_critic / 16;
#pragma unroll
  for (int g = 0; g < kHeadG; ++g)
    if (g < GA) in.ha[g] = ld4(H.h_actor + rr * H.ld_h_actor + 16 * g + 4 * q);
#pragma unroll
  for (int g = 0; g < kHeadG; ++g)
    if (g < GC) in.hc[g] = ld4(H.h_critic + rr * H.ld_h_critic + 16 * g + 4 * q);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    // chunks at or past A read chunk 0 (in bounds) and are never used
    const int c = 16 * t + 4 * q < a.num_actions ? 16 * t + 4 * q : 0;
    in.act[t] = ld4(a.actions + rr * a.ld_batch + c);
    in.om[t] = ld4(a.old_mean + rr * a.ld_batch + c);
    in.os[t] = ld4(a.old_std + rr * a.ld_batch + c);
  }
  in.old_logp = a.old_logp[rr * a.ld_batch];
  in.adv = a.advantages[rr * a.ld_batch];
  in.v_old = a.old_values[rr * a.ld_batch];
  in.ret = a.returns[rr * a.ld_batch];
}

// Sum over the four quarters of a row (lanes m, m + 16, m + 32, m + 48): every lane gets the same value.
template <typename T>
__device__ __forceinline__ T quarter_sum(T x) {
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}

template <int WAVES>
__global__ __launch_bounds__(64 * WAVES) void ppo_head_kernel(const HeadParams P, double* __restrict__ partials) {
  const LossParams& p = P.lp;
  const ppo_loss_args& a = p.a;
  const ppo_policy_head& H = P.h;
  const int A = a.num_actions;
  const int KA = H.k_actor, KC = H.k_critic;
  const int64_t R = a.rows;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = lane & 15, q = lane >> 4;
  const int NT = A > 16 ? 2 : 1;  // 16-wide action tiles
  constexpr int kThreads = 64 * WAVES;

  __shared__ __align__(16) float s_w[kHeadMaxA * kHeadWs];    // W_a [a][k], rows a >= A zero
  __shared__ __align__(16) float s_wt[kHeadMaxK * kHeadWts];  // W_a^T [k][a], columns a >= A zero
  __shared__ __align__(16) float s_wc[kHeadMaxK];
  __shared__ float s_b[kHeadMaxA], s_std[kHeadMaxA], s_var[kHeadMaxA], s_log[kHeadMaxA];
  __shared__ double s_red[WAVES][kFixedCols + PPO_MAX_ACTIONS];

  // the first tile's loads go out before the weights are staged, so both latencies overlap
  const int64_t tiles = ceil_div(R, kHeadRows);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * WAVES;
  int64_t tile = static_cast<int64_t>(blockIdx.x) * WAVES + wave;
  HeadTileIn in;
  if (tile < tiles) head_load_tile(P, tile, lane, in);

  {  // W_a as float4 rows: every load issued before the first LDS write
    constexpr int kPer = kHeadMaxA * kHeadMaxK / 4 / kThreads;
    const int cpr = KA / 4;  // float4 chunks per weight row
    f32x4 wv[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = threadIdx.x + u * kThreads;
      const int r = i / cpr, k = 4 * (i - r * cpr);
      const bool ok = i < kHeadMaxA * cpr && r < A;
      wv[u] = ld4(H.w_actor + (ok ? static_cast<int64_t>(r) * KA + k : 0));
      if (!ok) wv[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    constexpr int kWcPer = (kHeadMaxK + kThreads - 1) / kThreads;
    float wc[kWcPer];
#pragma unroll
    for (int u = 0; u < kWcPer; ++u) {
      const int k = threadIdx.x + u * kThreads;
      wc[u] = k < KC ? H.w_critic[k] : 0.0f;
    }
    float sp = 0.0f, b = 0.0f;
    if (threadIdx.x < A) {
      sp = a.std_param[threadIdx.x];
      b = H.b_actor[threadIdx.x];
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = threadIdx.x + u * kThreads;
      if (i < kHeadMaxA * cpr) {
        const int r = i / cpr, k = 4 * (i - r * cpr);
        st4(s_w + r * kHeadWs + k, wv[u]);
#pragma unroll
        for (int e = 0; e < 4; ++e) s_wt[(k + e) * kHeadWts + r] = wv[u][e];
      }
    }
#pragma unroll
    for (int u = 0; u < kWcPer; ++u)
      if (threadIdx.x + u * kThreads < KC) s_wc[threadIdx.x + u * kThreads] = wc[u];
    if (threadIdx.x < kHeadMaxA) {
      float sd = 1.0f, lg = 0.0f;
      if (threadIdx.x < A) std_from_param(sp, a.std_type, p.std_lo, p.std_hi, sd, lg);
      s_b[threadIdx.x] = b;
      s_std[threadIdx.x] = sd;
      s_var[threadIdx.x] = sd * sd;
      s_log[threadIdx.x] = lg;
    }
  }
  __syncthreads();
  const float b_c = H.b_critic[0];
  const int GA = KA / 16, GC = KC / 16;
  const float c_lp = static_cast<float>(kLogSqrt2Pi);

  double acc_surr = 0.0, acc_val = 0.0, acc_kl = 0.0;
  double acc_dstd[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) acc_dstd[v] = 0.0;

  for (; tile < tiles; tile += stride) {
    const int64_t row = tile * kHeadRows + m;
    const bool valid = row < R;

    // critic: value, value loss and its input-grad, finished before the actor's registers are needed
    float part = 0.0f;
#pragma unroll
    for (int g = 0; g < kHeadG; ++g) {
      if (g < GC) {
        const f32x4 w = ld4(s_wc + 16 * g + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) part = fmaf(in.hc[g][e], w[e], part);
      }
    }
    const float v = quarter_sum(part) + b_c;
    const float gv = p.inv_rows_value;  // c_v / R
    const float v_old = in.v_old, ret = in.ret;
    float vloss, dv;
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
    if (valid) {
#pragma unroll
      for (int g = 0; g < kHeadG; ++g) {
        if (g < GC) {
          const f32x4 w = ld4(s_wc + 16 * g + 4 * q);
          f32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = dv * w[e];
            o[e] = in.hc[g][e] > 0.0f ? x : x * (in.hc[g][e] + 1.0f);
          }
          st4(H.dz_critic + row * H.ld_dz_critic + 16 * g + 4 * q, o);
        }
      }
      if (q == 0) {
        a.d_value[row * a.ld_dvalue] = dv;
        if (H.value) H.value[row * H.ld_value] = v;
        acc_val += static_cast<double>(vloss);
      }
    }

    // actor forward: acc[t] = (h_a W_a^T) of action tile t, transposed in the lanes as described above
    f32x4 acc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (t < NT) {
#pragma unroll
        for (int g = 0; g < kHeadG; ++g) {
          if (g < GA) {
            const f32x4 w = ld4(s_w + (16 * t + m) * kHeadWs + 16 * g + 4 * q);
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2)
              acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[s2], in.ha[g][s2], acc[t], 0, 0, 0);
          }
        }
      }
    }

    // loss terms of the lane's actions (column j = 16t + 4q + r)
    float mu[8], dd[8];
    double t_acc = 0.0;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * t + 4 * q + r;
        const int v2 = 4 * t + r;
        mu[v2] = acc[t][r] + s_b[j];
        dd[v2] = 0.0f;
        if (j < A) {
          const float var = s_var[j];
          const float d = in.act[t][r] - mu[v2];
          dd[v2] = d;
          float tt = -(d * d) / (2.0f * var);
          tt = tt - s_log[j];
          tt = tt - c_lp;
          t_acc += static_cast<double>(tt);
          // torch kl_divergence(Normal(old), Normal(new)) = 0.5 * (var_ratio + t1 - 1 - log(var_ratio))
          const float sd = s_std[j];
          const float qq = in.os[t][r] / sd;
          const float vr = qq * qq;
          const float ee = (in.om[t][r] - mu[v2]) / sd;
          const float t1 = ee * ee;
          if (valid) acc_kl += static_cast<double>(0.5f * (((vr + t1) - 1.0f) - logf(vr)));
        }
      }
    }
    const float logp = static_cast<float>(quarter_sum(t_acc));
    const float ratio = expf(logp - in.old_logp);
    const float nadv = -in.adv;
    const float s1 = nadv * ratio;
    const float rc = fminf(fmaxf(ratio, p.ratio_lo), p.ratio_hi);
    const float s2 = nadv * rc;
    // d surrogate_loss / d ratio with torch's max / clamp conventions
    const float gs = p.inv_rows_surr;
    const float ga = s1 > s2 ? gs : (s1 == s2 ? gs * 0.5f : 0.0f);
    const float gb = s2 > s1 ? gs : (s1 == s2 ? gs * 0.5f : 0.0f);
    const bool in_clip = (ratio >= p.ratio_lo) && (ratio <= p.ratio_hi);
    const float g_ratio = ga * nadv + (in_clip ? gb * nadv : 0.0f);
    const float g_logp = valid ? g_ratio * ratio : 0.0f;
    if (valid && q == 0) acc_surr += static_cast<double>(fmaxf(s1, s2));
    float dm[8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * t + 4 * q + r;
        const int v2 = 4 * t + r;
        dm[v2] = 0.0f;
        if (j < A) {
          const float var = s_var[j];
          dm[v2] = (g_logp * dd[v2]) / var;
          // d logp / d log(std_j) = d^2 / var_j - 1
          acc_dstd[v2] += static_cast<double>(g_logp) * (static_cast<double>(dd[v2]) * dd[v2] / var - 1.0);
        }
      }
    }
    if (valid) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int c = 16 * t + 4 * q;
        if (c < A) {
          st4_masked(a.d_mean + row * a.ld_dmean, c, A, f32x4{dm[4 * t], dm[4 * t + 1], dm[4 * t + 2], dm[4 * t + 3]});
          if (H.mean) st4_masked(H.mean + row * H.ld_mean, c, A, f32x4{mu[4 * t], mu[4 * t + 1], mu[4 * t + 2],
                                                                         mu[4 * t + 3]});
        }
      }
    }

    // actor input-grad, 16 hidden units at a time: dz = (dloss/dmean W_a) * ELU'(h_a)
#pragma unroll
    for (int kt = 0; kt < kHeadG; ++kt) {
      if (kt < GA) {
        f32x4 acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (t < NT) {
            const f32x4 w = ld4(s_wt + (16 * kt + m) * kHeadWts + 16 * t + 4 * q);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(w[r], dm[4 * t + r], acc2, 0, 0, 0);
          }
        }
        if (valid) {
          const f32x4 hv = in.ha[kt];
          f32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = hv[e] > 0.0f ? acc2[e] : acc2[e] * (hv[e] + 1.0f);
          st4(H.dz_actor + row * H.ld_dz_actor + 16 * kt + 4 * q, o);
        }
      }
    }
    if (tile + stride < tiles) head_load_tile(P, tile + stride, lane, in);
  }

  // block partials: wave sums, the per-action std-gradient terms folded over the 16 rows of each quarter, then the
  // waves in a fixed order; column-major [cols][blocks] like ppo_loss_kernel's, for ppo_loss_finalize_kernel
  acc_surr = wave_sum(acc_surr);
  acc_val = wave_sum(acc_val);
  acc_kl = wave_sum(acc_kl);
#pragma unroll
  for (int v2 = 0; v2 < 8; ++v2) {
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) acc_dstd[v2] += __shfl_xor(acc_dstd[v2], off, 64);
  }
  if (lane == 0) {
    s_red[wave][0] = acc_surr;
    s_red[wave][1] = acc_val;
    s_red[wave][2] = acc_kl;
  }
  if (m == 0) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * t + 4 * q + r;
        if (j < A) s_red[wave][kFixedCols + j] = acc_dstd[4 * t + r];
      }
  }
  __syncthreads();
  const int cols = kFixedCols + A;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    double sum = 0.0;
    for (int w = 0; w < WAVES; ++w) sum += s_red[w][c];
    partials[static_cast<int64_t>(c) * gridDim.x + blockIdx.x] = sum;
  }
}

bool head_supported(int num_actions, int k_actor, int k_critic) {
  return num_actions >= 1 && num_actions <= kHeadMaxA && k_actor >= 16 && k_actor <= kHeadMaxK &&
         k_actor % 16 == 0 && k_critic >= 16 && k_critic <= kHeadMaxK && k_critic % 16 == 0;
}

// Wavefronts per block of the fused head kernel; in a build with PPO_HIP_TUNING, "PPO_HIP_HEAD_WAVES" (1, 2 or 4)
// overrides it (tuning aid).
int head_waves() {
#ifdef PPO_HIP_TUNING
  const char* e = std::getenv("PPO_HIP_HEAD_WAVES");
  const int w = e ? std::atoi(e) : kHeadWavesDefault;
  return (w == 1 || w == 2 || w == 4) ? w : kHeadWavesDefault;
#else
  return kHeadWavesDefault;
#endif
}

// Blocks of the fused head kernel: one 16-row tile per wave while that fits in 1024 blocks, else 1024 blocks that
// stride over the tiles (the partials the finalize reduces stay bounded).  Host arithmetic only: the workspace query
// must agree with the launch.
int64_t head_blocks(int64_t rows) {
  return std::max<int64_t>(1, std::min<int64_t>(1024, ceil_div(ceil_div(rows, kHeadRows), head_waves())));
}

int lanes_per_row(int num_actions) { return num_actions <= 32 ? 32 : 64; }

// Blocks of the loss kernel (= block partials the finalize reduces), at most 512 (measured: 26.5 us for loss +
// finalize at 512, 28.0 at 1024, 32.2 at 256 on 24,576 rows); in a build with PPO_HIP_TUNING, "PPO_HIP_LOSS_BLOCKS"
// overrides the cap (tuning aid).  Host arithmetic only: the workspace query must agree with the launch.
int64_t loss_blocks(int64_t rows, int num_actions) {
  const int groups = kLossThreads / lanes_per_row(num_actions);
#ifdef PPO_HIP_TUNING
  const char* e = std::getenv("PPO_HIP_LOSS_BLOCKS");
  const int64_t cap = e ? std::max(1, std::min(1024, std::atoi(e))) : 512;
#else
  const int64_t cap = 512;
#endif
  return std::max<int64_t>(1, std::min<int64_t>(cap, ceil_div(rows, groups)));
}

// head: the fused output-layer entry point, which computes mean / value itself (args->mean / value unused).
int make_params(const ppo_loss_args* args, LossParams& p, const char* who, bool head = false) {
  PPO_REQUIRE(args != nullptr, "%s: null args", who);
  const ppo_loss_args& a = *args;
  PPO_REQUIRE(a.rows > 0 && a.rows <= (int64_t)INT32_MAX * kLossThreads, "%s: rows=%lld", who, (long long)a.rows);
  PPO_REQUIRE(a.num_actions > 0 && a.num_actions <= PPO_MAX_ACTIONS, "%s: num_actions=%d outside [1, %d]", who,
              a.num_actions, PPO_MAX_ACTIONS);
  PPO_REQUIRE(a.std_type == PPO_STD_LOG || a.std_type == PPO_STD_SCALAR, "%s: std_type=%d", who, a.std_type);
  PPO_REQUIRE((head || (a.mean && a.value)) && a.actions && a.old_mean && a.old_std && a.old_logp && a.advantages &&
                  a.old_values && a.returns && a.std_param && a.d_mean && a.d_value,
              "%s: null pointer in args", who);
  PPO_REQUIRE((head || (a.ld_mean >= a.num_actions && a.ld_value >= 1)) && a.ld_dmean >= a.num_actions &&
                  a.ld_batch >= 1 && a.ld_dvalue >= 1,
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

int launch_finalize(const LossParams& p, const void* workspace, int64_t blocks, float* d_std_param,
                    ppo_device_state* state, int32_t adaptive, double desired_kl, double* trace, int32_t trace_rows,
                    ppo_stream_t stream) {
  // upstream compares the fp32 kl_mean with the Python floats desired_kl*2 and desired_kl/2, which torch rounds
  // to fp32 before comparing.
  const float kl_hi = static_cast<float>(desired_kl * 2.0);
  const float kl_lo = static_cast<float>(desired_kl / 2.0);
  const int ci = static_cast<int>(ceil_div(kFixedCols + p.a.num_actions, kFinWaves));
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(1), dim3(kFinThreads), 0, static_cast<hipStream_t>(stream), p,
                       static_cast<const double*>(workspace), static_cast<int>(blocks), d_std_param, state,
                       adaptive ? 1 : 0, kl_hi, kl_lo, trace, trace != nullptr ? trace_rows : 0);
  };
  static_assert(kFixedCols + PPO_MAX_ACTIONS <= 5 * kFinWaves, "five column rounds cover every column");
  switch (ci) {
    case 1: launch(ppo_loss_finalize_kernel<1>); break;
    case 2: launch(ppo_loss_finalize_kernel<2>); break;
    case 3: launch(ppo_loss_finalize_kernel<3>); break;
    case 4: launch(ppo_loss_finalize_kernel<4>); break;
    default: launch(ppo_loss_finalize_kernel<5>); break;
  }
  return check_launch("ppo_loss_finalize_kernel");
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
                                 double* trace, int32_t trace_rows, ppo_stream_t stream) {
  LossParams p{};
  int rc = make_params(args, p, "ppo_loss_finalize");
  PPO_REQUIRE(trace == nullptr || trace_rows > 0, "ppo_loss_finalize: trace_rows=%d", trace_rows);
  if (rc != PPO_OK) return rc;
  const size_t need = ppo_loss_workspace_bytes(args->rows, args->num_actions);
  PPO_REQUIRE(workspace != nullptr && workspace_bytes >= need, "ppo_loss_finalize: workspace too small");
  PPO_REQUIRE(d_std_param != nullptr && state != nullptr, "ppo_loss_finalize: null pointer");
  return launch_finalize(p, workspace, loss_blocks(args->rows, args->num_actions), d_std_param, state, adaptive,
                         desired_kl, trace, trace_rows, stream);
}

extern "C" int ppo_gauss_ppo_head_supported(int32_t num_actions, int32_t k_actor, int32_t k_critic) {
  return head_supported(num_actions, k_actor, k_critic) ? 1 : 0;
}

extern "C" size_t ppo_head_workspace_bytes(int64_t rows, int32_t num_actions) {
  if (rows <= 0 || num_actions <= 0 || num_actions > PPO_MAX_ACTIONS) return 0;
  return sizeof(double) * static_cast<size_t>(head_blocks(rows)) * (kFixedCols + num_actions);
}

extern "C" int ppo_gauss_ppo_head(const ppo_loss_args* args, const ppo_policy_head* head, void* workspace,
                                  size_t workspace_bytes, float* d_std_param, ppo_device_state* state,
                                  int32_t adaptive, double desired_kl, double* trace, int32_t trace_rows,
                                  ppo_stream_t stream) {
  static const char* who = "ppo_gauss_ppo_head";
  PPO_REQUIRE(args != nullptr && head != nullptr, "%s: null args / head", who);
  PPO_REQUIRE(trace == nullptr || trace_rows > 0, "%s: trace_rows=%d", who, trace_rows);
  const ppo_policy_head& h = *head;
  const ppo_loss_args& a = *args;
  PPO_REQUIRE(head_supported(a.num_actions, h.k_actor, h.k_critic),
              "%s: num_actions=%d k_actor=%d k_critic=%d not supported (num_actions <= %d, k_actor and k_critic "
              "multiples of 16, both <= %d)",
              who, a.num_actions, h.k_actor, h.k_critic, kHeadMaxA, kHeadMaxK);
  HeadParams P{};
  int rc = make_params(args, P.lp, who, true);
  if (rc != PPO_OK) return rc;
  PPO_REQUIRE(h.h_actor && h.w_actor && h.b_actor && h.h_critic && h.w_critic && h.b_critic && h.dz_actor &&
                  h.dz_critic,
              "%s: null pointer in head", who);
  PPO_REQUIRE(d_std_param != nullptr && state != nullptr, "%s: null pointer", who);
  // float4 rows: 16-byte aligned bases, leading dimensions in whole float4s
  auto vec_ok = [](const void* ptr, int64_t ld) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0 && ld % 4 == 0; };
  PPO_REQUIRE(vec_ok(h.w_actor, h.k_actor) && vec_ok(h.h_actor, h.ld_h_actor) && h.ld_h_actor >= h.k_actor && vec_ok(h.h_critic, h.ld_h_critic) &&
                  h.ld_h_critic >= h.k_critic && vec_ok(h.dz_actor, h.ld_dz_actor) && h.ld_dz_actor >= h.k_actor &&
                  vec_ok(h.dz_critic, h.ld_dz_critic) && h.ld_dz_critic >= h.k_critic &&
                  vec_ok(a.actions, a.ld_batch) && vec_ok(a.old_mean, a.ld_batch) && vec_ok(a.old_std, a.ld_batch) &&
                  vec_ok(a.d_mean, a.ld_dmean) && (h.mean == nullptr || (vec_ok(h.mean, h.ld_mean) &&
                                                                         h.ld_mean >= a.num_actions)) &&
                  (h.value == nullptr || h.ld_value >= 1),
              "%s: rows must be 16-byte aligned with leading dimensions that are multiples of 4 floats", who);
  P.h = h;
  const size_t need = ppo_head_workspace_bytes(a.rows, a.num_actions);
  PPO_REQUIRE(workspace != nullptr && workspace_bytes >= need, "%s: workspace too small (%zu < %zu)", who,
              workspace_bytes, need);
  const int64_t blocks = head_blocks(a.rows);
  auto launch = [&](auto kernel, int waves) {
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(64 * waves), 0,
                       static_cast<hipStream_t>(stream), P, static_cast<double*>(workspace));
  };
  switch (head_waves()) {
#ifdef PPO_HIP_TUNING
    case 1: launch(ppo_head_kernel<1>, 1); break;
    case 2: launch(ppo_head_kernel<2>, 2); break;
#endif
    default: launch(ppo_head_kernel<kHeadWavesDefault>, kHeadWavesDefault); break;
  }
  rc = check_launch("ppo_head_kernel");
  if (rc != PPO_OK) return rc;
  return launch_finalize(P.lp, workspace, blocks, d_std_param, state, adaptive, desired_kl, trace, trace_rows,
                         stream);
}
