// A12 + A13: per-group gradient-norm clipping (torch.nn.utils.clip_grad_norm_, rsl_rl/algorithms/ppo.py:309-310)
// fused with Adam (torch.optim.Adam, single-tensor path, ppo.py:311) over flat parameter / gradient / moment
// buffers; ppo_optim_step runs the same launches with the other optimisers upstream resolves (AdamW, SGD, RMSprop).  ppo_adam_step, two launches:
//   1. sum of squares of the gradient, one fp64 partial per 1024-element chunk (chunks never straddle groups);
//   2. every block re-reduces its group's partials in the same fixed order (so all blocks agree bit for bit),
//      derives the clip coefficient and streams p, g, m, v once: 16 B read + 12 B written per parameter
//      (+4 B rewriting the clipped gradient, which upstream leaves in .grad).
// ppo_adam_step_prenorm is launch 2 alone, on the per-group partial rows that the weight-grad reduce wrote while it
// stored the gradients (ppo_linear_bwd_dw_norm).
// The element update follows torch's fp32 operation order with contraction disabled.
#include <mutex>

#include "common.hpp"

#pragma clang fp contract(off)

// Scratch of ppo_adam_step_static: the per-chunk partial sums of squares in a file-scope device array instead of a
// caller workspace, so that call allocates nothing.  Every GPU the library runs on holds its own copy until the
// process ends.  In host code the array's name is not a device address: the address of the current device's copy
// comes from hipGetSymbolAddress (static_scratch below) and only that address is handed to kernels.
static __device__ __align__(256) double scratch[PPO_ADAM_STATIC_SCRATCH_DOUBLES];

namespace ppo {
namespace {

constexpr int kAdamThreads = 256;
constexpr int kChunk = 1024;  // ~420 blocks for the humanoid models: every CU busy
static_assert(kChunk == 4 * kAdamThreads, "vector path: one float4 per thread per chunk");

struct GroupTable {
  int64_t begin[PPO_MAX_PARAM_GROUPS + 1];
  int32_t first_chunk[PPO_MAX_PARAM_GROUPS + 1];
  int32_t num_groups;
};

__device__ inline int group_of_chunk(const GroupTable& t, int chunk) {
  int g = 0;
#pragma unroll
  for (int i = 1; i < PPO_MAX_PARAM_GROUPS; ++i)
    if (i < t.num_groups && chunk >= t.first_chunk[i]) g = i;
  return g;
}

__device__ inline double block_sum256(double x, double* red) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_down(x, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  double s = 0.0;
  for (int w = 0; w < kAdamThreads / 64; ++w) s += red[w];
  __syncthreads();
  return s;  // same value in every thread
}

// VEC: every group boundary is a multiple of 4 floats (the host checks), so each chunk is whole 16-byte vectors:
// one float4 per thread per 1024-element chunk.
template <bool VEC>
__global__ __launch_bounds__(kAdamThreads) void grad_sqnorm_kernel(const float* __restrict__ grads, GroupTable t,
                                                                   double* __restrict__ partials) {
  __shared__ double red[kAdamThreads / 64];
  const int chunk = blockIdx.x;
  const int g = group_of_chunk(t, chunk);
  const int64_t lo = t.begin[g] + static_cast<int64_t>(chunk - t.first_chunk[g]) * kChunk;
  const int64_t hi = min(lo + kChunk, t.begin[g + 1]);
  double acc = 0.0;
  if constexpr (VEC) {
    const int64_t i = lo + 4 * static_cast<int64_t>(threadIdx.x);
    if (i < hi) {
      const float4 q = *reinterpret_cast<const float4*>(grads + i);
      const double a = q.x, b = q.y, c = q.z, d = q.w;
      acc = ((a * a + b * b) + c * c) + d * d;
    }
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += kAdamThreads) {
      const double v = grads[i];
      acc += v * v;
    }
  }
  const double s = block_sum256(acc, red);
  if (threadIdx.x == 0) partials[chunk] = s;
}

// Mirrored parameters (ppo_param_mirror): element begin + r * cols + c of the flat buffer also goes to
// dst[r * ld + c].
struct MirrorTable {
  int64_t begin[PPO_MAX_PARAM_MIRRORS], end[PPO_MAX_PARAM_MIRRORS], ld[PPO_MAX_PARAM_MIRRORS];
  float* dst[PPO_MAX_PARAM_MIRRORS];
  int32_t cols[PPO_MAX_PARAM_MIRRORS];
  int32_t count;
};

__device__ __forceinline__ void mirror_store(const MirrorTable& mt, int64_t i, float p) {
#pragma unroll
  for (int k = 0; k < PPO_MAX_PARAM_MIRRORS; ++k) {
    if (k < mt.count && i >= mt.begin[k] && i < mt.end[k]) {
      const int64_t rel = i - mt.begin[k];
      const int64_t r = rel / mt.cols[k];
      mt.dst[k][r * mt.ld[k] + (rel - r * mt.cols[k])] = p;
    }
  }
}

struct AdamScalars {
  float max_norm, w1, b2, c2, eps, bc2_sqrt;
  double bc1;
  double weight_decay;  // AdamW: decoupled decay, p *= 1 - lr * weight_decay before the step
  float alpha, c_alpha;  // RMSprop: square_avg = alpha square_avg + (1 - alpha) g^2
};

// One parameter's update in torch's fp32 operation order.
__device__ __forceinline__ void adam_elem(float& p, float& g, float& m, float& v, float coef, float neg_step,
                                          const AdamScalars& s) {
  g = g * coef;
  m = m + s.w1 * (g - m);
  v = v * s.b2;
  v = v + (s.c2 * g) * g;
  const float denom = sqrtf(v) / s.bc2_sqrt + s.eps;
  p = p + (neg_step * m) / denom;
}

// The other optimisers upstream resolves (rsl_rl/utils/utils.py:71-96), torch's single-tensor update with the
// defaults upstream leaves them (torch/optim/{adamw,sgd,rmsprop}.py): AdamW = p *= fl(1 - lr wd) (Python double,
// rounded once), then Adam's update; SGD (no momentum, no decay) p = p - lr g (torch's vectorised add: one fused
// multiply-add); RMSprop (no momentum, not centred) square_avg = square_avg alpha + (1 - alpha) g g, p = p - lr g /
// (sqrt(square_avg) + eps).  m holds square_avg for RMSprop; SGD keeps no state.
__device__ __forceinline__ void sgd_elem(float& p, float& g, float coef, float neg_lr) {
  g = g * coef;
  p = fmaf(g, neg_lr, p);
}

__device__ __forceinline__ void rmsprop_elem(float& p, float& g, float& sa, float coef, float neg_lr,
                                             const AdamScalars& s) {
  g = g * coef;
  sa = sa * s.alpha;
  sa = sa + (s.c_alpha * g) * g;
  const float avg = sqrtf(sa) + s.eps;
  p = p + (neg_lr * g) / avg;
}

// PRE: the group's squared norm is the sum of column g of the PPO_DW_NORM_BLOCKS partial rows the weight-grad reduce
// wrote (ppo_adam_step_prenorm); else the sum of the group's per-chunk partials from grad_sqnorm_kernel.  KIND: the
// update rule (PPO_OPTIM_*); the Adam instantiations are the plain Adam kernel.
template <bool VEC, bool PRE, int KIND = PPO_OPTIM_ADAM>
__global__ __launch_bounds__(kAdamThreads) void adam_kernel(float* __restrict__ params, float* __restrict__ grads,
                                                            float* __restrict__ exp_avg,
                                                            float* __restrict__ exp_avg_sq, GroupTable t,
                                                            AdamScalars s, const double* __restrict__ partials,
                                                            ppo_device_state* __restrict__ state, MirrorTable mt) {
  constexpr bool kAdam = KIND == PPO_OPTIM_ADAM || KIND == PPO_OPTIM_ADAMW;
  constexpr bool kState0 = KIND != PPO_OPTIM_SGD, kState1 = kAdam;
  __shared__ double red[kAdamThreads / 64];
  const int chunk = blockIdx.x;
  const int g = group_of_chunk(t, chunk);
  double acc = 0.0;
  if constexpr (PRE) {
    for (int r = threadIdx.x; r < PPO_DW_NORM_BLOCKS; r += kAdamThreads) acc += partials[r * PPO_MAX_PARAM_GROUPS + g];
  } else {
    for (int c = t.first_chunk[g] + threadIdx.x; c < t.first_chunk[g + 1]; c += kAdamThreads) acc += partials[c];
  }
  const double sq = block_sum256(acc, red);
  const float total = static_cast<float>(sqrt(sq));
  const float coef = fminf(s.max_norm / (total + 1e-6f), 1.0f);
  const double lr = state->learning_rate;
  const float neg_step = static_cast<float>(kAdam ? -(lr / s.bc1) : -lr);
  const float decay = static_cast<float>(1.0 - lr * s.weight_decay);
  if (chunk == t.first_chunk[g] && threadIdx.x == 0 && g < 4) {
    state->total_norm[g] = total;
    state->clip_coef[g] = coef;
  }
  // one element: p, its gradient and the state this rule keeps
  auto update = [&](float& p, float& gr, float& m, float& v) {
    if constexpr (KIND == PPO_OPTIM_ADAM) {
      adam_elem(p, gr, m, v, coef, neg_step, s);
    } else if constexpr (KIND == PPO_OPTIM_ADAMW) {
      p = p * decay;
      adam_elem(p, gr, m, v, coef, neg_step, s);
    } else if constexpr (KIND == PPO_OPTIM_SGD) {
      sgd_elem(p, gr, coef, neg_step);
    } else {
      rmsprop_elem(p, gr, m, coef, neg_step, s);
    }
  };
  const int64_t lo = t.begin[g] + static_cast<int64_t>(chunk - t.first_chunk[g]) * kChunk;
  const int64_t hi = min(lo + kChunk, t.begin[g + 1]);
  if constexpr (VEC) {
    const int64_t i = lo + 4 * static_cast<int64_t>(threadIdx.x);
    if (i < hi) {
      float4 p = *reinterpret_cast<const float4*>(params + i);
      float4 gr = *reinterpret_cast<const float4*>(grads + i);
      float4 m = {0.0f, 0.0f, 0.0f, 0.0f}, v = {0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (kState0) m = *reinterpret_cast<const float4*>(exp_avg + i);
      if constexpr (kState1) v = *reinterpret_cast<const float4*>(exp_avg_sq + i);
      update(p.x, gr.x, m.x, v.x);
      update(p.y, gr.y, m.y, v.y);
      update(p.z, gr.z, m.z, v.z);
      update(p.w, gr.w, m.w, v.w);
      *reinterpret_cast<float4*>(params + i) = p;
      *reinterpret_cast<float4*>(grads + i) = gr;
      if constexpr (kState0) *reinterpret_cast<float4*>(exp_avg + i) = m;
      if constexpr (kState1) *reinterpret_cast<float4*>(exp_avg_sq + i) = v;
      if (mt.count > 0) {  // (a float4 may straddle a mirror's first or last element: per element)
        mirror_store(mt, i, p.x);
        mirror_store(mt, i + 1, p.y);
        mirror_store(mt, i + 2, p.z);
        mirror_store(mt, i + 3, p.w);
      }
    }
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += kAdamThreads) {
      float p = params[i], gr = grads[i], m = 0.0f, v = 0.0f;
      if constexpr (kState0) m = exp_avg[i];
      if constexpr (kState1) v = exp_avg_sq[i];
      update(p, gr, m, v);
      params[i] = p;
      grads[i] = gr;
      if constexpr (kState0) exp_avg[i] = m;
      if constexpr (kState1) exp_avg_sq[i] = v;
      if (mt.count > 0) mirror_store(mt, i, p);
    }
  }
}

int build_table(const int64_t* group_begin, int num_groups, GroupTable& t, int& chunks) {
  PPO_REQUIRE(group_begin != nullptr && num_groups >= 1 && num_groups <= PPO_MAX_PARAM_GROUPS,
              "ppo_adam_step: num_groups=%d outside [1, %d]", num_groups, PPO_MAX_PARAM_GROUPS);
  t = GroupTable{};
  t.num_groups = num_groups;
  int64_t c = 0;
  for (int g = 0; g <= num_groups; ++g) {
    t.begin[g] = group_begin[g];
    if (g > 0) PPO_REQUIRE(group_begin[g] > group_begin[g - 1], "ppo_adam_step: group %d is empty", g - 1);
  }
  PPO_REQUIRE(group_begin[0] == 0, "ppo_adam_step: group_begin[0] must be 0");
  for (int g = 0; g < num_groups; ++g) {
    t.first_chunk[g] = static_cast<int32_t>(c);
    c += ceil_div(group_begin[g + 1] - group_begin[g], kChunk);
    PPO_REQUIRE(c < INT32_MAX, "ppo_adam_step: too many parameters");
  }
  t.first_chunk[num_groups] = static_cast<int32_t>(c);
  for (int g = num_groups + 1; g <= PPO_MAX_PARAM_GROUPS; ++g) t.first_chunk[g] = INT32_MAX;
  chunks = static_cast<int>(c);
  return PPO_OK;
}

size_t workspace_bytes_for(int64_t num_params) {
  if (num_params <= 0) return 0;
  return sizeof(double) * static_cast<size_t>(ceil_div(num_params, kChunk) + PPO_MAX_PARAM_GROUPS);
}

// The current device's copy of `scratch`, looked up once per device (with that device current) and kept.
std::mutex g_scratch_mutex;
double* g_scratch[kMaxDevices] = {};

int static_scratch(double** out) {
  int dev = -1;
  PPO_HIP_CHECK(hipGetDevice(&dev));
  PPO_REQUIRE(dev >= 0 && dev < kMaxDevices, "ppo_adam_step_static: device %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    PPO_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    PPO_REQUIRE(p != nullptr, "ppo_adam_step_static: no device address for the scratch array");
    g_scratch[dev] = static_cast<double*>(p);
  }
  *out = g_scratch[dev];
  return PPO_OK;
}

// prenorm != nullptr: one launch taking the norms from the weight-grad reduce's partial rows; else the per-chunk
// norm pass into `workspace`, then the update.
// The rule-specific hyperparameters of ppo_optim_step (Adam: kind only).
struct OptimRule {
  int kind = PPO_OPTIM_ADAM;
  double weight_decay = 0.0, alpha = 0.0;
};

template <int KIND>
void launch_update(bool vec, bool pre, int chunks, hipStream_t st, float* params, float* grads, float* s0, float* s1,
                   const GroupTable& t, const AdamScalars& s, const double* partials, ppo_device_state* state,
                   const MirrorTable& mt) {
  if (pre) {
    if (vec) {
      hipLaunchKernelGGL((adam_kernel<true, true, KIND>), dim3(chunks), dim3(kAdamThreads), 0, st, params, grads, s0,
                         s1, t, s, partials, state, mt);
    } else {
      hipLaunchKernelGGL((adam_kernel<false, true, KIND>), dim3(chunks), dim3(kAdamThreads), 0, st, params, grads,
                         s0, s1, t, s, partials, state, mt);
    }
  } else if (vec) {
    hipLaunchKernelGGL((adam_kernel<true, false, KIND>), dim3(chunks), dim3(kAdamThreads), 0, st, params, grads, s0,
                       s1, t, s, partials, state, mt);
  } else {
    hipLaunchKernelGGL((adam_kernel<false, false, KIND>), dim3(chunks), dim3(kAdamThreads), 0, st, params, grads, s0,
                       s1, t, s, partials, state, mt);
  }
}

int adam_step(const char* who, float* params, float* grads, float* exp_avg, float* exp_avg_sq,
              const int64_t* group_begin, int32_t num_groups, double max_grad_norm, double beta1, double beta2,
              double eps, double bc1, double bc2_sqrt, ppo_device_state* state, void* workspace,
              size_t workspace_bytes, const double* prenorm, ppo_stream_t stream,
              const ppo_param_mirror* mirrors = nullptr, int num_mirrors = 0, const OptimRule& rule = OptimRule{}) {
  const bool adam = rule.kind == PPO_OPTIM_ADAM || rule.kind == PPO_OPTIM_ADAMW;
  PPO_REQUIRE(rule.kind >= PPO_OPTIM_ADAM && rule.kind <= PPO_OPTIM_RMSPROP, "%s: optimizer kind %d", who, rule.kind);
  PPO_REQUIRE(params && grads && state && (rule.kind == PPO_OPTIM_SGD || exp_avg) && (!adam || exp_avg_sq),
              "%s: null pointer", who);
  GroupTable t;
  int chunks = 0;
  int rc = build_table(group_begin, num_groups, t, chunks);
  if (rc != PPO_OK) return rc;
  MirrorTable mt{};
  PPO_REQUIRE(num_mirrors >= 0 && num_mirrors <= PPO_MAX_PARAM_MIRRORS && (num_mirrors == 0 || mirrors != nullptr),
              "%s: %d mirrors (at most %d, with their table)", who, num_mirrors, PPO_MAX_PARAM_MIRRORS);
  for (int k = 0; k < num_mirrors; ++k) {
    const ppo_param_mirror& q = mirrors[k];
    const int64_t end = q.begin + static_cast<int64_t>(q.rows) * q.cols;
    PPO_REQUIRE(q.dst != nullptr && q.rows > 0 && q.cols > 0 && q.ld_dst >= q.cols && q.begin >= 0 &&
                    end <= group_begin[num_groups],
                "%s: mirror %d malformed (begin=%lld rows=%d cols=%d ld=%lld)", who, k, (long long)q.begin, q.rows,
                q.cols, (long long)q.ld_dst);
    for (int j = 0; j < k; ++j)
      PPO_REQUIRE(end <= mt.begin[j] || q.begin >= mt.end[j], "%s: mirrors %d and %d overlap", who, j, k);
    mt.begin[k] = q.begin;
    mt.end[k] = end;
    mt.ld[k] = q.ld_dst;
    mt.dst[k] = q.dst;
    mt.cols[k] = q.cols;
  }
  mt.count = num_mirrors;
  if (prenorm == nullptr) {
    const size_t need = workspace_bytes_for(group_begin[num_groups]);
    PPO_REQUIRE(workspace != nullptr && workspace_bytes >= need, "%s: workspace too small (%zu < %zu)", who,
                workspace_bytes, need);
  }
  PPO_REQUIRE(!adam || (bc1 > 0.0 && bc2_sqrt > 0.0), "%s: bias corrections must be positive", who);
  AdamScalars s{};
  // torch passes max_norm, 1 - beta1, beta2, 1 - beta2 and eps as Python doubles that the fp32 kernels round once
  s.max_norm = static_cast<float>(max_grad_norm);
  s.w1 = static_cast<float>(1.0 - beta1);
  s.b2 = static_cast<float>(beta2);
  s.c2 = static_cast<float>(1.0 - beta2);
  s.eps = static_cast<float>(eps);
  s.bc1 = adam ? bc1 : 1.0;
  s.bc2_sqrt = static_cast<float>(adam ? bc2_sqrt : 1.0);
  s.weight_decay = rule.kind == PPO_OPTIM_ADAMW ? rule.weight_decay : 0.0;
  s.alpha = static_cast<float>(rule.alpha);
  s.c_alpha = static_cast<float>(1.0 - rule.alpha);
  hipStream_t st = static_cast<hipStream_t>(stream);
  bool vec = true;
  const void* bufs[] = {params, grads, exp_avg, exp_avg_sq};
  for (const void* b : bufs) vec = vec && reinterpret_cast<uintptr_t>(b) % 16 == 0;
  for (int g = 0; g <= num_groups; ++g) vec = vec && group_begin[g] % 4 == 0;
  const double* partials = prenorm;
  if (prenorm == nullptr) {
    double* ws = static_cast<double*>(workspace);
    if (vec) {
      hipLaunchKernelGGL(grad_sqnorm_kernel<true>, dim3(chunks), dim3(kAdamThreads), 0, st, grads, t, ws);
    } else {
      hipLaunchKernelGGL(grad_sqnorm_kernel<false>, dim3(chunks), dim3(kAdamThreads), 0, st, grads, t, ws);
    }
    rc = check_launch("grad_sqnorm_kernel");
    if (rc != PPO_OK) return rc;
    partials = ws;
  }
  const bool pre = prenorm != nullptr;
  switch (rule.kind) {
    case PPO_OPTIM_ADAMW:
      launch_update<PPO_OPTIM_ADAMW>(vec, pre, chunks, st, params, grads, exp_avg, exp_avg_sq, t, s, partials, state,
                                     mt);
      break;
    case PPO_OPTIM_SGD:
      launch_update<PPO_OPTIM_SGD>(vec, pre, chunks, st, params, grads, exp_avg, exp_avg_sq, t, s, partials, state,
                                   mt);
      break;
    case PPO_OPTIM_RMSPROP:
      launch_update<PPO_OPTIM_RMSPROP>(vec, pre, chunks, st, params, grads, exp_avg, exp_avg_sq, t, s, partials,
                                       state, mt);
      break;
    default:
      launch_update<PPO_OPTIM_ADAM>(vec, pre, chunks, st, params, grads, exp_avg, exp_avg_sq, t, s, partials, state,
                                    mt);
  }
  return check_launch("adam_kernel");
}

}  // namespace
}  // namespace ppo

using namespace ppo;

extern "C" size_t ppo_adam_workspace_bytes(int64_t num_params) { return workspace_bytes_for(num_params); }

extern "C" int ppo_adam_step(float* params, float* grads, float* exp_avg, float* exp_avg_sq,
                             const int64_t* group_begin, int32_t num_groups, double max_grad_norm, double beta1,
                             double beta2, double eps, double bc1, double bc2_sqrt, ppo_device_state* state,
                             void* workspace, size_t workspace_bytes, ppo_stream_t stream) {
  return adam_step("ppo_adam_step", params, grads, exp_avg, exp_avg_sq, group_begin, num_groups, max_grad_norm,
                   beta1, beta2, eps, bc1, bc2_sqrt, state, workspace, workspace_bytes, nullptr, stream);
}

extern "C" int ppo_adam_step_prenorm(float* params, float* grads, float* exp_avg, float* exp_avg_sq,
                                     const int64_t* group_begin, int32_t num_groups, double max_grad_norm,
                                     double beta1, double beta2, double eps, double bc1, double bc2_sqrt,
                                     ppo_device_state* state, const double* norm_partials, ppo_stream_t stream) {
  PPO_REQUIRE(norm_partials != nullptr, "ppo_adam_step_prenorm: null norm_partials");
  return adam_step("ppo_adam_step_prenorm", params, grads, exp_avg, exp_avg_sq, group_begin, num_groups,
                   max_grad_norm, beta1, beta2, eps, bc1, bc2_sqrt, state, nullptr, 0, norm_partials, stream);
}

extern "C" int ppo_adam_step_prenorm_mirror(float* params, float* grads, float* exp_avg, float* exp_avg_sq,
                                            const int64_t* group_begin, int32_t num_groups, double max_grad_norm,
                                            double beta1, double beta2, double eps, double bc1, double bc2_sqrt,
                                            ppo_device_state* state, const double* norm_partials,
                                            const ppo_param_mirror* mirrors, int32_t num_mirrors, ppo_stream_t stream) {
  PPO_REQUIRE(norm_partials != nullptr, "ppo_adam_step_prenorm_mirror: null norm_partials");
  return adam_step("ppo_adam_step_prenorm_mirror", params, grads, exp_avg, exp_avg_sq, group_begin, num_groups,
                   max_grad_norm, beta1, beta2, eps, bc1, bc2_sqrt, state, nullptr, 0, norm_partials, stream, mirrors,
                   num_mirrors);
}

// The same kernels on the static scratch: the parameter count is checked against the array's capacity before any
// HIP call; every partial is written before it is read within the call, so nothing needs clearing between calls.
extern "C" int ppo_adam_step_static(float* params, float* grads, float* exp_avg, float* exp_avg_sq,
                                    const int64_t* group_begin, int32_t num_groups, double max_grad_norm,
                                    double beta1, double beta2, double eps, double bc1, double bc2_sqrt,
                                    ppo_device_state* state, ppo_stream_t stream) {
  PPO_REQUIRE(group_begin != nullptr && num_groups >= 1 && num_groups <= PPO_MAX_PARAM_GROUPS,
              "ppo_adam_step_static: num_groups=%d outside [1, %d]", num_groups, PPO_MAX_PARAM_GROUPS);
  const int64_t n = group_begin[num_groups];
  PPO_REQUIRE(n > 0 && n <= PPO_ADAM_STATIC_MAX_PARAMS,
              "ppo_adam_step_static: %lld parameters; the static scratch holds the partials of at most %lld "
              "(use ppo_adam_step with a workspace)", (long long)n, (long long)PPO_ADAM_STATIC_MAX_PARAMS);
  static_assert(PPO_ADAM_STATIC_MAX_PARAMS / kChunk + PPO_MAX_PARAM_GROUPS <= PPO_ADAM_STATIC_SCRATCH_DOUBLES,
                "the static scratch must hold the partials of the largest accepted parameter count");
  double* ws = nullptr;
  if (int rc = static_scratch(&ws)) return rc;
  return adam_step("ppo_adam_step_static", params, grads, exp_avg, exp_avg_sq, group_begin, num_groups,
                   max_grad_norm, beta1, beta2, eps, bc1, bc2_sqrt, state, ws,
                   sizeof(double) * PPO_ADAM_STATIC_SCRATCH_DOUBLES, nullptr, stream);
}

extern "C" int ppo_optim_step(float* params, float* grads, float* state0, float* state1, const int64_t* group_begin,
                              int32_t num_groups, double max_grad_norm, const ppo_optim_config* config, double bc1,
                              double bc2_sqrt, ppo_device_state* state, const double* norm_partials, void* workspace,
                              size_t workspace_bytes, const ppo_param_mirror* mirrors, int32_t num_mirrors,
                              ppo_stream_t stream) {
  PPO_REQUIRE(config != nullptr, "ppo_optim_step: null config");
  const ppo_optim_config& c = *config;
  PPO_REQUIRE(c.kind >= PPO_OPTIM_ADAM && c.kind <= PPO_OPTIM_RMSPROP, "ppo_optim_step: kind=%d", c.kind);
  PPO_REQUIRE(c.kind != PPO_OPTIM_RMSPROP || (c.alpha >= 0.0 && c.alpha <= 1.0), "ppo_optim_step: alpha=%g",
              c.alpha);
  PPO_REQUIRE(c.weight_decay >= 0.0, "ppo_optim_step: weight_decay=%g", c.weight_decay);
  OptimRule rule;
  rule.kind = c.kind;
  rule.weight_decay = c.weight_decay;
  rule.alpha = c.alpha;
  return adam_step("ppo_optim_step", params, grads, state0, state1, group_begin, num_groups, max_grad_norm, c.beta1,
                   c.beta2, c.eps, bc1, bc2_sqrt, state, workspace, workspace_bytes, norm_partials, stream, mirrors,
                   num_mirrors, rule);
}
