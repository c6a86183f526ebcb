/*
 * ppo_hip.h -- C ABI of the MI355X (gfx950) PPO update library (libppo_hip.so).
 *
 * Every entry point takes caller-owned DEVICE pointers, int64 sizes and a HIP stream (hipStream_t passed as an
 * opaque pointer; NULL = the default stream), enqueues its kernels on that stream and returns without
 * synchronising.  Return value: PPO_OK (0) or a negative status; ppo_last_error() then describes the failure
 * (thread-local).  No entry point allocates device memory: scratch space is passed in by the caller, sized by the
 * matching *_workspace_bytes() query.  All arithmetic is fp32 with fp64 accumulators where a reduction spans rows.
 *
 * The comment above each entry point names the upstream rsl_rl v5.5.2 code (file:line) whose arithmetic it
 * replaces; the host side that calls these mirrors rsl_rl's PPO / RolloutStorage / MLPModel interface.
 */
#ifndef PPO_HIP_H_
#define PPO_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ppo_stream_t; /* a hipStream_t */

enum {
  PPO_OK = 0,
  PPO_EINVAL = -1,       /* bad argument: null pointer, negative or inconsistent size, workspace too small */
  PPO_EHIP = -2,         /* the HIP runtime reported an error (launch failure, ...) */
  PPO_EUNSUPPORTED = -3, /* shape or option outside what the kernels implement */
};

/* hidden-layer activations: rsl_rl's resolve_nn_activation names (rsl_rl/utils/utils.py:34-68) with torch's default
 * arguments: elu, selu, relu, crelu (CELU, alpha 1), lrelu (slope 0.01), tanh, sigmoid, softplus (beta 1, threshold
 * 20), gelu (erf), swish (SiLU), mish, identity */
enum {
  PPO_ACT_NONE = 0, PPO_ACT_ELU = 1, PPO_ACT_SELU = 2, PPO_ACT_RELU = 3, PPO_ACT_CELU = 4, PPO_ACT_LRELU = 5,
  PPO_ACT_TANH = 6, PPO_ACT_SIGMOID = 7, PPO_ACT_SOFTPLUS = 8, PPO_ACT_GELU = 9, PPO_ACT_SILU = 10, PPO_ACT_MISH = 11,
  PPO_ACT_IDENTITY = 12
};
#define PPO_ACT_COUNT 13
/* what an input-grad's z_prev holds: the activation's input (pre-activation) or its output h = act(z); the output
 * serves only the monotone activations (elu, selu, relu, crelu, lrelu, tanh, sigmoid, identity) */
enum { PPO_ELU_FROM_INPUT = 0, PPO_ELU_FROM_OUTPUT = 1 };
enum { PPO_STD_SCALAR = 0, PPO_STD_LOG = 1 };

/* Description of the last failure on the calling thread ("" if none). */
const char* ppo_last_error(void);
/* ABI version of this header (bumped on any layout change of the structs below). */
int ppo_abi_version(void);

/* ------------------------------------------------------------------------------------------------------------------
 * A1  GAE reverse-time scan.  Replaces the loop of rsl_rl/algorithms/ppo.py:175-188 (PPO.compute_returns).
 * rewards, values, returns, advantages: [T, N] fp32 (time-major, row t*N+n); dones: [T, N] uint8;
 * last_values: [N].  For t = T-1..0, in upstream's fp32 operation order (no contraction):
 *   nt = 1 - done[t];  delta = (r[t] + (nt*gamma)*V[t+1]) - V[t];  adv = delta + ((nt*gamma)*lam)*adv;
 *   ret[t] = adv + V[t]   (V[T] = last_values, adv starts at 0);   advantages = ret - V  (ppo.py:188).
 * T * N < 2^31.
 * ------------------------------------------------------------------------------------------------------------------ */
int ppo_gae(const float* rewards, const float* values, const uint8_t* dones, const float* last_values,
            float* returns, float* advantages, int64_t num_steps, int64_t num_envs, float gamma, float lam,
            ppo_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------------
 * A2  Advantage normalisation.  Replaces rsl_rl/algorithms/ppo.py:189-191 (global) and :213-216 (per mini-batch):
 *   out[i*out_stride] = (x[i*in_stride] - mean(x)) / (std_unbiased(x) + eps),  i < n.
 * mean and the unbiased std are reduced in fp64 (two passes), rounded to fp32 like torch's mean()/std().
 * n == 1 copies x unchanged (upstream skips the normalisation when numel() == 1).  in-place (out == x) allowed.
 * ------------------------------------------------------------------------------------------------------------------ */
size_t ppo_adv_normalize_workspace_bytes(int64_t n);
int ppo_adv_normalize(const float* x, int64_t in_stride, float* out, int64_t out_stride, int64_t n, float eps,
                      void* workspace, size_t workspace_bytes, ppo_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------------
 * A5  Permutation gather into a packed row table.  Replaces the per-mini-batch fancy indexing of
 * rsl_rl/storage/rollout_storage.py:232-259 (mini_batch_generator): because upstream draws ONE permutation per
 * update and reuses it for every epoch, gathering the whole rollout once in permutation order makes mini-batch i
 * the contiguous row range [i*B/M, (i+1)*B/M) of the table.
 *   dst[j*dst_stride + seg.dst_col + c] = f(seg.src[perm[j]*seg.src_stride + c]),  c < seg.width,
 * with f the identity, or the observation normaliser (x - mean[c]) / (std[c] + eps)
 * (rsl_rl/modules/normalization.py:46-48) when seg.norm_mean != NULL.  Data moves bit-exactly.  A segment of kind
 * PPO_GATHER_KEEP_U8 reads uint8 done flags d instead and writes 1 - d as fp32 (the recurrent update's per-step
 * state-keep factor, rsl_rl/modules/rnn.py:56-60 resets the state where a done was stored).  Every element is read
 * as the aligned 32-bit word that holds it, so fp32 sources must be 4-byte aligned and the word around each flag
 * must lie in the flags' allocation (true of any device allocation, whose size is rounded up to 256 bytes or more).
 * perm: int64 [rows], every entry in [0, src_rows).
 * ------------------------------------------------------------------------------------------------------------------ */
/* A column block of a row-major fp32 matrix: columns [0, width) of rows r * stride. */
typedef struct ppo_column_block {
  const float* src; /* [rows, stride] */
  int64_t stride;
  int32_t width;
  int32_t reserved;
} ppo_column_block;

enum { PPO_GATHER_FLOAT = 0, PPO_GATHER_KEEP_U8 = 1 };
typedef struct ppo_gather_segment {
  const void* src;        /* [src_rows, src_stride] fp32 (PPO_GATHER_FLOAT) or uint8 (PPO_GATHER_KEEP_U8) */
  int64_t src_stride;     /* elements */
  int32_t width;          /* elements copied per row */
  int32_t dst_col;        /* first destination column */
  const float* norm_mean; /* [width] or NULL (PPO_GATHER_FLOAT only) */
  const float* norm_std;  /* [width] (required with norm_mean) */
  float norm_eps;
  int32_t kind;           /* PPO_GATHER_FLOAT or PPO_GATHER_KEEP_U8 */
} ppo_gather_segment;

#define PPO_MAX_GATHER_SEGMENTS 16

int ppo_gather_rows(const int64_t* perm, int64_t rows, int64_t src_rows, const ppo_gather_segment* segments,
                    int32_t num_segments, float* dst, int64_t dst_stride, ppo_stream_t stream);

/* dst[r, c .. c + width_i) = cols[i].src[r * cols[i].stride + 0 .. width_i), column blocks side by side in order
 * (c = sum of the earlier widths; at most PPO_MAX_INTERLEAVE_FLOATS in all), for r < rows: the rollout's
 * per-transition scalars (log-prob, advantage, value, return) packed into one short record per row ahead of the
 * gather, which then reads one 16-byte piece per sampled row instead of four 4-byte ones (each pulling a whole cache
 * line).  No counterpart in the reference (upstream indexes the four [T*N, 1] tensors separately,
 * rollout_storage.py:244-258).  Data moves bit-exactly. */
#define PPO_MAX_INTERLEAVE_FLOATS 16
int ppo_interleave_columns(const ppo_column_block* cols, int32_t num_cols, int64_t rows, float* dst,
                           int64_t dst_stride, ppo_stream_t stream);

/* The permutation itself, host code: torch.randperm(n) as drawn from torch's CPU generator
 * (rsl_rl/storage/rollout_storage.py:232), i.e. a Fisher-Yates shuffle of 0..n-1 with z_i = draw_i mod (n - i)
 * over the generator's 32-bit MT19937 stream.  generator_state: the record torch.get_rng_state() returns
 * (state_bytes = 5056), advanced in place by the n - 1 draws (write it back with torch.set_rng_state()).
 * out: int64 [n] host memory.  PPO_EINVAL when the record's layout is not recognised (nothing is written). */
int ppo_host_randperm(uint8_t* generator_state, size_t state_bytes, int64_t n, int64_t* out);
/* The same shuffle in consecutive pieces: iterations [i0, i1) (0 <= i0 <= i1 <= n - 1) of it, drawing i1 - i0
 * values from the generator record and advancing it; out holds the result of iterations [0, i0) (it is set to the
 * identity when i0 = 0).  Positions [0, i1) of out are final afterwards.  Running [0, s) then [s, n - 1) gives
 * exactly ppo_host_randperm's permutation and generator state. */
int ppo_host_randperm_range(uint8_t* generator_state, size_t state_bytes, int64_t n, int64_t i0, int64_t i1,
                            int64_t* out);
/* Advances the same generator record past `draws` 32-bit outputs without producing them, host code.  Upstream's
 * update draws and discards a Normal sample of the mini-batch's [rows, A] means in every mini-batch (the stochastic
 * forward, rsl_rl/models/mlp_model.py:103-106 via rsl_rl/algorithms/ppo.py:228-233); on the CPU generator a float
 * normal_ of n >= 16 contiguous elements takes n uniform draws plus 16 more when n % 16 != 0, so skipping those keeps
 * the next rollout's noise where upstream's CPU run draws it. */
int ppo_host_rng_skip(uint8_t* generator_state, size_t state_bytes, int64_t draws);

/* ------------------------------------------------------------------------------------------------------------------
 * A6  Linear layers of rsl_rl/modules/mlp.py:27-95 (nn.Linear + nn.ELU), forward and hand-written backward, as
 * fp32-accurate MFMA GEMMs: where every operand of a call has 16-byte aligned rows (and, forward / input-grad, k is a
 * multiple of 16) on the bf16 matrix cores, each fp32 operand split into three bf16 parts and each fp32 product taken
 * as six bf16 products accumulated in fp32 (error of the fp32 MFMA's order); otherwise on the fp32 MFMA.  One call
 * runs up to PPO_MAX_LINEAR_PROBLEMS independent problems (e.g. actor and critic; the recurrent update's ten weight
 * gradients) over the same number of rows in a single grouped launch.  Weights use torch's layout: w[out, in],
 * row-major.
 * ------------------------------------------------------------------------------------------------------------------ */
#define PPO_MAX_LINEAR_PROBLEMS 12

/* forward: z = x w^T + b; with an activation (PPO_ACT_ELU ... PPO_ACT_IDENTITY) also h = act(z).  Replaces
 * nn.Linear.forward and the activation module's forward (rsl_rl/modules/mlp.py:91-95).  With an activation either
 * output may be NULL (not both): a backward that takes act' from h (PPO_ELU_FROM_OUTPUT, monotone activations) needs
 * only h; the others need z.  With PPO_ACT_NONE z is required and h is ignored. */
typedef struct ppo_linear_fwd_problem {
  const float* x; int64_t ldx; /* [rows, in] */
  const float* w;              /* [out, in] */
  const float* b;              /* [out] */
  float* z; int64_t ldz;       /* [rows, out] */
  float* h; int64_t ldh;       /* [rows, out] or NULL */
  int32_t in_features;
  int32_t out_features;
} ppo_linear_fwd_problem;

int ppo_linear_fwd(const ppo_linear_fwd_problem* problems, int32_t count, int64_t rows, int32_t activation,
                   ppo_stream_t stream);

/* backward to the layer input: dz_prev = (dz w) * act'(z_prev), act' of ELU = 1 if z > 0 else exp(z)
 * (torch's elu_backward on the input).  z_prev == NULL means no activation (plain dx = dz w).  With
 * elu_source = PPO_ELU_FROM_OUTPUT, z_prev holds h = elu(z) instead and act' = 1 if h > 0 else h + 1 (the same
 * derivative, exp(z) = expm1(z) + 1, evaluated from the forward's output so z need not be stored).
 * The workspace (ppo_linear_bwd_dx_workspace_bytes, 16-byte aligned) receives w^T of every problem when the
 * weights cannot be read as stored (rows not 16-byte aligned); it is required either way.
 * Replaces autograd's mm backward + EluBackward (rsl_rl/algorithms/ppo.py:298). */
typedef struct ppo_linear_bwd_dx_problem {
  const float* dz; int64_t lddz;         /* [rows, out] */
  const float* w;                        /* [out, in] */
  const float* z_prev; int64_t ldz_prev; /* [rows, in] or NULL */
  float* dz_prev; int64_t lddz_prev;     /* [rows, in] */
  int32_t in_features;
  int32_t out_features;
} ppo_linear_bwd_dx_problem;

size_t ppo_linear_bwd_dx_workspace_bytes(const ppo_linear_bwd_dx_problem* problems, int32_t count);
int ppo_linear_bwd_dx(const ppo_linear_bwd_dx_problem* problems, int32_t count, int64_t rows, int32_t elu_source,
                      void* workspace, size_t workspace_bytes, ppo_stream_t stream);
/* the same for any hidden-layer activation: dz_prev = (dz w) * act'(z_prev), z_prev the activation's input, or its
 * output with source = PPO_ELU_FROM_OUTPUT (monotone activations only; PPO_EINVAL otherwise).  ppo_linear_bwd_dx is
 * this call with PPO_ACT_ELU.  Replaces autograd's mm backward + the activation's backward (torch's
 * elu_backward / threshold_backward / leaky_relu_backward / tanh_backward / sigmoid_backward / softplus_backward /
 * gelu_backward / silu_backward / mish_backward). */
int ppo_linear_bwd_dx_act(const ppo_linear_bwd_dx_problem* problems, int32_t count, int64_t rows, int32_t activation,
                          int32_t source, void* workspace, size_t workspace_bytes, ppo_stream_t stream);

/* backward to the parameters: dw = dz^T x, db = sum_rows dz, reduced over rows in fixed-order split-K partials
 * (deterministic: no float atomics).  Replaces autograd's AddmmBackward for weight and bias. */
typedef struct ppo_linear_bwd_dw_problem {
  const float* dz; int64_t lddz; /* [rows, out] */
  const float* x; int64_t ldx;   /* [rows, in] */
  float* dw;                     /* [out, in] */
  float* db;                     /* [out], or NULL: no bias gradient (the column sums are skipped) */
  int32_t in_features;
  int32_t out_features;
  int32_t grad_norm_group;       /* ppo_linear_bwd_dw_norm: 0 = not counted, g + 1 = dw and db count in group g */
  int32_t reserved;              /* 0 */
} ppo_linear_bwd_dw_problem;

size_t ppo_linear_bwd_dw_workspace_bytes(const ppo_linear_bwd_dw_problem* problems, int32_t count, int64_t rows);
int ppo_linear_bwd_dw(const ppo_linear_bwd_dw_problem* problems, int32_t count, int64_t rows, void* workspace,
                      size_t workspace_bytes, ppo_stream_t stream);

/* A contiguous range [begin, end) of a flat gradient buffer that belongs to parameter group `group`. */
typedef struct ppo_grad_range {
  int64_t begin, end;
  int32_t group, reserved;
} ppo_grad_range;

/* ppo_linear_bwd_dw that also returns the fp64 sums of squares of the gradients it writes, per parameter group
 * (problems with grad_norm_group g + 1), for ppo_adam_step_prenorm: PPO_DW_NORM_BLOCKS partial rows of
 * PPO_MAX_PARAM_GROUPS doubles (row-major, every row written) in norm_partials.  The `num_extra` (<= PPO_MAX_EXTRA_GRADS)
 * ranges of extra_grads -- gradients the launch does not produce but that belong to a group's norm, such as the
 * distribution's std parameter, written before this call -- are added to the same partial rows.  No counterpart in the
 * reference (upstream's clip_grad_norm_ reads the gradients once more); the Adam step that follows then needs no pass
 * over the gradients of its own. */
#define PPO_DW_NORM_BLOCKS 512
#define PPO_MAX_EXTRA_GRADS 4
int ppo_linear_bwd_dw_norm(const ppo_linear_bwd_dw_problem* problems, int32_t count, int64_t rows, void* workspace,
                           size_t workspace_bytes, const float* extra_grads, const ppo_grad_range* extra,
                           int32_t num_extra, double* norm_partials, ppo_stream_t stream);

/* The same three GEMMs with launch flags (all problems of a call share them):
 *   PPO_GEMM_BF16_OPERANDS  bf16 operands: every operand element rounded to bf16 (to nearest even), the products
 *       of those exact in fp32 accumulation, fp32 outputs and epilogues -- the matrix products of upstream's
 *       use_mixed_precision (rsl_rl/algorithms/ppo.py:222-224: torch.autocast to bfloat16 over the forward and the
 *       loss, so their backward too), on the bf16 matrix cores at one product per k-group instead of bf16x6's six.
 *       Operands the bf16 kernels do not take (rows that are not 16-byte multiples, k not a multiple of 16) run on
 *       the fp32 kernels, i.e. at higher precision.  The bias gradient's column sums stay fp64 over the fp32 values.
 * flags = 0 is the plain entry point.  ppo_linear_bwd_dw_ex: norm_partials NULL (and no extra ranges) is
 * ppo_linear_bwd_dw, else ppo_linear_bwd_dw_norm. */
#define PPO_GEMM_BF16_OPERANDS 1
int ppo_linear_fwd_ex(const ppo_linear_fwd_problem* problems, int32_t count, int64_t rows, int32_t activation,
                      int32_t flags, ppo_stream_t stream);
int ppo_linear_bwd_dx_ex(const ppo_linear_bwd_dx_problem* problems, int32_t count, int64_t rows, int32_t activation,
                         int32_t source, int32_t flags, void* workspace, size_t workspace_bytes, ppo_stream_t stream);
int ppo_linear_bwd_dw_ex(const ppo_linear_bwd_dw_problem* problems, int32_t count, int64_t rows, int32_t flags,
                         void* workspace, size_t workspace_bytes, const float* extra_grads,
                         const ppo_grad_range* extra, int32_t num_extra, double* norm_partials, ppo_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------------
 * A7  Empirical observation normaliser, rsl_rl/modules/normalization.py:46-78.
 * ppo_obs_normalize: y = (x - mean) / (std + eps) over [rows, width] (forward, :46-48).
 * ppo_normalizer_update: batch moments of the concatenation of `num_segments` column blocks over `rows` rows
 * (fp64, two-pass: mean then biased variance), then the running update of (_mean, _var, _std, count) in upstream's
 * fp32 operation order (:58-78, single process).  state_mean/var/std: [dim]; count: one int64.
 * ------------------------------------------------------------------------------------------------------------------ */
int ppo_obs_normalize(const float* x, int64_t ldx, float* y, int64_t ldy, int64_t rows, int32_t width,
                      const float* mean, const float* std, float eps, ppo_stream_t stream);

size_t ppo_normalizer_update_workspace_bytes(int64_t rows, int32_t dim);
int ppo_normalizer_update(const ppo_column_block* blocks, int32_t num_blocks, int64_t rows, float* state_mean,
                          float* state_var, float* state_std, int64_t* count, void* workspace,
                          size_t workspace_bytes, ppo_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------------
 * A8-A11  Gaussian policy head + PPO losses, forward and backward, rsl_rl/algorithms/ppo.py:226-285 with
 * rsl_rl/modules/distribution.py:183-238 (state-independent std).  Per row r of a mini-batch of R rows:
 *   std = clamp(std_param) (scalar) or exp(clamp(log_std_param)) (log);
 *   logp = sum_a [-(a-mu)^2/(2 std^2) - log std - log sqrt(2 pi)];  ratio = exp(logp - old_logp);
 *   L_pi = mean_r max(-adv ratio, -adv clamp(ratio, 1-clip, 1+clip));
 *   L_v = mean_r max((V-R)^2, (V_old + clamp(V-V_old, -clip, clip) - R)^2)  (or mean (R-V)^2 unclipped);
 *   entropy_r = sum_a [0.5 + 0.5 log(2 pi) + log std];  loss = L_pi + c_v L_v - c_e mean(entropy);
 *   kl_r = sum_a 0.5 ((var_ratio + t1) - 1 - log var_ratio)  (torch's Normal/Normal KL, ppo.py:243).
 * Backward follows torch autograd: max() splits ties 50/50, clamp() passes the gradient on the closed interval.
 * Outputs d_mean [R, A] = dloss/dmu and d_value [R] = dloss/dV, plus per-block partial sums in `workspace`
 * (surrogate, value loss, kl, and the per-action std-parameter gradient) reduced by ppo_loss_finalize.
 * ------------------------------------------------------------------------------------------------------------------ */
typedef struct ppo_loss_args {
  int64_t rows;
  int32_t num_actions;
  int32_t std_type;         /* PPO_STD_SCALAR or PPO_STD_LOG */
  const float* mean;        /* [rows, ld_mean] new actor output */
  int64_t ld_mean;
  const float* value;       /* [rows] at stride ld_value: new critic output */
  int64_t ld_value;
  const float* actions;     /* [rows, A] at row stride ld_batch */
  const float* old_mean;    /* [rows, A] at row stride ld_batch */
  const float* old_std;     /* [rows, A] at row stride ld_batch */
  const float* old_logp;    /* [rows] at stride ld_batch */
  const float* advantages;  /* [rows] at stride ld_batch */
  const float* old_values;  /* [rows] at stride ld_batch */
  const float* returns;     /* [rows] at stride ld_batch */
  int64_t ld_batch;
  const float* std_param;   /* [A] the distribution parameter (std_param or log_std_param) */
  double std_lo, std_hi;    /* clamp range in the parameter's own space (log-space bounds for PPO_STD_LOG) */
  double clip_param;        /* ratio clamp [(float)(1-clip), (float)(1+clip)], value clamp +-(float)clip */
  double value_loss_coef;   /* used as fp32, like torch's Python-scalar multiply */
  double entropy_coef;
  int32_t use_clipped_value_loss;
  int32_t reserved;
  float* d_mean;            /* [rows, ld_dmean] */
  int64_t ld_dmean;
  float* d_value;           /* [rows] at stride ld_dvalue */
  int64_t ld_dvalue;
} ppo_loss_args;

#define PPO_MAX_ACTIONS 64

size_t ppo_loss_workspace_bytes(int64_t rows, int32_t num_actions);
int ppo_gauss_ppo_loss(const ppo_loss_args* args, void* workspace, size_t workspace_bytes, ppo_stream_t stream);

/* Device-resident optimisation state shared by ppo_loss_finalize and ppo_adam_step (fp64 like upstream's Python
 * floats).  The host reads it back once per update. */
typedef struct ppo_device_state {
  double learning_rate;       /* upstream PPO.learning_rate (ppo.py:120, :253-256) */
  double sum_value_loss;      /* sum over mini-batches of value_loss.item()        (ppo.py:317) */
  double sum_surrogate_loss;  /*                         surrogate_loss.item()     (ppo.py:318) */
  double sum_entropy;         /*                         entropy.mean().item()     (ppo.py:319) */
  float last_kl_mean;
  float last_value_loss;
  float last_surrogate_loss;
  float last_entropy;
  float total_norm[4];        /* per parameter group, last step (clip_grad_norm_'s total_norm) */
  float clip_coef[4];         /* per parameter group, last step */
  int32_t num_minibatches;    /* mini-batches finalised since the state was reset */
  int32_t reserved[3];
} ppo_device_state;

/* Reduces the loss partials of the last ppo_gauss_ppo_loss call (same rows / num_actions / workspace), writes the
 * fp32 losses, applies the adaptive-KL learning-rate rule of ppo.py:240-266 when adaptive != 0
 * (kl > 2 desired -> lr = max(1e-5, lr/1.5); 0 < kl < desired/2 -> lr = min(1e-2, lr*1.5); fp32 comparisons),
 * accumulates the loss sums, and writes the std-parameter gradient d_std_param [A] (entropy term and clamp mask
 * included).  trace, if not NULL, is a buffer of trace_rows rows of 5 doubles: row state->num_minibatches receives
 * {kl_mean, lr, surrogate, value, entropy} while that index is below trace_rows (later mini-batches are not
 * traced). */
int ppo_loss_finalize(const ppo_loss_args* args, const void* workspace, size_t workspace_bytes, float* d_std_param,
                      ppo_device_state* state, int32_t adaptive, double desired_kl, double* trace,
                      int32_t trace_rows, ppo_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------------
 * The output layers fused with the loss: one call does what the actor's and critic's output-layer forward
 * (rsl_rl/modules/mlp.py's last nn.Linear: mean = h_a W_a^T + b_a, value = h_c w_c^T + b_c), ppo_gauss_ppo_loss,
 * ppo_loss_finalize and the output layers' input-grad with ELU' of the layer below (the first step of
 * loss.backward() past the loss, ppo.py:297) do, for the update's MLP heads.  It reads args' batch columns and
 * writes d_mean / d_value (for the output layers' weight-grad) exactly like ppo_gauss_ppo_loss, and the loss state,
 * learning rate, trace (trace_rows as there) and d_std_param exactly like ppo_loss_finalize; args->mean / args->value are not read (the
 * head computes them and stores them to head->mean / head->value when those are not NULL).  The hidden layers'
 * gradients dz_actor / dz_critic are dloss/dz of the last hidden layers, ELU' taken from their outputs
 * (h > 0 ? 1 : h + 1).  Supported when ppo_gauss_ppo_head_supported() (num_actions <= 32, k_actor and k_critic
 * multiples of 16, both <= 128); every row pointer of h_*, dz_*, mean, d_mean, actions, old_mean and old_std
 * 16-byte aligned (aligned bases, leading dimensions multiples of 4), w_actor contiguous and 16-byte aligned.  The
 * A-wide runs of actions / old_mean / old_std are read as whole 16-byte chunks (up to 3 floats past column A-1 of a
 * row, inside the chunk that holds its last column).
 * ------------------------------------------------------------------------------------------------------------------ */
typedef struct ppo_policy_head {
  const float* h_actor;   /* [rows, k_actor] at row stride ld_h_actor: the actor's last hidden ELU output */
  int64_t ld_h_actor;
  const float* w_actor;   /* [num_actions, k_actor] row-major (nn.Linear weight) */
  const float* b_actor;   /* [num_actions] */
  const float* h_critic;  /* [rows, k_critic] at row stride ld_h_critic */
  int64_t ld_h_critic;
  const float* w_critic;  /* [1, k_critic] */
  const float* b_critic;  /* [1] */
  float* dz_actor;        /* out [rows, k_actor] at ld_dz_actor */
  int64_t ld_dz_actor;
  float* dz_critic;       /* out [rows, k_critic] at ld_dz_critic */
  int64_t ld_dz_critic;
  float* mean;            /* out, optional: [rows, num_actions] at ld_mean */
  int64_t ld_mean;
  float* value;           /* out, optional: [rows] at stride ld_value */
  int64_t ld_value;
  int32_t k_actor;
  int32_t k_critic;
} ppo_policy_head;

int ppo_gauss_ppo_head_supported(int32_t num_actions, int32_t k_actor, int32_t k_critic);
size_t ppo_head_workspace_bytes(int64_t rows, int32_t num_actions);
int ppo_gauss_ppo_head(const ppo_loss_args* args, const ppo_policy_head* head, void* workspace,
                       size_t workspace_bytes, float* d_std_param, ppo_device_state* state, int32_t adaptive,
                       double desired_kl, double* trace, int32_t trace_rows, ppo_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------------
 * Rollout-side Gaussian head for act() (rsl_rl/algorithms/ppo.py:124-135; rsl_rl/modules/distribution.py:183-232):
 * std = clamp(std_param) or exp(clamp(log_std_param)); with noise != NULL, actions = noise * std + mean
 * (torch.normal(mean, std) on a standard-normal draw); with noise == NULL the given actions are scored.
 * logp [rows] (optional) = sum_a log N(actions; mean, std); std_out [rows, A] (optional) = std per row, the
 * distribution_params[1] the rollout storage keeps.
 * ------------------------------------------------------------------------------------------------------------------ */
int ppo_gauss_sample(const float* mean, int64_t ld_mean, const float* std_param, int32_t std_type, double std_lo,
                     double std_hi, const float* noise, int64_t ld_noise, float* actions, int64_t ld_actions,
                     float* logp, float* std_out, int64_t ld_std, int64_t rows, int32_t num_actions,
                     ppo_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------------
 * A12+A13  Per-group gradient-norm clipping (torch.nn.utils.clip_grad_norm_, called per model at ppo.py:309-310)
 * fused with Adam (torch.optim.Adam single-tensor path, ppo.py:311) over ONE flat fp32 buffer per kind.
 * Groups are contiguous ranges [group_begin[g], group_begin[g+1]) of the flat buffers.
 *   total_g = ||grad[group g]||_2 (fp64);  coef_g = min(1, max_norm / (total_g + 1e-6));  g' = grad * coef_g;
 *   m = m + (1-b1) (g' - m);  v = v b2 + ((1-b2) g') g';  denom = sqrt(v) / bc2_sqrt + eps;
 *   p = p + ((-lr/bc1) m) / denom,   lr read from state->learning_rate,
 * bc1 = 1 - b1^step and bc2_sqrt = (1 - b2^step)^0.5 computed by the caller in double exactly as torch does.
 * grad is rewritten with the clipped values (upstream clips in place).
 * ------------------------------------------------------------------------------------------------------------------ */
#define PPO_MAX_PARAM_GROUPS 4

size_t ppo_adam_workspace_bytes(int64_t num_params);
int ppo_adam_step(float* params, float* grads, float* exp_avg, float* exp_avg_sq, const int64_t* group_begin,
                  int32_t num_groups, double max_grad_norm, double beta1, double beta2, double eps, double bc1,
                  double bc2_sqrt, ppo_device_state* state, void* workspace, size_t workspace_bytes,
                  ppo_stream_t stream);

/* ppo_adam_step with the group norms from ppo_linear_bwd_dw_norm's partial rows instead of a pass over the gradients
 * (one launch): total_g^2 = the sum of norm_partials[row][g] over the PPO_DW_NORM_BLOCKS rows in row order.  The
 * caller guarantees that the partials cover every gradient of every group exactly once (the weight-grad problems plus
 * the extra ranges); the update itself is ppo_adam_step's. */
int ppo_adam_step_prenorm(float* params, float* grads, float* exp_avg, float* exp_avg_sq, const int64_t* group_begin,
                          int32_t num_groups, double max_grad_norm, double beta1, double beta2, double eps,
                          double bc1, double bc2_sqrt, ppo_device_state* state, const double* norm_partials,
                          ppo_stream_t stream);

/* A parameter written a second time, into a buffer with another row stride, by the Adam step that updates it: the
 * rows x cols floats at params[begin] (row-major, row stride cols) also go to dst[r * ld_dst + c] (ld_dst >= cols;
 * columns past cols are not touched).  For a first layer whose input width is not a multiple of 16, the forward GEMM
 * reads a zero-padded copy of the weight with 16-float-aligned rows; written by the optimiser step itself, that copy
 * needs no launch of its own before each mini-batch. */
typedef struct ppo_param_mirror {
  int64_t begin;
  int32_t rows;
  int32_t cols;
  float* dst;
  int64_t ld_dst;
} ppo_param_mirror;
#define PPO_MAX_PARAM_MIRRORS 2

/* ppo_adam_step_prenorm that also writes up to PPO_MAX_PARAM_MIRRORS mirrored parameters (the updated values, bit
 * for bit).  No counterpart in the reference (upstream's parameters have one layout); the mirrors' ranges must not
 * overlap. */
int ppo_adam_step_prenorm_mirror(float* params, float* grads, float* exp_avg, float* exp_avg_sq,
                                 const int64_t* group_begin, int32_t num_groups, double max_grad_norm, double beta1,
                                 double beta2, double eps, double bc1, double bc2_sqrt, ppo_device_state* state,
                                 const double* norm_partials, const ppo_param_mirror* mirrors, int32_t num_mirrors,
                                 ppo_stream_t stream);

/* ppo_adam_step without a workspace argument: it allocates nothing and takes no caller memory besides its inputs and
 * outputs.  No counterpart in the reference (upstream's torch.optim.Adam allocates as it likes); it is for callers that
 * cannot allocate device memory -- code under HIP graph capture, tight training / serving loops, harnesses that
 * forbid hipMalloc.  Same kernels and results as ppo_adam_step, with the per-chunk norm partials in a static device
 * array of PPO_ADAM_STATIC_SCRATCH_DOUBLES doubles (64 KiB, one copy per GPU, held until the process ends), which
 * bounds the flat buffers to PPO_ADAM_STATIC_MAX_PARAMS floats: larger counts return PPO_EINVAL before any HIP call.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (concurrent streams or threads) race
 * and must be serialised by the caller.  Nothing in the array needs clearing between calls. */
#define PPO_ADAM_STATIC_SCRATCH_DOUBLES 8192
#define PPO_ADAM_STATIC_MAX_PARAMS ((int64_t)(PPO_ADAM_STATIC_SCRATCH_DOUBLES - PPO_MAX_PARAM_GROUPS) * 1024)
int ppo_adam_step_static(float* params, float* grads, float* exp_avg, float* exp_avg_sq, const int64_t* group_begin,
                         int32_t num_groups, double max_grad_norm, double beta1, double beta2, double eps, double bc1,
                         double bc2_sqrt, ppo_device_state* state, ppo_stream_t stream);

/* The optimisers upstream resolves by name (rsl_rl/utils/utils.py:71-96, constructed at rsl_rl/algorithms/ppo.py:99-102
 * with the learning rate only, so every other hyperparameter is torch's default), each with the same per-group clip
 * and in torch's single-tensor fp32 order:
 *   PPO_OPTIM_ADAM     ppo_adam_step's update (state0 = exp_avg, state1 = exp_avg_sq);
 *   PPO_OPTIM_ADAMW    p = p * fl(1 - lr * weight_decay), then Adam's update (torch.optim.AdamW, weight_decay 1e-2);
 *   PPO_OPTIM_SGD      p = p + g' * (-lr) as one fused multiply-add (torch.optim.SGD without momentum; no state);
 *   PPO_OPTIM_RMSPROP  sq = sq * alpha + ((1 - alpha) g') g';  p = p + ((-lr) g') / (sqrt(sq) + eps)
 *                      (torch.optim.RMSprop, alpha 0.99, eps 1e-8, no momentum, not centred; state0 = square_avg).
 * norm_partials != NULL: the group norms from ppo_linear_bwd_dw_norm's partial rows (as ppo_adam_step_prenorm, one
 * launch); else from a pass over the gradients into workspace (ppo_adam_workspace_bytes).  Up to
 * PPO_MAX_PARAM_MIRRORS mirrored parameters either way.  bc1 / bc2_sqrt: Adam and AdamW only (ignored otherwise). */
#define PPO_OPTIM_ADAM 0
#define PPO_OPTIM_ADAMW 1
#define PPO_OPTIM_SGD 2
#define PPO_OPTIM_RMSPROP 3
typedef struct ppo_optim_config {
  int32_t kind;        /* PPO_OPTIM_* */
  int32_t reserved;
  double beta1, beta2; /* Adam / AdamW */
  double eps;          /* Adam / AdamW / RMSprop */
  double weight_decay; /* AdamW */
  double alpha;        /* RMSprop */
} ppo_optim_config;
int ppo_optim_step(float* params, float* grads, float* state0, float* state1, const int64_t* group_begin,
                   int32_t num_groups, double max_grad_norm, const ppo_optim_config* config, double bc1,
                   double bc2_sqrt, ppo_device_state* state, const double* norm_partials, void* workspace,
                   size_t workspace_bytes, const ppo_param_mirror* mirrors, int32_t num_mirrors, ppo_stream_t stream);

/* ------------------------------------------------------------------------------------------------------------------
 * A15  LSTM / GRU of the recurrent models (torch nn.LSTM: gates i, f, g, o; torch nn.GRU: gates r, z, n; one layer
 * per call, stacked layers call again on the h of the layer below): rsl_rl/modules/rnn.py:22-86,
 * rsl_rl/models/rnn_model.py:76-84, the recurrent mini-batches of rsl_rl/storage/rollout_storage.py:262-331 and the
 * trajectory padding of rsl_rl/utils/utils.py:395-463.
 *
 * Upstream splits every env's steps into trajectories at the dones, pads them, runs the LSTM over each from the
 * state the rollout saved at its first step, and unpads.  A trajectory after a done starts from the zero state the
 * rollout saved after resetting, so the same outputs come from one sequence per env over the mini-batch's T steps,
 * from the state saved at step 0, with the state multiplied by keep_t = 1 - done_t after step t.  That is the form
 * evaluated here: rows are t * E + e (step-major), the envs of a mini-batch being E consecutive envs.
 *
 * Gate-interleaved layout ("_g"): row (or column) 4u + q holds slot q of hidden unit u, so that one 16-byte group
 * holds the four slots of a unit.  LSTM: slot q = gate q (i, f, g, o).  GRU: slots r, z, the hidden part of n
 * (W_hn h + b_hn) and the input part of n (W_in x + b_in); w_ih_g is zero in slot 2 and w_hh_g in slot 3, so the
 * input projection and the recurrent product are the LSTM's, and the cell n = tanh(slot 3 + r * slot 2),
 * h' = n + z (h - n) (torch's order) reads them apart.  The GRU's state h takes the place of the LSTM's cell state c
 * in every buffer (c0 = h0, c = h).  H must be a multiple of 4; every pointer 16-byte aligned and every leading
 * dimension a multiple of 4.
 * ------------------------------------------------------------------------------------------------------------------ */
#define PPO_MAX_LSTM_PROBLEMS 2
#define PPO_CELL_LSTM 0
#define PPO_CELL_GRU 1

/* torch-layout weights -> gate-interleaved copies: w_ih_g [4H, D], w_hh_g [4H, H], w_hh_gt = w_hh_g^T [H, 4H],
 * b_g = b_ih + b_hh [4H] (the gates' bias, nn.LSTM adds both). */
typedef struct ppo_lstm_pack_problem {
  const float* w_ih; const float* w_hh; const float* b_ih; const float* b_hh; /* [4H, D], [4H, H], [4H], [4H] */
  float* w_ih_g; float* w_hh_g; float* w_hh_gt; float* b_g;
  int32_t input_size;
  int32_t hidden;
} ppo_lstm_pack_problem;

int ppo_lstm_pack(const ppo_lstm_pack_problem* problems, int32_t count, ppo_stream_t stream);
/* The same for torch nn.GRU weights ([3H, D], [3H, H], [3H], [3H]; gates r, z, n) into the four-slot layout:
 * b_g = (b_ir + b_hr, b_iz + b_hz, b_hn, b_in) per unit. */
int ppo_gru_pack(const ppo_lstm_pack_problem* problems, int32_t count, ppo_stream_t stream);

/* One model's sequence over T steps x E envs.  The forward consumes gx = x w_ih_g^T + b_g for every row (from
 * ppo_linear_fwd) and writes, per step, the gate activations, the cell and hidden states, and hs (the state entering
 * each step: hs[0] = h0, hs[t+1] = h_t * keep_t), which the weight-gradient of w_hh reads as [T*E, H] (its first
 * T*E rows).  The backward runs t = T-1 .. 0: dL/dh_t = dh[t] + keep_t * (dgates[t+1] w_hh_g) and the carried cell
 * gradient give dgates[t] (pre-activation gate gradients, the operand of both weight-gradients and of the bias
 * gradient); dc is scratch (no initialisation needed). */
typedef struct ppo_lstm_seq_problem {
  const float* w_hh_g;                       /* [4H, H] */
  const float* w_hh_gt;                      /* [H, 4H] (backward) */
  const float* gx; int64_t ldgx;             /* [T*E, 4H] */
  const float* h0; const float* c0; int64_t ld0; /* [E, H] state entering step 0 */
  const float* keep; int64_t keep_stride;    /* 1 - done per row t*E + e, elements keep_stride floats apart */
  float* h; int64_t ldh;                     /* [T*E, H] h_t (before the reset) */
  float* hs;                                 /* [(T+1)*E, H], ld H */
  float* c;                                  /* [T*E, H] c_t (before the reset), ld H */
  float* gates;                              /* [T*E, 4H] activations, ld 4H */
  const float* dh; int64_t lddh;             /* backward: [T*E, H] dL/dh_t from the layers above */
  float* dgates;                             /* backward: [T*E, 4H], ld 4H */
  float* dc;                                 /* backward: [E, H] scratch, ld H */
  int32_t hidden;
  int32_t cell;                              /* PPO_CELL_LSTM or PPO_CELL_GRU; one value for all problems of a call */
} ppo_lstm_seq_problem;

/* Synchronisation buffer of the whole-sequence launches: int32 words for `count` problems of `envs` rows (-1 for an
 * invalid count or envs).  Word 0 is a sticky status: the library sets it non-zero when the blocks of a
 * whole-sequence launch stopped waiting for each other (after about 2 s; the outputs of that call are then invalid).
 * The caller zeroes the buffer once and reads word 0 whenever it checks for errors; a call that completes leaves the
 * other words at zero for the next one (and a forward call clears them before it starts).  After word 0 was found
 * non-zero the caller zeroes the whole buffer again: a backward call on the words a failed call left returns at
 * once with invalid outputs (word 0 stays set).  Calls that share a buffer must not overlap. */
int64_t ppo_lstm_seq_sync_words(int32_t count, int64_t envs);

/* sync = NULL: one launch per step.  sync != NULL (sync_words >= ppo_lstm_seq_sync_words(count, envs)): all steps
 * run in one launch when H is a multiple of 32 up to 256 and the device holds one row group's blocks at once, else
 * one launch per step.  The forward gives identical results either way; the backward's recurrent product sums in
 * another order (agreement to fp32 rounding). */
int ppo_lstm_seq_fwd(const ppo_lstm_seq_problem* problems, int32_t count, int64_t steps, int64_t envs,
                     int32_t* sync, int64_t sync_words, ppo_stream_t stream);
int ppo_lstm_seq_bwd(const ppo_lstm_seq_problem* problems, int32_t count, int64_t steps, int64_t envs,
                     int32_t* sync, int64_t sync_words, ppo_stream_t stream);

/* The layer's input projection for ppo_lstm_seq_fwd_proj: gx = x w_ih_g^T + b_g over all T*E rows (the
 * nn.LSTM / nn.GRU input products of rsl_rl/modules/rnn.py:35-52 in the gate-interleaved layout). */
typedef struct ppo_lstm_input_projection {
  const float* x; int64_t ldx;               /* [T*E, input_size] the layer's input, row t*E + e */
  const float* w_ih_g;                       /* [4H, input_size] gate-interleaved (ppo_lstm_pack / ppo_gru_pack) */
  const float* b_g;                          /* [4H] */
  int32_t input_size;
  int32_t reserved;
} ppo_lstm_input_projection;

/* ppo_lstm_seq_fwd with the input projection done by the call itself: gx is computed as ppo_linear_fwd_ex(x, w_ih_g,
 * b_g, no activation, flags) would compute it (flags: 0 or PPO_GEMM_BF16_OPERANDS), bit for bit.  For inputs of up to
 * 48 columns (a multiple of 16) with 16-byte rows, in a one-launch sequence, it runs inside that launch (each step's
 * products in the time its blocks wait for each other) and gx is left unwritten; otherwise as its own launch into gx
 * before the steps.  The problems' gx is scratch: its contents afterwards are unspecified. */
int ppo_lstm_seq_fwd_proj(const ppo_lstm_seq_problem* problems, const ppo_lstm_input_projection* proj, int32_t count,
                          int64_t steps, int64_t envs, int32_t flags, int32_t* sync, int64_t sync_words,
                          ppo_stream_t stream);

/* How long the blocks of a whole-sequence launch wait for each other before they give up and set the status word,
 * in ticks of the 100 MHz device clock, for every later launch of this process: ticks >= 0 sets that limit, ticks < 0
 * restores the default (200,000,000 = 2 s).  Returns the limit in force before the call.  A test hook (0 forces the
 * give-up path from the host; every kernel still runs to its end); no environment variable changes the limit.
 * No counterpart in the reference (nn.LSTM has no cross-block waits). */
int64_t ppo_lstm_seq_wait_limit(int64_t ticks);

/* gate-interleaved gradients -> torch-layout gradients (the bias gradient goes to both b_ih and b_hh). */
typedef struct ppo_lstm_grad_problem {
  const float* dw_ih_g; const float* dw_hh_g; const float* db_g;
  float* dw_ih; float* dw_hh; float* db_ih; float* db_hh;
  int32_t input_size;
  int32_t hidden;
} ppo_lstm_grad_problem;

int ppo_lstm_unpack_grads(const ppo_lstm_grad_problem* problems, int32_t count, ppo_stream_t stream);
/* The same into torch nn.GRU's layout ([3H, D], [3H, H], [3H], [3H]): the r and z bias gradients go to both biases,
 * slot 2's to b_hn and slot 3's to b_in. */
int ppo_gru_unpack_grads(const ppo_lstm_grad_problem* problems, int32_t count, ppo_stream_t stream);

/* ppo_lstm_unpack_grads / ppo_gru_unpack_grads that also add the fp64 sums of squares of the torch-layout gradients
 * they write to the norm_partials of the ppo_linear_bwd_dw_norm call before them on the same stream (problem i's to
 * group groups[i], 0 .. PPO_MAX_PARAM_GROUPS - 1; each partial row gets at most one addition per problem, in a fixed
 * order), so one ppo_adam_step_prenorm covers a recurrent model whose weight gradients the GEMM writes in the
 * gate-interleaved layout.  No counterpart in the reference (upstream's clip_grad_norm_ reads the gradients once
 * more). */
int ppo_lstm_unpack_grads_norm(const ppo_lstm_grad_problem* problems, const int32_t* groups, int32_t count,
                               double* norm_partials, ppo_stream_t stream);
int ppo_gru_unpack_grads_norm(const ppo_lstm_grad_problem* problems, const int32_t* groups, int32_t count,
                              double* norm_partials, ppo_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PPO_HIP_H_ */
