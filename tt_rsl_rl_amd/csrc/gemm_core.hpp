// Core of the fp32 MFMA GEMMs for gfx950, shared by the linear layers (gemm.hip) and the LSTM (lstm.hip).
//
// Two kernel families, both 256 threads = 4 wavefronts in a 2 x 2 arrangement over a BM x BN output tile, each
// wave owning (BM/2) x (BN/2) of 32 x 32 v_mfma_f32_32x32x2f32 accumulators, both fed by gfx950's direct
// global->LDS loads (buffer_load_dwordx4 / _dword ... lds: no register staging, no ds_write) into an LDS ring of
// stages with one barrier per BK-deep k-slab:
//
//   NT  C[m,n] = sum_k A[m,k] B[n,k]        both operands k-contiguous in memory
//       forward     z[r,o]   = sum_i x[r,i]  w[o,i]    A = x,  B = w           epilogue +b (ELU)
//       input-grad  dzp[r,i] = sum_o dz[r,o] wt[i,o]   A = dz, B = w^T (copied) epilogue * ELU'(z_prev)
//   TN  C[m,n] = sum_k A[k,m] B[k,n]        both operands m/n-contiguous ("k-major")
//       weight-grad dw[o,i]  = sum_r dz[r,o] x[r,i]    split-K partials, fixed-order reduction, fp64 db
//
// NT tiles are stored row-per-m in LDS with BK floats per row and the 16-byte chunks of each row XOR-swizzled by
// the row index, so a ds_read_b128 of 16 consecutive rows is bank-conflict free.  The k order inside a slab is
// permuted so that one ds_read_b128 per operand and lane supplies four consecutive MFMA k-steps: at step s of
// group g, lane half h contributes k = 8g + 4h + s for both operands (any bijection of k works if A and B agree).
// TN tiles are stored k-major (row per k, BM or BN floats), and rows are interleaved across the two 32-wide MFMA
// tiles of a wave (tile i takes m = 2*rho + i) so one ds_read_b64 feeds both tiles and the partial stores are
// float2-wide.  Reads of rows past M or N are clamped into the operand (their results are discarded); the NT K
// tail is loaded through a masked path with zeros, the TN one by the buffer's record limit.  Several independent problems (actor and critic, or all layers of
// the weight-grad) share one launch: the block index maps to (problem, split, tile) through per-problem block
// offsets, after an XCD-aware permutation that places consecutive tiles (which share an A panel) on one XCD / L2.
#pragma once

#include <atomic>
#include <cstdlib>
#include <cstring>

#include "common.hpp"

namespace ppo {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

enum Epilogue : int {
  EPI_BIAS = 0,
  EPI_BIAS_ELU = 1,
  EPI_ELU_GRAD = 2,
  EPI_STORE = 3,
  EPI_PARTIAL = 4,
  EPI_LSTM_FWD = 5,  // one LSTM step: gates -> cell / hidden state (lstm.hip)
  EPI_LSTM_BWD = 6,  // one LSTM backward step: hidden-state gradient -> gate gradients (lstm.hip)
  EPI_BIAS_ACT = 7,  // EPI_BIAS_ELU for the other activations (Problem::act)
  EPI_ACT_GRAD = 8,  // EPI_ELU_GRAD for the other activations
};
// The forward epilogues that add the bias and apply an activation, and the input-grad epilogues that multiply by its
// derivative: ELU's own (the kernels every workload here runs, unchanged by the others' existence) and the generic
// ones, which evaluate Problem::act per element.
constexpr bool epi_fwd_act(int e) { return e == EPI_BIAS_ELU || e == EPI_BIAS_ACT; }
constexpr bool epi_act_grad(int e) { return e == EPI_ELU_GRAD || e == EPI_ACT_GRAD; }
constexpr bool epi_generic(int e) { return e == EPI_BIAS_ACT || e == EPI_ACT_GRAD; }


// Per-step operands of the LSTM epilogues.  Rows are envs; gate-interleaved columns (4u + q = gate q of unit u).
struct LstmArgs {
  const float* gx;         // fwd: [E, 4H] input projection + both biases of this step
  const float* c_prev;     // [E, H] cell state entering the step (before the done reset)
  const float* keep_prev;  // 1 - done of the previous step per row (NULL: no reset, the step-0 state)
  const float* keep;       // 1 - done of this step per row
  float* gates;            // fwd: written [E, 4H] activations (i, f, g, o); bwd: read
  float* c;                // fwd: written c_t [E, H]; bwd: read
  float* h;                // fwd: written h_t [E, H] (ld ldh)
  float* hs;               // fwd: written h_t * keep, the next step's A operand [E, H]
  const float* dh;         // bwd: dL/dh_t from the layers above [E, H] (ld lddh)
  float* dgates;           // bwd: written dL/d(pre-activation) [E, 4H]
  float* dc;               // bwd: [E, H] cell gradient carried to the previous step (read unless first)
  int64_t ldgx, ldcp, ldh, lddh, keep_stride;
  int32_t hidden, first, last;  // bwd: first = no carried cell gradient yet, last = do not write dc
  int32_t cell;                 // PPO_CELL_LSTM or PPO_CELL_GRU (see gru_cell_fwd for the GRU's use of the buffers)
};

struct Problem {
  const float* A;
  const float* B;
  float* C;
  float* C2;
  const float* vec;  // bias [N]
  const float* aux;  // ELU'-source z_prev [M, N]
  double* colsum;    // [splits, M] sums of A over each split's k range (fp64: bias grads cancel heavily)
  int64_t lda, ldb, ldc, ldc2, ldaux;
  int64_t partial_stride;  // floats between split partials of C
  int32_t M, N, K;
  int32_t tiles_m, tiles_n, splits, k_chunk;
  int32_t block_begin;
  int32_t c_vec;            // NT epilogue: C (and C2 / aux when used) allow 16-byte accesses
  int32_t elu_from_output;  // input-grad: aux holds h = act(z) (act' from the output), else z
  int32_t act;              // EPI_BIAS_ELU / EPI_ELU_GRAD: the hidden layers' activation (PPO_ACT_*)
  int32_t b16;              // NT: B allows 16-byte direct loads (set by launch_nt)
  int32_t tn64;             // TN bf16x6: 128 x 64 output tiles (problems at most 64 columns wide)
  LstmArgs lstm;            // EPI_LSTM_*
};

// Logistic function and tanh of the LSTM cell on the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, each about
// 1 ulp): sigma(x) = 1 / (1 + 2^(-x log2 e)), tanh(x) = 2 sigma(2x) - 1 (absolute error a few 1e-8).  Both saturate
// at the ends: 2^(+inf) = inf and 1 / inf = 0.
__device__ __forceinline__ float sigmoid_hw(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}
__device__ __forceinline__ float tanh_hw(float x) { return __builtin_fmaf(2.0f, sigmoid_hw(2.0f * x), -1.0f); }

// ELU (alpha 1) of the forward epilogue: x for x > 0, else expm1(x), from two published pieces: on [-0.7, 0] the
// Taylor series of expm1 to degree 9 (x + x^2 (1/2! + x/3! + ... + x^7/9!), truncation below 1e-8 relative), below
// -0.7 the hardware 2^(x log2 e) minus 1 (v_exp_f32; no cancellation there, the result is below -0.5).  Within 1.2 ulp
// of expm1 (1.7 with a 1-ulp exp2) at about a quarter of a library expm1f's instructions, which matters because
// every output element of a hidden layer goes through it while the MFMA pipes wait.
__device__ __forceinline__ float elu_fwd(float x) {
  float p = 1.0f / 362880.0f;           // 1/9!
  p = fmaf(p, x, 1.0f / 40320.0f);      // 1/8!
  p = fmaf(p, x, 1.0f / 5040.0f);
  p = fmaf(p, x, 1.0f / 720.0f);
  p = fmaf(p, x, 1.0f / 120.0f);
  p = fmaf(p, x, 1.0f / 24.0f);
  p = fmaf(p, x, 1.0f / 6.0f);
  p = fmaf(p, x, 0.5f);
  const float near0 = fmaf(x * x, p, x);
  const float far = __builtin_amdgcn_exp2f(x * 1.4426950408889634f) - 1.0f;
  return x > 0.0f ? x : (x > -0.7f ? near0 : far);
}

// The hidden-layer activations of rsl_rl's MLP (rsl_rl/utils/utils.py:34-68, torch's modules with their default
// arguments) and their derivatives, as torch's CPU kernels evaluate them: SELU = scale (x or alpha (e^x - 1)),
// LeakyReLU slope 0.01, CELU alpha 1 = ELU, Softplus beta 1 threshold 20, GELU on erf, SiLU x sigma(x),
// Mish x tanh(softplus(x)).  act_grad(src) is act'(z) from the layer's input z, or, where the derivative is a
// function of the output h (every monotone one), from h: ELU / CELU h + 1 (h <= 0), SELU h + alpha scale, tanh
// 1 - h^2, sigmoid (1 - h) h.  ELU itself keeps elu_fwd (the epilogues test for it first).
constexpr float kSeluAlpha = 1.6732632423543772f, kSeluScale = 1.0507009873554805f;
constexpr float kSeluAS = kSeluAlpha * kSeluScale;

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

// (called, not inlined: one copy of every activation's code instead of one per output element)
__device__ __attribute__((noinline)) float act_fwd(int act, float x) {
  switch (act) {
    case PPO_ACT_SELU: return x > 0.0f ? x * kSeluScale : (expf(x) - 1.0f) * kSeluAS;
    case PPO_ACT_RELU: return x > 0.0f ? x : 0.0f;
    case PPO_ACT_LRELU: return x > 0.0f ? x : x * 0.01f;
    case PPO_ACT_TANH: return tanhf(x);
    case PPO_ACT_SIGMOID: return sigmoid_ref(x);
    case PPO_ACT_SOFTPLUS: return x > 20.0f ? x : log1pf(expf(x));
    case PPO_ACT_GELU: return x * 0.5f * (1.0f + erff(x * 0.70710678118654752f));
    case PPO_ACT_SILU: return x / (1.0f + expf(-x));
    case PPO_ACT_MISH: return x * tanhf(log1pf(expf(x)));
    case PPO_ACT_IDENTITY: return x;
    default: return elu_fwd(x);  // PPO_ACT_ELU, PPO_ACT_CELU
  }
}

// act'(.) of `src`: the output h when from_output (monotone activations only: the host checks), else the input z.
__device__ __attribute__((noinline)) float act_grad(int act, float src, bool from_output) {
  switch (act) {
    case PPO_ACT_SELU:
      return src > 0.0f ? kSeluScale : (from_output ? src + kSeluAS : kSeluAS * expf(src));
    case PPO_ACT_RELU: return src > 0.0f ? 1.0f : 0.0f;
    case PPO_ACT_LRELU: return src > 0.0f ? 1.0f : 0.01f;
    case PPO_ACT_TANH: {
      const float t = from_output ? src : tanhf(src);
      return 1.0f - t * t;
    }
    case PPO_ACT_SIGMOID: {
      const float y = from_output ? src : sigmoid_ref(src);
      return (1.0f - y) * y;
    }
    case PPO_ACT_SOFTPLUS: {
      const float z = expf(src);
      return src > 20.0f ? 1.0f : z / (z + 1.0f);
    }
    case PPO_ACT_GELU: {
      const float cdf = 0.5f * (1.0f + erff(src * 0.70710678118654752f));
      const float pdf = expf(-0.5f * src * src) * 0.39894228040143268f;
      return cdf + src * pdf;
    }
    case PPO_ACT_SILU: {
      const float sg = sigmoid_ref(src);
      return sg * (1.0f + src * (1.0f - sg));
    }
    case PPO_ACT_MISH: {
      const float sg = sigmoid_ref(src);
      const float ts = tanhf(log1pf(expf(src)));
      return ts + src * sg * (1.0f - ts * ts);
    }
    case PPO_ACT_IDENTITY: return 1.0f;
    default: return src > 0.0f ? 1.0f : (from_output ? src + 1.0f : expf(src));  // ELU, CELU
  }
}

template <bool V>
struct BoolC {
  static constexpr bool value = V;
};
template <int V>
struct IntC {
  static constexpr int value = V;
};

// Four outputs of an epilogue: o2 = act(o).  GEN = false: ELU (every workload here); GEN = true: any activation,
// chosen per element by `act` (a call: with every activation's code inlined per group of four outputs, the forward
// kernels grew 7x and ran 10x slower, measured).
template <bool GEN>
__device__ __forceinline__ void act_fwd4(int act, const f32x4& o, f32x4& o2) {
#pragma unroll
  for (int e = 0; e < 4; ++e) o2[e] = GEN ? act_fwd(act, o[e]) : elu_fwd(o[e]);
}

// o = x * act'(src); ELU's exactly as before the other activations existed (x itself where act' = 1).
template <bool GEN>
__device__ __forceinline__ void act_grad4(int act, int from_output, const f32x4& x, const f32x4& src, f32x4& o) {
  if constexpr (!GEN) {
    if (from_output) {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = src[e] > 0.0f ? x[e] : x[e] * (src[e] + 1.0f);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = src[e] > 0.0f ? x[e] : x[e] * expf(src[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = x[e] * act_grad(act, src[e], from_output != 0);
  }
}


struct Group {
  Problem p[PPO_MAX_LINEAR_PROBLEMS];
  int32_t count;
  int32_t xcds;  // > 1: the device's XCDs; block ids are permuted so each XCD gets a contiguous range of tiles
};

constexpr int kThreads = 256;

// Blocks are dispatched round-robin over the X XCDs; renumber them so that each XCD receives a contiguous range of
// logical tiles (a bijection of [0, n)).
__device__ inline int xcd_remap(int b, int n, int X) {
  const int q = n / X, r = n % X;
  const int xcd = b % X, slot = b / X;
  return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

struct TileCoord {
  int pi, split, tm, tn;
};

__device__ inline TileCoord locate(const Group& g) {
  const int b = g.xcds > 1 ? xcd_remap(blockIdx.x, gridDim.x, g.xcds) : static_cast<int>(blockIdx.x);
  int pi = 0;
#pragma unroll
  for (int i = 1; i < PPO_MAX_LINEAR_PROBLEMS; ++i) {
    if (i < g.count && b >= g.p[i].block_begin) pi = i;
  }
  const Problem& P = g.p[pi];
  const int local = b - P.block_begin;
  const int tiles_mn = P.tiles_m * P.tiles_n;
  TileCoord t;
  t.pi = pi;
  t.split = local / tiles_mn;
  const int r = local - t.split * tiles_mn;
  t.tm = r / P.tiles_n;
  t.tn = r - t.tm * P.tiles_n;
  return t;
}

// Direct global->LDS copy through a raw buffer: every lane moves BYTES from byte offset `off` of buffer r to
// lds_wave + lane * BYTES (lds_wave wave-uniform), and an offset at or past the buffer's record count reads zeros.
// Unlike the flat-encoded global_load_lds, the compiler's wait-count pass does not treat it as a possible LDS access
// that may complete out of order, so the LDS reads issued while it is in flight keep exact (not zero) wait counts.
template <int BYTES>
__device__ __forceinline__ void dma_buf(__amdgpu_buffer_rsrc_t r, uint32_t off, float* lds_wave) {
  static_assert(BYTES == 16 || BYTES == 4, "16- or 4-byte direct loads");
  auto* dst = (__attribute__((address_space(3))) void*)lds_wave;
  if constexpr (BYTES == 16) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, off, 0, 0, 0);
  } else {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 4, off, 0, 0, 0);
  }
}

// Raw buffer of `bytes` bytes at `base` (both wave-uniform), built from scalar registers: the compiler otherwise
// may compute the descriptor in vector registers and wrap every load that uses it in a per-lane loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_buffer(const float* base, int bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  float* const p = reinterpret_cast<float*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8; a field at its maximum
// does not wait).  The waits and the barrier are the compiler's builtins, not inline assembly: after an opaque asm
// statement the compiler's wait-count pass must assume unknown LDS / scalar-memory events are in flight, and every
// later LDS read it waits for becomes "lgkmcnt(0)" (measured: one full LDS round trip before each MFMA group).
// The builtins carry no memory ordering of their own, so compiler-only fences on both sides keep every memory
// access of the source on its side of the wait.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kWaitLgkm0 = 15 | (3 << 14) | (7 << 4);

// Waits until at most N of this wave's vector-memory operations are outstanding.  The LDS-direct loads count here
// (the compiler does not track them as LDS writes).  Loads complete in issue order.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0, "vmcnt");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(N < 63 ? N : 63));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Workgroup barrier of the LDS ring: this wave's LDS accesses are complete and the compiler moves no memory access
// across it.  Unlike __syncthreads(), whose workgroup release fence also drains every outstanding global load, it
// leaves the prefetched slabs in flight; their arrival is awaited explicitly with wait_slab().
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Ring of S LDS stages with prefetch distance S - 1: before computing slab kt a wave waits for its own loads of
// slab kt while the `later` (<= S - 2) slabs issued after it may stay in flight; L = loads per wave per slab.
// A cap of 63 outstanding only makes the wait stricter (loads retire in order).
template <int L, int S>
__device__ __forceinline__ void wait_slab(int later) {
  if constexpr (S >= 4) {
    if (later >= 2) {
      wait_vmcnt<2 * L>();
      return;
    }
  }
  if constexpr (S >= 3) {
    if (later >= 1) {
      wait_vmcnt<L>();
      return;
    }
  }
  wait_vmcnt<0>();
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ------------------------------------------------------------------------------------------------------------------
// NT: operands stored [x][k] (k contiguous); LDS tile [BX][BK] with swizzled 16-byte chunks.
// ------------------------------------------------------------------------------------------------------------------

// Physical chunk of logical chunk c in LDS row `row` is c ^ swz(row).  gfx950's LDS serves a ds_read_b128 16 lanes
// (16 x 16 bytes = all 64 banks) at a time; those lanes read one logical chunk of 16 consecutive rows, which the
// swizzle spreads over 16 distinct 16-byte bank groups (rows sharing a 256-byte window get different chunks).
template <int BK>
__device__ __forceinline__ int nt_swz(int row) {
  constexpr int CPR = BK / 4;
  static_assert(CPR == 4 || CPR == 8 || CPR == 16, "BK must be 16, 32 or 64");
  return CPR == 16 ? (row & 15) : CPR == 8 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}

// Direct loads of one NT operand: one full k-slab [x0, x0 + BX) x [k0, k0 + BK) per call, rows >= X clamped to X - 1.
// Each lane's byte offsets from the slab's first column are fixed for the whole k loop, so a slab costs one
// uniform (scalar) base pointer and one buffer_load ... lds per instruction.  Wave w issues instructions w, w+4, ...
template <int BX, int BK, bool W16>
struct NtLoader {
  static constexpr int CPR = BK / 4;
  static constexpr int NQ = W16 ? BX * BK / 256 : BX * BK / 64;
  static constexpr int PER = NQ / 4;
  static_assert(NQ % 4 == 0, "every wave must issue the same number of loads per slab");
  uint32_t off[PER];

  __device__ __forceinline__ void init(int64_t ld, int x0, int X, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int q = 4 * j + wave;
      int row, col;
      if constexpr (W16) {
        row = q * (64 / CPR) + lane / CPR;
        col = 4 * ((lane % CPR) ^ nt_swz<BK>(row));
      } else {
        row = q * (64 / BK) + lane / BK;
        const int f = lane % BK;
        col = 4 * ((f >> 2) ^ nt_swz<BK>(row)) + (f & 3);
      }
      const int64_t gx = min(x0 + row, X - 1);
      off[j] = static_cast<uint32_t>((gx * ld + col) * 4);
    }
  }
  // base: the operand's element (0, k0), wave-uniform.  The offsets stay under 4 GiB (the host rejects operands that
  // span more), so the buffer needs no bound of its own.
  __device__ __forceinline__ void issue(const float* base, float* lds_op, int wave) const {
    const __amdgpu_buffer_rsrc_t r = uniform_buffer(base, -1);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if constexpr (W16) {
        dma_buf<16>(r, off[j], lds_op + (4 * j + wave) * 256);
      } else {
        dma_buf<4>(r, off[j], lds_op + (4 * j + wave) * 64);
      }
    }
  }
};

// The partial last k-slab of an NT operand: masked element loads (k >= K -> 0), swizzled float4 LDS stores.
template <int BX, int BK>
__device__ __forceinline__ void nt_masked(const float* __restrict__ base, int64_t ld, int x0, int X, int k0, int K,
                                          float* lds_op) {
  constexpr int CPR = BK / 4;
  for (int q = threadIdx.x; q < BX * CPR; q += kThreads) {
    const int row = q / CPR, c = q % CPR;
    const float* src = base + static_cast<int64_t>(min(x0 + row, X - 1)) * ld;
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = k0 + 4 * c + e;
      v[e] = k < K ? src[k] : 0.0f;
    }
    *reinterpret_cast<f32x4*>(lds_op + row * BK + 4 * (c ^ nt_swz<BK>(row))) = v;
  }
}

// OCC: waves per SIMD the register allocation must allow (blocks of 4 waves per CU), traded against spills.
// Per-row operands of the LSTM step epilogues.  They do not depend on the product, so the kernels load them before
// their k loop and their latency hides behind it (loaded inside the epilogue, the stores between its row rounds keep
// the compiler from batching the loads of the next round).  Lane l finishes rows pr + 8 rr at columns pc .. pc + 3
// of each 32 x 32 tile (pr = l / 8, pc = 4 (l % 8)); with the k range split KS ways over the block's waves, split ks
// finishes the rounds rr = ks + KS k, k < 4 / KS.  r0 / c0 are the wave's first row / column.
template <int EPI, int TM, int TN, int KS>
struct LstmPre {
  __device__ __forceinline__ void load(const Problem&, int, int, int, int) {}
};

template <int TM, int TN, int KS>
struct LstmPre<EPI_LSTM_FWD, TM, TN, KS> {
  static constexpr int RR = 4 / KS;
  f32x4 gx[TM][TN][RR];
  float cp[TM][TN][RR];
  float kp[TM][RR];
  __device__ __forceinline__ void load(const Problem& P, int r0, int c0, int lane, int ks) {
    const LstmArgs& L = P.lstm;
    const int pr = lane >> 3, pc = 4 * (lane & 7);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int k = 0; k < RR; ++k) {
        const int64_t m = r0 + i * 32 + pr + 8 * (ks + KS * k);
        const bool in = m < P.M;
        kp[i][k] = in && L.keep_prev != nullptr ? L.keep_prev[m * L.keep_stride] : 1.0f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = c0 + j * 32 + pc;
          if (in && n < P.N) {
            gx[i][j][k] = *reinterpret_cast<const f32x4*>(L.gx + m * L.ldgx + n);
            cp[i][j][k] = L.c_prev[m * L.ldcp + (n >> 2)];
          } else {
            gx[i][j][k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            cp[i][j][k] = 0.0f;
          }
        }
      }
  }
};

template <int TM, int TN, int KS>
struct LstmPre<EPI_LSTM_BWD, TM, TN, KS> {
  static constexpr int RR = 4 / KS;
  float keep[TM][RR], kp[TM][RR];
  f32x4 dh[TM][TN][RR], ct[TM][TN][RR], cp[TM][TN][RR], dc[TM][TN][RR];
  f32x4 gt[TM][TN][RR][4];
  __device__ __forceinline__ void load(const Problem& P, int r0, int c0, int lane, int ks) {
    const LstmArgs& L = P.lstm;
    const int64_t H = L.hidden;
    const int pr = lane >> 3, pc = 4 * (lane & 7);
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int k = 0; k < RR; ++k) {
        const int64_t m = r0 + i * 32 + pr + 8 * (ks + KS * k);
        const bool in = m < P.M;
        keep[i][k] = in ? L.keep[m * L.keep_stride] : 0.0f;
        kp[i][k] = in && L.keep_prev != nullptr ? L.keep_prev[m * L.keep_stride] : 1.0f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = c0 + j * 32 + pc;
          if (in && n < P.N) {
            dh[i][j][k] = *reinterpret_cast<const f32x4*>(L.dh + m * L.lddh + n);
            ct[i][j][k] = *reinterpret_cast<const f32x4*>(L.c + m * H + n);
            cp[i][j][k] = *reinterpret_cast<const f32x4*>(L.c_prev + m * L.ldcp + n);
            dc[i][j][k] = L.first ? z : *reinterpret_cast<const f32x4*>(L.dc + m * H + n);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              gt[i][j][k][e] = *reinterpret_cast<const f32x4*>(L.gates + m * 4 * H + 4 * (n + e));
          } else {
            dh[i][j][k] = ct[i][j][k] = cp[i][j][k] = dc[i][j][k] = z;
#pragma unroll
            for (int e = 0; e < 4; ++e) gt[i][j][k][e] = z;
          }
        }
      }
  }
};

// LSTM forward cell for env m, gate columns n .. n+3 = gates i, f, g, o of hidden unit n / 4 (4H and every base are
// multiples of 4); x = this step's recurrent product, cp = c_{t-1} of the unit already multiplied by keep_prev.
// The cell arithmetic itself, shared with the whole-sequence kernel so that both give identical results.
struct LstmCellFwd {
  f32x4 act;  // i, f, g, o
  float c, h;
};
__device__ __forceinline__ LstmCellFwd lstm_cell_fwd(const f32x4& x, const f32x4& gx, float cp) {
  LstmCellFwd o;
  const float ig = sigmoid_hw(x[0] + gx[0]), fg = sigmoid_hw(x[1] + gx[1]);
  const float gg = tanh_hw(x[2] + gx[2]), og = sigmoid_hw(x[3] + gx[3]);
  o.c = __builtin_fmaf(fg, cp, ig * gg);  // (explicit: every kernel that inlines the cell rounds it the same way)
  o.h = og * tanh_hw(o.c);
  o.act = f32x4{ig, fg, gg, og};
  return o;
}

// GRU cell (torch nn.GRU: r = sigma(W_ir x + b_ir + W_hr h + b_hr), z likewise, n = tanh(W_in x + b_in + r (W_hn h +
// b_hn)), h' = (1 - z) n + z h, evaluated as torch's cell does: n + z (h - n)) on the LSTM's four-slot layout.  Slot q
// of unit u holds r, z, the hidden part of n (W_hn h + b_hn) and its input part (W_in x + b_in): w_ih_g has zero rows
// in slot 2, w_hh_g in slot 3, and b_g = (b_ir + b_hr, b_iz + b_hz, b_hn, b_in), so the input projection and the
// recurrent product are the LSTM's GEMMs.  x = the recurrent product (slot 3 exactly zero), gx = the projection (slot
// 2 exactly b_hn), hp = h_{t-1} of the unit multiplied by keep_prev.  The state the LSTM keeps in c is h itself here:
// c = h = h', act = (r, z, W_hn h + b_hn, n) for the backward.
__device__ __forceinline__ LstmCellFwd gru_cell_fwd(const f32x4& x, const f32x4& gx, float hp) {
  LstmCellFwd o;
  const float r = sigmoid_hw(x[0] + gx[0]), z = sigmoid_hw(x[1] + gx[1]);
  const float a = x[2] + gx[2];
  const float n = tanh_hw(__builtin_fmaf(r, a, x[3] + gx[3]));
  o.h = __builtin_fmaf(z, hp - n, n);
  o.c = o.h;
  o.act = f32x4{r, z, a, n};
  return o;
}

template <bool GRU>
__device__ __forceinline__ LstmCellFwd rnn_cell_fwd(const f32x4& x, const f32x4& gx, float cp) {
  if constexpr (GRU) {
    return gru_cell_fwd(x, gx, cp);
  } else {
    return lstm_cell_fwd(x, gx, cp);
  }
}

__device__ __forceinline__ void lstm_fwd_finish(const LstmArgs& L, int64_t m, int n, const f32x4& x, const f32x4& gx,
                                                float cp) {
  const int64_t H = L.hidden, u = n >> 2;
  const LstmCellFwd o = L.cell == PPO_CELL_GRU ? gru_cell_fwd(x, gx, cp) : lstm_cell_fwd(x, gx, cp);
  *reinterpret_cast<f32x4*>(L.gates + m * 4 * H + n) = o.act;
  L.c[m * H + u] = o.c;
  L.h[m * L.ldh + u] = o.h;
  L.hs[m * H + u] = o.h * L.keep[m * L.keep_stride];
}

// LSTM backward cell for env m, hidden units n .. n+3; x = (dgates of the next step) . W_hh for those units.
// The cell derivatives for 4 units (the arithmetic shared with the whole-sequence kernel): dpre[e] = the four gate
// pre-activation gradients of unit e, dcout = dL/dc carried to the previous step.
__device__ __forceinline__ void lstm_cell_bwd(const f32x4& x, float keep, float keep_prev, const f32x4& dhu,
                                              const f32x4& ct, const f32x4& cp, const f32x4& dcin,
                                              const f32x4 (&gt)[4], f32x4 (&dpre)[4], f32x4& dcout) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float ig = gt[e][0], fg = gt[e][1], gg = gt[e][2], og = gt[e][3];
    const float dh = dhu[e] + keep * x[e];
    const float tc = tanh_hw(ct[e]);
    const float dct = dcin[e] + dh * og * (1.0f - tc * tc);
    dpre[e] = f32x4{dct * gg * ig * (1.0f - ig), dct * (cp[e] * keep_prev) * fg * (1.0f - fg),
                    dct * ig * (1.0f - gg * gg), dh * tc * og * (1.0f - og)};
    dcout[e] = dct * fg * keep_prev;
  }
}

// GRU backward cell for env m, hidden units n .. n+3 (slots and act as gru_cell_fwd).  The state h_t reaches step
// t + 1 through the recurrent product (x, masked by keep) and directly through z h_t: dcin carries the latter,
// dh_{t+1} z_{t+1} keep_t, as the LSTM carries dL/dc.  dpre = (dr r (1 - r), dz z (1 - z), dn' r, dn') with
// dn' = dh (1 - z) (1 - n^2), dr = dn' (W_hn h + b_hn), dz = dh (h_{t-1} - n).
__device__ __forceinline__ void gru_cell_bwd(const f32x4& x, float keep, float keep_prev, const f32x4& dhu,
                                             const f32x4& cp, const f32x4& dcin, const f32x4 (&gt)[4],
                                             f32x4 (&dpre)[4], f32x4& dcout) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float r = gt[e][0], z = gt[e][1], a = gt[e][2], nn = gt[e][3];
    const float dh = (dhu[e] + keep * x[e]) + dcin[e];
    const float dn = dh * (1.0f - z) * (1.0f - nn * nn);
    const float dz = dh * (cp[e] * keep_prev - nn);
    dpre[e] = f32x4{dn * a * r * (1.0f - r), dz * z * (1.0f - z), dn * r, dn};
    dcout[e] = dh * z * keep_prev;
  }
}

template <bool GRU>
__device__ __forceinline__ void rnn_cell_bwd(const f32x4& x, float keep, float keep_prev, const f32x4& dhu,
                                             const f32x4& ct, const f32x4& cp, const f32x4& dcin,
                                             const f32x4 (&gt)[4], f32x4 (&dpre)[4], f32x4& dcout) {
  if constexpr (GRU) {
    gru_cell_bwd(x, keep, keep_prev, dhu, cp, dcin, gt, dpre, dcout);
  } else {
    lstm_cell_bwd(x, keep, keep_prev, dhu, ct, cp, dcin, gt, dpre, dcout);
  }
}

__device__ __forceinline__ void lstm_bwd_finish(const LstmArgs& L, int64_t m, int n, const f32x4& x, float keep,
                                                float keep_prev, const f32x4& dhu, const f32x4& ct, const f32x4& cp,
                                                const f32x4& dcin, const f32x4 (&gt)[4]) {
  const int64_t H = L.hidden;
  f32x4 dpre[4], dcout;
  if (L.cell == PPO_CELL_GRU) {
    gru_cell_bwd(x, keep, keep_prev, dhu, cp, dcin, gt, dpre, dcout);
  } else {
    lstm_cell_bwd(x, keep, keep_prev, dhu, ct, cp, dcin, gt, dpre, dcout);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) *reinterpret_cast<f32x4*>(L.dgates + m * 4 * H + 4 * (n + e)) = dpre[e];
  if (!L.last) *reinterpret_cast<f32x4*>(L.dc + m * H + n) = dcout;
}

// The NT tile's body; `lds` is the kernel's ring of S stages.
template <int BM, int BN, int BK, int S, int OCC, bool A16, bool B16, int EPI>
__device__ __forceinline__ void gemm_nt_tile(const Group& g, const TileCoord& tc, float* lds) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = (BM + BN) * BK;
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  static_assert(S >= 2 && S <= 4, "2..4 LDS stages");
  constexpr int L = NtLoader<BM, BK, A16>::PER + NtLoader<BN, BK, B16>::PER;

  const Problem& P = g.p[tc.pi];
  // problem fields as values: the loop's compiler barriers would otherwise re-read them from the argument block
  const float* const A = P.A;
  const float* const B = P.B;
  const int64_t lda = P.lda, ldb = P.ldb;
  const int row0 = tc.tm * BM, col0 = tc.tn * BN;
  const int M = P.M, N = P.N, K = P.K;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  NtLoader<BM, BK, A16> la;
  NtLoader<BN, BK, B16> lb;
  la.init(lda, row0, M, wave, lane);
  lb.init(ldb, col0, N, wave, lane);
  LstmPre<EPI, TM, TN, 1> pre;
  pre.load(P, row0 + wm * WM, col0 + wn * WN, lane, 0);
  const int nfull = K / BK;
  const int nk = (K + BK - 1) / BK;
  auto issue = [&](int kt, int stage) {
    float* st = lds + stage * STAGE;
    const int k0 = kt * BK;
    if (kt < nfull) {
      la.issue(A + k0, st, wave);
      lb.issue(B + k0, st + BM * BK, wave);
    } else {
      nt_masked<BM, BK>(A, lda, row0, M, k0, K, st);
      nt_masked<BN, BK>(B, ldb, col0, N, k0, K, st + BM * BK);
    }
  };
  // k-groups of 4 MFMA steps; the fragments of group g + 1 are read before the MFMAs of group g issue, and the
  // fragments of group 0 of slab kt + 1 before the MFMAs of the last group of slab kt: the slab-boundary wait and
  // barrier sit between the last fragment reads of slab kt and its last MFMAs, so no MFMA waits on an LDS read.
  constexpr int G = BK / 8;
  f32x4 fa[2][TM], fb[2][TN];
  auto load_group = [&](int kt, int buf, int gi) {
    const float* As = lds + (kt % S) * STAGE;
    const float* Bs = As + BM * BK;
    const int c = 2 * gi + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm * WM + 32 * i + (lane & 31);
      fa[buf][i] = *reinterpret_cast<const f32x4*>(As + r * BK + 4 * (c ^ nt_swz<BK>(r)));
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int r = wn * WN + 32 * j + (lane & 31);
      fb[buf][j] = *reinterpret_cast<const f32x4*>(Bs + r * BK + 4 * (c ^ nt_swz<BK>(r)));
    }
  };
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) issue(s, s);
  if (nk > 0) {
    wait_slab<L, S>(min(S - 2, nk - 1));
    lds_barrier();  // slab 0 is in LDS for every wave
    if (S - 1 < nk) issue(S - 1, S - 1);
    load_group(0, 0, 0);
  }
  int buf = 0;
  for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      if (gi + 1 < G) {
        load_group(kt, buf ^ 1, gi + 1);
      } else if (kt + 1 < nk) {
        // every wave has its fragments of slab kt (the barrier's lgkmcnt(0)), and slab kt + 1 has landed: slab
        // kt's stage is free for slab kt + S
        wait_slab<L, S>(min(S - 2, nk - 2 - kt));
        lds_barrier();
        if (kt + S < nk) issue(kt + S, kt % S);
        load_group(kt + 1, buf ^ 1, 0);
      }
      // scheduling fences: the compiler would otherwise sink the reads below the MFMAs and reuse one register set
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            // weights (B) as the MFMA's A operand: the accumulator holds the 32 x 32 tile of C transposed
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[buf][j][s], fa[buf][i][s], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      buf ^= 1;
    }
  }

  // Epilogue, one 32 x 32 accumulator tile at a time through a private 32 x 36-float LDS patch per wave (the ring is
  // free once every wave is past its last slab).  Element v of lane l of acc[i][j] is row l%32 and column
  // 8*(v/4) + 4*(l/32) + v%4 of the tile, so a lane writes 4 float4 runs into the patch; it then reads back 16-byte
  // chunks in row order (8 lanes per 128-byte row) and finishes them there: +bias / ELU, or * ELU'(z_prev), with
  // every global access a fully used 128-byte row segment (16-byte vectors when P.c_vec, elements at the N edge).
  static_assert(4 * 32 * 36 <= S * STAGE, "epilogue patches must fit in the LDS ring");
  constexpr int PS = 36;  // patch row stride: 144 bytes spreads the 16 rows of a ds_write_b128 over all banks
  lds_barrier();
  float* patch = lds + wave * 32 * PS;
  const int h = lane >> 5;
  const int pr = lane >> 3, pc = 4 * (lane & 7);  // read-back: row pr (+8 per step), columns pc .. pc + 3
  constexpr bool GEN = epi_generic(EPI);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 x = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        *reinterpret_cast<f32x4*>(patch + (lane & 31) * PS + 8 * q + 4 * h) = x;
      }
      const int n = col0 + wn * WN + j * 32 + pc;
      const bool n_in = n < N;
      const bool full = P.c_vec && n + 3 < N;
      f32x4 bias = {0.0f, 0.0f, 0.0f, 0.0f};
      if ((EPI == EPI_BIAS || epi_fwd_act(EPI)) && n_in) {
#pragma unroll
        for (int e = 0; e < 4; ++e) bias[e] = n + e < N ? P.vec[n + e] : 0.0f;
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int r = pr + 8 * rr;
        const f32x4 x = *reinterpret_cast<const f32x4*>(patch + r * PS + pc);
        const int m = row0 + wm * WM + i * 32 + r;
        if (m >= M || !n_in) continue;
        const int64_t mm = m;
        if constexpr (EPI == EPI_LSTM_FWD) {
          lstm_fwd_finish(P.lstm, mm, n, x, pre.gx[i][j][rr], pre.cp[i][j][rr] * pre.kp[i][rr]);
          continue;
        } else if constexpr (EPI == EPI_LSTM_BWD) {
          lstm_bwd_finish(P.lstm, mm, n, x, pre.keep[i][rr], pre.kp[i][rr], pre.dh[i][j][rr], pre.ct[i][j][rr],
                          pre.cp[i][j][rr], pre.dc[i][j][rr], pre.gt[i][j][rr]);
          continue;
        }
        f32x4 o, o2;
        if (EPI == EPI_BIAS || epi_fwd_act(EPI)) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = x[e] + bias[e];
          if (epi_fwd_act(EPI)) act_fwd4<GEN>(P.act, o, o2);
        } else if (epi_act_grad(EPI)) {
          f32x4 zp;
          if (full) {
            zp = *reinterpret_cast<const f32x4*>(P.aux + mm * P.ldaux + n);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) zp[e] = n + e < N ? P.aux[mm * P.ldaux + n + e] : 0.0f;
          }
          act_grad4<GEN>(P.act, P.elu_from_output, x, zp, o);
        } else {
          o = x;
        }
        // with ELU either output may be absent (h alone feeds the next layer and the input-grad)
        const bool st_c = !epi_fwd_act(EPI) || P.C != nullptr;
        const bool st_c2 = epi_fwd_act(EPI) && P.C2 != nullptr;
        if (full) {
          if (st_c) *reinterpret_cast<f32x4*>(P.C + mm * P.ldc + n) = o;
          if (st_c2) *reinterpret_cast<f32x4*>(P.C2 + mm * P.ldc2 + n) = o2;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (n + e < N) {
              if (st_c) P.C[mm * P.ldc + n + e] = o[e];
              if (st_c2) P.C2[mm * P.ldc2 + n + e] = o2[e];
            }
          }
        }
      }
    }
  }
}

// B16M: the second operand's loads are 16 bytes wide in every problem (1), 4 bytes in every problem (0), or chosen
// per problem from Problem::b16 (2: a grouped launch whose weights differ in alignment, e.g. a 99-wide critic input
// beside a 96-wide actor input; the branch is uniform per block).
template <int BM, int BN, int BK, int S, int OCC, bool A16, int B16M, int EPI>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm_nt_kernel(
    const Group g) {
  __shared__ __align__(16) float lds[S * (BM + BN) * BK];
  const TileCoord tc = locate(g);
  if constexpr (B16M == 2) {
    if (g.p[tc.pi].b16) {
      gemm_nt_tile<BM, BN, BK, S, OCC, A16, true, EPI>(g, tc, lds);
    } else {
      gemm_nt_tile<BM, BN, BK, S, OCC, A16, false, EPI>(g, tc, lds);
    }
  } else {
    gemm_nt_tile<BM, BN, BK, S, OCC, A16, B16M == 1, EPI>(g, tc, lds);
  }
}

// ------------------------------------------------------------------------------------------------------------------
// Persistent NT for the forward and input-grad epilogues (bias / bias+ELU / ELU' / plain store).
//
// A launch of one block per output tile runs as one or two waves of blocks that start together, so every block
// loads, multiplies and stores in the same phase: the epilogue's stores (an output tile is as many bytes as its
// operands at k = BM, BN) are a burst at HBM write speed that no MFMA work overlaps.  Here a grid of resident blocks
// walks the tiles (block b takes tiles r * grid + b', b' its XCD-contiguous slot) and the LDS ring streams k-slabs
// across tile boundaries: the first slabs of tile r + 1 are in flight while tile r's epilogue runs, and tile r's
// stores drain while tile r + 1 multiplies.  Vector-memory operations retire in issue order on this target, so the
// wait for the slab issued before an epilogue may leave that epilogue's stores outstanding: vmcnt(NSTORE), NSTORE
// being exactly the stores the epilogue issues.  To keep that count exact, every epilogue store is a buffer store
// issued by every lane (lanes outside the output get an offset past the buffer's end, which the hardware drops).
// Requirements (checked on the host): 16-byte aligned operands with leading dimensions that are multiples of 4,
// K a multiple of BK, 16-byte aligned outputs with N a multiple of 4, outputs smaller than 2 GiB.
// ------------------------------------------------------------------------------------------------------------------

// Tile t of a grouped launch (problems' tile ranges in block_begin, one split each).
__device__ inline TileCoord tile_at(const Group& g, int t) {
  int pi = 0;
#pragma unroll
  for (int i = 1; i < PPO_MAX_LINEAR_PROBLEMS; ++i)
    if (i < g.count && t >= g.p[i].block_begin) pi = i;
  const Problem& P = g.p[pi];
  const int local = t - P.block_begin;
  TileCoord c;
  c.pi = pi;
  c.split = 0;
  c.tm = local / P.tiles_n;
  c.tn = local - c.tm * P.tiles_n;
  return c;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
constexpr uint32_t kDropOffset = 0x80000000u;  // past every output buffer (the host keeps them under 2 GiB)

// Raw buffer over a row-major [rows, ld] fp32 output (null: a zero-length buffer, every store dropped).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_buffer(float* base, int rows, int64_t ld) {
  const int bytes = base != nullptr ? static_cast<int>(static_cast<int64_t>(rows) * ld * 4) : 0;
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000);
}

__device__ __forceinline__ void store_b128(__amdgpu_buffer_rsrc_t r, uint32_t off, const f32x4& v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 0);
}

// The epilogue of one wave's (TM x TN) 32 x 32 accumulator tiles (layout as in gemm_nt_tile): each tile through the
// wave's own LDS patch, finished in row order, TM * TN * 4 * OUTS buffer stores in every lane.
template <int TM, int TN, int EPI, bool GEN>
__device__ __forceinline__ void nt_pipe_epilogue_t(const Problem& P, const f32x16 (&acc)[TM][TN], int row0w,
                                                   int col0w, float* patch, int lane) {
  constexpr int PS = 36;
  const int h = lane >> 5;
  const int pr = lane >> 3, pc = 4 * (lane & 7);
  const int M = P.M, N = P.N;
  const __amdgpu_buffer_rsrc_t rc = out_buffer(epi_fwd_act(EPI) && P.C == nullptr ? nullptr : P.C, M, P.ldc);
  const __amdgpu_buffer_rsrc_t rc2 = out_buffer(epi_fwd_act(EPI) ? P.C2 : nullptr, M, P.ldc2);
  // every load of the epilogue before its first store: a wait for a load issued after a store would wait for the
  // store as well (in-order retirement)
  f32x4 bias[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    bias[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int n = col0w + j * 32 + pc;
    if ((EPI == EPI_BIAS || epi_fwd_act(EPI)) && n < N) bias[j] = *reinterpret_cast<const f32x4*>(P.vec + n);
  }
  f32x4 zsrc[epi_act_grad(EPI) ? TM : 1][epi_act_grad(EPI) ? TN : 1][4];
  if constexpr (epi_act_grad(EPI)) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int n = col0w + j * 32 + pc, m = row0w + i * 32 + pr + 8 * rr;
          zsrc[i][j][rr] = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
          if (m < M && n < N) zsrc[i][j][rr] = *reinterpret_cast<const f32x4*>(P.aux + int64_t(m) * P.ldaux + n);
        }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 x = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        *reinterpret_cast<f32x4*>(patch + (lane & 31) * PS + 8 * q + 4 * h) = x;
      }
      const int n = col0w + j * 32 + pc;
      const bool n_in = n < N;  // N % 4 == 0: columns n .. n + 3 are all in or all out
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int r = pr + 8 * rr;
        const f32x4 x = *reinterpret_cast<const f32x4*>(patch + r * PS + pc);
        const int m = row0w + i * 32 + r;
        const bool ok = m < M && n_in;
        const int64_t mm = ok ? m : 0;
        f32x4 o, o2;
        if constexpr (EPI == EPI_BIAS || epi_fwd_act(EPI)) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = x[e] + bias[j][e];
          if constexpr (epi_fwd_act(EPI)) act_fwd4<GEN>(P.act, o, o2);
        } else if constexpr (epi_act_grad(EPI)) {
          act_grad4<GEN>(P.act, P.elu_from_output, x, zsrc[i][j][rr], o);
        } else {
          o = x;
        }
        store_b128(rc, ok ? static_cast<uint32_t>((mm * P.ldc + n) * 4) : kDropOffset, o);
        if constexpr (epi_fwd_act(EPI))
          store_b128(rc2, ok ? static_cast<uint32_t>((mm * P.ldc2 + n) * 4) : kDropOffset, o2);
      }
    }
  }
}

template <int TM, int TN, int EPI>
__device__ __forceinline__ void nt_pipe_epilogue(const Problem& P, const f32x16 (&acc)[TM][TN], int row0w, int col0w,
                                                 float* patch, int lane) {
  nt_pipe_epilogue_t<TM, TN, EPI, epi_generic(EPI)>(P, acc, row0w, col0w, patch, lane);
}

template <int BM, int BN, int BK, int OCC, int EPI>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm_nt_pipe_kernel(
    const Group g, int tiles) {
  static_assert(EPI == EPI_BIAS || epi_fwd_act(EPI) || epi_act_grad(EPI) || EPI == EPI_STORE,
                "persistent NT: forward / input-grad epilogues");
  constexpr int S = 2;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int G = BK / 8;
  constexpr int PS = 36;
  constexpr int NSTORE = TM * TN * 4 * (epi_fwd_act(EPI) ? 2 : 1);
  static_assert(TM >= 1 && TN >= 1 && NSTORE < 63, "tile");
  __shared__ __align__(16) float lds[S * STAGE + 4 * 32 * PS];
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  float* const patch = lds + S * STAGE + wave * 32 * PS;
  const int nblk = gridDim.x;
  const int slot = g.xcds > 1 ? xcd_remap(blockIdx.x, nblk, g.xcds) : static_cast<int>(blockIdx.x);
  if (slot >= tiles) return;

  // issue cursor: the next k-slab to load (tile itile, slab ikt), LDS stage istage
  int itile = slot, ikt = 0, istage = 0, ink = 0;
  const float* iA = nullptr;
  const float* iB = nullptr;
  NtLoader<BM, BK, true> la;
  NtLoader<BN, BK, true> lb;
  auto cursor_tile = [&]() {
    const TileCoord c = tile_at(g, itile);
    const Problem& P = g.p[c.pi];
    iA = P.A;
    iB = P.B;
    ink = P.K / BK;
    la.init(P.lda, c.tm * BM, P.M, wave, lane);
    lb.init(P.ldb, c.tn * BN, P.N, wave, lane);
  };
  cursor_tile();
  auto issue_next = [&]() {
    float* st = lds + istage * STAGE;
    la.issue(iA + ikt * BK, st, wave);
    lb.issue(iB + ikt * BK, st + BM * BK, wave);
    istage ^= 1;
    if (++ikt == ink) {
      ikt = 0;
      itile += nblk;
      if (itile < tiles) cursor_tile();
    }
  };
  auto more = [&]() { return itile < tiles; };

  f32x4 fa[2][TM], fb[2][TN];
  auto load_group = [&](int stage, int buf, int gi) {
    const float* As = lds + stage * STAGE;
    const float* Bs = As + BM * BK;
    const int c = 2 * gi + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm * WM + 32 * i + (lane & 31);
      fa[buf][i] = *reinterpret_cast<const f32x4*>(As + r * BK + 4 * (c ^ nt_swz<BK>(r)));
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int r = wn * WN + 32 * j + (lane & 31);
      fb[buf][j] = *reinterpret_cast<const f32x4*>(Bs + r * BK + 4 * (c ^ nt_swz<BK>(r)));
    }
  };

  // prologue: slab 0 in LDS for every wave, slab 1 in flight, slab 0's first fragments in registers
  issue_next();
  wait_vmcnt<0>();
  lds_barrier();
  if (more()) issue_next();
  int cstage = 0, buf = 0;
  load_group(cstage, buf, 0);

  int ctile = slot;
  bool first = true;
  for (;;) {
    const TileCoord cc = tile_at(g, ctile);
    const Problem& P = g.p[cc.pi];
    const int nk = P.K / BK;
    const bool next_tile = ctile + nblk < tiles;
    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        if (gi + 1 < G) {
          load_group(cstage, buf ^ 1, gi + 1);
        } else {
          if (kt + 1 < nk || next_tile) {
            // the next slab (issued one slab ago, before the previous tile's epilogue when this is a tile's first
            // slab) has landed for every wave, and every wave is done with this slab's stage
            if (kt == 0 && !first) {
              wait_vmcnt<NSTORE>();
            } else {
              wait_vmcnt<0>();
            }
            lds_barrier();
            if (more()) issue_next();
          }
          // read on every path (after the last slab: stale values, never used), so both paths reach the MFMAs with
          // the same LDS reads in flight and the compiler's wait counts stay exact
          load_group(cstage ^ 1, buf ^ 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[buf][j][s4], fa[buf][i][s4], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        buf ^= 1;
      }
      cstage ^= 1;
    }
    nt_pipe_epilogue<TM, TN, EPI>(P, acc, cc.tm * BM + wm * WM, cc.tn * BN + wn * WN, patch, lane);
    if (!next_tile) break;
    ctile += nblk;
    first = false;
  }
}

// Blocks of kernel k the current device holds at once (0 when unknown), cached per device in `cache`.
template <typename K>
int resident_blocks(K kernel, std::atomic<int>* cache) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    v = std::max(per_cu, 0) * std::max(cus, 0) + 1;  // stored + 1: 0 marks "not queried yet"
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v - 1;
}

// ------------------------------------------------------------------------------------------------------------------
// NT with the k range split over the block's waves, for the LSTM step products (EPI_LSTM_FWD / _BWD only; operands
// 16-byte aligned).  A step's product is small (E x 4H forward, E x H backward) and long in k (H, 4H): one 32 x 32
// tile per wave with the whole k range is a long dependent MFMA chain, and 64 x 64 blocks leave CUs idle.  Here the 4
// waves form a (BM / 32) x (BN / 32) grid of 32 x 32 tiles times KS = 4 / (grid size) k splits: split ks takes
// k-groups [ks G / KS, (ks + 1) G / KS) of every slab.  The KS partial tiles meet in the epilogue's LDS patches,
// summed in a fixed order, and each split finishes 4 / KS of the row rounds.
// ------------------------------------------------------------------------------------------------------------------

template <int BM, int BN, int BK, int S, int OCC, int EPI>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm_nt_ks_kernel(
    const Group g) {
  static_assert(EPI == EPI_LSTM_FWD || EPI == EPI_LSTM_BWD, "k-split kernel: LSTM step epilogues");
  constexpr int WGM = BM / 32, WGN = BN / 32, NWT = WGM * WGN, KS = 4 / NWT;
  static_assert(BM % 32 == 0 && BN % 32 == 0 && NWT * KS == 4, "4 waves = wave tiles x k splits");
  constexpr int G = BK / 8, GPW = G / KS;
  static_assert(G % KS == 0 && GPW >= 1, "every split takes whole k-groups of each slab");
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int PS = 36;  // epilogue patch row stride (as in gemm_nt_kernel)
  constexpr int LDS = S * STAGE > 4 * 32 * PS ? S * STAGE : 4 * 32 * PS;
  constexpr int L = NtLoader<BM, BK, true>::PER + NtLoader<BN, BK, true>::PER;
  __shared__ __align__(16) float lds[LDS];

  const TileCoord tc = locate(g);
  const Problem& P = g.p[tc.pi];
  const float* const A = P.A;
  const float* const B = P.B;
  const int64_t lda = P.lda, ldb = P.ldb;
  const int row0 = tc.tm * BM, col0 = tc.tn * BN;
  const int M = P.M, N = P.N, K = P.K;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int ks = wave / NWT, wt = wave % NWT, wm = wt / WGN, wn = wt % WGN;

  f32x16 acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.0f;

  NtLoader<BM, BK, true> la;
  NtLoader<BN, BK, true> lb;
  la.init(lda, row0, M, wave, lane);
  lb.init(ldb, col0, N, wave, lane);
  LstmPre<EPI, 1, 1, KS> pre;
  pre.load(P, row0 + 32 * wm, col0 + 32 * wn, lane, ks);
  const int nfull = K / BK;
  const int nk = (K + BK - 1) / BK;
  auto issue = [&](int kt, int stage) {
    float* st = lds + stage * STAGE;
    const int k0 = kt * BK;
    if (kt < nfull) {
      la.issue(A + k0, st, wave);
      lb.issue(B + k0, st + BM * BK, wave);
    } else {
      nt_masked<BM, BK>(A, lda, row0, M, k0, K, st);
      nt_masked<BN, BK>(B, ldb, col0, N, k0, K, st + BM * BK);
    }
  };
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < nk) issue(st, st);
  for (int kt = 0; kt < nk; ++kt) {
    wait_slab<L, S>(min(S - 2, nk - 1 - kt));
    lds_barrier();
    if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
    const float* As = lds + (kt % S) * STAGE;
    const float* Bs = As + BM * BK;
    f32x4 fa[2], fb[2];
    auto load_group = [&](int buf, int gi) {
      const int c = 2 * gi + (lane >> 5);
      const int ra = 32 * wm + (lane & 31), rb = 32 * wn + (lane & 31);
      fa[buf] = *reinterpret_cast<const f32x4*>(As + ra * BK + 4 * (c ^ nt_swz<BK>(ra)));
      fb[buf] = *reinterpret_cast<const f32x4*>(Bs + rb * BK + 4 * (c ^ nt_swz<BK>(rb)));
    };
    load_group(0, ks * GPW);
#pragma unroll
    for (int q = 0; q < GPW; ++q) {
      if (q + 1 < GPW) load_group((q + 1) & 1, ks * GPW + q + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[q & 1][s4], fa[q & 1][s4], acc, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Epilogue: every wave stores its partial tile (transposed accumulator, as in gemm_nt_kernel) into its own patch;
  // then split ks sums the KS patches of its tile, split 0 first, for its row rounds and finishes them.
  lds_barrier();
  {
    float* patch = lds + wave * 32 * PS;
    const int h = lane >> 5;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 x = {acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
      *reinterpret_cast<f32x4*>(patch + (lane & 31) * PS + 8 * q + 4 * h) = x;
    }
  }
  lds_barrier();
  const int pr = lane >> 3, pc = 4 * (lane & 7);
  const int n = col0 + 32 * wn + pc;
#pragma unroll
  for (int k = 0; k < 4 / KS; ++k) {
    const int r = pr + 8 * (ks + KS * k);
    f32x4 x = *reinterpret_cast<const f32x4*>(lds + wt * 32 * PS + r * PS + pc);
#pragma unroll
    for (int sp = 1; sp < KS; ++sp) {
      const f32x4 y = *reinterpret_cast<const f32x4*>(lds + (sp * NWT + wt) * 32 * PS + r * PS + pc);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] += y[e];
    }
    const int m = row0 + 32 * wm + r;
    if (m >= M || n >= N) continue;
    if constexpr (EPI == EPI_LSTM_FWD) {
      lstm_fwd_finish(P.lstm, m, n, x, pre.gx[0][0][k], pre.cp[0][0][k] * pre.kp[0][k]);
    } else {
      lstm_bwd_finish(P.lstm, m, n, x, pre.keep[0][k], pre.kp[0][k], pre.dh[0][0][k], pre.ct[0][0][k],
                      pre.cp[0][0][k], pre.dc[0][0][k], pre.gt[0][0][k]);
    }
  }
}

// ------------------------------------------------------------------------------------------------------------------
// TN (weight-grad): operands stored [k][x] (x contiguous); LDS tile [BK][BX], unpadded.
// ------------------------------------------------------------------------------------------------------------------

// Direct loads of one TN operand: one k-slab, rows [k0, k0 + BK) x columns [x0, x0 + BX), per call, through a raw
// buffer that ends after the slab's last existing row (rows past it read zeros); columns past X read the last
// in-bounds chunk / element instead (the 16-byte form needs ld >= X rounded up to 4, which a leading dimension that
// is a multiple of 4 guarantees).  Per-lane byte offsets from the slab's first row are fixed.
template <int BX, int BK, bool W16>
struct TnLoader {
  static constexpr int NQ = W16 ? BK * BX / 256 : BK * BX / 64;
  static constexpr int PER = NQ / 4;
  static_assert(NQ % 4 == 0, "every wave must issue the same number of loads per slab");
  uint32_t off[PER];

  __device__ __forceinline__ void init(int64_t ld, int x0, int X, int wave, int lane) {
    const int xlast = W16 ? ((X - 1) >> 2) << 2 : X - 1;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int q = 4 * j + wave;
      const int flat = W16 ? 4 * (64 * q + lane) : 64 * q + lane;
      const int row = flat / BX, x = flat % BX;
      const int64_t gx = min(x0 + x, xlast);
      off[j] = static_cast<uint32_t>((row * ld + gx) * 4);
    }
  }
  // base: the operand's row k0, wave-uniform; rows (<= BK): the slab's rows that exist, the others read zeros.
  // Issues this wave's loads j0 .. j1 - 1 of the slab (all of them by default).
  __device__ __forceinline__ void issue(const float* base, int64_t ld, int rows, float* lds_op, int wave, int j0 = 0,
                                        int j1 = PER) const {
    const __amdgpu_buffer_rsrc_t r = uniform_buffer(base, static_cast<int>(rows * ld * 4));
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (j < j0 || j >= j1) continue;
      if constexpr (W16) {
        dma_buf<16>(r, off[j], lds_op + (4 * j + wave) * 256);
      } else {
        dma_buf<4>(r, off[j], lds_op + (4 * j + wave) * 64);
      }
    }
  }
};

template <int BM, int BN, int BK, int S, int OCC, bool A16, bool B16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm_tn_kernel(
    const Group g) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int STAGE = BK * (BM + BN);
  static_assert(TM == 2 && TN == 2, "TN kernel: 2 x 2 interleaved MFMA tiles per wave");
  static_assert(BK % 8 == 0, "TN slabs hold whole groups of 4 k-steps");
  static_assert(S >= 2 && S <= 4, "2..4 LDS stages");
  constexpr int L = TnLoader<BM, BK, A16>::PER + TnLoader<BN, BK, B16>::PER;
  constexpr int G = BK / 8;  // groups of 4 MFMA k-steps (8 rows of k) per slab
  __shared__ __align__(16) float lds[S * STAGE];

  const TileCoord tc = locate(g);
  const Problem& P = g.p[tc.pi];
  // problem fields as values: the loop's compiler barriers would otherwise re-read them from the argument block
  const float* const A = P.A;
  const float* const B = P.B;
  const int64_t lda = P.lda, ldb = P.ldb;
  const int row0 = tc.tm * BM, col0 = tc.tn * BN;
  const int M = P.M, N = P.N;
  const int k_begin = tc.split * P.k_chunk;
  const int k_end = min(P.K, k_begin + P.k_chunk);
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  const int h = lane >> 5, sg = lane & 31;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // Bias-gradient column sums from the A fragments already in registers: lane (h, sg) holds A[k][c] for the columns
  // c = wm * WM + 2 sg + i (i = 0, 1) at the rows k = h (mod 2) of the block's range, added in row order in fp64;
  // the two row parities meet in the end.  No LDS reads of their own, so no wait between the MFMAs.  Every wave
  // adds (the wn = 1 waves hold the same fragments) so the waves of a block take the same time.
  double colsum_acc[2] = {0.0, 0.0};
  const int span = max(k_end - k_begin, 0);
  const int nk = (span + BK - 1) / BK;
  TnLoader<BM, BK, A16> la;
  TnLoader<BN, BK, B16> lb;
  la.init(lda, row0, M, wave, lane);
  lb.init(ldb, col0, N, wave, lane);
  // Rows past k_end (the split's last, partial slab) read zeros; a slab wholly past it (the loop's look-ahead at the
  // end) becomes a zero fill that fetches nothing.  part = -1: every load of the slab; part = 0 .. 3: this wave's
  // loads of quarter `part` of each operand.
  constexpr int PA = TnLoader<BM, BK, A16>::PER, PB = TnLoader<BN, BK, B16>::PER;  // quarters [q PER / 4, ...)
  auto issue = [&](int kt, int stage, int part) {
    float* st = lds + stage * STAGE;
    const int k0 = k_begin + kt * BK;
    const int rows = max(0, min(BK, k_end - k0));
    if (part < 0) {
      la.issue(A + k0 * lda, lda, rows, st, wave);
      lb.issue(B + k0 * ldb, ldb, rows, st + BK * BM, wave);
    } else {
      la.issue(A + k0 * lda, lda, rows, st, wave, part * PA / 4, (part + 1) * PA / 4);
      lb.issue(B + k0 * ldb, ldb, rows, st + BK * BM, wave, part * PB / 4, (part + 1) * PB / 4);
    }
  };
  f32x2 fa[2][4], fb[2][4];
  auto load_group = [&](int stage, int buf, int gi) {
    const float* As = lds + stage * STAGE;
    const float* Bs = As + BK * BM;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kk = 8 * gi + 2 * st + h;
      fa[buf][st] = *reinterpret_cast<const f32x2*>(As + kk * BM + wm * WM + 2 * sg);
      fb[buf][st] = *reinterpret_cast<const f32x2*>(Bs + kk * BN + wn * WN + 2 * sg);
    }
  };

  if (nk > 0) {
    // prologue: slab 0 in LDS for every wave, slabs 1 .. S - 1 in flight, slab 0's first fragments in registers
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
      if (s < nk) issue(s, s, -1);
    wait_slab<L, S>(min(S - 2, nk - 1));
    lds_barrier();
    if (S - 1 < nk) issue(S - 1, S - 1, -1);
    load_group(0, 0, 0);
  }
  int buf = 0;
  for (int kt = 0; kt < nk; ++kt) {
    const int cstage = kt % S;
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const bool last = gi + 1 == G;
      if (!last) {
        load_group(cstage, buf ^ 1, gi + 1);
        // scheduling fence: the compiler would otherwise sink the reads below the MFMAs and reuse one register set
        __builtin_amdgcn_sched_barrier(0);
      } else {
        // The last group's fragments are in registers: once slab kt + 1 has landed for every wave and every wave is
        // done reading this stage, slab kt + S streams into it (on every slab, the last ones as zero fills, so the
        // loads share a block with the MFMAs below) and slab kt + 1's first fragments load under this group's
        // MFMAs (after the last slab: stale values, never used).
        wait_slab<L, S>(max(0, min(S - 2, nk - 2 - kt)));
        lds_barrier();
        load_group((kt + 1) % S, buf ^ 1, 0);
      }
#pragma unroll
      for (int st = 0; st < 4; ++st) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[buf][st][i], fb[buf][st][j], acc[i][j], 0, 0, 0);
          if (last && i == 0) {
            // a quarter of the next slab's loads per k-step, between MFMAs: a whole slab's loads issued back to back
            // fill the texture unit's queue and hold every wave of the CU at its next load with the MFMA pipe idle
            __builtin_amdgcn_sched_barrier(0);
            issue(kt + S, cstage, st);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) colsum_acc[i] += static_cast<double>(fa[buf][st][i]);
      }
      // keeps the group's adds here: the compiler would otherwise sink the whole chain behind the slab's last
      // branch, 32 dependent fp64 adds in a row between two MFMA groups
      asm volatile("" : "+v"(colsum_acc[0]), "+v"(colsum_acc[1]));
      __builtin_amdgcn_sched_barrier(0);
      buf ^= 1;
    }
  }
  wait_vmcnt<0>();  // the look-ahead's zero fills land before the block ends

  // Partial store.  Accumulator row rho = 8*(v/4) + 4*h + v%4 of tile i is m = 2*rho + i (TM == 2) or rho, and
  // column sg of tile j is n = 2*sg + j (TN == 2) or sg.
  float* Cs = P.C + static_cast<int64_t>(tc.split) * P.partial_stride;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int rho = 8 * (v >> 2) + 4 * h + (v & 3);
      const int m = row0 + wm * WM + (TM == 2 ? 2 * rho + i : rho);
      if (m >= M) continue;
      float* crow = Cs + static_cast<int64_t>(m) * P.ldc;
      if constexpr (TN == 2) {
        const int n = col0 + wn * WN + 2 * sg;
        if (n + 1 < N) {
          f32x2 o = {acc[i][0][v], acc[i][1][v]};
          *reinterpret_cast<f32x2*>(crow + n) = o;
        } else if (n < N) {
          crow[n] = acc[i][0][v];
        }
      } else {
        const int n = col0 + wn * WN + sg;
        if (n < N) crow[n] = acc[i][0][v];
      }
    }
  }
  if (P.colsum != nullptr && tc.tn == 0) {  // the two row parities of each column, h = 0 first
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const double other = __shfl_xor(colsum_acc[i], 32, 64);
      const double sum = h == 0 ? colsum_acc[i] + other : other + colsum_acc[i];
      const int m = row0 + wm * WM + 2 * sg + i;
      if (wn == 0 && h == 0 && m < M) P.colsum[static_cast<int64_t>(tc.split) * M + m] = sum;
    }
  }
}

// ------------------------------------------------------------------------------------------------------------------
// TN weight-grad on the bf16 matrix cores at fp32 accuracy.  Every operand element splits exactly into three bf16
// parts x = hi + mid + lo (each rounded to nearest from what the previous parts leave: 8 significant bits each, the
// 24 of fp32, for values in the normal range), and a product a b is taken as the six part products down to 16 bits
// below the leading one: lo.hi + mid.mid + hi.lo + mid.hi + hi.mid + hi.hi (small terms first); the three left out
// (mid.lo, lo.mid, lo.lo) are at most 2^-23 of |a b| together, the order of one fp32 rounding.  This is the
// published bf16x6 scheme (Henry, Tang and Heinecke, "Leveraging the bfloat16 artificial intelligence datatype for
// higher-precision computations", ARITH 2019).  Part products of bf16 values are exact in the fp32 accumulators.
// One v_mfma_f32_32x32x16_bf16 is 16 k-steps of a 32 x 32 tile at an eighth of the 32x32x2 fp32 MFMA's cycles per
// k-step, so the six take 3/4 of the fp32 MFMA's time... per 16 k-steps: 6 x 8 passes against 8 x 16.
//
// Each slab (16 rows of k) is staged through registers with 16-byte loads along the columns (the operands are
// k-major), split once per block (not once per wave that reads it), and written as bf16 parts into k-major planes;
// gfx950's transposing LDS read (ds_read_b64_tr_b16) then hands each lane 4 consecutive k of one column, two of them
// a wave's MFMA operand.  A slab's loads are issued two slabs ahead of its MFMAs (two register buffers), and its
// split into the free one of two stages runs between the MFMA groups of the slab before it, so each wave's VALU
// work overlaps its own MFMAs.  The fp64 bias sums come from the staged A values.
// ------------------------------------------------------------------------------------------------------------------

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Three-way split of two floats into packed bf16 pairs (element 0 in the low half).
__device__ __forceinline__ void split_bf16x3(float x0, float x1, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  float r0 = x0, r1 = x1;
  uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{r0, r1}), bf16x2));
  hi = u;
  r0 -= __builtin_bit_cast(float, u << 16);
  r1 -= __builtin_bit_cast(float, u & 0xffff0000u);
  u = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{r0, r1}), bf16x2));
  mid = u;
  r0 -= __builtin_bit_cast(float, u << 16);
  r1 -= __builtin_bit_cast(float, u & 0xffff0000u);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{r0, r1}), bf16x2));
}

// Two floats rounded to bf16 (to nearest even), packed (element 0 in the low half): the operands of the bf16-operand
// mode (PPO_GEMM_BF16_OPERANDS), whose products are the hi-part products of the bf16x6 scheme alone.
__device__ __forceinline__ uint32_t round_bf16x2(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{x0, x1}), bf16x2));
}

typedef short i16x4 __attribute__((ext_vector_type(4)));

// Byte offset of the 8-byte chunk c (4 bf16 columns) of row k in a k-major plane of W bf16 columns: the chunk index
// XOR-ed so that the 4 consecutive rows one transposing read takes (8 consecutive chunks each, per 32 lanes) fall on
// all 64 banks: W = 128 (256-byte rows) 8 (k % 4); W = 64 (128-byte rows: rows k and k + 1 already on different
// halves) 8 ((k / 2) % 2).
template <int W>
__device__ __forceinline__ int tn_chunk_off(int k, int c) {
  static_assert(W == 128 || W == 64, "plane width");
  return k * (W * 2) + ((c ^ (W == 128 ? 8 * (k & 3) : 8 * ((k >> 1) & 1))) << 3);
}

// One BM x BN tile (BN = 128, or 64 for narrow problems: then each wave owns 64 x 32 and B is staged one row per
// thread) of one split of the weight-grad.
// BF16: operands rounded to bf16 and one product per k-group (the bf16-operand mode); only part plane 0 is used.
template <int BN, bool FULL, bool BF16 = false>
__device__ __forceinline__ void tn_bx6_tile(const Group& g, const TileCoord tc, unsigned char* lds) {
  constexpr int BM = 128, BK = 16;
  constexpr int TN = BN / 64;                  // 32-column accumulator tiles per wave
  constexpr int PLANE = BK * BM * 2;           // bytes of one part of A: [16 rows of k][128 columns] bf16
  constexpr int PLANE_B = BK * BN * 2;         // one part of B
  constexpr int STAGE = 3 * (PLANE + PLANE_B);  // 3 parts x 2 operands
  constexpr int NBR = BN == 128 ? 2 : 1;       // B rows staged per thread and slab
  const Problem& P = g.p[tc.pi];
  const float* const A = P.A;
  const float* const B = P.B;
  const int64_t lda = P.lda, ldb = P.ldb;
  const int row0 = tc.tm * BM, col0 = tc.tn * BN;
  const int M = P.M, N = P.N;
  const int k_begin = tc.split * P.k_chunk;
  const int k_end = min(P.K, k_begin + P.k_chunk);
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  // slabs in pairs (the unrolled loop's two halves use the two register buffers); a slab past k_end is all zeros
  const int nk2 = (max(k_end - k_begin, 0) + 2 * BK - 1) / (2 * BK);
  // FULL (every chunk of the launch whole slab pairs: rows and split chunks multiples of 32): no per-row clamp and
  // no zeroing, each slab's address a wave-uniform offset from the lane's rows.  Only the blocks of the first column
  // tile that have a bias gradient sum columns; with and without, the loop has its own copy (no branch inside it).
  const bool want_colsum = P.colsum != nullptr && tc.tn == 0;

  // Staging: thread t loads the 4 columns 4 (t % 32) .. + 3 (clamped into the matrix: results past M / N are
  // discarded; ld % 4 == 0 keeps the chunk inside its row) of rows t / 32 and t / 32 + 8 of both operands' slab
  // (16-byte loads; a wave reads two 512-byte row pieces per load), rows at or past k_end as zeros.  Its part
  // chunks go to [row][column] planes (a row is 64 banks wide), the 8-byte chunk index XOR-ed with 8 (row % 4): the
  // transposing reads below take, per 32 lanes, 4 consecutive rows at 8 consecutive chunks, which this spreads over
  // all 64 banks.
  // (BN = 64: thread t loads the B columns 4 (t % 16) .. + 3 of slab row t / 16)
  const int sc = tid & 31, sk = tid >> 5;
  const int bsc = BN == 128 ? sc : tid & 15, bsk = BN == 128 ? sk : tid >> 4;
  const int mc_a = min(row0 + 4 * sc, ((M - 1) >> 2) << 2), mc_b = min(col0 + 4 * bsc, ((N - 1) >> 2) << 2);
  const float* const a_col = A + mc_a;
  const float* const b_col = B + mc_b;
  const int w_off0 = tn_chunk_off<BM>(sk, sc), w_off1 = tn_chunk_off<BM>(sk + 8, sc);
  const int wb_off0 = tn_chunk_off<BN>(bsk, bsc), wb_off1 = tn_chunk_off<BN>(bsk + 8, bsc);
  f32x4 stage_v[2][2 + NBR];  // two buffers of: A rows sk, sk + 8; B rows bsk (, bsk + 8)
  // Rows past k_end load row k_end - 1 and are zeroed afterwards: unconditional loads (no branch) keep the
  // compiler's wait counts for them exact across the loop.
  // FULL: the slab's rows from a wave-uniform base and 32-bit lane offsets (the launcher checks that 16 rows of
  // either operand span less than 2^31 bytes); the look-ahead past the end re-reads the last slab
  const int last_k0 = k_end - k_begin - BK;
  const uint32_t a_off[2] = {static_cast<uint32_t>((sk * lda + mc_a) * 4), static_cast<uint32_t>(((sk + 8) * lda + mc_a) * 4)};
  const uint32_t b_off[2] = {static_cast<uint32_t>((bsk * ldb + mc_b) * 4),
                             static_cast<uint32_t>(((bsk + 8) * ldb + mc_b) * 4)};
  auto load_slab = [&](int kt, f32x4 (&v)[2 + NBR]) __attribute__((always_inline)) {
    if constexpr (FULL) {
      const int64_t k0 = k_begin + min(kt * BK, last_k0);
      const unsigned char* const abase = reinterpret_cast<const unsigned char*>(A + k0 * lda);
      const unsigned char* const bbase = reinterpret_cast<const unsigned char*>(B + k0 * ldb);
#pragma unroll
      for (int h = 0; h < 2; ++h) v[h] = *reinterpret_cast<const f32x4*>(abase + a_off[h]);
#pragma unroll
      for (int h = 0; h < NBR; ++h) v[2 + h] = *reinterpret_cast<const f32x4*>(bbase + b_off[h]);
    } else {
      const int k0 = k_begin + kt * BK;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kc = min(k0 + sk + 8 * h, k_end - 1);
        v[h] = *reinterpret_cast<const f32x4*>(a_col + static_cast<int64_t>(kc) * lda);
      }
#pragma unroll
      for (int h = 0; h < NBR; ++h) {
        const int kc = min(k0 + bsk + 8 * h, k_end - 1);
        v[2 + h] = *reinterpret_cast<const f32x4*>(b_col + static_cast<int64_t>(kc) * ldb);
      }
    }
  };
  auto zero_tail = [&](int kt, f32x4 (&v)[2 + NBR]) {  // (applied where the values are used)
    const int k0 = k_begin + kt * BK;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (k0 + sk + 8 * h >= k_end) v[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < NBR; ++h)
      if (k0 + bsk + 8 * h >= k_end) v[2 + h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  };
  // q: A row sk, A row sk + 8, B row bsk (, B row bsk + 8)
  auto split_row = [&](const f32x4& v, int q, unsigned char* st) {
    unsigned char* c = st + (q < 2 ? ((q & 1) ? w_off1 : w_off0) : 3 * PLANE + ((q & 1) ? wb_off1 : wb_off0));
    if constexpr (BF16) {
      const uint32_t h0 = round_bf16x2(v[0], v[1]), h1 = round_bf16x2(v[2], v[3]);
      *reinterpret_cast<uint64_t*>(c) = (static_cast<uint64_t>(h1) << 32) | h0;
    } else {
      uint32_t h[2], md[2], l[2];
      split_bf16x3(v[0], v[1], h[0], md[0], l[0]);
      split_bf16x3(v[2], v[3], h[1], md[1], l[1]);
      const int pl = q < 2 ? PLANE : PLANE_B;
      *reinterpret_cast<uint64_t*>(c) = (static_cast<uint64_t>(h[1]) << 32) | h[0];
      *reinterpret_cast<uint64_t*>(c + pl) = (static_cast<uint64_t>(md[1]) << 32) | md[0];
      *reinterpret_cast<uint64_t*>(c + 2 * pl) = (static_cast<uint64_t>(l[1]) << 32) | l[0];
    }
  };
  double colsum_acc[4] = {0.0, 0.0, 0.0, 0.0};  // columns 4 sc + e of A over rows sk, sk + 8 of every slab, in order
  auto add_colsum = [&](const f32x4 (&v)[2 + NBR]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) colsum_acc[e] += static_cast<double>(v[0][e]) + static_cast<double>(v[1][e]);
  };

  f32x16 acc[2][TN];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // MFMA operand of 32 columns x 16 rows (lane l: column l % 32, rows 8 (l / 32) .. + 7) by two transposing reads:
  // within each 16 lanes, lane 4 r + i addresses row k0 + r, chunk i of its group's 16 columns, and lane d receives
  // rows k0 .. k0 + 3 of column d.
  const int grp = lane >> 4, gi = lane & 3, gr = (lane >> 2) & 3;
  const int rd_k = 8 * (grp >> 1) + gr, rd_c = 4 * (grp & 1) + gi;  // row (first read), chunk within 32 columns
  // (W: the plane's width in columns)
  auto frag = [&](auto w_c, const unsigned char* pl, int col32) {  // col32: first column of the 32 (a multiple of 32)
    constexpr int W = decltype(w_c)::value;
    const int c = col32 / 4 + rd_c;
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(pl + tn_chunk_off<W>(rd_k, c)));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(pl + tn_chunk_off<W>(rd_k + 4, c)));
    typedef short i16x8 __attribute__((ext_vector_type(8)));
    const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, v);
  };

  auto run = [&](auto colsum_c) __attribute__((always_inline)) {
  constexpr bool CS = decltype(colsum_c)::value;
  if (nk2 > 0) {  // slab 0 in stage 0, slab 1 in registers
    load_slab(0, stage_v[0]);
    load_slab(1, stage_v[1]);
    if constexpr (!FULL) zero_tail(0, stage_v[0]);
#pragma unroll
    for (int q = 0; q < 2 + NBR; ++q) split_row(stage_v[0][q], q, lds);
    if constexpr (CS) add_colsum(stage_v[0]);
    lds_barrier();
  }
  for (int kp = 0; kp < nk2; ++kp) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      // slab kt = 2 kp + u sits in stage u; slab kt + 1 in buffer u ^ 1 is split into stage u ^ 1 (which every wave
      // finished reading before the last barrier) between this slab's MFMA groups, while slab kt + 2 loads into
      // buffer u
      const int kt = 2 * kp + u;
      load_slab(kt + 2, stage_v[u]);
      __builtin_amdgcn_sched_barrier(0);
      const unsigned char* st = lds + u * STAGE;
      unsigned char* nst = lds + (u ^ 1) * STAGE;
      constexpr int NP = BF16 ? 1 : 3;  // part planes read
      bf16x8 fa[2][3], fb[TN][3];
#pragma unroll
      for (int pp = 0; pp < NP; ++pp) {
#pragma unroll
        for (int i = 0; i < 2; ++i) fa[i][pp] = frag(IntC<BM>{}, st + pp * PLANE, wm * 64 + 32 * i);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j][pp] = frag(IntC<BN>{}, st + 3 * PLANE + pp * PLANE_B, wn * (BN / 2) + 32 * j);
      }
      if constexpr (!FULL) zero_tail(kt + 1, stage_v[u ^ 1]);
      if constexpr (BF16) {  // the one product, then the next slab's rounding and its column sums
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i][0], fb[j][0], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 2 + NBR; ++q) split_row(stage_v[u ^ 1][q], q, nst);
        if (CS && (!FULL || kt + 1 < 2 * nk2)) add_colsum(stage_v[u ^ 1]);
        lds_barrier();
        continue;
      }
      constexpr int pa[6] = {2, 1, 0, 1, 0, 0}, pb[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
      for (int t = 0; t < 6; ++t) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i][pa[t]], fb[j][pb[t]], acc[i][j], 0, 0, 0);
        if (t < 2 + NBR) split_row(stage_v[u ^ 1][t], t, nst);
        // (FULL: the look-ahead past the last slab re-reads it; it must not count twice)
        if (t == 4 && CS && (!FULL || kt + 1 < 2 * nk2)) add_colsum(stage_v[u ^ 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      lds_barrier();
    }
  }
  };
  if (!FULL || want_colsum) {  // (the general case keeps one copy: a second one would not fit the registers)
    run(BoolC<true>{});
  } else {
    run(BoolC<false>{});
  }

  // partial store: accumulator element v of lane l is row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32 of its tile
  const int fr = lane & 31, fc = lane >> 5;
  float* Cs = P.C + static_cast<int64_t>(tc.split) * P.partial_stride;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = col0 + wn * (BN / 2) + 32 * j + fr;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = row0 + wm * 64 + 32 * i + 8 * (v >> 2) + 4 * fc + (v & 3);
        if (m < M && n < N) Cs[static_cast<int64_t>(m) * P.ldc + n] = acc[i][j][v];
      }
    }
  if (want_colsum) {  // column 4 sc + e: the 8 row groups sk = 0 .. 7 in order
    double* part = reinterpret_cast<double*>(lds);  // [8][128]
    lds_barrier();
#pragma unroll
    for (int e = 0; e < 4; ++e) part[sk * 128 + 4 * sc + e] = colsum_acc[e];
    lds_barrier();
    if (tid < 128 && row0 + tid < M) {
      double sum = part[tid];
      for (int r = 1; r < 8; ++r) sum += part[r * 128 + tid];
      P.colsum[static_cast<int64_t>(tc.split) * M + row0 + tid] = sum;
    }
  }
}

template <int OCC, bool FULL, bool BF16 = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm_tn_bx6_kernel(
    const Group g) {
  __shared__ __align__(16) unsigned char lds[2 * 6 * 16 * 128 * 2];  // two stages of the 128 x 128 tile's planes
  const TileCoord tc = locate(g);
  if (g.p[tc.pi].tn64) {
    tn_bx6_tile<64, FULL, BF16>(g, tc, lds);
  } else {
    tn_bx6_tile<128, FULL, BF16>(g, tc, lds);
  }
}

// ------------------------------------------------------------------------------------------------------------------
// NT (forward / input-grad) on the bf16 matrix cores at fp32 accuracy, with the part products of the weight-grad's
// bf16x6 kernel above: one BM x BN output tile per block (BM = 128, BN = 128 or 64; 4 waves in 2 x 2, each
// 64 x BN / 2), 16-deep k-slabs in NS LDS stages (two: 48 KiB with 128 x 128 tiles, three blocks per CU).  Both
// operands are k-contiguous: each staged row is read by four lanes (Q4, one 16-byte load of 4 consecutive k each) or
// two (two 16-byte loads of 8 k each), split into its bf16 parts and written to [rows][16] bf16 planes (16-byte
// chunks XOR-swapped on bit 3 of the row as in the weight-grad kernel).  A slab's loads go out NS iterations before
// its MFMAs into one of two register buffers, and its split lands in LDS one iteration later.  The accumulators have
// the fp32 NT kernels' layout (B fragment first), so the persistent kernel's epilogues finish the tile, through
// patches in the (then free) stage memory.
// ------------------------------------------------------------------------------------------------------------------
// BF16: operands rounded to bf16 and one product per k-group (the bf16-operand mode); only part plane 0 is used.
template <int BN, int OCC, int EPI, int NS, bool Q4, bool BKM = false, bool BF16 = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm_nt_bx6_kernel(
    const Group g) {
  static_assert(EPI == EPI_BIAS || epi_fwd_act(EPI) || epi_act_grad(EPI) || EPI == EPI_STORE,
                "bf16x6 NT: forward / input-grad epilogues");
  static_assert(BN == 128 || BN == 64, "tile");
  static_assert(!BKM || (BN == 128 && Q4), "k-major B: 128-wide tiles, four lanes per A row");
  constexpr int BM = 128, BK = 16;
  constexpr int TM = 2, TN = BN / 64;
  constexpr int PLANE_A = BM * BK * 2, PLANE_B = BN * BK * 2;  // bytes of one part of one operand
  constexpr int STAGE = 3 * (PLANE_A + PLANE_B);
  static_assert(NS == 2 || NS == 3, "LDS stages");
  constexpr int PS = 36;
  static_assert(4 * 32 * PS * 4 <= NS * STAGE, "epilogue patches fit in the stage memory");
  __shared__ __align__(16) unsigned char lds[NS * STAGE];

  const TileCoord tc = locate(g);
  const Problem& P = g.p[tc.pi];
  const float* const A = P.A;
  const float* const B = P.B;
  const int64_t lda = P.lda, ldb = P.ldb;
  const int row0 = tc.tm * BM, col0 = tc.tn * BN;
  const int M = P.M, N = P.N;
  const int nk = P.K / BK;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;

  // staging: Q4 -- four lanes per row, each one 16-byte load of 4 consecutive k (a wave's load covers 16 rows x 64
  // bytes), parts written as 8-byte halves of the chunks; else two lanes per row, each two 16-byte loads of 8
  // consecutive k (32 rows x 2 x 32 bytes), parts written as whole 16-byte chunks
  constexpr int LPR = Q4 ? 4 : 2;                 // lanes per staged row
  constexpr int RPP = kThreads / LPR;             // rows per staging pass
  constexpr int NA = BM / RPP;                    // A rows per thread
  constexpr int NB = BN >= RPP ? BN / RPP : 1;    // B rows per thread
  constexpr int LD = Q4 ? 1 : 2;                  // 16-byte loads per staged row
  const int sr = tid / LPR, sq = tid % LPR;       // first staged row, k part
  const bool stage_b = BN >= RPP || sr < BN;
  // (plain 16-byte global loads: this compiler turns element reads of __builtin_amdgcn_raw_buffer_load_b128's result
  // into one 4-byte load)
  const float* arow[NA];
  const float* brow[NB];
  int swz[NA > NB ? NA : NB];
#pragma unroll
  for (int i = 0; i < NA; ++i)
    arow[i] = A + static_cast<int64_t>(min(row0 + sr + i * RPP, M - 1)) * lda + (16 / LPR) * sq;
  // BKM: B is k-major (B[k][n], the weights of an input-grad as stored); thread t loads columns 4 (t % 32) .. + 3
  // (clamped into the row; ldb % 4 == 0) of slab rows t / 32 and t / 32 + 8, as the weight-grad kernel stages
  const int bsc = tid & 31, bsk = tid >> 5;
  int boff[2];
  if constexpr (BKM) {
    const float* const bcol = B + min(col0 + 4 * bsc, ((N - 1) >> 2) << 2);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      brow[h] = bcol + static_cast<int64_t>(bsk + 8 * h) * ldb;
      const int kr = bsk + 8 * h;  // [16 k][128 n] plane, 8-byte chunk index XOR-ed with 8 (k % 4)
      boff[h] = kr * (BN * 2) + (((bsc) ^ (8 * (kr & 3))) << 3);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NB; ++i)
      brow[i] = B + static_cast<int64_t>(min(col0 + (stage_b ? sr + i * RPP : 0), N - 1)) * ldb + (16 / LPR) * sq;
  }
#pragma unroll
  for (int i = 0; i < (NA > NB ? NA : NB); ++i) {  // byte offset of the thread's piece of row sr + i RPP in a plane
    const int r = sr + i * RPP;
    swz[i] = Q4 ? r * 32 + 16 * ((sq >> 1) ^ ((r >> 3) & 1)) + 8 * (sq & 1) : r * 32 + 16 * (sq ^ ((r >> 3) & 1));
  }
  // two register buffers: slab s is loaded NS iterations before its MFMAs and split into LDS one iteration later
  constexpr int NV = (NA + NB) * LD;
  u32x4 stage_v[2][NV];
  auto load_slab = [&](int kt, int rb) {  // the slab index is clamped into [0, nk): the look-ahead past the end re-reads
    const int k0 = min(kt, nk - 1) * BK;
    u32x4* const sv = stage_v[rb];
#pragma unroll
    for (int i = 0; i < NA; ++i)
#pragma unroll
      for (int l = 0; l < LD; ++l) sv[i * LD + l] = *reinterpret_cast<const u32x4*>(arow[i] + k0 + 4 * l);
    if constexpr (BKM) {
#pragma unroll
      for (int h = 0; h < 2; ++h) sv[NA + h] = *reinterpret_cast<const u32x4*>(brow[h] + static_cast<int64_t>(k0) * ldb);
    } else if (stage_b) {
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int l = 0; l < LD; ++l) sv[(NA + i) * LD + l] = *reinterpret_cast<const u32x4*>(brow[i] + k0 + 4 * l);
    }
  };
  auto split_piece = [&](int stage, int rb, int o) __attribute__((always_inline)) {
    unsigned char* st = lds + stage * STAGE;
    const u32x4* const sv = stage_v[rb];
    {
      if (o >= NA && !stage_b) return;
      const int i = o < NA ? o : o - NA;
      [[maybe_unused]] const int plane = o < NA ? PLANE_A : PLANE_B;
      unsigned char* row = st + (o < NA ? swz[i] : 3 * PLANE_A + (BKM ? boff[i] : swz[i]));
      uint32_t w[4 * LD];
#pragma unroll
      for (int l = 0; l < LD; ++l)
#pragma unroll
        for (int e = 0; e < 4; ++e) w[4 * l + e] = sv[o * LD + l][e];
      if constexpr (BF16) {
        uint32_t h[2 * LD];
#pragma unroll
        for (int q = 0; q < 2 * LD; ++q)
          h[q] = round_bf16x2(__builtin_bit_cast(float, w[2 * q]), __builtin_bit_cast(float, w[2 * q + 1]));
        if constexpr (Q4) {
          *reinterpret_cast<u32x2*>(row) = u32x2{h[0], h[1]};
        } else {
          *reinterpret_cast<u32x4*>(row) = u32x4{h[0], h[1], h[2], h[3]};
        }
        return;
      }
      uint32_t h[2 * LD], md[2 * LD], lo[2 * LD];
#pragma unroll
      for (int q = 0; q < 2 * LD; ++q)
        split_bf16x3(__builtin_bit_cast(float, w[2 * q]), __builtin_bit_cast(float, w[2 * q + 1]), h[q], md[q], lo[q]);
      if constexpr (Q4) {
        *reinterpret_cast<u32x2*>(row) = u32x2{h[0], h[1]};
        *reinterpret_cast<u32x2*>(row + plane) = u32x2{md[0], md[1]};
        *reinterpret_cast<u32x2*>(row + 2 * plane) = u32x2{lo[0], lo[1]};
      } else {
        *reinterpret_cast<u32x4*>(row) = u32x4{h[0], h[1], h[2], h[3]};
        *reinterpret_cast<u32x4*>(row + plane) = u32x4{md[0], md[1], md[2], md[3]};
        *reinterpret_cast<u32x4*>(row + 2 * plane) = u32x4{lo[0], lo[1], lo[2], lo[3]};
      }
    }
  };
  auto split_store = [&](int stage, int rb) {
#pragma unroll
    for (int o = 0; o < NA + NB; ++o) split_piece(stage, rb, o);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int fr = lane & 31, fc = lane >> 5;
  auto frag = [&](const unsigned char* pl, int r) {
    return *reinterpret_cast<const bf16x8*>(pl + r * 32 + 16 * (fc ^ ((r >> 3) & 1)));
  };
  // BKM: the B operand of 32 columns by transposing reads of the k-major plane, as in the weight-grad kernel
  const int grp = lane >> 4, gi = lane & 3, gr = (lane >> 2) & 3;
  const int rd_k = 8 * (grp >> 1) + gr, rd_c = 4 * (grp & 1) + gi;
  auto frag_t = [&](const unsigned char* pl, int col32) {
    const int c = col32 / 4 + rd_c;
    auto off = [](int kk, int cc) { return kk * (BN * 2) + ((cc ^ (8 * (kk & 3))) << 3); };
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(pl + off(rd_k, c)));
    const i16x4 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(pl + off(rd_k + 4, c)));
    typedef short i16x8 __attribute__((ext_vector_type(8)));
    const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, v);
  };

  if (nk > 0) {
    load_slab(0, 0);
    load_slab(1, 1);
    split_store(0, 0);
    if constexpr (NS == 3) {
      load_slab(2, 0);
      split_store(1, 1);
    }
    lds_barrier();
  }
  // slab s is loaded into register buffer s % 2 at iteration s - NS (the first NS in the prologue) and split into
  // LDS stage s % NS at iteration s - NS + 1, so iteration kt loads slab kt + NS and stores slab kt + NS - 1 (into the
  // stage of slab kt - 1, which every wave finished reading before the last barrier)
  auto step = [&](int kt, int cs, int rb_load, int rb_store) {
    load_slab(kt + NS, rb_load);
    __builtin_amdgcn_sched_barrier(0);  // (the compiler would sink the loads to their use)
    const unsigned char* st = lds + cs * STAGE;
    constexpr int NP = BF16 ? 1 : 3;  // part planes read
    bf16x8 fa[TM][3], fb[TN][3];
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i][pp] = frag(st + pp * PLANE_A, wm * 64 + 32 * i + fr);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j][pp] = BKM ? frag_t(st + 3 * PLANE_A + pp * PLANE_B, wn * (BN / 2) + 32 * j)
                        : frag(st + 3 * PLANE_A + pp * PLANE_B, wn * (BN / 2) + 32 * j + fr);
    }
    constexpr int pa[6] = {2, 1, 0, 1, 0, 0}, pb[6] = {0, 1, 2, 0, 1, 0};
    const int next = cs == 0 ? NS - 1 : cs - 1;
    if constexpr (BF16) {  // the one product, then the next slab's rounding
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j][0], fa[i][0], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      split_store(next, rb_store);
    } else if constexpr (BN == 128) {
      // the next slab's split, one staged row piece after each group of MFMAs: the wave's VALU work and LDS writes
      // issue while its MFMAs run (humanoid, per mini-batch: dx1 94 -> 88 us, fwd1 84 -> 83 us; the 64-wide tiles,
      // with half the MFMAs per group, measured 1 us slower that way)
#pragma unroll
      for (int t = 0; t < 6; ++t) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j][pb[t]], fa[i][pa[t]], acc[i][j], 0, 0, 0);
        if (t < NA + NB) split_piece(next, rb_store, t);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int o = 6; o < NA + NB; ++o) split_piece(next, rb_store, o);
    } else {
#pragma unroll
      for (int t = 0; t < 6; ++t)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j][pb[t]], fa[i][pa[t]], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      split_store(next, rb_store);
    }
    lds_barrier();
  };
  constexpr int RB_EVEN = NS % 2;  // the buffer iteration kt loads into, kt even
  int cs = 0, kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    step(kt, cs, RB_EVEN, 1 - RB_EVEN);
    cs = cs == NS - 1 ? 0 : cs + 1;
    step(kt + 1, cs, 1 - RB_EVEN, RB_EVEN);
    cs = cs == NS - 1 ? 0 : cs + 1;
  }
  if (kt < nk) step(kt, cs, RB_EVEN, 1 - RB_EVEN);
  float* const patch = reinterpret_cast<float*>(lds) + wave * 32 * PS;  // every wave is past the last barrier
  nt_pipe_epilogue<TM, TN, EPI>(P, acc, row0 + wm * 64, col0 + wn * (BN / 2), patch, lane);
}

// 16-byte direct loads need a 16-byte aligned base and a leading dimension that is a multiple of 4.
bool w16_ok(const float* base, int64_t ld) { return (reinterpret_cast<uintptr_t>(base) % 16 == 0) && ld % 4 == 0; }

int assign_blocks(Group& g, int count, int bm, int bn, const char* name, int& blocks) {
  blocks = 0;
  for (int i = 0; i < count; ++i) {
    Problem& p = g.p[i];
    p.tiles_m = static_cast<int>(ceil_div(p.M, bm));
    p.tiles_n = static_cast<int>(ceil_div(p.N, bn));
    p.block_begin = blocks;
    const int64_t nb = static_cast<int64_t>(p.tiles_m) * p.tiles_n * p.splits;
    if (blocks + nb > INT32_MAX) return fail(PPO_EUNSUPPORTED, "%s: grid too large", name);
    blocks += static_cast<int>(nb);
  }
  g.count = count;
  g.xcds = device_info().xcds;
#ifdef PPO_HIP_TUNING
  if (std::getenv("PPO_HIP_NO_XCD_REMAP") != nullptr) g.xcds = 1;
#endif
  for (int i = count; i < PPO_MAX_LINEAR_PROBLEMS; ++i) g.p[i].block_begin = INT32_MAX;
  return PPO_OK;
}

template <int BM, int BN, int BK, int S, int OCC, int EPI>
int launch_nt(Group& g, int count, hipStream_t s, const char* name) {
  int blocks;
  if (int rc = assign_blocks(g, count, BM, BN, name, blocks)) return rc;
  if (blocks == 0) return PPO_OK;
  bool a16 = true, all_b16 = true, any_b16 = false;
  for (int i = 0; i < count; ++i) {
    a16 = a16 && w16_ok(g.p[i].A, g.p[i].lda);
    g.p[i].b16 = w16_ok(g.p[i].B, g.p[i].ldb);
    all_b16 = all_b16 && g.p[i].b16;
    any_b16 = any_b16 || g.p[i].b16;
  }
  const dim3 grid(blocks), block(kThreads);
  if (a16) {
    if (all_b16) {
      hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, BK, S, OCC, true, 1, EPI>), grid, block, 0, s, g);
    } else if (any_b16) {
      hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, BK, S, OCC, true, 2, EPI>), grid, block, 0, s, g);
    } else {
      hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, BK, S, OCC, true, 0, EPI>), grid, block, 0, s, g);
    }
  } else {
    hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, BK, S, OCC, false, 0, EPI>), grid, block, 0, s, g);
  }
  return check_launch(name);
}

// Launch for problems whose operands are known to allow 16-byte loads (the caller has checked).
template <int BM, int BN, int BK, int S, int OCC, int EPI>
int launch_nt_aligned(Group& g, int count, hipStream_t s, const char* name) {
  int blocks;
  if (int rc = assign_blocks(g, count, BM, BN, name, blocks)) return rc;
  if (blocks == 0) return PPO_OK;
  for (int i = 0; i < count; ++i) g.p[i].b16 = 1;
  hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, BK, S, OCC, true, 1, EPI>), dim3(blocks), dim3(kThreads), 0, s, g);
  return check_launch(name);
}

// The k-split LSTM step kernel (operands known to allow 16-byte loads).
template <int BM, int BN, int BK, int S, int OCC, int EPI>
int launch_nt_ks(Group& g, int count, hipStream_t s, const char* name) {
  int blocks;
  if (int rc = assign_blocks(g, count, BM, BN, name, blocks)) return rc;
  if (blocks == 0) return PPO_OK;
  hipLaunchKernelGGL((gemm_nt_ks_kernel<BM, BN, BK, S, OCC, EPI>), dim3(blocks), dim3(kThreads), 0, s, g);
  return check_launch(name);
}

template <int BM, int BN, int BK, int S, int OCC>
int launch_tn(Group& g, int count, hipStream_t s, const char* name) {
  int blocks;
  if (int rc = assign_blocks(g, count, BM, BN, name, blocks)) return rc;
  if (blocks == 0) return PPO_OK;
  bool a16 = true, b16 = true;
  for (int i = 0; i < count; ++i) {
    a16 = a16 && w16_ok(g.p[i].A, g.p[i].lda);
    b16 = b16 && w16_ok(g.p[i].B, g.p[i].ldb);
  }
  if (a16 && b16) {
    hipLaunchKernelGGL((gemm_tn_kernel<BM, BN, BK, S, OCC, true, true>), dim3(blocks), dim3(kThreads), 0, s, g);
  } else if (a16) {
    hipLaunchKernelGGL((gemm_tn_kernel<BM, BN, BK, S, OCC, true, false>), dim3(blocks), dim3(kThreads), 0, s, g);
  } else if (b16) {
    hipLaunchKernelGGL((gemm_tn_kernel<BM, BN, BK, S, OCC, false, true>), dim3(blocks), dim3(kThreads), 0, s, g);
  } else {
    hipLaunchKernelGGL((gemm_tn_kernel<BM, BN, BK, S, OCC, false, false>), dim3(blocks), dim3(kThreads), 0, s, g);
  }
  return check_launch(name);
}

// The bf16x6 weight-grad when every problem's operands allow 16-byte loads (16-byte aligned, leading dimension a
// multiple of 4); PPO_EUNSUPPORTED otherwise.
template <int OCC>
int launch_tn_bx6(Group& g, int count, hipStream_t s, const char* name, bool bf16 = false) {
  bool full = true;  // every split chunk whole slab pairs, 16 rows of an operand under 2^31 bytes
  for (int i = 0; i < count; ++i) {
    const Problem& p = g.p[i];
    if (!w16_ok(p.A, p.lda) || !w16_ok(p.B, p.ldb)) return PPO_EUNSUPPORTED;
    full = full && p.K % 32 == 0 && p.k_chunk % 32 == 0 && 16 * std::max(p.lda, p.ldb) * 4 < (int64_t(1) << 31);
  }
  int blocks;
  if (int rc = assign_blocks(g, count, 128, 128, name, blocks)) return rc;
  // problems at most 64 columns wide: 128 x 64 tiles (the split plan gave them half the others' splits)
  blocks = 0;
  for (int i = 0; i < count; ++i) {
    Problem& p = g.p[i];
    p.tn64 = p.N <= 64 ? 1 : 0;
    p.tiles_n = static_cast<int>(ceil_div(p.N, p.tn64 ? 64 : 128));
    p.block_begin = blocks;
    blocks += p.tiles_m * p.tiles_n * p.splits;  // (at most the 128 x 128 count assign_blocks checked)
  }
  if (blocks == 0) return PPO_OK;
  if (bf16) {  // the bf16-operand mode: one product per k-group
    if (full) {
      hipLaunchKernelGGL((gemm_tn_bx6_kernel<OCC, true, true>), dim3(blocks), dim3(kThreads), 0, s, g);
    } else {
      hipLaunchKernelGGL((gemm_tn_bx6_kernel<(OCC < 2 ? OCC : 2), false, true>), dim3(blocks), dim3(kThreads), 0, s,
                         g);
    }
  } else if (full) {
    hipLaunchKernelGGL((gemm_tn_bx6_kernel<OCC, true>), dim3(blocks), dim3(kThreads), 0, s, g);
  } else {  // (the clamped, zeroed rows need more registers than three blocks per CU leave: two)
    hipLaunchKernelGGL((gemm_tn_bx6_kernel<(OCC < 2 ? OCC : 2), false>), dim3(blocks), dim3(kThreads), 0, s, g);
  }
  return check_launch(name);
}

// NT tile of a launch (BM x BN, k-slab depth, LDS stages, waves per SIMD).  The library ships the three the layers'
// shapes use (chosen by timing every tile on MI355X at 24,576-row mini-batches); a build with PPO_HIP_TUNING defined
// adds the others and the "PPO_HIP_GEMM_TILE" override (e.g. "128x128k16s2o3") for such sweeps.
enum Tile {
  T128x128k16s2o3, T128x64k32s2o4, T64x64k32s2o4,
#ifdef PPO_HIP_TUNING
  T128x128k16s3o3, T128x128k16s2o2, T128x128k32s2o2, T128x64k16s4o4, T64x64k32s2o5, T192x128k16s2o2,
  T128x128k64s2o1, T128x128k32s2o1, T256x128k32s2o1, T128x64k64s2o2
#endif
};

Tile pick_tile(Tile dflt) {
#ifdef PPO_HIP_TUNING
  const char* e = std::getenv("PPO_HIP_GEMM_TILE");
  if (e == nullptr) return dflt;
  static const struct {
    const char* name;
    Tile t;
  } kTiles[] = {{"128x128k16s2o3", T128x128k16s2o3}, {"128x128k16s3o3", T128x128k16s3o3},
                {"128x128k16s2o2", T128x128k16s2o2}, {"128x128k32s2o2", T128x128k32s2o2},
                {"128x64k16s4o4", T128x64k16s4o4},   {"128x64k32s2o4", T128x64k32s2o4},
                {"64x64k32s2o4", T64x64k32s2o4},     {"64x64k32s2o5", T64x64k32s2o5},
                {"192x128k16s2o2", T192x128k16s2o2}, {"128x128k64s2o1", T128x128k64s2o1},
                {"128x128k32s2o1", T128x128k32s2o1}, {"256x128k32s2o1", T256x128k32s2o1},
                {"128x64k64s2o2", T128x64k64s2o2}};
  for (const auto& k : kTiles)
    if (!std::strcmp(e, k.name)) return k.t;
#endif
  return dflt;
}

template <int EPI>
int launch_nt_tile(Tile t, Group& g, int count, hipStream_t s, const char* name) {
  switch (t) {
    case T128x64k32s2o4:
      return launch_nt<128, 64, 32, 2, 4, EPI>(g, count, s, name);
    case T64x64k32s2o4:
      return launch_nt<64, 64, 32, 2, 4, EPI>(g, count, s, name);
#ifdef PPO_HIP_TUNING
    case T128x128k16s3o3:
      return launch_nt<128, 128, 16, 3, 3, EPI>(g, count, s, name);
    case T128x128k16s2o2:
      return launch_nt<128, 128, 16, 2, 2, EPI>(g, count, s, name);
    case T128x128k32s2o2:
      return launch_nt<128, 128, 32, 2, 2, EPI>(g, count, s, name);
    case T128x64k16s4o4:
      return launch_nt<128, 64, 16, 4, 4, EPI>(g, count, s, name);
    case T64x64k32s2o5:
      return launch_nt<64, 64, 32, 2, 5, EPI>(g, count, s, name);
    case T192x128k16s2o2:
      return launch_nt<192, 128, 16, 2, 2, EPI>(g, count, s, name);
    case T128x128k64s2o1:
      return launch_nt<128, 128, 64, 2, 1, EPI>(g, count, s, name);
    case T128x128k32s2o1:
      return launch_nt<128, 128, 32, 2, 1, EPI>(g, count, s, name);
    case T256x128k32s2o1:
      return launch_nt<256, 128, 32, 2, 1, EPI>(g, count, s, name);
    case T128x64k64s2o2:
      return launch_nt<128, 64, 64, 2, 2, EPI>(g, count, s, name);
#endif
    default:
      return launch_nt<128, 128, 16, 2, 3, EPI>(g, count, s, name);
  }
}

}  // namespace
}  // namespace ppo
