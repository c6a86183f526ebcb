// A6 linear layers (rsl_rl/modules/mlp.py:27-95; autograd of nn.Linear / nn.ELU) as fp32-accurate MFMA GEMMs for
// gfx950.  Launches whose operands all have 16-byte rows run the bf16x6 kernels of gemm_core.hpp (each fp32 operand
// split into three bf16 parts, six bf16 MFMA products per fp32 product, fp32 accumulation); the others run the fp32
// MFMA kernels described here.
//
// Two fp32 kernel families, both 256 threads = 4 wavefronts in a 2 x 2 arrangement over a BM x BN output tile, each
// wave owning (BM/2) x (BN/2) of 32 x 32 v_mfma_f32_32x32x2f32 accumulators, both fed by gfx950's direct
// global->LDS loads (global_load_lds_dwordx4 / _dword: no register staging, no ds_write) into a two-stage LDS ring
// with one barrier per BK-deep k-slab:
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
// float2-wide.  Reads of rows past M or N are clamped into the operand (their results are discarded); the K tail
// is loaded through a masked path with zeros.  Several independent problems (actor and critic, or all layers of
// the weight-grad) share one launch: the block index maps to (problem, split, tile) through per-problem block
// offsets, after an XCD-aware permutation that places consecutive tiles (which share an A panel) on one XCD / L2.
#include <cstdlib>
#include <cstring>

#include "gemm_core.hpp"

namespace ppo {
namespace {

// Fixed-order reduction of split-K weight-grad partials: dw = sum_s partial[s], db = sum_s colsum[s].  A work item
// is 4 consecutive columns of one output row (the partials' rows are padded to ld = round4(in), so the loads are
// float4), summed split after split (every element in the same order as a scalar loop), then the bias entries.
//
// With a norm buffer (ppo_linear_bwd_dw_norm) the launch has exactly PPO_DW_NORM_BLOCKS blocks and every block also
// writes one row of PPO_MAX_PARAM_GROUPS fp64 partial sums of squares of the values it stored (its items in order,
// then a fixed-order block reduction), block 0 adding the squares of the caller's extra gradient ranges.
struct ReduceItem {
  const float* partial;  // [splits, out, ld]
  const double* colsum;  // [splits, out]
  float* dw;
  float* db;
  int64_t begin;         // first work item of this problem in the launch
  int64_t stride;        // floats between splits
  int32_t out, in, ld, splits;
  int32_t group;         // 0: not in a norm, g + 1: parameter group g
};
struct ReduceGroup {
  ReduceItem it[PPO_MAX_LINEAR_PROBLEMS];
  int32_t count;
  int64_t total;
  double* norm;  // [PPO_DW_NORM_BLOCKS][PPO_MAX_PARAM_GROUPS] or null
  const float* extra_grads;
  ppo_grad_range extra[PPO_MAX_EXTRA_GRADS];
  int32_t num_extra;
};

constexpr int kReduceBatch = 8;

// Adds x to the accumulator of group `group` (1-based; 0 adds nothing) with static register indexing.
__device__ __forceinline__ void add_sq(double (&sq)[PPO_MAX_PARAM_GROUPS], int group, double x) {
#pragma unroll
  for (int k = 0; k < PPO_MAX_PARAM_GROUPS; ++k)
    if (group == k + 1) sq[k] += x;
}

template <int THREADS>
__global__ __launch_bounds__(THREADS) void dw_reduce_kernel(const ReduceGroup g) {
  double sq[PPO_MAX_PARAM_GROUPS];
#pragma unroll
  for (int k = 0; k < PPO_MAX_PARAM_GROUPS; ++k) sq[k] = 0.0;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < g.total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int pi = 0;
#pragma unroll
    for (int i = 1; i < PPO_MAX_LINEAR_PROBLEMS; ++i)
      if (i < g.count && e >= g.it[i].begin) pi = i;
    const ReduceItem& R = g.it[pi];
    const int local = static_cast<int>(e - R.begin);  // < out * (ld / 4 + 1): 32-bit (checked on the host)
    const int q4 = R.ld >> 2;
    if (local < R.out * q4) {
      const int o = local / q4, i = 4 * (local - o * q4);
      const float* src = R.partial + static_cast<int64_t>(o) * R.ld + i;
      f32x4 acc = *reinterpret_cast<const f32x4*>(src);
      // splits 1, 2, ... added in order; kReduceBatch loads in flight at a time (clamped addresses past the last
      // split, discarded), not one dependent round trip per split
      for (int k0 = 1; k0 < R.splits; k0 += kReduceBatch) {
        f32x4 v[kReduceBatch];
#pragma unroll
        for (int j = 0; j < kReduceBatch; ++j)
          v[j] = *reinterpret_cast<const f32x4*>(src + static_cast<int64_t>(min(k0 + j, R.splits - 1)) * R.stride);
#pragma unroll
        for (int j = 0; j < kReduceBatch; ++j)
          if (k0 + j < R.splits) {
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] += v[j][c];
          }
      }
      float* out = R.dw + static_cast<int64_t>(o) * R.in + i;
      double s2 = 0.0;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (i + c < R.in) {
          out[c] = acc[c];
          s2 += static_cast<double>(acc[c]) * acc[c];
        }
      add_sq(sq, R.group, s2);
    } else {
      const int o = local - R.out * q4;
      double acc = 0.0;
      for (int k0 = 0; k0 < R.splits; k0 += kReduceBatch) {
        double v[kReduceBatch];
#pragma unroll
        for (int j = 0; j < kReduceBatch; ++j)
          v[j] = R.colsum[min(k0 + j, R.splits - 1) * static_cast<int64_t>(R.out) + o];
#pragma unroll
        for (int j = 0; j < kReduceBatch; ++j)
          if (k0 + j < R.splits) acc += v[j];
      }
      const float b = static_cast<float>(acc);
      R.db[o] = b;
      add_sq(sq, R.group, static_cast<double>(b) * b);
    }
  }
  if (g.norm == nullptr) return;
  if (blockIdx.x == 0) {
    for (int r = 0; r < g.num_extra; ++r)
      for (int64_t e = g.extra[r].begin + threadIdx.x; e < g.extra[r].end; e += blockDim.x) {
        const double x = g.extra_grads[e];
        add_sq(sq, g.extra[r].group + 1, x * x);
      }
  }
  __shared__ double red[THREADS / 64][PPO_MAX_PARAM_GROUPS];
#pragma unroll
  for (int k = 0; k < PPO_MAX_PARAM_GROUPS; ++k) {
    double x = sq[k];
    for (int off = 32; off > 0; off >>= 1) x += __shfl_down(x, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6][k] = x;
  }
  __syncthreads();
  if (threadIdx.x < PPO_MAX_PARAM_GROUPS) {
    double x = 0.0;
    for (int w = 0; w < THREADS / 64; ++w) x += red[w][threadIdx.x];
    g.norm[static_cast<int64_t>(blockIdx.x) * PPO_MAX_PARAM_GROUPS + threadIdx.x] = x;
  }
}

// w^T for the input-grad: wt[i, o] = w[o, i], ld of wt = out rounded up to 4.  32 x 32 tiles through LDS.
struct TransposeItem {
  const float* w;
  float* wt;
  int32_t out, in, ldt, tiles_in, block_begin, pad;
};
struct TransposeGroup {
  TransposeItem it[PPO_MAX_LINEAR_PROBLEMS];
  int32_t count;
};

__global__ __launch_bounds__(256) void transpose_kernel(const TransposeGroup g) {
  __shared__ float tile[32][33];
  int pi = 0;
#pragma unroll
  for (int i = 1; i < PPO_MAX_LINEAR_PROBLEMS; ++i)
    if (i < g.count && static_cast<int>(blockIdx.x) >= g.it[i].block_begin) pi = i;
  const TransposeItem& T = g.it[pi];
  const int local = blockIdx.x - T.block_begin;
  const int to = local / T.tiles_in, ti = local % T.tiles_in;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int o = to * 32 + r, i = ti * 32 + tx;
    tile[r][tx] = (o < T.out && i < T.in) ? T.w[static_cast<int64_t>(o) * T.in + i] : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int i = ti * 32 + r, o = to * 32 + tx;
    if (i < T.in && o < T.ldt) T.wt[static_cast<int64_t>(i) * T.ldt + o] = tile[tx][r];
  }
}

// Weight-grad: 128 x 128 tiles; split-K over the rows, in chunks that are multiples of the deepest (64-row) slab.
// The split count fills ONE wave of resident blocks and no more: the bf16x6 tile runs three blocks per CU (the fp32
// one two), so 768 blocks on the 256 CUs of a whole MI355X (fewer on a partitioned one).  A launch of 1,050 blocks
// (the humanoid weight-grads' 30 tiles x 35 splits, fp32 tile) leaves its last 26 blocks alone on the chip for a
// third of the kernel time; 30 x 17 = 510 blocks measured 280 us against 324.  The workspace query is host arithmetic (no device needed): it plans for the
// largest capacity, kDwMaxConcurrent, and a launch on a smaller device uses fewer splits, i.e. less workspace.
constexpr int kDwBM = 128, kDwBN = 128, kDwChunk = 64;
constexpr int kDwBlocksPerCu = 3;     // the bf16x6 kernel (168 VGPRs, 48 KiB LDS)
constexpr int kDwF32BlocksPerCu = 2;  // the fp32 kernel, for operands without 16-byte rows
constexpr int kDwMaxConcurrent = kDwBlocksPerCu * 256;

int dw_query_capacity() {
#ifdef PPO_HIP_TUNING
  if (const char* e = std::getenv("PPO_HIP_DW_BLOCKS")) return std::max(1, std::atoi(e));  // tuning aid
#endif
  return kDwMaxConcurrent;
}

int dw_launch_capacity(int blocks_per_cu) {
  const int cus = device_info().cus;
  const int cap = dw_query_capacity();
  return cus > 0 ? std::min(cap, blocks_per_cu * cus) : cap;
}

int dw_splits(int64_t tiles, int64_t rows, int capacity) {
  int64_t s = capacity / std::max<int64_t>(tiles, 1);
  s = std::min<int64_t>(s, std::max<int64_t>(1, rows / 256));
  s = std::max<int64_t>(1, std::min<int64_t>(s, 256));
  return static_cast<int>(s);
}

int64_t round4(int64_t n) { return (n + 3) / 4 * 4; }

struct DwPlan {
  int splits[PPO_MAX_LINEAR_PROBLEMS];
  int k_chunk[PPO_MAX_LINEAR_PROBLEMS];
  size_t partial_off[PPO_MAX_LINEAR_PROBLEMS];  // floats
  size_t colsum_off[PPO_MAX_LINEAR_PROBLEMS];   // floats (8-byte aligned: holds doubles)
  size_t total_floats;
};

// A problem at most 64 columns wide (in_features) runs on 128 x 64 tiles in the bf16x6 kernel (half a tile's work per
// block), so it gets half the splits of the others: every block of the launch then has about the same work.
bool dw_narrow(const ppo_linear_bwd_dw_problem& q) { return q.in_features <= kDwBN / 2; }

DwPlan plan_dw(const ppo_linear_bwd_dw_problem* probs, int count, int64_t rows, int capacity) {
  DwPlan plan{};
  int64_t halves = 0;  // work in half tiles (128 x 64)
  for (int i = 0; i < count; ++i)
    halves += ceil_div(probs[i].out_features, kDwBM) *
              (dw_narrow(probs[i]) ? 1 : 2 * ceil_div(probs[i].in_features, kDwBN));
  const int s_full = dw_splits((halves + 1) / 2, rows, capacity);
  size_t off = 0;
  for (int i = 0; i < count; ++i) {
    const int s = dw_narrow(probs[i]) ? std::max(1, s_full / 2) : s_full;
    const int64_t chunk = ceil_div(ceil_div(rows, s), kDwChunk) * kDwChunk;
    const int splits = static_cast<int>(ceil_div(rows, chunk));
    plan.splits[i] = splits;
    plan.k_chunk[i] = static_cast<int>(chunk);
    plan.partial_off[i] = off;
    off += static_cast<size_t>(splits) * probs[i].out_features * round4(probs[i].in_features);
    off = (off + 63) & ~static_cast<size_t>(63);
    plan.colsum_off[i] = off;
    off += 2 * static_cast<size_t>(splits) * probs[i].out_features;
    off = (off + 63) & ~static_cast<size_t>(63);
  }
  plan.total_floats = off;
  return plan;
}

// Input-grad workspace: one w^T per problem, [in, round4(out)], 256-byte aligned.
size_t dx_plan(const ppo_linear_bwd_dx_problem* probs, int count, size_t* offs) {
  size_t off = 0;
  for (int i = 0; i < count; ++i) {
    if (offs) offs[i] = off;
    off += static_cast<size_t>(probs[i].in_features) * round4(probs[i].out_features);
    off = (off + 63) & ~static_cast<size_t>(63);
  }
  return off;
}

// The persistent NT kernel when every problem of the launch meets its requirements (16-byte operands, whole
// k-slabs, 16-byte aligned outputs of a width divisible by 4 under 2 GiB, 16-byte aligned biases); PPO_EUNSUPPORTED
// otherwise, and the caller launches gemm_nt_kernel.
template <int BM, int BN, int BK, int OCC, int EPI>
int launch_nt_pipe(Group& g, int count, hipStream_t s, const char* name) {
  auto fits = [](const float* c, int64_t rows, int64_t ld) {
    return c == nullptr || (w16_ok(c, ld) && rows * ld * 4 < (int64_t(1) << 31));
  };
  for (int i = 0; i < count; ++i) {
    const Problem& p = g.p[i];
    if (!w16_ok(p.A, p.lda) || !w16_ok(p.B, p.ldb) || p.K % BK != 0 || p.N % 4 != 0) return PPO_EUNSUPPORTED;
    if (!fits(p.C, p.M, p.ldc) || (epi_fwd_act(EPI) && !fits(p.C2, p.M, p.ldc2))) return PPO_EUNSUPPORTED;
    if (epi_act_grad(EPI) && !w16_ok(p.aux, p.ldaux)) return PPO_EUNSUPPORTED;
    if ((EPI == EPI_BIAS || epi_fwd_act(EPI)) && reinterpret_cast<uintptr_t>(p.vec) % 16 != 0)
      return PPO_EUNSUPPORTED;
  }
  int tiles;
  if (int rc = assign_blocks(g, count, BM, BN, name, tiles)) return rc;
  if (tiles == 0) return PPO_OK;
  static std::atomic<int> cache[kMaxDevices];
  const int resident = resident_blocks(gemm_nt_pipe_kernel<BM, BN, BK, OCC, EPI>, cache);
  if (resident <= 0) return PPO_EUNSUPPORTED;
  hipLaunchKernelGGL((gemm_nt_pipe_kernel<BM, BN, BK, OCC, EPI>), dim3(std::min(tiles, resident)), dim3(kThreads), 0,
                     s, g, tiles);
  return check_launch(name);
}

// The bf16x6 NT kernel (fp32 accuracy on the bf16 matrix cores) when every problem of the launch meets its
// requirements (16-byte operands, whole 16-deep k-slabs, 16-byte aligned outputs of a width divisible by 4 under
// 2 GiB, 16-byte aligned biases / ELU' sources); PPO_EUNSUPPORTED otherwise.  128 x 128 output tiles in two LDS
// stages, three blocks per CU, four lanes per staged row: measured on MI355X in the 24,576-row humanoid update
// (ms per update, same box) 10.72 against 11.2 with three stages (two blocks per CU), 10.84 with two lanes per
// row and 11.4 with 128 x 64 tiles.  A PPO_HIP_TUNING build reads "PPO_HIP_BX6" = "bn[:stages[:four_lanes]]"
// (0: off).
template <int EPI, bool BKM = false>
int launch_nt_bx6(Group& g, int count, hipStream_t s, const char* name, bool bf16 = false) {
  auto fits = [](const float* c, int64_t rows, int64_t ld) {
    return c == nullptr || (w16_ok(c, ld) && rows * ld * 4 < (int64_t(1) << 31));
  };
  for (int i = 0; i < count; ++i) {
    const Problem& p = g.p[i];
    if (!w16_ok(p.A, p.lda) || !w16_ok(p.B, p.ldb) || p.K % 16 != 0 || p.N % 4 != 0) return PPO_EUNSUPPORTED;
    if (!fits(p.C, p.M, p.ldc) || (epi_fwd_act(EPI) && !fits(p.C2, p.M, p.ldc2))) return PPO_EUNSUPPORTED;
    if (epi_act_grad(EPI) && !w16_ok(p.aux, p.ldaux)) return PPO_EUNSUPPORTED;
    if ((EPI == EPI_BIAS || epi_fwd_act(EPI)) && reinterpret_cast<uintptr_t>(p.vec) % 16 != 0)
      return PPO_EUNSUPPORTED;
  }
  int bn = 128;
  [[maybe_unused]] int ns = 2, q4 = 1;
#ifdef PPO_HIP_TUNING
  if (const char* e = std::getenv("PPO_HIP_BX6")) {  // "bn[:ns[:q4]]"
    bn = std::atoi(e);
    if (const char* c = std::strchr(e, ':')) {
      ns = std::atoi(c + 1);
      if (const char* c2 = std::strchr(c + 1, ':')) q4 = std::atoi(c2 + 1);
    }
  }
  if ((bn != 64 && bn != 128) || (ns != 2 && ns != 3)) return PPO_EUNSUPPORTED;
  if (BKM && (bn != 128 || !q4 || ns != 2)) return PPO_EUNSUPPORTED;
  if (const char* e = std::getenv("PPO_HIP_BX6_KMAJOR"); BKM && e != nullptr && std::atoi(e) == 0)
    return PPO_EUNSUPPORTED;
#endif
  int blocks;
  if (int rc = assign_blocks(g, count, 128, bn, name, blocks)) return rc;
  if (blocks == 0) return PPO_OK;
#ifdef PPO_HIP_TUNING
  if (std::getenv("PPO_HIP_BX6") == nullptr)
#endif
  if (!BKM && 2 * blocks <= 3 * device_info().cus) {
    // 128 x 128 tiles would fill at most half of the three blocks per CU (a 128-wide output of a 24,576-row
    // mini-batch: 384 tiles): 128 x 64 tiles, twice as many blocks (humanoid fwd2 32.2 -> 31.3 us)
    bn = 64;
    if (int rc = assign_blocks(g, count, 128, bn, name, blocks)) return rc;
  }
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kThreads), 0, s, g);
    return check_launch(name);
  };
  if (bf16) {  // the bf16-operand mode: one product per k-group, the default tiles
    if constexpr (BKM) return go(gemm_nt_bx6_kernel<128, 3, EPI, 2, true, true, true>);
    if (bn == 64) return go(gemm_nt_bx6_kernel<64, 3, EPI, 2, true, false, true>);
    return go(gemm_nt_bx6_kernel<128, 3, EPI, 2, true, false, true>);
  }
  if constexpr (BKM) return go(gemm_nt_bx6_kernel<128, 3, EPI, 2, true, true>);
#ifdef PPO_HIP_TUNING
  if (bn == 64 || ns == 3 || !q4) {
    if (bn == 64 && ns == 2) return q4 ? go(gemm_nt_bx6_kernel<64, 3, EPI, 2, true>) : go(gemm_nt_bx6_kernel<64, 3, EPI, 2, false>);
    if (bn == 64) return q4 ? go(gemm_nt_bx6_kernel<64, 2, EPI, 3, true>) : go(gemm_nt_bx6_kernel<64, 2, EPI, 3, false>);
    if (ns == 3) return q4 ? go(gemm_nt_bx6_kernel<128, 2, EPI, 3, true>) : go(gemm_nt_bx6_kernel<128, 2, EPI, 3, false>);
    return go(gemm_nt_bx6_kernel<128, 3, EPI, 2, false>);
  }
#endif
  // two LDS stages (48 KiB with 128 x 128 tiles): three blocks per CU
  if (bn == 64) return go(gemm_nt_bx6_kernel<64, 3, EPI, 2, true>);
  return go(gemm_nt_bx6_kernel<128, 3, EPI, 2, true>);
}

// Tile of the persistent NT launches: 0 = none (gemm_nt_kernel only).  A PPO_HIP_TUNING build reads `var`
// (0 = off, 1..) for sweeps.
int pipe_tile(const char* var, int dflt) {
#ifdef PPO_HIP_TUNING
  if (const char* e = std::getenv(var)) return std::atoi(e);
#else
  (void)var;
#endif
  return dflt;
}

template <int EPI>
int launch_nt_pipe_tile(int t, Group& g, int count, hipStream_t s, const char* name) {
  switch (t) {
    case 1:  // (its ELU'-source registers would not fit 3 blocks per CU: not for the input-grads)
      if constexpr (epi_act_grad(EPI)) {
        return PPO_EUNSUPPORTED;
      } else {
        return launch_nt_pipe<128, 128, 16, 3, EPI>(g, count, s, name);
      }
    case 2:
      return launch_nt_pipe<128, 64, 16, 3, EPI>(g, count, s, name);
    case 3:
      return launch_nt_pipe<64, 64, 16, 4, EPI>(g, count, s, name);
#ifdef PPO_HIP_TUNING
    case 4:
      return launch_nt_pipe<64, 64, 32, 3, EPI>(g, count, s, name);
    case 5:
      if constexpr (epi_act_grad(EPI)) {
        return PPO_EUNSUPPORTED;
      } else {
        return launch_nt_pipe<128, 128, 32, 2, EPI>(g, count, s, name);
      }
    case 6:
      return launch_nt_pipe<128, 64, 32, 2, EPI>(g, count, s, name);
    case 7:
      return launch_nt_pipe<128, 128, 16, 2, EPI>(g, count, s, name);
    case 8:
      return launch_nt_pipe<128, 64, 16, 4, EPI>(g, count, s, name);
    case 9:
      return launch_nt_pipe<64, 128, 16, 4, EPI>(g, count, s, name);
    case 10:
      return launch_nt_pipe<64, 64, 16, 3, EPI>(g, count, s, name);
#endif
    default:
      return PPO_EUNSUPPORTED;
  }
}

bool rows_ok(int64_t rows) { return rows > 0 && rows <= INT32_MAX / 2; }

// The kernels address an NT operand with 32-bit byte offsets from its first element.
bool span_ok(int64_t rows, int64_t ld) { return rows * ld < (int64_t(1) << 30); }

}  // namespace
}  // namespace ppo

using namespace ppo;

namespace ppo {
namespace {

bool flags_ok(int32_t flags) { return (flags & ~PPO_GEMM_BF16_OPERANDS) == 0; }

}  // namespace
}  // namespace ppo

extern "C" int ppo_linear_fwd(const ppo_linear_fwd_problem* problems, int32_t count, int64_t rows, int32_t activation,
                              ppo_stream_t stream) {
  return ppo_linear_fwd_ex(problems, count, rows, activation, 0, stream);
}

extern "C" int ppo_linear_fwd_ex(const ppo_linear_fwd_problem* problems, int32_t count, int64_t rows,
                                 int32_t activation, int32_t flags, ppo_stream_t stream) {
  PPO_REQUIRE(flags_ok(flags), "ppo_linear_fwd: flags=%d", flags);
  const bool bf16 = (flags & PPO_GEMM_BF16_OPERANDS) != 0;
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LINEAR_PROBLEMS,
              "ppo_linear_fwd: count=%d outside [1, %d]", count, PPO_MAX_LINEAR_PROBLEMS);
  PPO_REQUIRE(rows_ok(rows), "ppo_linear_fwd: rows=%lld", (long long)rows);
  PPO_REQUIRE(activation >= PPO_ACT_NONE && activation < PPO_ACT_COUNT, "ppo_linear_fwd: activation=%d", activation);
  const bool elu = activation != PPO_ACT_NONE;  // (any activation: the bias + activation epilogue)
  Group g{};
  int max_n = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_linear_fwd_problem& q = problems[i];
    PPO_REQUIRE(q.x && q.w && q.b && (q.z || (elu && q.h)), "ppo_linear_fwd: problem %d has a null pointer", i);
    PPO_REQUIRE(q.in_features > 0 && q.out_features > 0, "ppo_linear_fwd: problem %d features", i);
    PPO_REQUIRE(q.ldx >= q.in_features && (q.z == nullptr || q.ldz >= q.out_features) &&
                    (!elu || q.h == nullptr || q.ldh >= q.out_features),
                "ppo_linear_fwd: problem %d leading dims", i);
    PPO_REQUIRE(span_ok(rows, q.ldx) && span_ok(q.out_features, q.in_features),
                "ppo_linear_fwd: problem %d: an operand spans 4 GiB or more", i);
    Problem& p = g.p[i];
    p.A = q.x; p.lda = q.ldx;
    p.B = q.w; p.ldb = q.in_features;
    p.C = q.z; p.ldc = q.ldz;
    p.C2 = q.h; p.ldc2 = q.ldh;
    p.vec = q.b;
    p.M = static_cast<int>(rows); p.N = q.out_features; p.K = q.in_features;
    p.splits = 1; p.k_chunk = q.in_features;
    p.c_vec = (q.z == nullptr || w16_ok(q.z, q.ldz)) && (!elu || q.h == nullptr || w16_ok(q.h, q.ldh));
    if (!elu) p.C2 = nullptr;
    p.act = activation;
    max_n = std::max(max_n, q.out_features);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  // measured on MI355X for 24576-row mini-batches: outputs wider than 128 like 128x128 tiles with 16-deep slabs,
  // narrower ones 128x64
  auto run = [&](auto epi_c, const char* name) {
    constexpr int EPI = decltype(epi_c)::value;
    const int brc = launch_nt_bx6<EPI>(g, count, s, name, bf16);
    if (brc != PPO_EUNSUPPORTED) return brc;
    const int prc = launch_nt_pipe_tile<EPI>(pipe_tile("PPO_HIP_PIPE_FWD", max_n > 128 ? 1 : 2), g, count, s, name);
    if (prc != PPO_EUNSUPPORTED) return prc;
    return launch_nt_tile<EPI>(pick_tile(max_n > 128 ? T128x128k16s2o3 : T128x64k32s2o4), g, count, s, name);
  };
  if (!elu) return run(IntC<EPI_BIAS>{}, "linear_fwd");
  if (activation == PPO_ACT_ELU) return run(IntC<EPI_BIAS_ELU>{}, "linear_fwd_elu");
  return run(IntC<EPI_BIAS_ACT>{}, "linear_fwd_act");
}

extern "C" size_t ppo_linear_bwd_dx_workspace_bytes(const ppo_linear_bwd_dx_problem* problems, int32_t count) {
  if (problems == nullptr || count < 1 || count > PPO_MAX_LINEAR_PROBLEMS) return 0;
  for (int i = 0; i < count; ++i)
    if (problems[i].in_features <= 0 || problems[i].out_features <= 0) return 0;
  return dx_plan(problems, count, nullptr) * sizeof(float);
}

namespace ppo {
namespace {

int check_dx_workspace(const ppo_linear_bwd_dx_problem* problems, int count, void* workspace, size_t workspace_bytes,
                       size_t* offs, const char* who) {
  const size_t need = dx_plan(problems, count, offs) * sizeof(float);
  PPO_REQUIRE(workspace != nullptr && workspace_bytes >= need, "%s: workspace too small (%zu < %zu)", who,
              workspace_bytes, need);
  PPO_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "%s: workspace must be 16-byte aligned", who);
  return PPO_OK;
}

// w^T of every problem into its slot of the input-grad workspace ([in, round4(out)], dx_plan's offsets).
int launch_transposes(const ppo_linear_bwd_dx_problem* problems, int count, float* ws, const size_t* offs,
                      hipStream_t s) {
  TransposeGroup tg{};
  int tblocks = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_linear_bwd_dx_problem& q = problems[i];
    TransposeItem& T = tg.it[i];
    T.w = q.w; T.wt = ws + offs[i]; T.out = q.out_features; T.in = q.in_features;
    T.ldt = static_cast<int>(round4(q.out_features));
    T.tiles_in = static_cast<int>(ceil_div(q.in_features, 32));
    T.block_begin = tblocks;
    tblocks += static_cast<int>(ceil_div(T.ldt, 32)) * T.tiles_in;
  }
  for (int i = count; i < PPO_MAX_LINEAR_PROBLEMS; ++i) tg.it[i].block_begin = INT32_MAX;
  tg.count = count;
  hipLaunchKernelGGL(transpose_kernel, dim3(tblocks), dim3(256), 0, s, tg);
  return check_launch("transpose_kernel");
}

// w^T of every problem into the workspace, then the input-grad GEMMs on those copies.
// act' can be evaluated from the activation's output (monotone activations: the output determines the input)
bool act_from_output_ok(int act) {
  return act == PPO_ACT_ELU || act == PPO_ACT_SELU || act == PPO_ACT_RELU || act == PPO_ACT_CELU ||
         act == PPO_ACT_LRELU || act == PPO_ACT_TANH || act == PPO_ACT_SIGMOID || act == PPO_ACT_IDENTITY;
}

int dx_gemm(const ppo_linear_bwd_dx_problem* problems, int32_t count, int64_t rows, int32_t activation,
            int32_t elu_source, void* workspace, size_t workspace_bytes, ppo_stream_t stream, const char* who,
            int32_t flags = 0) {
  PPO_REQUIRE(flags_ok(flags), "%s: flags=%d", who, flags);
  const bool bf16 = (flags & PPO_GEMM_BF16_OPERANDS) != 0;
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LINEAR_PROBLEMS, "%s: count=%d outside [1, %d]",
              who, count, PPO_MAX_LINEAR_PROBLEMS);
  PPO_REQUIRE(activation > PPO_ACT_NONE && activation < PPO_ACT_COUNT, "%s: activation=%d", who, activation);
  PPO_REQUIRE(elu_source == PPO_ELU_FROM_INPUT || elu_source == PPO_ELU_FROM_OUTPUT, "%s: source=%d", who,
              elu_source);
  PPO_REQUIRE(elu_source == PPO_ELU_FROM_INPUT || act_from_output_ok(activation),
              "%s: activation %d: its derivative needs the activation's input (source PPO_ELU_FROM_INPUT)", who,
              activation);
  PPO_REQUIRE(rows_ok(rows), "%s: rows=%lld", who, (long long)rows);
  bool any_act = false, any_plain = false;
  for (int i = 0; i < count; ++i) {
    const ppo_linear_bwd_dx_problem& q = problems[i];
    PPO_REQUIRE(q.dz && q.w && q.dz_prev, "%s: problem %d has a null pointer", who, i);
    PPO_REQUIRE(q.in_features > 0 && q.out_features > 0, "%s: problem %d features", who, i);
    PPO_REQUIRE(q.lddz >= q.out_features && q.lddz_prev >= q.in_features &&
                    (q.z_prev == nullptr || q.ldz_prev >= q.in_features),
                "%s: problem %d leading dims", who, i);
    PPO_REQUIRE(span_ok(rows, q.lddz) && span_ok(q.in_features, (q.out_features + 3) / 4 * 4),
                "%s: problem %d: an operand spans 4 GiB or more", who, i);
    (q.z_prev ? any_act : any_plain) = true;
  }
  PPO_REQUIRE(!(any_act && any_plain), "%s: mix of activation and plain problems in one call", who);
  size_t offs[PPO_MAX_LINEAR_PROBLEMS];
  if (int rc = check_dx_workspace(problems, count, workspace, workspace_bytes, offs, who)) return rc;
  float* ws = static_cast<float*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  Group g{};
  int max_n = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_linear_bwd_dx_problem& q = problems[i];
    Problem& p = g.p[i];
    p.A = q.dz; p.lda = q.lddz;
    p.B = q.w; p.ldb = q.in_features;
    p.C = q.dz_prev; p.ldc = q.lddz_prev;
    p.aux = q.z_prev; p.ldaux = q.ldz_prev;
    p.M = static_cast<int>(rows); p.N = q.in_features; p.K = q.out_features;
    p.splits = 1; p.k_chunk = q.out_features;
    p.c_vec = w16_ok(q.dz_prev, q.lddz_prev) && (q.z_prev == nullptr || w16_ok(q.z_prev, q.ldz_prev));
    p.elu_from_output = elu_source == PPO_ELU_FROM_OUTPUT;
    p.act = activation;
    max_n = std::max(max_n, q.in_features);
  }
  auto run = [&](auto epi_c, const char* name) {
    constexpr int EPI = decltype(epi_c)::value;
    // the bf16x6 kernel reads the weights as stored (k-major, 16-byte rows): no transpose
    const int krc = launch_nt_bx6<EPI, true>(g, count, s, name, bf16);
    if (krc != PPO_EUNSUPPORTED) return krc;
    // else w^T (k-contiguous) into the workspace for the other kernels
    if (int rc = launch_transposes(problems, count, ws, offs, s)) return rc;
    for (int i = 0; i < count; ++i) {
      g.p[i].B = ws + offs[i];
      g.p[i].ldb = round4(problems[i].out_features);
    }
    const int brc = launch_nt_bx6<EPI>(g, count, s, name, bf16);
    if (brc != PPO_EUNSUPPORTED) return brc;
    // measured on MI355X: 64x64 tiles for the 256..512-wide input grads, 128x64 for narrower ones
    const int prc = launch_nt_pipe_tile<EPI>(pipe_tile("PPO_HIP_PIPE_DX", max_n > 128 ? 3 : 2), g, count, s, name);
    if (prc != PPO_EUNSUPPORTED) return prc;
    return launch_nt_tile<EPI>(pick_tile(max_n > 128 ? T64x64k32s2o4 : T128x64k32s2o4), g, count, s, name);
  };
  if (!any_act) return run(IntC<EPI_STORE>{}, "linear_bwd_dx");
  if (activation == PPO_ACT_ELU) return run(IntC<EPI_ELU_GRAD>{}, "linear_bwd_dx_elu");
  return run(IntC<EPI_ACT_GRAD>{}, "linear_bwd_dx_act");
}

}  // namespace
}  // namespace ppo

extern "C" int ppo_linear_bwd_dx(const ppo_linear_bwd_dx_problem* problems, int32_t count, int64_t rows,
                                 int32_t elu_source, void* workspace, size_t workspace_bytes, ppo_stream_t stream) {
  return dx_gemm(problems, count, rows, PPO_ACT_ELU, elu_source, workspace, workspace_bytes, stream,
                 "ppo_linear_bwd_dx");
}

extern "C" int ppo_linear_bwd_dx_act(const ppo_linear_bwd_dx_problem* problems, int32_t count, int64_t rows,
                                     int32_t activation, int32_t source, void* workspace, size_t workspace_bytes,
                                     ppo_stream_t stream) {
  return dx_gemm(problems, count, rows, activation, source, workspace, workspace_bytes, stream,
                 "ppo_linear_bwd_dx_act");
}

extern "C" int ppo_linear_bwd_dx_ex(const ppo_linear_bwd_dx_problem* problems, int32_t count, int64_t rows,
                                    int32_t activation, int32_t source, int32_t flags, void* workspace,
                                    size_t workspace_bytes, ppo_stream_t stream) {
  return dx_gemm(problems, count, rows, activation, source, workspace, workspace_bytes, stream,
                 "ppo_linear_bwd_dx_ex", flags);
}

extern "C" size_t ppo_linear_bwd_dw_workspace_bytes(const ppo_linear_bwd_dw_problem* problems, int32_t count,
                                                    int64_t rows) {
  if (problems == nullptr || count < 1 || count > PPO_MAX_LINEAR_PROBLEMS || !rows_ok(rows)) return 0;
  for (int i = 0; i < count; ++i)
    if (problems[i].in_features <= 0 || problems[i].out_features <= 0) return 0;
  return plan_dw(problems, count, rows, dw_query_capacity()).total_floats * sizeof(float);
}

namespace ppo {
namespace {

int dw_gemm(const ppo_linear_bwd_dw_problem* problems, int32_t count, int64_t rows, void* workspace,
            size_t workspace_bytes, const float* extra_grads, const ppo_grad_range* extra, int32_t num_extra,
            double* norm, ppo_stream_t stream, int32_t flags = 0) {
  PPO_REQUIRE(flags_ok(flags), "ppo_linear_bwd_dw: flags=%d", flags);
  const bool bf16 = (flags & PPO_GEMM_BF16_OPERANDS) != 0;
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LINEAR_PROBLEMS,
              "ppo_linear_bwd_dw: count=%d outside [1, %d]", count, PPO_MAX_LINEAR_PROBLEMS);
  PPO_REQUIRE(rows_ok(rows), "ppo_linear_bwd_dw: rows=%lld", (long long)rows);
  for (int i = 0; i < count; ++i) {
    const ppo_linear_bwd_dw_problem& q = problems[i];
    PPO_REQUIRE(q.dz && q.x && q.dw, "ppo_linear_bwd_dw: problem %d has a null pointer", i);
    PPO_REQUIRE(q.in_features > 0 && q.out_features > 0, "ppo_linear_bwd_dw: problem %d features", i);
    PPO_REQUIRE(q.lddz >= q.out_features && q.ldx >= q.in_features, "ppo_linear_bwd_dw: problem %d leading dims", i);
    PPO_REQUIRE(static_cast<int64_t>(q.out_features) * (round4(q.in_features) + 4) < (int64_t(1) << 31),
                "ppo_linear_bwd_dw: problem %d: weight of %d x %d is too large", i, q.out_features, q.in_features);
    PPO_REQUIRE(q.grad_norm_group >= 0 && q.grad_norm_group <= PPO_MAX_PARAM_GROUPS,
                "ppo_linear_bwd_dw: problem %d: grad_norm_group %d outside [0, %d]", i, q.grad_norm_group,
                PPO_MAX_PARAM_GROUPS);
  }
  PPO_REQUIRE(num_extra >= 0 && num_extra <= PPO_MAX_EXTRA_GRADS && (num_extra == 0 || (extra && extra_grads)),
              "ppo_linear_bwd_dw_norm: %d extra gradient ranges (at most %d, with their buffer)", num_extra,
              PPO_MAX_EXTRA_GRADS);
  for (int r = 0; r < num_extra; ++r)
    PPO_REQUIRE(extra[r].begin >= 0 && extra[r].end >= extra[r].begin && extra[r].group >= 0 &&
                    extra[r].group < PPO_MAX_PARAM_GROUPS,
                "ppo_linear_bwd_dw_norm: extra range %d malformed", r);
  // the bf16x6 kernel takes operands with 16-byte rows (the fp32 kernel the rest, at fewer blocks per CU)
  bool bx6 = true;
  for (int i = 0; i < count; ++i)
    bx6 = bx6 && w16_ok(problems[i].dz, problems[i].lddz) && w16_ok(problems[i].x, problems[i].ldx);
  int occ = bx6 ? kDwBlocksPerCu : kDwF32BlocksPerCu;
#ifdef PPO_HIP_TUNING
  const char* cfg = std::getenv("PPO_HIP_DW_CFG");  // tuning aid: other slab depths / stages / occupancies
  if (cfg && !std::strcmp(cfg, "bx6o2")) occ = 2;
  if (cfg && std::strcmp(cfg, "bx6o2") && std::strcmp(cfg, "bx6")) {
    bx6 = false;
    occ = cfg[std::strlen(cfg) - 1] - '0';
  }
#endif
  const DwPlan plan = plan_dw(problems, count, rows, dw_launch_capacity(occ));
  PPO_REQUIRE(workspace != nullptr && workspace_bytes >= plan.total_floats * sizeof(float),
              "ppo_linear_bwd_dw: workspace too small (%zu < %zu)", workspace_bytes,
              plan.total_floats * sizeof(float));
  PPO_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "ppo_linear_bwd_dw: workspace must be 16-byte aligned");
  float* ws = static_cast<float*>(workspace);
  Group g{};
  ReduceGroup rg{};
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_linear_bwd_dw_problem& q = problems[i];
    Problem& p = g.p[i];
    const int64_t ldp = round4(q.in_features);
    p.A = q.dz; p.lda = q.lddz;
    p.B = q.x; p.ldb = q.ldx;
    p.C = ws + plan.partial_off[i]; p.ldc = ldp;
    p.partial_stride = static_cast<int64_t>(q.out_features) * ldp;
    p.colsum = q.db != nullptr ? reinterpret_cast<double*>(ws + plan.colsum_off[i]) : nullptr;
    p.M = q.out_features; p.N = q.in_features; p.K = static_cast<int>(rows);
    p.splits = plan.splits[i]; p.k_chunk = plan.k_chunk[i];
    ReduceItem& r = rg.it[i];
    r.partial = p.C; r.colsum = p.colsum; r.dw = q.dw; r.db = q.db;
    r.out = q.out_features; r.in = q.in_features; r.ld = static_cast<int>(ldp); r.splits = plan.splits[i];
    r.stride = p.partial_stride;
    r.group = norm != nullptr ? q.grad_norm_group : 0;
    r.begin = total;
    total += static_cast<int64_t>(q.out_features) * (ldp / 4 + (q.db != nullptr ? 1 : 0));
  }
  for (int i = count; i < PPO_MAX_LINEAR_PROBLEMS; ++i) rg.it[i].begin = INT64_MAX;
  rg.count = count;
  rg.total = total;
  rg.norm = norm;
  rg.extra_grads = extra_grads;
  for (int r = 0; r < num_extra; ++r) rg.extra[r] = extra[r];
  rg.num_extra = num_extra;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc;
#ifdef PPO_HIP_TUNING
  if (cfg && !std::strcmp(cfg, "bk16s2o3")) {
    rc = launch_tn<kDwBM, kDwBN, 16, 2, 3>(g, count, s, "linear_bwd_dw");
  } else if (cfg && !std::strcmp(cfg, "bk16s3o3")) {
    rc = launch_tn<kDwBM, kDwBN, 16, 3, 3>(g, count, s, "linear_bwd_dw");
  } else if (cfg && !std::strcmp(cfg, "bk32s2o1")) {
    rc = launch_tn<kDwBM, kDwBN, 32, 2, 1>(g, count, s, "linear_bwd_dw");
  } else if (cfg && !std::strcmp(cfg, "bk16s4o2")) {
    rc = launch_tn<kDwBM, kDwBN, 16, 4, 2>(g, count, s, "linear_bwd_dw");
  } else if (cfg && !std::strcmp(cfg, "f32o2")) {
    rc = launch_tn<kDwBM, kDwBN, 32, 2, 2>(g, count, s, "linear_bwd_dw");
  } else if (bx6 && occ == 2) {
    rc = launch_tn_bx6<2>(g, count, s, "linear_bwd_dw");
  } else
#endif
  if (bx6) {
    rc = launch_tn_bx6<kDwBlocksPerCu>(g, count, s, "linear_bwd_dw", bf16);
  } else {
    rc = launch_tn<kDwBM, kDwBN, 32, 2, kDwF32BlocksPerCu>(g, count, s, "linear_bwd_dw");
  }
  if (rc != PPO_OK) return rc;
  if (norm != nullptr && total > PPO_DW_NORM_BLOCKS * 256) {
    // the norm rows fix the block count: wider blocks keep one work item per thread (the LSTMs' weight-grads)
    hipLaunchKernelGGL(dw_reduce_kernel<1024>, dim3(PPO_DW_NORM_BLOCKS), dim3(1024), 0, s, rg);
  } else {
    const int64_t blocks = norm != nullptr ? PPO_DW_NORM_BLOCKS : std::min<int64_t>(ceil_div(total, 256), 4096);
    hipLaunchKernelGGL(dw_reduce_kernel<256>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, rg);
  }
  return check_launch("dw_reduce_kernel");
}

}  // namespace
}  // namespace ppo

extern "C" int ppo_linear_bwd_dw(const ppo_linear_bwd_dw_problem* problems, int32_t count, int64_t rows,
                                 void* workspace, size_t workspace_bytes, ppo_stream_t stream) {
  return dw_gemm(problems, count, rows, workspace, workspace_bytes, nullptr, nullptr, 0, nullptr, stream);
}

extern "C" int ppo_linear_bwd_dw_norm(const ppo_linear_bwd_dw_problem* problems, int32_t count, int64_t rows,
                                      void* workspace, size_t workspace_bytes, const float* extra_grads,
                                      const ppo_grad_range* extra, int32_t num_extra, double* norm_partials,
                                      ppo_stream_t stream) {
  PPO_REQUIRE(norm_partials != nullptr, "ppo_linear_bwd_dw_norm: null norm_partials");
  return dw_gemm(problems, count, rows, workspace, workspace_bytes, extra_grads, extra, num_extra, norm_partials,
                 stream);
}

extern "C" int ppo_linear_bwd_dw_ex(const ppo_linear_bwd_dw_problem* problems, int32_t count, int64_t rows,
                                    int32_t flags, void* workspace, size_t workspace_bytes, const float* extra_grads,
                                    const ppo_grad_range* extra, int32_t num_extra, double* norm_partials,
                                    ppo_stream_t stream) {
  PPO_REQUIRE(norm_partials != nullptr || num_extra == 0, "ppo_linear_bwd_dw_ex: extra ranges need norm_partials");
  return dw_gemm(problems, count, rows, workspace, workspace_bytes, extra_grads, extra, num_extra, norm_partials,
                 stream, flags);
}
