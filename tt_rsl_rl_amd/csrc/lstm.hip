// A15 LSTM of the recurrent models (torch nn.LSTM; rsl_rl/modules/rnn.py:22-86) on gfx950.  Every entry point
// works on one layer; stacked layers are run one after another by the caller (layer k's input = layer k-1's h).
//
// The input projection x w_ih^T + b of all T steps is one GEMM (ppo_linear_fwd on the gate-interleaved weights), or,
// for inputs of at most 64 columns, part of the whole-sequence forward launch (ppo_lstm_seq_fwd_proj).
// The recurrence is one kernel per step: the NT GEMM of gemm_core.hpp computes hs[t] w_hh_g^T (rows = envs,
// columns = gates of 4 hidden units per 16-byte group) and its LSTM epilogue applies the cell equations
// (i, f, o = sigmoid, g = tanh; c_t = f c_{t-1} + i g; h_t = o tanh(c_t)), writing the activations for the backward
// and the next step's operand hs[t+1] = h_t * keep_t.  The backward step computes dgates[t+1] w_hh_g (rows = envs,
// columns = hidden units) and its epilogue applies the cell derivatives, carrying dL/dc to the previous step.
// Actor and critic share every launch.  The two weight gradients are plain split-K GEMMs over all T*E rows
// (ppo_linear_bwd_dw: dgates^T hs and dgates^T x).
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "gemm_core.hpp"

namespace ppo {
namespace {

struct PackItem {
  const float* w_ih;
  const float* w_hh;
  const float* b_ih;
  const float* b_hh;
  float* w_ih_g;
  float* w_hh_g;
  float* w_hh_gt;
  float* b_g;
  int64_t D, H, begin;  // begin: first flat element of this problem in the launch
  int32_t gru;          // torch nn.GRU weights (r, z, n) into the four-slot layout of gru_cell_fwd
};
struct PackGroup {
  PackItem it[PPO_MAX_LSTM_PROBLEMS];
  int32_t count;
  int64_t total;
};

// Flat element e of a problem: [0, 4HD) w_ih_g, [.., +4HH) w_hh_g, [.., +4HH) w_hh_gt, [.., +4H) b_g; each output
// element is written by exactly one thread (reads are gathers from the torch layout).  32-bit index arithmetic (the
// host checks that a launch has fewer than 2^31 elements): a 64-bit division is a long subroutine per element.
__global__ __launch_bounds__(256) void lstm_pack_kernel(const PackGroup g) {
  const uint32_t total = static_cast<uint32_t>(g.total), b1 = static_cast<uint32_t>(g.it[1].begin);
  for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const PackItem& P = g.it[(g.count > 1 && e >= b1) ? 1 : 0];
    uint32_t k = e - static_cast<uint32_t>(P.begin);
    const uint32_t H = static_cast<uint32_t>(P.H), D = static_cast<uint32_t>(P.D), G = 4 * H;
    // torch gate of slot q (-1: a zero row).  LSTM: slot q = gate q (i, f, g, o) of both weights.  GRU: slots r, z
    // of both weights, slot 2 = n of w_hh only, slot 3 = n of w_ih only.
    auto gate_ih = [&](uint32_t q) -> int { return P.gru ? (q < 2 ? static_cast<int>(q) : q == 3 ? 2 : -1) : static_cast<int>(q); };
    auto gate_hh = [&](uint32_t q) -> int { return P.gru ? (q < 3 ? static_cast<int>(q) : -1) : static_cast<int>(q); };
    if (k < G * D) {  // w_ih_g[4u+q][d] = w_ih[gate(q) H + u][d]
      const uint32_t n = k / D, d = k - n * D;
      const int q = gate_ih(n & 3);
      P.w_ih_g[k] = q < 0 ? 0.0f : P.w_ih[(q * H + (n >> 2)) * D + d];
      continue;
    }
    k -= G * D;
    if (k < G * H) {  // w_hh_g[4u+q][j] = w_hh[gate(q) H + u][j]
      const uint32_t n = k / H, j = k - n * H;
      const int q = gate_hh(n & 3);
      P.w_hh_g[k] = q < 0 ? 0.0f : P.w_hh[(q * H + (n >> 2)) * H + j];
      continue;
    }
    k -= G * H;
    if (k < G * H) {  // w_hh_gt[j][4u+q] = w_hh_g[4u+q][j]
      const uint32_t j = k / G, n = k - j * G;
      const int q = gate_hh(n & 3);
      P.w_hh_gt[k] = q < 0 ? 0.0f : P.w_hh[(q * H + (n >> 2)) * H + j];
      continue;
    }
    k -= G * H;  // b_g[4u+q] = b_ih[gate_ih(q) H + u] + b_hh[gate_hh(q) H + u] (a missing gate adds nothing)
    const uint32_t u = k >> 2;
    const int qi = gate_ih(k & 3), qh = gate_hh(k & 3);
    if (qi >= 0 && qh >= 0) {
      P.b_g[k] = P.b_ih[qi * H + u] + P.b_hh[qh * H + u];
    } else {
      P.b_g[k] = qi >= 0 ? P.b_ih[qi * H + u] : P.b_hh[qh * H + u];
    }
  }
}

struct GradItem {
  const float* dw_ih_g;
  const float* dw_hh_g;
  const float* db_g;
  float* dw_ih;
  float* dw_hh;
  float* db_ih;
  float* db_hh;
  int64_t D, H, begin;
  int32_t gru;  // torch nn.GRU layout ([3H, D], [3H, H], [3H]) from the four-slot layout of gru_cell_fwd
};
struct GradGroup {
  GradItem it[PPO_MAX_LSTM_PROBLEMS];
  int32_t count;
  int64_t total;
  double* norm;                          // NORM: [PPO_DW_NORM_BLOCKS][PPO_MAX_PARAM_GROUPS] partial rows, added to
  int32_t group[PPO_MAX_LSTM_PROBLEMS];  // problem i's parameter group
};

// Flat element e of a problem: [0, GD) dw_ih, [.., +GH) dw_hh, [.., +G) db_ih and db_hh (torch layout, written once
// each; G = 4H rows for the LSTM, 3H for the GRU).  The LSTM's bias gradient goes to both b_ih and b_hh; the GRU's n
// gate has separate input and hidden biases (slots 3 and 2).
//
// NORM: the launch has at most PPO_DW_NORM_BLOCKS blocks and block b adds the fp64 sums of squares of the values it
// wrote (per problem: the thread's elements in order, then a fixed-order block reduction) to row b of the partials
// the weight-gradient launch before it wrote (problem 0's sum first, then problem 1's), so the optimiser's clip norms
// cover the torch-layout gradients (each bias gradient of an LSTM counted for both b_ih and b_hh, as torch sees them).
template <bool NORM, int THREADS = 256>
__global__ __launch_bounds__(THREADS) void lstm_unpack_kernel(const GradGroup g) {
  const uint32_t total = static_cast<uint32_t>(g.total), b1 = static_cast<uint32_t>(g.it[1].begin);
  double sq[PPO_MAX_LSTM_PROBLEMS] = {};
  for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const int pi = (g.count > 1 && e >= b1) ? 1 : 0;
    const GradItem& P = g.it[pi];
    auto put = [&](float* dst, float v) {
      *dst = v;
      if constexpr (NORM) {
        const double x = static_cast<double>(v) * v;
        if (pi == 0) sq[0] += x; else sq[1] += x;
      }
    };
    uint32_t k = e - static_cast<uint32_t>(P.begin);
    const uint32_t H = static_cast<uint32_t>(P.H), D = static_cast<uint32_t>(P.D), G = (P.gru ? 3 : 4) * H;
    // torch row r = q H + u -> interleaved row 4u + slot
    auto slot_ih = [&](uint32_t r) -> uint32_t {
      const uint32_t q = r / H;
      return 4 * (r - q * H) + (P.gru && q == 2 ? 3 : q);
    };
    auto slot_hh = [&](uint32_t r) -> uint32_t {
      const uint32_t q = r / H;
      return 4 * (r - q * H) + q;
    };
    if (k < G * D) {
      const uint32_t r = k / D, d = k - r * D;
      put(P.dw_ih + k, P.dw_ih_g[slot_ih(r) * D + d]);
      continue;
    }
    k -= G * D;
    if (k < G * H) {
      const uint32_t r = k / H, j = k - r * H;
      put(P.dw_hh + k, P.dw_hh_g[slot_hh(r) * H + j]);
      continue;
    }
    k -= G * H;
    put(P.db_ih + k, P.db_g[slot_ih(k)]);
    put(P.db_hh + k, P.db_g[slot_hh(k)]);
  }
  if constexpr (NORM) {
    __shared__ double red[THREADS / 64][PPO_MAX_LSTM_PROBLEMS];
#pragma unroll
    for (int p = 0; p < PPO_MAX_LSTM_PROBLEMS; ++p) {
      double x = sq[p];
      for (int off = 32; off > 0; off >>= 1) x += __shfl_down(x, off, 64);
      if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6][p] = x;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      double* row = g.norm + static_cast<int64_t>(blockIdx.x) * PPO_MAX_PARAM_GROUPS;
      for (int p = 0; p < g.count; ++p) {
        double x = 0.0;
        for (int w = 0; w < THREADS / 64; ++w) x += red[w][p];
        row[g.group[p]] += x;
      }
    }
  }
}

// hs[0] = h0 for every problem (rows E, H floats each); with a sync buffer, block 0 also clears its words 1 ..
// sync_words - 1 for the whole-sequence launch that follows (the status word 0 stays).
struct CopyItem {
  const float* src;
  float* dst;
  int64_t ld_src, begin;
};
struct CopyGroup {
  CopyItem it[PPO_MAX_LSTM_PROBLEMS];
  int32_t count;
  int64_t H, total;
  int32_t* sync;
  int32_t sync_words;
};

__global__ __launch_bounds__(256) void lstm_copy_state_kernel(const CopyGroup g) {
  if (g.sync != nullptr && blockIdx.x == 0)
    for (int i = 1 + threadIdx.x; i < g.sync_words; i += blockDim.x) g.sync[i] = 0;
  const uint32_t total = static_cast<uint32_t>(g.total), b1 = static_cast<uint32_t>(g.it[1].begin);
  const uint32_t H = static_cast<uint32_t>(g.H);
  for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const CopyItem& C = g.it[(g.count > 1 && e >= b1) ? 1 : 0];
    const uint32_t k = e - static_cast<uint32_t>(C.begin), row = k / H, col = k - row * H;
    C.dst[k] = C.src[static_cast<int64_t>(row) * C.ld_src + col];
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// ---- Whole-sequence forward: one launch for all T steps ----
//
// Block (problem p, row-group slot g, column block cb) holds gate columns [64 cb, 64 cb + 64) of w_hh_g (64 x H
// floats) in LDS for the whole sequence and computes rows [64 rg, 64 rg + 64) of every step, for rg = g, g + slots,
// ...  Step t of a row group reads hs[t] of its rows, which all ncb column blocks of that row group write at step
// t - 1.  hs[t + 1] is written and hs[t] read through the L2 of the XCD when all blocks of the row group run on it
// (the usual case, see writers_on_xcd), else with device-scope (sc1) accesses, which the XCDs' separate L2 caches
// keep coherent; neither needs a whole-cache write-back or invalidate.  After its stores have completed (vmcnt 0) a
// block adds 1 to the row group's counter (word 0 of the row group's 128-byte line), and before step t a block polls
// the counter until it reaches ncb t; after its last step a block counts out (seq_count_out), and the last block of
// the row group to do so zeroes the counter, so a call that completes leaves its counters at zero for the next call
// (the forward's state-copy launch clears them too).  The host sizes the grid to the blocks the device holds at once
// (occupancy query), so the peers of a row group are resident together.  A wait still gives up after kSeqSpinTicks of the 100 MHz real-time clock: it
// sets the sticky status word and the abort word, every block then leaves at its next wait, and the caller sees
// status != 0 (no hang).
//
// The MFMA sequence per accumulator (32-deep k slabs, k-groups of 8, element s of the f32x4 fragments) and the cell
// arithmetic are those of the per-step kernel on 64 x 64 tiles, so both paths give identical results.
//
// PROJ: the input projection gx = x w_ih_g^T + b_g of the lane's cell outputs is computed in the launch with the
// projection GEMM's own arithmetic (gemm_nt_bx6_kernel: each operand element split into three bf16 parts, or rounded
// to bf16 alone in the bf16-operand mode; the six products of a 16-deep k-slab in that kernel's order with the
// weights as the first operand, slabs in order, then + b_g), so gx is bit for bit what ppo_linear_fwd(_ex) writes.
// A step's x rows and the block's w_ih_g rows (L2-resident) are loaded at the top of the previous step, split and
// multiplied after that step's signal, in the time the row group's blocks take to see each other's counts.
constexpr int kSeqRows = 64, kSeqCols = 64, kSeqBK = 32;
constexpr int kSeqMaxSlabs = 8;  // H <= 256: the w_hh_g slice is 64 KB of LDS, two blocks per CU
constexpr int kSeqProjSlabs = 3;  // fused input projection: inputs of at most 3 16-deep k-slabs (48 columns)
constexpr int kSyncHeader = 32;  // int32 words ahead of the row-group lines: [0] status (sticky), [1] abort
constexpr int kSyncStride = 32;  // one 128-byte line per row group: [0] counter, [1 + j] XCD of block j
constexpr int kBufferWord3 = 0x00020000;  // raw buffer descriptor, 32-bit data (gfx9 family)
constexpr int kDeviceScope = 16;          // buffer-load cache policy: sc1, coherent at device scope
constexpr uint64_t kSeqSpinTicks = 200000000ull;  // 2 s of the 100 MHz clock (ppo_lstm_seq_wait_limit)

struct SeqFwdItem {
  const float* w;  // w_hh_g [4H, H]
  const float* gx;
  const float* x;    // fused projection: the layer input [T*E, D] (ld ldx), w_ih_g [4H, D], b_g [4H]
  const float* wih;
  const float* bg;
  int64_t ldx;
  int32_t kp;        // D / 16
  const float* c0;
  const float* keep;
  float* gates;
  float* c;
  float* h;
  float* hs;
  int64_t ldgx, ld0, keep_stride, ldh;
};
struct SeqFwdArgs {
  SeqFwdItem it[PPO_MAX_LSTM_PROBLEMS];
  int32_t* sync;
  uint64_t spin_ticks;
  int32_t H, E, T, nrg, ncb, slots;
  int32_t xcds;  // XCDs of the device (block b runs on XCD b % xcds)
  int32_t bf16;  // fused projection with bf16 operands (PPO_GEMM_BF16_OPERANDS)
};

// Waits until *ctr >= target; every thread of the block returns the same verdict (false: the sequence was aborted).
// `flag` is an LDS word that no wave touches between the previous workgroup barrier and this one.  The data the
// counter announces is read afterwards either through the L2 that all its writers share or with device-scope loads,
// so the poll needs no cache invalidate.
__device__ __forceinline__ bool seq_wait(int32_t* sync, int32_t* ctr, int target, volatile float* flag,
                                         uint64_t spin_ticks) {
  if (threadIdx.x == 0) {
    float ok = 1.0f;
    if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      const uint64_t t0 = wall_clock64();
      while (true) {
        __builtin_amdgcn_s_sleep(1);
        if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) break;
        if (__hip_atomic_load(sync + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
          ok = 0.0f;
          break;
        }
        if (wall_clock64() - t0 > spin_ticks) {
          __hip_atomic_store(sync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(sync + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = 0.0f;
          break;
        }
      }
    }
    *flag = ok;
  }
  __syncthreads();
  return *flag != 0.0f;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// x[q] belongs to unit 2q + hl of the lane's pair (lanes l and l + 32); returns units 4 hl .. 4 hl + 3 of the pair.
__device__ __forceinline__ f32x4 trade_halves(const float (&x)[4], int hl) {
  const float r0 = __shfl_xor(hl ? x[0] : x[2], 32), r1 = __shfl_xor(hl ? x[1] : x[3], 32);
  return hl ? f32x4{r0, x[2], r1, x[3]} : f32x4{x[0], r0, x[1], r1};
}

// Eight consecutive k of one MFMA operand row (v0: k 0..3, v1: k 4..7) as a 32x32x16 bf16 fragment in each of its
// three bf16 parts, split as the bf16x6 GEMMs' staging splits them (split_bf16x3 on consecutive pairs).
__device__ __forceinline__ void split_frag(const f32x4& v0, const f32x4& v1, bf16x8 (&part)[3]) {
  uint32_t h[4], m[4], l[4];
  split_bf16x3(v0[0], v0[1], h[0], m[0], l[0]);
  split_bf16x3(v0[2], v0[3], h[1], m[1], l[1]);
  split_bf16x3(v1[0], v1[1], h[2], m[2], l[2]);
  split_bf16x3(v1[2], v1[3], h[3], m[3], l[3]);
  part[0] = __builtin_bit_cast(bf16x8, u32x4{h[0], h[1], h[2], h[3]});
  part[1] = __builtin_bit_cast(bf16x8, u32x4{m[0], m[1], m[2], m[3]});
  part[2] = __builtin_bit_cast(bf16x8, u32x4{l[0], l[1], l[2], l[3]});
}

// This wave's XCD (accelerator complex die): the hardware register XCC_ID.
__device__ __forceinline__ int xcd_id() {
  int v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
  return v;
}

// Row-group line: word 0 the counter, word 1 + j the XCD (+ 1) of the row group's block j, published before the
// block's first count.  True when all nblk writers run on XCD `mine`.  Every block of the row group reads the same
// words, so all of them reach the same verdict.  When true, the row group's exchange goes through that XCD's L2:
// ordinary stores (complete once the L2 has them) and ordinary loads (none of those lines was read earlier in the
// launch, so no copy older than the stores sits in an L1).  The blocks are numbered so that a row group's blocks land
// on one XCD under round-robin dispatch; where they do not, the exchange stays device-scope (sc1) stores and loads,
// which the separate L2s keep coherent.
__device__ __forceinline__ bool writers_on_xcd(const int32_t* line, int nblk, int mine) {
  const int lane = threadIdx.x & 63;
  const int v = lane < nblk ? __hip_atomic_load(line + 1 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : mine + 1;
  return __all(v == mine + 1);
}

// Block numbering of the sequence kernels: the grid is P = problems x slots row-group slots of nblk blocks each.
// Blocks are dispatched round-robin over the X XCDs of the device (block b to XCD b % X, checked at run time by
// writers_on_xcd), so a slot's blocks share an XCD when they are X apart: b = x + X (j + nblk k) for slot
// pg = x + X k.  Within the XCD, block j of slot k is then followed by block j + 1 of the same slot, so that a CU's
// second resident block (one XCD pass later) belongs to another row group and the two do not run their MFMA phases
// in lockstep.  When P is not a multiple of X: pg = b % P, j = b / P.
__device__ __forceinline__ void seq_block(int nblk, int xcds, int& pg, int& j) {
  const int b = blockIdx.x, P = gridDim.x / nblk;
  if (xcds > 1 && P % xcds == 0) {
    const int i = b / xcds;
    j = i % nblk;
    pg = b % xcds + xcds * (i / nblk);
  } else {
    pg = b % P;
    j = b / P;
  }
}

// Counts the block in for the row group once every wave's device-scope stores of the step have completed.
__device__ __forceinline__ void seq_signal(int32_t* ctr) {
  wait_vmcnt<0>();
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Counts the block out of its row group's pass, after its last wait (only thread 0 reads the counter): one more
// increment per block on top of the step counts, so the block whose increment brings the counter to `total` (the
// blocks' T - 1 step counts and one count-out each) comes after every read of the counter in this call, and it
// zeroes the counter for the next call on the same buffer.  Every wait's target is at most the final step count,
// which the counter has reached before any block counts out, so the extra increments release no wait early.  A call
// that gave up leaves its counters as they were (the caller zeroes the buffer after reading a non-zero status).
__device__ __forceinline__ void seq_count_out(int32_t* ctr, int total) {
  if (threadIdx.x == 0 && __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1)
    __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int NS, bool GRU, bool PROJ>
__global__ __launch_bounds__(256) void lstm_seq_fwd_kernel(const SeqFwdArgs a) {
  constexpr int BK = kSeqBK, WSLAB = kSeqCols * BK, ASLAB = kSeqRows * BK;
  __shared__ __align__(16) float wl[NS * WSLAB];
  __shared__ __align__(16) float al[2 * ASLAB];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1, hl = lane >> 5;
  int pg, cb;
  seq_block(a.ncb, a.xcds, pg, cb);
  const int p = pg / a.slots, g = pg % a.slots;
  const int xcd = xcd_id();
  const SeqFwdItem& S = a.it[p];
  const int64_t H = a.H, E = a.E;
  const int n0 = cb * kSeqCols;
  // slice of w_hh_g: slab s, row r, 16-byte chunk cc at wl[s WSLAB + r BK + 4 (cc ^ swz(r))], the per-step layout
  for (int i = tid; i < kSeqCols * 8 * NS; i += 256) {
    const int row = i / (8 * NS), c4 = i % (8 * NS), sl = c4 >> 3, cc = c4 & 7;
    const f32x4 v = *reinterpret_cast<const f32x4*>(S.w + (n0 + row) * H + 4 * c4);
    *reinterpret_cast<f32x4*>(wl + sl * WSLAB + row * BK + 4 * (cc ^ nt_swz<BK>(row))) = v;
  }
  // the lane's cell outputs: env row wm*32 + lane%32 of the tile, gate columns ncol + 8q (q = 0..3) = 4 units
  const int ncol = n0 + wn * 32 + 4 * hl;
  // PROJ: the wave's w_ih_g rows (gate columns n0 + wn*32 + lane%32), k 8 (lane/32) .. + 7 of each 16-deep slab
  constexpr int KPM = PROJ ? kSeqProjSlabs : 1;
  [[maybe_unused]] const float* const wr =
      PROJ ? S.wih + static_cast<int64_t>(n0 + wn * 32 + (lane & 31)) * (16 * S.kp) + 8 * hl : nullptr;
  int32_t* const ctr0 = a.sync + kSyncHeader + p * a.nrg * kSyncStride;
  volatile float* const flag = al + ASLAB;  // free between a step's last barrier and the next wait's barrier
  for (int rg = g; rg < a.nrg; rg += a.slots) {
    __syncthreads();  // the previous row group's last slab reads are done; the slice is staged (first pass)
    int32_t* const line = ctr0 + rg * kSyncStride;
    if (tid == 0) __hip_atomic_store(line + 1 + cb, xcd + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool peers = false;  // every writer of the row group on this XCD (known after the first wait)
    const int64_t m0 = static_cast<int64_t>(rg) * kSeqRows;
    const int64_t m = m0 + wm * 32 + (lane & 31);
    const bool in = m < E;
    const int64_t mc = in ? m : E - 1;
    float cp[4];  // c_{t-1} * keep_{t-1} of the lane's units (the GRU: h_{t-1} * keep_{t-1}); step 0: c0
#pragma unroll
    for (int q = 0; q < 4; ++q) cp[q] = S.c0[mc * S.ld0 + ((ncol + 8 * q) >> 2)];
    // this thread's two 16-byte chunks of every 64 x 32 slab of hs[t]: rows clamped to E - 1
    int64_t aoff[2];
    int lofs[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = tid + 256 * j, row = i >> 3, cc = i & 7;
      aoff[j] = std::min<int64_t>(m0 + row, E - 1) * H + 4 * cc;
      lofs[j] = row * BK + 4 * (cc ^ nt_swz<BK>(row));
    }
    // PROJ: the operands of a step's input projection (its x row of the lane, the block's w_ih_g rows, the bias) are
    // loaded a step ahead, at the top of the previous step (whose hs stores and signal then find them landed), and
    // multiplied after that step's signal, while the row group's other blocks pick the signal up
    [[maybe_unused]] f32x4 xr[KPM][2], wv[KPM][2], pbias[4];
    auto proj_load = [&](int64_t row) __attribute__((always_inline)) {
      const float* const xp = S.x + row * S.ldx + 8 * hl;
#pragma unroll
      for (int kt = 0; kt < KPM; ++kt) {
        if (kt < S.kp) {
          xr[kt][0] = *reinterpret_cast<const f32x4*>(xp + 16 * kt);
          xr[kt][1] = *reinterpret_cast<const f32x4*>(xp + 16 * kt + 4);
          wv[kt][0] = *reinterpret_cast<const f32x4*>(wr + 16 * kt);
          wv[kt][1] = *reinterpret_cast<const f32x4*>(wr + 16 * kt + 4);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) pbias[q] = *reinterpret_cast<const f32x4*>(S.bg + ncol + 8 * q);
    };
    auto proj_compute = [&](f32x4 (&out)[4]) __attribute__((always_inline)) {
      f32x16 pacc;
#pragma unroll
      for (int v = 0; v < 16; ++v) pacc[v] = 0.0f;
      constexpr int pa[6] = {2, 1, 0, 1, 0, 0}, pb[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
      for (int kt = 0; kt < KPM; ++kt) {
        if (kt < S.kp) {
          bf16x8 xpl[3], wpl[3];
          split_frag(xr[kt][0], xr[kt][1], xpl);
          split_frag(wv[kt][0], wv[kt][1], wpl);
          if (a.bf16) {
            pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wpl[0], xpl[0], pacc, 0, 0, 0);
          } else {
#pragma unroll
            for (int u = 0; u < 6; ++u)
              pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wpl[pb[u]], xpl[pa[u]], pacc, 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) out[q][e] = pacc[4 * q + e] + pbias[q][e];
    };
    f32x4 gx[4];
    if constexpr (PROJ) {  // step 0's
      proj_load(mc);
      proj_compute(gx);
    }
    for (int t = 0; t < a.T; ++t) {
      const int64_t rowt = static_cast<int64_t>(t) * E + mc;
      if constexpr (PROJ) {
        if (t + 1 < a.T) proj_load(rowt + E);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) gx[q] = *reinterpret_cast<const f32x4*>(S.gx + rowt * S.ldgx + ncol + 8 * q);
      }
      const float keep = S.keep[rowt * S.keep_stride];
      if (t > 0) {
        if (!seq_wait(a.sync, line, a.ncb * t, flag, a.spin_ticks)) return;
        if (t == 1) peers = writers_on_xcd(line, a.ncb, xcd);
      }
      const __amdgpu_buffer_rsrc_t At = __builtin_amdgcn_make_buffer_rsrc(
          S.hs + static_cast<int64_t>(t) * E * H, 0, static_cast<int>(E * H * 4), kBufferWord3);
      f32x4 ra[NS][2];
      auto load_hs = [&](auto policy) {
#pragma unroll
        for (int sl = 0; sl < NS; ++sl)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            ra[sl][j] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(At, static_cast<int>(4 * (aoff[j] + sl * BK)), 0,
                                                             decltype(policy)::value));
      };
      if (t == 0 || peers) {  // hs[0] was written before the launch
        load_hs(std::integral_constant<int, 0>{});
      } else {
        load_hs(std::integral_constant<int, kDeviceScope>{});
      }
      f32x16 acc;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
      for (int j = 0; j < 2; ++j) *reinterpret_cast<f32x4*>(al + lofs[j]) = ra[0][j];
      lds_barrier();
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
        const float* As = al + (sl & 1) * ASLAB;
        const float* Ws = wl + sl * WSLAB;
        const int rA = wm * 32 + (lane & 31), rB = wn * 32 + (lane & 31);
#pragma unroll
        for (int gi = 0; gi < BK / 8; ++gi) {
          const int c = 2 * gi + hl;
          const f32x4 fa = *reinterpret_cast<const f32x4*>(As + rA * BK + 4 * (c ^ nt_swz<BK>(rA)));
          const f32x4 fb = *reinterpret_cast<const f32x4*>(Ws + rB * BK + 4 * (c ^ nt_swz<BK>(rB)));
#pragma unroll
          for (int k = 0; k < 4; ++k) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[k], fa[k], acc, 0, 0, 0);
        }
        if (sl + 1 < NS) {
          // the other buffer's slab sl - 1 was read by every wave before the previous barrier
#pragma unroll
          for (int j = 0; j < 2; ++j)
            *reinterpret_cast<f32x4*>(al + ((sl + 1) & 1) * ASLAB + lofs[j]) = ra[sl + 1][j];
          lds_barrier();
        }
      }
      // the cell for the lane's units 2q + hl (of the wave's 8); lanes l and l + 32 (same row) then trade halves so
      // that each holds 4 consecutive units (hl = 0: units 0..3, hl = 1: units 4..7) and stores 16 bytes per array
      f32x4 act[4];
      float cv[4], hv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 x = {acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
        const LstmCellFwd o = rnn_cell_fwd<GRU>(x, gx[q], cp[q]);
        act[q] = o.act;
        cv[q] = o.c;
        hv[q] = o.h;
        cp[q] = o.c * keep;
      }
      const f32x4 c4 = trade_halves(cv, hl), h4 = trade_halves(hv, hl);
      const f32x4 hs4 = {h4[0] * keep, h4[1] * keep, h4[2] * keep, h4[3] * keep};
      const int64_t ub = ((n0 + wn * 32) >> 2) + 4 * hl;
      // hs[t + 1] first (the other blocks read it: through this XCD's L2 when they all run here, else device
      // scope), then the count, then the outputs nobody waits for
      if (in) {
        const __amdgpu_buffer_rsrc_t Hs = __builtin_amdgcn_make_buffer_rsrc(
            S.hs + static_cast<int64_t>(t + 1) * E * H, 0, static_cast<int>(E * H * 4), kBufferWord3);
        const u32x4 v = __builtin_bit_cast(u32x4, hs4);
        const int off = static_cast<int>(4 * (mc * H + ub));
        if (peers) {
          __builtin_amdgcn_raw_buffer_store_b128(v, Hs, off, 0, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b128(v, Hs, off, 0, kDeviceScope);
        }
      }
      if (t + 1 < a.T) seq_signal(line);
      if constexpr (PROJ) {
        if (t + 1 < a.T) proj_compute(gx);  // the next step's (the cell is done with this one's)
      }
      if (in) {
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<f32x4*>(S.gates + rowt * 4 * H + ncol + 8 * q) = act[q];
        *reinterpret_cast<f32x4*>(S.c + rowt * H + ub) = c4;
        *reinterpret_cast<f32x4*>(S.h + rowt * S.ldh + ub) = h4;
      }
    }
    seq_count_out(line, a.ncb * a.T);
  }
}



// ---- Whole-sequence backward: one launch for all T steps ----
//
// Block (problem p, row-group slot g, unit block ub) holds rows [32 ub, 32 ub + 32) of w_hh_gt (32 units x 4H, LDS,
// 16-byte chunks XOR-swizzled by row) for the whole sequence and runs t = T-1 .. 0 for rows [64 rg, 64 rg + 64).
// Step t's product dgates[t+1] w_hh_g (k = 4H) reads all 4H columns of dgates[t+1] of its rows, which the nub unit
// blocks of the row group write at step t + 1: the same device-scope exchange and per-row-group counters as the
// forward.  Wave w takes rows 16 w .. 16 w + 15 of the row group and both 16-unit halves of the block's units on
// v_mfma_f32_16x16x4f32 with the weights as the first operand, so a lane's accumulator holds 4 consecutive units of
// one env row: the shape the cell derivatives take.  dgates[t+1] goes from memory straight into registers,
// kSeqBwdAhead 64-deep k slabs ahead of the MFMAs (no LDS, no barrier inside a step); the carried dL/dc stays in
// registers from step to step.
constexpr int kSeqBwdUnits = 32, kSeqBwdKS = 64, kSeqBwdAhead = 4;
constexpr int kSeqBwdMaxSlabs = 16;  // 4H <= 1024: the w_hh_gt slice is 128 KB of LDS, one block per CU

struct SeqBwdItem {
  const float* wt;  // w_hh_gt [H, 4H]
  const float* c0;
  const float* keep;
  const float* gates;
  const float* c;
  const float* dh;
  float* dgates;
  int64_t ld0, keep_stride, lddh;
};
struct SeqBwdArgs {
  SeqBwdItem it[PPO_MAX_LSTM_PROBLEMS];
  int32_t* sync;
  uint64_t spin_ticks;
  int32_t H, E, T, nrg, nub, slots;
  int32_t xcds;
};

template <int NS, bool GRU>
__global__ __launch_bounds__(256) void lstm_seq_bwd_kernel(const SeqBwdArgs a) {
  constexpr int K = kSeqBwdKS * NS, KC = K / 4, U = kSeqBwdUnits, AH = kSeqBwdAhead < NS ? kSeqBwdAhead : NS;
  __shared__ __align__(16) float wl[U * K];
  __shared__ float flag_word;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int lr = lane & 15, lq = lane >> 4;
  int pg, ub;
  seq_block(a.nub, a.xcds, pg, ub);
  const int p = pg / a.slots, g = pg % a.slots;
  const int xcd = xcd_id();
  const SeqBwdItem& S = a.it[p];
  const int64_t H = a.H, E = a.E;
  const int u0 = ub * U;
  for (int i = tid; i < U * KC; i += 256) {
    const int row = i / KC, c = i % KC;
    const f32x4 v = *reinterpret_cast<const f32x4*>(S.wt + (u0 + row) * K + 4 * c);
    *reinterpret_cast<f32x4*>(wl + row * K + 4 * (c ^ (row & 15))) = v;
  }
  __syncthreads();
  int32_t* const ctr0 = a.sync + kSyncHeader + p * a.nrg * kSyncStride;
  for (int rg = g; rg < a.nrg; rg += a.slots) {
    int32_t* const line = ctr0 + rg * kSyncStride;
    if (tid == 0) __hip_atomic_store(line + 1 + ub, xcd + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool l2 = false;
    const int64_t m = static_cast<int64_t>(rg) * kSeqRows + 16 * wave + lr;
    const bool in = m < E;
    const int64_t mc = in ? m : E - 1;
    f32x4 dc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};  // dL/dc_t carried from step t + 1
    for (int t = a.T - 1; t >= 0; --t) {
      const int64_t rowt = static_cast<int64_t>(t) * E + mc;
      // the cell's operands (written before the launch): this row, units n .. n + 3 of each half
      const float keep = S.keep[rowt * S.keep_stride];
      const float kp = t > 0 ? S.keep[(rowt - E) * S.keep_stride] : 1.0f;
      f32x4 dhu[2], ct[2], cp[2], gt[2][4];
#pragma unroll
      for (int ti = 0; ti < 2; ++ti) {
        const int n = u0 + 16 * ti + 4 * lq;
        dhu[ti] = *reinterpret_cast<const f32x4*>(S.dh + rowt * S.lddh + n);
        ct[ti] = *reinterpret_cast<const f32x4*>(S.c + rowt * H + n);
        cp[ti] = t > 0 ? *reinterpret_cast<const f32x4*>(S.c + (rowt - E) * H + n)
                       : *reinterpret_cast<const f32x4*>(S.c0 + mc * S.ld0 + n);
#pragma unroll
        for (int e = 0; e < 4; ++e) gt[ti][e] = *reinterpret_cast<const f32x4*>(S.gates + rowt * 4 * H + 4 * (n + e));
      }
      // 4 partial sums per half (k-groups j = 0..3 of every slab): 8 independent MFMA chains per wave, so a
      // single wave per SIMD keeps the matrix pipe busy
      f32x4 acc[2][4];
#pragma unroll
      for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[ti][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (t + 1 < a.T) {
        // dgates[t + 1] complete for the row group: every unit block has finished T - 1 - t steps
        if (!seq_wait(a.sync, line, a.nub * (a.T - 1 - t), &flag_word, a.spin_ticks)) return;
        if (t + 2 == a.T) l2 = writers_on_xcd(line, a.nub, xcd);
        const __amdgpu_buffer_rsrc_t Dg = __builtin_amdgcn_make_buffer_rsrc(
            S.dgates + static_cast<int64_t>(t + 1) * E * K, 0, static_cast<int>(E * K * 4), kBufferWord3);
        const int abase = static_cast<int>(4 * (mc * K + 4 * lq));
        // slab sl, k-group j (16 deep): the lane's 4 consecutive k of its row; one copy of the loop per load policy
        auto product = [&](auto policy) {
          f32x4 ra[NS][4];
          f32x4 fw[2][4][2];  // the weight fragments of two slabs: the next slab's are read under this one's MFMAs
          auto issue = [&](int sl) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              ra[sl][j] = __builtin_bit_cast(
                  f32x4, __builtin_amdgcn_raw_buffer_load_b128(Dg, abase + 4 * (kSeqBwdKS * sl + 16 * j), 0,
                                                               decltype(policy)::value));
          };
          auto wfrag = [&](int sl) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int c = (kSeqBwdKS * sl + 16 * j) / 4 + lq;
#pragma unroll
              for (int ti = 0; ti < 2; ++ti) {
                const int row = 16 * ti + lr;
                fw[sl & 1][j][ti] = *reinterpret_cast<const f32x4*>(wl + row * K + 4 * (c ^ (row & 15)));
              }
            }
          };
#pragma unroll
          for (int sl = 0; sl < AH; ++sl) issue(sl);
          wfrag(0);
#pragma unroll
          for (int sl = 0; sl < NS; ++sl) {
            // scheduling fences: the compiler would otherwise move each load next to its use (fewer registers,
            // but one slab's load latency exposed per slab)
            __builtin_amdgcn_sched_barrier(0);
            if (sl + AH < NS) issue(sl + AH);
            if (sl + 1 < NS) wfrag(sl + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
              for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int ti = 0; ti < 2; ++ti)
                  acc[ti][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fw[sl & 1][j][ti][s4], ra[sl][j][s4], acc[ti][j],
                                                                    0, 0, 0);
          }
        };
        if (l2) {
          product(std::integral_constant<int, 0>{});
        } else {
          product(std::integral_constant<int, kDeviceScope>{});
        }
      }
      f32x4 dpre[2][4];
#pragma unroll
      for (int ti = 0; ti < 2; ++ti) {
        const f32x4 x = (acc[ti][0] + acc[ti][1]) + (acc[ti][2] + acc[ti][3]);
        f32x4 dcout;
        rnn_cell_bwd<GRU>(x, keep, kp, dhu[ti], ct[ti], cp[ti], dc[ti], gt[ti], dpre[ti], dcout);
        dc[ti] = dcout;
      }
      // dgates[t]: the next step's operand (through this XCD's L2 when every writer of the row group runs here, else
      // device scope), then the count
      if (in) {
        const __amdgpu_buffer_rsrc_t Dt = __builtin_amdgcn_make_buffer_rsrc(
            S.dgates + static_cast<int64_t>(t) * E * K, 0, static_cast<int>(E * K * 4), kBufferWord3);
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const u32x4 v = __builtin_bit_cast(u32x4, dpre[ti][e]);
            const int off = static_cast<int>(4 * (mc * K + 4 * (u0 + 16 * ti + 4 * lq + e)));
            if (l2) {
              __builtin_amdgcn_raw_buffer_store_b128(v, Dt, off, 0, 0);
            } else {
              __builtin_amdgcn_raw_buffer_store_b128(v, Dt, off, 0, kDeviceScope);
            }
          }
      }
      if (t > 0) seq_signal(line);
    }
    seq_count_out(line, a.nub * a.T);
    __syncthreads();  // flag_word is reused by the next row group's first wait
  }
}

int64_t grid_for(int64_t total) { return std::max<int64_t>(1, std::min<int64_t>(ceil_div(total, 256), 8192)); }

int check_seq(const ppo_lstm_seq_problem* probs, int32_t count, int64_t steps, int64_t envs, bool bwd,
              const char* who) {
  PPO_REQUIRE(probs != nullptr && count >= 1 && count <= PPO_MAX_LSTM_PROBLEMS, "%s: count=%d outside [1, %d]", who,
              count, PPO_MAX_LSTM_PROBLEMS);
  PPO_REQUIRE(steps >= 1 && envs >= 1 && steps * envs <= INT32_MAX / 8, "%s: steps=%lld envs=%lld", who,
              (long long)steps, (long long)envs);
  for (int i = 0; i < count; ++i) {
    const ppo_lstm_seq_problem& q = probs[i];
    const int64_t H = q.hidden;
    PPO_REQUIRE(H >= 4 && H % 4 == 0 && H <= 4096, "%s: problem %d hidden=%d must be a positive multiple of 4", who,
                i, q.hidden);
    PPO_REQUIRE(q.cell == PPO_CELL_LSTM || q.cell == PPO_CELL_GRU, "%s: problem %d cell=%d", who, i, q.cell);
    PPO_REQUIRE(q.cell == probs[0].cell, "%s: the problems of one call must share the cell type", who);
    PPO_REQUIRE(q.w_hh_g && q.gx && q.h0 && q.c0 && q.keep && q.h && q.hs && q.c && q.gates,
                "%s: problem %d has a null pointer", who, i);
    PPO_REQUIRE(!bwd || (q.w_hh_gt && q.dh && q.dgates && q.dc), "%s: problem %d: backward buffers missing", who, i);
    PPO_REQUIRE(q.ldgx >= 4 * H && q.ldgx % 4 == 0 && q.ld0 >= H && q.ld0 % 4 == 0 && q.ldh >= H && q.ldh % 4 == 0 &&
                    q.keep_stride >= 1 && (!bwd || (q.lddh >= H && q.lddh % 4 == 0)),
                "%s: problem %d leading dims", who, i);
    const void* ptrs[] = {q.w_hh_g, q.gx, q.h0, q.c0, q.h, q.hs, q.c, q.gates};
    for (const void* p : ptrs) PPO_REQUIRE(aligned16(p), "%s: problem %d: pointers must be 16-byte aligned", who, i);
    if (bwd) {
      const void* bp[] = {q.w_hh_gt, q.dh, q.dgates, q.dc};
      for (const void* p : bp) PPO_REQUIRE(aligned16(p), "%s: problem %d: pointers must be 16-byte aligned", who, i);
    }
    PPO_REQUIRE((steps + 1) * envs * 4 * H < (int64_t(1) << 30), "%s: problem %d: sequence spans 4 GiB or more", who,
                i);
  }
  return PPO_OK;
}

// Per-step GEMM configuration: "64x64" is the plain NT kernel (whole k range per wave); the others are the k-split
// kernel with the named block tile ("32x64": 2 splits, "32x32k64": 4 splits over 64-deep slabs, ...).  Measured at
// E = 1024, H = 256 (two problems): the forward step (k = H) takes ~21 us with every tile, the backward step
// (k = 4H) 31 us on 64 x 64 and 19 us on 32x32k64, whose 4 splits cut each wave's dependent MFMA chain to a quarter
// and give 4x the blocks.  In a build with PPO_HIP_TUNING, "PPO_HIP_LSTM_FWD_CFG" / "PPO_HIP_LSTM_BWD_CFG" override
// the defaults (tuning aid).  The backward instantiations with 2 splits allow fewer waves per SIMD: their prefetched
// epilogue operands take registers.
template <int EPI>
int launch_step(Group& g, int count, hipStream_t s, const char* name) {
  constexpr bool fwd = EPI == EPI_LSTM_FWD;
  constexpr int O2 = fwd ? 4 : 2;
#ifdef PPO_HIP_TUNING
  const char* e = std::getenv(fwd ? "PPO_HIP_LSTM_FWD_CFG" : "PPO_HIP_LSTM_BWD_CFG");
  const char* cfg = e != nullptr ? e : fwd ? "64x64" : "32x32k64";
  if (!std::strcmp(cfg, "32x64")) return launch_nt_ks<32, 64, 32, 2, O2, EPI>(g, count, s, name);
  if (!std::strcmp(cfg, "64x32")) return launch_nt_ks<64, 32, 32, 2, O2, EPI>(g, count, s, name);
  if (!std::strcmp(cfg, "32x64k64")) return launch_nt_ks<32, 64, 64, 2, O2, EPI>(g, count, s, name);
  if (!std::strcmp(cfg, "32x32k64")) return launch_nt_ks<32, 32, 64, 2, 4, EPI>(g, count, s, name);
  if (!std::strcmp(cfg, "32x32k32")) return launch_nt_ks<32, 32, 32, 3, 4, EPI>(g, count, s, name);
  return launch_nt_aligned<64, 64, 32, 2, O2, EPI>(g, count, s, name);
#else
  if constexpr (fwd) {
    return launch_nt_aligned<64, 64, 32, 2, O2, EPI>(g, count, s, name);
  } else {
    return launch_nt_ks<32, 32, 64, 2, 4, EPI>(g, count, s, name);
  }
#endif
}

int64_t seq_row_groups(int64_t envs) { return ceil_div(envs, static_cast<int64_t>(kSeqRows)); }

// How long a block of a sequence kernel waits for the others before it gives up (100 MHz ticks): kSeqSpinTicks,
// unless a caller set another limit through ppo_lstm_seq_wait_limit (tests force the give-up path that way; every
// kernel still runs to its end).  No environment variable changes it.
std::atomic<int64_t> g_seq_wait_limit{-1};

uint64_t seq_spin_ticks() {
  const int64_t v = g_seq_wait_limit.load(std::memory_order_relaxed);
  return v >= 0 ? static_cast<uint64_t>(v) : kSeqSpinTicks;
}

// Launches the whole-sequence forward when the shape allows it and the device holds at least one row-group slot
// (count * ncb blocks) at once.  Returns PPO_OK, an error, or PPO_EUNSUPPORTED to ask for the per-step launches.
template <int NS, bool GRU, bool PROJ>
int launch_seq_fwd(SeqFwdArgs& a, int count, hipStream_t s) {
  static std::atomic<int> cache[kMaxDevices];
  const int resident = resident_blocks(lstm_seq_fwd_kernel<NS, GRU, PROJ>, cache);
  const int per_slot = count * a.ncb;
  const int slots = std::min(a.nrg, resident / per_slot);
  if (slots < 1) return PPO_EUNSUPPORTED;
  a.slots = slots;  // (the state-copy launch before this one cleared the sync words)
  hipLaunchKernelGGL((lstm_seq_fwd_kernel<NS, GRU, PROJ>), dim3(count * slots * a.ncb), dim3(256), 0, s, a);
  return check_launch("lstm_seq_fwd_kernel");
}

template <bool GRU, bool PROJ>
int seq_fwd_slabs(SeqFwdArgs& a, int64_t H, int count, hipStream_t s) {
  switch (H / kSeqBK) {
    case 1: return launch_seq_fwd<1, GRU, PROJ>(a, count, s);
    case 2: return launch_seq_fwd<2, GRU, PROJ>(a, count, s);
    case 3: return launch_seq_fwd<3, GRU, PROJ>(a, count, s);
    case 4: return launch_seq_fwd<4, GRU, PROJ>(a, count, s);
    case 5: return launch_seq_fwd<5, GRU, PROJ>(a, count, s);
    case 6: return launch_seq_fwd<6, GRU, PROJ>(a, count, s);
    case 7: return launch_seq_fwd<7, GRU, PROJ>(a, count, s);
    default: return launch_seq_fwd<8, GRU, PROJ>(a, count, s);
  }
}

// proj: the problems' input projections computed in the launch (nullptr: gx is read); bf16: their operands in bf16
int seq_fwd(const ppo_lstm_seq_problem* probs, const ppo_lstm_input_projection* proj, bool bf16, int count,
            int64_t steps, int64_t envs, int32_t* sync, hipStream_t s) {
  const int64_t H = probs[0].hidden;
  if (H % kSeqBK != 0 || H / kSeqBK > kSeqMaxSlabs) return PPO_EUNSUPPORTED;
  SeqFwdArgs a{};
  for (int i = 0; i < count; ++i) {
    const ppo_lstm_seq_problem& q = probs[i];
    SeqFwdItem& it = a.it[i];
    it.w = q.w_hh_g; it.gx = q.gx; it.c0 = q.c0; it.keep = q.keep;
    it.gates = q.gates; it.c = q.c; it.h = q.h; it.hs = q.hs;
    it.ldgx = q.ldgx; it.ld0 = q.ld0; it.keep_stride = q.keep_stride; it.ldh = q.ldh;
    if (proj != nullptr) {
      it.x = proj[i].x; it.ldx = proj[i].ldx; it.wih = proj[i].w_ih_g; it.bg = proj[i].b_g;
      it.kp = proj[i].input_size / 16;
    }
  }
  a.bf16 = bf16 ? 1 : 0;
  a.sync = sync;
  a.spin_ticks = seq_spin_ticks();
  a.xcds = std::max(device_info().xcds, 1);
  a.H = static_cast<int32_t>(H);
  a.E = static_cast<int32_t>(envs);
  a.T = static_cast<int32_t>(steps);
  a.nrg = static_cast<int32_t>(seq_row_groups(envs));
  a.ncb = static_cast<int32_t>(4 * H / kSeqCols);
  const bool gru = probs[0].cell == PPO_CELL_GRU;
  if (proj != nullptr) return gru ? seq_fwd_slabs<true, true>(a, H, count, s) : seq_fwd_slabs<false, true>(a, H, count, s);
  return gru ? seq_fwd_slabs<true, false>(a, H, count, s) : seq_fwd_slabs<false, false>(a, H, count, s);
}

template <int NS, bool GRU>
int launch_seq_bwd(SeqBwdArgs& a, int count, hipStream_t s) {
  static std::atomic<int> cache[kMaxDevices];
  const int resident = resident_blocks(lstm_seq_bwd_kernel<NS, GRU>, cache);
  const int per_slot = count * a.nub;
  const int slots = std::min(a.nrg, resident / per_slot);
  if (slots < 1) return PPO_EUNSUPPORTED;
  a.slots = slots;
  // (the counters start at zero: a zeroed buffer, or the previous call's count-outs)
  hipLaunchKernelGGL((lstm_seq_bwd_kernel<NS, GRU>), dim3(count * slots * a.nub), dim3(256), 0, s, a);
  return check_launch("lstm_seq_bwd_kernel");
}

template <bool GRU>
int seq_bwd_slabs(SeqBwdArgs& a, int64_t H, int count, hipStream_t s) {
  switch (4 * H / kSeqBwdKS) {
    case 2: return launch_seq_bwd<2, GRU>(a, count, s);
    case 4: return launch_seq_bwd<4, GRU>(a, count, s);
    case 6: return launch_seq_bwd<6, GRU>(a, count, s);
    case 8: return launch_seq_bwd<8, GRU>(a, count, s);
    case 10: return launch_seq_bwd<10, GRU>(a, count, s);
    case 12: return launch_seq_bwd<12, GRU>(a, count, s);
    case 14: return launch_seq_bwd<14, GRU>(a, count, s);
    default: return launch_seq_bwd<16, GRU>(a, count, s);
  }
}

int seq_bwd(const ppo_lstm_seq_problem* probs, int count, int64_t steps, int64_t envs, int32_t* sync,
            hipStream_t s) {
  const int64_t H = probs[0].hidden;
  if (H % kSeqBwdUnits != 0 || 4 * H / kSeqBwdKS > kSeqBwdMaxSlabs) return PPO_EUNSUPPORTED;
  SeqBwdArgs a{};
  for (int i = 0; i < count; ++i) {
    const ppo_lstm_seq_problem& q = probs[i];
    SeqBwdItem& it = a.it[i];
    it.wt = q.w_hh_gt; it.c0 = q.c0; it.keep = q.keep; it.gates = q.gates; it.c = q.c; it.dh = q.dh;
    it.dgates = q.dgates; it.ld0 = q.ld0; it.keep_stride = q.keep_stride; it.lddh = q.lddh;
  }
  a.sync = sync;
  a.spin_ticks = seq_spin_ticks();
  a.xcds = std::max(device_info().xcds, 1);
  a.H = static_cast<int32_t>(H);
  a.E = static_cast<int32_t>(envs);
  a.T = static_cast<int32_t>(steps);
  a.nrg = static_cast<int32_t>(seq_row_groups(envs));
  a.nub = static_cast<int32_t>(H / kSeqBwdUnits);
  return probs[0].cell == PPO_CELL_GRU ? seq_bwd_slabs<true>(a, H, count, s) : seq_bwd_slabs<false>(a, H, count, s);
}

int check_sync(int32_t* sync, int64_t sync_words, int count, int64_t envs, const char* who) {
  if (sync == nullptr) return PPO_OK;
  const int64_t need = kSyncHeader + count * seq_row_groups(envs) * kSyncStride;
  PPO_REQUIRE(sync_words >= need, "%s: sync buffer of %lld int32 words, %lld needed", who, (long long)sync_words,
              (long long)need);
  PPO_REQUIRE(reinterpret_cast<uintptr_t>(sync) % 4 == 0, "%s: sync must be 4-byte aligned", who);
  return PPO_OK;
}

}  // namespace
}  // namespace ppo

using namespace ppo;

namespace ppo {
namespace {

int pack(const ppo_lstm_pack_problem* problems, int32_t count, bool gru, ppo_stream_t stream, const char* who) {
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LSTM_PROBLEMS, "%s: count=%d", who, count);
  PackGroup g{};
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_lstm_pack_problem& q = problems[i];
    PPO_REQUIRE(q.w_ih && q.w_hh && q.b_ih && q.b_hh && q.w_ih_g && q.w_hh_g && q.w_hh_gt && q.b_g,
                "%s: problem %d has a null pointer", who, i);
    PPO_REQUIRE(q.input_size >= 1 && q.hidden >= 4 && q.hidden % 4 == 0, "%s: problem %d sizes", who, i);
    PackItem& P = g.it[i];
    P.w_ih = q.w_ih; P.w_hh = q.w_hh; P.b_ih = q.b_ih; P.b_hh = q.b_hh;
    P.w_ih_g = q.w_ih_g; P.w_hh_g = q.w_hh_g; P.w_hh_gt = q.w_hh_gt; P.b_g = q.b_g;
    P.D = q.input_size; P.H = q.hidden; P.begin = total; P.gru = gru;
    total += 4 * P.H * P.D + 8 * P.H * P.H + 4 * P.H;
  }
  PPO_REQUIRE(total <= INT32_MAX, "%s: %lld elements (at most 2^31 - 1 per call)", who, (long long)total);
  g.count = count;
  g.total = total;
  hipLaunchKernelGGL(lstm_pack_kernel, dim3(grid_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream), g);
  return check_launch("lstm_pack_kernel");
}

int unpack(const ppo_lstm_grad_problem* problems, int32_t count, bool gru, const int32_t* groups, double* norm,
           ppo_stream_t stream, const char* who) {
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LSTM_PROBLEMS, "%s: count=%d", who, count);
  GradGroup g{};
  if (norm != nullptr) {
    PPO_REQUIRE(groups != nullptr, "%s: null groups", who);
    PPO_REQUIRE(reinterpret_cast<uintptr_t>(norm) % 8 == 0, "%s: norm_partials must be 8-byte aligned", who);
    for (int i = 0; i < count; ++i) {
      PPO_REQUIRE(groups[i] >= 0 && groups[i] < PPO_MAX_PARAM_GROUPS, "%s: groups[%d]=%d (0 .. %d)", who, i,
                  groups[i], PPO_MAX_PARAM_GROUPS - 1);
      g.group[i] = groups[i];
    }
    g.norm = norm;
  }
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_lstm_grad_problem& q = problems[i];
    PPO_REQUIRE(q.dw_ih_g && q.dw_hh_g && q.db_g && q.dw_ih && q.dw_hh && q.db_ih && q.db_hh,
                "%s: problem %d has a null pointer", who, i);
    PPO_REQUIRE(q.input_size >= 1 && q.hidden >= 4 && q.hidden % 4 == 0, "%s: problem %d sizes", who, i);
    GradItem& P = g.it[i];
    P.dw_ih_g = q.dw_ih_g; P.dw_hh_g = q.dw_hh_g; P.db_g = q.db_g;
    P.dw_ih = q.dw_ih; P.dw_hh = q.dw_hh; P.db_ih = q.db_ih; P.db_hh = q.db_hh;
    P.D = q.input_size; P.H = q.hidden; P.begin = total; P.gru = gru;
    total += (gru ? 3 : 4) * P.H * (P.D + P.H + 1);
  }
  PPO_REQUIRE(total <= INT32_MAX, "%s: %lld elements (at most 2^31 - 1 per call)", who, (long long)total);
  g.count = count;
  g.total = total;
  if (norm != nullptr && total > PPO_DW_NORM_BLOCKS * 256) {
    // the norm rows cap the block count: wider blocks keep about one element per thread
    hipLaunchKernelGGL((lstm_unpack_kernel<true, 1024>), dim3(PPO_DW_NORM_BLOCKS), dim3(1024), 0,
                       static_cast<hipStream_t>(stream), g);
  } else if (norm != nullptr) {
    hipLaunchKernelGGL(lstm_unpack_kernel<true>, dim3(grid_for(total)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), g);
  } else {
    hipLaunchKernelGGL(lstm_unpack_kernel<false>, dim3(grid_for(total)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), g);
  }
  return check_launch("lstm_unpack_kernel");
}

}  // namespace
}  // namespace ppo

extern "C" int ppo_lstm_pack(const ppo_lstm_pack_problem* problems, int32_t count, ppo_stream_t stream) {
  return pack(problems, count, false, stream, "ppo_lstm_pack");
}

extern "C" int ppo_gru_pack(const ppo_lstm_pack_problem* problems, int32_t count, ppo_stream_t stream) {
  return pack(problems, count, true, stream, "ppo_gru_pack");
}

extern "C" int ppo_lstm_unpack_grads(const ppo_lstm_grad_problem* problems, int32_t count, ppo_stream_t stream) {
  return unpack(problems, count, false, nullptr, nullptr, stream, "ppo_lstm_unpack_grads");
}

extern "C" int ppo_gru_unpack_grads(const ppo_lstm_grad_problem* problems, int32_t count, ppo_stream_t stream) {
  return unpack(problems, count, true, nullptr, nullptr, stream, "ppo_gru_unpack_grads");
}

extern "C" int ppo_lstm_unpack_grads_norm(const ppo_lstm_grad_problem* problems, const int32_t* groups, int32_t count,
                                          double* norm_partials, ppo_stream_t stream) {
  static const char* who = "ppo_lstm_unpack_grads_norm";
  PPO_REQUIRE(norm_partials != nullptr, "%s: null norm_partials", who);
  return unpack(problems, count, false, groups, norm_partials, stream, who);
}

extern "C" int ppo_gru_unpack_grads_norm(const ppo_lstm_grad_problem* problems, const int32_t* groups, int32_t count,
                                         double* norm_partials, ppo_stream_t stream) {
  static const char* who = "ppo_gru_unpack_grads_norm";
  PPO_REQUIRE(norm_partials != nullptr, "%s: null norm_partials", who);
  return unpack(problems, count, true, groups, norm_partials, stream, who);
}

extern "C" int64_t ppo_lstm_seq_sync_words(int32_t count, int64_t envs) {
  if (count < 1 || count > PPO_MAX_LSTM_PROBLEMS || envs < 1) return -1;
  return kSyncHeader + count * seq_row_groups(envs) * kSyncStride;
}

extern "C" int64_t ppo_lstm_seq_wait_limit(int64_t ticks) {
  const int64_t previous = g_seq_wait_limit.exchange(ticks < 0 ? -1 : ticks, std::memory_order_relaxed);
  return previous < 0 ? static_cast<int64_t>(kSeqSpinTicks) : previous;
}

namespace ppo {
namespace {

// The input projections can be computed inside the whole-sequence launch with exactly the arithmetic of the
// projection GEMM: inputs of 16..64 columns (a multiple of 16) and every operand as the bf16x6 GEMM takes it
// (16-byte rows: x, w_ih_g, b_g, gx), so that ppo_linear_fwd(_ex) would run the bf16x6 kernel on them.
bool proj_fusable(const ppo_lstm_seq_problem* probs, const ppo_lstm_input_projection* proj, int count,
                  int64_t steps, int64_t envs) {
  for (int i = 0; i < count; ++i) {
    const ppo_lstm_input_projection& r = proj[i];
    const int64_t rows = steps * envs;
    if (r.input_size % 16 != 0 || r.input_size > 16 * kSeqProjSlabs) return false;
    if (!w16_ok(r.x, r.ldx) || !w16_ok(r.w_ih_g, r.input_size) || !aligned16(r.b_g)) return false;
    if (!w16_ok(probs[i].gx, probs[i].ldgx) || rows * probs[i].ldgx * 4 >= (int64_t(1) << 31)) return false;
    if (rows * r.ldx >= (int64_t(1) << 30)) return false;
  }
  return true;
}

// gx = x w_ih_g^T + b_g for every problem, as ppo_linear_fwd_ex.
int launch_projections(const ppo_lstm_seq_problem* probs, const ppo_lstm_input_projection* proj, int count,
                       int64_t rows, int32_t flags, ppo_stream_t stream) {
  ppo_linear_fwd_problem lp[PPO_MAX_LSTM_PROBLEMS]{};
  for (int i = 0; i < count; ++i) {
    lp[i].x = proj[i].x; lp[i].ldx = proj[i].ldx;
    lp[i].w = proj[i].w_ih_g; lp[i].b = proj[i].b_g;
    lp[i].z = const_cast<float*>(probs[i].gx); lp[i].ldz = probs[i].ldgx;
    lp[i].in_features = proj[i].input_size;
    lp[i].out_features = static_cast<int32_t>(4 * probs[i].hidden);
  }
  return ppo_linear_fwd_ex(lp, count, rows, PPO_ACT_NONE, flags, stream);
}

int seq_fwd_entry(const ppo_lstm_seq_problem* problems, const ppo_lstm_input_projection* proj, int32_t flags,
                  int32_t count, int64_t steps, int64_t envs, int32_t* sync, int64_t sync_words,
                  ppo_stream_t stream, const char* who) {
  if (int rc = check_seq(problems, count, steps, envs, false, who)) return rc;
  if (int rc = check_sync(sync, sync_words, count, envs, who)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  bool fuse = false;
  if (proj != nullptr) {
    PPO_REQUIRE((flags & ~PPO_GEMM_BF16_OPERANDS) == 0, "%s: flags=%d", who, flags);
    for (int i = 0; i < count; ++i) {
      const ppo_lstm_input_projection& r = proj[i];
      PPO_REQUIRE(r.x != nullptr && r.w_ih_g != nullptr && r.b_g != nullptr, "%s: projection %d has a null pointer",
                  who, i);
      PPO_REQUIRE(r.input_size > 0 && r.ldx >= r.input_size, "%s: projection %d: input_size=%d ldx=%lld", who, i,
                  r.input_size, (long long)r.ldx);
    }
    fuse = sync != nullptr && steps > 1 && proj_fusable(problems, proj, count, steps, envs);
  }
  const int64_t E = envs;
  CopyGroup cg{};
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    PPO_REQUIRE(problems[i].hidden == problems[0].hidden, "ppo_lstm_seq_fwd: problems must share the hidden size");
    cg.it[i].src = problems[i].h0;
    cg.it[i].dst = problems[i].hs;
    cg.it[i].ld_src = problems[i].ld0;
    cg.it[i].begin = total;
    total += E * problems[i].hidden;
  }
  PPO_REQUIRE(total <= INT32_MAX, "%s: %lld state elements (at most 2^31 - 1 per call)", who, (long long)total);
  cg.count = count;
  cg.H = problems[0].hidden;
  cg.total = total;
  if (sync != nullptr && steps > 1) {  // the counters of the whole-sequence launch, cleared in the same launch
    cg.sync = sync;
    cg.sync_words = static_cast<int32_t>(kSyncHeader + count * seq_row_groups(envs) * kSyncStride);
  }
  hipLaunchKernelGGL(lstm_copy_state_kernel, dim3(grid_for(total)), dim3(256), 0, s, cg);
  if (int rc = check_launch("lstm_copy_state_kernel")) return rc;
  if (fuse) {
    const int rc = seq_fwd(problems, proj, (flags & PPO_GEMM_BF16_OPERANDS) != 0, count, steps, envs, sync, s);
    if (rc != PPO_EUNSUPPORTED) return rc;
  }
  if (proj != nullptr) {  // the projections as their own launch, then the sequence on gx
    if (int rc = launch_projections(problems, proj, count, steps * E, flags, stream)) return rc;
  }
  if (sync != nullptr && steps > 1) {
    const int rc = seq_fwd(problems, nullptr, false, count, steps, envs, sync, s);
    if (rc != PPO_EUNSUPPORTED) return rc;
  }
  for (int64_t t = 0; t < steps; ++t) {
    Group g{};
    for (int i = 0; i < count; ++i) {
      const ppo_lstm_seq_problem& q = problems[i];
      const int64_t H = q.hidden;
      Problem& p = g.p[i];
      p.A = q.hs + t * E * H; p.lda = H;
      p.B = q.w_hh_g; p.ldb = H;
      p.M = static_cast<int>(E); p.N = static_cast<int>(4 * H); p.K = static_cast<int>(H);
      p.splits = 1; p.k_chunk = p.K;
      LstmArgs& L = p.lstm;
      L.gx = q.gx + t * E * q.ldgx; L.ldgx = q.ldgx;
      if (t == 0) {
        L.c_prev = q.c0; L.ldcp = q.ld0; L.keep_prev = nullptr;
      } else {
        L.c_prev = q.c + (t - 1) * E * H; L.ldcp = H; L.keep_prev = q.keep + (t - 1) * E * q.keep_stride;
      }
      L.keep = q.keep + t * E * q.keep_stride; L.keep_stride = q.keep_stride;
      L.gates = q.gates + t * E * 4 * H;
      L.c = q.c + t * E * H;
      L.h = q.h + t * E * q.ldh; L.ldh = q.ldh;
      L.hs = q.hs + (t + 1) * E * H;
      L.hidden = static_cast<int>(H);
      L.cell = q.cell;
    }
    if (int rc = launch_step<EPI_LSTM_FWD>(g, count, s, "lstm_step_fwd")) return rc;
  }
  return PPO_OK;
}

}  // namespace
}  // namespace ppo

extern "C" int ppo_lstm_seq_fwd(const ppo_lstm_seq_problem* problems, int32_t count, int64_t steps, int64_t envs,
                                int32_t* sync, int64_t sync_words, ppo_stream_t stream) {
  return seq_fwd_entry(problems, nullptr, 0, count, steps, envs, sync, sync_words, stream, "ppo_lstm_seq_fwd");
}

extern "C" int ppo_lstm_seq_fwd_proj(const ppo_lstm_seq_problem* problems, const ppo_lstm_input_projection* proj,
                                     int32_t count, int64_t steps, int64_t envs, int32_t flags, int32_t* sync,
                                     int64_t sync_words, ppo_stream_t stream) {
  PPO_REQUIRE(proj != nullptr, "ppo_lstm_seq_fwd_proj: projections are required");
  return seq_fwd_entry(problems, proj, flags, count, steps, envs, sync, sync_words, stream, "ppo_lstm_seq_fwd_proj");
}

extern "C" int ppo_lstm_seq_bwd(const ppo_lstm_seq_problem* problems, int32_t count, int64_t steps, int64_t envs,
                                int32_t* sync, int64_t sync_words, ppo_stream_t stream) {
  if (int rc = check_seq(problems, count, steps, envs, true, "ppo_lstm_seq_bwd")) return rc;
  if (int rc = check_sync(sync, sync_words, count, envs, "ppo_lstm_seq_bwd")) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t E = envs;
  if (sync != nullptr && steps > 1) {
    const int rc = seq_bwd(problems, count, steps, envs, sync, s);
    if (rc != PPO_EUNSUPPORTED) return rc;
  }
  for (int64_t t = steps - 1; t >= 0; --t) {
    Group g{};
    for (int i = 0; i < count; ++i) {
      const ppo_lstm_seq_problem& q = problems[i];
      const int64_t H = q.hidden;
      Problem& p = g.p[i];
      // dL/dh_t from step t+1 = dgates[t+1] w_hh_g; nothing at the last step (K = 0)
      p.A = t + 1 < steps ? q.dgates + (t + 1) * E * 4 * H : q.dgates; p.lda = 4 * H;
      p.B = q.w_hh_gt; p.ldb = 4 * H;
      p.M = static_cast<int>(E); p.N = static_cast<int>(H); p.K = t + 1 < steps ? static_cast<int>(4 * H) : 0;
      p.splits = 1; p.k_chunk = p.K;
      LstmArgs& L = p.lstm;
      if (t == 0) {
        L.c_prev = q.c0; L.ldcp = q.ld0; L.keep_prev = nullptr;
      } else {
        L.c_prev = q.c + (t - 1) * E * H; L.ldcp = H; L.keep_prev = q.keep + (t - 1) * E * q.keep_stride;
      }
      L.keep = q.keep + t * E * q.keep_stride; L.keep_stride = q.keep_stride;
      L.gates = q.gates + t * E * 4 * H;
      L.c = q.c + t * E * H;
      L.dh = q.dh + t * E * q.lddh; L.lddh = q.lddh;
      L.dgates = q.dgates + t * E * 4 * H;
      L.dc = q.dc;
      L.hidden = static_cast<int>(H);
      L.first = t + 1 == steps;
      L.last = t == 0;
      L.cell = q.cell;
    }
    if (int rc = launch_step<EPI_LSTM_BWD>(g, count, s, "lstm_step_bwd")) return rc;
  }
  return PPO_OK;
}
