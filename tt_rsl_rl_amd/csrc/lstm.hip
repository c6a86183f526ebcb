// A15 LSTM of the recurrent models (torch nn.LSTM, one layer; rsl_rl/modules/rnn.py:22-86) on gfx950.
//
// The input projection x w_ih^T + b of all T steps is one GEMM (ppo_linear_fwd on the gate-interleaved weights).
// The recurrence is one kernel per step: the NT GEMM of gemm_core.hpp computes hs[t] w_hh_g^T (rows = envs,
// columns = gates of 4 hidden units per 16-byte group) and its LSTM epilogue applies the cell equations
// (i, f, o = sigmoid, g = tanh; c_t = f c_{t-1} + i g; h_t = o tanh(c_t)), writing the activations for the backward
// and the next step's operand hs[t+1] = h_t * keep_t.  The backward step computes dgates[t+1] w_hh_g (rows = envs,
// columns = hidden units) and its epilogue applies the cell derivatives, carrying dL/dc to the previous step.
// Actor and critic share every launch.  The two weight gradients are plain split-K GEMMs over all T*E rows
// (ppo_linear_bwd_dw: dgates^T hs and dgates^T x).
#include <cstring>

#include "gemm_core.hpp"

namespace ppo {
namespace {

// Gate-interleaved index of torch row r = q*H + u is 4u + q.
__device__ __forceinline__ int64_t interleave(int64_t r, int64_t H) { return 4 * (r % H) + r / H; }

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
};
struct PackGroup {
  PackItem it[PPO_MAX_LSTM_PROBLEMS];
  int32_t count;
  int64_t total;
};

// Flat element e of a problem: [0, 4HD) w_ih_g, [.., +4HH) w_hh_g, [.., +4HH) w_hh_gt, [.., +4H) b_g; each output
// element is written by exactly one thread (reads are gathers from the torch layout).
__global__ __launch_bounds__(256) void lstm_pack_kernel(const PackGroup g) {
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < g.total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const PackItem& P = g.it[(g.count > 1 && e >= g.it[1].begin) ? 1 : 0];
    int64_t k = e - P.begin;
    const int64_t H = P.H, D = P.D, G = 4 * H;
    if (k < G * D) {  // w_ih_g[4u+q][d] = w_ih[qH+u][d]
      const int64_t n = k / D, d = k % D;
      P.w_ih_g[k] = P.w_ih[((n & 3) * H + (n >> 2)) * D + d];
      continue;
    }
    k -= G * D;
    if (k < G * H) {  // w_hh_g[4u+q][j] = w_hh[qH+u][j]
      const int64_t n = k / H, j = k % H;
      P.w_hh_g[k] = P.w_hh[((n & 3) * H + (n >> 2)) * H + j];
      continue;
    }
    k -= G * H;
    if (k < G * H) {  // w_hh_gt[j][4u+q] = w_hh[qH+u][j]
      const int64_t j = k / G, n = k % G;
      P.w_hh_gt[k] = P.w_hh[((n & 3) * H + (n >> 2)) * H + j];
      continue;
    }
    k -= G * H;  // b_g[4u+q] = b_ih[qH+u] + b_hh[qH+u]
    const int64_t r = (k & 3) * H + (k >> 2);
    P.b_g[k] = P.b_ih[r] + P.b_hh[r];
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
};
struct GradGroup {
  GradItem it[PPO_MAX_LSTM_PROBLEMS];
  int32_t count;
  int64_t total;
};

// Flat element e of a problem: [0, 4HD) dw_ih, [.., +4HH) dw_hh, [.., +4H) db_ih and db_hh (torch layout, written
// once each).
__global__ __launch_bounds__(256) void lstm_unpack_kernel(const GradGroup g) {
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < g.total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const GradItem& P = g.it[(g.count > 1 && e >= g.it[1].begin) ? 1 : 0];
    int64_t k = e - P.begin;
    const int64_t H = P.H, D = P.D, G = 4 * H;
    if (k < G * D) {
      const int64_t r = k / D, d = k % D;
      P.dw_ih[k] = P.dw_ih_g[interleave(r, H) * D + d];
      continue;
    }
    k -= G * D;
    if (k < G * H) {
      const int64_t r = k / H, j = k % H;
      P.dw_hh[k] = P.dw_hh_g[interleave(r, H) * H + j];
      continue;
    }
    k -= G * H;
    const float v = P.db_g[interleave(k, H)];
    P.db_ih[k] = v;
    P.db_hh[k] = v;
  }
}

// hs[0] = h0 for every problem (rows E, H floats each).
struct CopyItem {
  const float* src;
  float* dst;
  int64_t ld_src, begin;
};
struct CopyGroup {
  CopyItem it[PPO_MAX_LSTM_PROBLEMS];
  int32_t count;
  int64_t H, total;
};

__global__ __launch_bounds__(256) void lstm_copy_state_kernel(const CopyGroup g) {
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < g.total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const CopyItem& C = g.it[(g.count > 1 && e >= g.it[1].begin) ? 1 : 0];
    const int64_t k = e - C.begin, row = k / g.H, col = k % g.H;
    C.dst[k] = C.src[row * C.ld_src + col];
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

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
// and give 4x the blocks.  "PPO_HIP_LSTM_FWD_CFG" / "PPO_HIP_LSTM_BWD_CFG" override the defaults (tuning aid).  The
// backward instantiations with 2 splits allow fewer waves per SIMD: their prefetched epilogue operands take
// registers.
template <int EPI>
int launch_step(Group& g, int count, hipStream_t s, const char* name) {
  constexpr bool fwd = EPI == EPI_LSTM_FWD;
  constexpr int O2 = fwd ? 4 : 2;
  const char* e = std::getenv(fwd ? "PPO_HIP_LSTM_FWD_CFG" : "PPO_HIP_LSTM_BWD_CFG");
  const char* cfg = e != nullptr ? e : fwd ? "64x64" : "32x32k64";
  if (!std::strcmp(cfg, "32x64")) return launch_nt_ks<32, 64, 32, 2, O2, EPI>(g, count, s, name);
  if (!std::strcmp(cfg, "64x32")) return launch_nt_ks<64, 32, 32, 2, O2, EPI>(g, count, s, name);
  if (!std::strcmp(cfg, "32x64k64")) return launch_nt_ks<32, 64, 64, 2, O2, EPI>(g, count, s, name);
  if (!std::strcmp(cfg, "32x32k64")) return launch_nt_ks<32, 32, 64, 2, 4, EPI>(g, count, s, name);
  if (!std::strcmp(cfg, "32x32k32")) return launch_nt_ks<32, 32, 32, 3, 4, EPI>(g, count, s, name);
  return launch_nt_aligned<64, 64, 32, 2, O2, EPI>(g, count, s, name);
}

}  // namespace
}  // namespace ppo

using namespace ppo;

extern "C" int ppo_lstm_pack(const ppo_lstm_pack_problem* problems, int32_t count, ppo_stream_t stream) {
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LSTM_PROBLEMS, "ppo_lstm_pack: count=%d", count);
  PackGroup g{};
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_lstm_pack_problem& q = problems[i];
    PPO_REQUIRE(q.w_ih && q.w_hh && q.b_ih && q.b_hh && q.w_ih_g && q.w_hh_g && q.w_hh_gt && q.b_g,
                "ppo_lstm_pack: problem %d has a null pointer", i);
    PPO_REQUIRE(q.input_size >= 1 && q.hidden >= 4 && q.hidden % 4 == 0, "ppo_lstm_pack: problem %d sizes", i);
    PackItem& P = g.it[i];
    P.w_ih = q.w_ih; P.w_hh = q.w_hh; P.b_ih = q.b_ih; P.b_hh = q.b_hh;
    P.w_ih_g = q.w_ih_g; P.w_hh_g = q.w_hh_g; P.w_hh_gt = q.w_hh_gt; P.b_g = q.b_g;
    P.D = q.input_size; P.H = q.hidden; P.begin = total;
    total += 4 * P.H * P.D + 8 * P.H * P.H + 4 * P.H;
  }
  g.count = count;
  g.total = total;
  hipLaunchKernelGGL(lstm_pack_kernel, dim3(grid_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream), g);
  return check_launch("lstm_pack_kernel");
}

extern "C" int ppo_lstm_unpack_grads(const ppo_lstm_grad_problem* problems, int32_t count, ppo_stream_t stream) {
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LSTM_PROBLEMS, "ppo_lstm_unpack_grads: count=%d",
              count);
  GradGroup g{};
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_lstm_grad_problem& q = problems[i];
    PPO_REQUIRE(q.dw_ih_g && q.dw_hh_g && q.db_g && q.dw_ih && q.dw_hh && q.db_ih && q.db_hh,
                "ppo_lstm_unpack_grads: problem %d has a null pointer", i);
    PPO_REQUIRE(q.input_size >= 1 && q.hidden >= 4 && q.hidden % 4 == 0, "ppo_lstm_unpack_grads: problem %d sizes", i);
    GradItem& P = g.it[i];
    P.dw_ih_g = q.dw_ih_g; P.dw_hh_g = q.dw_hh_g; P.db_g = q.db_g;
    P.dw_ih = q.dw_ih; P.dw_hh = q.dw_hh; P.db_ih = q.db_ih; P.db_hh = q.db_hh;
    P.D = q.input_size; P.H = q.hidden; P.begin = total;
    total += 4 * P.H * P.D + 4 * P.H * P.H + 4 * P.H;
  }
  g.count = count;
  g.total = total;
  hipLaunchKernelGGL(lstm_unpack_kernel, dim3(grid_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream), g);
  return check_launch("lstm_unpack_kernel");
}

extern "C" int ppo_lstm_seq_fwd(const ppo_lstm_seq_problem* problems, int32_t count, int64_t steps, int64_t envs,
                                ppo_stream_t stream) {
  if (int rc = check_seq(problems, count, steps, envs, false, "ppo_lstm_seq_fwd")) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
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
  cg.count = count;
  cg.H = problems[0].hidden;
  cg.total = total;
  hipLaunchKernelGGL(lstm_copy_state_kernel, dim3(grid_for(total)), dim3(256), 0, s, cg);
  if (int rc = check_launch("lstm_copy_state_kernel")) return rc;
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
    }
    if (int rc = launch_step<EPI_LSTM_FWD>(g, count, s, "lstm_step_fwd")) return rc;
  }
  return PPO_OK;
}

extern "C" int ppo_lstm_seq_bwd(const ppo_lstm_seq_problem* problems, int32_t count, int64_t steps, int64_t envs,
                                ppo_stream_t stream) {
  if (int rc = check_seq(problems, count, steps, envs, true, "ppo_lstm_seq_bwd")) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t E = envs;
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
    }
    if (int rc = launch_step<EPI_LSTM_BWD>(g, count, s, "lstm_step_bwd")) return rc;
  }
  return PPO_OK;
}
