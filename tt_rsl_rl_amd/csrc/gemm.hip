// A6 linear layers (rsl_rl/modules/mlp.py:27-95; autograd of nn.Linear / nn.ELU) as fp32 MFMA GEMMs for gfx950.
//
// One templated kernel computes C = A B over BM x BN output tiles with 256 threads: 4 wavefronts in a 2 x 2
// arrangement, each owning a (BM/2) x (BN/2) sub-tile of 32 x 32 v_mfma_f32_32x32x2f32 accumulators.  A and B are
// staged through double-buffered LDS in BK-deep k-slabs stored k-major, so every MFMA operand fetch is one
// ds_read_b32 per lane and each slab costs a single barrier; the next slab is fetched from global memory into
// registers (float4 where the leading dimension allows, chosen per problem at launch) while the current one is
// multiplied.  A(m,k) and B(k,n) are read either k-contiguous or m/n-contiguous (template flags), which covers the
// three products of a layer without transposing anything in memory:
//   forward     z[r,o]   = sum_i x[r,i]  w[o,i]   A = x  (k-contig)   B = w (k-contig)   epilogue +b, ELU
//   input-grad  dzp[r,i] = sum_o dz[r,o] w[o,i]   A = dz (k-contig)   B = w (n-contig)   epilogue * ELU'(z_prev)
//   weight-grad dw[o,i]  = sum_r dz[r,o] x[r,i]   A = dz (m-contig)   B = x (n-contig)   split-K partials
// The weight-grad kernel also sums its A slab over k (blocks of the first n tile only), which yields the bias
// gradient db[o] = sum_r dz[r,o] in fp64.  Split-K partials are reduced in a fixed order by a second kernel, so the
// result is deterministic.  Several independent problems (actor and critic, or all layers of the weight-grad)
// share one launch: the block index is mapped to (problem, split, tile) through per-problem block offsets, after
// an XCD-aware permutation that places consecutive tiles (which share an A panel) on the same XCD / L2.
#include <cstdlib>
#include <cstring>

#include "common.hpp"

namespace ppo {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum Epilogue : int { EPI_BIAS = 0, EPI_BIAS_ELU = 1, EPI_ELU_GRAD = 2, EPI_STORE = 3, EPI_PARTIAL = 4 };

struct Problem {
  const float* A;
  const float* B;
  float* C;
  float* C2;
  const float* vec;  // bias [N]
  const float* aux;  // ELU'-source z_prev [M, N]
  double* colsum;    // [splits, M] row sums of A over each split's k range (fp64: bias grads cancel heavily)
  int64_t lda, ldb, ldc, ldc2, ldaux;
  int64_t partial_stride;  // floats between split partials of C
  int32_t M, N, K;
  int32_t tiles_m, tiles_n, splits, k_chunk;
  int32_t block_begin;
  int32_t a_vec, b_vec;    // float4 global loads along the contiguous dimension are valid for this problem
};

struct Group {
  Problem p[PPO_MAX_LINEAR_PROBLEMS];
  int32_t count;
  int32_t xcd_remap;  // 1: permute block ids so each XCD gets a contiguous range of tiles
};

constexpr int kThreads = 256;
constexpr int kXcds = 8;

// Blocks are dispatched round-robin over the XCDs; renumber them so that each XCD receives a contiguous range of
// logical tiles (a bijection of [0, n)).
__device__ inline int xcd_remap(int b, int n) {
  const int q = n / kXcds, r = n % kXcds;
  const int xcd = b % kXcds, slot = b / kXcds;
  return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// Loads one BK-deep slab of a BM-wide (A) or BN-wide (B) operand into registers and stores it k-major into LDS.
// KMAJ: element (x, k) at base[(x0 + x) * ld + k0 + k]; otherwise at base[(k0 + k) * ld + x0 + x].
template <int BX, int BK, bool KMAJ, bool VEC>
struct Slab {
  static constexpr int kElems = BX * BK / kThreads;
  static_assert(kElems % 4 == 0, "slab must give every thread a multiple of 4 elements");
  float r[kElems];
  int valid[kElems / 4];  // float4 path: leading elements of each vector inside the operand (the rest -> 0)

  // Issues the loads only: nothing here consumes the loaded registers, so the wait for them lands in store(),
  // after the MFMAs of the current slab.
  __device__ inline void load(const float* __restrict__ base, int64_t ld, int x0, int X, int k0, int k_end) {
    const int tid = threadIdx.x;
    if (VEC) {
#pragma unroll
      for (int i = 0; i < kElems / 4; ++i) {
        const int q = tid + kThreads * i;
        int x, k;
        if (KMAJ) {
          x = q / (BK / 4);
          k = (q % (BK / 4)) * 4;
        } else {
          k = q / (BX / 4);
          x = (q % (BX / 4)) * 4;
        }
        const int gx = x0 + x, gk = k0 + k;
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        int n = 0;
        if (KMAJ) {
          if (gx < X && gk < k_end) {
            v = *reinterpret_cast<const f32x4*>(base + gx * ld + gk);
            n = min(4, k_end - gk);
          }
        } else {
          if (gk < k_end && gx < X) {
            v = *reinterpret_cast<const f32x4*>(base + gk * ld + gx);
            n = min(4, X - gx);
          }
        }
        valid[i] = n;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[4 * i + j] = v[j];
      }
    } else {
#pragma unroll
      for (int i = 0; i < kElems; ++i) {
        const int q = tid + kThreads * i;
        const int x = KMAJ ? q / BK : q % BX;
        const int k = KMAJ ? q % BK : q / BX;
        const int gx = x0 + x, gk = k0 + k;
        float v = 0.0f;
        if (gx < X && gk < k_end) v = KMAJ ? base[gx * ld + gk] : base[gk * ld + gx];
        r[i] = v;
      }
    }
  }

  template <int LDS_W>
  __device__ inline void store(float (*lds)[LDS_W]) {
    const int tid = threadIdx.x;
    if (VEC) {
#pragma unroll
      for (int i = 0; i < kElems / 4; ++i) {
        const int q = tid + kThreads * i;
        float e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = j < valid[i] ? r[4 * i + j] : 0.0f;
        if (KMAJ) {
          const int x = q / (BK / 4), k = (q % (BK / 4)) * 4;
#pragma unroll
          for (int j = 0; j < 4; ++j) lds[k + j][x] = e[j];
        } else {
          const int k = q / (BX / 4), x = (q % (BX / 4)) * 4;
          f32x4 v = {e[0], e[1], e[2], e[3]};
          *reinterpret_cast<f32x4*>(&lds[k][x]) = v;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < kElems; ++i) {
        const int q = tid + kThreads * i;
        const int x = KMAJ ? q / BK : q % BX;
        const int k = KMAJ ? q % BK : q / BX;
        lds[k][x] = r[i];
      }
    }
  }
};

template <int BM, int BN, int BK, bool A_KMAJ, bool B_KMAJ, bool A_VEC, bool B_VEC, int EPI>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const Group g) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int PAD = 4;
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  __shared__ __align__(16) float As[2][BK][BM + PAD];
  __shared__ __align__(16) float Bs[2][BK][BN + PAD];

  const int b = g.xcd_remap ? xcd_remap(blockIdx.x, gridDim.x) : static_cast<int>(blockIdx.x);
  int pi = 0;
#pragma unroll
  for (int i = 1; i < PPO_MAX_LINEAR_PROBLEMS; ++i) {
    if (i < g.count && b >= g.p[i].block_begin) pi = i;
  }
  const Problem& P = g.p[pi];
  const int local = b - P.block_begin;
  const int tiles_mn = P.tiles_m * P.tiles_n;
  const int split = local / tiles_mn;
  const int t = local - split * tiles_mn;
  const int tm = t / P.tiles_n;
  const int tn = t - tm * P.tiles_n;
  const int row0 = tm * BM;
  const int col0 = tn * BN;
  const int k_begin = split * P.k_chunk;
  const int k_end = min(P.K, k_begin + P.k_chunk);
  const int M = P.M, N = P.N;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  Slab<BM, BK, A_KMAJ, A_VEC> sa;
  Slab<BN, BK, B_KMAJ, B_VEC> sb;
  const bool do_colsum = (EPI == EPI_PARTIAL) && (P.colsum != nullptr) && (tn == 0);
  double colsum_acc = 0.0;

  const int nk = k_begin < k_end ? static_cast<int>(ceil_div(k_end - k_begin, BK)) : 0;
  if (nk > 0) {
    sa.load(P.A, P.lda, row0, M, k_begin, k_end);
    sb.load(P.B, P.ldb, col0, N, k_begin, k_end);
    sa.store(As[0]);
    sb.store(Bs[0]);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      const int k0 = k_begin + (kt + 1) * BK;
      sa.load(P.A, P.lda, row0, M, k0, k_end);
      sb.load(P.B, P.ldb, col0, N, k0, k_end);
    }
    if (do_colsum && tid < BM) {
#pragma unroll
      for (int kk = 0; kk < BK; ++kk) colsum_acc += static_cast<double>(As[cur][kk][tid]);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      const int k = kk + (lane >> 5);
      float a[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = As[cur][k][wm * WM + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[j] = Bs[cur][k][wn * WN + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      sa.store(As[cur ^ 1]);
      sb.store(Bs[cur ^ 1]);
    }
    __syncthreads();
  }

  // Epilogue.  MFMA 32x32 output layout: element v of lane l is row 8*(v/4) + 4*(l/32) + v%4, column l%32.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int c = col0 + wn * WN + j * 32 + (lane & 31);
      if (c >= N) continue;
      float bias = 0.0f;
      if (EPI == EPI_BIAS || EPI == EPI_BIAS_ELU) bias = P.vec[c];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = row0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (r >= M) continue;
        const float x = acc[i][j][v];
        const int64_t rr = r;
        if (EPI == EPI_BIAS) {
          P.C[rr * P.ldc + c] = x + bias;
        } else if (EPI == EPI_BIAS_ELU) {
          const float z = x + bias;
          P.C[rr * P.ldc + c] = z;
          P.C2[rr * P.ldc2 + c] = z > 0.0f ? z : expm1f(z);
        } else if (EPI == EPI_ELU_GRAD) {
          const float zp = P.aux[rr * P.ldaux + c];
          P.C[rr * P.ldc + c] = zp > 0.0f ? x : x * expf(zp);
        } else if (EPI == EPI_STORE) {
          P.C[rr * P.ldc + c] = x;
        } else {  // EPI_PARTIAL
          P.C[split * P.partial_stride + rr * P.ldc + c] = x;
        }
      }
    }
  }
  if (do_colsum && tid < BM && row0 + tid < M) P.colsum[static_cast<int64_t>(split) * M + row0 + tid] = colsum_acc;
}

// Fixed-order reduction of split-K weight-grad partials: dw = sum_s partial[s], db = sum_s colsum[s].
struct ReduceItem {
  const float* partial;  // [splits, out*in]
  const double* colsum;  // [splits, out]
  float* dw;
  float* db;
  int64_t begin;         // first flat element of this item in the launch
  int32_t out, in, splits, pad;
};
struct ReduceGroup {
  ReduceItem it[PPO_MAX_LINEAR_PROBLEMS];
  int32_t count;
  int64_t total;
};

__global__ __launch_bounds__(256) void dw_reduce_kernel(const ReduceGroup g) {
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < g.total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int pi = 0;
#pragma unroll
    for (int i = 1; i < PPO_MAX_LINEAR_PROBLEMS; ++i)
      if (i < g.count && e >= g.it[i].begin) pi = i;
    const ReduceItem& R = g.it[pi];
    const int64_t local = e - R.begin;
    const int64_t nw = static_cast<int64_t>(R.out) * R.in;
    if (local < nw) {
      float s = 0.0f;
      for (int k = 0; k < R.splits; ++k) s += R.partial[k * nw + local];
      R.dw[local] = s;
    } else {
      const int64_t o = local - nw;
      double s = 0.0;
      for (int k = 0; k < R.splits; ++k) s += R.colsum[k * static_cast<int64_t>(R.out) + o];
      R.db[o] = static_cast<float>(s);
    }
  }
}

template <int BM, int BN, int BK, bool AK, bool BKM, int EPI>
int launch(Group& g, int count, hipStream_t s, const char* name) {
  int blocks = 0;
  bool avec = std::getenv("PPO_HIP_GEMM_SCALAR") == nullptr, bvec = avec;
  for (int i = 0; i < count; ++i) {
    Problem& p = g.p[i];
    p.tiles_m = static_cast<int>(ceil_div(p.M, BM));
    p.tiles_n = static_cast<int>(ceil_div(p.N, BN));
    p.block_begin = blocks;
    const int64_t nb = static_cast<int64_t>(p.tiles_m) * p.tiles_n * p.splits;
    if (blocks + nb > INT32_MAX) return fail(PPO_EUNSUPPORTED, "%s: grid too large", name);
    blocks += static_cast<int>(nb);
    avec = avec && p.a_vec;
    bvec = bvec && p.b_vec;
  }
  g.count = count;
  g.xcd_remap = std::getenv("PPO_HIP_NO_XCD_REMAP") == nullptr;
  for (int i = count; i < PPO_MAX_LINEAR_PROBLEMS; ++i) g.p[i].block_begin = INT32_MAX;
  if (blocks == 0) return PPO_OK;
  // float4 global loads only when every problem of the launch allows them
  if (avec && bvec) {
    hipLaunchKernelGGL((gemm_kernel<BM, BN, BK, AK, BKM, true, true, EPI>), dim3(blocks), dim3(kThreads), 0, s, g);
  } else if (avec) {
    hipLaunchKernelGGL((gemm_kernel<BM, BN, BK, AK, BKM, true, false, EPI>), dim3(blocks), dim3(kThreads), 0, s, g);
  } else if (bvec) {
    hipLaunchKernelGGL((gemm_kernel<BM, BN, BK, AK, BKM, false, true, EPI>), dim3(blocks), dim3(kThreads), 0, s, g);
  } else {
    hipLaunchKernelGGL((gemm_kernel<BM, BN, BK, AK, BKM, false, false, EPI>), dim3(blocks), dim3(kThreads), 0, s, g);
  }
  return check_launch(name);
}

// float4 loads along the contiguous dimension need a 16-byte aligned base, a leading dimension that is a multiple
// of 4, and -- because a partial float4 at the end of a row is read whole and masked -- a leading dimension of at
// least the contiguous extent rounded up to 4 (the caller's buffer holds rows x ld floats).
bool vec_ok(const float* base, int64_t ld, int64_t contiguous_extent) {
  return (reinterpret_cast<uintptr_t>(base) % 16 == 0) && ld % 4 == 0 && ld >= (contiguous_extent + 3) / 4 * 4;
}

// Tile of a launch: "PPO_HIP_GEMM_TILE" (e.g. "128x64k32") overrides the size-based choice (tuning aid).
enum Tile { T128x128k32, T128x128k16, T128x64k32, T64x64k32, T256x128k16 };

Tile pick_tile(Tile dflt) {
  const char* e = std::getenv("PPO_HIP_GEMM_TILE");
  if (e == nullptr) return dflt;
  if (!std::strcmp(e, "128x128k32")) return T128x128k32;
  if (!std::strcmp(e, "128x128k16")) return T128x128k16;
  if (!std::strcmp(e, "128x64k32")) return T128x64k32;
  if (!std::strcmp(e, "64x64k32")) return T64x64k32;
  if (!std::strcmp(e, "256x128k16")) return T256x128k16;
  return dflt;
}

template <bool AK, bool BKM, int EPI>
int launch_tile(Tile t, Group& g, int count, hipStream_t s, const char* name) {
  switch (t) {
    case T128x128k16:
      return launch<128, 128, 16, AK, BKM, EPI>(g, count, s, name);
    case T128x64k32:
      return launch<128, 64, 32, AK, BKM, EPI>(g, count, s, name);
    case T64x64k32:
      return launch<64, 64, 32, AK, BKM, EPI>(g, count, s, name);
    case T256x128k16:
      return launch<256, 128, 16, AK, BKM, EPI>(g, count, s, name);
    default:
      return launch<128, 128, 32, AK, BKM, EPI>(g, count, s, name);
  }
}

// Split-K policy for the weight-grad: enough blocks to cover the chip (~4 per CU), slabs of at least 256 rows.
// Tile: "PPO_HIP_DW_TILE" overrides the default 128x128k32 (tuning aid).
constexpr int kDwBK = 32;  // split-K chunks are multiples of the largest BK

Tile dw_tile() {
  const char* e = std::getenv("PPO_HIP_DW_TILE");
  if (e == nullptr) return T128x128k16;
  if (!std::strcmp(e, "128x128k32")) return T128x128k32;
  if (!std::strcmp(e, "128x64k32")) return T128x64k32;
  if (!std::strcmp(e, "64x64k32")) return T64x64k32;
  if (!std::strcmp(e, "256x128k16")) return T256x128k16;
  return T128x128k16;
}

void tile_dims(Tile t, int& bm, int& bn) {
  switch (t) {
    case T128x64k32: bm = 128; bn = 64; break;
    case T64x64k32: bm = 64; bn = 64; break;
    case T256x128k16: bm = 256; bn = 128; break;
    default: bm = 128; bn = 128; break;
  }
}

int dw_splits(int64_t tiles, int64_t rows) {
  const int64_t target = 1024;
  int64_t s = ceil_div(target, std::max<int64_t>(tiles, 1));
  s = std::min<int64_t>(s, std::max<int64_t>(1, rows / 256));
  s = std::max<int64_t>(1, std::min<int64_t>(s, 256));
  return static_cast<int>(s);
}

struct DwPlan {
  int splits[PPO_MAX_LINEAR_PROBLEMS];
  int k_chunk[PPO_MAX_LINEAR_PROBLEMS];
  size_t partial_off[PPO_MAX_LINEAR_PROBLEMS];  // floats
  size_t colsum_off[PPO_MAX_LINEAR_PROBLEMS];   // floats (8-byte aligned: holds doubles)
  size_t total_floats;
};

DwPlan plan_dw(const ppo_linear_bwd_dw_problem* probs, int count, int64_t rows) {
  DwPlan plan{};
  int bm, bn;
  tile_dims(dw_tile(), bm, bn);
  int64_t tiles = 0;
  for (int i = 0; i < count; ++i)
    tiles += ceil_div(probs[i].out_features, bm) * ceil_div(probs[i].in_features, bn);
  const int s = dw_splits(tiles, rows);
  size_t off = 0;
  for (int i = 0; i < count; ++i) {
    const int64_t chunk = ceil_div(ceil_div(rows, s), kDwBK) * kDwBK;
    const int splits = static_cast<int>(ceil_div(rows, chunk));
    plan.splits[i] = splits;
    plan.k_chunk[i] = static_cast<int>(chunk);
    plan.partial_off[i] = off;
    off += static_cast<size_t>(splits) * probs[i].out_features * probs[i].in_features;
    off = (off + 63) & ~static_cast<size_t>(63);
    plan.colsum_off[i] = off;
    off += 2 * static_cast<size_t>(splits) * probs[i].out_features;
    off = (off + 63) & ~static_cast<size_t>(63);
  }
  plan.total_floats = off;
  return plan;
}

bool rows_ok(int64_t rows) { return rows > 0 && rows <= INT32_MAX / 2; }

}  // namespace
}  // namespace ppo

using namespace ppo;

extern "C" int ppo_linear_fwd(const ppo_linear_fwd_problem* problems, int32_t count, int64_t rows, int32_t activation,
                              ppo_stream_t stream) {
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LINEAR_PROBLEMS,
              "ppo_linear_fwd: count=%d outside [1, %d]", count, PPO_MAX_LINEAR_PROBLEMS);
  PPO_REQUIRE(rows_ok(rows), "ppo_linear_fwd: rows=%lld", (long long)rows);
  PPO_REQUIRE(activation == PPO_ACT_NONE || activation == PPO_ACT_ELU, "ppo_linear_fwd: activation=%d", activation);
  Group g{};
  int max_n = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_linear_fwd_problem& q = problems[i];
    PPO_REQUIRE(q.x && q.w && q.b && q.z, "ppo_linear_fwd: problem %d has a null pointer", i);
    PPO_REQUIRE(q.in_features > 0 && q.out_features > 0, "ppo_linear_fwd: problem %d features", i);
    PPO_REQUIRE(q.ldx >= q.in_features && q.ldz >= q.out_features, "ppo_linear_fwd: problem %d leading dims", i);
    PPO_REQUIRE(activation == PPO_ACT_NONE || (q.h != nullptr && q.ldh >= q.out_features),
                "ppo_linear_fwd: problem %d needs h for ELU", i);
    Problem& p = g.p[i];
    p.A = q.x; p.lda = q.ldx;
    p.B = q.w; p.ldb = q.in_features;
    p.C = q.z; p.ldc = q.ldz;
    p.C2 = q.h; p.ldc2 = q.ldh;
    p.vec = q.b;
    p.M = static_cast<int>(rows); p.N = q.out_features; p.K = q.in_features;
    p.splits = 1; p.k_chunk = q.in_features;
    p.a_vec = vec_ok(q.x, q.ldx, q.in_features);
    p.b_vec = vec_ok(q.w, q.in_features, q.in_features);
    max_n = std::max(max_n, q.out_features);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  // measured on MI355X for 24576-row mini-batches: wide outputs like 128x128 tiles, 128..256-wide outputs 128x64,
  // narrow output layers 64x64
  const Tile t = pick_tile(max_n > 256 ? T128x128k16 : (max_n > 64 ? T128x64k32 : T64x64k32));
  if (activation == PPO_ACT_ELU) return launch_tile<true, true, EPI_BIAS_ELU>(t, g, count, s, "linear_fwd_elu");
  return launch_tile<true, true, EPI_BIAS>(t, g, count, s, "linear_fwd");
}

extern "C" int ppo_linear_bwd_dx(const ppo_linear_bwd_dx_problem* problems, int32_t count, int64_t rows,
                                 ppo_stream_t stream) {
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LINEAR_PROBLEMS,
              "ppo_linear_bwd_dx: count=%d outside [1, %d]", count, PPO_MAX_LINEAR_PROBLEMS);
  PPO_REQUIRE(rows_ok(rows), "ppo_linear_bwd_dx: rows=%lld", (long long)rows);
  Group g{};
  bool any_act = false, any_plain = false;
  int max_n = 0;
  for (int i = 0; i < count; ++i) {
    const ppo_linear_bwd_dx_problem& q = problems[i];
    PPO_REQUIRE(q.dz && q.w && q.dz_prev, "ppo_linear_bwd_dx: problem %d has a null pointer", i);
    PPO_REQUIRE(q.in_features > 0 && q.out_features > 0, "ppo_linear_bwd_dx: problem %d features", i);
    PPO_REQUIRE(q.lddz >= q.out_features && q.lddz_prev >= q.in_features &&
                    (q.z_prev == nullptr || q.ldz_prev >= q.in_features),
                "ppo_linear_bwd_dx: problem %d leading dims", i);
    (q.z_prev ? any_act : any_plain) = true;
    Problem& p = g.p[i];
    p.A = q.dz; p.lda = q.lddz;
    p.B = q.w; p.ldb = q.in_features;
    p.C = q.dz_prev; p.ldc = q.lddz_prev;
    p.aux = q.z_prev; p.ldaux = q.ldz_prev;
    p.M = static_cast<int>(rows); p.N = q.in_features; p.K = q.out_features;
    p.splits = 1; p.k_chunk = q.out_features;
    p.a_vec = vec_ok(q.dz, q.lddz, q.out_features);
    p.b_vec = vec_ok(q.w, q.in_features, q.in_features);
    max_n = std::max(max_n, q.in_features);
  }
  PPO_REQUIRE(!(any_act && any_plain), "ppo_linear_bwd_dx: mix of activation and plain problems in one call");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // measured on MI355X: 64x64 tiles for every input-grad shape of the [512, 256, 128] MLPs
  const Tile t = pick_tile(T64x64k32);
  if (any_act) return launch_tile<true, false, EPI_ELU_GRAD>(t, g, count, s, "linear_bwd_dx_elu");
  return launch_tile<true, false, EPI_STORE>(t, g, count, s, "linear_bwd_dx");
}

extern "C" size_t ppo_linear_bwd_dw_workspace_bytes(const ppo_linear_bwd_dw_problem* problems, int32_t count,
                                                    int64_t rows) {
  if (problems == nullptr || count < 1 || count > PPO_MAX_LINEAR_PROBLEMS || !rows_ok(rows)) return 0;
  for (int i = 0; i < count; ++i)
    if (problems[i].in_features <= 0 || problems[i].out_features <= 0) return 0;
  return plan_dw(problems, count, rows).total_floats * sizeof(float);
}

extern "C" int ppo_linear_bwd_dw(const ppo_linear_bwd_dw_problem* problems, int32_t count, int64_t rows,
                                 void* workspace, size_t workspace_bytes, ppo_stream_t stream) {
  PPO_REQUIRE(problems != nullptr && count >= 1 && count <= PPO_MAX_LINEAR_PROBLEMS,
              "ppo_linear_bwd_dw: count=%d outside [1, %d]", count, PPO_MAX_LINEAR_PROBLEMS);
  PPO_REQUIRE(rows_ok(rows), "ppo_linear_bwd_dw: rows=%lld", (long long)rows);
  for (int i = 0; i < count; ++i) {
    const ppo_linear_bwd_dw_problem& q = problems[i];
    PPO_REQUIRE(q.dz && q.x && q.dw && q.db, "ppo_linear_bwd_dw: problem %d has a null pointer", i);
    PPO_REQUIRE(q.in_features > 0 && q.out_features > 0, "ppo_linear_bwd_dw: problem %d features", i);
    PPO_REQUIRE(q.lddz >= q.out_features && q.ldx >= q.in_features, "ppo_linear_bwd_dw: problem %d leading dims", i);
  }
  const DwPlan plan = plan_dw(problems, count, rows);
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
    p.A = q.dz; p.lda = q.lddz;
    p.B = q.x; p.ldb = q.ldx;
    p.C = ws + plan.partial_off[i]; p.ldc = q.in_features;
    p.partial_stride = static_cast<int64_t>(q.out_features) * q.in_features;
    p.colsum = reinterpret_cast<double*>(ws + plan.colsum_off[i]);
    p.M = q.out_features; p.N = q.in_features; p.K = static_cast<int>(rows);
    p.splits = plan.splits[i]; p.k_chunk = plan.k_chunk[i];
    p.a_vec = vec_ok(q.dz, q.lddz, q.out_features);
    p.b_vec = vec_ok(q.x, q.ldx, q.in_features);
    ReduceItem& r = rg.it[i];
    r.partial = p.C; r.colsum = p.colsum; r.dw = q.dw; r.db = q.db;
    r.out = q.out_features; r.in = q.in_features; r.splits = plan.splits[i];
    r.begin = total;
    total += static_cast<int64_t>(q.out_features) * q.in_features + q.out_features;
  }
  for (int i = count; i < PPO_MAX_LINEAR_PROBLEMS; ++i) rg.it[i].begin = INT64_MAX;
  rg.count = count;
  rg.total = total;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = launch_tile<false, false, EPI_PARTIAL>(dw_tile(), g, count, s, "linear_bwd_dw");
  if (rc != PPO_OK) return rc;
  const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), 4096);
  hipLaunchKernelGGL(dw_reduce_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, rg);
  return check_launch("dw_reduce_kernel");
}
