// A5 permutation gather (rsl_rl/storage/rollout_storage.py:232-259) and the observation-normaliser forward
// (rsl_rl/modules/normalization.py:46-48), fused: one pass over the rollout per update writes the packed,
// permuted, normalised row table that every mini-batch of every epoch then reads contiguously (for the recurrent
// update also the keep = 1 - done column, from the stored uint8 dones).
//
// The copied floats of a row, segment after segment, are numbered 0 .. total-1 ("flat columns"); lane l of a
// wavefront owns flat columns l, l + 64, ... (kSlots of them per pass), so consecutive lanes read consecutive floats of
// a segment and write consecutive destination floats.  The flat column -> (segment, column) map depends only on the
// segment widths: each wave derives it once per pass (from a copy of the segment table in LDS) and then moves
// kRowsPerIter rows per iteration, issuing all their loads before any store so a wave waits for memory once per
// iteration rather than once per segment.
#include <atomic>
#include <cstdlib>

#include "common.hpp"

#pragma clang fp contract(off)

namespace ppo {
namespace {

struct GatherArgs {
  ppo_gather_segment seg[PPO_MAX_GATHER_SEGMENTS];
  int32_t prefix[PPO_MAX_GATHER_SEGMENTS + 1];  // first flat column of each segment; prefix[num_segments] = total
  int32_t num_segments;
  // gather_rows_vec_kernel: segments [0, num_vec) move as float4 chunks (vprefix: first chunk of each, vprefix[num_vec]
  // = the chunk count), segments [num_vec, num_segments) as floats (prefix, from 0 at segment num_vec)
  int32_t vprefix[PPO_MAX_GATHER_SEGMENTS + 1];
  int32_t num_vec;
};

// Source pointers are global memory; read back from the LDS copy of the segment table they would otherwise be
// generic (flat) pointers, whose loads also count as LDS operations and defeat the wait counters.
typedef const uint32_t __attribute__((address_space(1))) global_u32;
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kGatherThreads = 256;
constexpr int kWavesPerBlock = kGatherThreads / kWave;

constexpr int kGatherRowsPerIter = 4;
// Row iterations per wave of gather_rows_vec_kernel at most (measured, gather alone: humanoid's 98,304 rows 54.5 us
// with one iteration per wave, 49.9 with two, 48.2 with eight; flat48_65k's 1,572,864 rows 413 / 412 / 423 us: an
// iteration's loads wait for the previous iteration's stores to have read their registers)
constexpr int64_t kGatherMaxIters = 2;

// kSlots: flat columns per lane per pass (64 kSlots floats of a row; the launcher takes the fewest that cover a row,
// up to 8); kRowsPerIter: rows whose loads a wave has in flight at once (4: 96 against 105 us with 2 for the humanoid
// table's 98,304 rows of 295 copied floats, 131 us with 8)
template <int kSlots, int kRowsPerIter>
__global__ __launch_bounds__(kGatherThreads) void gather_rows_kernel(const int64_t* __restrict__ perm, int64_t rows,
                                                                     int64_t src_rows, GatherArgs args,
                                                                     float* __restrict__ dst, int64_t dst_stride) {
  __shared__ ppo_gather_segment seg[PPO_MAX_GATHER_SEGMENTS];
  if (threadIdx.x < args.num_segments) seg[threadIdx.x] = args.seg[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave_id = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  const int64_t wave_count = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  const int total = args.prefix[args.num_segments];
  for (int f0 = 0; f0 < total; f0 += kWave * kSlots) {
    // this lane's flat columns of the pass -> source address and row stride (bytes), destination column,
    // normaliser.  Every source element is read as the aligned 32-bit word that holds it: the float itself, or for a
    // keep segment the word around the uint8 done flag (inside the flags' allocation), from which the byte is taken.
    uintptr_t src[kSlots];
    int64_t stride[kSlots];
    int dcol[kSlots];
    bool valid[kSlots], keep[kSlots];
    float mu[kSlots], den[kSlots];
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
      const int fc = f0 + lane + kWave * k;
      int s = 0;
      for (int i = 1; i < args.num_segments; ++i) s = fc >= args.prefix[i] ? i : s;
      const int col = fc - args.prefix[s];
      const ppo_gather_segment& g = seg[s];
      const bool in = fc < total;
      const bool u8 = in && g.kind == PPO_GATHER_KEEP_U8;
      const int esz = u8 ? 1 : 4;
      // a lane without a column this slot reads element (0, 0) of the first segment and discards it
      src[k] = reinterpret_cast<uintptr_t>(in ? g.src : seg[0].src) + (in ? col * esz : 0);
      valid[k] = in;
      keep[k] = u8;
      stride[k] = in ? g.src_stride * esz : 0;
      dcol[k] = g.dst_col + col;
      const bool norm = in && g.norm_mean != nullptr;
      mu[k] = norm ? g.norm_mean[col] : 0.0f;
      den[k] = norm ? g.norm_std[col] + g.norm_eps : 1.0f;
    }
    for (int64_t j0 = wave_id * kRowsPerIter; j0 < rows; j0 += wave_count * kRowsPerIter) {
      int64_t sr[kRowsPerIter];
#pragma unroll
      for (int r = 0; r < kRowsPerIter; ++r) {
        const int64_t j = j0 + r;
        const int64_t p = j < rows ? perm[j] : -1;
        sr[r] = p >= 0 && p < src_rows ? p : -1;  // never read outside the source (the host checks perm)
      }
      // every load unconditional and in straight-line code (rows outside [0, rows) read source row 0), so the
      // wave issues all of them before it waits
      float v[kRowsPerIter][kSlots];
      uint32_t word[kRowsPerIter][kSlots];
      int shift[kRowsPerIter][kSlots];
#pragma unroll
      for (int r = 0; r < kRowsPerIter; ++r) {
        const int64_t row = sr[r] >= 0 ? sr[r] : 0;
#pragma unroll
        for (int k = 0; k < kSlots; ++k) {
          const uintptr_t a = src[k] + row * stride[k];
          word[r][k] = *reinterpret_cast<global_u32*>(a & ~static_cast<uintptr_t>(3));
          shift[r][k] = static_cast<int>(a & 3) * 8;
        }
      }
      // then all arithmetic (plain copies take mu = 0, den = 1: (x - 0) / 1 == x exactly; keep = 1 - done), then all
      // stores: a store counts in the same counter as the loads, so interleaving them would make every wait drain the
      // stores too
#pragma unroll
      for (int r = 0; r < kRowsPerIter; ++r)
#pragma unroll
        for (int k = 0; k < kSlots; ++k) {
          const float x = keep[k] ? 1.0f - static_cast<float>((word[r][k] >> shift[r][k]) & 0xffu)
                                  : __uint_as_float(word[r][k]);
          v[r][k] = (x - mu[k]) / den[k];
        }
      __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic above the (predicated) stores
#pragma unroll
      for (int r = 0; r < kRowsPerIter; ++r)
#pragma unroll
        for (int k = 0; k < kSlots; ++k)
          if (sr[r] >= 0 && valid[k]) dst[(j0 + r) * dst_stride + dcol[k]] = v[r][k];
    }
  }
}

// Rows whose segments are mostly whole, 16-byte aligned float4 runs (fp32 source 16-byte aligned with a leading
// dimension a multiple of 4, width and destination column multiples of 4, in a 16-byte aligned table whose stride is
// a multiple of 4): lane l owns the float4 chunks l, l + 64, ... of those segments (kV slots, one 16-byte load and
// store each) and the flat columns l, l + 64, ... of the others (kS slots, 4-byte), every row in one pass.  A wave
// moves kRowsPerIter rows per iteration with all their loads in flight before the arithmetic and the stores, as in
// gather_rows_kernel, whose results it reproduces bit for bit (the same (x - mean) / (std + eps) per float).
template <int kV, int kS, int kRowsPerIter>
__global__ __launch_bounds__(kGatherThreads) void gather_rows_vec_kernel(const int64_t* __restrict__ perm,
                                                                         int64_t rows, int64_t src_rows,
                                                                         GatherArgs args, float* __restrict__ dst,
                                                                         int64_t dst_stride) {
  __shared__ ppo_gather_segment seg[PPO_MAX_GATHER_SEGMENTS];
  if (threadIdx.x < args.num_segments) seg[threadIdx.x] = args.seg[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  // (wave-uniform as far as the compiler can see, so the permutation entries below are scalar loads, which wait on
  // their own counter instead of behind this wave's row stores)
  const int64_t wave_id = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock +
                          __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t wave_count = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  const int nv = args.num_vec, ns = args.num_segments;
  const int vtotal = args.vprefix[nv], stotal = args.prefix[ns];
  // the lane's chunks: source address, row stride (bytes), destination column, normaliser (4 columns each)
  uintptr_t vsrc[kV];
  int64_t vstride[kV];
  int vcol[kV];
  bool vvalid[kV];
  f32x4 vmu[kV], vden[kV];
#pragma unroll
  for (int k = 0; k < kV; ++k) {
    const int fc = lane + kWave * k;
    int s = 0;
    for (int i = 1; i < nv; ++i) s = fc >= args.vprefix[i] ? i : s;
    const ppo_gather_segment& g = seg[s];
    const bool in = fc < vtotal;
    const int col = in ? 4 * (fc - args.vprefix[s]) : 0;
    vvalid[k] = in;
    vsrc[k] = reinterpret_cast<uintptr_t>(in ? g.src : seg[0].src) + col * 4;
    vstride[k] = in ? g.src_stride * 4 : 0;
    vcol[k] = g.dst_col + col;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool norm = in && g.norm_mean != nullptr;
      vmu[k][e] = norm ? g.norm_mean[col + e] : 0.0f;
      vden[k][e] = norm ? g.norm_std[col + e] + g.norm_eps : 1.0f;
    }
  }
  // the lane's single floats (as gather_rows_kernel's)
  uintptr_t src[kS > 0 ? kS : 1];
  int64_t stride[kS > 0 ? kS : 1];
  int dcol[kS > 0 ? kS : 1];
  bool valid[kS > 0 ? kS : 1], keep[kS > 0 ? kS : 1];
  float mu[kS > 0 ? kS : 1], den[kS > 0 ? kS : 1];
#pragma unroll
  for (int k = 0; k < kS; ++k) {
    const int fc = lane + kWave * k;
    int s = nv;
    for (int i = nv + 1; i < ns; ++i) s = fc >= args.prefix[i] ? i : s;
    const bool in = fc < stotal && ns > nv;
    const ppo_gather_segment& g = seg[in ? s : 0];
    const int col = in ? fc - args.prefix[s] : 0;
    const bool u8 = in && g.kind == PPO_GATHER_KEEP_U8;
    const int esz = u8 ? 1 : 4;
    src[k] = reinterpret_cast<uintptr_t>(in ? g.src : seg[0].src) + (in ? col * esz : 0);
    valid[k] = in;
    keep[k] = u8;
    stride[k] = in ? g.src_stride * esz : 0;
    dcol[k] = g.dst_col + col;
    const bool norm = in && g.norm_mean != nullptr;
    mu[k] = norm ? g.norm_mean[col] : 0.0f;
    den[k] = norm ? g.norm_std[col] + g.norm_eps : 1.0f;
  }
  typedef const f32x4 __attribute__((address_space(1))) global_f32x4;
  // The grid holds about the blocks the device keeps resident, so a wave walks several iterations; the permutation
  // entries of its next iteration are loaded right after this iteration's row loads, and an iteration waits for one
  // memory round trip instead of two (the entry, then the row it names).
  // (32-bit row indices, rows < 2^30 (the launcher checks): the loop's compares stay scalar, and no vector register
  // that a row store of the iteration still reads is taken for them)
  const int rows32 = static_cast<int>(rows), step = static_cast<int>(wave_count) * kRowsPerIter;
  int64_t pn[kRowsPerIter];
  auto load_perm = [&](int j0) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < kRowsPerIter; ++r) {
      const int j = j0 + r;
      pn[r] = j < rows32 ? perm[j] : -1;
    }
  };
  load_perm(static_cast<int>(wave_id) * kRowsPerIter);
  for (int j0 = static_cast<int>(wave_id) * kRowsPerIter; j0 < rows32; j0 += step) {
    int64_t sr[kRowsPerIter];
#pragma unroll
    for (int r = 0; r < kRowsPerIter; ++r)
      sr[r] = pn[r] >= 0 && pn[r] < src_rows ? pn[r] : -1;  // never read outside the source (the host checks perm)
    f32x4 vv[kRowsPerIter][kV];
    uint32_t word[kRowsPerIter][kS > 0 ? kS : 1];
    int shift[kRowsPerIter][kS > 0 ? kS : 1];
#pragma unroll
    for (int r = 0; r < kRowsPerIter; ++r) {
      const int64_t row = sr[r] >= 0 ? sr[r] : 0;
#pragma unroll
      for (int k = 0; k < kV; ++k) vv[r][k] = *reinterpret_cast<global_f32x4*>(vsrc[k] + row * vstride[k]);
#pragma unroll
      for (int k = 0; k < kS; ++k) {
        const uintptr_t a = src[k] + row * stride[k];
        word[r][k] = *reinterpret_cast<global_u32*>(a & ~static_cast<uintptr_t>(3));
        shift[r][k] = static_cast<int>(a & 3) * 8;
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // (the next entries' loads after the rows', so the wait below skips them)
    load_perm(j0 + step);
    float v[kRowsPerIter][kS > 0 ? kS : 1];
#pragma unroll
    for (int r = 0; r < kRowsPerIter; ++r) {
#pragma unroll
      for (int k = 0; k < kV; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) vv[r][k][e] = (vv[r][k][e] - vmu[k][e]) / vden[k][e];
#pragma unroll
      for (int k = 0; k < kS; ++k) {
        const float x = keep[k] ? 1.0f - static_cast<float>((word[r][k] >> shift[r][k]) & 0xffu)
                                : __uint_as_float(word[r][k]);
        v[r][k] = (x - mu[k]) / den[k];
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic above the (predicated) stores
#pragma unroll
    for (int r = 0; r < kRowsPerIter; ++r) {
      if (sr[r] < 0) continue;
      float* const drow = dst + (j0 + r) * dst_stride;
#pragma unroll
      for (int k = 0; k < kV; ++k)
        if (vvalid[k]) *reinterpret_cast<f32x4*>(drow + vcol[k]) = vv[r][k];
#pragma unroll
      for (int k = 0; k < kS; ++k)
        if (valid[k]) drow[dcol[k]] = v[r][k];
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

// One thread per output element (row r = t / W, column c = t % W of the W-float rows): consecutive threads write
// consecutive floats of the destination and read consecutive rows of each source block.
struct InterleaveArgs {
  ppo_column_block col[PPO_MAX_INTERLEAVE_FLOATS];
  int32_t first[PPO_MAX_INTERLEAVE_FLOATS];  // first output column of each block
  int32_t num_cols, width;
};

__global__ __launch_bounds__(256) void interleave_kernel(const InterleaveArgs a, int64_t rows, float* __restrict__ dst,
                                                         int64_t dst_stride) {
  const uint32_t total = static_cast<uint32_t>(rows) * a.width;  // < 2^31 (checked on the host)
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < total; t += gridDim.x * blockDim.x) {
    const uint32_t r = t / a.width;
    const int c = static_cast<int>(t - r * a.width);
    int b = 0;
#pragma unroll
    for (int i = 1; i < PPO_MAX_INTERLEAVE_FLOATS; ++i)
      if (i < a.num_cols && c >= a.first[i]) b = i;
    dst[static_cast<int64_t>(r) * dst_stride + c] = a.col[b].src[static_cast<int64_t>(r) * a.col[b].stride + (c - a.first[b])];
  }
}

// Blocks of a gather kernel the current device holds at once (0 when unknown), queried once per instantiation and
// device.
template <typename K>
int64_t resident_gather_blocks(K kernel) {
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kGatherThreads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    v = std::max(per_cu, 0) * std::max(cus, 0) + 1;  // stored + 1: 0 marks "not queried yet"
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v - 1;
}

}  // namespace
}  // namespace ppo

using namespace ppo;

extern "C" int ppo_interleave_columns(const ppo_column_block* cols, int32_t num_cols, int64_t rows, float* dst,
                                      int64_t dst_stride, ppo_stream_t stream) {
  PPO_REQUIRE(cols && dst, "ppo_interleave_columns: null pointer");
  PPO_REQUIRE(rows > 0 && num_cols > 0 && num_cols <= PPO_MAX_INTERLEAVE_FLOATS,
              "ppo_interleave_columns: rows=%lld num_cols=%d", (long long)rows, num_cols);
  InterleaveArgs a{};
  int total = 0;
  for (int i = 0; i < num_cols; ++i) {
    PPO_REQUIRE(cols[i].src != nullptr && cols[i].width > 0 && cols[i].stride >= cols[i].width,
                "ppo_interleave_columns: column block %d malformed", i);
    a.col[i] = cols[i];
    a.first[i] = total;
    total += cols[i].width;
    PPO_REQUIRE(total <= PPO_MAX_INTERLEAVE_FLOATS, "ppo_interleave_columns: more than %d floats per row",
                PPO_MAX_INTERLEAVE_FLOATS);
  }
  PPO_REQUIRE(dst_stride >= total, "ppo_interleave_columns: dst_stride %lld < %d", (long long)dst_stride, total);
  PPO_REQUIRE(rows * total < (int64_t(1) << 31), "ppo_interleave_columns: %lld rows of %d floats are too many",
              (long long)rows, total);
  a.num_cols = num_cols;
  a.width = total;
  const int64_t blocks = std::min<int64_t>(ceil_div(rows * total, 256), 16384);
  hipLaunchKernelGGL(interleave_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a, rows, dst, dst_stride);
  return check_launch("interleave_kernel");
}

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
  int64_t total = 0;
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
    PPO_REQUIRE(g.kind == PPO_GATHER_FLOAT || (g.kind == PPO_GATHER_KEEP_U8 && g.norm_mean == nullptr),
                "ppo_gather_rows: segment %d: kind %d (a keep segment takes no normaliser)", s, g.kind);
    PPO_REQUIRE(g.kind != PPO_GATHER_FLOAT || reinterpret_cast<uintptr_t>(g.src) % 4 == 0,
                "ppo_gather_rows: segment %d: fp32 source not 4-byte aligned", s);
    args.seg[s] = g;
    args.prefix[s] = static_cast<int32_t>(total);
    total += g.width;
    PPO_REQUIRE(total <= INT32_MAX / 2, "ppo_gather_rows: rows of %lld floats are too wide", (long long)total);
  }
  args.prefix[num_segments] = static_cast<int32_t>(total);
  // float4 chunks for the segments that allow them (16-byte aligned sources of a stride and width that are multiples
  // of 4, destination columns multiples of 4 in a 16-byte aligned table of such a stride), when each lane's share of
  // a row fits 4 chunk slots and 4 float slots (one pass)
  {
    const bool dst16 = reinterpret_cast<uintptr_t>(dst) % 16 == 0 && dst_stride % 4 == 0;
    auto vec_ok = [&](const ppo_gather_segment& g) {
      return dst16 && g.kind == PPO_GATHER_FLOAT && reinterpret_cast<uintptr_t>(g.src) % 16 == 0 &&
             g.src_stride % 4 == 0 && g.width % 4 == 0 && g.dst_col % 4 == 0;
    };
    GatherArgs va{};
    int n = 0;
    int64_t chunks = 0, floats = 0;
    for (int pass = 0; pass < 2; ++pass)
      for (int s = 0; s < num_segments; ++s) {
        const ppo_gather_segment& g = segments[s];
        if (vec_ok(g) != (pass == 0)) continue;
        va.seg[n] = g;
        if (pass == 0) {
          va.vprefix[n] = static_cast<int32_t>(chunks);
          chunks += g.width / 4;
        } else {
          va.prefix[n] = static_cast<int32_t>(floats);
          floats += g.width;
        }
        if (pass == 0) va.num_vec = n + 1;
        ++n;
      }
    va.num_segments = num_segments;
    va.vprefix[va.num_vec] = static_cast<int32_t>(chunks);
    va.prefix[num_segments] = static_cast<int32_t>(floats);
    const int kv = static_cast<int>(ceil_div(chunks, static_cast<int64_t>(kWave)));
    const int ks = static_cast<int>(ceil_div(floats, static_cast<int64_t>(kWave)));
    if (va.num_vec > 0 && kv <= 4 && ks <= 4 && rows < (int64_t(1) << 30)) {
      auto gov = [&](auto kernel) {
        constexpr int R = kGatherRowsPerIter;
        // the blocks the device holds at once, or more where a wave would otherwise take more than kGatherMaxIters
        // iterations
        const int64_t need = ceil_div(rows, static_cast<int64_t>(kWavesPerBlock) * R);
        const int64_t res = resident_gather_blocks(kernel);
        const int64_t blocks = std::min<int64_t>(
            res > 0 ? std::max<int64_t>(std::min(need, res), ceil_div(need, kGatherMaxIters)) : need, 65536);
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kGatherThreads), 0,
                           static_cast<hipStream_t>(stream), perm, rows, src_rows, va, dst, dst_stride);
        return check_launch("gather_rows_vec_kernel");
      };
      constexpr int R = kGatherRowsPerIter;
#define PPO_GATHER_VEC(V)                                         \
  switch (ks) {                                                   \
    case 0: return gov(gather_rows_vec_kernel<V, 0, R>);          \
    case 1: return gov(gather_rows_vec_kernel<V, 1, R>);          \
    case 2: return gov(gather_rows_vec_kernel<V, 2, R>);          \
    case 3: return gov(gather_rows_vec_kernel<V, 3, R>);          \
    default: return gov(gather_rows_vec_kernel<V, 4, R>);         \
  }
      switch (kv) {
        case 1: PPO_GATHER_VEC(1)
        case 2: PPO_GATHER_VEC(2)
        case 3: PPO_GATHER_VEC(3)
        default: PPO_GATHER_VEC(4)
      }
#undef PPO_GATHER_VEC
    }
  }
  // the fewest slots that cover a row (a slot past the row still issues its load), 8 for wider rows (more passes)
  const int slots = static_cast<int>(std::min<int64_t>(ceil_div(total, static_cast<int64_t>(kWave)), 8));
  auto go = [&](auto kernel, int r) {
    const int64_t blocks = std::min<int64_t>(ceil_div(rows, static_cast<int64_t>(kWavesPerBlock) * r), 65536);
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kGatherThreads), 0,
                       static_cast<hipStream_t>(stream), perm, rows, src_rows, args, dst, dst_stride);
    return check_launch("gather_rows_kernel");
  };
#ifdef PPO_HIP_TUNING
  if (const char* e = std::getenv("PPO_HIP_GATHER_ROWS"); e != nullptr && std::atoi(e) == 2) {
    return slots <= 4 ? go(gather_rows_kernel<4, 2>, 2) : go(gather_rows_kernel<8, 2>, 2);
  }
#endif
  constexpr int R = kGatherRowsPerIter;
  switch (slots) {
    case 1: return go(gather_rows_kernel<1, R>, R);
    case 2: return go(gather_rows_kernel<2, R>, R);
    case 3: return go(gather_rows_kernel<3, R>, R);
    case 4: return go(gather_rows_kernel<4, R>, R);
    case 5: return go(gather_rows_kernel<5, R>, R);
    case 6: return go(gather_rows_kernel<6, R>, R);
    case 7: return go(gather_rows_kernel<7, R>, R);
    default: return go(gather_rows_kernel<8, R>, R);
  }
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
