// The update's mini-batch permutation (rsl_rl/storage/rollout_storage.py:232: `torch.randperm(B)`), host code.
//
// On the CPU, torch.randperm(n) is a Fisher-Yates shuffle driven by the CPU generator's 32-bit Mersenne Twister
// stream: r = identity; for i = 0 .. n-2: z = draw_i mod (n - i); swap(r[i], r[i + z]), which leaves the generator
// n - 1 draws further on.  The update takes its permutation from that generator so that the mini-batches are
// bit-identical to upstream's CPU run after the same seed; torch's loop takes ~13 ns per element (1.3 ms for the
// 98,304 rows of a 4096 x 24 rollout) while the GPU waits.  Here the same permutation and the same generator state
// are produced in three passes: all n - 1 draws (MT19937 twisted a block of 624 words at a time), all moduli (a
// vectorisable double quotient with an exact integer correction), then the swaps, which alone are sequential.
//
// The shuffle also runs as consecutive ranges of iterations [i0, i1) (ppo_host_randperm_range): iteration i only
// swaps positions >= i, so positions [0, i1) are final after the first range and their rows can be used while the
// rest of the shuffle runs; the generator record carries the stream position from one range to the next.
//
// The generator state is exchanged as the record torch.get_rng_state() returns (5056 bytes): the initial seed, the
// MT19937 read position (`left`, `next`) and its 624 state words (each stored in 64 bits), then cached normal
// samples that the shuffle does not touch.  The caller passes the record in and writes it back with
// torch.set_rng_state().
//
// The update also advances the generator past the samples upstream's stochastic forward draws and discards in every
// mini-batch (rsl_rl/models/mlp_model.py:103-106 via rsl_rl/algorithms/ppo.py:228-233): ppo_host_rng_skip moves the
// stream on by a number of draws without producing them, so the next rollout draws where upstream's would.
//
// MT19937 (Matsumoto & Nishimura, 1998): the standard recurrence and output tempering.
#include "common.hpp"

#include <cstring>
#include <vector>

namespace ppo {
namespace {

constexpr int kMtN = 624;
constexpr int kMtM = 397;
constexpr uint32_t kMtMatrixA = 0x9908b0dfu;
constexpr size_t kStateBytes = 5056;
constexpr size_t kWordsOffset = 24;  // uint64 seed, int32 left, int32 seeded, uint64 next

struct Mt19937 {
  uint32_t w[kMtN];
  int left;  // draws remaining before the next twist + 1 (torch's convention: 1 right after seeding)
  int next;  // index of the next word to temper

  static uint32_t mix(uint32_t u, uint32_t v, uint32_t far) {
    const uint32_t y = (u & 0x80000000u) | (v & 0x7fffffffu);
    return far ^ (y >> 1) ^ ((0u - (y & 1u)) & kMtMatrixA);  // branch-free, so the twist loops vectorise
  }
  // in place, in index order: word i combines words i, i+1 and i+M (mod N), the last ones already new
  void twist() {
    int i = 0;
    for (; i < kMtN - kMtM; ++i) w[i] = mix(w[i], w[i + 1], w[i + kMtM]);
    for (; i < kMtN - 1; ++i) w[i] = mix(w[i], w[i + 1], w[i + kMtM - kMtN]);
    w[kMtN - 1] = mix(w[kMtN - 1], w[0], w[kMtM - 1]);
    left = kMtN;
    next = 0;
  }

  static uint32_t temper(uint32_t y) {
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
  }

  // Advance the stream by `count` draws without producing them: only the twists matter (tempering touches the
  // outputs, not the state).
  void skip(int64_t count) {
    while (count > 0) {
      if (--left == 0) twist();
      const int64_t run = std::min<int64_t>(count, left);
      next += static_cast<int>(run);
      left -= static_cast<int>(run - 1);
      count -= run;
    }
  }

  // out[0 .. count): the next `count` draws.
  void draws(uint32_t* out, int64_t count) {
    int64_t k = 0;
    while (k < count) {
      if (--left == 0) twist();
      // the words [next, kMtN) can be tempered without another twist: left - 1 more draws after this one
      const int64_t run = std::min<int64_t>(count - k, left);
      for (int64_t j = 0; j < run; ++j) out[k + j] = temper(w[next + j]);
      next += static_cast<int>(run);
      left -= static_cast<int>(run - 1);
      k += run;
    }
  }
};

int load_state(const uint8_t* rec, Mt19937& mt) {
  int32_t left, seeded;
  uint64_t next;
  std::memcpy(&left, rec + 8, 4);
  std::memcpy(&seeded, rec + 12, 4);
  std::memcpy(&next, rec + 16, 8);
  PPO_REQUIRE(left >= 1 && left <= kMtN && next <= static_cast<uint64_t>(kMtN) && seeded == 1,
              "ppo_host_randperm: generator record not recognised (left=%d next=%llu seeded=%d)", left,
              (unsigned long long)next, seeded);
  for (int i = 0; i < kMtN; ++i) {
    uint64_t v;
    std::memcpy(&v, rec + kWordsOffset + 8 * static_cast<size_t>(i), 8);
    PPO_REQUIRE(v <= 0xffffffffull, "ppo_host_randperm: generator record not recognised (word %d)", i);
    mt.w[i] = static_cast<uint32_t>(v);
  }
  mt.left = left;
  mt.next = static_cast<int>(next);
  return PPO_OK;
}

void store_state(const Mt19937& mt, uint8_t* rec) {
  const int32_t left = mt.left;
  const uint64_t next = static_cast<uint64_t>(mt.next);
  std::memcpy(rec + 8, &left, 4);
  std::memcpy(rec + 16, &next, 8);
  for (int i = 0; i < kMtN; ++i) {
    const uint64_t v = mt.w[i];
    std::memcpy(rec + kWordsOffset + 8 * static_cast<size_t>(i), &v, 8);
  }
}

}  // namespace
}  // namespace ppo

using namespace ppo;

namespace ppo {
namespace {

// Iterations [i0, i1) of the shuffle on `out`, which holds the result of iterations [0, i0) (the identity for
// i0 = 0): z_i = draw mod (n - i), swap(out[i], out[i + z_i]).  Iteration i only touches positions >= i, so after
// the call out[0, i1) is final.
int shuffle_range(uint8_t* generator_state, size_t state_bytes, int64_t n, int64_t i0, int64_t i1, int64_t* out,
                  const char* who) {
  PPO_REQUIRE(generator_state != nullptr && out != nullptr, "%s: null pointer", who);
  PPO_REQUIRE(state_bytes == kStateBytes, "%s: generator record of %zu bytes (expected %zu)", who, state_bytes,
              kStateBytes);
  PPO_REQUIRE(n >= 1 && n < (int64_t(1) << 31), "%s: n=%lld", who, (long long)n);
  PPO_REQUIRE(i0 >= 0 && i0 <= i1 && i1 <= n - 1, "%s: iterations [%lld, %lld) outside [0, %lld)", who,
              (long long)i0, (long long)i1, (long long)(n - 1));
  Mt19937 mt;
  if (int rc = load_state(generator_state, mt)) return rc;
  if (i0 == 0)
    for (int64_t i = 0; i < n; ++i) out[i] = i;
  const int64_t m = i1 - i0;
  if (m > 0) {
    std::vector<uint32_t> z(static_cast<size_t>(m));
    mt.draws(z.data(), m);
    // z_i = draw_i mod (n - i) through a double quotient (exact operands < 2^32; the rounded quotient is at most
    // one too large, which the correction undoes), so the loop vectorises instead of issuing integer divides
    for (int64_t k = 0; k < m; ++k) {
      const double d = static_cast<double>(n - i0 - k), x = static_cast<double>(z[k]);
      double r = x - static_cast<double>(static_cast<int64_t>(x / d)) * d;
      r = r < 0.0 ? r + d : r;
      z[k] = static_cast<uint32_t>(r);
    }
    // the swaps are sequential; their targets are known, so the line of a later swap is fetched ahead
    constexpr int64_t kAhead = 16;
    for (int64_t k = 0; k < m; ++k) {
      const int64_t i = i0 + k;
      if (k + kAhead < m) __builtin_prefetch(out + i + kAhead + z[k + kAhead], 1);
      const int64_t j = i + z[k];
      const int64_t t = out[i];
      out[i] = out[j];
      out[j] = t;
    }
  }
  store_state(mt, generator_state);
  return PPO_OK;
}

}  // namespace
}  // namespace ppo

// Skip `draws` 32-bit outputs of the generator record's stream (no outputs produced).
extern "C" int ppo_host_rng_skip(uint8_t* generator_state, size_t state_bytes, int64_t draws) {
  PPO_REQUIRE(generator_state != nullptr, "ppo_host_rng_skip: null pointer");
  PPO_REQUIRE(state_bytes == kStateBytes, "ppo_host_rng_skip: generator record of %zu bytes (expected %zu)",
              state_bytes, kStateBytes);
  PPO_REQUIRE(draws >= 0, "ppo_host_rng_skip: draws=%lld", (long long)draws);
  Mt19937 mt;
  if (int rc = load_state(generator_state, mt)) return rc;
  mt.skip(draws);
  store_state(mt, generator_state);
  return PPO_OK;
}

extern "C" int ppo_host_randperm(uint8_t* generator_state, size_t state_bytes, int64_t n, int64_t* out) {
  return shuffle_range(generator_state, state_bytes, n, 0, n - 1, out, "ppo_host_randperm");
}

extern "C" int ppo_host_randperm_range(uint8_t* generator_state, size_t state_bytes, int64_t n, int64_t i0,
                                       int64_t i1, int64_t* out) {
  return shuffle_range(generator_state, state_bytes, n, i0, i1, out, "ppo_host_randperm_range");
}
