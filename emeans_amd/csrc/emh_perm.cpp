// numpy's legacy permutation (RandomState(seed).permutation(n),
// crates/emeans-core/src/rng.rs:19-102): MT19937 words, numpy's masked
// rejection random_interval, and the shuffle from the last index down.
//
// Every training run draws two of these before its first batch can start
// (the initial centroids and the first epoch's order), so this file is plain
// host C++ built by the system C++ compiler, which turns the two-candidate
// rejection below into branch-free selects.

#include <cstddef>
#include <cstdint>
#include <utility>

namespace emh {
namespace host {

namespace {

constexpr int N = 624, M = 397;

struct Words {
  uint32_t mt[N];
  uint32_t out[N];  // the current block of tempered words
  int pos = N;

  explicit Words(uint32_t seed) {
    uint32_t s = seed;
    for (int i = 0; i < N; i++) {
      mt[i] = s;
      s = 1812433253u * (s ^ (s >> 30)) + (uint32_t)(i + 1);
    }
  }
  static uint32_t twist(uint32_t a, uint32_t b, uint32_t c) {
    const uint32_t y = (a & 0x80000000u) | (b & 0x7fffffffu);
    return c ^ (y >> 1) ^ ((0u - (y & 1u)) & 0x9908b0dfu);
  }
  static uint32_t temper(uint32_t y) {
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    return y ^ (y >> 18);
  }
  void refill() {
    int i = 0;
    for (; i < N - M; i++) mt[i] = twist(mt[i], mt[i + 1], mt[i + M]);
    for (; i < N - 1; i++) mt[i] = twist(mt[i], mt[i + 1], mt[i + M - N]);
    mt[N - 1] = twist(mt[N - 1], mt[0], mt[M - 1]);
    for (int j = 0; j < N; j++) out[j] = temper(mt[j]);
    pos = 0;
  }
  uint32_t next() {
    if (pos == N) refill();
    return out[pos++];
  }
  // random_interval(max) for 0 < max < 2^32: two candidate words are tested
  // at once, so the loop branches only when both are rejected; the words
  // consumed are the same as testing them one at a time.
  uint32_t interval(uint32_t max) {
    const uint32_t m = 0xffffffffu >> __builtin_clz(max);
    for (;;) {
      if (pos >= N - 1) {
        const uint32_t v = next() & m;
        if (v <= max) return v;
        continue;
      }
      const uint32_t v1 = out[pos] & m, v2 = out[pos + 1] & m;
      const bool a1 = v1 <= max, a2 = v2 <= max;
      if (a1 | a2) {
        pos += a1 ? 1 : 2;
        return a1 ? v1 : v2;
      }
      pos += 2;
    }
  }
  // random_interval(max) for max >= 2^32 (two words per candidate).
  uint64_t interval64(uint64_t max) {
    uint64_t mask = max;
    mask |= mask >> 1;
    mask |= mask >> 2;
    mask |= mask >> 4;
    mask |= mask >> 8;
    mask |= mask >> 16;
    mask |= mask >> 32;
    for (;;) {
      const uint64_t hi = next();
      const uint64_t v = ((hi << 32) | next()) & mask;
      if (v <= max) return v;
    }
  }
};

}  // namespace

void mt_permutation(uint32_t seed, size_t n, uint32_t* p) {
  Words w(seed);
  for (size_t i = 0; i < n; i++) p[i] = (uint32_t)i;
  size_t i = n;
  for (; i > 1 && i - 1 > 0xffffffffull; i--) std::swap(p[i - 1], p[w.interval64(i - 1)]);
  for (; i > 1; i--) std::swap(p[i - 1], p[w.interval((uint32_t)(i - 1))]);
}

}  // namespace host
}  // namespace emh
