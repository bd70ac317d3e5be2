// numpy's legacy permutation (RandomState(seed).permutation(n),
// crates/emeans-core/src/rng.rs:19-102): MT19937 words, numpy's masked
// rejection random_interval, and the shuffle from the last index down.
//
// Every training run draws two of these before its first batch can start
// (the initial centroids and the first epoch's order), so the draws are
// restated for speed, consuming exactly the words numpy consumes:
//  - random_interval(max) takes the next word w while (w & mask) > max, and
//    max falls by one per draw: over the word stream that is one pass with a
//    running max that drops at each taken word. No word position depends on
//    the previous draw's value;
//  - in a chunk of S words the max falls by at most S, so a word at or below
//    max - S is taken and one above max is not, whatever came before it.
//    Chunks with no word in between and no mask change are decided without
//    the running max (8 words at a time with AVX2 where the CPU has it); the
//    rest go word by word;
//  - the swaps of a block's draws follow its scan, in draw order.
// Plain host C++, built by the system C++ compiler.

#include <immintrin.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <thread>
#include <utility>
#include <vector>

namespace emh {
namespace host {

namespace {

constexpr int N = 624, M = 397;

// Left-pack tables: for each 8-bit mask, the indices of its set bits in order.
struct PackLut {
  uint64_t idx[256];
  PackLut() {
    for (int msk = 0; msk < 256; msk++) {
      uint64_t v = 0;
      int o = 0;
      for (int b = 0; b < 8; b++)
        if (msk >> b & 1) v |= (uint64_t)b << (8 * o++);
      idx[msk] = v;
    }
  }
};
const PackLut kLut;

// Words k..e (e - k a multiple of 8) decided against thr: stores the taken
// (v <= thr) masked words in order at jb + nj and returns the new count;
// *unc gets whether some word lies in (thr, mx].
__attribute__((target("avx2"))) int pack_avx2(const uint32_t* out, int k, int e, uint32_t m,
                                              uint32_t thr, uint32_t mx, uint32_t* jb, int nj,
                                              uint32_t* unc) {
  const __m256i vm = _mm256_set1_epi32((int)m);
  const __m256i bias = _mm256_set1_epi32((int)0x80000000u);
  const __m256i vthr = _mm256_set1_epi32((int)(thr ^ 0x80000000u));
  const __m256i vmx = _mm256_set1_epi32((int)(mx ^ 0x80000000u));
  __m256i u = _mm256_setzero_si256();
  for (int t = k; t < e; t += 8) {
    const __m256i v = _mm256_and_si256(_mm256_loadu_si256((const __m256i*)(out + t)), vm);
    const __m256i vb = _mm256_xor_si256(v, bias);
    const __m256i gt = _mm256_cmpgt_epi32(vb, vthr);  // v > thr
    const __m256i gtm = _mm256_cmpgt_epi32(vb, vmx);  // v > mx
    u = _mm256_or_si256(u, _mm256_andnot_si256(gtm, gt));
    const int msk = ~_mm256_movemask_ps(_mm256_castsi256_ps(gt)) & 0xff;
    const __m256i perm = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)&kLut.idx[msk]));
    _mm256_storeu_si256((__m256i*)(jb + nj), _mm256_permutevar8x32_epi32(v, perm));
    nj += __builtin_popcount((unsigned)msk);
  }
  *unc = !_mm256_testz_si256(u, u);
  return nj;
}

const bool kAvx2 = __builtin_cpu_supports("avx2");

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
  __attribute__((target_clones("avx2", "default"))) void refill() {
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

// The draws for i = n - 1 .. 1 below 2^32 (max = i - 1 for draw i, from i = n
// down), a block of words at a time: sink(i0, jb, nj) gets the block's nj
// taken values in draw order, the first for i = i0.
template <class Sink>
void draws(Words& w, size_t i, Sink&& sink) {
  // The running max mx, its mask m, and lo = m >> 1, the max at which the
  // mask halves.
  uint32_t m = 0xffffffffu >> __builtin_clz((uint32_t)(i - 1));
  uint32_t lo = m >> 1;
  uint32_t jb[N + 8];    // a block's draws (slack for 8-wide stores)
  constexpr int S = 64;  // words decided together
  while (i > 1) {
    if (w.pos == N) w.refill();
    const size_t i0 = i;
    int k = w.pos, nj = 0;
    uint32_t mx = (uint32_t)(i - 1);
    while (k < N) {
      const int e = k + S < N ? k + S : N;
      // The max falls by at most e - k within the chunk: a word at or below
      // mx - S is taken whatever came before it, one above mx is not. With
      // no word in between and no mask change, the chunk needs no running max.
      if (mx > lo + (uint32_t)S) {
        const uint32_t thr = mx - (uint32_t)S;
        const int nj0 = nj;
        uint32_t unc = 0;
        int t = k;
        if (kAvx2) {
          const int e8 = k + ((e - k) & ~7);
          nj = pack_avx2(w.out, k, e8, m, thr, mx, jb, nj, &unc);
          t = e8;
        }
        for (; t < e; t++) {
          const uint32_t v = w.out[t] & m;
          jb[nj] = v;
          nj += (int)(v <= thr);
          unc |= (uint32_t)(v > thr) & (uint32_t)(v <= mx);
        }
        if (!unc) {
          mx -= (uint32_t)(nj - nj0);
          k = e;
          continue;
        }
        nj = nj0;
      }
      bool done = false;
      for (; k < e; k++) {
        const uint32_t v = w.out[k] & m;
        jb[nj] = v;
        const uint32_t acc = v <= mx;
        nj += (int)acc;
        mx -= acc;
        if (mx == lo) {
          if (mx == 0) {
            k++;
            done = true;
            break;
          }
          m >>= 1;
          lo = m >> 1;
        }
      }
      if (done) break;
    }
    w.pos = k;
    i = (size_t)mx + 1;
    sink(i0, jb, nj);
  }
}

}  // namespace

void mt_permutation(uint32_t seed, size_t n, uint32_t* p) {
  Words w(seed);
  if (n - 1 > 0xffffffffull || n < (size_t)(1u << 15)) {
    for (size_t i = 0; i < n; i++) p[i] = (uint32_t)i;
    size_t i = n;
    for (; i > 1 && i - 1 > 0xffffffffull; i--) std::swap(p[i - 1], p[w.interval64(i - 1)]);
    if (i <= 1) return;
    draws(w, i, [&](size_t i0, const uint32_t* jb, int nj) {
      for (int t = 0; t < nj; t++) std::swap(p[i0 - 1 - t], p[jb[t]]);
    });
    return;
  }
  // Larger n: the swaps depend only on the draws, so a second thread makes
  // them in draw order, following the drawing thread through `avail`.
  static thread_local std::vector<uint32_t> buf;  // this (drawing) thread's
  if (buf.size() < n) buf.resize(n);
  uint32_t* const js = buf.data();
  std::atomic<size_t> avail{0};
  const size_t total = n - 1;  // draws for i = n .. 2
  std::thread swapper([&] {
    for (size_t i = 0; i < n; i++) p[i] = (uint32_t)i;
    size_t t = 0;
    while (t < total) {
      size_t lim;
      while ((lim = avail.load(std::memory_order_acquire)) == t) _mm_pause();
      for (; t < lim; t++) std::swap(p[n - 1 - t], p[js[t]]);
    }
  });
  size_t made = 0;
  draws(w, n, [&](size_t, const uint32_t* jb, int nj) {
    std::memcpy(js + made, jb, (size_t)nj * 4);
    made += (size_t)nj;
    avail.store(made, std::memory_order_release);
  });
  swapper.join();
}

}  // namespace host
}  // namespace emh
