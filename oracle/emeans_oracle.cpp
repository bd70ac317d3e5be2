// emeans oracle: a CPU restatement of the reference's float order.
//
// TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP backend:
// only tests, the smoke check and the CPU-baseline leg of the benchmark load
// it. The product (emeans_amd) never links, loads or calls it.
//
// Every function restates one piece of the Rust reference (samhvw8/emeans,
// crates/emeans-core) and cites the file:line it follows. The float order is
// the reference CPU backend's (`cpu-fused` for top-1, `core/cpu.rs` for the
// exact ops): every dot product is one sequential fused multiply-add chain
// over the dimensions starting from +0; norms are sequential unfused f32 sums
// of rounded squares; scatter sums add rows in selection order; the EMA and
// split are plain f32 operations with no contraction. Build with
// -ffp-contract=off (the Makefile does) so that the compiler fuses nothing
// the reference does not.
//
// How each part is pinned (tests/test_oracle_golden.py):
//   RandomState, recipe, schedule      reference.json mt19937/recipes/alphas, bit-exact,
//                                      and numpy's own legacy RandomState
//   the whole training loop            reference.json runs (5 faiss runs: last-pass
//                                      labels and nsplit exact, obj 1e-5, centroids 1e-4)
//   top1 / knn                         f64 brute force (non-tie labels exact) and the
//                                      defining fma chain on small cases
//   scatter / ema / split / norms      f64 closed forms and the reference's special cases
//   dedup                              the reference's known-answer dedup tests
//                                      (emeans-cluster/tests/dedup.rs:112-300) on
//                                      their own data, and hand-built graphs

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <cstdio>
#include <map>
#include <set>
#include <unordered_map>
#include <vector>
#include <string>
#ifdef __AVX2__
#include <immintrin.h>
#endif
#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// ------------------------------------------------------------------ MT19937
// numpy legacy RandomState; crates/emeans-core/src/rng.rs:13-102.
struct RandomState {
  static constexpr int N = 624, M = 397;
  uint32_t mt[N];
  int pos;
  explicit RandomState(uint32_t seed) {  // rng.rs:19-29
    uint32_t s = seed;
    for (int i = 0; i < N; i++) {
      mt[i] = s;
      s = 1812433253u * (s ^ (s >> 30)) + (uint32_t)(i + 1);
    }
    pos = N;
  }
  void generate() {  // rng.rs:31-44
    for (int i = 0; i < N; i++) {
      uint32_t y = (mt[i] & 0x80000000u) | (mt[(i + 1) % N] & 0x7fffffffu);
      uint32_t v = mt[(i + M) % N] ^ (y >> 1);
      if (y & 1u) v ^= 0x9908b0dfu;
      mt[i] = v;
    }
    pos = 0;
  }
  uint32_t next_u32() {  // rng.rs:46-56
    if (pos == N) generate();
    uint32_t y = mt[pos++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    return y ^ (y >> 18);
  }
  uint64_t next_u64() {  // rng.rs:58-60
    uint64_t hi = next_u32();
    uint64_t lo = next_u32();
    return (hi << 32) | lo;
  }
  double random_sample() {  // rng.rs:63-67
    double a = (double)(next_u32() >> 5);
    double b = (double)(next_u32() >> 6);
    return (a * 67108864.0 + b) / 9007199254740992.0;
  }
  uint64_t random_interval(uint64_t max) {  // rng.rs:70-92
    if (max == 0) return 0;
    uint64_t mask = max;
    for (int s : {1, 2, 4, 8, 16, 32}) mask |= mask >> s;
    if (max <= 0xffffffffull) {
      for (;;) {
        uint64_t v = (uint64_t)next_u32() & mask;
        if (v <= max) return v;
      }
    }
    for (;;) {
      uint64_t v = next_u64() & mask;
      if (v <= max) return v;
    }
  }
  void permutation(size_t n, uint32_t* out) {  // rng.rs:95-102
    for (size_t i = 0; i < n; i++) out[i] = (uint32_t)i;
    for (size_t i = n; i-- > 1;) {
      size_t j = (size_t)random_interval(i);
      std::swap(out[i], out[j]);
    }
  }
};

// ------------------------------------------------------------------- recipe
// crates/emeans-core/src/recipe.rs
constexpr double ALPHA_MIN_FACTOR = 0.1;       // recipe.rs:10
constexpr size_t CHECK_UNUSED_EVERY = 5;       // recipe.rs:12
constexpr float INIT_USAGE = 1.0f / 65536.0f;  // recipe.rs:14
constexpr double SPLIT_EPSILON = 1e-4;         // recipe.rs:16
constexpr double UNUSED_THRESHOLD = 0.1;       // recipe.rs:18
constexpr size_t NO_REVIVAL_MAX_D = 2;         // recipe.rs:20
constexpr size_t AUTO_QUALITY_MAX_D = 16;      // recipe.rs:22

enum Law { LAW_AUTO = 0, LAW_THROUGHPUT = 1, LAW_QUALITY = 2 };

size_t round_power_of_two(double value) {  // recipe.rs:69-80
  if (value <= 1.0) return 1;
  double low = std::ldexp(1.0, (int)std::floor(std::log2(value)));
  double high = 2.0 * low;
  return (size_t)((value / low < high / value) ? low : high);
}

double step_law(size_t n, size_t k, double nepochs, size_t b) {  // recipe.rs:83-91
  double a = 0.8244 * std::pow((double)k, -0.4617) * std::pow((double)b, 0.9003) *
             std::pow((double)n, -0.4498) * std::pow(nepochs, -0.1057);
  return std::min(std::max(a, 1e-4), 1.0);
}

// recipe.rs:96-124; `law` already resolved when batch_size == 0 (None).
void resolve_batch_and_step(size_t n, size_t k, double nepochs, int law, size_t batch_size,
                            int has_alpha0, double alpha0, size_t* b_out, double* a_out) {
  size_t b;
  if (batch_size > 0) {
    b = std::min(batch_size, n);
  } else {
    double c = law == LAW_THROUGHPUT ? 0.035134 : 0.00439175;
    double raw = c * std::pow((double)k, 0.134749) * std::pow((double)n, 0.876473) *
                 std::pow(nepochs, 0.813344);
    b = round_power_of_two(raw);
    if (law == LAW_THROUGHPUT)
      b = std::min(b, round_power_of_two((double)n / 2.0));
    else
      b = std::min(b, n / 2);
    b = std::max(std::min(b, n), (size_t)1);
  }
  *b_out = b;
  *a_out = has_alpha0 ? alpha0 : step_law(n, k, nepochs, b);
}

std::vector<size_t> epoch_rows(size_t n, double nepochs) {  // recipe.rs:127-140
  double whole = std::floor(nepochs);
  size_t remainder = (size_t)std::nearbyint((nepochs - whole) * (double)n);
  size_t w = (size_t)whole;
  if (w == 0) return {remainder};
  std::vector<size_t> rows(w - 1, n);
  if (remainder > 0) rows.push_back(remainder);
  rows.push_back(n);
  return rows;
}

uint32_t epoch_seed(uint32_t seed, size_t epoch) {  // recipe.rs:143-145
  return (uint32_t)(((uint64_t)seed * 1000003ull + (uint64_t)epoch) % (1ull << 32));
}

double scheduled_alpha(double alpha0, size_t step, size_t total) {  // recipe.rs:148-152
  double fraction = (double)std::min(step, total) / (double)std::max(total, (size_t)1);
  double cosine = 0.5 * (1.0 + std::cos(M_PI * fraction));
  return alpha0 * (ALPHA_MIN_FACTOR + (1.0 - ALPHA_MIN_FACTOR) * cosine);
}

// -------------------------------------------------------------- f32 helpers

// Sequential f32 sum of rounded squares: assign.rs:150-155 (`row_norms`).
inline float sq_norm(const float* r, size_t d) {
  float s = 0.0f;
  for (size_t t = 0; t < d; t++) {
    float p = r[t] * r[t];
    s = s + p;
  }
  return s;
}

// faiss normalize_into for one row: core/cpu.rs:219-230 (= model.rs:954-967).
inline void normalize_row(float* r, size_t d) {
  float mx = 0.0f;
  for (size_t t = 0; t < d; t++) mx = std::fmax(mx, std::fabs(r[t]));
  float s = mx > 0.0f ? mx : 1.0f;
  for (size_t t = 0; t < d; t++) r[t] = r[t] / s;
  float norm = std::sqrt(sq_norm(r, d));
  s = norm > 0.0f ? norm : 1.0f;
  for (size_t t = 0; t < d; t++) r[t] = r[t] / s;
}

// numpy FLOAT_pairwise_sum: model.rs:970-1002.
float numpy_sum_f32(const float* a, size_t n) {
  if (n < 8) {
    float res = 0.0f;
    for (size_t i = 0; i < n; i++) res = res + a[i];
    return res;
  } else if (n <= 128) {
    float r[8];
    for (int j = 0; j < 8; j++) r[j] = a[j];
    size_t i = 8;
    for (; i < n - n % 8; i += 8)
      for (int j = 0; j < 8; j++) r[j] = r[j] + a[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; i++) res = res + a[i];
    return res;
  } else {
    size_t n2 = n / 2;
    n2 -= n2 % 8;
    return numpy_sum_f32(a, n2) + numpy_sum_f32(a + n2, n - n2);
  }
}

// --------------------------------------------------------------- top-1 (cpu-fused)
// assign/fused.rs:111-301 and assign.rs:423-502. Each dot is one fma chain over
// t = 0..d-1 starting from +0 (fused.rs:241-260, test 383-404). IP: the
// largest dot, L2: the smallest `cnorm[j] - 2 dot`; a strict scan in column
// order, so ties keep the lowest id (assign.rs:420-493). Score: the dot (IP)
// or max(|x|^2 + v, 0) (assign.rs:497-502).

constexpr int MR = 6;   // rows per microkernel tile (fused.rs:23)
constexpr int NR = 16;  // centroids per microkernel tile (fused.rs:25)

// acc[i][j] = fma chain over t of a[t][i] * b[t][j] (packed panels).
inline void micro(const float* a, const float* b, size_t d, float acc[MR][NR]) {
#ifdef __AVX2__
  __m256 c[MR][2];
  for (int i = 0; i < MR; i++) c[i][0] = c[i][1] = _mm256_setzero_ps();
  for (size_t t = 0; t < d; t++) {
    __m256 b0 = _mm256_loadu_ps(b + t * NR);
    __m256 b1 = _mm256_loadu_ps(b + t * NR + 8);
    for (int i = 0; i < MR; i++) {
      __m256 ai = _mm256_broadcast_ss(a + t * MR + i);
      c[i][0] = _mm256_fmadd_ps(ai, b0, c[i][0]);
      c[i][1] = _mm256_fmadd_ps(ai, b1, c[i][1]);
    }
  }
  for (int i = 0; i < MR; i++) {
    _mm256_storeu_ps(acc[i], c[i][0]);
    _mm256_storeu_ps(acc[i] + 8, c[i][1]);
  }
#else
  for (int i = 0; i < MR; i++)
    for (int j = 0; j < NR; j++) acc[i][j] = 0.0f;
  for (size_t t = 0; t < d; t++)
    for (int i = 0; i < MR; i++) {
      float ai = a[t * MR + i];
      for (int j = 0; j < NR; j++) acc[i][j] = std::fma(ai, b[t * NR + j], acc[i][j]);
    }
#endif
}

// Rows `r` of a selection: x[ids[r]] when ids, else x[r].
inline const float* row_of(const float* x, const uint32_t* ids, size_t r, size_t d) {
  return x + (size_t)(ids ? ids[r] : r) * d;
}

void pack_centroids(const float* c, size_t k, size_t d, std::vector<float>& out) {  // fused.rs:86-98
  size_t panels = (k + NR - 1) / NR;
  out.assign(panels * d * NR, 0.0f);
  for (size_t p = 0; p < panels; p++)
    for (size_t j = 0; j < (size_t)NR && p * NR + j < k; j++)
      for (size_t t = 0; t < d; t++) out[p * d * NR + t * NR + j] = c[(p * NR + j) * d + t];
}

// Fused top-1 of selection positions [lo, hi): labels/scores written at the positions.
void top1(const float* x, size_t d, const uint32_t* ids, size_t lo, size_t hi, const float* c,
          size_t k, int ip, uint32_t* labels, float* scores) {
  if (hi <= lo) return;
  std::vector<float> cn(k);
  if (!ip)
    for (size_t j = 0; j < k; j++) cn[j] = sq_norm(c + j * d, d);  // assign.rs:346-349
  std::vector<float> bp;
  pack_centroids(c, k, d, bp);
  size_t panels = (k + NR - 1) / NR;
  size_t n = hi - lo;
  size_t tasks = (n + MR - 1) / MR;
#pragma omp parallel for schedule(dynamic, 4)
  for (size_t tsk = 0; tsk < tasks; tsk++) {
    size_t r0 = lo + tsk * MR;
    size_t nr = std::min((size_t)MR, hi - r0);
    std::vector<float> a(d * MR, 0.0f);
    for (size_t i = 0; i < nr; i++) {
      const float* xr = row_of(x, ids, r0 + i, d);
      for (size_t t = 0; t < d; t++) a[t * MR + i] = xr[t];
    }
    float best[MR];
    uint32_t bj[MR];
    for (int i = 0; i < MR; i++) {
      best[i] = ip ? -INFINITY : INFINITY;
      bj[i] = 0;
    }
    float acc[MR][NR];
    for (size_t p = 0; p < panels; p++) {
      micro(a.data(), bp.data() + p * d * NR, d, acc);
      size_t cols = std::min((size_t)NR, k - p * NR);
      for (size_t i = 0; i < nr; i++)
        for (size_t j = 0; j < cols; j++) {
          size_t id = p * NR + j;
          if (ip) {
            float v = acc[i][j];
            if (v > best[i]) {
              best[i] = v;
              bj[i] = (uint32_t)id;
            }
          } else {
            float two = 2.0f * acc[i][j];
            float v = cn[id] - two;
            if (v < best[i]) {
              best[i] = v;
              bj[i] = (uint32_t)id;
            }
          }
        }
    }
    for (size_t i = 0; i < nr; i++) {
      labels[r0 + i] = bj[i];
      if (ip) {
        scores[r0 + i] = best[i];
      } else {
        float xn = sq_norm(row_of(x, ids, r0 + i, d), d);
        scores[r0 + i] = std::fmax(xn + best[i], 0.0f);
      }
    }
  }
}

// ------------------------------------------------------------ scatter / EMA / split

// core/cpu.rs:118-143 + scatter_rows 337-375: counts and per-label sums of the
// selected rows, added in selection order in f32; sums and counts overwritten;
// `acc += sums` when given. Labels are read at the selection positions.
void scatter_add(const float* x, size_t d, const uint32_t* ids, size_t lo, size_t hi,
                 const uint32_t* labels, size_t k, float* sums, uint32_t* counts, float* acc) {
  // group_by_label (cpu.rs:233-252): stable counting sort.
  std::vector<size_t> start(k + 1, 0);
  for (size_t p = lo; p < hi; p++) start[labels[p] + 1]++;
  for (size_t j = 0; j < k; j++) start[j + 1] += start[j];
  std::vector<size_t> fill(start.begin(), start.end() - 1), order(hi - lo);
  for (size_t p = lo; p < hi; p++) order[fill[labels[p]]++] = p;
  for (size_t j = 0; j < k; j++) counts[j] = (uint32_t)(start[j + 1] - start[j]);
#pragma omp parallel for schedule(dynamic, 8)
  for (size_t j = 0; j < k; j++) {
    float* s = sums + j * d;
    for (size_t t = 0; t < d; t++) s[t] = 0.0f;
    for (size_t q = start[j]; q < start[j + 1]; q++) {
      const float* r = row_of(x, ids, order[q], d);
      for (size_t t = 0; t < d; t++) s[t] = s[t] + r[t];
    }
    if (acc)
      for (size_t t = 0; t < d; t++) acc[j * d + t] = acc[j * d + t] + s[t];
  }
}

// core/cpu.rs:389-432 (`ema_here`): faiss update in f32, no FMA.
void ema_update(float* pos, float* usage, const float* sums, const uint32_t* counts, size_t k,
                size_t d, float alpha, float decay, int replace) {
  if (!replace)
    for (size_t j = 0; j < k; j++) usage[j] = usage[j] * decay;
#pragma omp parallel for schedule(static)
  for (size_t j = 0; j < k; j++) {
    if (counts[j] == 0) continue;
    float count = (float)counts[j];
    float retained = replace ? 0.0f : usage[j];
    float step = alpha * count;
    float mass = retained + step;
    float weight = step / mass;
    for (size_t t = 0; t < d; t++) {
      float mean = sums[j * d + t] / count;
      float& cc = pos[j * d + t];
      if (weight == 1.0f) {
        cc = mean;
      } else {
        float diff = mean - cc;
        float w = weight * diff;
        cc = cc + w;
      }
    }
    usage[j] = mass;
  }
}

// core/mod.rs:374-399 (`apply_splits`).
void apply_splits(float* pos, float* usage, size_t d, const uint32_t* pairs, size_t npairs) {
  const float eps = (float)SPLIT_EPSILON;
  std::vector<float> donor(d), child(d);
  for (size_t q = 0; q < npairs; q++) {
    size_t s = pairs[2 * q], t = pairs[2 * q + 1];
    const float* c = pos + s * d;
    bool same = true;
    for (size_t i = 0; i < d; i++) {
      float off = eps * (i % 2 == 0 ? 1.0f : -1.0f);
      float lo = 1.0f - off, hi = 1.0f + off;
      donor[i] = c[i] * lo;
      child[i] = c[i] * hi;
      same = same && donor[i] == child[i];
    }
    if (same) {
      float up = std::nextafter(child[0], INFINITY);
      child[0] = std::isfinite(up) ? up : std::nextafter(child[0], -INFINITY);
    }
    float half = usage[s] / 2.0f;
    usage[s] = half;
    std::memcpy(pos + s * d, donor.data(), d * 4);
    usage[t] = half;
    std::memcpy(pos + t * d, child.data(), d * 4);
  }
}

// core/mod.rs:339-370 (`plan_revival`): (donor, dead) pairs.
std::vector<std::pair<uint32_t, uint32_t>> plan_revival(const float* usage, size_t k, double tau,
                                                        RandomState& rng) {
  float total = numpy_sum_f32(usage, k);
  float threshold = (total * (float)tau) / (float)k;
  std::vector<char> unused(k), donors(k);
  size_t n_unused = 0, n_donors = 0;
  for (size_t j = 0; j < k; j++) {
    unused[j] = usage[j] < threshold;
    n_unused += unused[j];
    donors[j] = !unused[j] && usage[j] > 0.0f;
    n_donors += donors[j];
  }
  size_t nsplit = std::min(n_unused, n_donors);
  std::vector<std::pair<uint32_t, uint32_t>> plan;
  if (nsplit == 0) return plan;
  std::vector<double> uni(k);
  for (size_t j = 0; j < k; j++) uni[j] = std::max(rng.random_sample(), 2.2250738585072014e-308);
  std::vector<std::pair<double, size_t>> keyed;
  for (size_t j = 0; j < k; j++)
    if (donors[j]) keyed.push_back({(double)std::log(usage[j]) - std::log(-std::log(uni[j])), j});
  // Larger key first (total order), equal keys: higher index first.
  auto total_key = [](double v) {
    int64_t b;
    std::memcpy(&b, &v, 8);
    return b ^ (int64_t)(((uint64_t)(b >> 63)) >> 1);
  };
  std::stable_sort(keyed.begin(), keyed.end(), [&](const auto& a, const auto& b) {
    int64_t ka = total_key(a.first), kb = total_key(b.first);
    if (ka != kb) return ka > kb;
    return a.second > b.second;
  });
  size_t t = 0;
  for (size_t q = 0; q < nsplit; q++) {
    while (!unused[t]) t++;
    plan.push_back({(uint32_t)keyed[q].second, (uint32_t)t});
    t++;
  }
  return plan;
}

// core/mod.rs:404-429 (`closing_means`).
void closing_means(const float* positions, const float* sums, const double* counts, size_t k,
                   size_t d, int spherical, float* out) {
  std::memcpy(out, positions, k * d * 4);
  for (size_t j = 0; j < k; j++) {
    float* c = out + j * d;
    if (counts[j] > 0.0) {
      float nf = (float)counts[j];
      for (size_t t = 0; t < d; t++) c[t] = sums[j * d + t] / nf;
    }
    if (spherical) normalize_row(c, d);
  }
}

// ------------------------------------------------------------------ top-k
// Exact kNN by inner product (core/src/knn.rs:53-107; reference.rs:48-84):
// best first by larger score then lower id; exclude_self skips j == i; pad
// id u32::MAX, score -inf. Dots are the fma chain of the fused top-1 (the
// reference CPU kNN takes its dots from the un-vendored `gemm` crate, whose
// order the reference's own tests pin only to 1e-5).
void knn(const float* q, size_t m, const float* data, size_t n, size_t d, size_t kk,
         int exclude_self, uint32_t* ids, float* sims) {
  std::vector<float> bp;
  pack_centroids(data, n, d, bp);
  size_t panels = (n + NR - 1) / NR;
  size_t tasks = (m + MR - 1) / MR;
#pragma omp parallel for schedule(dynamic, 1)
  for (size_t tsk = 0; tsk < tasks; tsk++) {
    size_t r0 = tsk * MR, nr = std::min((size_t)MR, m - r0);
    std::vector<float> a(d * MR, 0.0f);
    for (size_t i = 0; i < nr; i++)
      for (size_t t = 0; t < d; t++) a[t * MR + i] = q[(r0 + i) * d + t];
    std::vector<float> sc(MR * kk, -INFINITY);
    std::vector<uint32_t> id(MR * kk, 0xffffffffu);
    std::vector<size_t> worst(MR, 0);
    float acc[MR][NR];
    for (size_t p = 0; p < panels; p++) {
      micro(a.data(), bp.data() + p * d * NR, d, acc);
      size_t cols = std::min((size_t)NR, n - p * NR);
      for (size_t i = 0; i < nr; i++) {
        float* s = &sc[i * kk];
        uint32_t* ii = &id[i * kk];
        for (size_t jj = 0; jj < cols; jj++) {
          size_t j = p * NR + jj;
          if (exclude_self && j == r0 + i) continue;
          float v = acc[i][jj];
          size_t w = worst[i];
          // Ids arrive in increasing order: replace the worst kept entry (lowest
          // score, then highest id) only when strictly better (knn.rs:82-96).
          if (v > s[w]) {
            s[w] = v;
            ii[w] = (uint32_t)j;
            size_t nw = 0;
            for (size_t t = 1; t < kk; t++) {
              bool worse = s[t] < s[nw] || (s[t] == s[nw] && ii[t] > ii[nw]);
              if (worse) nw = t;
            }
            worst[i] = nw;
          }
        }
      }
    }
    for (size_t i = 0; i < nr; i++) {
      std::vector<std::pair<float, uint32_t>> pr(kk);
      for (size_t t = 0; t < kk; t++) pr[t] = {sc[i * kk + t], id[i * kk + t]};
      // knn.rs:97-99: score descending in IEEE total order, then id ascending.
      std::sort(pr.begin(), pr.end(), [](const auto& a, const auto& b) {
        int32_t ka, kb;
        std::memcpy(&ka, &a.first, 4);
        std::memcpy(&kb, &b.first, 4);
        ka ^= (int32_t)(((uint32_t)(ka >> 31)) >> 1);
        kb ^= (int32_t)(((uint32_t)(kb >> 31)) >> 1);
        if (ka != kb) return ka > kb;
        return a.second < b.second;
      });
      for (size_t t = 0; t < kk; t++) {
        ids[(r0 + i) * kk + t] = pr[t].second;
        sims[(r0 + i) * kk + t] = pr[t].second == 0xffffffffu ? -INFINITY : pr[t].first;
      }
    }
  }
}

}  // namespace

// =================================================================== C ABI
extern "C" {

// --- RandomState
void* orc_rng_new(uint32_t seed) { return new RandomState(seed); }
void orc_rng_free(void* r) { delete (RandomState*)r; }
double orc_rng_random_sample(void* r) { return ((RandomState*)r)->random_sample(); }
void orc_rng_permutation(void* r, uint64_t n, uint32_t* out) {
  ((RandomState*)r)->permutation(n, out);
}

// --- recipe
void orc_resolve_batch_and_step(uint64_t n, uint64_t k, double nepochs, int law,
                                uint64_t batch_size, int has_alpha0, double alpha0,
                                uint64_t* b, double* a) {
  size_t bb;
  resolve_batch_and_step(n, k, nepochs, law, batch_size, has_alpha0, alpha0, &bb, a);
  *b = bb;
}
int orc_resolve_law(int law, uint64_t d) {  // recipe.rs:45-53
  if (law == LAW_AUTO) return d <= AUTO_QUALITY_MAX_D ? LAW_QUALITY : LAW_THROUGHPUT;
  return law;
}
uint64_t orc_epoch_rows(uint64_t n, double nepochs, uint64_t* out, uint64_t cap) {
  auto r = epoch_rows(n, nepochs);
  for (size_t i = 0; i < r.size() && i < cap; i++) out[i] = r[i];
  return r.size();
}
double orc_scheduled_alpha(double alpha0, uint64_t step, uint64_t total) {
  return scheduled_alpha(alpha0, step, total);
}
uint32_t orc_epoch_seed(uint32_t seed, uint64_t e) { return epoch_seed(seed, e); }
double orc_unused_threshold(uint64_t d) { return d <= NO_REVIVAL_MAX_D ? 0.0 : UNUSED_THRESHOLD; }
float orc_numpy_sum_f32(const float* a, uint64_t n) { return numpy_sum_f32(a, n); }

// --- the layer-1 ops, CPU float order
void orc_top1(const float* x, uint64_t d, const uint32_t* ids, uint64_t lo, uint64_t hi,
              const float* c, uint64_t k, int ip, uint32_t* labels, float* scores) {
  top1(x, d, ids, lo, hi, c, k, ip, labels, scores);
}
void orc_row_norms(const float* m, uint64_t rows, uint64_t d, float* out) {
#pragma omp parallel for
  for (size_t i = 0; i < rows; i++) out[i] = sq_norm(m + i * d, d);
}
void orc_normalize_rows(const float* src, uint64_t rows, uint64_t d, float* dst) {
#pragma omp parallel for
  for (size_t i = 0; i < rows; i++) {
    std::memcpy(dst + i * d, src + i * d, d * 4);
    normalize_row(dst + i * d, d);
  }
}
void orc_scatter_add(const float* x, uint64_t d, const uint32_t* ids, uint64_t lo, uint64_t hi,
                     const uint32_t* labels, uint64_t k, float* sums, uint32_t* counts,
                     float* acc) {
  scatter_add(x, d, ids, lo, hi, labels, k, sums, counts, acc);
}
void orc_ema_update(float* pos, float* usage, const float* sums, const uint32_t* counts,
                    uint64_t k, uint64_t d, double alpha) {
  // EmaStep::new (core/mod.rs:189-197): f64 alpha cast like numpy.
  ema_update(pos, usage, sums, counts, k, d, (float)alpha, (float)(1.0 - alpha), alpha == 1.0);
}
void orc_apply_splits(float* pos, float* usage, uint64_t d, const uint32_t* pairs,
                      uint64_t npairs) {
  apply_splits(pos, usage, d, pairs, npairs);
}
// Returns the number of pairs written to `pairs` (2 u32 each, capacity k pairs).
uint64_t orc_plan_revival(const float* usage, uint64_t k, double tau, void* rng,
                          uint32_t* pairs) {
  auto p = plan_revival(usage, k, tau, *(RandomState*)rng);
  for (size_t q = 0; q < p.size(); q++) {
    pairs[2 * q] = p[q].first;
    pairs[2 * q + 1] = p[q].second;
  }
  return p.size();
}
void orc_closing_means(const float* positions, const float* sums, const double* counts,
                       uint64_t k, uint64_t d, int spherical, float* out) {
  closing_means(positions, sums, counts, k, d, spherical, out);
}
void orc_knn(const float* q, uint64_t m, const float* data, uint64_t n, uint64_t d, uint64_t kk,
             int exclude_self, uint32_t* ids, float* sims) {
  knn(q, m, data, n, d, kk, exclude_self, ids, sims);
}
void orc_set_threads(int t) {
#ifdef _OPENMP
  if (t > 0) omp_set_num_threads(t);
#else
  (void)t;
#endif
}
int orc_get_threads() {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

// --- Emeans::train on the CPU device loop (model.rs:700-811 + core/train.rs:60-303).
struct OrcTrainCfg {
  uint64_t k, d;
  double nepochs;
  uint64_t batch_size;  // 0 = batch law
  int has_alpha0;
  double alpha0;
  int batch_law;  // 0 auto, 1 throughput, 2 quality
  uint32_t seed;
  int spherical;
  int has_unused_threshold;
  double unused_threshold;
  uint64_t assignment_chunk_size;  // 0 = 65536
};

struct OrcTrainOut {
  float* centroids;   // k*d
  float* positions;   // k*d
  float* usage;       // k
  int32_t* labels;    // n (last-pass labels)
  double* obj;        // per epoch (capacity 64)
  double* imbalance;  // per epoch
  uint64_t* nsplit;   // per epoch
  uint64_t n_epochs;
  uint64_t n_splits;
  uint64_t batch_size;
  double alpha0;
  uint64_t total_steps;
};

// Emeans::train_rows (model.rs:772-811) from its three starts: init == null
// and positions == null: k sampled rows (train); init: given centroids
// (train_from -> begin, model.rs:306-316); positions + usage: saved EMA state
// (train_resume -> begin_with_state, model.rs:318-336). Returns 0, or 1 for
// bad shapes, 2 for state the reference refuses (non-finite centroids or
// positions, masses not finite and >= 0).
int orc_train_from(const float* x, uint64_t n, const OrcTrainCfg* cfg, const float* init,
                   const float* positions, const float* usage_in, OrcTrainOut* out) {
  const size_t k = cfg->k, d = cfg->d;
  if (n < k || d == 0 || k == 0) return 1;
  const bool sph = cfg->spherical != 0;
  const bool ip = sph;
  std::vector<float> pos(k * d);
  std::vector<float> usage(k, INIT_USAGE);
  if (positions) {
    if (!usage_in) return 1;
    std::memcpy(pos.data(), positions, k * d * 4);
    std::memcpy(usage.data(), usage_in, k * 4);
    for (size_t j = 0; j < k; j++)
      if (!std::isfinite(usage[j]) || usage[j] < 0.0f) return 2;
  } else {
    if (init) {
      std::memcpy(pos.data(), init, k * d * 4);
    } else if (n == k) {  // model.rs:789-796
      std::memcpy(pos.data(), x, k * d * 4);
    } else {
      std::vector<uint32_t> perm(n);
      RandomState(cfg->seed).permutation(n, perm.data());
      for (size_t j = 0; j < k; j++) std::memcpy(&pos[j * d], x + (size_t)perm[j] * d, d * 4);
    }
    if (sph)
      for (size_t j = 0; j < k; j++) normalize_row(&pos[j * d], d);  // model.rs:311-314
  }
  for (size_t i = 0; i < k * d; i++)
    if (!std::isfinite(pos[i])) return 2;  // model.rs:349-352
  // Recipe (recipe.rs:200-254).
  int law = orc_resolve_law(cfg->batch_law, d);
  size_t bsz;
  double alpha0;
  resolve_batch_and_step(n, k, cfg->nepochs, law, cfg->batch_size, cfg->has_alpha0, cfg->alpha0,
                         &bsz, &alpha0);
  auto erows = epoch_rows(n, cfg->nepochs);
  size_t total_steps = 0;
  for (size_t r : erows) total_steps += (r + bsz - 1) / bsz;
  double tau = cfg->has_unused_threshold ? cfg->unused_threshold : orc_unused_threshold(d);
  size_t chunk = cfg->assignment_chunk_size ? cfg->assignment_chunk_size : 65536;
  // Device loop (train.rs:92-303) on host vectors.
  std::vector<uint32_t> order(n), labels_ep(n);
  std::vector<float> scores_ep(n), readout(sph ? k * d : k), sums(k * d), pass(k * d, 0.0f);
  std::vector<uint32_t> counts(k);
  RandomState split_rng(cfg->seed);
  size_t n_splits = 0, step = 0;
  std::vector<double> pass_counts(k, 0.0);
  for (size_t epoch = 0; epoch < erows.size(); epoch++) {
    size_t rows = erows[epoch];
    bool last = epoch + 1 == erows.size();
    RandomState(epoch_seed(cfg->seed, epoch)).permutation(n, order.data());
    size_t splits_before = n_splits;
    for (size_t b = 0; b < rows; b += bsz) {
      size_t e = std::min(b + bsz, rows);
      if (sph)
        orc_normalize_rows(pos.data(), k, d, readout.data());
      else
        orc_row_norms(pos.data(), k, d, readout.data());
      const float* cents = sph ? readout.data() : pos.data();
      for (size_t c0 = b; c0 < e; c0 += chunk) {
        size_t c1 = std::min(c0 + chunk, e);
        top1(x, d, order.data(), c0, c1, cents, k, ip, labels_ep.data(), scores_ep.data());
      }
      scatter_add(x, d, order.data(), b, e, labels_ep.data(), k, sums.data(), counts.data(),
                  last ? pass.data() : nullptr);
      double alpha = scheduled_alpha(alpha0, step, total_steps);
      orc_ema_update(pos.data(), usage.data(), sums.data(), counts.data(), k, d, alpha);
      if ((step + 1) % CHECK_UNUSED_EVERY == 0) {
        auto plan = plan_revival(usage.data(), k, tau, split_rng);
        std::vector<uint32_t> flat;
        for (auto& pr : plan) {
          flat.push_back(pr.first);
          flat.push_back(pr.second);
        }
        apply_splits(pos.data(), usage.data(), d, flat.data(), plan.size());
        n_splits += plan.size();
      }
      step++;
    }
    // Epoch statistics (train.rs:224-279).
    double obj_epoch = 0.0;
    for (size_t b = 0; b < rows; b += bsz) {
      size_t e = std::min(b + bsz, rows);
      double obj_batch = 0.0;
      for (size_t c0 = b; c0 < e; c0 += chunk) {
        size_t c1 = std::min(c0 + chunk, e);
        double obj = 0.0;
        if (sph) {
          obj += 2.0 * (double)(c1 - c0);
          for (size_t p = c0; p < c1; p++) obj += (double)(-2.0f * scores_ep[p]);
        } else {
          for (size_t p = c0; p < c1; p++) obj += (double)scores_ep[p];
        }
        obj_batch += obj;
      }
      obj_epoch += obj_batch;
    }
    std::vector<uint64_t> hist(k, 0);
    for (size_t p = 0; p < rows; p++) hist[labels_ep[p]]++;
    double count_square = 0.0;
    for (size_t j = 0; j < k; j++) count_square += (double)hist[j] * (double)hist[j];
    if (epoch < 64) {
      out->obj[epoch] = obj_epoch;
      out->imbalance[epoch] = (double)k * count_square / ((double)rows * (double)rows);
      out->nsplit[epoch] = n_splits - splits_before;
    }
    if (last) {
      for (size_t j = 0; j < k; j++) pass_counts[j] = (double)hist[j];
      if (out->labels) {
        for (size_t i = 0; i < n; i++) out->labels[i] = -1;
        for (size_t p = 0; p < rows; p++) out->labels[order[p]] = (int32_t)labels_ep[p];
      }
    }
  }
  closing_means(pos.data(), pass.data(), pass_counts.data(), k, d, sph, out->centroids);
  if (out->positions) std::memcpy(out->positions, pos.data(), k * d * 4);
  if (out->usage) std::memcpy(out->usage, usage.data(), k * 4);
  out->n_epochs = erows.size();
  out->n_splits = n_splits;
  out->batch_size = bsz;
  out->alpha0 = alpha0;
  out->total_steps = total_steps;
  return 0;
}

int orc_train(const float* x, uint64_t n, const OrcTrainCfg* cfg, OrcTrainOut* out) {
  return orc_train_from(x, n, cfg, nullptr, nullptr, nullptr, out);
}

// --- dedup_with_neighbors (crates/emeans-cluster/src/dedup.rs:186-358), with the
// reference's side inputs: created_unix (NaN = unknown) with max_gap_secs
// (has_gap), burst ids (burst[i] < 0 = none) and priority (each may be null).
static float dot_seq(const float* a, const float* b, size_t d) {  // dedup.rs:158-160
  float s = 0.0f;
  for (size_t t = 0; t < d; t++) {
    float p = a[t] * b[t];
    s = s + p;
  }
  return s;
}

namespace {
struct OrcUnionFind {  // dedup.rs:126-156: lower root wins
  std::vector<uint32_t> p;
  explicit OrcUnionFind(size_t n) : p(n) {
    for (size_t i = 0; i < n; i++) p[i] = (uint32_t)i;
  }
  uint32_t find(uint32_t i) {
    while (p[i] != i) {
      uint32_t q = p[i];
      p[i] = p[q];
      i = q;
    }
    return i;
  }
  void unite(uint32_t a, uint32_t b) {
    uint32_t ra = find(a), rb = find(b);
    if (ra != rb) p[std::max(ra, rb)] = std::min(ra, rb);
  }
};
}  // namespace

uint64_t orc_dedup(const float* x, uint64_t n, uint64_t d, const uint32_t* nb_ids,
                   const float* nb_sims, uint64_t kk, float sim_threshold, float rep_threshold,
                   int has_gap, double max_gap_secs, const double* created_unix,
                   const int64_t* burst, const float* priority, uint32_t* group_of,
                   uint32_t* reps, uint32_t* anchors, uint32_t* sizes, uint64_t* linked_pairs,
                   uint64_t* split_components) {
  // time_ok (dedup.rs:213-221)
  auto time_ok = [&](size_t i, size_t j) {
    if (!has_gap || !created_unix) return true;
    const double ti = created_unix[i], tj = created_unix[j];
    if (!std::isfinite(ti) || !std::isfinite(tj)) return true;
    return std::fabs(ti - tj) <= max_gap_secs;
  };
  auto row = [&](size_t i) { return x + i * d; };
  // Burst units (always together), then link components seeded with them (dedup.rs:224-239).
  OrcUnionFind unit(n);
  if (burst) {
    std::map<int64_t, uint32_t> first;
    for (size_t i = 0; i < n; i++) {
      if (burst[i] < 0) continue;
      auto it = first.emplace(burst[i], (uint32_t)i).first;
      unit.unite(it->second, (uint32_t)i);
    }
  }
  OrcUnionFind comp(n);
  for (uint32_t i = 0; i < n; i++) comp.unite(unit.find(i), i);
  std::vector<uint32_t> degree(n, 0);
  std::set<std::pair<uint32_t, uint32_t>> pairs;
  for (size_t i = 0; i < n; i++)  // dedup.rs:240-254
    for (size_t t = 0; t < kk; t++) {
      const uint32_t j = nb_ids[i * kk + t];
      const float s = nb_sims[i * kk + t];
      if (j == 0xffffffffu || s < sim_threshold || !time_ok(i, j)) continue;
      comp.unite((uint32_t)i, j);
      auto key = std::make_pair((uint32_t)std::min<size_t>(i, j), (uint32_t)std::max<size_t>(i, j));
      if (pairs.insert(key).second) {
        degree[i]++;
        degree[j]++;
      }
    }
  // Members of each component in row order; each row's burst unit (dedup.rs:256-261).
  std::map<uint32_t, std::vector<uint32_t>> members;
  for (uint32_t i = 0; i < n; i++) members[comp.find(i)].push_back(i);
  std::vector<uint32_t> unit_of(n);
  for (uint32_t i = 0; i < n; i++) unit_of[i] = unit.find(i);
  // Star cover (dedup.rs:263-309).
  std::vector<std::pair<std::vector<uint32_t>, uint32_t>> groups;
  size_t split = 0;
  for (auto& kv : members) {
    const std::vector<uint32_t>& rows = kv.second;
    if (rows.size() == 1) {
      groups.push_back({rows, rows[0]});
      continue;
    }
    std::map<uint32_t, std::vector<uint32_t>> units;
    for (uint32_t r : rows) units[unit_of[r]].push_back(r);
    std::vector<uint32_t> order = rows;
    std::sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) {
      if (degree[a] != degree[b]) return degree[a] > degree[b];
      return a < b;
    });
    std::set<uint32_t> taken;
    const size_t before = groups.size();
    for (uint32_t c : order) {
      const uint32_t cu = unit_of[c];
      if (taken.count(cu)) continue;
      taken.insert(cu);
      std::vector<uint32_t> g = units[cu];
      std::vector<uint32_t> rest;
      for (auto& u : units)
        if (!taken.count(u.first)) rest.push_back(u.first);
      std::vector<bool> joins;
      for (uint32_t u : rest) {  // every row of a unit must fit the anchor
        bool all = true;
        for (uint32_t r : units[u])
          all = all && time_ok(r, c) && dot_seq(row(r), row(c), d) >= rep_threshold;
        joins.push_back(all);
      }
      for (size_t q = 0; q < rest.size(); q++)
        if (joins[q]) {
          taken.insert(rest[q]);
          g.insert(g.end(), units[rest[q]].begin(), units[rest[q]].end());
        }
      std::sort(g.begin(), g.end());
      groups.push_back({g, c});
    }
    if (groups.size() - before > 1) split++;
  }
  std::stable_sort(groups.begin(), groups.end(),
                   [](const auto& a, const auto& b) { return a.first[0] < b.first[0]; });
  // Representatives: priority, then mean similarity, then lowest id (dedup.rs:315-340).
  for (size_t gi = 0; gi < groups.size(); gi++) {
    const std::vector<uint32_t>& g = groups[gi].first;
    anchors[gi] = groups[gi].second;
    sizes[gi] = (uint32_t)g.size();
    uint32_t rep = g[0];
    if (g.size() > 1) {
      float bp = -INFINITY;
      double bm = -INFINITY;
      uint32_t ba = 0xffffffffu;
      for (uint32_t a : g) {
        double sum = 0.0;
        for (uint32_t b : g)
          if (b != a) sum += (double)dot_seq(row(a), row(b), d);
        const double mean = sum / (double)(g.size() - 1);
        const float p = priority ? priority[a] : 0.0f;
        if (p > bp || (p == bp && mean > bm)) {
          bp = p;
          bm = mean;
          ba = a;
        }
      }
      rep = ba;
    }
    reps[gi] = rep;
    for (uint32_t r : g) group_of[r] = (uint32_t)gi;
  }
  *linked_pairs = pairs.size();
  *split_components = split;
  return groups.size();
}

// --- kmeans_pp (crates/emeans-cluster/src/auto.rs:401-455): k-means++ seeding
// with the cosine distance 1 - x.y; kmax row ids in pick order. The dots are
// dedup.rs's order: rounded products added in sequence (no fma).
uint64_t orc_kmeans_pp(const float* x, uint64_t n, uint64_t d, uint64_t kmax, uint32_t seed,
                       uint32_t* picks) {
  kmax = std::min(kmax, n);
  if (kmax == 0) return 0;
  RandomState rng(seed);
  const size_t first = (size_t)rng.random_interval(n - 1);
  std::vector<uint32_t> pk{(uint32_t)first};
  std::vector<float> best(n, -INFINITY);
  std::vector<double> w(n);
  size_t last = first;
  while (pk.size() < kmax) {
    const float* c = x + last * d;
    for (size_t i = 0; i < n; i++) {
      const float s = dot_seq(x + i * d, c, d);
      if (s > best[i]) best[i] = s;
    }
    double total = 0.0;
    for (size_t i = 0; i < n; i++) {
      const double dist = std::fmax(1.0 - (double)best[i], 0.0);  // f64::max
      w[i] = dist * dist;
      total += w[i];
    }
    size_t next;
    if (total > 0.0) {
      double u = rng.random_sample() * total;
      size_t j = n - 1;
      for (size_t i = 0; i < n; i++) {
        if (u < w[i]) {
          j = i;
          break;
        }
        u -= w[i];
      }
      if (w[j] == 0.0) {  // the farthest row; the last of equal maxima (Iterator::max_by)
        size_t m = 0;
        for (size_t i = 1; i < n; i++)
          if (!(w[i] < w[m])) m = i;
        j = m;
      }
      next = j;
    } else {
      next = 0;
      for (size_t i = 0; i < n; i++)
        if (std::find(pk.begin(), pk.end(), (uint32_t)i) == pk.end()) {
          next = i;
          break;
        }
    }
    pk.push_back((uint32_t)next);
    last = next;
  }
  std::memcpy(picks, pk.data(), pk.size() * 4);
  return pk.size();
}

// --- gemm_nt (crates/emeans-core/src/assign.rs:813-825) as Hierarchy::grow
// calls it (crates/emeans-cluster/src/incremental.rs:423-440): out[i * nb + j]
// = a_i . b_j. The reference takes these from the `gemm` crate; here each is
// one fma chain over t in order from +0, the order of the top-1 dots.
void orc_dots(const float* a, uint64_t m, const float* b, uint64_t nb, uint64_t d, float* out) {
  for (size_t i = 0; i < m; i++)
    for (size_t j = 0; j < nb; j++) {
      float acc = 0.0f;
      for (size_t t = 0; t < d; t++) acc = std::fma(a[i * d + t], b[j * d + t], acc);
      out[i * nb + j] = acc;
    }
}

// --- internal_scores (crates/emeans-cluster/src/metrics.rs:113-268): cosine
// silhouette, Calinski-Harabasz, Davies-Bouldin and the spherical objective of
// `labels` (< k) on unit rows. The row-by-cluster-sum dots come from the
// `gemm` crate in the reference; here they are one fma chain each over t in
// order. Everything else keeps the reference's f64 order, with its parallel
// sums taken in index order. out: silhouette, CH, DB, objective; sizes k.
int orc_internal_scores(const float* x, uint64_t n, uint64_t d, const uint32_t* labels,
                        uint64_t k, double* out, uint64_t* sizes_out, uint64_t* k_eff_out) {
  for (size_t i = 0; i < n; i++)
    if (labels[i] >= k) return 1;
  std::vector<uint64_t> sizes(k, 0);
  std::vector<double> sums(k * d, 0.0);
  for (size_t i = 0; i < n; i++) {
    sizes[labels[i]]++;
    double* s = &sums[labels[i] * d];
    for (size_t t = 0; t < d; t++) s[t] += (double)x[i * d + t];
  }
  std::vector<size_t> live;
  for (size_t j = 0; j < k; j++)
    if (sizes[j] > 0) live.push_back(j);
  const size_t ke = live.size();
  std::vector<float> sums32(ke * d);
  std::vector<double> sq(ke, 0.0);
  std::vector<size_t> slot(k, SIZE_MAX);
  for (size_t s = 0; s < ke; s++) {
    slot[live[s]] = s;
    for (size_t t = 0; t < d; t++) {
      const double v = sums[live[s] * d + t];
      sums32[s * d + t] = (float)v;
      sq[s] += v * v;
    }
  }
  std::vector<double> xx(n);
  for (size_t i = 0; i < n; i++) {
    double a = 0.0;
    for (size_t t = 0; t < d; t++) a += (double)x[i * d + t] * (double)x[i * d + t];
    xx[i] = a;
  }
  double sil_sum = 0.0, obj_sum = 0.0;
  std::vector<double> scatter(ke, 0.0);
  std::vector<float> g(ke);
  for (size_t i = 0; i < n; i++) {
    for (size_t s = 0; s < ke; s++) {
      float acc = 0.0f;
      for (size_t t = 0; t < d; t++) acc = std::fma(x[i * d + t], sums32[s * d + t], acc);
      g[s] = acc;
    }
    const size_t own = slot[labels[i]];
    const double na = (double)sizes[live[own]];
    const double dot_own = (double)g[own];
    const double dist = std::sqrt(std::fmax(xx[i] - 2.0 * dot_own / na + sq[own] / (na * na), 0.0));
    const double cos_c = dot_own / std::fmax(std::sqrt(sq[own]), 1e-30);
    const double obj = 2.0 - 2.0 * cos_c;
    double sil = 0.0;
    if (!(ke < 2 || na < 2.0)) {
      const double a = 1.0 - (dot_own - xx[i]) / (na - 1.0);
      double b = INFINITY;
      for (size_t s = 0; s < ke; s++)
        if (s != own) b = std::fmin(b, 1.0 - (double)g[s] / (double)sizes[live[s]]);
      const double m = std::fmax(a, b);
      sil = m > 0.0 ? (b - a) / m : 0.0;
    }
    sil_sum += sil;
    obj_sum += obj;
    scatter[own] += dist;
  }
  const double nf = (double)std::max<uint64_t>(n, 1);
  double total_xx = 0.0;
  for (size_t i = 0; i < n; i++) total_xx += xx[i];
  double wsum = 0.0;
  for (size_t s = 0; s < ke; s++) wsum += sq[s] / (double)sizes[live[s]];
  const double within = total_xx - wsum;
  std::vector<double> grand(d, 0.0);
  for (size_t s = 0; s < ke; s++)
    for (size_t t = 0; t < d; t++) grand[t] += sums[live[s] * d + t];
  double gsq = 0.0;
  for (size_t t = 0; t < d; t++) gsq += grand[t] * grand[t];
  const double total = total_xx - gsq / nf;
  const double between = total - within;
  const double ch = (ke < 2 || n <= ke || within <= 0.0)
                        ? 0.0
                        : (between / (double)(ke - 1)) / (within / (double)(n - ke));
  double db = 0.0;
  if (ke >= 2) {
    double acc = 0.0;
    for (size_t a = 0; a < ke; a++) {
      double worst = 0.0;
      for (size_t b = 0; b < ke; b++) {
        if (b == a) continue;
        double m2 = 0.0;
        for (size_t t = 0; t < d; t++) {
          const double p = sums[live[a] * d + t] / (double)sizes[live[a]];
          const double q = sums[live[b] * d + t] / (double)sizes[live[b]];
          m2 += (p - q) * (p - q);
        }
        const double m = std::sqrt(m2);
        const double sa = scatter[a] / (double)sizes[live[a]], sb = scatter[b] / (double)sizes[live[b]];
        const double r = m > 0.0 ? (sa + sb) / m : INFINITY;
        worst = std::fmax(worst, r);
      }
      acc += worst;
    }
    db = acc / (double)ke;
  }
  out[0] = sil_sum / nf;
  out[1] = ch;
  out[2] = db;
  out[3] = obj_sum / nf;
  for (size_t j = 0; j < k; j++) sizes_out[j] = sizes[j];
  *k_eff_out = ke;
  return 0;
}

// --- Test-data generators of the reference's own tests.
// core/contract.rs:40-60 (`mixture`): Box-Muller over MT19937 random_sample, f64.
void orc_contract_mixture(uint64_t n, uint64_t d, uint64_t centers, double sigma, int unit,
                          uint32_t seed, float* out) {
  RandomState rng(seed);
  auto gauss = [&]() {
    double u1 = std::max(rng.random_sample(), 1e-300);
    double u2 = rng.random_sample();
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2);
  };
  std::vector<double> cs(centers * d);
  for (auto& v : cs) v = gauss();
  std::vector<double> row(d);
  for (size_t i = 0; i < n; i++) {
    const double* c = &cs[(i % centers) * d];
    for (size_t t = 0; t < d; t++) row[t] = c[t] + sigma * gauss();
    double s = 1.0;
    if (unit) {
      double q = 0.0;
      for (size_t t = 0; t < d; t++) q += row[t] * row[t];
      s = std::max(std::sqrt(q), 1e-12);
    }
    for (size_t t = 0; t < d; t++) out[i * d + t] = (float)(row[t] / s);
  }
}

// tests/common/mod.rs:7-35 (`mixture` of the model/kernel tests): f32 data.
void orc_common_mixture(uint64_t n, uint64_t d, uint64_t centers, float spread, int spherical,
                        uint32_t seed, float* out) {
  RandomState rng(seed);
  auto normal = [&]() {
    double u1 = std::max(rng.random_sample(), 1e-300);
    double u2 = rng.random_sample();
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2));
  };
  std::vector<float> c(centers * d);
  for (auto& v : c) v = 3.0f * normal();
  for (size_t i = 0; i < n; i++) {
    size_t j = i % centers;
    for (size_t t = 0; t < d; t++) {
      float nz = spread * normal();
      out[i * d + t] = c[j * d + t] + nz;
    }
    if (spherical) {
      float norm = std::sqrt(sq_norm(out + i * d, d));
      for (size_t t = 0; t < d; t++) out[i * d + t] = out[i * d + t] / norm;
    }
  }
}

}  // extern "C"
