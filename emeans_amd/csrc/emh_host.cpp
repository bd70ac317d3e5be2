// Host side of the device loop and its callers, on the gfx950 context:
//  - the seeded draws the reference keeps on the host: numpy-legacy MT19937
//    (crates/emeans-core/src/rng.rs), the recipe and cosine schedule
//    (recipe.rs), the revival plan (core/mod.rs:339-370) and closing means
//    (core/mod.rs:404-429);
//  - layer 2, core::train::run (core/train.rs:60-303) and Emeans::train
//    (model.rs:700-811): every batch op queued on the context's stream, the
//    host waiting only for the revival check (every 5 steps), the epoch's
//    labels and scores, and the end; the next epoch's permutation and the
//    epoch statistics run on helper threads;
//  - assign_all / assign_on (assign.rs:785-809, core/mod.rs:249-330),
//    knn_self / knn (emeans-cluster/src/knn.rs:17-64) and dedup
//    (emeans-cluster/src/dedup.rs:163-358) with its time and burst rules.

#include <algorithm>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <functional>
#include <initializer_list>
#include <future>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <unordered_map>
#include <string>
#include <thread>
#include <vector>

#include "emh_internal.h"

namespace emh {
namespace host {

// ------------------------------------------------------------------ MT19937
// RandomState(seed).permutation(n) into p (emh_perm.cpp).
void mt_permutation(uint32_t seed, size_t n, uint32_t* p);

class RandomState {  // rng.rs:13-102
 public:
  explicit RandomState(uint32_t seed) {
    uint32_t s = seed;
    for (int i = 0; i < N; i++) {
      mt_[i] = s;
      s = 1812433253u * (s ^ (s >> 30)) + (uint32_t)(i + 1);
    }
    pos_ = N;
  }
  uint32_t next_u32() {
    if (pos_ == N) refill();
    return out_[pos_++];
  }
  double random_sample() {
    uint32_t a = next_u32() >> 5, b = next_u32() >> 6;
    return ((double)a * 67108864.0 + (double)b) / 9007199254740992.0;
  }
  // numpy legacy random_interval: masked rejection in [0, max]. For max below
  // 2^32 two candidate words are tested at once, so the loop branches only
  // when both are rejected; the words consumed are the same as one at a time.
  uint64_t interval(uint64_t max) {
    if (max == 0) return 0;
    if (max <= 0xffffffffull) {
      const uint32_t mx = (uint32_t)max, m = 0xffffffffu >> __builtin_clz(mx);
      for (;;) {
        if (pos_ >= N - 1) {
          const uint32_t v = next_u32() & m;
          if (v <= mx) return v;
          continue;
        }
        const uint32_t v1 = out_[pos_] & m, v2 = out_[pos_ + 1] & m;
        const bool a1 = v1 <= mx, a2 = v2 <= mx;
        if (a1 | a2) {
          pos_ += a1 ? 1 : 2;
          return a1 ? v1 : v2;
        }
        pos_ += 2;
      }
    }
    uint64_t mask = max;
    mask |= mask >> 1;
    mask |= mask >> 2;
    mask |= mask >> 4;
    mask |= mask >> 8;
    mask |= mask >> 16;
    mask |= mask >> 32;
    for (;;) {
      const uint64_t hi = next_u32();
      const uint64_t v = ((hi << 32) | next_u32()) & mask;
      if (v <= max) return v;
    }
  }
  // numpy's legacy shuffle: for i = n-1 down to 1, swap p[i] with p[interval(i)].
  static std::vector<uint32_t> permutation(uint32_t seed, size_t n) {
    std::vector<uint32_t> p(n);
    mt_permutation(seed, n, p.data());
    return p;
  }
  // The same draws as interval() from a fresh state (emh_perm.cpp).
  static void permutation_into(uint32_t seed, size_t n, uint32_t* p) { mt_permutation(seed, n, p); }

 private:
  static constexpr int N = 624, M = 397;
  static uint32_t twist(uint32_t a, uint32_t b, uint32_t c) {  // MT19937 recurrence
    const uint32_t y = (a & 0x80000000u) | (b & 0x7fffffffu);
    return c ^ (y >> 1) ^ ((0u - (y & 1u)) & 0x9908b0dfu);
  }
  static uint32_t temper(uint32_t y) {
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    return y ^ (y >> 18);
  }
  // The next N words of the state, tempered into out_.
  void refill() {
    int i = 0;
    for (; i < N - M; i++) mt_[i] = twist(mt_[i], mt_[i + 1], mt_[i + M]);
    for (; i < N - 1; i++) mt_[i] = twist(mt_[i], mt_[i + 1], mt_[i + M - N]);
    mt_[N - 1] = twist(mt_[N - 1], mt_[0], mt_[M - 1]);
    for (int j = 0; j < N; j++) out_[j] = temper(mt_[j]);
    pos_ = 0;
  }
  uint32_t mt_[N];
  uint32_t out_[N];
  int pos_;
};

// ------------------------------------------------------------------- recipe
struct Recipe {
  size_t batch_size = 0;
  double alpha0 = 0;
  std::vector<size_t> epoch_rows;
  size_t total_steps = 0;
  double tau = 0;
  size_t chunk = 65536;
};

size_t pow2_round(double v) {  // recipe.rs:69-80
  if (v <= 1.0) return 1;
  double lo = std::ldexp(1.0, (int)std::floor(std::log2(v)));
  return (size_t)(v / lo < (2.0 * lo) / v ? lo : 2.0 * lo);
}

Recipe resolve(size_t n, size_t k, size_t d, const emh_config& cfg) {  // recipe.rs:200-254
  Recipe r;
  int law = cfg.batch_law;
  if (law == 0) law = d <= 16 ? 2 : 1;  // auto: quality at d <= 16
  const double T = cfg.nepochs;
  size_t b;
  if (cfg.batch_size > 0) {
    b = std::min((size_t)cfg.batch_size, n);
  } else {
    const double cb = law == 1 ? 0.035134 : 0.00439175;
    const double raw = cb * std::pow((double)k, 0.134749) * std::pow((double)n, 0.876473) *
                       std::pow(T, 0.813344);
    b = pow2_round(raw);
    b = law == 1 ? std::min(b, pow2_round((double)n / 2.0)) : std::min(b, n / 2);
    b = std::max<size_t>(std::min(b, n), 1);
  }
  r.batch_size = b;
  if (cfg.has_alpha0) {
    r.alpha0 = cfg.alpha0;
  } else {
    double a = 0.8244 * std::pow((double)k, -0.4617) * std::pow((double)b, 0.9003) *
               std::pow((double)n, -0.4498) * std::pow(T, -0.1057);
    r.alpha0 = std::min(std::max(a, 1e-4), 1.0);
  }
  // epoch_rows (recipe.rs:127-140)
  const double whole = std::floor(T);
  const size_t rem = (size_t)std::nearbyint((T - whole) * (double)n);
  const size_t w = (size_t)whole;
  if (w == 0) {
    r.epoch_rows = {rem};
  } else {
    r.epoch_rows.assign(w - 1, n);
    if (rem > 0) r.epoch_rows.push_back(rem);
    r.epoch_rows.push_back(n);
  }
  for (size_t e : r.epoch_rows) r.total_steps += (e + b - 1) / b;
  r.tau = cfg.has_unused_threshold ? cfg.unused_threshold : (d <= 2 ? 0.0 : 0.1);
  r.chunk = cfg.assignment_chunk_size ? (size_t)cfg.assignment_chunk_size : 65536;
  return r;
}

uint32_t epoch_seed(uint32_t seed, size_t e) {  // recipe.rs:143-145
  return (uint32_t)(((uint64_t)seed * 1000003ull + e) & 0xffffffffull);
}

double scheduled_alpha(double a0, size_t step, size_t total) {  // recipe.rs:148-152
  const double f = (double)std::min(step, total) / (double)std::max<size_t>(total, 1);
  const double cosine = 0.5 * (1.0 + std::cos(M_PI * f));
  return a0 * (0.1 + 0.9 * cosine);
}

// numpy float32 pairwise sum (model.rs:970-1002).
float np_sum(const float* a, size_t n) {
  if (n < 8) {
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s = s + a[i];
    return s;
  }
  if (n <= 128) {
    float r[8];
    for (int j = 0; j < 8; j++) r[j] = a[j];
    size_t i = 8;
    const size_t stop = n - n % 8;
    for (; i < stop; i += 8)
      for (int j = 0; j < 8; j++) r[j] = r[j] + a[i + j];
    float s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; i++) s = s + a[i];
    return s;
  }
  size_t h = n / 2;
  h -= h % 8;
  return np_sum(a, h) + np_sum(a + h, n - h);
}

// The Gumbel terms ln(-ln u) of the next k uniforms of a revival stream
// (u = random_sample() floored at the smallest normal f64, core/mod.rs:355-357).
std::vector<double> gumbel_terms(RandomState& rng, size_t k) {
  std::vector<double> g(k);
  for (size_t j = 0; j < k; j++)
    g[j] = std::log(-std::log(std::max(rng.random_sample(), 2.2250738585072014e-308)));
  return g;
}

// Revival plan (core/mod.rs:339-370): clusters under tau * mean mass take a
// donor drawn by Gumbel top-k on ln N. The k uniforms are drawn only if a split
// happens: `draw` returns their Gumbel terms (gumbel_terms of the stream).
template <class Draw>
std::vector<uint32_t> plan_revival(const std::vector<float>& usage, double tau, Draw&& draw) {
  const size_t k = usage.size();
  const float thr = (np_sum(usage.data(), k) * (float)tau) / (float)k;
  std::vector<uint32_t> dead;
  std::vector<char> donor(k);
  size_t ndonor = 0;
  for (size_t j = 0; j < k; j++) {
    const bool u = usage[j] < thr;
    if (u) dead.push_back((uint32_t)j);
    donor[j] = !u && usage[j] > 0.0f;
    ndonor += donor[j];
  }
  const size_t nsplit = std::min(dead.size(), ndonor);
  std::vector<uint32_t> pairs;
  if (nsplit == 0) return pairs;
  const std::vector<double> g = draw();
  struct Key {
    int64_t ord;
    uint32_t j;
  };
  std::vector<Key> keys;
  keys.reserve(ndonor);
  for (size_t j = 0; j < k; j++) {
    if (!donor[j]) continue;
    double v = (double)std::log(usage[j]) - g[j];  // f32 ln, then f64
    int64_t b;
    std::memcpy(&b, &v, 8);
    b ^= (int64_t)(((uint64_t)(b >> 63)) >> 1);  // IEEE total order as an integer
    keys.push_back({b, (uint32_t)j});
  }
  // Larger key first, equal keys: higher index first. The order is total, so
  // the nsplit first of a selection, sorted, are those of a full sort.
  const auto before = [](const Key& a, const Key& b) {
    return a.ord != b.ord ? a.ord > b.ord : a.j > b.j;
  };
  if (nsplit < keys.size()) std::nth_element(keys.begin(), keys.begin() + nsplit, keys.end(), before);
  std::sort(keys.begin(), keys.begin() + nsplit, before);
  for (size_t q = 0; q < nsplit; q++) {
    pairs.push_back(keys[q].j);
    pairs.push_back(dead[q]);
  }
  return pairs;
}

void normalize_row(float* r, size_t d) {  // model.rs:954-967
  float mx = 0.0f;
  for (size_t t = 0; t < d; t++) mx = std::fmax(mx, std::fabs(r[t]));
  const float s = mx > 0.0f ? mx : 1.0f;
  for (size_t t = 0; t < d; t++) r[t] = r[t] / s;
  float q = 0.0f;
  for (size_t t = 0; t < d; t++) {
    float p = r[t] * r[t];
    q = q + p;
  }
  const float nr = std::sqrt(q);
  const float s2 = nr > 0.0f ? nr : 1.0f;
  for (size_t t = 0; t < d; t++) r[t] = r[t] / s2;
}

// ------------------------------------------------------------ device buffers
// A call's device buffer: its own allocation, or a piece of an Arena laid
// over one of the context's kept blocks (arena_for), which it does not free.
struct Buf {
  void* p = nullptr;
  bool own = false;
  Buf() = default;
  Buf(emh_ctx*, size_t bytes) : own(true) {
    if (bytes) EMH_HIP(hipMalloc(&p, bytes));
  }
  Buf(Arena& a, size_t bytes) {
    if (bytes) p = a.take(bytes);
  }
  ~Buf() {
    if (own && p) (void)hipFree(p);
  }
  Buf(const Buf&) = delete;
  Buf& operator=(const Buf&) = delete;
  float* f() const { return (float*)p; }
  uint32_t* u() const { return (uint32_t*)p; }
};

// An Arena over the context's kept block s, large enough for Bufs of the
// given byte sizes taken in that order. The block only grows, so after the
// first call of a size the call allocates and frees nothing; the work that
// used the block last is on the same context's streams, which every user
// drains before it returns.
Arena arena_for(Scratch& s, std::initializer_list<size_t> sizes) {
  size_t total = 0;
  for (size_t b : sizes) total += (b + 255) & ~size_t(255);
  Arena a;
  a.base = (char*)s.get(std::max<size_t>(total, 256));
  a.cap = total;
  return a;
}

void h2d(emh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!bytes) return;
  EMH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  EMH_HIP(hipStreamSynchronize(c->stream));
}
void d2h(emh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (bytes) EMH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  EMH_HIP(hipStreamSynchronize(c->stream));
}
void check_flags(emh_ctx* c) {
  uint32_t w[SW_WORDS];
  d2h(c, w, c->small, sizeof w);
  if (w[SW_BAD_LABEL] || w[SW_BAD_ID]) {
    launch_fill_u32(c, c->small + SW_BAD_LABEL, 1, 0);
    launch_fill_u32(c, c->small + SW_BAD_ID, 1, 0);
    EMH_HIP(hipStreamSynchronize(c->stream));
    throw Failure(w[SW_BAD_LABEL] ? "label out of range" : "row id out of range");
  }
}

// A HIP event without timing.
// Waits until the device posts seq into *word (pinned host memory, written at
// system scope by a kernel on c's stream): a spin, with a stream
// synchronization after 50 ms so that a failed launch surfaces as an error.
void wait_posted(emh_ctx* c, const uint32_t* word, uint32_t seq) {
  const auto t0 = std::chrono::steady_clock::now();
  for (uint32_t i = 1;; i++) {
    if (__atomic_load_n(word, __ATOMIC_ACQUIRE) == seq) return;
    if ((i & 1023) == 0 &&
        std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(50)) {
      EMH_HIP(hipStreamSynchronize(c->stream));
      EMH_ENSURE(__atomic_load_n(word, __ATOMIC_ACQUIRE) == seq, "revival check word not posted");
      return;
    }
    __builtin_ia32_pause();
  }
}

struct Event {
  hipEvent_t e = nullptr;
  Event() { EMH_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming)); }
  ~Event() {
    if (e) (void)hipEventDestroy(e);
  }
  Event(const Event&) = delete;
  Event& operator=(const Event&) = delete;
  void record(hipStream_t s) { EMH_HIP(hipEventRecord(e, s)); }
  void wait() { EMH_HIP(hipEventSynchronize(e)); }  // returns at once if never recorded
};

// Errors the kernels flagged in the small block (a copy of it in w).
void raise_flags(emh_ctx* c, const uint32_t* w) {
  if (!(w[SW_BAD_LABEL] || w[SW_BAD_ID] || w[SW_BAD_INIT])) return;
  for (int s : {SW_BAD_LABEL, SW_BAD_ID, SW_BAD_INIT}) launch_fill_u32(c, c->small + s, 1, 0);
  EMH_HIP(hipStreamSynchronize(c->stream));
  if (w[SW_BAD_INIT]) throw Invalid("initial centroids must be finite");
  throw Failure(w[SW_BAD_LABEL] ? "label out of range" : "row id out of range");
}

// Threads for the host work beside the device loop (the next epoch's order,
// Gumbel terms, epoch statistics, the final copies). They live as long as the
// process: starting a thread per task would put its start-up on the loop's
// path. Tasks only wait on HIP events of work already queued, never on each
// other, so four threads cannot all block on what a queued task would do.
class Helpers {
 public:
  static Helpers& get() {
    static Helpers* h = new Helpers(4);  // never destroyed: idle threads end with the process
    return *h;
  }
  template <class F>
  auto run(F&& f) -> std::future<decltype(f())> {
    using R = decltype(f());
    auto task = std::make_shared<std::packaged_task<R()>>(std::forward<F>(f));
    std::future<R> fut = task->get_future();
    {
      std::lock_guard<std::mutex> g(m_);
      q_.emplace_back([task] { (*task)(); });
    }
    cv_.notify_one();
    return fut;
  }

 private:
  explicit Helpers(int n) {
    for (int i = 0; i < n; i++) std::thread([this] { loop(); }).detach();
  }
  void loop() {
    for (;;) {
      std::function<void()> f;
      {
        std::unique_lock<std::mutex> l(m_);
        cv_.wait(l, [&] { return !q_.empty(); });
        f = std::move(q_.front());
        q_.pop_front();
      }
      f();
    }
  }
  std::mutex m_;
  std::condition_variable cv_;
  std::deque<std::function<void()>> q_;
};

template <class F>
auto beside(F&& f) {
  return Helpers::get().run(std::forward<F>(f));
}

// Pageable host memory to the device at DMA speed: pieces of STAGE bytes go
// through the context's two pinned staging halves, copied in by this thread
// and three helpers while the copy stream moves the other half to the device.
// The copy stream first waits for `after` (when given); work queued on the
// context stream after the call sees the data. Returns once every piece is in
// staging; the last DMAs may still run.
constexpr size_t STAGE = size_t(32) << 20;
void upload(emh_ctx* c, void* dst, const void* src, size_t bytes, hipEvent_t after = nullptr) {
  if (!bytes) return;
  hipStream_t cs = c->copies();
  if (after) EMH_HIP(hipStreamWaitEvent(cs, after, 0));
  char* half[2] = {(char*)c->pin_stage[0].get(STAGE), (char*)c->pin_stage[1].get(STAGE)};
  const char* s = (const char*)src;
  for (size_t off = 0, pc = 0; off < bytes; off += STAGE, pc++) {
    const int h = (int)(pc & 1);
    const size_t len = std::min(STAGE, bytes - off);
    EMH_HIP(hipEventSynchronize(c->ev_stage[h]));  // the last copy out of this half is done
    constexpr int T = 4;
    const size_t part = (len / T + 63) & ~size_t(63);
    std::future<void> f[T - 1];
    for (int t = 1; t < T; t++) {
      const size_t a = std::min(len, t * part), b = std::min(len, a + part);
      f[t - 1] = beside([=] { std::memcpy(half[h] + a, s + off + a, b - a); });
    }
    std::memcpy(half[h], s + off, std::min(len, part));
    for (auto& x : f) x.get();
    EMH_HIP(hipMemcpyAsync((char*)dst + off, half[h], len, hipMemcpyHostToDevice,
                           cs));
    EMH_HIP(hipEventRecord(c->ev_stage[h], cs));
  }
  EMH_HIP(hipEventRecord(c->ev_stage[2], cs));
  EMH_HIP(hipStreamWaitEvent(c->stream, c->ev_stage[2], 0));
}

void copy_async(emh_ctx* c, void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
  if (bytes) EMH_HIP(hipMemcpyAsync(dst, src, bytes, kind, c->stream));
}

// The start's arguments (model.rs:306-336): one kind of start, the right
// shapes, masses finite and >= 0.
void check_init(const emh_config* cfg, const emh_train_init* init) {
  if (!init) return;
  const int kinds = (init->centroids != nullptr) + (init->centroids_dev != nullptr) +
                    (init->positions != nullptr);
  EMH_ENSURE(kinds <= 1, "give initial centroids or EMA state, not both");
  EMH_ENSURE(!init->usage || init->positions, "usage comes with positions");
  if (init->centroids_dev)
    EMH_ENSURE(init->centroids_dev->kind == 0 && init->centroids_dev->len == cfg->k * cfg->d,
               "init centroids must be k x d");
  if (init->positions) {
    EMH_ENSURE(init->usage, "positions need their usage (k masses)");
    for (size_t j = 0; j < cfg->k; j++)
      EMH_ENSURE(std::isfinite(init->usage[j]) && init->usage[j] >= 0.0f,
                 "usage must be finite and >= 0");
  }
}

void check_cfg(size_t n, const emh_config* cfg, const emh_train_out* out) {
  EMH_ENSURE(cfg && out && out->centroids, "null argument");
  EMH_ENSURE(!out->centroids_dev ||
                 (out->centroids_dev->kind == 0 && out->centroids_dev->len == cfg->k * cfg->d),
             "centroids_dev must be a k x d f32 buffer");
  EMH_ENSURE(cfg->d > 0 && cfg->k > 0, "d and k must be positive");
  EMH_ENSURE(std::isfinite(cfg->nepochs) && cfg->nepochs > 0.0, "nepochs must be positive");
  EMH_ENSURE(!cfg->has_unused_threshold || cfg->unused_threshold >= 0.0,
             "unused_threshold must be >= 0 (0 disables revival)");
  EMH_ENSURE(cfg->batch_law >= 0 && cfg->batch_law <= 2, "unknown batch law");
  EMH_ENSURE(n >= cfg->k, "need at least k = %llu rows, got %zu", (unsigned long long)cfg->k, n);
  const Recipe r = resolve(n, cfg->k, cfg->d, *cfg);
  for (size_t e : r.epoch_rows) EMH_ENSURE(e > 0, "nepochs gives an empty epoch for n = %zu", n);
}

// Emeans::train_rows (model.rs:772-811) with the data on the device, driving
// core::train::run (core/train.rs:60-303), then the closing means
// (core/mod.rs:404-429).
//
// The host never idles the device for a whole step: host<->device traffic
// goes through pinned buffers and events. At a revival check (every 5th step)
// the masses the step's EMA will leave depend only on the step's counts, so
// they are computed and copied out right after the count kernel; the host
// plans the revival while the device still runs the step's sums and EMA. The
// epoch's labels and scores are copied out asynchronously and the statistics
// wait for them on a helper thread; the next epoch's order is drawn on
// another and copied in from a pinned buffer.
void train_dev(emh_ctx* c, const float* x, size_t n, const emh_config& cfg,
               const emh_train_init* init, emh_train_out* out) {
  const auto t_start = std::chrono::steady_clock::now();
  const size_t k = cfg.k, d = cfg.d;
  const bool sph = cfg.spherical != 0;
  const Recipe R = resolve(n, k, d, cfg);
  const size_t bsz = R.batch_size, chunk = std::max<size_t>(R.chunk, 1);
  const size_t n_epochs = R.epoch_rows.size();
  const bool capture = cfg.capture_assignments && out->labels;

  float* h_usage = (float*)c->pin_usage.get(k * 4);
  uint32_t* h_plan = (uint32_t*)c->pin_plan.get(2 * k * 4);
  uint32_t* h_small = (uint32_t*)c->pin_small.get(3 * SW_WORDS * 4);
  uint32_t* h_small0 = h_small + SW_WORDS;
  // The revival check's completion word, posted by the mass preview kernel.
  uint32_t* h_seq = h_small + 2 * SW_WORDS;
  __atomic_store_n(h_seq, 0u, __ATOMIC_RELAXED);
  uint32_t seq_no = 0;
  uint32_t* h_order[2];
  uint32_t* h_lab[2];
  float* h_sco[2];
  for (int i = 0; i < 2; i++) {
    h_order[i] = (uint32_t*)c->pin_order[i].get(n * 4);
    h_lab[i] = (uint32_t*)c->pin_lab[i].get(n * 4);
    h_sco[i] = (float*)c->pin_sco[i].get(n * 4);
  }
  // The split kernel reads the plan where the host writes it (pinned memory
  // mapped into the device's address space): no copy between planning and
  // the split. The next plan is written only after the next revival check's
  // preview has posted its word, and that kernel runs after this split.
  uint32_t* d_plan = nullptr;
  EMH_HIP(hipHostGetDevicePointer((void**)&d_plan, h_plan, 0));
  // Likewise the revival check's masses and small-block words are written by
  // the mass preview kernel straight into h_usage and h_small.
  float* d_usage_h = nullptr;
  uint32_t* d_small_h = nullptr;
  EMH_HIP(hipHostGetDevicePointer((void**)&d_usage_h, h_usage, 0));
  EMH_HIP(hipHostGetDevicePointer((void**)&d_small_h, h_small, 0));
  float* h_out = (float*)c->pin_out.get((2 * k * d + k) * 4);
  // ev_order[b]: epoch order b is on the device and h_order[b] free again (copy
  // stream); ev_done[b]: the epoch that used order/labels/scores b has run
  // (main stream); ev_epoch[b]: its scores and label counts are on the host.
  Event ev_init, ev_order[2], ev_done[2], ev_epoch[2], ev_last, ev_posout;
  // The copies' stream: the copy stream, beside the kernels; for a small run
  // the context stream itself, where the copies are a few KB and a wait
  // across streams (a barrier packet between hardware queues) would cost more
  // than the overlap saves. cross_wait orders stream s after event e, which
  // was recorded on the other stream; with one stream, order is implicit.
  hipStream_t cps = n <= ONE_STREAM_ROWS ? c->stream : c->copies();
  auto cross_wait = [&](hipStream_t s, hipEvent_t e) {
    if (cps != c->stream) EMH_HIP(hipStreamWaitEvent(s, e, 0));
  };

  // Epochs alternate between two sets of order/labels/scores buffers, so the
  // copies of one epoch's run on the copy stream beside the next epoch's kernels.
  const size_t rb = n * 4, kb = k * 4, cb = k * d * 4, ob = (sph ? k * d : k) * 4;
  Arena ar = arena_for(c->trun, {rb, rb, rb, rb, rb, rb, cb, kb, ob, cb, kb, cb, kb, kb, kb});
  Buf order0(ar, rb), order1(ar, rb), lab0(ar, rb), lab1(ar, rb), sco0(ar, rb), sco1(ar, rb),
      pos(ar, cb), mass(ar, kb), readout(ar, ob), sums(ar, cb), counts(ar, kb), pass(ar, cb),
      tally0(ar, kb), tally1(ar, kb), init_ids(ar, kb);
  uint32_t* d_order[2] = {order0.u(), order1.u()};
  struct Drain {  // nothing queued may outlive the buffers, also on an error
    emh_ctx* c;
    ~Drain() {
      if (c->copy_stream) (void)hipStreamSynchronize(c->copy_stream);
      (void)hipStreamSynchronize(c->stream);
    }
  } drain{c};
  // Epoch e's order: drawn into h_order[e % 2] once the last copy out of it is
  // done, then copied (copy stream) into d_order[e % 2] once the epoch that
  // last used that buffer has run. Runs on a helper thread.
  auto fill_order = [&](size_t epoch) {
    const int buf = (int)(epoch & 1);
    ev_order[buf].wait();
    RandomState::permutation_into(epoch_seed(cfg.seed, epoch), n, h_order[buf]);
    cross_wait(cps, ev_done[buf].e);
    EMH_HIP(hipMemcpyAsync(d_order[buf], h_order[buf], R.epoch_rows[epoch] * 4,
                           hipMemcpyHostToDevice, cps));
    ev_order[buf].record(cps);
  };
  // The revival stream (RandomState(seed)) serves only revivals, k uniforms
  // per revival that splits: the next k Gumbel terms are drawn ahead.
  RandomState split_rng(cfg.seed);
  // Helper tasks (the next epoch's order, Gumbel terms, epoch statistics)
  // reference this frame, and their futures do not wait when destroyed: on
  // any exit, an error included, Join waits for those still running before
  // anything they use goes.
  std::future<void> next;
  std::future<std::vector<double>> gnext;
  std::future<emh_epoch_stats> pending;
  std::future<void> init_perm;
  struct Join {
    std::future<void>& a;
    std::future<std::vector<double>>& b;
    std::future<emh_epoch_stats>& p;
    std::future<void>& q;
    ~Join() {
      if (a.valid()) a.wait();
      if (b.valid()) b.wait();
      if (p.valid()) p.wait();
      if (q.valid()) q.wait();
    }
  } join{next, gnext, pending, init_perm};
  // The first epoch's order and the initial centroids' rows (permutation(n)
  // [..k], model.rs:783-790) are drawn on helpers from the start, while this
  // thread queues the split of the rows.
  const bool resume = init && init->positions;
  const bool draw_init = !resume && !(init && (init->centroids || init->centroids_dev)) && n != k;
  next = beside([&] { fill_order(0); });
  if (draw_init)  // into h_order[1], unused until epoch 1
    init_perm = beside([&] { RandomState::permutation_into(cfg.seed, n, h_order[1]); });
  // When the batches take the split-operand screen, every row's halves once
  // (slab-major, with |x|^2; fp16 for the two-pass screen of SCREEN_F16,
  // else bf16): each batch then gathers its rows' halves by id instead of
  // splitting them again.
  SplitRows pre_rows{};
  const SplitRows* pre = nullptr;
  c->xpre_of = emh_ctx::SplitOf{};  // xpre is rewritten (or left stale) below
  bool run_f16 = false;
  if (split_screen(c, bsz, d, k, sph) && n < (1u << 25)) {
    run_f16 = c->screen == SCREEN_F16;
    pre_rows = SplitRows{c->xpre.get(halves_bytes(n, d)), (float*)c->xpre_norm.get(n * 4), n,
                         n * 128, run_f16};
    launch_halves(c, x, n, d, nullptr, 0, n, (void*)pre_rows.xs, (float*)pre_rows.xn, nullptr,
                  nullptr, run_f16);
    pre = &pre_rows;
    c->xpre_of.ptr = x;  // which buffer: emh_train_dev names it once the run has ended
    c->xpre_of.n = n;
    c->xpre_of.d = d;
    c->xpre_of.f16 = run_f16;
  }
  // L2 batches on the split-operand screen keep the centroids split for the
  // run: a full split after each row-norms readout (the first batch, and
  // after a revival moved rows), then the EMA rewrites the rows it moves.
  const bool keep_csplit = pre && !sph;
  void* tsplit = keep_csplit ? c->tsplit.get(halves_bytes(k, d)) : nullptr;
  // The bound's centroid maxima: halves_blocks(k) pairs after a full split,
  // then one pair per EMA block, or per cluster after a small batch's update.
  // A revival's split appends one pair per split (at most k / 2) to those.
  const size_t tpart_pairs = halves_blocks(k) + std::max(ema_blocks(k), k) + k;
  uint32_t* tpart_h = keep_csplit ? (uint32_t*)c->tsplit_part.get(tpart_pairs * 8) : nullptr;
  const uint32_t* tpart_end = keep_csplit ? tpart_h + 2 * tpart_pairs : nullptr;
  uint32_t* tpart_e = keep_csplit ? tpart_h + 2 * halves_blocks(k) : nullptr;
  SplitCents pcents{tsplit, tpart_h, (int)halves_blocks(k), run_f16};
  // When the batches' top-1 runs the screen with d % 4 == 0 (the check and
  // the queued-row scan), or the latency-bound exact scan alone (small k),
  // it tallies the labels it writes (counts and the chunk histograms of the
  // counting sort), so scatter_add needs no count launch; the EMA clears
  // both for the next batch.
  const bool tally = top1_tallies(c, bsz, d, k, sph) && scatter_tallied(bsz, k);
  const size_t tstride = tally_stride(bsz);
  uint32_t* tcnt = tally ? (uint32_t*)c->tally_cnt.get(tstride * k * 4) : nullptr;
  if (tally) launch_fill_u32(c, tcnt, tstride * k, 0);
  uint32_t* d_lab[2] = {lab0.u(), lab1.u()};
  // The epoch's label counts, tallied batch by batch by the EMA launches: the
  // statistics' histogram, and for the last pass the closing means' counts.
  uint32_t* d_tally[2] = {tally0.u(), tally1.u()};
  float* d_sco[2] = {sco0.f(), sco1.f()};
  // The start (model.rs:772-797): saved EMA state as it is (begin_with_state);
  // else initial centroids, given (begin) or the rows permutation(n)[..k],
  // normalized when spherical (model.rs:306-316), masses INIT_USAGE
  // (recipe.rs:14).
  if (resume) {
    h2d(c, pos.p, init->positions, k * d * 4);
    h2d(c, mass.p, init->usage, k * 4);
  } else {
    if (init && init->centroids) {
      h2d(c, pos.p, init->centroids, k * d * 4);
    } else if (init && init->centroids_dev) {
      EMH_HIP(hipMemcpyAsync(pos.p, init->centroids_dev->ptr, k * d * 4, hipMemcpyDeviceToDevice,
                             c->stream));
    } else if (n == k) {
      EMH_HIP(hipMemcpyAsync(pos.p, x, k * d * 4, hipMemcpyDeviceToDevice, c->stream));
    } else {
      init_perm.get();
      copy_async(c, init_ids.p, h_order[1], k * 4, hipMemcpyHostToDevice);
      launch_gather_rows(c, x, n, d, init_ids.u(), k, pos.f());
    }
    if (sph) {
      launch_normalize_rows(c, pos.f(), k, d, readout.f());
      EMH_HIP(hipMemcpyAsync(pos.p, readout.p, k * d * 4, hipMemcpyDeviceToDevice, c->stream));
    }
    const float init_usage = 1.0f / 65536.0f;
    uint32_t init_bits;
    std::memcpy(&init_bits, &init_usage, 4);
    launch_fill_u32(c, mass.u(), k, init_bits);
  }
  launch_check_finite(c, pos.f(), k * d, c->small + SW_BAD_INIT);
  launch_fill_u32(c, pass.u(), k * d, 0);
  launch_fill_u32(c, counts.u(), k, 0);  // each EMA leaves them at zero for the next batch
  copy_async(c, h_small0, c->small, SW_WORDS * 4, hipMemcpyDeviceToHost);
  ev_order[1].record(c->stream);  // the initial ids are out of h_order[1]
  ev_init.record(c->stream);
  // The check of the initial centroids (finite) is read once the first
  // batch's top-1 is queued, so the device is not idle meanwhile.
  bool init_checked = false;
  if (cfg.verbose)
    fprintf(stderr, "Clustering %zu points in %zuD to %zu clusters, %g epochs (batch %zu, alpha0 %.3f%s)\n",
            n, d, k, cfg.nepochs, bsz, R.alpha0, sph ? ", spherical" : "");

  gnext = beside([&] { return gumbel_terms(split_rng, k); });
  // After a revival used them, the next block is drawn on a helper once the
  // next batch's kernels are queued, off the GPU's path.
  auto take_gumbel = [&] { return gnext.get(); };
  bool refill = false;
  size_t n_splits = 0, step = 0;
  bool norms_stale = true;  // L2 readout: the EMA keeps the norms of the rows it moves
  // Spherical readout: the EMA writes the normalized rows it moves, so a full
  // normalize_rows runs only at the start and after a revival's splits.
  const bool ema_readout = sph && d <= EMA_READOUT_MAX_D;
  bool readout_stale = true;
  std::vector<emh_epoch_stats> stats;
  for (size_t epoch = 0; epoch < n_epochs; epoch++) {
    const size_t rows = R.epoch_rows[epoch];
    const bool last = epoch + 1 == n_epochs;
    const int buf = (int)(epoch & 1);
    next.get();
    cross_wait(c->stream, ev_order[buf].e);  // this epoch's order is in
    cross_wait(c->stream, ev_epoch[buf].e);  // labels of epoch - 2 are out
    if (!last) next = beside([&, e1 = epoch + 1] { fill_order(e1); });
    launch_fill_u32(c, d_tally[buf], k, 0);
    uint32_t* order = d_order[buf];
    uint32_t* lab = d_lab[buf];
    float* sco = d_sco[buf];
    const size_t splits_before = n_splits;
    for (size_t b = 0; b < rows; b += bsz) {
      const size_t e = std::min(b + bsz, rows);
      if (sph) {
        if (!ema_readout || readout_stale) launch_normalize_rows(c, pos.f(), k, d, readout.f());
        readout_stale = false;
      } else if (norms_stale) {
        launch_row_norms(c, pos.f(), k, d, readout.f());
        norms_stale = false;
        if (keep_csplit) {
          launch_halves(c, pos.f(), k, d, nullptr, 0, k, tsplit, (float*)c->csplit_norm.get(k * 4),
                        readout.f(), tpart_h, run_f16);
          pcents.part = tpart_h;
          pcents.nparts = (int)halves_blocks(k);
        }
      }
      const float* cents = sph ? readout.f() : pos.f();
      const float* cn = sph ? nullptr : readout.f();
      const LabelTally tl{tcnt, counts.u(), b, tstride};
      for (size_t c0 = b; c0 < e; c0 += chunk) {
        const size_t c1 = std::min(c0 + chunk, e);
        // After the first step the previous EMA cleared the screen's words.
        launch_top1(c, x, n, d, order, c0, c1, cents, cn, k, sph, lab, sco,
                    step > 0 && c0 == b, nullptr, pre, keep_csplit ? &pcents : nullptr,
                    tally ? &tl : nullptr);
      }
      if (!init_checked) {
        ev_init.wait();
        raise_flags(c, h_small0);
        init_checked = true;
      }
      if (refill) {  // the next check's Gumbel terms, drawn while the GPU works
        gnext = beside([&] { return gumbel_terms(split_rng, k); });
        refill = false;
      }
      const double alpha = scheduled_alpha(R.alpha0, step, R.total_steps);
      const float af = (float)alpha, df = (float)(1.0 - alpha);
      const int replace = alpha == 1.0;
      const bool check = (step + 1) % 5 == 0;  // CHECK_UNUSED_EVERY (recipe.rs:12)
      // scatter_add in two segments: counts, then (after the revival check's
      // mass preview, which needs only the counts) the ordered sums.
      const bool tsc = prof_take(c, EMH_PROF_SCATTER);
      if (!tally) {
        ProfScope p(c, EMH_PROF_SCATTER, 0.0, tsc, false);
        launch_scatter_count(c, b, e, lab, k, counts.u(), true);
      }
      if (check)
        launch_mass_preview(c, mass.f(), counts.u(), k, af, df, replace, d_usage_h, d_small_h,
                            d_small_h + 2 * SW_WORDS, ++seq_no);
      if (tally && update_small(e - b, d, sph)) {
        // A small batch (the automatic-k sweeps' fits): placement, sums and
        // the EMA step in one launch, the same bits.
        ProfScope p(c, EMH_PROF_SCATTER,
                    scatter_bytes(e - b, k, d, true, last) + ema_bytes(k, d), tsc);
        launch_update_small(c, x, n, d, order, b, e, lab, k, counts.u(), tcnt, tstride * k,
                            last ? pass.f() : nullptr, pos.f(), mass.f(), af, df, replace,
                            sph ? nullptr : readout.f(), tsplit, tpart_e,
                            sph ? readout.f() : nullptr, d_tally[buf], run_f16);
        if (keep_csplit) {
          pcents.part = tpart_e;
          pcents.nparts = (int)k;
        }
      } else {
        {
          ProfScope p(c, EMH_PROF_SCATTER, scatter_bytes(e - b, k, d, true, last), tsc);
          launch_scatter_sums(c, x, n, d, order, b, e, lab, k, sums.f(),
                              last ? pass.f() : nullptr, tally ? counts.u() : nullptr, tcnt,
                              tstride);
        }
        ProfScope p(c, EMH_PROF_EMA, ema_bytes(k, d), prof_take(c, EMH_PROF_EMA));
        launch_ema(c, pos.f(), mass.f(), sums.f(), counts.u(), k, d, af, df, replace,
                   sph ? nullptr : readout.f(), true, d_tally[buf], true, tsplit, tpart_e, tcnt,
                   tally ? tstride * k : 0, ema_readout ? readout.f() : nullptr, run_f16);
        if (keep_csplit) {
          pcents.part = tpart_e;
          pcents.nparts = (int)ema_blocks(k);
        }
      }
      if (check) {
        wait_posted(c, h_seq, seq_no);
        raise_flags(c, h_small);
        std::vector<float> usage(h_usage, h_usage + k);
        std::vector<uint32_t> plan = plan_revival(usage, R.tau, take_gumbel);
        if (!plan.empty()) {
          const size_t np = plan.size() / 2;
          std::memcpy(h_plan, plan.data(), plan.size() * 4);
          if (!sph && d <= SPLIT_FUSED_MAX_D) {
            // Donors and dead are disjoint. The split also leaves the moved
            // rows' norms and (split screen) halves, and appends a bound
            // partial per pair: no full row_norms and halves pass follows.
            uint32_t* app = keep_csplit ? const_cast<uint32_t*>(pcents.part) +  // tpart_h's
                                              2 * (size_t)pcents.nparts
                                        : nullptr;
            EMH_ENSURE(!keep_csplit || app + 2 * np <= tpart_end, "bound partials overflow");
            launch_split_fused(c, pos.f(), mass.f(), d_plan, np, d, k, readout.f(),
                               keep_csplit ? tsplit : nullptr, app, run_f16);
            if (keep_csplit) pcents.nparts += (int)np;
          } else {
            launch_split(c, pos.f(), mass.f(), d_plan, np, d, true);
            norms_stale = true;
          }
          n_splits += np;
          readout_stale = true;
        }
        refill = !gnext.valid();  // scheduled after the next batch's launches
      }
      step++;
    }
    // Epoch end: labels and scores go out; the statistics (train.rs:224-279)
    // wait for them on a helper thread.
    ev_done[buf].record(c->stream);
    cross_wait(cps, ev_done[buf].e);
    EMH_HIP(hipMemcpyAsync(h_lab[buf], d_tally[buf], k * 4, hipMemcpyDeviceToHost, cps));
    EMH_HIP(hipMemcpyAsync(h_sco[buf], sco, rows * 4, hipMemcpyDeviceToHost, cps));
    ev_epoch[buf].record(cps);
    if (pending.valid()) stats.push_back(pending.get());  // frees the other buffer pair
    const size_t nsplit = n_splits - splits_before;
    pending = beside([&, rows, buf, nsplit, epoch, st = step]() {
      ev_epoch[buf].wait();
      const double t =
          std::chrono::duration<double>(std::chrono::steady_clock::now() - t_start).count();
      const float* sc = h_sco[buf];
      // The objective: one in-order f64 chain per (batch, chunk), as
      // train.rs adds them; eight chains run interleaved (each with the same
      // adds in the same order), then the batches' sums are added in order.
      struct Chain {
        size_t c0, c1;
        double s;
      };
      std::vector<Chain> ch;
      std::vector<size_t> nper;  // chunks per batch
      for (size_t b = 0; b < rows; b += bsz) {
        const size_t e = std::min(b + bsz, rows);
        size_t m = 0;
        for (size_t c0 = b; c0 < e; c0 += chunk, m++) {
          const size_t c1 = std::min(c0 + chunk, e);
          ch.push_back({c0, c1, sph ? 2.0 * (double)(c1 - c0) : 0.0});
        }
        nper.push_back(m);
      }
      auto term = [&](float v) { return sph ? (double)(-2.0f * v) : (double)v; };
      for (size_t g0 = 0; g0 < ch.size(); g0 += 8) {
        const size_t ng = std::min<size_t>(8, ch.size() - g0);
        size_t len = ch[g0].c1 - ch[g0].c0;
        for (size_t g = 1; g < ng; g++) len = std::min(len, ch[g0 + g].c1 - ch[g0 + g].c0);
        double acc[8];
        const float* ptr[8];
        for (size_t g = 0; g < 8; g++) {  // lanes past ng repeat chain g0 and are discarded
          const Chain& q = ch[g0 + (g < ng ? g : 0)];
          acc[g] = q.s;
          ptr[g] = sc + q.c0;
        }
        for (size_t i = 0; i < len; i++)
          for (int g = 0; g < 8; g++) acc[g] += term(ptr[g][i]);
        for (size_t g = 0; g < ng; g++) {
          Chain& q = ch[g0 + g];
          for (size_t i = len; i < q.c1 - q.c0; i++) acc[g] += term(ptr[g][i]);
          q.s = acc[g];
        }
      }
      double obj_epoch = 0.0;
      for (size_t b = 0, i = 0; b < nper.size(); b++) {
        double obj_batch = 0.0;
        for (size_t m = 0; m < nper[b]; m++, i++) obj_batch += ch[i].s;
        obj_epoch += obj_batch;
      }
      const uint32_t* hist = h_lab[buf];  // the epoch's tallied counts
      double sq = 0.0;
      for (size_t j = 0; j < k; j++) sq += (double)hist[j] * (double)hist[j];
      emh_epoch_stats es;
      es.obj = obj_epoch;
      es.time = t;
      es.imbalance_factor = (double)k * sq / ((double)rows * (double)rows);
      es.nsplit = nsplit;
      if (cfg.verbose)
        fprintf(stderr, "  Epoch %zu / %zu (%zu rows), iteration %zu (%.2f s): objective=%.17g\n",
                epoch + 1, n_epochs, rows, st, t, obj_epoch);
      return es;
    });
  }
  // The end: positions and masses are final after the last EMA and go out on
  // the copy stream while the closing means (core/mod.rs:404-429: the last
  // pass's label counts, sums / count; the counts were tallied batch by batch
  // by the last pass's EMA launches) and the labels by data row are computed;
  // the host copies into the caller's arrays run in parallel.
  const size_t rows_last = R.epoch_rows.back();
  const int lb = (int)((n_epochs - 1) & 1);
  ev_last.record(c->stream);
  cross_wait(cps, ev_last.e);
  EMH_HIP(hipMemcpyAsync(h_out + k * d, pos.p, k * d * 4, hipMemcpyDeviceToHost, cps));
  EMH_HIP(hipMemcpyAsync(h_out + 2 * k * d, mass.p, k * 4, hipMemcpyDeviceToHost, cps));
  ev_posout.record(cps);
  launch_closing(c, pos.f(), pass.f(), d_tally[lb], k, d, sums.f());
  const float* C = sums.f();
  if (sph) {
    launch_normalize_rows(c, sums.f(), k, d, pass.f());
    C = pass.f();
  }
  if (out->centroids_dev)
    EMH_HIP(hipMemcpyAsync(out->centroids_dev->ptr, C, k * d * 4, hipMemcpyDeviceToDevice,
                           c->stream));
  copy_async(c, h_out, C, k * d * 4, hipMemcpyDeviceToHost);
  uint32_t* h_rowlab = h_lab[lb ^ 1];  // free: its epoch's statistics are done
  if (out->labels && capture) {
    launch_labels_by_row(c, d_order[lb], d_lab[lb], rows_last, n, d_lab[lb ^ 1]);
    copy_async(c, h_rowlab, d_lab[lb ^ 1], n * 4, hipMemcpyDeviceToHost);
  }
  copy_async(c, h_small, c->small, SW_WORDS * 4, hipMemcpyDeviceToHost);
  auto side = beside([&] {
    ev_posout.wait();
    if (out->positions) std::memcpy(out->positions, h_out + k * d, k * d * 4);
    if (out->usage) std::memcpy(out->usage, h_out + 2 * k * d, k * 4);
  });
  struct JoinSide {  // an error below must not leave the task using this frame
    std::future<void>& f;
    ~JoinSide() {
      if (f.valid()) f.wait();
    }
  } join_side{side};
  EMH_HIP(hipStreamSynchronize(c->stream));
  stats.push_back(pending.get());
  raise_flags(c, h_small);
  // The outputs: the centroids in four pieces (three on helpers), the labels
  // beside them.
  {
    constexpr int T = 4;
    const size_t cb = k * d * 4, part = (cb / T + 63) & ~size_t(63);
    std::future<void> f[T];
    struct JoinAll {  // no piece may outlive this frame, also on an error
      std::future<void>* f;
      ~JoinAll() {
        for (int t = 0; t < T; t++)
          if (f[t].valid()) f[t].wait();
      }
    } join_all{f};
    for (int t = 1; t < T; t++) {
      const size_t a = std::min(cb, t * part), b = std::min(cb, a + part);
      if (a < b)
        f[t] = beside([=] { std::memcpy((char*)out->centroids + a, (const char*)h_out + a, b - a); });
    }
    if (out->labels)
      f[0] = beside([&] {
        if (capture)
          std::memcpy(out->labels, h_rowlab, n * 4);
        else
          std::fill(out->labels, out->labels + n, -1);
      });
    std::memcpy(out->centroids, h_out, std::min(cb, part));
    for (auto& x : f)
      if (x.valid()) x.get();
  }
  side.get();
  out->n_epochs = n_epochs;
  for (size_t e = 0; e < n_epochs && e < out->max_epochs; e++)
    if (out->stats) out->stats[e] = stats[e];
  out->n_splits = n_splits;
  out->batch_size = bsz;
  out->alpha0 = R.alpha0;
  out->total_steps = R.total_steps;
  out->fallback_rows = (uint32_t)(h_small[SW_FALLBACK_TOTAL] - h_small0[SW_FALLBACK_TOTAL]);
}

// dedup_with_neighbors (dedup.rs:186-358).
float dot_seq(const float* a, const float* b, size_t d) {  // dedup.rs:158-160
  float s = 0.0f;
  for (size_t t = 0; t < d; t++) {
    float p = a[t] * b[t];
    s = s + p;
  }
  return s;
}

// Disjoint sets whose root is always the lowest row of its set: a union
// hangs the higher root under the lower (dedup.rs:139-155), so results do
// not depend on the order of the unions.
struct LowRootSets {
  std::vector<uint32_t> up;
  explicit LowRootSets(size_t n) : up(n) {
    for (size_t i = 0; i < n; i++) up[i] = (uint32_t)i;
  }
  uint32_t root(uint32_t i) {
    while (up[i] != i) {
      up[i] = up[up[i]];
      i = up[i];
    }
    return i;
  }
  void join(uint32_t a, uint32_t b) {
    a = root(a);
    b = root(b);
    if (a != b) up[std::max(a, b)] = std::min(a, b);
  }
};

// Rows bucketed by a key that is itself a row id (a set's lowest row): for
// each key in ascending order, its rows in ascending order.
struct Buckets {
  std::vector<uint32_t> start, rows;
  Buckets(const std::vector<uint32_t>& key, size_t n) : start(n + 1, 0), rows(n) {
    for (size_t i = 0; i < n; i++) start[key[i] + 1]++;
    for (size_t k = 0; k < n; k++) start[k + 1] += start[k];
    std::vector<uint32_t> at(start.begin(), start.end() - 1);
    for (size_t i = 0; i < n; i++) rows[at[key[i]]++] = (uint32_t)i;
  }
  size_t size(uint32_t k) const { return start[k + 1] - start[k]; }
  const uint32_t* begin(uint32_t k) const { return rows.data() + start[k]; }
  const uint32_t* end(uint32_t k) const { return rows.data() + start[k + 1]; }
};

struct DedupSide {
  const double* t = nullptr;
  const int64_t* burst = nullptr;
  const float* priority = nullptr;
  bool gap = false;
  double max_gap = 0.0;
};

size_t dedup_groups(const float* x, size_t n, size_t d, const uint32_t* nb_ids,
                    const float* nb_sims, size_t kk, float sim_t, float rep_t,
                    const DedupSide& side, uint32_t* group_of, uint32_t* reps, uint32_t* anchors,
                    uint32_t* sizes, size_t* linked, size_t* split_components) {
  // A link or a star membership needs the two rows' times within the gap
  // when both are known (dedup.rs:213-221).
  auto time_ok = [&](size_t i, size_t j) {
    if (!side.gap || !side.t || !std::isfinite(side.t[i]) || !std::isfinite(side.t[j]))
      return true;
    return std::fabs(side.t[i] - side.t[j]) <= side.max_gap;
  };
  auto row = [&](size_t i) { return x + i * d; };
  // Burst units: the rows of one burst id (dedup.rs:224-233).
  LowRootSets unit(n);
  if (side.burst) {
    std::unordered_map<int64_t, uint32_t> first;
    for (size_t i = 0; i < n; i++)
      if (side.burst[i] >= 0) unit.join(first.emplace(side.burst[i], (uint32_t)i).first->second,
                                        (uint32_t)i);
  }
  std::vector<uint32_t> unit_of(n);
  for (size_t i = 0; i < n; i++) unit_of[i] = unit.root((uint32_t)i);
  // Components: the units, joined by the links that pass the threshold and
  // the time rule (dedup.rs:234-254). A row's degree counts its distinct links.
  LowRootSets comp(n);
  for (size_t i = 0; i < n; i++) comp.join(unit_of[i], (uint32_t)i);
  std::vector<uint64_t> links;
  for (size_t i = 0; i < n; i++)
    for (size_t t = 0; t < kk; t++) {
      const uint32_t j = nb_ids[i * kk + t];
      if (j == 0xffffffffu || j >= n || nb_sims[i * kk + t] < sim_t || !time_ok(i, j)) continue;
      comp.join((uint32_t)i, j);
      const uint64_t a = std::min<uint64_t>(i, j), b = std::max<uint64_t>(i, j);
      links.push_back(a << 32 | b);
    }
  std::sort(links.begin(), links.end());
  links.erase(std::unique(links.begin(), links.end()), links.end());
  std::vector<uint32_t> degree(n, 0);
  for (uint64_t l : links) {
    degree[l >> 32]++;
    degree[l & 0xffffffffu]++;
  }
  std::vector<uint32_t> comp_of(n);
  for (size_t i = 0; i < n; i++) comp_of[i] = comp.root((uint32_t)i);
  const Buckets members(comp_of, n), units(unit_of, n);
  // Star cover of each component (dedup.rs:263-309): the untaken row with the
  // most links (then the lowest id) anchors a group; its own burst unit is in
  // it whatever the similarity; every other untaken unit joins when all its
  // rows are within rep_t of the anchor and pass the time rule.
  std::vector<std::pair<std::vector<uint32_t>, uint32_t>> groups;
  size_t split = 0;
  std::vector<char> taken(n, 0);
  std::vector<uint32_t> comp_units, order;
  for (uint32_t c0 = 0; c0 < n; c0++) {
    if (members.size(c0) == 0) continue;
    if (members.size(c0) == 1) {
      groups.push_back({{c0}, c0});
      continue;
    }
    comp_units.clear();  // the component's unit roots, ascending
    order.assign(members.begin(c0), members.end(c0));
    for (uint32_t r : order)
      if (unit_of[r] == r) comp_units.push_back(r);
    std::sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) {
      return degree[a] != degree[b] ? degree[a] > degree[b] : a < b;
    });
    const size_t before = groups.size();
    for (uint32_t c : order) {
      const uint32_t cu = unit_of[c];
      if (taken[cu]) continue;
      taken[cu] = 1;
      std::vector<uint32_t> g(units.begin(cu), units.end(cu));
      for (uint32_t u : comp_units) {
        if (taken[u]) continue;
        bool fits = true;
        for (const uint32_t* r = units.begin(u); fits && r != units.end(u); ++r)
          fits = time_ok(*r, c) && dot_seq(row(*r), row(c), d) >= rep_t;
        if (fits) {
          taken[u] = 1;
          g.insert(g.end(), units.begin(u), units.end(u));
        }
      }
      std::sort(g.begin(), g.end());
      groups.push_back({std::move(g), c});
    }
    if (groups.size() - before > 1) split++;
  }
  std::sort(groups.begin(), groups.end(),
            [](const auto& a, const auto& b) { return a.first[0] < b.first[0]; });
  // Representatives (dedup.rs:315-340): the highest priority, then the highest
  // mean similarity to the other members (an f64 sum in member order), then
  // the lowest id.
  for (size_t gi = 0; gi < groups.size(); gi++) {
    const auto& g = groups[gi].first;
    anchors[gi] = groups[gi].second;
    sizes[gi] = (uint32_t)g.size();
    uint32_t rep = g[0];
    if (g.size() > 1) {
      float bp = -INFINITY;
      double bm = -INFINITY;
      rep = 0xffffffffu;
      for (uint32_t a : g) {
        double s = 0.0;
        for (uint32_t b : g)
          if (b != a) s += (double)dot_seq(row(a), row(b), d);
        const double mean = s / (double)(g.size() - 1);
        const float p = side.priority ? side.priority[a] : 0.0f;
        if (p > bp || (p == bp && mean > bm)) {
          bp = p;
          bm = mean;
          rep = a;
        }
      }
    }
    reps[gi] = rep;
    for (uint32_t r : g) group_of[r] = (uint32_t)gi;
  }
  *linked = links.size();
  *split_components = split;
  return groups.size();
}

// ------------------------------------------------------------- auto-k pieces
// kmeans_pp (emeans-cluster/src/auto.rs:401-455) on rows resident on the
// device: each pick's row dots raise every row's best cosine on the device
// (k_pp_best); the D^2 weights, their f64 sum and the draw run here in row
// order, as the reference's.
std::vector<uint32_t> kmeans_pp_dev(emh_ctx* c, const float* x, size_t n, size_t d, size_t kmax,
                                    uint32_t seed) {
  kmax = std::min(kmax, n);
  std::vector<uint32_t> picks;
  if (kmax == 0) return picks;
  RandomState rng(seed);
  size_t last = (size_t)rng.interval(n - 1);
  picks.push_back((uint32_t)last);
  Arena ar = arena_for(c->kpp, {n * 4});
  Buf best(ar, n * 4);
  launch_fill_u32(c, best.u(), n, 0xff800000u);  // -inf
  float* hb = (float*)c->pin_aux.get(n * 4);
  std::vector<double> w(n);
  std::vector<char> picked(n, 0);
  picked[last] = 1;
  while (picks.size() < kmax) {
    launch_pp_best(c, x, n, d, last, best.f());
    copy_async(c, hb, best.p, n * 4, hipMemcpyDeviceToHost);
    EMH_HIP(hipStreamSynchronize(c->stream));
    double total = 0.0;
    for (size_t i = 0; i < n; i++) {
      const double dist = std::fmax(1.0 - (double)hb[i], 0.0);
      w[i] = dist * dist;
      total += w[i];
    }
    size_t next = 0;
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
      if (w[j] == 0.0) {  // rounding landed on a zero weight: the last of the largest
        size_t m = 0;
        for (size_t i = 1; i < n; i++)
          if (!(w[i] < w[m])) m = i;
        j = m;
      }
      next = j;
    } else {  // every row coincides with a pick: the first unpicked row
      while (next < n && picked[next]) next++;
      if (next == n) next = 0;
    }
    picks.push_back((uint32_t)next);
    picked[next] = 1;
    last = next;
  }
  return picks;
}

// internal_scores (emeans-cluster/src/metrics.rs:113-268) of labels (n, on
// the device, < k) on unit rows resident on the device. The cluster sums and
// every row's terms come from the device; the row-order f64 sums, the
// Calinski-Harabasz dispersions and the Davies-Bouldin ratios run here.
void internal_scores_dev(emh_ctx* c, const float* x, size_t n, size_t d, const uint32_t* labels_d,
                         size_t k, emh_internal* out, uint64_t* sizes_out) {
  std::vector<uint32_t> lab(n);
  copy_async(c, lab.data(), labels_d, n * 4, hipMemcpyDeviceToHost);
  EMH_HIP(hipStreamSynchronize(c->stream));
  std::vector<uint64_t> sizes(k, 0);
  for (size_t i = 0; i < n; i++) {
    EMH_ENSURE(lab[i] < k, "label out of range");
    sizes[lab[i]]++;
  }
  std::vector<uint32_t> live, slot(k, 0xffffffffu);
  for (size_t j = 0; j < k; j++)
    if (sizes[j] > 0) {
      slot[j] = (uint32_t)live.size();
      live.push_back((uint32_t)j);
    }
  const size_t ke = live.size();
  // Rows grouped by cluster, in row order within each (a stable counting sort).
  std::vector<uint32_t> start(ke + 1, 0), rid(n), own(n);
  for (size_t s = 0; s < ke; s++) start[s + 1] = start[s] + (uint32_t)sizes[live[s]];
  {
    std::vector<uint32_t> at(start.begin(), start.end() - 1);
    for (size_t i = 0; i < n; i++) {
      own[i] = slot[lab[i]];
      rid[at[own[i]]++] = (uint32_t)i;
    }
  }
  Arena ar = arena_for(c->iscore, {n * 4, (ke + 1) * 4, n * 4, ke * d * 8, ke * d * 4, ke * 8,
                                    ke * 8, n * ke * 4, n * 8, n * 8, n * 8, n * 8});
  Buf rid_d(ar, n * 4), start_d(ar, (ke + 1) * 4), own_d(ar, n * 4), sums_d(ar, ke * d * 8),
      s32_d(ar, ke * d * 4), size_d(ar, ke * 8), sq_d(ar, ke * 8), g_d(ar, n * ke * 4),
      xx_d(ar, n * 8), sil_d(ar, n * 8), obj_d(ar, n * 8), dist_d(ar, n * 8);
  h2d(c, rid_d.p, rid.data(), n * 4);
  h2d(c, start_d.p, start.data(), (ke + 1) * 4);
  h2d(c, own_d.p, own.data(), n * 4);
  std::vector<double> sums(ke * d), sq(ke, 0.0), size(ke);
  if (ke > 0) launch_sum64(c, x, d, rid_d.u(), start_d.u(), ke, (double*)sums_d.p);
  d2h(c, sums.data(), sums_d.p, ke * d * 8);
  std::vector<float> s32(ke * d);
  for (size_t s = 0; s < ke; s++) {
    size[s] = (double)sizes[live[s]];
    for (size_t t = 0; t < d; t++) {
      const double v = sums[s * d + t];
      s32[s * d + t] = (float)v;
      sq[s] += v * v;
    }
  }
  h2d(c, s32_d.p, s32.data(), ke * d * 4);
  h2d(c, size_d.p, size.data(), ke * 8);
  h2d(c, sq_d.p, sq.data(), ke * 8);
  std::vector<double> xx(n), sil(n), obj(n), dist(n);
  if (n > 0) {
    if (ke > 0) {
      launch_row_dots(c, x, n, d, s32_d.f(), ke, g_d.f(), (double*)xx_d.p);
      launch_iscore_terms(c, n, ke, g_d.f(), (double*)xx_d.p, own_d.u(), (double*)size_d.p,
                          (double*)sq_d.p, (double*)sil_d.p, (double*)obj_d.p, (double*)dist_d.p);
    }
    d2h(c, xx.data(), xx_d.p, n * 8);
    d2h(c, sil.data(), sil_d.p, n * 8);
    d2h(c, obj.data(), obj_d.p, n * 8);
    d2h(c, dist.data(), dist_d.p, n * 8);
  }
  double sil_sum = 0.0, obj_sum = 0.0, total_xx = 0.0;
  std::vector<double> scatter(ke, 0.0);
  for (size_t i = 0; i < n; i++) {
    sil_sum += sil[i];
    obj_sum += obj[i];
    scatter[own[i]] += dist[i];
  }
  for (size_t i = 0; i < n; i++) total_xx += xx[i];
  const double nf = (double)std::max<size_t>(n, 1);
  double wsum = 0.0;
  for (size_t s = 0; s < ke; s++) wsum += sq[s] / size[s];
  const double within = total_xx - wsum;
  std::vector<double> grand(d, 0.0);
  for (size_t s = 0; s < ke; s++)
    for (size_t t = 0; t < d; t++) grand[t] += sums[s * d + t];
  double gsq = 0.0;
  for (size_t t = 0; t < d; t++) gsq += grand[t] * grand[t];
  const double between = (total_xx - gsq / nf) - within;
  out->calinski_harabasz = (ke < 2 || n <= ke || within <= 0.0)
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
          const double p = sums[a * d + t] / size[a], q = sums[b * d + t] / size[b];
          m2 += (p - q) * (p - q);
        }
        const double m = std::sqrt(m2);
        const double r = m > 0.0 ? (scatter[a] / size[a] + scatter[b] / size[b]) / m : INFINITY;
        worst = std::fmax(worst, r);
      }
      acc += worst;
    }
    db = acc / (double)ke;
  }
  out->k_eff = ke;
  out->silhouette = sil_sum / nf;
  out->davies_bouldin = db;
  out->objective = obj_sum / nf;
  if (sizes_out)
    for (size_t j = 0; j < k; j++) sizes_out[j] = sizes[j];
}

}  // namespace host
}  // namespace emh

namespace {
template <class F>
int guard2(F&& f) {
  try {
    f();
    return EMH_OK;
  } catch (const emh::Invalid& e) {
    emh::set_last_error(e.what());
    return EMH_INVALID;
  } catch (const std::exception& e) {
    emh::set_last_error(e.what());
    return EMH_ERROR;
  } catch (...) {
    emh::set_last_error("unknown error");
    return EMH_ERROR;
  }
}
}  // namespace

using namespace emh::host;

namespace {
// dedup_with_neighbors' argument checks (dedup.rs:193-211).
DedupSide check_dedup(const float* x, size_t n, size_t d, const emh_dedup_input* in,
                      const emh_dedup_config* cfg, const emh_dedup_result* out) {
  EMH_ENSURE(d > 0, "x must be n x d");
  EMH_ENSURE(cfg && out, "null argument");
  EMH_ENSURE(cfg->sim_threshold >= -1.0f && cfg->sim_threshold <= 1.0f,
             "sim_threshold must be in [-1, 1]");
  EMH_ENSURE(n == 0 || (x && out->group_of && out->representatives && out->anchors && out->sizes),
             "null argument");
  DedupSide s;
  if (in) {
    s.t = in->created_unix;
    s.burst = in->burst;
    s.priority = in->priority;
  }
  if (s.priority)
    for (size_t i = 0; i < n; i++)
      EMH_ENSURE(!std::isnan(s.priority[i]), "priority must not be NaN");
  s.gap = cfg->has_max_gap_secs != 0;
  s.max_gap = cfg->max_gap_secs;
  return s;
}
float rep_threshold(const emh_dedup_config* cfg) {
  return cfg->has_rep_threshold ? cfg->rep_threshold : cfg->sim_threshold;
}
}  // namespace

extern "C" {

int emh_train_dev(emh_ctx* c, const emh_buf* x, size_t n, const emh_config* cfg,
                  const emh_train_init* init, emh_train_out* out) {
  return guard2([&] {
    EMH_ENSURE(c && x && x->kind == 0, "x must be an f32 buffer");
    check_cfg(n, cfg, out);
    check_init(cfg, init);
    EMH_ENSURE(x->len == n * cfg->d, "x must be n x d");
    EMH_HIP(hipSetDevice(c->device));
    if (out->centroids_dev) ++out->centroids_dev->gen;
    train_dev(c, (const float*)x->ptr, n, *cfg, init, out);
    // The run split x's rows: an assignment of the same rows may take them,
    // while the buffer keeps these contents (Assigner::bind_data keeps the
    // bound copy only while bound, assign.rs:75-83).
    if (c->xpre_of.ptr == x->ptr && c->xpre_of.n == n && x->owned && !x->exposed) {
      c->xpre_of.serial = x->serial;
      c->xpre_of.gen = x->gen;
      c->xpre_of.valid = true;
    }
  });
}

int emh_train(emh_ctx* c, const float* x, size_t n, const emh_config* cfg,
              const emh_train_init* init, emh_train_out* out) {
  return guard2([&] {
    EMH_ENSURE(c && x, "null argument");
    check_cfg(n, cfg, out);
    check_init(cfg, init);
    EMH_HIP(hipSetDevice(c->device));
    Buf xd(c, n * cfg->d * 4);  // Device::bind: the data set goes to the device once
    upload(c, xd.p, x, n * cfg->d * 4);
    train_dev(c, xd.f(), n, *cfg, init, out);
  });
}

int emh_assign(emh_ctx* c, const float* x, size_t n, size_t d, const float* cents, size_t k,
               int metric, size_t chunk, uint32_t* labels, float* scores) {
  return guard2([&] {
    EMH_ENSURE(c && d > 0 && k > 0 && cents, "bad arguments");
    EMH_ENSURE(metric == EMH_L2 || metric == EMH_IP, "unknown metric");
    if (n == 0) return;
    EMH_ENSURE(x && labels && scores, "null argument");
    EMH_HIP(hipSetDevice(c->device));
    chunk = chunk ? chunk : 65536;
    // Centroids and their norms go up once for all chunks.
    Buf cb(c, k * d * 4), cn(c, k * 4);
    upload(c, cb.p, cents, k * d * 4);
    if (metric == EMH_L2) emh::launch_row_norms(c, cb.f(), k, d, cn.f());
    // A pipeline over the chunks: chunk i + 1 is staged in and copied to the
    // device while chunk i's kernels run; the device row buffers, labels and
    // scores alternate, and chunk i's results reach the caller's arrays (from
    // pinned memory) while chunk i + 1 runs.
    const size_t m = std::min(chunk, n);
    Buf xb0(c, m * d * 4), xb1(c, m * d * 4), lb0(c, m * 4), lb1(c, m * 4), sb0(c, m * 4),
        sb1(c, m * 4);
    float* xb[2] = {xb0.f(), xb1.f()};
    uint32_t* lb[2] = {lb0.u(), lb1.u()};
    float* sb[2] = {sb0.f(), sb1.f()};
    uint32_t* hl[2] = {(uint32_t*)c->pin_lab[0].get(m * 4), (uint32_t*)c->pin_lab[1].get(m * 4)};
    float* hs[2] = {(float*)c->pin_sco[0].get(m * 4), (float*)c->pin_sco[1].get(m * 4)};
    Event used[2], out[2];  // chunk's kernels done with its rows; its results in pinned memory
    size_t pend = SIZE_MAX;  // the chunk whose results wait for the caller's arrays
    auto deliver = [&](size_t i) {
      const size_t b = i * chunk, e = std::min(b + chunk, n);
      out[i & 1].wait();
      std::memcpy(labels + b, hl[i & 1], (e - b) * 4);
      std::memcpy(scores + b, hs[i & 1], (e - b) * 4);
    };
    for (size_t i = 0, b = 0; b < n; i++, b += chunk) {
      const size_t e = std::min(b + chunk, n);
      const int h = (int)(i & 1);
      upload(c, xb[h], x + b * d, (e - b) * d * 4, i >= 2 ? used[h].e : nullptr);
      emh::launch_top1(c, xb[h], e - b, d, nullptr, 0, e - b, cb.f(),
                       metric == EMH_L2 ? cn.f() : nullptr, k, metric == EMH_IP, lb[h], sb[h]);
      used[h].record(c->stream);
      if (pend != SIZE_MAX) deliver(pend);  // before reusing its pinned halves
      copy_async(c, hl[h], lb[h], (e - b) * 4, hipMemcpyDeviceToHost);
      copy_async(c, hs[h], sb[h], (e - b) * 4, hipMemcpyDeviceToHost);
      out[h].record(c->stream);
      pend = i;
    }
    deliver(pend);
    check_flags(c);
    EMH_HIP(hipStreamSynchronize(c->copies()));  // staging is free again
  });
}

int emh_assign_dev(emh_ctx* c, const emh_buf* x, size_t n, size_t d, const emh_buf* cents,
                   size_t k, int metric, size_t chunk, emh_buf* labels, emh_buf* scores) {
  return guard2([&] {
    EMH_ENSURE(c && x && cents && labels && scores, "null argument");
    EMH_ENSURE(d > 0 && k > 0, "d and k must be positive");
    EMH_ENSURE(metric == EMH_L2 || metric == EMH_IP, "unknown metric");
    EMH_ENSURE(x->kind == 0 && cents->kind == 0 && scores->kind == 0 && labels->kind == 1,
               "buffer kinds: x, centroids, scores f32; labels u32");
    EMH_ENSURE(x->len >= n * d && cents->len >= k * d, "x n x d, centroids k x d");
    EMH_ENSURE(labels->len >= n && scores->len >= n, "outputs too short");
    if (n == 0) return;
    EMH_HIP(hipSetDevice(c->device));
    ++scores->gen;
    chunk = chunk ? chunk : 65536;
    emh::Arena ar = arena_for(c->cnorm, {metric == EMH_L2 ? k * 4 : 0});
    Buf cn(ar, metric == EMH_L2 ? k * 4 : 0);
    if (metric == EMH_L2) emh::launch_row_norms(c, (const float*)cents->ptr, k, d, cn.f());
    // The rows' halves, when the context's last training run split these very
    // rows, in the format the screen mode takes, and nothing has written them
    // since.
    const emh_ctx::SplitOf& so = c->xpre_of;
    const bool reuse = so.valid && so.ptr == x->ptr && so.serial == x->serial &&
                       so.gen == x->gen && !x->exposed && so.d == d && n <= so.n &&
                       so.f16 == (c->screen == emh::SCREEN_F16);
    const emh::SplitRows pre{c->xpre.ptr, (const float*)c->xpre_norm.ptr, so.n, so.n * 128,
                             so.f16};
    for (size_t b = 0; b < n; b += chunk) {
      const size_t e = std::min(b + chunk, n);
      emh::launch_top1(c, (const float*)x->ptr, n, d, nullptr, b, e, (const float*)cents->ptr,
                       metric == EMH_L2 ? cn.f() : nullptr, k, metric == EMH_IP,
                       (uint32_t*)labels->ptr, (float*)scores->ptr, false, nullptr,
                       reuse ? &pre : nullptr);
    }
    EMH_HIP(hipStreamSynchronize(c->stream));  // cn's block is reused by the next call
  });
}

int emh_knn(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
            size_t kk, int exclude_self, uint32_t* ids, float* sims) {
  return emh_topk(c, q, m, data, n, d, kk, exclude_self, ids, sims);
}


int emh_dedup_neighbors(const float* x, size_t n, size_t d, const uint32_t* nb_ids,
                        const float* nb_sims, size_t kk, const emh_dedup_input* in,
                        const emh_dedup_config* cfg, emh_dedup_result* out) {
  return guard2([&] {
    const DedupSide s = check_dedup(x, n, d, in, cfg, out);
    EMH_ENSURE(n == 0 || (kk > 0 && nb_ids && nb_sims), "neighbours must have one row per row of x");
    size_t lp = 0, sc = 0;
    const size_t g = dedup_groups(x, n, d, nb_ids, nb_sims, kk, cfg->sim_threshold,
                                  rep_threshold(cfg), s, out->group_of, out->representatives,
                                  out->anchors, out->sizes, &lp, &sc);
    if (out->nn_sim)
      for (size_t i = 0; i < n; i++) out->nn_sim[i] = nb_sims[i * kk];
    out->n_groups = g;
    out->linked_pairs = lp;
    out->split_components = sc;
  });
}

int emh_dedup(emh_ctx* c, const float* x, size_t n, size_t d, const emh_dedup_input* in,
              const emh_dedup_config* cfg, emh_dedup_result* out) {
  return guard2([&] {
    EMH_ENSURE(c, "null context");
    check_dedup(x, n, d, in, cfg, out);
    const size_t k = std::max<size_t>(std::min<size_t>(cfg->k, n > 0 ? n - 1 : 0), 1);  // dedup.rs:172
    std::vector<uint32_t> ids(n * k, 0xffffffffu);
    std::vector<float> sims(n * k, -INFINITY);
    if (n > 1) {
      EMH_ENSURE(k <= (size_t)emh::KLONG, "dedup on the GPU searches at most %d neighbours",
                 emh::KLONG);
      if (emh_topk(c, x, n, x, n, d, k, 1, ids.data(), sims.data()) != EMH_OK)
        throw emh::Failure(emh_last_error());
    }
    if (emh_dedup_neighbors(x, n, d, ids.data(), sims.data(), k, in, cfg, out) != EMH_OK)
      throw emh::Failure(emh_last_error());
  });
}

int emh_kmeans_pp(emh_ctx* c, const emh_buf* x, size_t n, size_t d, size_t kmax, uint32_t seed,
                  uint32_t* picks, size_t* n_picks) {
  return guard2([&] {
    EMH_ENSURE(c && x && x->kind == 0 && picks && n_picks, "null argument");
    EMH_ENSURE(d > 0 && x->len >= n * d, "x must be n x d");
    EMH_ENSURE(n < (1ull << 32), "kmeans_pp: too many rows");
    EMH_HIP(hipSetDevice(c->device));
    const std::vector<uint32_t> p = kmeans_pp_dev(c, (const float*)x->ptr, n, d, kmax, seed);
    std::memcpy(picks, p.data(), p.size() * 4);
    *n_picks = p.size();
  });
}

int emh_internal_scores(emh_ctx* c, const emh_buf* x, size_t n, size_t d, const emh_buf* labels,
                        size_t k, emh_internal* out, uint64_t* sizes) {
  return guard2([&] {
    EMH_ENSURE(c && x && labels && out, "null argument");
    EMH_ENSURE(x->kind == 0 && labels->kind == 1, "x f32, labels u32");
    EMH_ENSURE(d > 0 && x->len >= n * d, "x must be n x d");
    EMH_ENSURE(labels->len >= n, "one label per row");
    EMH_ENSURE(k > 0 && n < (1ull << 32), "bad shape");
    EMH_HIP(hipSetDevice(c->device));
    emh_internal r{};
    internal_scores_dev(c, (const float*)x->ptr, n, d, (const uint32_t*)labels->ptr, k, &r, sizes);
    *out = r;
  });
}

int emh_dots(emh_ctx* c, const emh_buf* a, size_t m, const emh_buf* b, size_t nb, size_t d,
             emh_buf* out) {
  return guard2([&] {
    EMH_ENSURE(c && a && b && out, "null argument");
    EMH_ENSURE(a->kind == 0 && b->kind == 0 && out->kind == 0, "a, b and out must be f32 buffers");
    EMH_ENSURE(d > 0 && d < (1ull << 31), "d must be positive");
    EMH_ENSURE(nb < (1ull << 31), "dots: too many b rows");
    EMH_ENSURE(a->len >= m * d && b->len >= nb * d, "a must be m x d and b nb x d");
    EMH_ENSURE(out->len >= m * nb, "out must hold m x nb");
    if (m == 0 || nb == 0) return;
    EMH_HIP(hipSetDevice(c->device));
    ++out->gen;
    emh::launch_row_dots(c, (const float*)a->ptr, m, d, (const float*)b->ptr, nb, (float*)out->ptr,
                    nullptr);
  });
}

// Host-side pieces of the loop, exported for checks that need no device.
void emh_host_permutation(uint32_t seed, uint64_t n, uint32_t* out) {
  RandomState::permutation_into(seed, n, out);
}
double emh_host_random_sample(uint32_t seed, uint64_t skip) {
  RandomState r(seed);
  for (uint64_t i = 0; i < skip; i++) r.random_sample();
  return r.random_sample();
}
int emh_host_recipe(uint64_t n, const emh_config* cfg, uint64_t* batch_size, double* alpha0,
                    uint64_t* epoch_rows, uint64_t cap, uint64_t* n_epochs, uint64_t* total) {
  return guard2([&] {
    EMH_ENSURE(cfg && batch_size && alpha0 && n_epochs && total, "null argument");
    Recipe r = resolve(n, cfg->k, cfg->d, *cfg);
    *batch_size = r.batch_size;
    *alpha0 = r.alpha0;
    *n_epochs = r.epoch_rows.size();
    for (size_t e = 0; e < r.epoch_rows.size() && e < cap; e++) epoch_rows[e] = r.epoch_rows[e];
    *total = r.total_steps;
  });
}
double emh_host_scheduled_alpha(double alpha0, uint64_t step, uint64_t total) {
  return scheduled_alpha(alpha0, step, total);
}
// Revival plan from a fresh RandomState(seed); returns the number of pairs written.
uint64_t emh_host_plan_revival(const float* usage, uint64_t k, double tau, uint32_t seed,
                               uint32_t* pairs) {
  RandomState r(seed);
  std::vector<float> u(usage, usage + k);
  std::vector<uint32_t> p = plan_revival(u, tau, [&] { return gumbel_terms(r, k); });
  std::memcpy(pairs, p.data(), p.size() * 4);
  return p.size() / 2;
}
float emh_host_numpy_sum_f32(const float* a, uint64_t n) { return np_sum(a, n); }

}  // extern "C"
