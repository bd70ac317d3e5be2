// Internal declarations of the gfx950 backend: the context, buffers, error
// plumbing and the kernel launchers each .hip file provides.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/emeans_hip.h"

namespace emh {

// A failed check inside the library; turned into EMH_INVALID / EMH_ERROR at the ABI.
struct Invalid : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};

#define EMH_ENSURE(cond, ...)                                  \
  do {                                                         \
    if (!(cond)) {                                             \
      char _m[512];                                            \
      snprintf(_m, sizeof _m, __VA_ARGS__);                    \
      throw ::emh::Invalid(_m);                                \
    }                                                          \
  } while (0)

#define EMH_HIP(call)                                                               \
  do {                                                                              \
    hipError_t _e = (call);                                                         \
    if (_e != hipSuccess) {                                                         \
      char _m[512];                                                                 \
      snprintf(_m, sizeof _m, "%s failed: %s (%s:%d)", #call, hipGetErrorString(_e), \
               __FILE__, __LINE__);                                                 \
      throw ::emh::Failure(_m);                                                     \
    }                                                                               \
  } while (0)

void set_last_error(const std::string& m);

// Device scratch that grows on demand and is reused by later calls.
struct Scratch {
  void* ptr = nullptr;
  size_t bytes = 0;
  void* get(size_t need) {
    if (need > bytes) {
      // Queued kernels may still read the old block: wait before freeing it.
      if (ptr) {
        EMH_HIP(hipDeviceSynchronize());
        EMH_HIP(hipFree(ptr));
      }
      ptr = nullptr;
      size_t b = need + need / 4 + 4096;
      EMH_HIP(hipMalloc(&ptr, b));
      bytes = b;
    }
    return ptr;
  }
  // The same, with a new block zeroed in stream order (counters that every
  // use leaves at zero again).
  void* get_zeroed(size_t need, hipStream_t s) {
    if (need > bytes) {
      get(need);
      EMH_HIP(hipMemsetAsync(ptr, 0, bytes, s));
    }
    return ptr;
  }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
};

// Where an op takes its per-call device scratch: the context's growing
// buffers (no Arena), or one fixed block carved in order, 256-byte aligned,
// with the regions that must start at zero cleared by a fill kernel on every
// call. Carving past the block's end throws (the callers check the size first).
struct Arena {
  char* base = nullptr;
  size_t cap = 0, used = 0;
  void* take(size_t bytes) {
    const size_t at = (used + 255) & ~size_t(255);
    if (at + bytes > cap) throw Invalid("scratch block too small for this call");
    used = at + bytes;
    return base + at;
  }
};

// Pinned host memory that grows on demand and is reused by later calls.
struct Pinned {
  void* ptr = nullptr;
  size_t bytes = 0;
  void* get(size_t need) {
    if (need > bytes) {
      if (ptr) {
        EMH_HIP(hipDeviceSynchronize());  // queued copies may still use it
        EMH_HIP(hipHostFree(ptr));
      }
      ptr = nullptr;
      size_t b = need + need / 4 + 4096;
      EMH_HIP(hipHostMalloc(&ptr, b, hipHostMallocDefault));
      bytes = b;
    }
    return ptr;
  }
  void release() {
    if (ptr) (void)hipHostFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
};

// Top-1 / top-k path (emh_set_screen): the exact kernels alone, or the MFMA
// screen ahead of the exact check: bf16 three-pass (SCREEN_BF3), f32, or
// (SCREEN_F16) fp16 two-pass on the split-operand top-1 screen with every
// other screen in bf16 three-pass. Rows or centroids beyond |x| = 32768 make
// the fp16 bound NaN: those rows take the exact scan.
enum ScreenMode : int { SCREEN_OFF = 0, SCREEN_BF3 = 1, SCREEN_F32 = 2, SCREEN_F16 = 3 };
// Top-1 calls of at most this many exact items (rows x max(ceil(k / 64), 2))
// run the exact kernels alone by default: there one launch takes less time
// than the screen's three (d = 768: the screen ~60 us at any size up to 8,192
// rows for k <= 16, ~85 us for k = 64 .. 256 up to 4,096 rows).
constexpr size_t EXACT_BELOW = 4096;
// Direct selections of at most this many items of the latency-bound scan
// (k_queued1: 4 rows x 16 centroids each, plus one per 4 rows for L2) take
// that scan instead of k_exact1 (~13 us against ~32 us at 64 items).
constexpr size_t QUEUED_DIRECT = 1024;
// A top-1 call's exact items.
inline size_t exact_items(size_t n, size_t k) {
  const size_t g = (k + 63) / 64;
  return n * (g < 2 ? 2 : g);
}

// Words of the context's small device block.
enum SmallWord : int {
  SW_FALLBACK_COUNT = 0,  // rows appended to the exact kernel's list by the current call
  SW_CMAX2 = 1,           // max over centroids of |c|^2 (f32 bits)
  SW_CNMAX = 2,           // max over centroids of the given cnorm (f32 bits)
  SW_BAD_LABEL = 3,       // set when scatter_add saw a label >= k
  SW_FALLBACK_TOTAL = 4,  // running total of rescanned rows (u32, wraps)
  SW_BAD_ID = 5,          // set when a selection named a row id >= n
  SW_TICKET = 6,          // blocks of the scatter count kernel that have finished (reset by the last)
  SW_NBIG = 7,            // clusters of the current scatter with more rows than the per-column path takes
  SW_BAD_INIT = 8,        // set when a training run's initial centroids are not finite
  SW_WORDS = 16,
};

}  // namespace emh

struct emh_buf {
  void* ptr = nullptr;
  size_t len = 0;   // elements
  int kind = 0;     // 0 f32, 1 u32
  bool owned = true;
  int device = -1;  // where the library allocated it
  // Which buffer and which contents, for the split rows a context keeps: a
  // serial number unique over the process, a generation every entry point
  // that writes the buffer advances, and whether its address was handed out
  // (emh_buf_ptr), after which writes can come from outside.
  uint64_t serial = 0;
  uint64_t gen = 0;
  mutable bool exposed = false;
};

struct emh_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  // Host<->device staging that overlaps the kernels, made on first use
  // (copies()): the runtime gives each new stream the least-used hardware
  // queue, so contexts made together (the automatic-k sweeps' four) get
  // their kernel streams on different queues when no copy stream comes
  // between them.
  hipStream_t copy_stream = nullptr;
  hipStream_t copies() {
    if (!copy_stream) EMH_HIP(hipStreamCreateWithFlags(&copy_stream, hipStreamNonBlocking));
    return copy_stream;
  }
  int cus = 256;
  int screen = emh::SCREEN_BF3;
  size_t exact_below = emh::EXACT_BELOW;  // emh_set_exact_below
  uint32_t* small = nullptr;  // SW_WORDS u32 on the device
  char* scratch = nullptr;    // the device's fixed scratch block (emh_top1_noalloc)
  uint64_t fallback_total = 0;
  emh::Scratch cand, fblist, order, start, misc, knn_tmp, xnorm, bigj, chunkcnt, tickets;
  emh::Scratch xsplit, csplit, csplit_norm, csplit_part;  // split-operand screen: a call's rows, centroids
  emh::Scratch xpre, xpre_norm;              // a training run's rows, split once
  // What xpre holds: the rows [0, n) of buffer `serial` at generation `gen`
  // (d dimensions, at address ptr); valid only for a buffer the library owns.
  struct SplitOf {
    bool valid = false;
    const void* ptr = nullptr;
    uint64_t serial = 0, gen = 0;
    size_t n = 0, d = 0;
    bool f16 = false;  // the halves' format (emh_halves.h)
  } xpre_of;
  emh::Scratch tsplit, tsplit_part;          // a training run's centroids, kept split by the EMA
  emh::Scratch tally_cnt;                    // a training run's label tally (chunk histograms)
  emh::Scratch klong;                        // top-k beyond 16: a query block's scores
  // Per-call buffers of the entry points that run many times in a row (a
  // training run's, k-means++'s, internal_scores', the assignment's norms):
  // carved from a block kept between calls, since hipFree waits for the
  // whole device, the other contexts' streams included.
  emh::Scratch trun, kpp, iscore, cnorm;
  emh::Scratch preview_ticket;  // k_mass_preview's last-block ticket (left at zero)
  // Host staging of the device loop: masses, plan, flags, epoch orders and
  // epoch labels/scores (double-buffered), results.
  emh::Pinned pin_usage, pin_plan, pin_small, pin_order[2], pin_lab[2], pin_sco[2], pin_out;
  // Staged uploads from pageable host memory (emh_host.cpp, upload): two
  // pinned halves, each with the event of the last copy that read it, and the
  // event the context stream waits on for the whole upload.
  emh::Pinned pin_stage[2];
  emh::Pinned pin_aux;  // kmeans_pp's best cosines on the way to the host
  hipEvent_t ev_stage[3] = {nullptr, nullptr, nullptr};
  std::string name = "hip-gfx950";
  // Op timing (emh_profile): event pairs on the context stream around every
  // prof-th instance of each timed op (EMH_PROF_*), with the algorithmic
  // units (FLOP or bytes) each instance covers; an op of several launches
  // records one pair per launch segment and counts once.
  int prof[EMH_PROF_OPS] = {};               // period per op (0: off)
  uint64_t prof_count[EMH_PROF_OPS] = {};    // instances seen since profiling was switched on
  struct Timed {
    hipEvent_t a, b;
    int op;
    double units;  // on the instance's last segment
    bool last;     // the instance's last segment
  };
  std::vector<Timed> timed;
  struct ProfSum {
    double ms = 0.0, units = 0.0;
    uint64_t instances = 0;
  };
  ProfSum prof_sum[EMH_PROF_OPS];
  std::vector<hipEvent_t> ev_pool;  // events for the timing, reused across reads
  size_t ev_used = 0;
  hipEvent_t pool_event() {
    if (ev_used == ev_pool.size()) {
      hipEvent_t e;
      EMH_HIP(hipEventCreate(&e));
      ev_pool.push_back(e);
    }
    return ev_pool[ev_used++];
  }
};

namespace emh {

inline dim3 grid1(size_t n, int per) { return dim3((unsigned)((n + per - 1) / per)); }

// Whether this instance of op is timed (every prof-th instance while profiling is on).
inline bool prof_take(emh_ctx* c, int op) {
  return c->prof[op] && c->prof_count[op]++ % (uint64_t)c->prof[op] == 0;
}

// Brackets a segment of one op instance (one or more launches) with events
// when `take`; `last` marks the instance's final segment, which carries its
// algorithmic units.
struct ProfScope {
  emh_ctx* c;
  hipEvent_t a = nullptr, b = nullptr;
  int op;
  double units;
  bool last;
  ProfScope(emh_ctx* ctx, int op_, double units_, bool take, bool last_ = true)
      : c(ctx), op(op_), units(units_), last(last_) {
    if (!take) return;
    a = c->pool_event();
    b = c->pool_event();
    EMH_HIP(hipEventRecord(a, c->stream));
  }
  ~ProfScope() {
    if (!a) return;
    if (hipEventRecord(b, c->stream) == hipSuccess) c->timed.push_back({a, b, op, units, last});
  }
};

// Algorithmic HBM bytes of one scatter_add of `rows` selected rows (row
// reads, labels, ids when given, sums and counts written, the accumulator
// read and written when given) and of one ema_update (positions read and
// written, sums read, masses read and written, counts read).
inline double scatter_bytes(size_t rows, size_t k, size_t d, bool ids, bool acc) {
  return 4.0 * ((double)rows * (double)d + (double)rows + (ids ? (double)rows : 0.0) +
                (double)k * (double)d + (double)k + (acc ? 2.0 * (double)k * (double)d : 0.0));
}
inline double ema_bytes(size_t k, size_t d) { return 4.0 * (3.0 * (double)k * (double)d + 4.0 * (double)k); }

// ---- launchers (emh_ops.hip)
void launch_fill_u32(emh_ctx* c, uint32_t* p, size_t n, uint32_t v);
void launch_row_norms(emh_ctx* c, const float* m, size_t rows, size_t d, float* out);
void launch_normalize_rows(emh_ctx* c, const float* src, size_t rows, size_t d, float* dst);
// With clear_screen_words, also zeroes the small-block words launch_top1
// clears before its screen (the fallback count and the bound maxima), so the
// next top-1 may skip that fill. With tally, also adds counts into it. With
// zero_counts, leaves counts at zero once read (the next batch's
// launch_scatter_count adds into them). With csplit (norms needed), also
// rewrites the halves (launch_halves' layout, k rows; fp16 with f16, else
// bf16) of the rows it
// moves and leaves the bound's centroid maxima of its ema_blocks(k) blocks in
// cpart, as launch_halves' part does. With zero_words, also clears
// zero_words[0..nzero) (a tally's chunk histograms). With readout (spherical
// runs, no norms, d <= EMA_READOUT_MAX_D), each moved row's normalize_rows
// readout is written there too (rows that did not move keep theirs).
constexpr size_t EMA_READOUT_MAX_D = 1024;
void launch_ema(emh_ctx* c, float* pos, float* usage, const float* sums, const uint32_t* counts,
                size_t k, size_t d, float alpha, float decay, int replace, float* norms = nullptr,
                bool clear_screen_words = false, uint32_t* tally = nullptr,
                bool zero_counts = false, void* csplit = nullptr, uint32_t* cpart = nullptr,
                uint32_t* zero_words = nullptr, size_t nzero = 0, float* readout = nullptr,
                bool f16 = false);
size_t ema_blocks(size_t k);
// The masses launch_ema will leave, into out (usage untouched); with
// small_out, also a copy of the small block's words; with seq_out, then seq
// into *seq_out once all of that is written. out, small_out and seq_out may be
// pinned host memory mapped into the device's address space.
void launch_mass_preview(emh_ctx* c, const float* usage, const uint32_t* counts, size_t k,
                         float alpha, float decay, int replace, float* out,
                         uint32_t* small_out = nullptr, uint32_t* seq_out = nullptr,
                         uint32_t seq = 0);
// counts = histogram of labels[0..n) (labels >= k skipped).
void launch_hist(emh_ctx* c, const uint32_t* labels, size_t n, size_t k, uint32_t* counts);
// Closing means: out[j] = sums[j] / counts[j] where counts[j] > 0, else pos[j].
void launch_closing(emh_ctx* c, const float* pos, const float* sums, const uint32_t* counts,
                    size_t k, size_t d, float* out);
// out[0..n) = -1, then out[order[p]] = lab[p] for p < rows.
void launch_labels_by_row(emh_ctx* c, const uint32_t* order, const uint32_t* lab, size_t rows,
                          size_t n, uint32_t* out);
// *flag = 1 when any of v[0..n) is not finite.
void launch_check_finite(emh_ctx* c, const float* v, size_t n, uint32_t* flag);
void launch_split(emh_ctx* c, float* pos, float* usage, const uint32_t* pairs_dev, size_t npairs,
                  size_t d, bool independent);
// launch_split of independent pairs that also writes the two moved rows'
// norms (L2 readout) and, when given, their halves (csplit, k rows; fp16 with
// f16, else bf16) and
// one bound partial pair per pair (cpart[2 q], cpart[2 q + 1]); d at most
// SPLIT_FUSED_MAX_D.
constexpr size_t SPLIT_FUSED_MAX_D = 1024;
void launch_split_fused(emh_ctx* c, float* pos, float* usage, const uint32_t* pairs_dev,
                        size_t npairs, size_t d, size_t k, float* norms, void* csplit,
                        uint32_t* cpart, bool f16);
void launch_gather_rows(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                        size_t m, float* out);

// ---- emh_scatter.hip
void launch_scatter(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids, size_t lo,
                    size_t hi, const uint32_t* labels, size_t k, float* sums, uint32_t* counts,
                    float* acc);
// The same in two halves: counts (and the cluster offsets), then the ordered
// sums; the caller may queue work that needs only the counts in between.
// counts_zero: counts holds zeros on entry (launch_ema with zero_counts left
// them so), which saves a fill.
void launch_scatter_count(emh_ctx* c, size_t lo, size_t hi, const uint32_t* labels, size_t k,
                          uint32_t* counts, bool counts_zero = false);
// counts_tallied: the labels' counts and chunk histograms come from the
// top-1 call that wrote them (LabelTally with cnt = tally_cnt, stride =
// tally_stride), and
// launch_scatter_count was not called; the placement then scans the counts
// itself. Needs scatter_tallied(hi - lo, k).
void launch_scatter_sums(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                         size_t lo, size_t hi, const uint32_t* labels, size_t k, float* sums,
                         float* acc, const uint32_t* counts_tallied = nullptr,
                         const uint32_t* tally_cnt = nullptr, size_t tally_stride = 0);

// Training runs of at most this many rows queue their host<->device copies
// on the context stream instead of the copy stream.
constexpr size_t ONE_STREAM_ROWS = 65536;

// ---- emh_update.hip: a small training batch's scatter_add and EMA step in one
// launch (the same bits as launch_scatter_sums then launch_ema).
constexpr size_t UPDATE_SMALL_BATCH = 256;  // most positions per batch
constexpr size_t UPDATE_SMALL_MAX_D = 1024;
// Whether a batch of n positions with d dimensions takes it.
bool update_small(size_t n, size_t d, bool spherical);
// Labels lo .. hi tallied into counts (and tcnt, ntcnt words) by the batch's
// top-1 call. As launch_scatter_sums (tallied) then launch_ema with
// clear_screen_words and zero_counts: moves the centroids that got rows
// (pos, usage; norms and, with csplit, the halves for L2 runs, fp16 with f16;
// readout
// for spherical ones), adds the sums into acc (when given) and counts into
// tally, and leaves counts and tcnt at zero. With csplit, cpart[2 j] =
// cpart[2 j + 1] = norms[j] bits for every cluster j (k pairs).
void launch_update_small(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                         size_t lo, size_t hi, const uint32_t* labels, size_t k, uint32_t* counts,
                         uint32_t* tcnt, size_t ntcnt, float* acc, float* pos, float* usage,
                         float alpha, float decay, int replace, float* norms, void* csplit,
                         uint32_t* cpart, float* readout, uint32_t* tally, bool f16);

// ---- emh_autok.hip (kmeans_pp and internal_scores of the automatic-k callers)
// best[i] = max(best[i], dot(x[i], x[last])), the dot in sequence without fma.
void launch_pp_best(emh_ctx* c, const float* x, size_t n, size_t d, size_t last, float* best);
// sums[s][t] = f64 sum over rows rid[start[s] .. start[s + 1]) of x[row][t], in order.
void launch_sum64(emh_ctx* c, const float* x, size_t d, const uint32_t* rid,
                  const uint32_t* start, size_t ke, double* sums);
// g[i][s] = fma chain of x[i] . sums32[s] (i < n, s < ke); xx[i] = f64 sum of squares.
void launch_row_dots(emh_ctx* c, const float* x, size_t n, size_t d, const float* sums32,
                     size_t ke, float* g, double* xx);
// Per-row silhouette, objective and distance terms (metrics.rs:158-184).
void launch_iscore_terms(emh_ctx* c, size_t n, size_t ke, const float* g, const double* xx,
                         const uint32_t* own, const double* size, const double* sq, double* sil,
                         double* obj, double* dist);

// ---- emh_screen.hip (top-1 and top-k orchestration)
// words_clear: the caller zeroed the screen's small-block words since the
// last top-1 (launch_ema with clear_screen_words), so the fill is skipped.
// ar: take the per-call scratch from this fixed block instead of the
// context's buffers (no allocation; the call is not profiled).
// Rows split into bf16 halves ahead of the calls (launch_halves over all nx
// rows of x, slab-major with slab stride `slab` bytes), with their |x|^2:
// the screen gathers them by id instead of splitting each call's selection.
struct SplitRows {
  const void* xs;
  const float* xn;
  size_t nx, slab;
  bool f16 = false;  // fp16 halves (else bf16; emh_halves.h)
};
// Positions per chunk of scatter_add's chunked counting sort.
constexpr int TALLY_CP = 256;
// The labels a top-1 call writes, tallied for the scatter_add of the same
// positions that follows it (launch_scatter_sums with tallied): for each
// labelled position p, cnt[label stride + (p - lo) / TALLY_CP] and
// counts[label] grow by one (label-major chunk histograms: a label's chunks
// are contiguous, stride = tally_stride(positions)). Both must be zero on
// entry (launch_ema clears them), and every position must get a label (ids
// in range).
struct LabelTally {
  uint32_t* cnt;
  uint32_t* counts;
  size_t lo, stride;
};
// Whether a scatter_add of n positions with k labels can take tallied labels
// (the chunked path), and its chunk count.
bool scatter_tallied(size_t n, size_t k);
inline size_t scatter_chunks(size_t n) { return (n + TALLY_CP - 1) / TALLY_CP; }
inline size_t tally_stride(size_t n) { return (scatter_chunks(n) + 3) & ~(size_t)3; }
// Centroids split ahead of the call (launch_halves over the k centroids, or
// launch_ema's csplit for the rows it moved), with the bound's centroid
// maxima in nparts (max |c|^2, max cnorm) pairs.
struct SplitCents {
  const void* cs;
  const uint32_t* part;
  int nparts;
  bool f16 = false;  // fp16 halves (else bf16)
};
// pre: x's rows already split, pc: the centroids (used when the call takes
// the split-operand screen; see split_screen).
// tally: tally the labels (see LabelTally; the call must screen with d % 4 ==
// 0, where the check and the queued-row scan write every label: a tallied call
// screens also when its rows are fewer than the context's exact_below).
void launch_top1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids, size_t lo, size_t hi,
                 const float* cents, const float* cnorm, size_t k, bool ip, uint32_t* labels,
                 float* scores, bool words_clear = false, Arena* ar = nullptr,
                 const SplitRows* pre = nullptr, const SplitCents* pc = nullptr,
                 const LabelTally* tally = nullptr);
// Whether top-1 calls of n rows with d dimensions and k centroids take the
// split-operand screen (k_screen4), whose rows a caller may split ahead.
bool split_screen(emh_ctx* c, size_t n, size_t d, size_t k, bool ip);
// Whether top-1 calls of n rows with d dimensions and k centroids run a
// screen (and so the check and the queued-row scan). A tallied call always
// does, whatever its rows.
bool top1_screens(emh_ctx* c, size_t n, size_t d, size_t k, bool ip);
// Whether a top-1 call of n rows (and of any fewer) can tally the labels it
// writes: the screen with d % 4 == 0, or the latency-bound exact scan.
bool top1_tallies(emh_ctx* c, size_t n, size_t d, size_t k, bool ip);
// Split rows of x (n rows, or ids[lo..lo+n)) into halves in out (fp16 with
// f16, else bf16; emh_halves.h), slab-major, with their |x|^2 in norm; with
// part, each of the
// halves_blocks(n) blocks leaves the largest |x|^2 of its rows and the
// largest cnorm in part[2 b], part[2 b + 1] (emh_screen4.hip). Bytes of out:
// halves_bytes(n, d).
void launch_halves(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids, size_t lo,
                   size_t n, void* out, float* norm, const float* cnorm, uint32_t* part,
                   bool f16 = false);
inline size_t halves_bytes(size_t n, size_t d) { return n * ((d + 31) / 32) * 128; }
inline size_t halves_blocks(size_t n) { return (n + 7) / 8; }
// out[0], out[1] = the largest part[2 i], part[2 i + 1] over i < nparts (f32
// bits as u32), for a screen whose blocks would otherwise each read more than
// PART_MAX_ONCE partials.
constexpr size_t PART_MAX_ONCE = 1024;
void launch_part_max(emh_ctx* c, const uint32_t* part, size_t nparts, uint32_t* out);
// Bytes of fixed-block scratch launch_top1 takes for a call of n rows (an
// upper bound: each region rounded up to 256 bytes).
size_t top1_scratch_bytes(emh_ctx* c, size_t n, size_t d, size_t k, bool ip);

// With rep, the screen runs and its lists are measured (launch_margin) instead
// of checked: nothing is written to ids or sims.
void launch_topk(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                 size_t kk, bool exclude_self, uint32_t* ids, float* sims,
                 emh_screen_report* rep = nullptr);
// Exact top-k for 16 < kk <= KLONG (emh_topk_long.hip): no screen.
constexpr int KLONG = 4096;
void launch_topk_long(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                      size_t kk, bool exclude_self, uint32_t* ids, float* sims);
// The screen stage of a top-1 call, its lists measured instead of checked.
void screen_margin_top1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                        size_t lo, size_t hi, const float* cents, const float* cnorm, size_t k,
                        bool ip, emh_screen_report* out);

}  // namespace emh
