/* emeans_hip.h -- C ABI of the MI355X (gfx950) backend of emeans.
 *
 * Layer 1 of the reference is the `Device` trait
 * (crates/emeans-core/src/core/mod.rs:71-178): buffers that live on the
 * backend plus the ops of one e-means batch. Each `emh_*` entry point below
 * replaces one method of that trait, or one caller that the reference writes
 * generically over it, and cites the line it replaces. A Rust shim crate binds
 * these with `extern "C"` and implements `Device` + `Assigner` on top.
 *
 * Conventions (the reference's FFI rules, crates/emeans-ffi/src/lib.rs:26-140):
 *  - every call returns EMH_OK (0), EMH_INVALID (1, bad argument) or EMH_ERROR (2);
 *  - on failure nothing is written to the out-parameters and a message for the
 *    calling thread is available from emh_last_error();
 *  - no C++ exception crosses the ABI.
 * Threading: one emh_ctx is one HIP stream on one device and is not thread-safe;
 * the caller serializes calls on a context (the Rust shim holds `&mut`).
 * Ordering: ops are queued on the context's stream; only emh_read_* and
 * emh_sync wait for the device (core/mod.rs:70).
 */
#ifndef EMEANS_HIP_H
#define EMEANS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EMH_OK 0
#define EMH_INVALID 1
#define EMH_ERROR 2

/* Metric (crates/emeans-core/src/assign.rs:14-21). */
#define EMH_L2 0
#define EMH_IP 1

typedef struct emh_ctx emh_ctx;
/* A device buffer of f32 or u32 (Device::F / Device::U). */
typedef struct emh_buf emh_buf;

/* Message of the last failed call on this thread (emeans-ffi/src/lib.rs:95-140). */
const char* emh_last_error(void);

/* ------------------------------------------------------------------ context */
/* Backend construction: make_assigner(Backend::Custom{"hip"}) -> the engine
 * (emeans-cluster/src/backend.rs:170-178; the CUDA analogue is CudaCore::new,
 * emeans-cuda/src/lib.rs:302-503). Fails with EMH_ERROR when there is no
 * gfx950 device. */
int emh_create(int device, emh_ctx** out);
int emh_destroy(emh_ctx* ctx);
/* Device::name (core/mod.rs:77): "hip-gfx950". */
const char* emh_name(const emh_ctx* ctx);
/* Device::flush (core/mod.rs:93). */
int emh_flush(emh_ctx* ctx);
/* Wait for all queued work (the wait half of Device::read_*). */
int emh_sync(emh_ctx* ctx);
/* The HIP stream the context queues on (hipStream_t), for interop. */
void* emh_stream(emh_ctx* ctx);

/* ------------------------------------------------------------------ buffers */
/* Device::bind (core/mod.rs:81): copy the data set x (len floats) to the device.
 * Always copies (assign.rs:75-83). */
int emh_bind(emh_ctx* ctx, const float* x, size_t len, emh_buf** out);
/* Device::upload_f32 / upload_u32 (core/mod.rs:82-83). */
int emh_upload_f32(emh_ctx* ctx, const float* v, size_t len, emh_buf** out);
int emh_upload_u32(emh_ctx* ctx, const uint32_t* v, size_t len, emh_buf** out);
/* Device::zeros_f32 / zeros_u32 (core/mod.rs:84-85). */
int emh_zeros_f32(emh_ctx* ctx, size_t len, emh_buf** out);
int emh_zeros_u32(emh_ctx* ctx, size_t len, emh_buf** out);
/* Device::write_f32 / write_u32 (core/mod.rs:86-88): b[offset..offset+len] = v,
 * after queued work that uses b. */
int emh_write_f32(emh_ctx* ctx, emh_buf* b, size_t offset, const float* v, size_t len);
int emh_write_u32(emh_ctx* ctx, emh_buf* b, size_t offset, const uint32_t* v, size_t len);
/* Device::read_f32 / read_u32 (core/mod.rs:89-91): wait, then copy b[lo..hi). */
int emh_read_f32(emh_ctx* ctx, const emh_buf* b, size_t lo, size_t hi, float* dst);
int emh_read_u32(emh_ctx* ctx, const emh_buf* b, size_t lo, size_t hi, uint32_t* dst);
/* Drop of the backend's buffer type. Waits for ctx's queued work first. A
 * block of at most 64 MB is kept for the next buffer of the same size on the
 * device (at most 1 GB a device, released with the device's last context), and
 * the context that takes it waits on the device for the work the other
 * contexts had queued when it was freed; a buffer whose address went out
 * (emh_buf_ptr) is freed at once. The handle is gone after the call, also
 * when it fails. */
int emh_free(emh_ctx* ctx, emh_buf* b);
/* A non-owning view of caller device memory (for example a torch tensor) as a
 * buffer; freeing the view does not free the memory. kind: 0 f32, 1 u32. */
int emh_wrap(emh_ctx* ctx, void* dev_ptr, size_t len, int kind, emh_buf** out);
void* emh_buf_ptr(const emh_buf* b);
size_t emh_buf_len(const emh_buf* b);

/* --------------------------------------------------------------------- ops */
/* Device::top1 (core/mod.rs:97-112): for every selected position p in
 * [lo, hi), row x[ids[p]] (ids != NULL) or x[p]; labels[p] = nearest of the k
 * centroids (largest inner product, or smallest squared L2), ties to the lower
 * id; scores[p] its score. cnorm (squared centroid norms) is required for L2.
 * Only positions in [lo, hi) are written. Labels and scores equal the
 * reference CPU backend's (cpu-fused, assign/fused.rs) bit for bit. */
int emh_top1(emh_ctx* ctx, const emh_buf* x, size_t d, const emh_buf* ids, size_t lo, size_t hi,
             const emh_buf* centroids, const emh_buf* cnorm, size_t k, int metric,
             emh_buf* labels, emh_buf* scores);

/* emh_top1 that allocates nothing. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, checks and results (the same bits) as emh_top1; the per-call
 * scratch (screen candidate lists, the queue of rows for the exact scan, row
 * norms, queue words) comes from one fixed 32 MiB block of device memory per
 * GPU, held until the process ends. The screened path (k >= 2, d >= 32)
 * takes 40 bytes per row per centroid part (1 to 8 parts, fewer as the call
 * has more rows) plus about 21 bytes per row: some 500,000 rows per call at
 * d % 4 == 0; with d % 4 != 0, or without the screen, 8 ceil(k / 64) bytes
 * per row more. A call whose scratch would exceed the block fails with
 * EMH_INVALID before anything is queued.
 * Every call on a GPU shares that GPU's block, which keeps the last call's
 * contents. Calls from different streams or contexts on one GPU run one
 * after another: each call's stream waits for the previous call's work
 * (an event per GPU, recorded at the end of each call). A stream under HIP
 * graph capture takes no part in that ordering: calls captured into graphs
 * that run at once on one GPU race, so the caller orders such graphs. The
 * call is not timed by emh_profile. */
int emh_top1_noalloc(emh_ctx* ctx, const emh_buf* x, size_t d, const emh_buf* ids, size_t lo,
                     size_t hi, const emh_buf* centroids, const emh_buf* cnorm, size_t k,
                     int metric, emh_buf* labels, emh_buf* scores);

/* Device::topk (core/mod.rs:114-124): best kk data rows per query by inner
 * product, best first (larger score, then lower id); with exclude_self query
 * i is data row i and is skipped; missing: id 0xFFFFFFFF, score -inf.
 * kk <= 16 (GPU_KMAX, emeans-core/src/knn.rs:16) runs the MFMA screen; for
 * 16 < kk <= 4096, where the reference's knn (emeans-cluster/src/knn.rs:42)
 * turns to its CPU search (core/src/knn.rs:53-107), an exact search on the
 * GPU with the same results; larger kk fails with EMH_INVALID.
 * Host pointers in and out (the reference signature). */
int emh_topk(emh_ctx* ctx, const float* queries, size_t m, const float* data, size_t n, size_t d,
             size_t kk, int exclude_self, uint32_t* ids, float* sims);
/* The same on device buffers (queries/data resident; ids/sims m*kk). */
int emh_topk_dev(emh_ctx* ctx, const emh_buf* queries, size_t m, const emh_buf* data, size_t n,
                 size_t d, size_t kk, int exclude_self, emh_buf* ids, emh_buf* sims);

/* Device::scatter_add (core/mod.rs:126-139): counts[j] = selected rows with
 * label j, sums[j] = those rows added in selection order in f32 (bit-equal to
 * the CPU's row-order sums); both overwritten; acc += sums when acc != NULL.
 * labels are read at the selection positions. */
int emh_scatter_add(emh_ctx* ctx, const emh_buf* x, size_t d, const emh_buf* ids, size_t lo,
                    size_t hi, const emh_buf* labels, size_t k, emh_buf* sums, emh_buf* counts,
                    emh_buf* acc);

/* Device::row_norms (core/mod.rs:141-142): sequential f32 sum of squares. */
int emh_row_norms(emh_ctx* ctx, const emh_buf* m, size_t rows, size_t d, emh_buf* out);

/* Device::normalize_rows (core/mod.rs:144-151): faiss normalize_into. */
int emh_normalize_rows(emh_ctx* ctx, const emh_buf* src, size_t rows, size_t d, emh_buf* dst);

/* Device::split (core/mod.rs:153-162): apply a revival plan of npairs
 * (donor, dead) pairs given as 2*npairs u32 (host memory); bit-equal to
 * apply_splits (core/mod.rs:374-399). usage has k = emh_buf_len(usage) floats. */
int emh_split(emh_ctx* ctx, emh_buf* positions, emh_buf* usage, const uint32_t* pairs,
              size_t npairs, size_t d);

/* Device::ema_update (core/mod.rs:164-177) with EmaStep (core/mod.rs:182-197):
 * alpha = (float)alpha64, decay = (float)(1 - alpha64), replace = alpha64 == 1. */
int emh_ema_update(emh_ctx* ctx, emh_buf* positions, emh_buf* usage, const emh_buf* sums,
                   const emh_buf* counts, size_t k, size_t d, float alpha, float decay,
                   int replace);

/* ----------------------------------------------- layer 2 and its callers */
/* Config (crates/emeans-core/src/model.rs:24-76). Zero/negative "has_*" means None. */
typedef struct emh_config {
  uint64_t k, d;
  double nepochs;               /* 5.0 */
  uint64_t batch_size;          /* 0 = batch law */
  int has_alpha0;
  double alpha0;
  int batch_law;                /* 0 auto, 1 throughput, 2 quality */
  uint32_t seed;                /* 1234 */
  int spherical;
  int has_unused_threshold;
  double unused_threshold;
  uint64_t assignment_chunk_size; /* 0 = 65536 */
  int capture_assignments;
  int verbose;
} emh_config;

/* Per-epoch statistics (EpochStats, model.rs:80-89). */
typedef struct emh_epoch_stats {
  double obj;
  double time;
  double imbalance_factor;
  uint64_t nsplit;
} emh_epoch_stats;

/* Results of one training run; arrays are caller-allocated: centroids,
 * positions k*d, usage k, labels n (may be NULL), stats capacity max_epochs. */
typedef struct emh_train_out {
  float* centroids;
  float* positions;
  float* usage;
  int32_t* labels;
  emh_epoch_stats* stats;
  uint64_t max_epochs;
  uint64_t n_epochs;
  uint64_t n_splits;
  uint64_t batch_size;
  double alpha0;
  uint64_t total_steps;
  uint64_t fallback_rows; /* rows the exact top-1 kernel rescanned (screen misses) */
  emh_buf* centroids_dev; /* optional: the centroids also land in this k*d f32 buffer */
} emh_train_out;

/* The start of a training run (the Job's positions and usage,
 * core/train.rs:33-58). All NULL: k sampled rows (Emeans::train,
 * model.rs:786-797). centroids or centroids_dev (k x d, host or device): given
 * initial centroids, normalized when spherical, masses 2^-16 (train_from ->
 * begin, model.rs:705-736, 306-316). positions (k x d) with usage (k), host:
 * saved EMA state taken as it is (train_resume -> begin_with_state,
 * model.rs:739-749, 318-336); masses must be finite and >= 0. Initial
 * centroids and positions must be finite. */
typedef struct emh_train_init {
  const float* centroids;
  const emh_buf* centroids_dev;
  const float* positions;
  const float* usage;
} emh_train_init;

/* Emeans::train / train_from / train_resume (model.rs:700-811) driving the
 * device loop core::train::run (core/train.rs:60-303) on this context: the
 * start given by init (NULL: sampled centroids), the seeded epoch
 * permutations and revival draws on the host, every batch op on the device.
 * x is n*d host floats, copied to the device once. */
int emh_train(emh_ctx* ctx, const float* x, size_t n, const emh_config* cfg,
              const emh_train_init* init, emh_train_out* out);
/* The same with the data already on the device (x: n*d f32 buffer). */
int emh_train_dev(emh_ctx* ctx, const emh_buf* x, size_t n, const emh_config* cfg,
                  const emh_train_init* init, emh_train_out* out);

/* Emeans::assign (model.rs:898-919) -> assign_all (assign.rs:785-809) ->
 * assign_on (core/mod.rs:249-330) on this context: labels/scores of every row
 * of x (n*d host floats) against k centroids. chunk = rows per call (0 = 65536). */
int emh_assign(emh_ctx* ctx, const float* x, size_t n, size_t d, const float* centroids,
               size_t k, int metric, size_t chunk, uint32_t* labels, float* scores);

/* assign_on with everything resident on the device: labels/scores (n entries)
 * of the n rows of x against k centroids (k*d f32 buffer), in chunks of
 * `chunk` rows (0 = 65536); L2 centroid norms are computed on the device
 * (row_norms, as assign_on does, core/mod.rs:265-272). */
int emh_assign_dev(emh_ctx* ctx, const emh_buf* x, size_t n, size_t d, const emh_buf* centroids,
                   size_t k, int metric, size_t chunk, emh_buf* labels, emh_buf* scores);

/* knn_self / knn (emeans-cluster/src/knn.rs:17-64) on this context. */
int emh_knn(emh_ctx* ctx, const float* queries, size_t m, const float* data, size_t n, size_t d,
            size_t kk, int exclude_self, uint32_t* ids, float* sims);

/* DedupConfig (emeans-cluster/src/dedup.rs:39-62). */
typedef struct emh_dedup_config {
  uint64_t k;                /* neighbours searched per row (10) */
  float sim_threshold;       /* cosine that links two rows (0.95) */
  int has_rep_threshold;     /* 0: rep_threshold = sim_threshold */
  float rep_threshold;       /* cosine to the star's anchor needed to join it */
  int has_max_gap_secs;      /* 0: similarity alone decides */
  double max_gap_secs;       /* largest time gap of a link when both rows have a time */
} emh_dedup_config;

/* DedupInput (dedup.rs:65-76): optional per-row side information; each
 * pointer is NULL or has n entries. */
typedef struct emh_dedup_input {
  const double* created_unix; /* creation time (s); NaN = unknown */
  const int64_t* burst;       /* burst id (the caller's interned id); < 0 = none */
  const float* priority;      /* representative preference, higher wins; no NaN */
} emh_dedup_input;

/* DedupResult (dedup.rs:79-102): caller-allocated arrays, group_of and
 * nn_sim with n entries (nn_sim may be NULL), representatives, anchors and
 * sizes with capacity n; the counts are written by the call. */
typedef struct emh_dedup_result {
  uint32_t* group_of;
  uint32_t* representatives;
  uint32_t* anchors;
  uint32_t* sizes;
  float* nn_sim;
  uint64_t n_groups;
  uint64_t linked_pairs;
  uint64_t split_components;
} emh_dedup_result;

/* dedup_with_neighbors (dedup.rs:186-358) on the host: links (cosine >=
 * sim_threshold and, when both rows have a time and max_gap_secs is set,
 * |t_i - t_j| <= max_gap_secs), burst units (rows of one burst id always in one
 * group), union-find components, the star cover (a burst joins an anchor only
 * when every one of its rows fits; the anchor's own burst is exempt) and the
 * representatives. nb_ids / nb_sims: kk neighbours per row, as knn_self gives. */
int emh_dedup_neighbors(const float* x, size_t n, size_t d, const uint32_t* nb_ids,
                        const float* nb_sims, size_t kk, const emh_dedup_input* input,
                        const emh_dedup_config* cfg, emh_dedup_result* out);

/* dedup (dedup.rs:163-183): knn_self with k = min(cfg->k, n - 1) (at least 1)
 * on this context, then the host groups. The GPU keeps at most 16 neighbours. */
int emh_dedup(emh_ctx* ctx, const float* x, size_t n, size_t d, const emh_dedup_input* input,
              const emh_dedup_config* cfg, emh_dedup_result* out);

/* --------------------------------------------- the automatic-k callers */
/* kmeans_pp (emeans-cluster/src/auto.rs:401-455): k-means++ seeding with the
 * cosine distance 1 - x.y on the rows of x (n x d f32 buffer, unit rows):
 * min(kmax, n) row ids in pick order (picks has kmax entries), the same as the
 * reference's for the same seed. */
int emh_kmeans_pp(emh_ctx* ctx, const emh_buf* x, size_t n, size_t d, size_t kmax,
                  uint32_t seed, uint32_t* picks, size_t* n_picks);

/* Internal (emeans-cluster/src/metrics.rs:95-111). */
typedef struct emh_internal {
  uint64_t k_eff;             /* non-empty clusters */
  double silhouette;          /* mean cosine-distance silhouette */
  double calinski_harabasz;
  double davies_bouldin;
  double objective;           /* mean 2 - 2 cos to the normalized cluster mean */
} emh_internal;
/* internal_scores (metrics.rs:113-268) of labels (n entries < k, u32
 * buffer) on the unit rows of x (n x d f32 buffer); sizes (k, may be NULL)
 * gets the rows per label. The reference takes the row-by-cluster-sum dots
 * from the gemm crate; here each is one fma chain over the columns in order
 * (the scores agree with scikit-learn's within the reference's 1e-5). */
int emh_internal_scores(emh_ctx* ctx, const emh_buf* x, size_t n, size_t d, const emh_buf* labels,
                        size_t k, emh_internal* out, uint64_t* sizes);

/* gemm_nt (emeans-core/src/assign.rs:813-825) as Hierarchy::grow calls it
 * (emeans-cluster/src/incremental.rs:423-440): out[i * nb + j] = a_i . b_j for
 * a (m x d f32 buffer) and b (nb x d f32 buffer) into out (f32 buffer of at
 * least m * nb entries). Each dot is one fma chain over the columns in order;
 * the reference's gemm-crate order is not reproduced (its callers compare
 * dots with thresholds). Queued; read out to wait. */
int emh_dots(emh_ctx* ctx, const emh_buf* a, size_t m, const emh_buf* b, size_t nb, size_t d,
             emh_buf* out);

/* ------------------------------------------------- host replay (no device) */
/* The seeded host-side pieces of the device loop, exported so that callers and
 * tests can check them without a GPU. They never touch the device. */
/* RandomState::new(seed).permutation(n) (crates/emeans-core/src/rng.rs:19,95):
 * numpy-legacy MT19937 shuffle; out has n entries. */
void emh_host_permutation(uint32_t seed, uint64_t n, uint32_t* out);
/* The (skip+1)-th RandomState::random_sample() of a fresh RandomState::new(seed)
 * (rng.rs:63). */
double emh_host_random_sample(uint32_t seed, uint64_t skip);
/* Recipe::resolve (recipe.rs:200-254) for n rows: batch size, alpha0, rows of
 * each epoch (first `cap` written to epoch_rows), epoch count, total steps. */
int emh_host_recipe(uint64_t n, const emh_config* cfg, uint64_t* batch_size, double* alpha0,
                    uint64_t* epoch_rows, uint64_t cap, uint64_t* n_epochs, uint64_t* total);
/* scheduled_alpha (recipe.rs:148-152): the cosine schedule in f64. */
double emh_host_scheduled_alpha(double alpha0, uint64_t step, uint64_t total);
/* plan_revival (core/mod.rs:339-370) with a fresh RandomState::new(seed):
 * (donor, dead) pairs written to pairs (capacity 2k); returns the pair count. */
uint64_t emh_host_plan_revival(const float* usage, uint64_t k, double tau, uint32_t seed,
                               uint32_t* pairs);
/* numpy_sum_f32 (model.rs:970-1002): numpy's pairwise f32 sum. */
float emh_host_numpy_sum_f32(const float* a, uint64_t n);

/* ------------------------------------------------------------ diagnostics */
/* Which screen a top-1 or top-k call ran (emh_screen_report.variant). */
#define EMH_SCREEN_NONE 0        /* no screen: k < 2, d < 32 or emh_set_screen(ctx, 0) */
#define EMH_SCREEN_BIG_TAGGED 1  /* large-tile bf16 screen, one tile per part, tagged keys */
#define EMH_SCREEN_BIG_SORTED 2  /* large-tile bf16 screen, several tiles per part */
#define EMH_SCREEN_SMALL_BF16 3  /* 128 x 128 bf16 screen (d % 4 != 0, and small kNN calls) */
#define EMH_SCREEN_SMALL_F32 4   /* 128 x 128 f32 screen (emh_set_screen(ctx, 2)) */
#define EMH_SCREEN_BIG_KNN 5     /* kNN: 128 x 256 bf16 screen over operands split once */
#define EMH_SCREEN_BIG_F16 6     /* large-tile fp16 two-pass screen, one tile per part, tagged keys */
typedef struct emh_screen_report {
  int variant;          /* EMH_SCREEN_* */
  int parts;            /* centroid (or data row) parts per row tile */
  int tiles_per_part;
  uint64_t pairs;       /* list entries re-scored */
  uint64_t over;        /* entries whose |screen key - exact key| exceeded the bound E */
  double max_ratio;     /* max |screen key - exact key| / E over the entries */
  double max_dot_ratio; /* max dot error / the bound's dot term (split + MFMA model), after
                           the allowances that are IEEE rounding of the keys or the tag */
} emh_screen_report;
/* Diagnostics of the screen's exactness argument (no counterpart in the
 * reference): run the screen of emh_top1 (or of emh_topk_dev) on the same
 * arguments, then re-score every entry of its candidate lists with the exact
 * fma-chain key the check uses and report how far the screen's key was from
 * it, relative to the per-row bound E the check trusts. Writes no labels,
 * scores, ids or sims; waits for the device. */
int emh_screen_margin(emh_ctx* ctx, const emh_buf* x, size_t d, const emh_buf* ids, size_t lo,
                      size_t hi, const emh_buf* centroids, const emh_buf* cnorm, size_t k,
                      int metric, emh_screen_report* out);
int emh_screen_margin_topk(emh_ctx* ctx, const emh_buf* queries, size_t m, const emh_buf* data,
                           size_t n, size_t d, int exclude_self, emh_screen_report* out);
/* Rows the exact top-1 / top-k kernels rescanned since the context was made
 * (the screen's misses; EMEANS_CUDA_SCREEN_STATS analogue, emeans-cuda lib.rs:278-287). */
uint64_t emh_fallback_rows(emh_ctx* ctx);
/* Select the top-1 / top-k path: 1 = MFMA screen in bf16 three-pass arithmetic
 * + exact check (default), 3 = the same with the split-operand top-1 screen
 * (k_screen4) in fp16 two-pass arithmetic (a third fewer MFMAs, a bound 2.7
 * times looser at d = 768; rows or centroids beyond |x| = 32768 take the exact
 * scan), 2 = MFMA screen in f32 arithmetic + exact check, 0 = exact kernels
 * only (the reference "FP32 kernel alone", emeans-cuda tests/contract.rs:27-37).
 * Results are the same bits in every mode. */
int emh_set_screen(emh_ctx* ctx, int on);
/* Top-1 calls of at most `items` exact items (rows x max(ceil(k / 64), 2))
 * run the exact kernels alone even when the mode screens (default 4096: there
 * one exact launch takes less time than the screen's three); 0 screens every
 * call the mode screens and keeps the exact scan of a call without the screen
 * on its throughput kernel. A training run decides once, by its batch size.
 * Results are the same bits either way. No reference counterpart (a
 * performance knob of this backend, like emh_set_screen). */
int emh_set_exact_below(emh_ctx* ctx, uint64_t items);
/* Ops that emh_profile times. */
#define EMH_PROF_SCREEN 0  /* the MFMA screen kernel of top-1 and top-k; units: 2 rows k d FLOP */
#define EMH_PROF_SCATTER 1 /* scatter_add (count and ordered-sum launches); units: HBM bytes */
#define EMH_PROF_EMA 2     /* ema_update; units: HBM bytes */
#define EMH_PROF_OPS 3
/* Time every on-th instance of each op above with HIP events on the
 * context's stream (0: off; 1: every instance; a larger period keeps the
 * events' own cost out of the timed work). No counterpart in the reference,
 * whose CUDA backend is profiled externally (.okf/results/cuda-kernels.md);
 * emh_profile_read_op waits, then returns and resets op's totals: milliseconds,
 * instances timed, and the algorithmic units they cover (FLOP for the
 * screen; bytes per the formulas rows d 4 + rows 4 (labels) [+ rows 4 (ids)]
 * + k d 4 + k 4 [+ 2 k d 4 (acc)] for scatter_add and 3 k d 4 + 4 k 4 for
 * ema_update). emh_profile_read is emh_profile_read_op for the screen. */
int emh_profile(emh_ctx* ctx, int on);
/* The same for one op (EMH_PROF_*), the others unchanged. */
int emh_profile_op(emh_ctx* ctx, int op, int on);
int emh_profile_read_op(emh_ctx* ctx, int op, double* ms, uint64_t* instances, double* units);
int emh_profile_read(emh_ctx* ctx, double* ms, uint64_t* launches, double* flop);

#ifdef __cplusplus
}
#endif
#endif /* EMEANS_HIP_H */
