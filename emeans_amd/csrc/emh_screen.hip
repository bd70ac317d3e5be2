// Fused top-1 (Device::top1, core/mod.rs:97-112) and exact top-k
// (Device::topk, core/mod.rs:114-124) for gfx950: the MFMA screen and the
// orchestration of the check (emh_rescore.hip) and exact scans (emh_verify.hip).
//
// Exactness: the reference CPU backend (cpu-fused, assign/fused.rs) scores
// every (row, centroid) pair with one sequential f32 fma chain over the d
// dimensions. The screen computes the same dot products on the bf16 MFMA in
// three passes (x.c ~ xh.ch + xh.cl + xl.ch, the halves rounded to nearest
// even, f32 accumulation), so its scores differ from the chain's by about
// 2^-16 |x| |c| plus the accumulation's rounding. The path therefore has three
// stages:
//
//  1. screen (MFMA, the dense x . C^T contraction): per part (a range of
//     centroid tiles) each row keeps the L smallest screen keys (key = -dot
//     for IP, |c|^2 - 2 dot for L2) with their ids, in registers; the n x k
//     score matrix never leaves the CU.
//  2. check: bound the screen error E rigorously from |x| and max|c|. A
//     part's list holds every centroid of the part whose screen key is at
//     most best + 2E when the list is not full or its L-th key is above
//     best + 2E; with every part so, the centroids that can win are among
//     the lists' entries within best + 2E: re-score exactly those (at most
//     C1) with the fma chain and take the smallest exact key, lower id on
//     ties. Otherwise queue the row.
//  3. exact: the full fma-chain scan of the queued rows over all k centroids.
//
// The same stages with a longer list, merged over the parts, give the exact
// top-k of kNN.
//
// Bound (screen_bound, emh_select.h): the chain is within gamma_d sum|x_t c_t|
// of the exact dot (gamma_d = d u / (1 - d u), u = 2^-24) and sum|x_t c_t| <=
// |x| |c|; the screen adds the split's dropped and rounded parts
// (<= 3.05 * 2^-16 |x| |c|) and the MFMA chain's rounding (each MFMA within
// 16 u of its terms' magnitudes); L2 keys add the rounding of |c|^2 - 2 dot
// on both sides (one rounding in the screen's fma, two in the check's). E
// carries a 12.5% margin for its own rounding.

#include "emh_screen_kern.h"

namespace emh {
namespace {

// The 128 x 128 screens in the context's arithmetic (f32 in SCREEN_F32, else bf16).
void launch_screen_t1(emh_ctx* c, const ScreenArgs& a, bool ip) {
  if (c->screen == SCREEN_F32)
    launch_screen_t1_f32(c, a, ip);
  else
    launch_screen_t1_bf3(c, a, ip);
}
void launch_screen_kn(emh_ctx* c, const ScreenArgs& a, bool exclude_self) {
  if (c->screen == SCREEN_F32)
    exclude_self ? launch_screen_kn_f32_self(c, a) : launch_screen_kn_f32_any(c, a);
  else
    exclude_self ? launch_screen_kn_bf3_self(c, a) : launch_screen_kn_bf3_any(c, a);
}

int choose_parts(int row_tiles, int ntiles, int cus, int per_cu = 2) {
  // Enough blocks for per_cu per CU (all resident at once), never more parts
  // than tiles, and at most MAX_PARTS lists per row for the verify to merge.
  int want = (per_cu * cus + row_tiles - 1) / row_tiles;
  return std::max(1, std::min(std::min(want, ntiles), MAX_PARTS));
}

}  // namespace

namespace {
// The screen's launch geometry for n rows against k centroids. split: the
// call may take the split-operand screen (k_screen4: fp16 or bf16, k >= 64
// and at most MAX_PARTS tiles of 256 centroids, one tile per part with
// tagged keys; any d >= 32). Otherwise (and for the no-allocation entry, which
// has no room to split a selection) the large-tile screen that splits its
// slabs itself (k_screen3, d % 4 == 0, k >= 64) or the 128 x 128 screens.
struct Top1Geom {
  bool screen, big, split;
  int row_tiles, ntiles, parts, tpp;
};
Top1Geom top1_geom(emh_ctx* c, size_t n, size_t d, size_t k, bool ip, bool split,
                   bool small_exact) {
  Top1Geom g{};
  // The screen for any k >= 2 with d >= 32: below that, and for k = 1, the
  // exact scan is as fast. (At small k the exact scan's items leave most
  // lanes idle: 900,000 rows against 40 centroids took 10x the screen's time.)
  // With small_exact, calls of at most c->exact_below exact items, or small
  // enough for the latency-bound scan, take the exact kernels too: one launch
  // beats the screen's three there.
  g.screen = c->screen && k >= 2 && d >= 32 &&
             !(small_exact && (exact_items(n, k) <= c->exact_below ||
                               queued_direct(c, n, d, k, ip)));
  if (!g.screen) return g;
  const int nt3 = (int)((k + TC3 - 1) / TC3);
  // (k_screen4 addresses a slab's rows with 32-bit offsets: fewer than 2^25 rows.)
  // A selection that gives the large tiles fewer blocks than half the CUs (an
  // epoch's tail batch: 3,392 rows x 1,024 centroids in 56 blocks took 55 us)
  // takes the 128 x 128 screen, whose 216 blocks there take 45 us.
  const size_t blocks3 = (n + TR3 - 1) / TR3 * (size_t)nt3;
  const bool few = 2 * blocks3 < (size_t)c->cus;
  if (split && !few && c->screen != SCREEN_F32 && k >= 64 && nt3 <= MAX_PARTS &&
      n < (1u << 25)) {
    g.big = g.split = true;
    g.row_tiles = (int)((n + TR3 - 1) / TR3);
    g.ntiles = g.parts = nt3;
    g.tpp = 1;
    return g;
  }
  // The large-tile bf16 screen (one 512-thread block per CU, 256-centroid
  // tiles) when d % 4 == 0 and k >= 64; smaller k fill a 128-centroid tile
  // better.
  g.big = c->screen != SCREEN_F32 && d % 4 == 0 && k >= 64 && !(split && few);
  const int TR = g.big ? TR3 : 128;
  g.row_tiles = (int)((n + TR - 1) / TR);
  g.ntiles = (int)((k + (g.big ? TC3 : TC) - 1) / (g.big ? TC3 : TC));
  g.parts = choose_parts(g.row_tiles, g.ntiles, c->cus, g.big ? 1 : 2);
  g.tpp = (g.ntiles + g.parts - 1) / g.parts;
  g.parts = (g.ntiles + g.tpp - 1) / g.tpp;
  return g;
}
}  // namespace

bool split_screen(emh_ctx* c, size_t n, size_t d, size_t k, bool ip) {
  return top1_geom(c, n, d, k, ip, true, true).split;
}
bool top1_screens(emh_ctx* c, size_t n, size_t d, size_t k, bool ip) {
  return top1_geom(c, n, d, k, ip, false, true).screen;
}
bool top1_tallies(emh_ctx* c, size_t n, size_t d, size_t k, bool ip) {
  // queued_direct holds for every smaller selection too (its items grow with n).
  return d % 4 == 0 && (top1_screens(c, n, d, k, ip) || queued_direct(c, n, d, k, ip));
}

size_t top1_scratch_bytes(emh_ctx* c, size_t n, size_t d, size_t k, bool ip) {
  const Top1Geom g = top1_geom(c, n, d, k, ip, false, true);
  if (!g.screen) return exact1_scratch_bytes(c, n, d, k, ip, false);
  auto r = [](size_t b) { return (b + 255) & ~size_t(255); };
  return r((size_t)g.parts * n * L1 * sizeof(Cand)) + 2 * r(n * 4) +
         exact1_scratch_bytes(c, n, d, k, ip, true);
}

namespace {
// The screen stage of a top-1 call: its lists, their parts, the rows' |x|^2,
// the check's queue and the arithmetic the check's bound must follow.
struct Top1Screen {
  Top1Geom g;
  Cand* cand = nullptr;
  uint32_t* fb = nullptr;
  float* xnorm = nullptr;
  bool tagged = false;
  bool f16 = false;  // the split-operand screen ran in fp16 two-pass arithmetic
  int L = L1;  // entries per part list: L1S for the sorted insert's, L1F for the fp16 screen's
};

// The split-operand screen's arithmetic: fp16 two-pass in SCREEN_F16, else
// bf16 three-pass.
bool split_f16(const emh_ctx* c) { return c->screen == SCREEN_F16; }

Top1Screen screen_top1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                       size_t lo, size_t n, const float* cents, const float* cnorm, size_t k,
                       bool ip, bool words_clear, Arena* ar, const SplitRows* pre,
                       const SplitCents* pc, bool small_exact) {
  Top1Screen s;
  s.g = top1_geom(c, n, d, k, ip, !ar, small_exact);
  if (!s.g.screen) return s;
  const Top1Geom& g = s.g;
  const bool f16 = g.split && split_f16(c);
  const size_t cbytes = (size_t)g.parts * n * (f16 ? L1F : L1) * sizeof(Cand);
  s.cand = (Cand*)(ar ? ar->take(cbytes) : c->cand.get(cbytes));
  s.fb = (uint32_t*)(ar ? ar->take(n * 4) : c->fblist.get(n * 4));
  s.xnorm = (float*)(ar ? ar->take(n * 4) : c->xnorm.get(n * 4));
  if (!words_clear)  // fallback count, cmax2, cnmax (the screen or the split fills the maxima)
    launch_fill_u32(c, c->small, 3, 0);
  const unsigned blocks = (unsigned)(g.row_tiles * g.parts);
  s.tagged = g.big && g.tpp == 1;
  s.L = f16 ? L1F : g.big && !s.tagged ? L1S : L1;
  if (g.split) {
    // The centroids' halves and the bound's centroid maxima (the caller's,
    // split ahead, or split here), then the rows' halves (the caller's, or
    // this selection's), all in the call's format.
    EMH_ENSURE(!pre || pre->f16 == f16, "top1: rows split in the other format");
    EMH_ENSURE(!pc || pc->f16 == f16, "top1: centroids split in the other format");
    s.f16 = f16;
    const void* cs;
    const uint32_t* part;
    int nparts;
    if (pc) {
      cs = pc->cs;
      part = pc->part;
      nparts = pc->nparts;
    } else {
      void* cw = c->csplit.get(halves_bytes(k, d));
      uint32_t* pw = (uint32_t*)c->csplit_part.get(halves_blocks(k) * 8);
      launch_halves(c, cents, k, d, nullptr, 0, k, cw, (float*)c->csplit_norm.get(k * 4),
                    ip ? nullptr : cnorm, pw, f16);
      cs = cw;
      part = pw;
      nparts = (int)halves_blocks(k);
    }
    Screen4Args a{blocks,   nullptr,  0,      nullptr, 0,       d,       nullptr,
                  0,        n,        cs,     k * 128, cnorm,   k,       1,
                  g.parts,  g.ntiles, s.cand, s.xnorm, part,    nparts,  f16};
    if (pre) {
      a.xs = pre->xs;
      a.xslab = pre->slab;
      a.xn = pre->xn;
      a.nx = pre->nx;
      a.ids = ids;
      a.lo = lo;
    } else {
      void* xs = c->xsplit.get(halves_bytes(n, d));
      launch_halves(c, x, nx, d, ids, lo, n, xs, s.xnorm, nullptr, nullptr, f16);
      a.xs = xs;
      a.xslab = n * 128;
      a.xn = s.xnorm;
      a.nx = n;
    }
    ProfScope prof(c, EMH_PROF_SCREEN, 2.0 * (double)n * (double)k * (double)d,
                   prof_take(c, EMH_PROF_SCREEN));
    launch_screen4(c, a, ip);
    return s;
  }
  ProfScope prof(c, EMH_PROF_SCREEN, 2.0 * (double)n * (double)k * (double)d,
                 !ar && prof_take(c, EMH_PROF_SCREEN));
  const ScreenArgs a{blocks, x, nx, d, ids, lo, n, cents, cnorm, k, g.tpp, g.parts, g.ntiles,
                     s.cand, s.xnorm};
  // One tile per part: tagged keys (the cheap fold); more: the sorted
  // insert, which skips most keys once the lists hold good ones.
  if (g.big)
    launch_screen3(c, a, ip, s.tagged);
  else
    launch_screen_t1(c, a, ip);
  return s;
}

// The check's bound arithmetic: the screen's (BoundKind).
int bound_kind(const emh_ctx* c, const Top1Screen& s) {
  if (c->screen == SCREEN_F32) return BOUND_F32;
  if (s.f16) return BOUND_F16_TAGGED;
  return s.tagged ? BOUND_BF16_TAGGED : BOUND_BF16;
}
}  // namespace

void launch_top1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids, size_t lo,
                 size_t hi, const float* cents, const float* cnorm, size_t k, bool ip,
                 uint32_t* labels, float* scores, bool words_clear, Arena* ar,
                 const SplitRows* pre, const SplitCents* pc, const LabelTally* tally) {
  if (hi <= lo) return;
  const size_t n = hi - lo;
  EMH_ENSURE(d <= 16384, "top1: d = %zu above the supported 16384", d);
  EMH_ENSURE(n < (1u << 31) && k < (1u << 31), "top1: shape too large");
  // A tallying call takes the screen, or the latency-bound exact scan, which
  // tallies too; never k_exact1.
  const bool small_exact = !tally || queued_direct(c, n, d, k, ip);
  const Top1Screen s = screen_top1(c, x, nx, d, ids, lo, n, cents, cnorm, k, ip, words_clear, ar,
                                   pre, pc, small_exact);
  EMH_ENSURE(!tally || (d % 4 == 0 && (s.g.screen || queued_direct(c, n, d, k, ip))),
             "top1: labels are tallied only by the screen or the queued-row scan, d %% 4 == 0");
  if (!s.g.screen) {
    launch_exact1(c, x, nx, d, ids, lo, n, nullptr, cents, cnorm, k, ip, labels, scores, ar,
                  tally);
    return;
  }
  launch_verify1(c, x, nx, d, ids, lo, n, cents, cnorm, k, ip, s.cand, s.g.parts, s.xnorm, labels,
                 scores, s.fb, bound_kind(c, s), tally, s.L);
  launch_exact1(c, x, nx, d, ids, lo, n, s.fb, cents, cnorm, k, ip, labels, scores, ar, tally);
}

void screen_margin_top1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                        size_t lo, size_t hi, const float* cents, const float* cnorm, size_t k,
                        bool ip, emh_screen_report* out) {
  *out = emh_screen_report{};
  if (hi <= lo) return;
  const size_t n = hi - lo;
  EMH_ENSURE(d <= 16384 && n < (1u << 31) && k < (1u << 31), "top1: shape too large");
  const Top1Screen s =
      screen_top1(c, x, nx, d, ids, lo, n, cents, cnorm, k, ip, false, nullptr, nullptr, nullptr,
                  false);
  if (!s.g.screen) return;  // variant 0: no screen, nothing to measure
  out->variant = s.f16     ? EMH_SCREEN_BIG_F16
                 : s.g.big ? (s.tagged ? EMH_SCREEN_BIG_TAGGED : EMH_SCREEN_BIG_SORTED)
                           : (c->screen == SCREEN_F32 ? EMH_SCREEN_SMALL_F32 : EMH_SCREEN_SMALL_BF16);
  out->parts = s.g.parts;
  out->tiles_per_part = s.g.tpp;
  launch_margin(c, x, nx, d, ids, lo, n, cents, cnorm, ip, s.cand, s.g.parts, s.L, s.xnorm,
                bound_kind(c, s), out);
}

void launch_topk(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                 size_t kk, bool exclude_self, uint32_t* ids, float* sims, emh_screen_report* rep) {
  if (m == 0) return;
  if (kk > (size_t)KMAX && !rep) {  // beyond the screen's lists: the exact top-k
    launch_topk_long(c, q, m, data, n, d, kk, exclude_self, ids, sims);
    return;
  }
  EMH_ENSURE(kk >= 1 && kk <= (size_t)KMAX, "topk: kk = %zu must be in 1..16", kk);
  EMH_ENSURE(d <= 16384, "topk: d = %zu above the supported 16384", d);
  EMH_ENSURE(m < (1u << 31) && n < (1u << 31), "topk: shape too large");
  if (n > 0 && screen4kn_fits(c, m, n, d)) {
    // The operands split once, the 128 x 256 DMA-fed screen, then the same check.
    Cand* cand = nullptr;
    float* xnorm = nullptr;
    const int parts = screen4kn(c, q, m, data, n, d, kk, exclude_self, &cand, &xnorm);
    if (rep) {
      *rep = emh_screen_report{};
      rep->variant = EMH_SCREEN_BIG_KNN;
      rep->parts = parts;
      rep->tiles_per_part = 0;
      launch_margin(c, q, m, d, nullptr, 0, m, data, nullptr, true, cand, parts, LK, xnorm,
                    BOUND_BF16, rep);
      return;
    }
    uint32_t* fb = (uint32_t*)c->fblist.get(m * 4);
    launch_verifyk(c, q, m, data, n, d, kk, cand, parts, xnorm, ids, sims, fb);
    launch_exactk(c, q, m, data, n, d, kk, exclude_self, fb, ids, sims);
    return;
  }
  const int TR = 64;
  const int row_tiles = (int)((m + TR - 1) / TR);
  const int ntiles = (int)((n + TC - 1) / TC);
  int parts = choose_parts(row_tiles, std::max(ntiles, 1), c->cus);
  const int tpp = (std::max(ntiles, 1) + parts - 1) / parts;
  parts = (std::max(ntiles, 1) + tpp - 1) / tpp;
  Cand* cand = (Cand*)c->cand.get((size_t)parts * m * LK * sizeof(Cand));
  uint32_t* fb = (uint32_t*)c->fblist.get(m * 4);
  float* xnorm = (float*)c->xnorm.get(m * 4);
  launch_fill_u32(c, c->small, 3, 0);
  if (n > 0) {
    ProfScope prof(c, EMH_PROF_SCREEN, 2.0 * (double)m * (double)n * (double)d,
                   prof_take(c, EMH_PROF_SCREEN));
    const unsigned blocks = (unsigned)(row_tiles * parts);
    launch_screen_kn(c, ScreenArgs{blocks, q, m, d, nullptr, 0, m, data, nullptr, n, tpp, parts,
                                   ntiles, cand, xnorm},
                     exclude_self);
  } else {
    parts = 1;
    launch_fill_u32(c, (uint32_t*)cand, m * LK * 2, NONE);  // empty lists
    launch_fill_u32(c, (uint32_t*)xnorm, m, 0);
  }
  if (rep) {  // the diagnostic: measure the lists, change nothing
    *rep = emh_screen_report{};
    if (n == 0) return;
    rep->variant = c->screen == SCREEN_F32 ? EMH_SCREEN_SMALL_F32 : EMH_SCREEN_SMALL_BF16;
    rep->parts = parts;
    rep->tiles_per_part = tpp;
    launch_margin(c, q, m, d, nullptr, 0, m, data, nullptr, true, cand, parts, LK, xnorm,
                  c->screen != SCREEN_F32 ? BOUND_BF16 : BOUND_F32, rep);
    return;
  }
  launch_verifyk(c, q, m, data, n, d, kk, cand, parts, xnorm, ids, sims, fb);
  launch_exactk(c, q, m, data, n, d, kk, exclude_self, fb, ids, sims);
}

}  // namespace emh
