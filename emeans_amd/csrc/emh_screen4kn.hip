// The kNN screen over operands split ahead of time (k_screen4kn): the first
// stage of the exact top-k (Device::topk, core/mod.rs:114-124) for queries and
// data rows split once into bf16 halves by k_halves, fed to the MFMAs through
// the LDS-DMA ring of the top-1 screen (k_screen4). Every workgroup streams all
// data rows of its part, so the split is what the earlier kNN screen (which
// split each slab it staged, in every workgroup) repeated.
//
// Tile: 128 queries x 256 data rows; wave w owns queries 64 (w % 2) .. + 64
// and data rows 64 (w / 2) .. + 64 (2 x 2 blocks of 32 x 32, the data rows as
// the MFMA's A, the queries as its B, so lane l holds query l % 32 of each
// block). Per 16 dimensions the same three bf16 MFMAs as the other screens
// (hi.hi, hi.lo, lo.hi), so the check's error bound E covers the keys.
//
// At the end of each data tile the keys (-dot) fold into per-lane lists of
// the L smallest (key, id), in registers. The two lane halves hold the same
// 32 queries in different data columns; one swap across them gives lane
// (l % 32, half y) both halves' keys of query 32 y + l % 32 of its wave, so a
// lane keeps one list. A key enters when it is at most the lane's own kk-th
// key plus 2E' (E' >= E: the check's bound on the same inputs, with margin
// for the rounding of that sum). The check settles a query when the merged
// list is not full or its L-th key lies beyond the merged kk-th key plus 2E;
// the merged kk-th key is at most any lane's, and a lane's kk-th key only
// falls, so every key the check needs was within its lane's threshold when it
// arrived: it is in the lane's list unless that list was full of smaller
// keys, and then the merged list's L-th key is below it, which sends the
// query to the exact scan. The four lists of a query (one per wave of its
// row) merge into the part's list at the end.

#include <algorithm>

#include "emh_screen4.h"

namespace emh {
namespace {

constexpr int TRK = 128;                         // queries per tile
constexpr int TCK = 256;                         // data rows per tile
constexpr int SK_ROWS = TRK * SLAB_BYTES;        // a stage's queries: 16 KB
constexpr int SK_STAGE = (TRK + TCK) * SLAB_BYTES;  // queries and data: 48 KB

template <int L, bool SELF>
__global__ __launch_bounds__(512, 1) void k_screen4kn(
    const char* __restrict__ qs, size_t qslab, const float* __restrict__ qn, int m,
    const char* __restrict__ xs, size_t xslab, int n, int d, int kk, int tiles_per_part,
    int parts, int ntiles, Cand* __restrict__ cand, float* __restrict__ xnorm,
    const uint32_t* __restrict__ cmax_part, int nparts, uint32_t* __restrict__ small) {
  constexpr int WA = 2, WN = 2;  // data and query 32-blocks per wave
  constexpr int PER = 6;         // DMAs per step per wave: 2 of queries, 4 of data
  __shared__ __attribute__((aligned(1024))) char s0[SK_STAGE], s1[SK_STAGE];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w & 1, wc = w >> 1;
  const int li = lane & 31, h = lane >> 5;
  const uint32_t wi = xcd_swizzle(blockIdx.x, gridDim.x);
  const int rt = (int)(wi / (uint32_t)parts), part = (int)(wi % (uint32_t)parts);
  const int t0 = part * tiles_per_part;
  const int t1 = min(ntiles, t0 + tiles_per_part);
  if (t0 >= t1) return;
  const int row0 = rt * TRK;
  const int d32 = (d + 31) >> 5;

  // Loader: DMA j of wave w fills LDS rows 64 j + 8 w + lane / 8 of an operand
  // (j < 2 for the queries, j < 4 for the data); lane's 16 bytes land in slot
  // lane % 8 of its row, which holds chunk (lane % 8) ^ swz(row). Queries past
  // m read query 0, data rows past n read row n - 1: neither is ever kept.
  const int lrow = w * 8 + (lane >> 3);
  const int lq = ((lane & 7) ^ swz(lrow)) << 4;
  uint32_t qo[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int r = row0 + j * 64 + lrow;
    qo[j] = (uint32_t)(r < m ? r : 0) * SLAB_BYTES + lq;
  }
  int lt = t0, lj = 0;  // load cursor: the step whose slabs the next DMAs fetch
  const int nsteps = (t1 - t0) * d32;
  auto dma_part = [&](char* X, int q) __attribute__((always_inline)) {
    if (q < 2) {
      dma16o(qs + lj * qslab, qo[q], X + (q * 64 + w * 8) * SLAB_BYTES);
    } else {
      const int j = q - 2;
      const int tl = min(lt, t1 - 1);
      const int row = min(tl * TCK + j * 64 + lrow, n - 1);
      dma16o(xs + lj * xslab, (uint32_t)row * SLAB_BYTES + lq,
             X + SK_ROWS + (j * 64 + w * 8) * SLAB_BYTES);
    }
  };
  auto advance = [&]() __attribute__((always_inline)) {
    const bool wrap = ++lj == d32;
    lj = wrap ? 0 : lj;
    lt += wrap ? 1 : 0;
  };

  const int sw = swz(li);  // LDS rows 64 wr + 32 y + li and 64 wc + 32 a + li
  struct Rows {
    v8bf bh[WN], bl[WN];
  };
  auto read_rows = [&](const char* X, int ks, Rows& o) __attribute__((always_inline)) {
    const int oh = ((4 * ks + h) ^ sw) << 4, ol = ((4 * ks + 2 + h) ^ sw) << 4;
#pragma unroll
    for (int y = 0; y < WN; y++) {
      const char* p = X + (wr * 64 + y * 32 + li) * SLAB_BYTES;
      o.bh[y] = *reinterpret_cast<const v8bf*>(p + oh);
      o.bl[y] = *reinterpret_cast<const v8bf*>(p + ol);
    }
  };
  v8bf ah[WA], al[WA];
  auto read_data = [&](const char* X, int ks, int a) __attribute__((always_inline)) {
    const int oh = ((4 * ks + h) ^ sw) << 4, ol = ((4 * ks + 2 + h) ^ sw) << 4;
    const char* p = X + SK_ROWS + (wc * 64 + a * 32 + li) * SLAB_BYTES;
    ah[a] = *reinterpret_cast<const v8bf*>(p + oh);
    al[a] = *reinterpret_cast<const v8bf*>(p + ol);
  };

  // The query whose list this lane keeps (after the swap, y = h).
  const uint32_t qown = (uint32_t)(row0 + wr * 64 + h * 32 + li);

  // 2E' per query: the check's bound from the split's |q|^2 and the data's
  // largest |x|^2 (the split's per-block partials; block 0 leaves it for the
  // check), with a margin for its own rounding.
  float thr_e;
  {
    uint32_t ma, mb;
    part_max(cmax_part, nparts, ma, mb);
    if (blockIdx.x == 0 && tid == 0) small[SW_CMAX2] = ma;
    const float cm2 = __uint_as_float(ma);
    const float xv = qown < (uint32_t)m ? qn[qown] : 0.f;
    thr_e = 2.0f * 1.0078125f * screen_bound(xv, cm2, 0.f, d, false, BOUND_BF16);
  }

  float lkey[L];
  uint32_t lid[L];
  float lim = INFINITY;  // min(L-th key, kk-th key + 2E'): keys above it never enter
#pragma unroll
  for (int e = 0; e < L; e++) {
    lkey[e] = INFINITY;
    lid[e] = NONE;
  }
  // After an insert: the new limit. The list is sorted ascending (never NaN),
  // so the kk-th key is the largest of the first kk: a max over a masked
  // unrolled chain. (kk is a runtime value. A chain of selects of list
  // elements was folded by the compiler into one indexed read, which put the
  // list in LDS: 48 KB more per block and bank-conflicting stores of the
  // whole list on every insert.)
  auto relimit = [&]() __attribute__((always_inline)) {
    float kth = lkey[0];
#pragma unroll
    for (int e = 1; e < L; e++) kth = fmaxf(kth, e < kk ? lkey[e] : -INFINITY);
    const float t = kth + thr_e + fabsf(kth) * 9.5367431640625e-07f + 1e-42f;  // + 2^-20 |kth|
    lim = fminf(lkey[L - 1], t);  // a NaN bound leaves the L-th key
  };
  auto offer = [&](float v, uint32_t gj) __attribute__((always_inline)) {
    float key = gj < (uint32_t)n ? 0.0f - v : INFINITY;
    if (SELF && gj == qown) key = INFINITY;
    const bool in = key <= lim;  // NaN never
    if (__ballot(in) != 0ull) {
      insert_nb<L>(lkey, lid, in ? key : INFINITY, gj);
      relimit();
    }
  };

  v16f acc[WA][WN];
#pragma unroll
  for (int a = 0; a < WA; a++)
#pragma unroll
    for (int y = 0; y < WN; y++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[a][y][r] = 0.f;

  // A data tile's keys into the lists; the accumulators start over. 32 x 32
  // accumulator layout: element r of lane l is (data row 8 (r / 4) +
  // 4 (l / 32) + r % 4 of the block, query l % 32 of query block y); block y's
  // queries are kept by the lanes of half y. First every element is compared
  // with its query's limit (dot >= -lim is key <= lim, exactly; a block's
  // maximum first), and the wave notes the (a, r) positions of block y where
  // some lane's element passes;
  // then, for those positions only, the element and its partner half's (one
  // swap) go to the query's list. Most positions pass nowhere once the lists
  // hold good keys, and the insert is written once per block y.
  auto fold = [&](int tile) __attribute__((always_inline)) {
    const float lp = __shfl_xor(lim, 32, 64);  // the partner lane's limit
    const float nl[WN] = {-(h == 0 ? lim : lp), -(h == 1 ? lim : lp)};
    uint32_t pos[WN] = {0u, 0u};  // bit 16 a + r: some lane's element passes (wave-uniform)
#pragma unroll
    for (int y = 0; y < WN; y++)
#pragma unroll
      for (int a = 0; a < WA; a++) {
        // The block's largest element first (fmaxf passes over NaN, which
        // never passes): once the lists hold good keys most blocks have no
        // passing element in any lane, and one ballot skips their sixteen.
        float mx = acc[a][y][0];
#pragma unroll
        for (int r = 1; r < 16; r++) mx = fmaxf(mx, acc[a][y][r]);
        if (__ballot(mx >= nl[y]) != 0ull) {
#pragma unroll
          for (int r = 0; r < 16; r++)
            pos[y] |= __ballot(acc[a][y][r] >= nl[y]) != 0ull ? 1u << (16 * a + r) : 0u;
        }
      }
#pragma unroll
    for (int y = 0; y < WN; y++) {
      for (uint32_t mk = pos[y]; mk != 0u; mk &= mk - 1u) {
        const int p = __builtin_ctz(mk), a = p >> 4, r = p & 15;
        // The element by selects (an indexed read would move acc to memory).
        float v = acc[0][y][0];
#pragma unroll
        for (int q = 1; q < 16 * WA; q++) v = p == q ? acc[q >> 4][y][q & 15] : v;
        const float o = __shfl_xor(v, 32, 64);
        const uint32_t g = (uint32_t)(tile * TCK + wc * 64 + a * 32 + 8 * (r >> 2) + (r & 3));
        const float nan = __uint_as_float(0x7fc00000u);  // never kept: the other half's query
        offer(h == y ? v : nan, g + 4 * h);
        offer(h == y ? o : nan, g + 4 * (1 - h));
      }
    }
#pragma unroll
    for (int a = 0; a < WA; a++)
#pragma unroll
      for (int y = 0; y < WN; y++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[a][y][r] = 0.f;
  };

  auto mfma6 = [&](int a, const Rows& b) __attribute__((always_inline)) {
#pragma unroll
    for (int y = 0; y < WN; y++)
      acc[a][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[a], b.bh[y], acc[a][y], 0, 0, 0);
#pragma unroll
    for (int y = 0; y < WN; y++)
      acc[a][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[a], b.bl[y], acc[a][y], 0, 0, 0);
#pragma unroll
    for (int y = 0; y < WN; y++)
      acc[a][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[a], b.bh[y], acc[a][y], 0, 0, 0);
  };
  // Prologue: steps 0 and 1 into stages 0 and 1; step 0's first operands.
#pragma unroll
  for (int q = 0; q < PER; q++) dma_part(s0, q);
  advance();
#pragma unroll
  for (int q = 0; q < PER; q++) dma_part(s1, q);
  advance();
  wait_vm<PER>();  // step 0's DMAs are in (step 1's stay in flight)
  __builtin_amdgcn_s_barrier();
  Rows r0, r1;
  read_rows(s0, 0, r0);
#pragma unroll
  for (int a = 0; a < WA; a++) read_data(s0, 0, a);
  int ct = t0, cj = 0;  // compute cursor: tile and slab of the current step
  // One step (a 32-dimension slab, two MFMA steps), as k_screen4's: the
  // second MFMA step's operands are read during the first, a barrier mid-slab
  // (every wave's DMAs of the next step are in, and no wave reads this stage
  // again), then the next step's first operands and the DMAs of the step after
  // it go out between the second MFMA step's groups. A tile's last slab ends
  // with its fold.
  auto step = [&](auto stage_no) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_no)::value;
    char* cur = S == 0 ? s0 : s1;
    const char* next = S == 0 ? s1 : s0;
#pragma unroll
    for (int a = 0; a < WA; a++) {
      mfma6(a, r0);
      __builtin_amdgcn_sched_barrier(0);
      if (a == 0) read_rows(cur, 1, r1);
      read_data(cur, 1, a);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm<0>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int a = 0; a < WA; a++) {
      mfma6(a, r1);
      __builtin_amdgcn_sched_barrier(0);
      if (a == 0) read_rows(next, 0, r0);
      read_data(next, 0, a);
#pragma unroll
      for (int q = 0; q < PER / WA; q++) dma_part(cur, a * (PER / WA) + q);
      if (a == WA - 1) advance();
      __builtin_amdgcn_sched_barrier(0);
    }
    if (++cj == d32) {
      fold(ct);
      cj = 0;
      ++ct;
    }
  };
  for (int st = 0; st < nsteps; st += 2) {
    step(StageNo<0>{});
    if (st + 1 < nsteps) step(StageNo<1>{});
  }
  wait_vm<0>();  // the DMAs past the last step have landed (the merge reuses stages)

  // The queries' |q|^2 for the check.
  if (part == 0 && tid < TRK) {
    const int r = row0 + tid;
    if (r < m) xnorm[r] = qn[r];
  }
  // Merge the four lists of each query (one per wave column wc), two wave
  // columns a round: keys in stage 0, ids in stage 1, list c (wc % 2) of
  // query r at c CS + r RS (RS odd: a wave's 64 lanes, 64 queries, hit 64
  // banks).
  constexpr int RS = L | 1, CS = TRK * RS;
  static_assert(2 * CS * 4 <= SK_STAGE, "merge space");
  float* MK = reinterpret_cast<float*>(s0);
  uint32_t* MI = reinterpret_cast<uint32_t*>(s1);
  float mk[L];
  uint32_t mi[L];
#pragma unroll
  for (int e = 0; e < L; e++) {
    mk[e] = INFINITY;
    mi[e] = NONE;
  }
  for (int round = 0; round < 2; round++) {
    __syncthreads();
    if ((wc >> 1) == round) {
      const int row = wr * 64 + h * 32 + li;
#pragma unroll
      for (int e = 0; e < L; e++) {
        MK[(wc & 1) * CS + row * RS + e] = lkey[e];
        MI[(wc & 1) * CS + row * RS + e] = lid[e];
      }
    }
    __syncthreads();
    if (tid < TRK) {
      for (int c = 0; c < 2; c++) {
#pragma unroll
        for (int e = 0; e < L; e++) {
          const uint32_t id = MI[c * CS + tid * RS + e];
          if (id != NONE) insert<L>(mk, mi, MK[c * CS + tid * RS + e], id);
        }
      }
    }
  }
  if (tid < TRK && row0 + tid < m) {
    Cand* out = cand + ((size_t)(row0 + tid) * parts + part) * L;  // [row][part][L]
#pragma unroll
    for (int e = 0; e < L; e++) out[e] = Cand{mk[e], mi[e]};
  }
}

}  // namespace

bool screen4kn_fits(emh_ctx* c, size_t m, size_t n, size_t d) {
  // (bf16 three-pass in every mode but SCREEN_OFF and SCREEN_F32)
  return c->screen != SCREEN_OFF && c->screen != SCREEN_F32 && d >= 32 && m >= 256 && n >= 512 &&
         m < (1u << 25) && n < (1u << 25);
}

int screen4kn(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
              size_t kk, bool exclude_self, Cand** cand_out, float** xnorm_out) {
  // The data rows split once (with their |x|^2 and per-block maxima of it);
  // the queries too, unless they are the data.
  const bool same = q == data && m == n;
  void* xs = c->csplit.get(halves_bytes(n, d));
  float* xn = (float*)c->csplit_norm.get(n * 4);
  // Past PART_MAX_ONCE partials, one workgroup reduces them ahead of the
  // screen, whose every block would otherwise read them all.
  const size_t hb = halves_blocks(n);
  uint32_t* part = (uint32_t*)c->csplit_part.get((hb + 1) * 8);
  launch_halves(c, data, n, d, nullptr, 0, n, xs, xn, nullptr, part);
  int nparts = (int)hb;
  if (hb > PART_MAX_ONCE) {
    launch_part_max(c, part, hb, part + 2 * hb);
    part += 2 * hb;
    nparts = 1;
  }
  const void* qs = xs;
  const float* qn = xn;
  if (!same) {
    void* qw = c->xsplit.get(halves_bytes(m, d));
    float* qnw = (float*)c->misc.get(m * 4);
    launch_halves(c, q, m, d, nullptr, 0, m, qw, qnw, nullptr, nullptr);
    qs = qw;
    qn = qnw;
  }
  const int row_tiles = (int)((m + TRK - 1) / TRK);
  const int ntiles = (int)((n + TCK - 1) / TCK);
  // Parts (data-tile ranges) per query tile only while there are fewer query
  // tiles than CUs: the blocks running at once on an XCD then stream the same
  // data tiles, which its L2 serves. (C4, 3,907 query tiles: 561 ms with one
  // part, 747 ms with three, though three fill the last wave of blocks better.)
  int parts = std::max(1, std::min(std::min((c->cus + row_tiles - 1) / row_tiles, ntiles),
                                   MAX_PARTS));
  const int tpp = (ntiles + parts - 1) / parts;
  parts = (ntiles + tpp - 1) / tpp;
  Cand* cand = (Cand*)c->cand.get((size_t)parts * m * LK * sizeof(Cand));
  float* xnorm = (float*)c->xnorm.get(m * 4);
  launch_fill_u32(c, c->small, 3, 0);
  auto kern = exclude_self ? k_screen4kn<LK, true> : k_screen4kn<LK, false>;
  ProfScope prof(c, EMH_PROF_SCREEN, 2.0 * (double)m * (double)n * (double)d,
                 prof_take(c, EMH_PROF_SCREEN));
  hipLaunchKernelGGL(kern, dim3((unsigned)(row_tiles * parts)), dim3(512), 0, c->stream,
                     (const char*)qs, m * (size_t)SLAB_BYTES, qn, (int)m, (const char*)xs,
                     n * (size_t)SLAB_BYTES, (int)n, (int)d, (int)kk, tpp, parts, ntiles, cand,
                     xnorm, part, nparts, c->small);
  EMH_HIP(hipGetLastError());
  *cand_out = cand;
  *xnorm_out = xnorm;
  return parts;
}

}  // namespace emh
