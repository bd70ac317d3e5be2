// The large-tile top-1 screen over operands split ahead of time (k_screen4),
// and the kernel that splits rows or centroids into halves (k_halves).
// Shared by emh_screen4.hip (launchers) and nothing else.
//
// k_screen3 splits every slab it stages (f32 loads, three conversions per
// element, LDS stores), once per row tile and centroid part, and runs its
// eight waves in lockstep between those stagings, so the MFMA pipe idles
// through each. Here the halves come from HBM as they will sit in LDS:
//  - rows are split once per bound matrix (a training run splits all of its
//    rows up front and every batch gathers them by id) or once per call, and
//    centroids once per batch, into slabs of 32 dimensions: 128 bytes per
//    row, one cache line (hi, hi, lo, lo chunks of 8 dimensions for each
//    16-dimension MFMA step), stored slab-major (slab j of every row
//    contiguous); dimensions past d are zero;
//  - slabs stream into a two-stage LDS ring by LDS DMA (global_load_lds, 16
//    bytes per lane, eight rows per instruction, no registers): the cost of
//    such a load goes with the cache lines it touches, and a row of a slab is
//    one line;
//  - a step's DMAs for the next slab go out between its groups of MFMAs, so
//    one wave's loads are issued while the other wave on its SIMD runs MFMAs.
// Two arithmetics, by the halves' format: bf16 three-pass (per 16 dimensions
// hi.hi, hi.lo, lo.hi: k_screen3's sequence, so the same keys and bound) and
// fp16 two-pass (centroid hi against row hi, then row lo: a third fewer
// MFMAs and operand reads, within a bound 2.7 times the bf16 one at d = 768;
// the centroids' lo halves are not read).
#pragma once

#include <type_traits>

#include "emh_dma.h"
#include "emh_halves.h"
#include "emh_screen_kern.h"

namespace emh {
namespace {

constexpr int S4_HALF = TR3 * SLAB_BYTES;  // one operand's slab in LDS: 32 KB
constexpr int S4_STAGE = 2 * S4_HALF;      // rows and centroids: 64 KB

// Chunks of a slab row: 4 kk + (0, 1) the hi halves of dimensions 16 kk +
// (0-7, 8-15), 4 kk + (2, 3) their lo halves, for MFMA step kk = 0, 1. In LDS
// the chunks of row r are XOR-swizzled by swz(r). A b128 read of an operand
// has lane l read row 32 y + (l % 32) at chunk c + l / 32 (c even); the 64
// banks serve sixteen 16-byte groups at a time, and row r's group is
// 8 (r % 2) + slot. With swz, the sixteen lanes l .. l + 15 (l % 16 == 0)
// and the eight-lane pairs l .. l + 7, l + 32 .. l + 39 (l % 8 == 0) each hit
// sixteen different groups: within a parity the rows' swz values differ in
// bits 1-2 over rows 2 j + p (j < 4) and in bit 0 between the two halves of
// sixteen rows, and c + l / 32 only flips bit 0. ((r >> 1) & 7 alone was
// conflict-free only for the first grouping.)
__device__ __forceinline__ int swz(int r) { return (((r >> 1) & 3) << 1) | ((r >> 3) & 1); }

// The largest of part[2 i] and of part[2 i + 1] over i < nparts (f32 bits
// compared as u32: a NaN or negative value wins), in every lane of the wave.
// Each lane's loads of a batch of PMB partials are issued together: a loop
// of load-then-max would wait once per 64 partials.
constexpr int PMB = 16;
__device__ __forceinline__ void part_max(const uint32_t* __restrict__ part, int nparts,
                                         uint32_t& ma, uint32_t& mb) {
  const int lane = threadIdx.x & 63;
  ma = 0;
  mb = 0;
  for (int i0 = 0; i0 < nparts; i0 += 64 * PMB) {
    uint2 v[PMB];
#pragma unroll
    for (int u = 0; u < PMB; u++) {
      const int i = i0 + 64 * u + lane;
      v[u] = i < nparts ? reinterpret_cast<const uint2*>(part)[i] : make_uint2(0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < PMB; u++) {
      ma = max(ma, v[u].x);
      mb = max(mb, v[u].y);
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    ma = max(ma, (uint32_t)__shfl_xor((int)ma, o, 64));
    mb = max(mb, (uint32_t)__shfl_xor((int)mb, o, 64));
  }
}

template <bool VEC4>
__device__ __forceinline__ void load32(const float* p, int col, int d, float (&v)[32]) {
  if (VEC4 && col + 32 <= d) {
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const float4 t = *reinterpret_cast<const float4*>(p + col + 4 * q);
      v[4 * q] = t.x;
      v[4 * q + 1] = t.y;
      v[4 * q + 2] = t.z;
      v[4 * q + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 32; e++) v[e] = col + e < d ? p[col + e] : 0.f;
  }
}

// Split rows ids[lo + g] (lo + g without ids; an id >= nx reads row 0) for
// g < n into out (fp16 halves when f16, else bf16), in selection order and
// slab-major: slab j of row g at
// out + (j n + g) 128 bytes. norm[g] = the row's |x|^2 (f32, summed in any
// order: the screen bound's input). With part: block b writes the largest
// |x|^2 of its rows and, with cnorm, the largest cnorm[g] (f32 bits; a NaN or
// negative value wins) to part[2 b], part[2 b + 1]: the bound's centroid
// inputs, which the screen reduces (no atomics on one word).
// Block b takes rows 8 b .. 8 b + 7, two per wave. A wave reads a row in
// 256-dimension segments, 16 contiguous bytes per lane (one 1 KB run per
// load instruction), and lane l writes the hi and lo quads of its four
// dimensions (8 bytes each) into slab 8 s + l / 8: eight lanes fill one
// slab row, so each store instruction covers eight whole 128-byte lines.
template <bool VEC4>
__global__ __launch_bounds__(256) void k_halves(const float* __restrict__ x, size_t nx, int d,
                                                const uint32_t* __restrict__ ids, size_t lo,
                                                size_t n, char* __restrict__ out,
                                                float* __restrict__ norm,
                                                const float* __restrict__ cnorm,
                                                uint32_t* __restrict__ part, int f16) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int d32 = (d + 31) >> 5, nseg = (d32 + 7) >> 3;
  const int js = lane >> 3, c4 = lane & 7;
  const int hoff = quad_hi_offset(c4);
  size_t g[2];
  bool valid[2];
  const float* xr[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    g[i] = (size_t)blockIdx.x * 8 + 2 * w + i;
    valid[i] = g[i] < n;
    size_t id = 0;
    if (valid[i]) {
      id = ids ? (size_t)ids[lo + g[i]] : lo + g[i];
      if (id >= nx) id = 0;
    }
    xr[i] = x + id * (size_t)d;
  }
  float sq[2] = {0.f, 0.f};
#pragma unroll 3
  for (int s = 0; s < nseg; s++) {
    const int j = 8 * s + js;
    if (j >= d32) break;
    const int col = 32 * j + 4 * c4;
    float4 v[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
      if (VEC4) {
        v[i] = col < d ? *reinterpret_cast<const float4*>(xr[i] + col) : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        v[i].x = col < d ? xr[i][col] : 0.f;
        v[i].y = col + 1 < d ? xr[i][col + 1] : 0.f;
        v[i].z = col + 2 < d ? xr[i][col + 2] : 0.f;
        v[i].w = col + 3 < d ? xr[i][col + 3] : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
      sq[i] = fmaf(v[i].x, v[i].x, sq[i]);
      sq[i] = fmaf(v[i].y, v[i].y, sq[i]);
      sq[i] = fmaf(v[i].z, v[i].z, sq[i]);
      sq[i] = fmaf(v[i].w, v[i].w, sq[i]);
      uint2 hi, lw;
      split_quad(v[i], hi, lw, f16 != 0);
      if (valid[i]) {
        char* o = out + ((size_t)j * n + g[i]) * SLAB_BYTES + hoff;
        *reinterpret_cast<uint2*>(o) = hi;
        *reinterpret_cast<uint2*>(o + 32) = lw;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) sq[i] += __shfl_xor(sq[i], m, 64);
    if (valid[i] && lane == 0) norm[g[i]] = sq[i];
  }
  if (part) {
    uint32_t ma = 0u, mb = 0u;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      if (valid[i]) {
        ma = max(ma, __float_as_uint(sq[i]));
        if (cnorm) mb = max(mb, __float_as_uint(cnorm[g[i]]));
      }
    }
    __shared__ uint32_t red[2][4];
    if (lane == 0) {
      red[0][w] = ma;
      red[1][w] = mb;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      part[2 * blockIdx.x] = max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3]));
      part[2 * blockIdx.x + 1] = max(max(red[1][0], red[1][1]), max(red[1][2], red[1][3]));
    }
  }
}

// A compile-time stage number: each access then names one LDS array.
template <int I>
using StageNo = std::integral_constant<int, I>;

// The screen. Block: NW waves over TR3 = 256 rows x TC3 = 256 centroids per
// tile (k_screen3's block tile). xs: the split rows of the
// data (row id of slab j at xs + j xslab + 128 id), gathered by ids[lo + r]
// (lo + r without ids); xn: their |x|^2, copied to xnorm[r] by part 0 unless
// xn is xnorm; cs: the split centroids (slab stride cslab); cnorm: their
// norms (L2). Ring: step s (tile t0 + s / d32, slab s % d32) sits in stage
// s % 2. Step s waits for its own DMAs, passes a barrier (every wave's DMAs of
// step s are in, and every wave is done with stage (s + 1) % 2), then runs
// its MFMAs while it issues the DMAs of step s + 1 into the other stage.
template <int L, bool L2, int NW, bool F16>
__global__ __launch_bounds__(NW * 64, 1) void k_screen4(
    const char* __restrict__ xs, size_t xslab, const float* __restrict__ xn, size_t nx, int d,
    const uint32_t* __restrict__ ids, size_t lo, int nrows, const char* __restrict__ cs,
    size_t cslab, const float* __restrict__ cnorm, int k, int tiles_per_part, int parts,
    int ntiles, Cand* __restrict__ cand, float* __restrict__ xnorm,
    const uint32_t* __restrict__ cmax_part, int nparts, uint32_t* __restrict__ small) {
  // NW = 8: wave w owns rows 64 (w % 4) .. + 64 (WN = 2 row blocks) and
  // centroids 128 (w / 4) .. + 128, two waves per SIMD; NW = 4: rows
  // 128 (w % 2) .. + 128 (WN = 4), one wave per SIMD with 256 accumulators.
  constexpr int WA = 4, WN = 8 / (NW / 2);  // A (centroid) and B (row) 32-blocks per wave
  constexpr int RW = 32 * WN;               // rows per wave
  constexpr int ND = 32 / NW;               // DMAs per operand per step per wave
  __shared__ __attribute__((aligned(1024))) char s0[S4_STAGE], s1[S4_STAGE];
  __shared__ __attribute__((aligned(16))) float Ns[4][TC3];  // tile norms, by tile % 4

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w % (NW / 2), wc = w / (NW / 2);
  const int li = lane & 31, h = lane >> 5;
  const uint32_t wi = xcd_swizzle(blockIdx.x, gridDim.x);
  const int rt = (int)(wi / (uint32_t)parts), part = (int)(wi % (uint32_t)parts);
  const int t0 = part * tiles_per_part;
  const int t1 = min(ntiles, t0 + tiles_per_part);
  if (t0 >= t1) return;
  const int row0 = rt * TR3;
  const int d32 = (d + 31) >> 5;

  // Loader: DMA j (0 .. ND - 1) of wave w fills LDS rows 8 NW j + 8 w + lane / 8
  // of an operand; lane's 16 bytes land in slot lane % 8 of its row, which
  // holds chunk (lane % 8) ^ swz(row) (8 NW j is a multiple of 32). Rows past
  // the selection (or with a bad id) read data row 0; their lists are never
  // written.
  const int lrow = w * 8 + (lane >> 3);
  const int lq = ((lane & 7) ^ swz(lrow)) << 4;
  uint32_t xo[ND];  // byte offsets of the lanes' rows in a slab (nx < 2^25)
#pragma unroll
  for (int j = 0; j < ND; j++) {
    const int r = row0 + j * 8 * NW + lrow;
    uint32_t id = 0;
    if (r < nrows) {
      const size_t p = lo + (size_t)r;
      const size_t v = ids ? (size_t)ids[p] : p;
      id = v < nx ? (uint32_t)v : 0u;
    }
    xo[j] = id * SLAB_BYTES + lq;
  }
  // Load cursor: the step whose slabs the next DMAs fetch (tile lt, slab
  // lj). Every step issues the next step's DMAs; past the last step they
  // fetch the last tile's slabs again into a stage that nothing reads, so the
  // code of a step has no branches.
  int lt = t0, lj = 0;
  const int nsteps = (t1 - t0) * d32;
  // DMA q of the current load step into stage X: q < ND rows, then ND
  // centroids (the last: and the tile's norms).
  auto dma_part = [&](char* X, int q) __attribute__((always_inline)) {
    const int j = q % ND;
    char* dst = X + (q / ND) * S4_HALF + (j * 8 * NW + w * 8) * SLAB_BYTES;
    if (q < ND) {
      dma16o(xs + lj * xslab, xo[j], dst);
    } else {
      const int tl = min(lt, t1 - 1);
      const int row = min(tl * TC3 + j * 8 * NW + lrow, k - 1);
      dma16o(cs + lj * cslab, (uint32_t)row * SLAB_BYTES + lq, dst);
      if (L2 && q == 2 * ND - 1)  // 64 norms per wave (waves w and w + 4 alike)
        dma4(cnorm + min(tl * TC3 + (w & 3) * 64 + lane, k - 1), &Ns[tl & 3][(w & 3) * 64]);
    }
  };
  auto advance = [&]() __attribute__((always_inline)) {
    const bool wrap = ++lj == d32;
    lj = wrap ? 0 : lj;
    lt += wrap ? 1 : 0;
  };

  // Operand reads of MFMA step kk (0, 1) of a slab from its stage X: lane
  // half h takes dimensions 16 kk + 8 h .. + 7 (chunk 4 kk + h of the hi
  // half, 4 kk + 2 + h of the lo half).
  const int sw = swz(li);  // rows wr * RW + y * 32 + li: swz(row) = sw
  // Operand registers: 8 halves of one format (fp16 or bf16).
  typedef std::conditional_t<F16, v8h, v8bf> Op;
  struct Rows {
    Op bh[WN], bl[WN];
  };
  auto read_rows = [&](const char* X, int kk, Rows& o) __attribute__((always_inline)) {
    const int oh = ((4 * kk + h) ^ sw) << 4, ol = ((4 * kk + 2 + h) ^ sw) << 4;
#pragma unroll
    for (int y = 0; y < WN; y++) {
      const char* p = X + (wr * RW + y * 32 + li) * SLAB_BYTES;
      o.bh[y] = *reinterpret_cast<const Op*>(p + oh);
      o.bl[y] = *reinterpret_cast<const Op*>(p + ol);
    }
  };
  Op ah[WA], al[WA];  // centroid operands: each refreshed right after its MFMAs (al: bf16)
  auto read_cent = [&](const char* X, int kk, int a) __attribute__((always_inline)) {
    const int oh = ((4 * kk + h) ^ sw) << 4, ol = ((4 * kk + 2 + h) ^ sw) << 4;
    const char* p = X + S4_HALF + (wc * 128 + a * 32 + li) * SLAB_BYTES;
    ah[a] = *reinterpret_cast<const Op*>(p + oh);
    if (!F16) al[a] = *reinterpret_cast<const Op*>(p + ol);
  };

  float lkey[WN][L];  // per-row lists, filled by the fold after the loop
  uint32_t lid[WN][L];
  v16f acc[WA][WN];
#pragma unroll
  for (int a = 0; a < WA; a++)
#pragma unroll
    for (int y = 0; y < WN; y++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[a][y][r] = 0.f;

  // The fold keeps, per lane and row, the L smallest keys of the lane's
  // columns among those within its own smallest key m plus twice the bound
  // E' >= E the check uses (screen_bound on the same inputs, with a margin
  // for its own rounding and for the tags' 63 ulps). The check settles a row
  // only when every part's merged list is complete within the row's best key
  // b <= m plus 2E: a key within b + 2E is within m + 2E' of its lane, so it
  // is in the lane's list unless that list is full of smaller keys, and then
  // the merged list is full with its last key within b + 2E, which sends the
  // row to the exact scan. A NaN bound inserts nothing (the row goes to the
  // exact scan). Keys beyond the threshold, nearly all of them, cost a
  // compare each instead of an insert.
  float thr_e[WN];  // 2E' per row of the lane
  {
    // The bound's centroid maxima from the centroid split's per-block
    // partials (max of the f32 bits: a NaN or negative value wins); block 0
    // leaves them in the small block for the check.
    uint32_t ma, mb;
    part_max(cmax_part, nparts, ma, mb);
    if (blockIdx.x == 0 && tid == 0) {
      small[SW_CMAX2] = ma;
      small[SW_CNMAX] = L2 ? mb : 0u;
    }
    const float cm2 = __uint_as_float(ma), cnm = L2 ? __uint_as_float(mb) : 0.f;
#pragma unroll
    for (int y = 0; y < WN; y++) {
      const int r = row0 + wr * RW + y * 32 + li;
      float xv = 0.f;
      if (r < nrows) {
        const size_t p = lo + (size_t)r;
        const size_t id = ids ? (size_t)ids[p] : p;
        xv = xn[id < nx ? id : 0];
      }
      thr_e[y] = 2.0f * 1.0078125f *
                 screen_bound(xv, cm2, cnm, d, L2, F16 ? BOUND_F16_TAGGED : BOUND_BF16_TAGGED);
    }
  }
  auto threshold = [&](float m, int y) __attribute__((always_inline)) {
    return m + thr_e[y] + fabsf(m) * 1.52587890625e-05f + 1e-42f;  // + 2^-16 |m|: the tags
  };
  // A part of one tile: each key carries its lane-local column tag 16 a + r
  // in its low 6 mantissa bits (the bound covers the change), so that an
  // insert of bare floats keeps the lane's L smallest per row; the tags then
  // give the ids. (A tagged +inf or NaN is a NaN, which no compare takes.)
  // The lane's smallest tagged key is always within its threshold: it opens
  // the list, and the insert pass (a wave-wide branch, taken when any lane
  // has a key to insert) is left with the near-ties, which are rare; keys
  // carry distinct tags, so the list is the one inserting every key gives.
  auto fold_tagged = [&](int tile) __attribute__((always_inline)) {
    const float* ns = Ns[tile & 3];
    float m[WN], tm[WN];  // the lane's smallest key, and smallest tagged key
#pragma unroll
    for (int y = 0; y < WN; y++) m[y] = tm[y] = INFINITY;
#pragma unroll
    for (int a = 0; a < WA; a++) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int c0 = wc * 128 + a * 32 + 8 * q + 4 * h;
        const float4 n4 = L2 ? *reinterpret_cast<const float4*>(ns + c0) : make_float4(0, 0, 0, 0);
        const float nv[4] = {n4.x, n4.y, n4.z, n4.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int r = 4 * q + e;
          const float nn = tile * TC3 + c0 + e < k ? nv[e] : INFINITY;
#pragma unroll
          for (int y = 0; y < WN; y++) {
            const float v = acc[a][y][r];
            const float key = L2 ? fmaf(-2.0f, v, nn) : nn - v;  // one rounding: within E
            m[y] = fminf(m[y], key);
            const float tagged =
                __uint_as_float((__float_as_uint(key) & ~63u) | (uint32_t)(16 * a + r));
            tm[y] = fminf(tm[y], tagged);  // a tagged +-inf is a NaN: never the minimum
            acc[a][y][r] = tagged;
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // one centroid block's accumulators at a time
    }
    float thr[WN], tk[WN][L];
#pragma unroll
    for (int y = 0; y < WN; y++) {
      thr[y] = threshold(m[y], y);
      tk[y][0] = tm[y] <= thr[y] ? tm[y] : INFINITY;  // not when the bound is NaN
#pragma unroll
      for (int e = 1; e < L; e++) tk[y][e] = INFINITY;
    }
#pragma unroll
    for (int a = 0; a < WA; a++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
#pragma unroll
        for (int y = 0; y < WN; y++) {
          const float tagged = acc[a][y][r];
          const bool in = tagged <= thr[y] && tagged != tm[y];
          if (__ballot(in) != 0ull) insert_key<L>(tk[y], in ? tagged : INFINITY);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int y = 0; y < WN; y++) {
#pragma unroll
      for (int e = 0; e < L; e++) {
        const float kv = tk[y][e];
        const uint32_t tg = __float_as_uint(kv) & 63u;
        const int ci = wc * 128 + (int)(tg >> 4) * 32 + 8 * (int)((tg & 15u) >> 2) + 4 * h +
                       (int)(tg & 3u);
        lkey[y][e] = kv;
        lid[y][e] = kv < INFINITY ? (uint32_t)(tile * TC3 + ci) : NONE;
      }
    }
  };

  constexpr int PER = 2 * ND + (L2 ? 1 : 0);  // DMAs per step per wave
  auto mfma = [](const Op& p, const Op& q, const v16f& c) __attribute__((always_inline)) {
    if constexpr (F16)
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(p, q, c, 0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(p, q, c, 0, 0, 0);
  };
  // One centroid block's MFMAs of a 16-dimension step: hi.hi, hi.lo, then
  // (bf16) lo.hi.
  auto mfma6 = [&](int a, const Rows& b) __attribute__((always_inline)) {
#pragma unroll
    for (int y = 0; y < WN; y++) acc[a][y] = mfma(ah[a], b.bh[y], acc[a][y]);
#pragma unroll
    for (int y = 0; y < WN; y++) acc[a][y] = mfma(ah[a], b.bl[y], acc[a][y]);
    if constexpr (!F16) {
#pragma unroll
      for (int y = 0; y < WN; y++) acc[a][y] = mfma(al[a], b.bh[y], acc[a][y]);
    }
  };
  // Prologue: steps 0 and 1 into stages 0 and 1; step 0's first operands.
#pragma unroll
  for (int q = 0; q < 2 * ND; q++) dma_part(s0, q);
  advance();
#pragma unroll
  for (int q = 0; q < 2 * ND; q++) dma_part(s1, q);
  advance();
  wait_vm<PER>();  // step 0's DMAs are in (step 1's stay in flight)
  __builtin_amdgcn_s_barrier();
  Rows r0, r1;  // row operands of the first and second MFMA steps of a slab
  read_rows(s0, 0, r0);
#pragma unroll
  for (int a = 0; a < WA; a++) read_cent(s0, 0, a);
  // One step s (a 32-dimension slab in stage s % 2, two MFMA steps), as
  // groups of 3 WN MFMAs (one centroid block each) with the fences keeping
  // each group's other work after it:
  //  - first MFMA step: its groups are followed by the reads of the second
  //    step's operands they no longer need;
  //  - the wave's reads are done and its DMAs of step s + 1 have landed;
  //    barrier: every wave's have, and no wave reads stage s % 2 again;
  //  - second MFMA step: its groups are followed by the reads of step s + 1's
  //    first operands (stage (s + 1) % 2) and the DMAs of step s + 2 into
  //    stage s % 2.
  // So the next step's MFMAs start on operands already in registers, and a
  // wave's reads and DMAs go out while the other wave on its SIMD runs
  // MFMAs. Past the last step the reads fetch stale stages and the DMAs
  // fetch the last tile again, which nothing uses.
  auto step = [&](auto stage_no) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_no)::value;
    char* cur = S == 0 ? s0 : s1;
    const char* next = S == 0 ? s1 : s0;
#pragma unroll
    for (int a = 0; a < WA; a++) {
      mfma6(a, r0);
      __builtin_amdgcn_sched_barrier(0);
      if (a == 0) read_rows(cur, 1, r1);
      read_cent(cur, 1, a);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm<0>();  // this wave's DMAs of step s + 1 have landed
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): its reads of stage s % 2 are done
    __builtin_amdgcn_s_barrier();  // ... and every wave's
#pragma unroll
    for (int a = 0; a < WA; a++) {
      mfma6(a, r1);
      __builtin_amdgcn_sched_barrier(0);
      if (a == 0) read_rows(next, 0, r0);
      read_cent(next, 0, a);
#pragma unroll
      for (int q = 0; q < ND / 2; q++) dma_part(cur, a * (ND / 2) + q);
      if (a == WA - 1) advance();
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int st = 0; st < nsteps; st += 2) {
    step(StageNo<0>{});
    if (st + 1 < nsteps) step(StageNo<1>{});
  }
  wait_vm<0>();  // the DMAs past the last step have landed (the merge reuses stages)
  fold_tagged(t0);

  // The rows' |x|^2 for the check (the split's sums).
  if (part == 0 && xn != xnorm && tid < TR3) {
    const int r = row0 + tid;
    if (r < nrows) {
      const size_t p = lo + (size_t)r;
      size_t id = ids ? (size_t)ids[p] : p;
      if (id >= nx) id = 0;
      xnorm[r] = xn[id];
    }
  }
  // Merge the four partial lists of each row (two lane halves x two centroid
  // waves): keys in stage 0, ids in stage 1, entry e of contribution c for
  // row r at c CS + r RS + e. RS is odd, so the merge's reads (one row per
  // lane) touch 64 different banks; CS is 32 banks past a multiple of 64, so
  // the two lane halves' stores (rows li, contributions 2 wc + h) do too.
  constexpr int RS = L | 1, CS = (TR3 * RS + 63) / 64 * 64 + 32;
  float* MK = reinterpret_cast<float*>(s0);
  uint32_t* MI = reinterpret_cast<uint32_t*>(s1);
  static_assert(4 * CS * 4 <= S4_STAGE, "merge space");
  __syncthreads();
#pragma unroll
  for (int y = 0; y < WN; y++) {
    const int row = wr * RW + y * 32 + li;
    const int contrib = wc * 2 + h;
#pragma unroll
    for (int e = 0; e < L; e++) {
      MK[contrib * CS + row * RS + e] = lkey[y][e];
      MI[contrib * CS + row * RS + e] = lid[y][e];
    }
  }
  __syncthreads();
  for (int row = tid; row < TR3; row += NW * 64) {
    if (row0 + row >= nrows) continue;
    float mk[L];
    uint32_t mi[L];
#pragma unroll
    for (int e = 0; e < L; e++) {
      mk[e] = INFINITY;
      mi[e] = NONE;
    }
    for (int c = 0; c < 4; c++) {
#pragma unroll
      for (int e = 0; e < L; e++) {
        const uint32_t id = MI[c * CS + row * RS + e];
        if (id != NONE) insert<L>(mk, mi, MK[c * CS + row * RS + e], id);
      }
    }
    Cand* out = cand + ((size_t)(row0 + row) * parts + part) * L;  // [row][part][L]
#pragma unroll
    for (int e = 0; e < L; e++) out[e] = Cand{mk[e], mi[e]};
  }
}

}  // namespace
}  // namespace emh
