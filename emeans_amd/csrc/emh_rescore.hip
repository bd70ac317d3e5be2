// The check behind the MFMA screen (emh_screen.hip): per row, bound the
// screen's error, decide from the centroid parts' candidate lists whether the
// candidates are complete, and either queue the row for the exact scan
// (emh_verify.hip) or re-score its candidates with the reference's float order:
//   dot = one fma chain over t = 0..d-1 from +0 (assign/fused.rs:241-260);
//   L2 key = cnorm[j] - 2 dot (two roundings, assign.rs:461);
//   |x|^2 = sequential sum of rounded squares (assign.rs:150-155);
//   score = dot (IP) or max(|x|^2 + key, 0) (L2, assign.rs:497-502);
//   ties to the lower id.
// Top-1 with d % 4 == 0 (k_check1): the rows and their candidates are staged
// through LDS in chunks by loader waves while compute waves run the chains.
// Top-k and the top-1 case d % 4 != 0 (k_verify): one thread per (row,
// candidate) pair runs a chain, reading the row and the candidate from global
// memory with PF float4 loads of each in flight.

#include <cstring>

#include "emh_select.h"

namespace emh {
namespace {

constexpr int PF = 16;  // float4 loads of each operand in flight per chain

// Exact fma chain of x and c (the cpu-fused dot); acc starts at +0.
template <bool VEC4>
__device__ __forceinline__ float chain(const float* __restrict__ xr, const float* __restrict__ cr,
                                       int d) {
  float acc = 0.f;
  if (VEC4) {
    const float4* c4 = reinterpret_cast<const float4*>(cr);
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    const int d4 = d >> 2;
    int t = 0;
    for (; t + PF <= d4; t += PF) {
      float4 a[PF], b[PF];
#pragma unroll
      for (int u = 0; u < PF; u++) {
        a[u] = x4[t + u];
        b[u] = c4[t + u];
      }
#pragma unroll
      for (int u = 0; u < PF; u++) {
        acc = fmaf(a[u].x, b[u].x, acc);
        acc = fmaf(a[u].y, b[u].y, acc);
        acc = fmaf(a[u].z, b[u].z, acc);
        acc = fmaf(a[u].w, b[u].w, acc);
      }
    }
    for (; t < d4; t++) {
      const float4 a = x4[t], b = c4[t];
      acc = fmaf(a.x, b.x, acc);
      acc = fmaf(a.y, b.y, acc);
      acc = fmaf(a.z, b.z, acc);
      acc = fmaf(a.w, b.w, acc);
    }
  } else {
    for (int t = 0; t < d; t++) acc = fmaf(xr[t], cr[t], acc);
  }
  return acc;
}

// Sequential f32 sum of rounded squares.
template <bool VEC4>
__device__ __forceinline__ float seq_sq(const float* __restrict__ xr, int d) {
  float s = 0.f;
  if (VEC4) {
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    const int d4 = d >> 2;
    int t = 0;
    for (; t + PF <= d4; t += PF) {
      float4 a[PF];
#pragma unroll
      for (int u = 0; u < PF; u++) a[u] = x4[t + u];
#pragma unroll
      for (int u = 0; u < PF; u++) {
        float p0 = a[u].x * a[u].x, p1 = a[u].y * a[u].y, p2 = a[u].z * a[u].z,
              p3 = a[u].w * a[u].w;
        s = s + p0;
        s = s + p1;
        s = s + p2;
        s = s + p3;
      }
    }
    for (; t < d4; t++) {
      const float4 a = x4[t];
      float p0 = a.x * a.x, p1 = a.y * a.y, p2 = a.z * a.z, p3 = a.w * a.w;
      s = s + p0;
      s = s + p1;
      s = s + p2;
      s = s + p3;
    }
  } else {
    for (int t = 0; t < d; t++) {
      float p = xr[t] * xr[t];
      s = s + p;
    }
  }
  return s;
}

// Block: 256 threads, R rows (positions lo + r0 ...). KNN: rows are queries,
// "centroids" the data rows, and the kk best by exact dot are written per
// query (labels/scores then hold m x kk ids/sims).
template <int L, int R, bool KNN, bool VEC4>
__global__ __launch_bounds__(256) void k_verify(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int nrows, const float* __restrict__ cents, const float* __restrict__ cnorm, int k, int ip,
    int kk, const Cand* __restrict__ cand, int parts, const float* __restrict__ xnorm,
    uint32_t* __restrict__ labels, float* __restrict__ scores, uint32_t* __restrict__ fb,
    uint32_t* __restrict__ small, int bound) {
  constexpr int PMAX = R * (KNN ? L : C1 + 1);  // pairs (+ the |x|^2 chain per top-1 row)
  __shared__ Cand cst[R * MAX_PARTS * L];
  __shared__ uint32_t prow[PMAX], pcid[PMAX];
  __shared__ float pres[PMAX];
  __shared__ int cnt[R], off[R + 1];
  __shared__ uint32_t rowid[R];
  __shared__ int rstate[R];
  const int tid = threadIdx.x;
  const int r0 = blockIdx.x * R;
  const int rows = min(R, nrows - r0);
  const bool l2 = !KNN && !ip;

  if (tid < rows) {
    const size_t p = lo + (size_t)(r0 + tid);
    const size_t xid = ids ? (size_t)ids[p] : p;
    if (xid >= nx) small[SW_BAD_ID] = 1;
    rowid[tid] = xid < nx ? (uint32_t)xid : NONE;
  }
  // The block's candidate lists (rows x parts x L, contiguous) into LDS.
  {
    const int ne = rows * parts * L;
    const uint2* src = reinterpret_cast<const uint2*>(cand + (size_t)r0 * parts * L);
    uint2* dst = reinterpret_cast<uint2*>(cst);
    for (int i0 = tid; i0 < ne; i0 += 256 * 4) {
      uint2 v[4];
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (i0 + 256 * u < ne) v[u] = src[i0 + 256 * u];
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (i0 + 256 * u < ne) dst[i0 + 256 * u] = v[u];
    }
  }
  __syncthreads();
  // One thread per row. kNN: merge (each part's list is ascending, so a part
  // is done at its first entry not below the current L-th key), bound, decide.
  // Top-1: per part, as k_check1 decides (a part's list holds all of its
  // centroids within thr when not full or when its last key is above thr).
  float key[L];
  uint32_t id[L];
  float thr = 0.f;
  if (tid < rows) {
    const Cand* c = cst + tid * parts * L;
    if (KNN) {
#pragma unroll
      for (int e = 0; e < L; e++) {
        key[e] = INFINITY;
        id[e] = NONE;
      }
      for (int q = 0; q < parts; q++)
        for (int e = 0; e < L; e++) {
          const Cand v = c[q * L + e];
          if (v.id == NONE || !(v.key < key[L - 1])) break;
          insert<L>(key, id, v.key, v.id);
        }
    }
    int state = 0, nc = 0;
    if (rowid[tid] != NONE) {
      const float E = screen_bound(xnorm[r0 + tid], __uint_as_float(small[SW_CMAX2]),
                                   __uint_as_float(small[SW_CNMAX]), d, l2, bound);
      bool complete;
      if (KNN) {
        thr = key[kk - 1] + 2.0f * E;
        complete = id[L - 1] == NONE || key[L - 1] > thr;
        if (complete)
#pragma unroll
          for (int e = 0; e < L - 1; e++) nc += id[e] != NONE && (key[e] <= thr || thr != thr);
      } else {
        float best = INFINITY;
        bool anyv = false;
        for (int q = 0; q < parts; q++)
          if (c[q * L].id != NONE) {
            anyv = true;
            best = fminf(best, c[q * L].key);
          }
        thr = best + 2.0f * E;
        bool cert = true;
        int tot = 0;
        for (int q = 0; q < parts; q++) {
          const Cand last = c[q * L + L - 1];
          if (last.id != NONE && !(last.key > thr)) cert = false;
          for (int e = 0; e < L; e++) {
            const Cand v = c[q * L + e];
            tot += v.id != NONE && (v.key <= thr || thr != thr);
          }
        }
        complete = anyv && cert && tot <= C1;
        if (complete) nc = tot + (l2 ? 1 : 0);
      }
      if (complete) {
        state = 1;
      } else {
        nc = 0;
        const uint32_t f = atomicAdd(&small[SW_FALLBACK_COUNT], 1u);
        fb[f] = KNN ? (uint32_t)(r0 + tid) : (uint32_t)(lo + r0 + tid);
      }
    }
    rstate[tid] = state;
    cnt[tid] = nc;
  }
  __syncthreads();
  if (tid == 0) {
    int s = 0;
    for (int r = 0; r < rows; r++) {
      off[r] = s;
      s += cnt[r];
    }
    off[rows] = s;
  }
  __syncthreads();
  if (tid < rows && rstate[tid]) {
    int o = off[tid];
    if (KNN) {
#pragma unroll
      for (int e = 0; e < L - 1; e++)
        if (id[e] != NONE && (key[e] <= thr || thr != thr)) {
          prow[o] = tid;
          pcid[o] = id[e];
          o++;
        }
    } else {
      const Cand* c = cst + tid * parts * L;
      for (int i = 0; i < parts * L; i++) {
        const Cand v = c[i];
        if (v.id != NONE && (v.key <= thr || thr != thr)) {
          prow[o] = tid;
          pcid[o] = v.id;
          o++;
        }
      }
    }
    if (l2) {
      prow[o] = tid;
      pcid[o] = NONE;
    }
  }
  __syncthreads();
  // One thread per pair runs its chain.
  const int np = off[rows];
  for (int s = tid; s < np; s += 256) {
    const float* xr = x + (size_t)rowid[prow[s]] * d;
    const uint32_t cid = pcid[s];
    pres[s] = cid == NONE ? seq_sq<VEC4>(xr, d) : chain<VEC4>(xr, cents + (size_t)cid * d, d);
  }
  __syncthreads();
  // One thread per row picks the exact best.
  if (tid < rows && rstate[tid]) {
    const int a = off[tid], b = off[tid + 1];
    if (!KNN) {
      float best = INFINITY, xn = 0.f;
      uint32_t bid = NONE;
      for (int s = a; s < b; s++) {
        const uint32_t cid = pcid[s];
        if (cid == NONE) {
          xn = pres[s];
          continue;
        }
        float kx;
        if (ip) {
          kx = -pres[s];
        } else {
          float two = 2.0f * pres[s];
          kx = cnorm[cid] - two;
        }
        if (kx < best || (kx == best && cid < bid)) {
          best = kx;
          bid = cid;
        }
      }
      if (bid == NONE) {
        bid = 0;
        best = INFINITY;
      }
      const size_t p = lo + (size_t)(r0 + tid);
      labels[p] = bid;
      scores[p] = ip ? -best : fmaxf(xn + best, 0.0f);
    } else {
      // Kept set: the kk best by (dot desc, id asc), IEEE; output order: IEEE
      // total order descending, then id (knn.rs:82-103).
      float dv[L];
      uint32_t di[L];
      int m = 0;
      for (int s = a; s < b && m < L; s++) {
        dv[m] = pres[s];
        di[m] = pcid[s];
        m++;
      }
      for (int i = 0; i < m; i++)
        for (int j = i + 1; j < m; j++) {
          bool sw = dv[j] > dv[i] || (dv[j] == dv[i] && di[j] < di[i]);
          if (sw) {
            float t = dv[i]; dv[i] = dv[j]; dv[j] = t;
            uint32_t u = di[i]; di[i] = di[j]; di[j] = u;
          }
        }
      const int kept = m < kk ? m : kk;
      for (int i = 0; i < kept; i++)
        for (int j = i + 1; j < kept; j++) {
          int32_t ki = total_key(dv[i]), kj = total_key(dv[j]);
          bool sw = kj > ki || (kj == ki && di[j] < di[i]);
          if (sw) {
            float t = dv[i]; dv[i] = dv[j]; dv[j] = t;
            uint32_t u = di[i]; di[i] = di[j]; di[j] = u;
          }
        }
      uint32_t* io = labels + (size_t)(r0 + tid) * kk;
      float* so = scores + (size_t)(r0 + tid) * kk;
      for (int e = 0; e < kk; e++) {
        io[e] = e < kept ? di[e] : NONE;
        so[e] = e < kept ? dv[e] : -INFINITY;
      }
    }
  }
}

constexpr int R1 = 16;  // rows per block, top-1
constexpr int RK = 16;  // rows per block, top-k

// ---- Top-1 check with the rows staged through LDS (d % 4 == 0).
//
// Decision per part, without a merge. With thr = best + 2E, le(key) = key <=
// thr || thr is NaN, and lists holding only finite keys (the screen never
// keeps +inf or NaN), a part's list holds every centroid of the part whose
// screen key satisfies le when the list is not full or its last key is above
// thr. The row is settled when some entry is valid, every part is so, and at
// most C1 entries satisfy le; its candidates are then exactly those entries.
// Eight threads per row scan one part's list each and combine with lane
// shuffles.
//
// Chains. The block's settled rows (x) and their candidates (centroid rows)
// are staged in CDC-float chunks into a double-buffered LDS tile by waves 2-3,
// which keep CNR chunks of loads in flight in registers; waves 0-1 run the
// chains from LDS: wave 0 one lane per (row, candidate) fma chain, wave 1 one
// lane per row for the |x|^2 chain (L2). Every chunk costs each wave one
// barrier. Blocks whose rows have more than CCAP candidates in total take
// further passes over the chunks.
constexpr int CR = 32;              // rows per block
constexpr int CCAP = 64;            // candidate slots per pass (one chain lane each)
constexpr int CSLOT = CR + CCAP;    // staged rows per chunk
constexpr int CDC = 64;             // floats per chunk
constexpr int CDC4 = CDC / 4;
constexpr int CDP4 = CDC4 + 1;      // LDS row stride in float4: conflict-free chain reads
constexpr int CNR = 2;              // chunks in flight per loading thread
constexpr int CNQ = CSLOT * CDC4 / 128;  // float4 per loading thread per chunk
static_assert(CSLOT * CDC4 % 128 == 0, "chunk split");

typedef float v4f __attribute__((ext_vector_type(4)));

// f(integral_constant<0>) ... f(integral_constant<N - 1>), in order.
template <int N, typename F>
__device__ __forceinline__ void unroll_steps(F&& f) {
  if constexpr (N > 0) {
    unroll_steps<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

template <int L>
__global__ __launch_bounds__(256) void k_check1(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int nrows, const float* __restrict__ cents, const float* __restrict__ cnorm, int ip,
    const Cand* __restrict__ cand, int parts, const float* __restrict__ xnorm,
    uint32_t* __restrict__ labels, float* __restrict__ scores, uint32_t* __restrict__ fb,
    uint32_t* __restrict__ small, int bound, uint32_t* __restrict__ tcnt,
    uint32_t* __restrict__ tcounts, size_t tlo, size_t tstride) {
  __shared__ v4f stage[2][CSLOT * CDP4];
  __shared__ uint32_t xrow[CR];  // x row of each settled row, NONE otherwise
  __shared__ int rcnt[CR], roff[CR + 1], rset[CR];
  __shared__ uint32_t prow[CR * C1], pcid[CR * C1];
  __shared__ float pdot[CR * C1], pcn[CR * C1], rnorm[CR];
  const int tid = threadIdx.x;
  const int r0 = blockIdx.x * CR;
  const int rows = min(CR, nrows - r0);
  const bool l2 = !ip;
  {
    const int r = tid >> 3, j = tid & 7;
    const bool live = r < rows;
    float key[L];
    uint32_t idv[L];
#pragma unroll
    for (int e = 0; e < L; e++) {
      key[e] = INFINITY;
      idv[e] = NONE;
    }
    uint32_t xid = NONE;
    float xn = 0.f;
    bool badid = false;
    if (live) {
      const size_t p = lo + (size_t)(r0 + r);
      const size_t xi = ids ? (size_t)ids[p] : p;
      badid = xi >= nx;
      xid = badid ? NONE : (uint32_t)xi;
      xn = xnorm[r0 + r];
      if (j < parts) {
        const Cand* c = cand + ((size_t)(r0 + r) * parts + j) * L;
#pragma unroll
        for (int e = 0; e < L; e++) {
          const Cand v = c[e];
          key[e] = v.key;
          idv[e] = v.id;
        }
      }
    }
    // Each list is ascending with its valid entries first: the row's best key
    // is the smallest head.
    float best = idv[0] != NONE ? key[0] : INFINITY;
    int anyv = idv[0] != NONE;
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
      best = fminf(best, __shfl_xor(best, m));
      anyv |= __shfl_xor(anyv, m);
    }
    const bool vrow = live && !badid;
    uint32_t inc = 0;
    int cj = 0, cert = 1;
    if (vrow) {
      const float E = screen_bound(xn, __uint_as_float(small[SW_CMAX2]),
                                   __uint_as_float(small[SW_CNMAX]), d, l2, bound);
      const float thr = best + 2.0f * E;
#pragma unroll
      for (int e = 0; e < L; e++)
        if (idv[e] != NONE && (key[e] <= thr || thr != thr)) {
          inc |= 1u << e;
          cj++;
        }
      // This part's list holds all of its centroids within thr: not full, or
      // its last key above thr (never with a NaN thr).
      cert = idv[L - 1] == NONE || key[L - 1] > thr;
    }
    int tot = cj, incl = cj;
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
      tot += __shfl_xor(tot, m);
      cert &= __shfl_xor(cert, m);
      const int v = __shfl_up(incl, m, 8);
      if (j >= m) incl += v;
    }
    const bool settled = vrow && anyv && cert && tot <= C1;
    if (j == 0) {
      xrow[r] = settled ? xid : NONE;
      rcnt[r] = settled ? tot : 0;
      rset[r] = settled;
      if (live && badid) small[SW_BAD_ID] = 1;
      if (vrow && !settled) {
        const uint32_t f = atomicAdd(&small[SW_FALLBACK_COUNT], 1u);
        fb[f] = (uint32_t)(lo + r0 + r);
      }
    }
    __syncthreads();
    if (tid < 64) {
      int v = tid < CR ? rcnt[tid] : 0;
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) {
        const int u = __shfl_up(v, m);
        if (tid >= m) v += u;
      }
      if (tid < CR) roff[tid + 1] = v;
      if (tid == 0) roff[0] = 0;
    }
    __syncthreads();
    if (settled) {
      int o = roff[r] + incl - cj;
#pragma unroll
      for (int e = 0; e < L; e++)
        if ((inc >> e) & 1u) {
          prow[o] = (uint32_t)r;
          pcid[o] = idv[e];
          o++;
        }
    }
    __syncthreads();
  }
  const int npairs = roff[CR];
  const int d4 = d >> 2;
  const int nch = (d + CDC - 1) / CDC;
  const int wave = tid >> 6, lane = tid & 63;
  for (int pb = 0; pb < npairs; pb += CCAP) {
    const int np = min(CCAP, npairs - pb);
    const bool dl = wave == 0 && lane < np;
    const bool nl = l2 && pb == 0 && wave == 1 && lane < CR && rset[lane];
    float acc = 0.f, nrm = 0.f, cn = 0.f;
    if (wave >= 2) {
      // Loaders. Float4 i of a chunk is slot i / CDC4, column i % CDC4; past
      // the used slots (and past d in the last chunk) the index is clamped, so
      // every thread issues the same loads each step and the waits stay exact.
      const int nlast = (CR + np) * CDC4 - 1;
      const int lt = tid - 128;
      const v4f* src[CNQ];
      int col[CNQ], dst[CNQ];
#pragma unroll
      for (int q = 0; q < CNQ; q++) {
        const int i = min(lt + 128 * q, nlast);
        const int slot = i / CDC4;
        const float* base;
        if (slot < CR) {
          const uint32_t xr = xrow[slot];
          base = x + (size_t)(xr == NONE ? 0u : xr) * d;
        } else {
          base = cents + (size_t)pcid[pb + slot - CR] * d;
        }
        src[q] = reinterpret_cast<const v4f*>(base);
        col[q] = i % CDC4;
        dst[q] = slot * CDP4 + col[q];
      }
      v4f rb[CNR][CNQ];
#pragma unroll
      for (int s = 0; s < CNR; s++)
#pragma unroll
        for (int q = 0; q < CNQ; q++) rb[s][q] = src[q][min(min(s, nch - 1) * CDC4 + col[q], d4 - 1)];
#pragma unroll
      for (int q = 0; q < CNQ; q++) stage[0][dst[q]] = rb[0][q];
#pragma unroll
      for (int q = 0; q < CNQ; q++) rb[0][q] = src[q][min(min(CNR, nch - 1) * CDC4 + col[q], d4 - 1)];
      __syncthreads();
      // Step c stores chunk c + 1 (register set (c + 1) % CNR) and refills
      // that set with chunk c + 1 + CNR; the set index is a constant in each
      // unrolled step, so the sets stay in registers.
      auto step = [&](auto U, int c0) __attribute__((always_inline)) {
        constexpr int s = (decltype(U)::value + 1) % CNR;
        const int c = c0 + decltype(U)::value;
#pragma unroll
        for (int q = 0; q < CNQ; q++) stage[(c + 1) & 1][dst[q]] = rb[s][q];
        const int cn2 = min(c + 1 + CNR, nch - 1);
#pragma unroll
        for (int q = 0; q < CNQ; q++) rb[s][q] = src[q][min(cn2 * CDC4 + col[q], d4 - 1)];
        __syncthreads();
      };
      for (int c0 = 0; c0 < nch; c0 += CNR)
        unroll_steps<CNR>([&](auto U) __attribute__((always_inline)) { step(U, c0); });
    } else {
      const int xs = dl ? (int)prow[pb + lane] : (nl ? lane : 0);
      const int cs = CR + (dl ? lane : 0);
      if (dl && l2) cn = cnorm[pcid[pb + lane]];
      __syncthreads();
      // As many barriers as the loaders: nch rounded up to a multiple of CNR.
      const int nsteps = (nch + CNR - 1) / CNR * CNR;
      for (int c = 0; c < nsteps; c++) {
        if (c < nch) {
          const int n4 = min(CDC4, d4 - c * CDC4);
          const v4f* xp = &stage[c & 1][xs * CDP4];
          if (dl) {
            const v4f* cp = &stage[c & 1][cs * CDP4];
            if (n4 == CDC4) {
              // The chunk's operands are read into registers before the
              // chain starts, so the chain waits for LDS once per chunk
              // rather than once per four fmas.
              v4f xa[CDC4], wa[CDC4];
#pragma unroll
              for (int f = 0; f < CDC4; f++) {
                xa[f] = xp[f];
                wa[f] = cp[f];
              }
              __builtin_amdgcn_sched_barrier(0);
#pragma unroll
              for (int f = 0; f < CDC4; f++) {
                acc = fmaf(xa[f].x, wa[f].x, acc);
                acc = fmaf(xa[f].y, wa[f].y, acc);
                acc = fmaf(xa[f].z, wa[f].z, acc);
                acc = fmaf(xa[f].w, wa[f].w, acc);
              }
            } else {
              for (int f = 0; f < n4; f++) {
                const v4f a = xp[f], w = cp[f];
                acc = fmaf(a.x, w.x, acc);
                acc = fmaf(a.y, w.y, acc);
                acc = fmaf(a.z, w.z, acc);
                acc = fmaf(a.w, w.w, acc);
              }
            }
          } else if (nl) {
            if (n4 == CDC4) {
              v4f xa[CDC4];
#pragma unroll
              for (int f = 0; f < CDC4; f++) xa[f] = xp[f];
              __builtin_amdgcn_sched_barrier(0);
#pragma unroll
              for (int f = 0; f < CDC4; f++) {
                const v4f a = xa[f];
                const float p0 = a.x * a.x, p1 = a.y * a.y, p2 = a.z * a.z, p3 = a.w * a.w;
                nrm = nrm + p0;
                nrm = nrm + p1;
                nrm = nrm + p2;
                nrm = nrm + p3;
              }
            } else {
              for (int f = 0; f < n4; f++) {
                const v4f a = xp[f];
                const float p0 = a.x * a.x, p1 = a.y * a.y, p2 = a.z * a.z, p3 = a.w * a.w;
                nrm = nrm + p0;
                nrm = nrm + p1;
                nrm = nrm + p2;
                nrm = nrm + p3;
              }
            }
          }
        }
        __syncthreads();
      }
    }
    if (dl) {
      pdot[pb + lane] = acc;
      pcn[pb + lane] = cn;
    }
    if (nl) rnorm[lane] = nrm;
    __syncthreads();
  }
  // One thread per settled row picks the exact best (ties to the lower id).
  uint32_t mylab = NONE;
  if (tid < rows && rset[tid]) {
    const int a = roff[tid], b = roff[tid + 1];
    float bk = INFINITY;
    uint32_t bid = NONE;
    for (int s = a; s < b; s++) {
      const uint32_t cid = pcid[s];
      float kx;
      if (ip) {
        kx = -pdot[s];
      } else {
        const float two = 2.0f * pdot[s];
        kx = pcn[s] - two;
      }
      if (kx < bk || (kx == bk && cid < bid)) {
        bk = kx;
        bid = cid;
      }
    }
    if (bid == NONE) {
      bid = 0;
      bk = INFINITY;
    }
    const size_t p = lo + (size_t)(r0 + tid);
    labels[p] = bid;
    scores[p] = ip ? -bk : fmaxf(rnorm[tid] + bk, 0.0f);
    mylab = bid;
  }
  if (tcnt) {
    // The tally: the block's rows lie in one chunk of TALLY_CP positions (lo
    // - tlo is a multiple of it), so the first row of each label adds the
    // label's rows in the block, one atomic per (block, label) on each word.
    __shared__ uint32_t tl[CR];
    if (tid < CR) tl[tid] = mylab;
    __syncthreads();
    if (tid < CR && mylab != NONE) {
      uint32_t cntl = 0;
      bool first = true;
      for (int j = 0; j < CR; j++) {
        const bool same = tl[j] == mylab;
        cntl += same;
        first = first && !(same && j < tid);
      }
      if (first) {
        const size_t ch = (lo - tlo + (size_t)r0) / TALLY_CP;
        atomicAdd(&tcnt[(size_t)mylab * tstride + ch], cntl);
        atomicAdd(&tcounts[mylab], cntl);
      }
    }
  }
}

// One thread per list entry: the entry's exact key (the check's fma chain
// over t = 0..d-1 from +0; IP -dot, L2 cnorm - 2 dot) against its screen key.
// out[0]: entries measured; out[1]: entries beyond E; out[2]: the largest
// |screen key - exact key| / E; out[3]: the largest dot error over the bound's
// dot term, after the allowances that are IEEE rounding (L2: one rounding of
// each key) or the tag (tagged keys): max(0, |dk| - u(|ks| + |ke|) - 2^-17 |ks|)
// / ((2 for L2) edot). Ratios are f32 bits (>= 0, so their bits order as the
// values). Entries with a non-finite key or bound are not measured (their rows
// go to the exact scan).
__global__ __launch_bounds__(256) void k_margin(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    size_t nrows, const float* __restrict__ cents, const float* __restrict__ cnorm, int ip,
    const Cand* __restrict__ cand, int per_row, const float* __restrict__ xnorm,
    const uint32_t* __restrict__ small, int bound, unsigned long long* __restrict__ out) {
  const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nrows * (size_t)per_row) return;
  const size_t r = e / (size_t)per_row;
  const Cand cd = cand[e];
  if (cd.id == NONE || !isfinite(cd.key)) return;
  const size_t p = lo + r;
  const size_t xi = ids ? (size_t)ids[p] : p;
  if (xi >= nx) return;
  const float* xr = x + xi * (size_t)d;
  const float* cr = cents + (size_t)cd.id * d;
  float acc = 0.f;
  for (int t = 0; t < d; t++) acc = fmaf(xr[t], cr[t], acc);
  const float kx = ip ? -acc : cnorm[cd.id] - 2.0f * acc;
  float edot = 0.f;
  const float E = screen_bound(xnorm[r], __uint_as_float(small[SW_CMAX2]),
                               __uint_as_float(small[SW_CNMAX]), d, !ip, bound, &edot);
  if (!isfinite(kx) || !isfinite(E) || !(E > 0.f) || !(edot > 0.f)) return;
  const float dk = fabsf(cd.key - kx);
  const float ratio = dk / E;
  const float u = 5.9604645e-08f;
  const float allow = (ip ? 0.f : 1.0000002f * u * (fabsf(cd.key) + fabsf(kx))) +
                      (bound == BOUND_BF16_TAGGED || bound == BOUND_F16_TAGGED
                           ? 7.63e-6f * fabsf(cd.key) + 8.9e-44f
                           : 0.f);
  const float dot_ratio = fmaxf(dk - allow, 0.f) / ((ip ? 1.0f : 2.0f) * edot);
  atomicAdd(&out[0], 1ull);
  if (ratio > 1.0f) atomicAdd(&out[1], 1ull);
  atomicMax(&out[2], (unsigned long long)__float_as_uint(ratio));
  atomicMax(&out[3], (unsigned long long)__float_as_uint(dot_ratio));
}

}  // namespace

void launch_margin(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                   size_t lo, size_t n, const float* cents, const float* cnorm, bool ip,
                   const Cand* cand, int parts, int L, const float* xnorm, int bound,
                   emh_screen_report* rep) {
  unsigned long long* w = nullptr;
  EMH_HIP(hipMalloc(&w, 4 * sizeof(unsigned long long)));
  unsigned long long h[4] = {0, 0, 0, 0};
  try {
    EMH_HIP(hipMemcpyAsync(w, h, sizeof h, hipMemcpyHostToDevice, c->stream));
    const size_t total = n * (size_t)parts * L;
    hipLaunchKernelGGL(k_margin, grid1(total, 256), dim3(256), 0, c->stream, x, nx, (int)d, ids,
                       lo, n, cents, cnorm, ip ? 1 : 0, cand, parts * L, xnorm, c->small, bound,
                       w);
    EMH_HIP(hipGetLastError());
    EMH_HIP(hipMemcpyAsync(h, w, sizeof h, hipMemcpyDeviceToHost, c->stream));
    EMH_HIP(hipStreamSynchronize(c->stream));
  } catch (...) {
    (void)hipFree(w);
    throw;
  }
  EMH_HIP(hipFree(w));
  uint32_t bits[2] = {(uint32_t)h[2], (uint32_t)h[3]};
  float mr[2];
  std::memcpy(mr, bits, 8);
  rep->pairs = h[0];
  rep->over = h[1];
  rep->max_ratio = mr[0];
  rep->max_dot_ratio = mr[1];
}

void launch_verify1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                    size_t lo, size_t n, const float* cents, const float* cnorm, size_t k, bool ip,
                    const Cand* cand, int parts, const float* xnorm, uint32_t* labels,
                    float* scores, uint32_t* fb, int bound, const LabelTally* tally, int L) {
  const dim3 g((unsigned)((n + R1 - 1) / R1));
  static_assert(TALLY_CP % CR == 0, "a check block's rows lie in one tally chunk");
  EMH_ENSURE(!tally || (d % 4 == 0 && lo >= tally->lo && (lo - tally->lo) % TALLY_CP == 0),
             "check: a tally needs d %% 4 == 0 and chunk-aligned positions");
  EMH_ENSURE(L == L1 || L == L1F || (L == L1S && d % 4 == 0), "check: lists of %d entries", L);
  if (d % 4 == 0)
    hipLaunchKernelGGL(L == L1S ? k_check1<L1S> : L == L1F ? k_check1<L1F> : k_check1<L1>,
                       dim3((unsigned)((n + CR - 1) / CR)), dim3(256), 0, c->stream, x,
                       nx, (int)d, ids, lo, (int)n, cents, cnorm, ip ? 1 : 0, cand, parts, xnorm,
                       labels, scores, fb, c->small, bound, tally ? tally->cnt : nullptr,
                       tally ? tally->counts : nullptr, tally ? tally->lo : 0,
                       tally ? tally->stride : 0);
  else
    hipLaunchKernelGGL((L == L1F ? k_verify<L1F, R1, false, false> : k_verify<L1, R1, false, false>),
                       g, dim3(256), 0, c->stream, x, nx, (int)d, ids, lo, (int)n, cents, cnorm,
                       (int)k, ip ? 1 : 0, 1, cand, parts, xnorm, labels, scores, fb, c->small,
                       bound);
  EMH_HIP(hipGetLastError());
}

void launch_verifyk(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                    size_t kk, const Cand* cand, int parts, const float* xnorm, uint32_t* ids,
                    float* sims, uint32_t* fb) {
  const dim3 g((unsigned)((m + RK - 1) / RK));
  const int bound = c->screen == SCREEN_F32 ? BOUND_F32 : BOUND_BF16;
  if (d % 4 == 0)
    hipLaunchKernelGGL((k_verify<LK, RK, true, true>), g, dim3(256), 0, c->stream, q, m, (int)d,
                       nullptr, (size_t)0, (int)m, data, nullptr, (int)n, 1, (int)kk, cand, parts,
                       xnorm, ids, sims, fb, c->small, bound);
  else
    hipLaunchKernelGGL((k_verify<LK, RK, true, false>), g, dim3(256), 0, c->stream, q, m,
                       (int)d, nullptr, (size_t)0, (int)m, data, nullptr, (int)n, 1, (int)kk,
                       cand, parts, xnorm, ids, sims, fb, c->small, bound);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
