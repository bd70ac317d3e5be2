// The exact stages behind the MFMA screen (emh_screen.hip, which also gathers
// the error bound's inputs max_j |c_j|^2 and max_j cnorm[j]):
//
//  k_verify    per block of up to 16 rows staged in LDS: merge the parts'
//              candidate lists, bound the screen error, and either queue the
//              row for the exact scan or re-score its candidates with the
//              reference's fma chain, one thread per (row, candidate) pair;
//  k_exact_*   the exact scan of queued rows over all centroids, split into
//              (8 rows x 64 centroids) items so that a handful of rows still
//              spreads over the whole chip, then a per-row reduction.
//
// Float order (the reference CPU backend, assign/fused.rs + assign.rs):
// dot = fma chain over t = 0..d-1 from +0; L2 key = cnorm[j] - 2 dot (two
// roundings); |x|^2 = sequential sum of rounded squares; score = dot (IP) or
// max(|x|^2 + key, 0) (L2); ties to the lower id; a key that is NaN or +inf
// never wins, and a row where nothing wins gets label 0 and the initial score.

#include "emh_select.h"

namespace emh {
namespace {

constexpr int WAVE = 64;
constexpr int RMAX = 16;  // rows per verify block


// Exact fma chain of an LDS row with a global row (the cpu-fused dot), with
// the global loads issued 16 float4 ahead.
template <bool VEC4>
__device__ __forceinline__ float chain(const float* xr, const float* cr, int d) {
  float acc = 0.f;
  if (VEC4) {
    const float4* c4 = reinterpret_cast<const float4*>(cr);
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    const int d4 = d >> 2;
    int t = 0;
    for (; t + 16 <= d4; t += 16) {
      float4 v[16];
#pragma unroll
      for (int u = 0; u < 16; u++) v[u] = c4[t + u];
#pragma unroll
      for (int u = 0; u < 16; u++) {
        float4 xv = x4[t + u];
        acc = fmaf(xv.x, v[u].x, acc);
        acc = fmaf(xv.y, v[u].y, acc);
        acc = fmaf(xv.z, v[u].z, acc);
        acc = fmaf(xv.w, v[u].w, acc);
      }
    }
    for (; t < d4; t++) {
      float4 v = c4[t], xv = x4[t];
      acc = fmaf(xv.x, v.x, acc);
      acc = fmaf(xv.y, v.y, acc);
      acc = fmaf(xv.z, v.z, acc);
      acc = fmaf(xv.w, v.w, acc);
    }
  } else {
    for (int t = 0; t < d; t++) acc = fmaf(xr[t], cr[t], acc);
  }
  return acc;
}

// --------------------------------------------------------------- verify
// Block: 256 threads, R <= 32 rows (positions lo + r0 .. lo + r0 + R) staged in
// LDS with row stride XS (d + 4 for VEC4, else d + 1, so rows fall on
// different banks). KNN: rows are queries, "centroids" the data rows, and
// the kk best by exact dot are written per query.
template <int L, bool KNN, bool VEC4>
__global__ __launch_bounds__(256) void k_verify(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int nrows, const float* __restrict__ cents, const float* __restrict__ cnorm, int k, int ip,
    int kk, const Cand* __restrict__ cand, int parts, int R, uint32_t* __restrict__ labels,
    float* __restrict__ scores, uint32_t* __restrict__ fb, uint32_t* __restrict__ small) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  constexpr int PMAX = RMAX * L;
  __shared__ uint32_t prow[PMAX], pcid[PMAX];
  __shared__ float pres[PMAX];
  __shared__ Cand cst[RMAX * MAX_PARTS * L];
  __shared__ float xnb[RMAX];
  __shared__ int cnt[RMAX], off[RMAX + 1];
  __shared__ uint32_t rowid[RMAX];
  __shared__ int rstate[RMAX];
  const int XS = VEC4 ? d + 4 : d + 1;
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
  __syncthreads();
  // Phase 0: the rows into LDS (coalesced, 8 loads in flight per thread).
  if (VEC4) {
    const int d4 = d >> 2, total = rows * d4;
    for (int i0 = tid; i0 < total; i0 += 256 * 8) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int i = i0 + 256 * u;
        v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < total) {
          const int r = i / d4, c = i - r * d4;
          const uint32_t xid = rowid[r];
          if (xid != NONE) v[u] = reinterpret_cast<const float4*>(x + (size_t)xid * d)[c];
        }
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int i = i0 + 256 * u;
        if (i < total) {
          const int r = i / d4, c = i - r * d4;
          *reinterpret_cast<float4*>(&xs[r * XS + 4 * c]) = v[u];
        }
      }
    }
  } else {
    for (int i = tid; i < rows * d; i += 256) {
      const int r = i / d, c = i - r * d;
      const uint32_t xid = rowid[r];
      xs[r * XS + c] = xid != NONE ? x[(size_t)xid * d + c] : 0.f;
    }
  }
  __syncthreads();
  // Phase 1: |x|^2 in any order for the bound (8 threads per row).
  {
    const int r = tid >> 3, part = tid & 7;
    float s = 0.f;
    if (r < rows)
      for (int t = part; t < d; t += 8) {
        float v = xs[r * XS + t];
        s += v * v;
      }
    s += __shfl_xor(s, 1, WAVE);
    s += __shfl_xor(s, 2, WAVE);
    s += __shfl_xor(s, 4, WAVE);
    if (part == 0 && r < rows) xnb[r] = s;
  }
  __syncthreads();
  // Phase 2: the block's candidate lists (rows x parts x L, contiguous) into
  // LDS; then one thread per row decides and lists its (row, candidate) pairs.
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
  float key[L];
  uint32_t id[L];
  float thr = 0.f;
  if (tid < rows) {
    merge_parts<L>(cst + tid * parts * L, parts, key, id);
    int state = 0, nc = 0;
    if (rowid[tid] != NONE) {
      const float E = screen_bound(xnb[tid], __uint_as_float(small[SW_CMAX2]),
                                   __uint_as_float(small[SW_CNMAX]), d, l2);
      thr = (KNN ? key[kk - 1] : key[0]) + 2.0f * E;
      const bool complete = KNN ? (id[L - 1] == NONE || key[L - 1] > thr)
                                : (id[0] != NONE && (id[L - 1] == NONE || key[L - 1] > thr));
      if (complete) {
        state = 1;
#pragma unroll
        for (int e = 0; e < L - 1; e++) nc += id[e] != NONE && (key[e] <= thr || thr != thr);
        nc += l2;
      } else {
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
#pragma unroll
    for (int e = 0; e < L - 1; e++)
      if (id[e] != NONE && (key[e] <= thr || thr != thr)) {
        prow[o] = tid;
        pcid[o] = id[e];
        o++;
      }
    if (l2) {
      prow[o] = tid;
      pcid[o] = NONE;
    }
  }
  __syncthreads();
  // Phase 3: one thread per pair runs its chain.
  const int np = off[rows];
  for (int s = tid; s < np; s += 256) {
    const float* xr = xs + prow[s] * XS;
    const uint32_t cid = pcid[s];
    float acc = 0.f;
    if (cid == NONE) {
      for (int t = 0; t < d; t++) {
        float q2 = xr[t] * xr[t];
        acc = acc + q2;
      }
    } else {
      acc = chain<VEC4>(xr, cents + (size_t)cid * d, d);
    }
    pres[s] = acc;
  }
  __syncthreads();
  // Phase 4: one thread per row picks the exact best.
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

// ------------------------------------------------------------- exact top-1
// Item = (group of RG rows, chunk of CJ centroids): one wave, lane = centroid,
// RG chains per lane over d in tiles of TD dimensions staged in LDS.
constexpr int CJ = 64, RG = 8, TD = 64;

template <bool VEC4>
__global__ __launch_bounds__(64) void k_exact_part(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int n_direct, const uint32_t* __restrict__ list, const uint32_t* __restrict__ small,
    const float* __restrict__ cents, const float* __restrict__ cnorm, int k, int ip,
    Cand* __restrict__ partial) {
  __shared__ float ct[CJ][TD + 1];
  __shared__ __attribute__((aligned(16))) float xt[RG][TD];
  __shared__ uint32_t xid_s[RG];
  const int nrows = list ? (int)small[SW_FALLBACK_COUNT] : n_direct;
  const int nch = (k + CJ - 1) / CJ;
  const int ngr = (nrows + RG - 1) / RG;
  const int lane = threadIdx.x;
  for (int item = blockIdx.x; item < ngr * nch; item += gridDim.x) {
    const int g = item / nch, q = item - g * nch;
    if (lane < RG) {
      const int f = g * RG + lane;
      uint32_t xid = NONE;
      if (f < nrows) {
        const size_t p = list ? (size_t)list[f] : lo + (size_t)f;
        const size_t id = ids ? (size_t)ids[p] : p;
        xid = id < nx ? (uint32_t)id : NONE;
      }
      xid_s[lane] = xid;
    }
    __syncthreads();
    const int j = q * CJ + lane;
    float acc[RG];
#pragma unroll
    for (int r = 0; r < RG; r++) acc[r] = 0.f;
    for (int t0 = 0; t0 < d; t0 += TD) {
      const int tl = min(TD, d - t0);
      for (int i = lane; i < CJ * (TD / 4); i += WAVE) {
        const int r = i / (TD / 4), c4 = i % (TD / 4);
        const int jj = min(q * CJ + r, k - 1);
        const float* cr = cents + (size_t)jj * d;
        const int col = t0 + 4 * c4;
        float4 v;
        if (VEC4 && col + 4 <= d) {
          v = *reinterpret_cast<const float4*>(cr + col);
        } else {
          v.x = col + 0 < d ? cr[col + 0] : 0.f;
          v.y = col + 1 < d ? cr[col + 1] : 0.f;
          v.z = col + 2 < d ? cr[col + 2] : 0.f;
          v.w = col + 3 < d ? cr[col + 3] : 0.f;
        }
        ct[r][4 * c4 + 0] = v.x;
        ct[r][4 * c4 + 1] = v.y;
        ct[r][4 * c4 + 2] = v.z;
        ct[r][4 * c4 + 3] = v.w;
      }
      for (int i = lane; i < RG * TD; i += WAVE) {
        const int r = i / TD, c = i % TD;
        const uint32_t xid = xid_s[r];
        xt[r][c] = (xid != NONE && t0 + c < d) ? x[(size_t)xid * d + t0 + c] : 0.f;
      }
      __syncthreads();
      for (int tt = 0; tt < tl; tt++) {
        const float cv = ct[lane][tt];
#pragma unroll
        for (int r = 0; r < RG; r++) acc[r] = fmaf(xt[r][tt], cv, acc[r]);
      }
      __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < RG; r++) {
      float kx = INFINITY;
      uint32_t id = NONE;
      if (j < k && xid_s[r] != NONE) {
        if (ip) {
          kx = -acc[r];
        } else {
          float two = 2.0f * acc[r];
          kx = cnorm[j] - two;
        }
        id = (uint32_t)j;
        if (!(kx < INFINITY)) {  // NaN or +inf never wins
          kx = INFINITY;
          id = NONE;
        }
      }
      for (int o = 32; o > 0; o >>= 1) {
        float k2 = __shfl_xor(kx, o, WAVE);
        uint32_t i2 = __shfl_xor(id, o, WAVE);
        if (k2 < kx || (k2 == kx && i2 < id)) {
          kx = k2;
          id = i2;
        }
      }
      const int f = g * RG + r;
      if (lane == 0 && f < nrows) partial[(size_t)f * nch + q] = Cand{kx, id};
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void k_exact_final(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int n_direct, const uint32_t* __restrict__ list, uint32_t* __restrict__ small, int k, int ip,
    const Cand* __restrict__ partial, uint32_t* __restrict__ labels, float* __restrict__ scores) {
  const int nrows = list ? (int)small[SW_FALLBACK_COUNT] : n_direct;
  const int nch = (k + CJ - 1) / CJ;
  if (list && blockIdx.x == 0 && threadIdx.x == 0) small[SW_FALLBACK_TOTAL] += (uint32_t)nrows;
  for (int f = blockIdx.x * blockDim.x + threadIdx.x; f < nrows; f += gridDim.x * blockDim.x) {
    const size_t p = list ? (size_t)list[f] : lo + (size_t)f;
    const size_t xid = ids ? (size_t)ids[p] : p;
    if (xid >= nx) {
      small[SW_BAD_ID] = 1;
      continue;
    }
    float best = INFINITY;
    uint32_t bid = NONE;
    for (int q = 0; q < nch; q++) {
      const Cand c = partial[(size_t)f * nch + q];
      if (c.id != NONE && (c.key < best || (c.key == best && c.id < bid))) {
        best = c.key;
        bid = c.id;
      }
    }
    if (bid == NONE) {
      bid = 0;
      best = INFINITY;
    }
    labels[p] = bid;
    if (ip) {
      scores[p] = -best;
    } else {
      const float* xr = x + xid * (size_t)d;
      float xn = 0.f;
      for (int t = 0; t < d; t++) {
        float q2 = xr[t] * xr[t];
        xn = xn + q2;
      }
      scores[p] = fmaxf(xn + best, 0.0f);
    }
  }
}

// ------------------------------------------------------------- exact top-k
// One workgroup per queued query: each thread keeps the kk best of its strided
// share (j increasing, replace the worst only when strictly better, as
// knn.rs:82-96), then the workgroup picks the kk best of the 256 lists.
__global__ __launch_bounds__(256) void k_exactk(const float* __restrict__ q, int d,
                                                const float* __restrict__ data, int n, int kk,
                                                int exclude_self, const uint32_t* __restrict__ list,
                                                uint32_t* __restrict__ small,
                                                uint32_t* __restrict__ ids_out,
                                                float* __restrict__ sims_out) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  __shared__ float sk[256 * KMAX];
  __shared__ uint32_t si[256 * KMAX];
  __shared__ float wbest[4];
  __shared__ uint32_t wbid[4];
  __shared__ int wslot[4];
  const size_t nrows = small[SW_FALLBACK_COUNT];
  if (blockIdx.x == 0 && threadIdx.x == 0) small[SW_FALLBACK_TOTAL] += (uint32_t)nrows;
  for (size_t f = blockIdx.x; f < nrows; f += gridDim.x) {
    const size_t r = list[f];
    const float* qr = q + r * (size_t)d;
    for (int t = threadIdx.x; t < d; t += blockDim.x) xs[t] = qr[t];
    __syncthreads();
    float sc[KMAX];
    uint32_t ii[KMAX];
    for (int e = 0; e < KMAX; e++) {
      sc[e] = -INFINITY;
      ii[e] = NONE;
    }
    int worst = 0;
    for (int j = threadIdx.x; j < n; j += blockDim.x) {
      if (exclude_self && (size_t)j == r) continue;
      const float* c = data + (size_t)j * d;
      float a = 0.f;
      for (int t = 0; t < d; t++) a = fmaf(xs[t], c[t], a);
      if (a > sc[worst]) {
        sc[worst] = a;
        ii[worst] = (uint32_t)j;
        worst = 0;
        for (int e = 1; e < kk; e++) {
          bool worse = sc[e] < sc[worst] || (sc[e] == sc[worst] && ii[e] > ii[worst]);
          if (worse) worst = e;
        }
      }
    }
    for (int e = 0; e < KMAX; e++) {
      sk[threadIdx.x * KMAX + e] = e < kk ? sc[e] : -INFINITY;
      si[threadIdx.x * KMAX + e] = e < kk ? ii[e] : NONE;
    }
    __syncthreads();
    float outd[KMAX];
    uint32_t outi[KMAX];
    int got = 0;
    for (int e = 0; e < kk; e++) {
      float b = -INFINITY;
      uint32_t bi = NONE;
      int slot = -1;
      for (int s = threadIdx.x; s < 256 * KMAX; s += blockDim.x) {
        const uint32_t j = si[s];
        if (j == NONE) continue;
        const float v = sk[s];
        if (slot < 0 || v > b || (v == b && j < bi)) {
          b = v;
          bi = j;
          slot = s;
        }
      }
      for (int o = 32; o > 0; o >>= 1) {
        float b2 = __shfl_xor(b, o, WAVE);
        uint32_t i2 = __shfl_xor(bi, o, WAVE);
        int s2 = __shfl_xor(slot, o, WAVE);
        if (s2 >= 0 && (slot < 0 || b2 > b || (b2 == b && i2 < bi))) {
          b = b2;
          bi = i2;
          slot = s2;
        }
      }
      if ((threadIdx.x & 63) == 0) {
        wbest[threadIdx.x >> 6] = b;
        wbid[threadIdx.x >> 6] = bi;
        wslot[threadIdx.x >> 6] = slot;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        int bw = -1;
        for (int w = 0; w < 4; w++) {
          if (wslot[w] < 0) continue;
          if (bw < 0 || wbest[w] > wbest[bw] || (wbest[w] == wbest[bw] && wbid[w] < wbid[bw]))
            bw = w;
        }
        wslot[0] = bw < 0 ? -1 : wslot[bw];
        wbest[0] = bw < 0 ? -INFINITY : wbest[bw];
        wbid[0] = bw < 0 ? NONE : wbid[bw];
        if (bw >= 0) si[wslot[0]] = NONE;
      }
      __syncthreads();
      if (wslot[0] >= 0) {
        outd[got] = wbest[0];
        outi[got] = wbid[0];
        got++;
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      // Output order: IEEE total order descending, then id.
      for (int a = 0; a < got; a++)
        for (int b = a + 1; b < got; b++) {
          int32_t ka = total_key(outd[a]), kb = total_key(outd[b]);
          if (kb > ka || (kb == ka && outi[b] < outi[a])) {
            float t = outd[a]; outd[a] = outd[b]; outd[b] = t;
            uint32_t u = outi[a]; outi[a] = outi[b]; outi[b] = u;
          }
        }
      for (int e = 0; e < kk; e++) {
        ids_out[r * kk + e] = e < got ? outi[e] : NONE;
        sims_out[r * kk + e] = e < got ? outd[e] : -INFINITY;
      }
    }
    __syncthreads();
  }
}

int verify_rows(size_t d) {  // rows per verify block: <= RMAX (3 blocks per CU at d = 768)
  size_t xs = d + 4;
  return (int)std::max<size_t>(1, std::min<size_t>(RMAX, 32768 / xs));
}

}  // namespace

void launch_verify1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                    size_t lo, size_t n, const float* cents, const float* cnorm, size_t k, bool ip,
                    const Cand* cand, int parts, uint32_t* labels, float* scores, uint32_t* fb) {
  const int R = verify_rows(d);
  const bool vec4 = d % 4 == 0;
  const size_t lds = (size_t)R * (vec4 ? d + 4 : d + 1) * sizeof(float);
  const dim3 g((unsigned)((n + R - 1) / R));
  if (vec4)
    hipLaunchKernelGGL((k_verify<L1, false, true>), g, dim3(256), lds, c->stream, x, nx, (int)d,
                       ids, lo, (int)n, cents, cnorm, (int)k, ip ? 1 : 0, 1, cand, parts, R,
                       labels, scores, fb, c->small);
  else
    hipLaunchKernelGGL((k_verify<L1, false, false>), g, dim3(256), lds, c->stream, x, nx, (int)d,
                       ids, lo, (int)n, cents, cnorm, (int)k, ip ? 1 : 0, 1, cand, parts, R,
                       labels, scores, fb, c->small);
  EMH_HIP(hipGetLastError());
}

void launch_exact1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                   size_t lo, size_t n, const uint32_t* list, const float* cents,
                   const float* cnorm, size_t k, bool ip, uint32_t* labels, float* scores) {
  if (n == 0) return;
  const size_t nch = (k + CJ - 1) / CJ;
  Cand* partial = (Cand*)c->knn_tmp.get(n * nch * sizeof(Cand));
  // Queued rows: the count lives on the device, so the grid covers the worst case.
  const size_t items = ((n + RG - 1) / RG) * nch;
  // Queued rows are few: a grid of 2 blocks per CU covers them, and blocks
  // past the device-side count exit at once.
  const unsigned g = (unsigned)std::min<size_t>(items, (size_t)(list ? 2 : 8) * c->cus);
  if (d % 4 == 0)
    hipLaunchKernelGGL(k_exact_part<true>, dim3(g), dim3(64), 0, c->stream, x, nx, (int)d, ids,
                       lo, (int)n, list, c->small, cents, cnorm, (int)k, ip ? 1 : 0, partial);
  else
    hipLaunchKernelGGL(k_exact_part<false>, dim3(g), dim3(64), 0, c->stream, x, nx, (int)d, ids,
                       lo, (int)n, list, c->small, cents, cnorm, (int)k, ip ? 1 : 0, partial);
  EMH_HIP(hipGetLastError());
  const unsigned g2 = (unsigned)std::min<size_t>((n + 255) / 256, (size_t)4 * c->cus);
  hipLaunchKernelGGL(k_exact_final, dim3(g2), dim3(256), 0, c->stream, x, nx, (int)d, ids, lo,
                     (int)n, list, c->small, (int)k, ip ? 1 : 0, partial, labels, scores);
  EMH_HIP(hipGetLastError());
}

void launch_verifyk(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                    size_t kk, const Cand* cand, int parts, uint32_t* ids, float* sims,
                    uint32_t* fb) {
  const int R = verify_rows(d);
  const bool vec4 = d % 4 == 0;
  const size_t lds = (size_t)R * (vec4 ? d + 4 : d + 1) * sizeof(float);
  const dim3 g((unsigned)((m + R - 1) / R));
  if (vec4)
    hipLaunchKernelGGL((k_verify<LK, true, true>), g, dim3(256), lds, c->stream, q, m, (int)d,
                       nullptr, (size_t)0, (int)m, data, nullptr, (int)n, 1, (int)kk, cand, parts,
                       R, ids, sims, fb, c->small);
  else
    hipLaunchKernelGGL((k_verify<LK, true, false>), g, dim3(256), lds, c->stream, q, m, (int)d,
                       nullptr, (size_t)0, (int)m, data, nullptr, (int)n, 1, (int)kk, cand, parts,
                       R, ids, sims, fb, c->small);
  EMH_HIP(hipGetLastError());
}

void launch_exactk(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                   size_t kk, bool exclude_self, const uint32_t* fb, uint32_t* ids, float* sims) {
  (void)m;
  hipLaunchKernelGGL(k_exactk, dim3(2 * c->cus), dim3(256), d * sizeof(float), c->stream, q,
                     (int)d, data, (int)n, (int)kk, exclude_self ? 1 : 0, fb, c->small, ids, sims);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
