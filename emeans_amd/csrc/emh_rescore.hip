// The check behind the MFMA screen (emh_screen.hip): per row, merge the
// centroid parts' candidate lists, bound the screen's error, and either queue
// the row for the exact scan (emh_verify.hip) or re-score its candidates with
// the reference's float order:
//   dot = one fma chain over t = 0..d-1 from +0 (assign/fused.rs:241-260);
//   L2 key = cnorm[j] - 2 dot (two roundings, assign.rs:461);
//   |x|^2 = sequential sum of rounded squares (assign.rs:150-155);
//   score = dot (IP) or max(|x|^2 + key, 0) (L2, assign.rs:497-502);
//   ties to the lower id.
// One thread per (row, candidate) pair runs a chain, reading the row and the
// candidate from global memory (L2/MALL-resident after the screen) with PF
// float4 loads of each in flight; the small LDS footprint keeps many blocks
// per CU so the chains' latency overlaps.

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
    uint32_t* __restrict__ small) {
  constexpr int PMAX = R * L;
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
  // One thread per row: merge (each part's list is ascending, so a part is
  // done at its first entry not below the current L-th key), bound, decide.
  float key[L];
  uint32_t id[L];
  float thr = 0.f;
  if (tid < rows) {
#pragma unroll
    for (int e = 0; e < L; e++) {
      key[e] = INFINITY;
      id[e] = NONE;
    }
    const Cand* c = cst + tid * parts * L;
    for (int q = 0; q < parts; q++)
      for (int e = 0; e < L; e++) {
        const Cand v = c[q * L + e];
        if (v.id == NONE || !(v.key < key[L - 1])) break;
        insert<L>(key, id, v.key, v.id);
      }
    int state = 0, nc = 0;
    if (rowid[tid] != NONE) {
      const float E = screen_bound(xnorm[r0 + tid], __uint_as_float(small[SW_CMAX2]),
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

}  // namespace

void launch_verify1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                    size_t lo, size_t n, const float* cents, const float* cnorm, size_t k, bool ip,
                    const Cand* cand, int parts, const float* xnorm, uint32_t* labels,
                    float* scores, uint32_t* fb) {
  const dim3 g((unsigned)((n + R1 - 1) / R1));
  if (d % 4 == 0)
    hipLaunchKernelGGL((k_verify<L1, R1, false, true>), g, dim3(256), 0, c->stream, x, nx,
                       (int)d, ids, lo, (int)n, cents, cnorm, (int)k, ip ? 1 : 0, 1, cand, parts,
                       xnorm, labels, scores, fb, c->small);
  else
    hipLaunchKernelGGL((k_verify<L1, R1, false, false>), g, dim3(256), 0, c->stream, x, nx,
                       (int)d, ids, lo, (int)n, cents, cnorm, (int)k, ip ? 1 : 0, 1, cand, parts,
                       xnorm, labels, scores, fb, c->small);
  EMH_HIP(hipGetLastError());
}

void launch_verifyk(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                    size_t kk, const Cand* cand, int parts, const float* xnorm, uint32_t* ids,
                    float* sims, uint32_t* fb) {
  const dim3 g((unsigned)((m + RK - 1) / RK));
  if (d % 4 == 0)
    hipLaunchKernelGGL((k_verify<LK, RK, true, true>), g, dim3(256), 0, c->stream, q, m, (int)d,
                       nullptr, (size_t)0, (int)m, data, nullptr, (int)n, 1, (int)kk, cand, parts,
                       xnorm, ids, sims, fb, c->small);
  else
    hipLaunchKernelGGL((k_verify<LK, RK, true, false>), g, dim3(256), 0, c->stream, q, m,
                       (int)d, nullptr, (size_t)0, (int)m, data, nullptr, (int)n, 1, (int)kk,
                       cand, parts, xnorm, ids, sims, fb, c->small);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
