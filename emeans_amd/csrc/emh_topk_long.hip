// Exact top-k for more neighbours than the screen's lists hold (kk above
// KMAX = 16, up to KLONG). Device::topk (core/mod.rs:114-124) serves
// kk <= GPU_KMAX in the reference; larger k runs its CPU search (knn.rs:42,
// core/src/knn.rs:53-107). Here both stay on the GPU, with that search's
// results:
//
//  - k_dots: the exact dots of a block of queries against every data row,
//    each the sequential f32 fma chain over the d dimensions (the float order
//    of every other score in this library), into scratch;
//  - k_select_long: one workgroup per query keeps the kk best data rows by a
//    radix select over the scores (larger score first, the lower id among
//    equal scores: the rows the reference keeps by replacing its worst entry
//    only on a strictly larger score while ids increase, knn.rs:82-96), then
//    sorts them by score descending in IEEE total order, then id ascending
//    (knn.rs:97-99). NaN and -inf scores are never kept (no score is larger
//    than the -inf a slot starts with); exclude_self skips j == i; missing
//    entries are id 0xFFFFFFFF, score -inf.

#include <algorithm>

#include "emh_select.h"

namespace emh {
namespace {

constexpr int DT = 64;  // queries and data rows per dots tile
constexpr int DK = 16;  // dimensions per LDS slab
constexpr int DP = DT + 4;  // padded slab row: the transposed stores hit 64 banks

// S[i ldS + j] = chain over t < d of q[q0 + i][t] * x[j][t], i < qb, j < n.
// Thread (ty, tx) of 16 x 16 computes queries 4 ty .. + 3 against data rows
// 4 tx .. + 3: sixteen independent chains, two b128 LDS reads per 16 fmas.
__global__ __launch_bounds__(256) void k_dots(const float* __restrict__ q, size_t q0, int qb,
                                              const float* __restrict__ x, int n, int d,
                                              float* __restrict__ S, size_t ldS) {
  __shared__ __attribute__((aligned(16))) float Qs[DK][DP];
  __shared__ __attribute__((aligned(16))) float Xs[DK][DP];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int j0 = blockIdx.x * DT, i0 = blockIdx.y * DT;
  // Loader: thread tid stages row tid / 4, dimensions 4 (tid % 4) .. + 3 of a slab.
  const int lr = tid >> 2, lc = 4 * (tid & 3);
  const int qi = min(i0 + lr, qb - 1), xj = min(j0 + lr, n - 1);  // clamped: valid rows only
  const float* qrow = q + (q0 + (size_t)qi) * (size_t)d;
  const float* xrow = x + (size_t)xj * (size_t)d;
  float acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int b = 0; b < 4; b++) acc[a][b] = 0.f;
  for (int t0 = 0; t0 < d; t0 += DK) {
    const int tn = min(DK, d - t0);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int t = t0 + lc + e;
      Qs[lc + e][lr] = t < d ? qrow[t] : 0.f;
      Xs[lc + e][lr] = t < d ? xrow[t] : 0.f;
    }
    __syncthreads();
    for (int t = 0; t < tn; t++) {  // dimensions past d never enter a chain
      const float4 qa = *reinterpret_cast<const float4*>(&Qs[t][4 * ty]);
      const float4 xb = *reinterpret_cast<const float4*>(&Xs[t][4 * tx]);
      const float qv[4] = {qa.x, qa.y, qa.z, qa.w};
      const float xv[4] = {xb.x, xb.y, xb.z, xb.w};
#pragma unroll
      for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = fmaf(qv[a], xv[b], acc[a][b]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < 4; a++) {
    const int i = i0 + 4 * ty + a;
    if (i >= qb) break;
    float* o = S + (size_t)i * ldS;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int j = j0 + 4 * tx + b;
      if (j < n) o[j] = acc[a][b];
    }
  }
}

// Ascending unsigned image of a float's IEEE total order.
__device__ __forceinline__ uint32_t ord_total(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_ord(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
// The selection's key: 0 for a score that is never kept (NaN, -inf, the
// query itself), else the ascending image of its IEEE value (-0 == +0:
// adding +0 turns -0 into +0). Every kept key is above ord_total(-inf) > 0.
__device__ __forceinline__ uint32_t sel_key(float v, bool skip) {
  if (skip || !(v > -INFINITY)) return 0u;
  return ord_total(v + 0.0f);
}

constexpr int NT = 1024;  // threads per selecting workgroup
constexpr int NW = NT / 64;

// Block-wide exclusive prefix of one flag per thread, and the block's total.
__device__ __forceinline__ int block_rank(bool f, int* wsum, int& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const unsigned long long b = __ballot(f);
  const int below = __popcll(b & ((1ull << lane) - 1ull));
  if (lane == 0) wsum[w] = __popcll(b);
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int v = 0; v < NW; v++) {
    const int c = wsum[v];
    before += v < w ? c : 0;
    total += c;
  }
  __syncthreads();
  return before + below;
}

// Workgroup i: the kk best data rows of query q0 + i from its scores
// S[i ldS ..], written to ids / sims row q0 + i. P (a power of two >= kk)
// slots of sort keys in LDS.
template <int P>
__global__ __launch_bounds__(NT) void k_select_long(const float* __restrict__ S, size_t ldS,
                                                    int n, size_t q0, int kk, int exclude_self,
                                                    uint32_t* __restrict__ ids,
                                                    float* __restrict__ sims) {
  __shared__ unsigned long long sk[P];
  __shared__ uint32_t hist[2048];
  __shared__ int wsum[NW];
  __shared__ uint32_t sh_prefix, sh_rem, sh_all;
  const int tid = threadIdx.x;
  const size_t qi = q0 + blockIdx.x;
  const float* row = S + (size_t)blockIdx.x * ldS;
  auto key_at = [&](int j) { return sel_key(row[j], exclude_self && (size_t)j == qi); };

  // Radix select of the kk-th largest key: digits of 11, 11 and 10 bits.
  uint32_t prefix = 0, pmask = 0;
  uint32_t rem = (uint32_t)kk;
  bool all = false;  // fewer kept scores than kk: every one is taken
  for (int pass = 0; pass < 3 && !all; pass++) {
    const int shift = pass == 0 ? 21 : pass == 1 ? 10 : 0;
    const int nb = pass == 2 ? 1024 : 2048;
    for (int b = tid; b < nb; b += NT) hist[b] = 0u;
    __syncthreads();
    for (int j = tid; j < n; j += NT) {
      const uint32_t k = key_at(j);
      if (k != 0u && (k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & (nb - 1)], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // Lane l sums bins from the top: segment [nb - (l + 1) s, nb - l s).
      const int s = nb / 64;
      const int hi = nb - tid * s;
      uint32_t seg = 0;
      for (int b = hi - 1; b >= hi - s; b--) seg += hist[b];
      uint32_t incl = seg;  // inclusive prefix over lanes 0 .. tid (top bins first)
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o, 64);
        if (tid >= o) incl += t;
      }
      const uint32_t total = __shfl(incl, 63, 64);
      if (pass == 0 && total <= rem) {
        if (tid == 0) sh_all = 1u;
      } else {
        const uint32_t excl = incl - seg;
        if (excl < rem && rem <= incl) {  // the digit is in this lane's segment
          uint32_t above = excl;
          for (int b = hi - 1; b >= hi - s; b--) {
            const uint32_t c = hist[b];
            if (above + c >= rem) {
              sh_prefix = prefix | ((uint32_t)b << shift);
              sh_rem = rem - above;
              break;
            }
            above += c;
          }
        }
        if (tid == 0) sh_all = 0u;
      }
    }
    __syncthreads();
    all = sh_all != 0u;
    if (!all) {
      prefix = sh_prefix;
      rem = sh_rem;
      pmask |= (uint32_t)(nb - 1) << shift;
    }
    __syncthreads();
  }
  // Keys above T = prefix are all kept (kk - rem of them); of the keys equal
  // to T, the rem with the lowest ids. With `all`, every kept key.
  const uint32_t T = prefix;
  const uint32_t n_gt = all ? 0u : (uint32_t)kk - rem, need = all ? 0u : rem;
  uint32_t got_gt = 0, got_eq = 0;
  for (int j0 = 0; j0 < n; j0 += NT) {
    const int j = j0 + tid;
    const uint32_t k = j < n ? key_at(j) : 0u;
    const bool gt = all ? k != 0u : k > T;
    const bool eq = !all && k != 0u && k == T;
    int tot_gt, tot_eq;
    const int rg = block_rank(gt, wsum, tot_gt);
    const int re = block_rank(eq, wsum, tot_eq);
    const float v = j < n ? row[j] : 0.f;
    const unsigned long long sortkey =
        ((unsigned long long)(~ord_total(v)) << 32) | (unsigned long long)(uint32_t)j;
    if (gt) sk[got_gt + rg] = sortkey;
    if (eq && got_eq + re < need) sk[n_gt + got_eq + re] = sortkey;
    got_gt += tot_gt;
    got_eq += tot_eq;
  }
  const uint32_t cnt = all ? got_gt : (uint32_t)kk;
  for (int s = tid; s < P; s += NT)
    if ((uint32_t)s >= cnt) sk[s] = ~0ull;
  __syncthreads();
  // Bitonic sort of the P keys, ascending: score descending, then id ascending.
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = tid; t < P / 2; t += NT) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const unsigned long long a = sk[lo], b = sk[hi];
        if ((a > b) == up) {
          sk[lo] = b;
          sk[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int t = tid; t < kk; t += NT) {
    const size_t o = qi * (size_t)kk + t;
    if ((uint32_t)t < cnt) {
      const unsigned long long e = sk[t];
      ids[o] = (uint32_t)e;
      sims[o] = from_ord(~(uint32_t)(e >> 32));
    } else {
      ids[o] = NONE;
      sims[o] = -INFINITY;
    }
  }
}

template <int P>
void select_long(emh_ctx* c, unsigned blocks, const float* S, size_t ldS, size_t n, size_t q0,
                 size_t kk, bool exclude_self, uint32_t* ids, float* sims) {
  hipLaunchKernelGGL(k_select_long<P>, dim3(blocks), dim3(NT), 0, c->stream, S, ldS, (int)n, q0,
                     (int)kk, exclude_self ? 1 : 0, ids, sims);
  EMH_HIP(hipGetLastError());
}

}  // namespace

void launch_topk_long(emh_ctx* c, const float* q, size_t m, const float* data, size_t n,
                      size_t d, size_t kk, bool exclude_self, uint32_t* ids, float* sims) {
  EMH_ENSURE(kk > (size_t)KMAX && kk <= (size_t)KLONG, "topk: kk = %zu outside %d..%d", kk,
             KMAX + 1, KLONG);
  EMH_ENSURE(m < (1u << 31) && n < (1u << 31) && d < (1u << 31), "topk: shape too large");
  if (m == 0) return;
  // Scores of a block of queries against all data rows: about 1 GiB of
  // scratch, at least one 64-query tile.
  const size_t ldS = std::max<size_t>((n + 3) & ~size_t(3), 4);
  const size_t budget = size_t(1) << 30;
  size_t qb = std::max<size_t>(budget / (ldS * 4) / DT * DT, DT);
  qb = std::min(std::min(qb, size_t(65535) * DT), m);  // grid.y of k_dots within 65535
  float* S = (float*)c->klong.get(qb * ldS * 4);
  for (size_t q0 = 0; q0 < m; q0 += qb) {
    const size_t nb = std::min(qb, m - q0);
    if (n > 0) {
      const dim3 g((unsigned)((n + DT - 1) / DT), (unsigned)((nb + DT - 1) / DT));
      hipLaunchKernelGGL(k_dots, g, dim3(256), 0, c->stream, q, q0, (int)nb, data, (int)n,
                         (int)d, S, ldS);
      EMH_HIP(hipGetLastError());
    }
    const unsigned blocks = (unsigned)nb;
    if (kk <= 32)
      select_long<32>(c, blocks, S, ldS, n, q0, kk, exclude_self, ids, sims);
    else if (kk <= 256)
      select_long<256>(c, blocks, S, ldS, n, q0, kk, exclude_self, ids, sims);
    else
      select_long<KLONG>(c, blocks, S, ldS, n, q0, kk, exclude_self, ids, sims);
  }
}

}  // namespace emh
