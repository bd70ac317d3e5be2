// Fused top-1 (Device::top1, core/mod.rs:97-112) and exact top-k
// (Device::topk, core/mod.rs:114-124) for gfx950.
//
// Exactness: the reference CPU backend (cpu-fused, assign/fused.rs) scores
// every (row, centroid) pair with one sequential f32 fma chain over the d
// dimensions. FP32 MFMA accumulates in its own order, so its scores can differ
// from the chain's by a few ulps times d. The path therefore has three stages:
//
//  1. screen (MFMA, the dense x . C^T contraction): each row keeps the L
//     smallest screen keys (key = -dot for IP, |c|^2 - 2 dot for L2) with
//     their ids, in registers; the n x k score matrix never leaves the CU.
//  2. verify (one thread per row): merge the partial lists; bound the screen
//     error E rigorously from |x| and max|c|; if the L-th smallest key is
//     above best + 2E, every centroid that can win is among the first L-1,
//     so re-score exactly those within best + 2E with the fma chain and take
//     the smallest exact key, lower id on ties. Otherwise queue the row.
//  3. exact (one workgroup per queued row): the full fma-chain scan over all
//     k centroids, the reference float order, ties to the lower id.
//
// The same stages with a longer list give the exact top-k of kNN.
//
// Bound: for any summation order of d products, |computed - exact dot| <=
// gamma_d * sum|x_t c_t| (gamma_d = d u / (1 - d u), u = 2^-24), and
// sum|x_t c_t| <= |x| |c|. The chain and the MFMA (taken at 2 gamma_d, plus a
// denormal-flush floor of d 2^-124) give |dot' - dot| <= 3 gamma_d |x| cmax;
// L2 keys add the rounding of |c|^2 - 2 dot on both sides. E carries a 12.5%
// margin for its own rounding.

#include "emh_internal.h"

namespace emh {
namespace {

constexpr int WAVE = 64;
constexpr int BK = 32;       // dimensions per LDS slab
constexpr int LDK = BK + 4;  // padded LDS row (floats): 144 B, conflict-free b128 reads
constexpr int TC = 128;      // centroids per tile (two 32-blocks per wave, two waves)
constexpr uint32_t NONE = 0xffffffffu;

typedef float v16f __attribute__((ext_vector_type(16)));

struct Cand {
  float key;
  uint32_t id;
};

// Insert (v, j) into an ascending list of L keys (the list keeps the L smallest).
template <int L>
__device__ __forceinline__ void insert(float (&key)[L], uint32_t (&id)[L], float v, uint32_t j) {
  if (!(v < key[L - 1])) return;
  key[L - 1] = v;
  id[L - 1] = j;
#pragma unroll
  for (int e = L - 1; e > 0; e--) {
    bool sw = key[e] < key[e - 1];
    float a = key[e - 1], b = key[e];
    uint32_t ia = id[e - 1], ib = id[e];
    key[e - 1] = sw ? b : a;
    key[e] = sw ? a : b;
    id[e - 1] = sw ? ib : ia;
    id[e] = sw ? ia : ib;
  }
}

// Work item of block `bid` of `nb`: blocks are dealt round-robin to the 8 XCDs
// (consecutive ids land on different XCDs), so number each XCD's blocks
// consecutively. The centroid parts of one row tile then run on one XCD at
// about the same time and share its L2.
__device__ __forceinline__ uint32_t xcd_swizzle(uint32_t bid, uint32_t nb) {
  uint32_t xcd = bid & 7, q = bid >> 3;
  uint32_t m = nb >> 3, r = nb & 7;
  return xcd * m + min(xcd, r) + q;
}

__device__ __forceinline__ float4 load4(const float* p, int col, int d, bool vec4) {
  if (p == nullptr) return make_float4(0.f, 0.f, 0.f, 0.f);
  if (vec4 && col + 4 <= d) return *reinterpret_cast<const float4*>(p + col);
  float4 v;
  v.x = col + 0 < d ? p[col + 0] : 0.f;
  v.y = col + 1 < d ? p[col + 1] : 0.f;
  v.z = col + 2 < d ? p[col + 2] : 0.f;
  v.w = col + 3 < d ? p[col + 3] : 0.f;
  return v;
}

// ---------------------------------------------------------------- screen
// Block: 256 threads = 4 waves; wave w: wr = w & 1 (row half), wc = w >> 1
// (centroid half). Block tile: TR = 64*WN rows x TC centroids per tile;
// each wave owns 32*WN rows x 64 centroids = (2 x WN) 32x32 MFMA blocks.
// MFMA v_mfma_f32_32x32x2_f32: A = centroids (M), B = rows (N); lane l holds
// row n = l % 32 of each block, so a row's keys stay in two lanes of a wave.
// The screen sums the K dimension in any order: lane half h = l / 32 takes
// dimensions [h*16, h*16 + 16) of each slab, four per b128 LDS read.
template <int WN, int L, bool L2, bool KNN>
__global__ __launch_bounds__(256, 2) void k_screen(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int nrows, const float* __restrict__ cents, const float* __restrict__ cnorm, int k,
    int tiles_per_part, int parts, int ntiles, bool vec4, Cand* __restrict__ cand) {
  constexpr int TR = 64 * WN;
  constexpr int XL = TR * BK / 4 / 256;  // float4 loads per thread per slab (rows)
  constexpr int CL = TC * BK / 4 / 256;  // float4 loads per thread per slab (centroids)
  // One LDS block: the X and C slabs (double-buffered), reused for the final merge.
  __shared__ __attribute__((aligned(16))) float smem[2 * (TR + TC) * LDK];
  __shared__ float Ns[2][TC];
  float (*Xs)[TR * LDK] = reinterpret_cast<float (*)[TR * LDK]>(smem);
  float (*Cs)[TC * LDK] = reinterpret_cast<float (*)[TC * LDK]>(smem + 2 * TR * LDK);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w & 1, wc = w >> 1;
  const int li = lane & 31, h = lane >> 5;
  const uint32_t wi = xcd_swizzle(blockIdx.x, gridDim.x);
  const int rt = (int)(wi / (uint32_t)parts), part = (int)(wi % (uint32_t)parts);
  const int t0 = part * tiles_per_part;
  const int t1 = min(ntiles, t0 + tiles_per_part);
  if (t0 >= t1) return;
  const int row0 = rt * TR;

  // Rows this thread loads: (tid >> 3) + 32u, float4 column (tid & 7).
  const float* xp[XL];
#pragma unroll
  for (int u = 0; u < XL; u++) {
    int r = row0 + (tid >> 3) + 32 * u;
    if (r < nrows) {
      size_t p = lo + (size_t)r;
      size_t xid = ids ? (size_t)ids[p] : p;
      xp[u] = xid < nx ? x + xid * (size_t)d : nullptr;
    } else {
      xp[u] = nullptr;
    }
  }
  const int c4 = (tid & 7) * 4;

  // Global query index of each row this lane scores (kNN exclude_self).
  uint32_t qrow[WN];
#pragma unroll
  for (int y = 0; y < WN; y++) qrow[y] = (uint32_t)(lo + row0 + wr * 32 * WN + y * 32 + li);

  float lkey[WN][L];
  uint32_t lid[WN][L];
#pragma unroll
  for (int y = 0; y < WN; y++)
#pragma unroll
    for (int e = 0; e < L; e++) {
      lkey[y][e] = INFINITY;
      lid[y][e] = NONE;
    }

  v16f acc[2][WN];
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int y = 0; y < WN; y++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[a][y][r] = 0.f;

  const int nslabs = (d + BK - 1) / BK;
  const int nsteps = (t1 - t0) * nslabs;
  float4 xr[XL], cr[CL];
  float nreg = 0.f;

  auto gload = [&](int st) {
    int tile = t0 + st / nslabs, slab = st % nslabs;
    int col = slab * BK + c4;
#pragma unroll
    for (int u = 0; u < XL; u++) xr[u] = load4(xp[u], col, d, vec4);
#pragma unroll
    for (int u = 0; u < CL; u++) {
      int j = tile * TC + (tid >> 3) + 32 * u;
      cr[u] = load4(j < k ? cents + (size_t)j * d : nullptr, col, d, vec4);
    }
    if (slab == 0 && tid < TC) {
      int j = tile * TC + tid;
      nreg = j < k ? (L2 ? cnorm[j] : 0.f) : INFINITY;
    }
  };
  auto lstore = [&](int st) {
    int buf = st & 1, slab = st % nslabs, tile = t0 + st / nslabs;
#pragma unroll
    for (int u = 0; u < XL; u++)
      *reinterpret_cast<float4*>(&Xs[buf][((tid >> 3) + 32 * u) * LDK + c4]) = xr[u];
#pragma unroll
    for (int u = 0; u < CL; u++)
      *reinterpret_cast<float4*>(&Cs[buf][((tid >> 3) + 32 * u) * LDK + c4]) = cr[u];
    if (slab == 0 && tid < TC) Ns[tile & 1][tid] = nreg;
  };

  gload(0);
  lstore(0);
  __syncthreads();
  for (int st = 0; st < nsteps; st++) {
    const int buf = st & 1;
    if (st + 1 < nsteps) gload(st + 1);
    const float* cs = Cs[buf];
    const float* xs = Xs[buf];
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) {
      const int kk = h * 16 + s4 * 4;
      float4 a0 = *reinterpret_cast<const float4*>(&cs[(wc * 64 + li) * LDK + kk]);
      float4 a1 = *reinterpret_cast<const float4*>(&cs[(wc * 64 + 32 + li) * LDK + kk]);
      float4 b[WN];
#pragma unroll
      for (int y = 0; y < WN; y++)
        b[y] = *reinterpret_cast<const float4*>(&xs[(wr * 32 * WN + y * 32 + li) * LDK + kk]);
#pragma unroll
      for (int y = 0; y < WN; y++) {
        acc[0][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.x, b[y].x, acc[0][y], 0, 0, 0);
        acc[1][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.x, b[y].x, acc[1][y], 0, 0, 0);
      }
#pragma unroll
      for (int y = 0; y < WN; y++) {
        acc[0][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.y, b[y].y, acc[0][y], 0, 0, 0);
        acc[1][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.y, b[y].y, acc[1][y], 0, 0, 0);
      }
#pragma unroll
      for (int y = 0; y < WN; y++) {
        acc[0][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.z, b[y].z, acc[0][y], 0, 0, 0);
        acc[1][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.z, b[y].z, acc[1][y], 0, 0, 0);
      }
#pragma unroll
      for (int y = 0; y < WN; y++) {
        acc[0][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.w, b[y].w, acc[0][y], 0, 0, 0);
        acc[1][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.w, b[y].w, acc[1][y], 0, 0, 0);
      }
    }
    if (st % nslabs == nslabs - 1) {
      // Tile done: fold its keys into the per-row lists.
      const int tile = t0 + st / nslabs;
      const float* ns = Ns[tile & 1];
#pragma unroll
      for (int a = 0; a < 2; a++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          // 32x32 accumulator layout: element (m, n) with n = lane % 32,
          // m = 8 (r / 4) + 4 (lane / 32) + r % 4.
          const int ci = wc * 64 + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          const uint32_t gj = (uint32_t)(tile * TC + ci);
          const float nn = ns[ci];
#pragma unroll
          for (int y = 0; y < WN; y++) {
            float v = acc[a][y][r];
            float key = L2 ? nn - 2.0f * v : nn - v;
            if (KNN && gj == qrow[y]) key = INFINITY;
            insert<L>(lkey[y], lid[y], key, gj);
            acc[a][y][r] = 0.f;
          }
        }
      }
    }
    if (st + 1 < nsteps) lstore(st + 1);
    __syncthreads();
  }

  // Merge the four partial lists of each row (two lane halves x two waves).
  Cand* M = reinterpret_cast<Cand*>(smem);  // [TR][4][L]
  static_assert(TR * 4 * L * 8 <= (int)(sizeof(float) * 2 * (TR + TC) * LDK), "merge space");
  __syncthreads();
#pragma unroll
  for (int y = 0; y < WN; y++) {
    const int row = wr * 32 * WN + y * 32 + li;
    const int contrib = wc * 2 + h;
#pragma unroll
    for (int e = 0; e < L; e++) M[(row * 4 + contrib) * L + e] = Cand{lkey[y][e], lid[y][e]};
  }
  __syncthreads();
  for (int row = tid; row < TR; row += 256) {
    if (row0 + row >= nrows) continue;
    float mk[L];
    uint32_t mi[L];
#pragma unroll
    for (int e = 0; e < L; e++) {
      mk[e] = INFINITY;
      mi[e] = NONE;
    }
    for (int q = 0; q < 4 * L; q++) {
      Cand cq = M[row * 4 * L + q];
      if (cq.id != NONE) insert<L>(mk, mi, cq.key, cq.id);
    }
    Cand* out = cand + ((size_t)part * nrows + row0 + row) * L;
#pragma unroll
    for (int e = 0; e < L; e++) out[e] = Cand{mk[e], mi[e]};
  }
}

// ------------------------------------------------------------ bound inputs
// small[SW_CMAX2] = max_j |c_j|^2 (any order), small[SW_CNMAX] = max_j cnorm[j].
__global__ __launch_bounds__(256) void k_prep(const float* __restrict__ cents, int k, int d,
                                              const float* __restrict__ cnorm,
                                              uint32_t* __restrict__ small) {
  int lane = threadIdx.x & 63;
  int j = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (j >= k) return;
  const float* c = cents + (size_t)j * d;
  float s = 0.f;
  for (int t = lane; t < d; t += WAVE) s += c[t] * c[t];
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, WAVE);
  if (lane == 0) {
    atomicMax(&small[SW_CMAX2], __float_as_uint(s));
    if (cnorm) atomicMax(&small[SW_CNMAX], __float_as_uint(cnorm[j]));
  }
}

__device__ __forceinline__ float screen_bound(float xn, float cmax2, float cnmax, int d, bool l2) {
  const float u = 5.9604645e-08f;  // 2^-24
  const float du = (float)d * u;
  const float g = du / (1.0f - du);
  const float S = (sqrtf(xn) * (1.0f + g)) * (sqrtf(cmax2) * (1.0f + g));
  const float edot = 3.0f * g * S + (float)d * 4.7019774e-38f;  // d 2^-124
  float e = l2 ? 2.0f * edot + 2.0f * u * (cnmax + 2.0f * S) : edot;
  return e * 1.125f;
}

// Sequential f32 sum of rounded squares (assign.rs:150-155).
__device__ __forceinline__ float seq_norm(const float* r, int d, bool vec4) {
  float s = 0.f;
  int t = 0;
  if (vec4)
    for (; t + 4 <= d; t += 4) {
      float4 v = *reinterpret_cast<const float4*>(r + t);
      float a = v.x * v.x, b = v.y * v.y, c = v.z * v.z, e = v.w * v.w;
      s = s + a;
      s = s + b;
      s = s + c;
      s = s + e;
    }
  for (; t < d; t++) {
    float a = r[t] * r[t];
    s = s + a;
  }
  return s;
}

// Exact fma chains of x against up to 4 rows (the cpu-fused dot, fused.rs:241-260).
__device__ __forceinline__ void chains4(const float* xr, const float* c0, const float* c1,
                                        const float* c2, const float* c3, int d, bool vec4,
                                        float& a0, float& a1, float& a2, float& a3) {
  a0 = a1 = a2 = a3 = 0.f;
  int t = 0;
  if (vec4)
    for (; t + 4 <= d; t += 4) {
      float4 xv = *reinterpret_cast<const float4*>(xr + t);
      float4 v0 = *reinterpret_cast<const float4*>(c0 + t);
      float4 v1 = *reinterpret_cast<const float4*>(c1 + t);
      float4 v2 = *reinterpret_cast<const float4*>(c2 + t);
      float4 v3 = *reinterpret_cast<const float4*>(c3 + t);
      a0 = fmaf(xv.x, v0.x, a0); a0 = fmaf(xv.y, v0.y, a0); a0 = fmaf(xv.z, v0.z, a0); a0 = fmaf(xv.w, v0.w, a0);
      a1 = fmaf(xv.x, v1.x, a1); a1 = fmaf(xv.y, v1.y, a1); a1 = fmaf(xv.z, v1.z, a1); a1 = fmaf(xv.w, v1.w, a1);
      a2 = fmaf(xv.x, v2.x, a2); a2 = fmaf(xv.y, v2.y, a2); a2 = fmaf(xv.z, v2.z, a2); a2 = fmaf(xv.w, v2.w, a2);
      a3 = fmaf(xv.x, v3.x, a3); a3 = fmaf(xv.y, v3.y, a3); a3 = fmaf(xv.z, v3.z, a3); a3 = fmaf(xv.w, v3.w, a3);
    }
  for (; t < d; t++) {
    float xv = xr[t];
    a0 = fmaf(xv, c0[t], a0);
    a1 = fmaf(xv, c1[t], a1);
    a2 = fmaf(xv, c2[t], a2);
    a3 = fmaf(xv, c3[t], a3);
  }
}

// Merge the parts' lists of position r into one ascending list of L.
template <int L>
__device__ __forceinline__ void merge_parts(const Cand* cand, int parts, int nrows, int r,
                                            float (&key)[L], uint32_t (&id)[L]) {
#pragma unroll
  for (int e = 0; e < L; e++) {
    key[e] = INFINITY;
    id[e] = NONE;
  }
  for (int q = 0; q < parts; q++) {
    const Cand* c = cand + ((size_t)q * nrows + r) * L;
    for (int e = 0; e < L; e++) {
      Cand v = c[e];
      if (v.id == NONE) break;
      insert<L>(key, id, v.key, v.id);
    }
  }
}

// --------------------------------------------------------------- top-1 verify
template <int L>
__global__ __launch_bounds__(256) void k_verify1(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int nrows, const float* __restrict__ cents, const float* __restrict__ cnorm, int k, int ip,
    const Cand* __restrict__ cand, int parts, bool vec4, uint32_t* __restrict__ labels,
    float* __restrict__ scores, uint32_t* __restrict__ fblist, uint32_t* __restrict__ small) {
  int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= nrows) return;
  float key[L];
  uint32_t id[L];
  merge_parts<L>(cand, parts, nrows, r, key, id);
  const size_t p = lo + (size_t)r;
  const size_t xid = ids ? (size_t)ids[p] : p;
  if (xid >= nx) {  // reported at the next read; outputs left as they were
    small[SW_BAD_ID] = 1;
    return;
  }
  const float* xr = x + xid * (size_t)d;
  const float xn = seq_norm(xr, d, vec4);
  const float E = screen_bound(xn, __uint_as_float(small[SW_CMAX2]),
                               __uint_as_float(small[SW_CNMAX]), d, !ip);
  const float thr = key[0] + 2.0f * E;
  const bool complete = id[0] != NONE && (id[L - 1] == NONE || key[L - 1] > thr);
  if (!complete) {
    uint32_t f = atomicAdd(&small[SW_FALLBACK_COUNT], 1u);
    fblist[f] = (uint32_t)p;
    return;
  }
  float best = INFINITY;
  uint32_t bid = NONE;
  for (int e0 = 0; e0 < L - 1; e0 += 4) {
    uint32_t cid[4];
    bool ok[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      int e = e0 + q;
      ok[q] = e < L - 1 && id[e] != NONE && key[e] <= thr;
      cid[q] = ok[q] ? id[e] : id[0];
    }
    if (!ok[0] && !ok[1] && !ok[2] && !ok[3]) break;
    float a[4];
    chains4(xr, cents + (size_t)cid[0] * d, cents + (size_t)cid[1] * d,
            cents + (size_t)cid[2] * d, cents + (size_t)cid[3] * d, d, vec4, a[0], a[1], a[2],
            a[3]);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      if (!ok[q]) continue;
      float kx;
      if (ip) {
        kx = -a[q];
      } else {
        float two = 2.0f * a[q];
        kx = cnorm[cid[q]] - two;
      }
      if (kx < best || (kx == best && cid[q] < bid)) {
        best = kx;
        bid = cid[q];
      }
    }
  }
  if (bid == NONE) {  // unreachable when complete; keep the CPU's defaults
    bid = 0;
    best = INFINITY;
  }
  labels[p] = bid;
  scores[p] = ip ? -best : fmaxf(xn + best, 0.0f);
}

// ------------------------------------------------------------- top-1 exact
// One workgroup per row: the reference scan, every centroid's fma chain, the
// smallest key, lower id on ties (assign.rs:420-493); score as finish_score.
// Rows: positions lo..hi, or the queued list (count read on the device).
__global__ __launch_bounds__(256) void k_exact1(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    size_t hi, const uint32_t* __restrict__ list, uint32_t* __restrict__ small,
    const float* __restrict__ cents, const float* __restrict__ cnorm, int k, int ip,
    uint32_t* __restrict__ labels, float* __restrict__ scores) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  __shared__ float bk[256];
  __shared__ uint32_t bi[256];
  const size_t nrows = list ? (size_t)small[SW_FALLBACK_COUNT] : hi - lo;
  if (list && blockIdx.x == 0 && threadIdx.x == 0) small[SW_FALLBACK_TOTAL] += (uint32_t)nrows;
  for (size_t f = blockIdx.x; f < nrows; f += gridDim.x) {
    const size_t p = list ? (size_t)list[f] : lo + f;
    const size_t xid = ids ? (size_t)ids[p] : p;
    if (xid >= nx) {  // uniform over the block: skip the row, report at the next read
      if (threadIdx.x == 0) small[SW_BAD_ID] = 1;
      continue;
    }
    const float* xr = x + xid * (size_t)d;
    for (int t = threadIdx.x; t < d; t += blockDim.x) xs[t] = xr[t];
    __syncthreads();
    float best = INFINITY;
    uint32_t bid = NONE;
    for (int j = threadIdx.x; j < k; j += blockDim.x) {
      const float* c = cents + (size_t)j * d;
      float a = 0.f;
      for (int t = 0; t < d; t++) a = fmaf(xs[t], c[t], a);
      float kx;
      if (ip) {
        kx = -a;
      } else {
        float two = 2.0f * a;
        kx = cnorm[j] - two;
      }
      if (kx < best) {
        best = kx;
        bid = (uint32_t)j;
      }
    }
    bk[threadIdx.x] = best;
    bi[threadIdx.x] = bid;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if ((int)threadIdx.x < o) {
        float k2 = bk[threadIdx.x + o];
        uint32_t i2 = bi[threadIdx.x + o];
        if (k2 < bk[threadIdx.x] || (k2 == bk[threadIdx.x] && i2 < bi[threadIdx.x])) {
          bk[threadIdx.x] = k2;
          bi[threadIdx.x] = i2;
        }
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      float b = bk[0];
      uint32_t j = bi[0];
      if (j == NONE) {  // nothing beat the initial value: label 0, initial score
        j = 0;
        b = INFINITY;
      }
      labels[p] = j;
      if (ip) {
        scores[p] = -b;
      } else {
        float xn = 0.f;
        for (int t = 0; t < d; t++) {
          float q = xs[t] * xs[t];
          xn = xn + q;
        }
        scores[p] = fmaxf(xn + b, 0.0f);
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------- top-k verify
// Keys are -dot. The kept set is the kk best by (dot desc, id asc), IEEE
// compares; the output order is dot descending in IEEE total order, then id
// (knn.rs:82-103).
__device__ __forceinline__ int32_t total_key(float v) {
  int32_t b = __float_as_int(v);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

__device__ __forceinline__ void write_topk(float* dots, uint32_t* cid, int nc, int kk,
                                           uint32_t* ids_out, float* sims_out) {
  // Selection by (dot desc, id asc) with IEEE compares.
  for (int a = 0; a < nc; a++)
    for (int b = a + 1; b < nc; b++) {
      bool sw = dots[b] > dots[a] || (dots[b] == dots[a] && cid[b] < cid[a]);
      if (sw) {
        float t = dots[a]; dots[a] = dots[b]; dots[b] = t;
        uint32_t u = cid[a]; cid[a] = cid[b]; cid[b] = u;
      }
    }
  int m = nc < kk ? nc : kk;
  // Final order: total order descending, then id.
  for (int a = 0; a < m; a++)
    for (int b = a + 1; b < m; b++) {
      int32_t ka = total_key(dots[a]), kb = total_key(dots[b]);
      bool sw = kb > ka || (kb == ka && cid[b] < cid[a]);
      if (sw) {
        float t = dots[a]; dots[a] = dots[b]; dots[b] = t;
        uint32_t u = cid[a]; cid[a] = cid[b]; cid[b] = u;
      }
    }
  for (int e = 0; e < kk; e++) {
    ids_out[e] = e < m ? cid[e] : NONE;
    sims_out[e] = e < m ? dots[e] : -INFINITY;
  }
}

template <int L>
__global__ __launch_bounds__(128) void k_verifyk(
    const float* __restrict__ q, int d, size_t m, const float* __restrict__ data, int n, int kk,
    const Cand* __restrict__ cand, int parts, bool vec4, uint32_t* __restrict__ ids_out,
    float* __restrict__ sims_out, uint32_t* __restrict__ fblist, uint32_t* __restrict__ small) {
  int r = blockIdx.x * blockDim.x + threadIdx.x;
  if ((size_t)r >= m) return;
  float key[L];
  uint32_t id[L];
  merge_parts<L>(cand, parts, (int)m, r, key, id);
  const float* qr = q + (size_t)r * d;
  const float qn = seq_norm(qr, d, vec4);
  const float E = screen_bound(qn, __uint_as_float(small[SW_CMAX2]), 0.f, d, false);
  const float thr = key[kk - 1] + 2.0f * E;
  const bool complete = id[L - 1] == NONE || key[L - 1] > thr;
  if (!complete) {
    uint32_t f = atomicAdd(&small[SW_FALLBACK_COUNT], 1u);
    fblist[f] = (uint32_t)r;
    return;
  }
  float dots[L];
  uint32_t cid[L];
  int nc = 0;
  for (int e0 = 0; e0 < L - 1; e0 += 4) {
    uint32_t c4[4];
    bool ok[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      int e = e0 + t;
      ok[t] = e < L - 1 && id[e] != NONE && (key[e] <= thr || !(thr == thr));
      c4[t] = ok[t] ? id[e] : (id[0] == NONE ? 0u : id[0]);
    }
    if (!ok[0] && !ok[1] && !ok[2] && !ok[3]) break;
    float a[4];
    chains4(qr, data + (size_t)c4[0] * d, data + (size_t)c4[1] * d, data + (size_t)c4[2] * d,
            data + (size_t)c4[3] * d, d, vec4, a[0], a[1], a[2], a[3]);
#pragma unroll
    for (int t = 0; t < 4; t++)
      if (ok[t]) {
        dots[nc] = a[t];
        cid[nc] = c4[t];
        nc++;
      }
  }
  write_topk(dots, cid, nc, kk, ids_out + (size_t)r * kk, sims_out + (size_t)r * kk);
}

// ------------------------------------------------------------- top-k exact
// One workgroup per queued query: each thread keeps the kk best of its strided
// share (j increasing, replace the worst only when strictly better, as
// knn.rs:82-96), then the workgroup picks the kk best of the 256 lists.
constexpr int KMAX = 16;
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
    // kk rounds: the best remaining entry by (score desc, id asc), IEEE.
    float outd[KMAX];
    uint32_t outi[KMAX];
    int got = 0;
    for (int e = 0; e < kk; e++) {
      float b = -INFINITY;
      uint32_t bi = NONE;
      int slot = -1;
      for (int s = threadIdx.x; s < 256 * KMAX; s += blockDim.x) {
        uint32_t j = si[s];
        if (j == NONE) continue;
        float v = sk[s];
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
    if (threadIdx.x == 0) write_topk(outd, outi, got, kk, ids_out + r * kk, sims_out + r * kk);
    __syncthreads();
  }
}

int choose_parts(int row_tiles, int ntiles, int cus) {
  // Enough blocks for ~4 per CU (2 resident), never more parts than tiles.
  int want = (4 * cus + row_tiles - 1) / row_tiles;
  return std::max(1, std::min(want, ntiles));
}

}  // namespace

constexpr int L1 = 5;   // top-1 list: 4 candidates + the bound
constexpr int LK = 24;  // top-k list: kk <= 16 plus 7 spare + the bound

void launch_top1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids, size_t lo, size_t hi,
                 const float* cents, const float* cnorm, size_t k, bool ip, uint32_t* labels,
                 float* scores) {
  if (hi <= lo) return;
  const size_t n = hi - lo;
  EMH_ENSURE(d <= 16384, "top1: d = %zu above the supported 16384", d);
  EMH_ENSURE(n < (1u << 31) && k < (1u << 31), "top1: shape too large");
  const bool vec4 = d % 4 == 0;
  const size_t xs_bytes = d * sizeof(float);
  const bool screen = c->screen && k >= 64 && d >= 32;
  if (!screen) {
    unsigned g = (unsigned)std::min<size_t>(n, 65535);
    hipLaunchKernelGGL(k_exact1, dim3(g), dim3(256), xs_bytes, c->stream, x, nx, (int)d, ids, lo,
                       hi, nullptr, c->small, cents, cnorm, (int)k, ip ? 1 : 0, labels, scores);
    EMH_HIP(hipGetLastError());
    return;
  }
  const int TR = 128;
  const int row_tiles = (int)((n + TR - 1) / TR);
  const int ntiles = (int)((k + TC - 1) / TC);
  int parts = choose_parts(row_tiles, ntiles, c->cus);
  const int tpp = (ntiles + parts - 1) / parts;
  parts = (ntiles + tpp - 1) / tpp;
  Cand* cand = (Cand*)c->cand.get((size_t)parts * n * L1 * sizeof(Cand));
  uint32_t* fb = (uint32_t*)c->fblist.get(n * 4);
  launch_fill_u32(c, c->small, 3, 0);  // fallback count, cmax2, cnmax
  hipLaunchKernelGGL(k_prep, grid1(k, 4), dim3(256), 0, c->stream, cents, (int)k, (int)d,
                     ip ? nullptr : cnorm, c->small);
  EMH_HIP(hipGetLastError());
  const unsigned blocks = (unsigned)(row_tiles * parts);
  ProfScope prof(c, 2.0 * (double)n * (double)k * (double)d);
  if (ip)
    hipLaunchKernelGGL((k_screen<2, L1, false, false>), dim3(blocks), dim3(256), 0, c->stream, x,
                       nx, (int)d, ids, lo, (int)n, cents, cnorm, (int)k, tpp, parts, ntiles, vec4,
                       cand);
  else
    hipLaunchKernelGGL((k_screen<2, L1, true, false>), dim3(blocks), dim3(256), 0, c->stream, x,
                       nx, (int)d, ids, lo, (int)n, cents, cnorm, (int)k, tpp, parts, ntiles, vec4,
                       cand);
  EMH_HIP(hipGetLastError());
  hipLaunchKernelGGL((k_verify1<L1>), grid1(n, 256), dim3(256), 0, c->stream, x, nx, (int)d, ids,
                     lo, (int)n, cents, cnorm, (int)k, ip ? 1 : 0, cand, parts, vec4, labels,
                     scores, fb, c->small);
  EMH_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_exact1, dim3(2 * c->cus), dim3(256), xs_bytes, c->stream, x, nx, (int)d,
                     ids, lo, hi, fb, c->small, cents, cnorm, (int)k, ip ? 1 : 0, labels, scores);
  EMH_HIP(hipGetLastError());
}

void launch_topk(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                 size_t kk, bool exclude_self, uint32_t* ids, float* sims) {
  if (m == 0) return;
  EMH_ENSURE(kk >= 1 && kk <= (size_t)KMAX, "topk: kk = %zu must be in 1..16", kk);
  EMH_ENSURE(d <= 16384, "topk: d = %zu above the supported 16384", d);
  EMH_ENSURE(m < (1u << 31) && n < (1u << 31), "topk: shape too large");
  const bool vec4 = d % 4 == 0;
  const int TR = 64;
  const int row_tiles = (int)((m + TR - 1) / TR);
  const int ntiles = (int)((n + TC - 1) / TC);
  int parts = choose_parts(row_tiles, std::max(ntiles, 1), c->cus);
  const int tpp = (std::max(ntiles, 1) + parts - 1) / parts;
  parts = (std::max(ntiles, 1) + tpp - 1) / tpp;
  Cand* cand = (Cand*)c->cand.get((size_t)parts * m * LK * sizeof(Cand));
  uint32_t* fb = (uint32_t*)c->fblist.get(m * 4);
  launch_fill_u32(c, c->small, 3, 0);
  if (n > 0) {
    hipLaunchKernelGGL(k_prep, grid1(n, 4), dim3(256), 0, c->stream, data, (int)n, (int)d,
                       nullptr, c->small);
    EMH_HIP(hipGetLastError());
    ProfScope prof(c, 2.0 * (double)m * (double)n * (double)d);
    if (exclude_self)
      hipLaunchKernelGGL((k_screen<1, LK, false, true>), dim3((unsigned)(row_tiles * parts)),
                         dim3(256), 0, c->stream, q, m, (int)d, nullptr, (size_t)0, (int)m, data,
                         nullptr, (int)n, tpp, parts, ntiles, vec4, cand);
    else
      hipLaunchKernelGGL((k_screen<1, LK, false, false>), dim3((unsigned)(row_tiles * parts)),
                         dim3(256), 0, c->stream, q, m, (int)d, nullptr, (size_t)0, (int)m, data,
                         nullptr, (int)n, tpp, parts, ntiles, vec4, cand);
    EMH_HIP(hipGetLastError());
  } else {
    parts = 1;
    launch_fill_u32(c, (uint32_t*)cand, m * LK * 2, NONE);  // empty lists
  }
  hipLaunchKernelGGL((k_verifyk<LK>), grid1(m, 128), dim3(128), 0, c->stream, q, (int)d, m, data,
                     (int)n, (int)kk, cand, parts, vec4, ids, sims, fb, c->small);
  EMH_HIP(hipGetLastError());
  hipLaunchKernelGGL(k_exactk, dim3(2 * c->cus), dim3(256), d * sizeof(float), c->stream, q,
                     (int)d, data, (int)n, (int)kk, exclude_self ? 1 : 0, fb, c->small, ids, sims);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
