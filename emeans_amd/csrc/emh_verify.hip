// The exact scans behind the MFMA screen (emh_screen.hip) and its check
// (emh_rescore.hip), for the rows the check could not settle:
//
//  k_exact1    top-1: the rows' scan over all centroids, split into
//              (4 rows x 64 centroids) items; the block that completes a row
//              group's last item reduces the group's rows (one launch). For
//              a selection without the screen, and queued rows when d % 4 != 0;
//  k_queued1   top-1 for the rows the check queues (d % 4 == 0): short
//              (4 rows x 16 centroids) items, one burst of DMA copies and one
//              chain per lane each, the winners folded by 64-bit atomics;
//  k_exactk    top-k: one block per queued query over all data rows.
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

// ------------------------------------------------------------- exact top-1
// Item = (group of RG rows, chunk of CJ centroids): one wave, lane = centroid,
// RG chains per lane. The dimensions go in tiles of TD: a tile of the chunk's
// centroids and the group's rows is loaded into registers (every load of the
// tile in flight at once) while the previous tile is consumed from LDS.
constexpr int CJ = 64, RG = 4, TD = 64, TDP = TD + 4;
constexpr int CL4 = CJ * TD / 4 / WAVE;  // float4 loads per lane per tile (centroids)
constexpr int XL4 = RG * TD / 4 / WAVE;  // float4 loads per lane per tile (rows)

// Columns col..col+3 of a row, zero past d. Branch-free: every load is issued
// (at a clamped column) and the zeros are selected afterwards, so a tile's
// loads stay in flight together instead of each waiting on a branch.
template <bool VEC4>
__device__ __forceinline__ float4 load_tile4(const float* row, int col, int d, bool valid = true) {
  if (VEC4) {  // d % 4 == 0: col < d implies col + 4 <= d
    const float4 v = *reinterpret_cast<const float4*>(row + min(col, d - 4));
    const bool in = valid && col < d;
    return make_float4(in ? v.x : 0.f, in ? v.y : 0.f, in ? v.z : 0.f, in ? v.w : 0.f);
  }
  float e[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const float v = row[min(col + u, d - 1)];
    e[u] = valid && col + u < d ? v : 0.f;
  }
  return make_float4(e[0], e[1], e[2], e[3]);
}

// The end of row group g (rows g*RG ...): each row's smallest chunk minimum
// (lower id on ties; a row where nothing wins gets label 0 and the initial
// score) and, for L2, its |x|^2 as a sequential sum of rounded squares: the
// wave stages the group's squares in LDS (sq, RG rows of SEG floats per pass)
// and lane r adds row r's in order. One wave.
constexpr int SEG = CJ * TDP / RG;
__device__ __attribute__((noinline)) void finish_group(const float* __restrict__ x, size_t nx, int d,
                             const uint32_t* __restrict__ ids, size_t lo,
                             const uint32_t* __restrict__ list, uint32_t* __restrict__ small,
                             int nch, int ip, const Cand* __restrict__ partial, int g, int nrows,
                             float* sq, uint32_t* __restrict__ labels,
                             float* __restrict__ scores) {
  const int lane = threadIdx.x;
  float mybest = INFINITY;  // lane r < RG: row r's best key and id
  uint32_t mybid = NONE;
  size_t myp = 0;
  const float* xr[RG];
  bool ok[RG];
#pragma unroll
  for (int r = 0; r < RG; r++) {
    const int f = g * RG + r;
    ok[r] = false;
    xr[r] = x;
    if (f >= nrows) continue;  // uniform
    const size_t p = list ? (size_t)list[f] : lo + (size_t)f;
    const size_t xid = ids ? (size_t)ids[p] : p;
    if (xid >= nx) {
      if (lane == 0) small[SW_BAD_ID] = 1;
      continue;
    }
    ok[r] = true;
    xr[r] = x + xid * (size_t)d;
    float best = INFINITY;
    uint32_t bid = NONE;
    for (int q = lane; q < nch; q += WAVE) {
      const Cand c = partial[(size_t)f * nch + q];
      if (c.id != NONE && (c.key < best || (c.key == best && c.id < bid))) {
        best = c.key;
        bid = c.id;
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float b2 = __shfl_xor(best, o, WAVE);
      const uint32_t i2 = __shfl_xor(bid, o, WAVE);
      if (i2 != NONE && (b2 < best || (b2 == best && i2 < bid))) {
        best = b2;
        bid = i2;
      }
    }
    if (lane == r) {
      mybest = best;
      mybid = bid;
      myp = p;
    }
  }
  float xn = 0.f;
  if (!ip) {
    for (int t0 = 0; t0 < d; t0 += SEG) {
      const int tl = min(SEG, d - t0);
#pragma unroll
      for (int r = 0; r < RG; r++) {
        if (!ok[r]) continue;  // uniform
        for (int i0 = 0; i0 < tl; i0 += WAVE * 8) {
          float v[8];
#pragma unroll
          for (int u = 0; u < 8; u++) {
            const int i = i0 + lane + WAVE * u;
            v[u] = i < tl ? xr[r][t0 + i] : 0.f;
          }
#pragma unroll
          for (int u = 0; u < 8; u++) {
            const int i = i0 + lane + WAVE * u;
            if (i < tl) sq[r * SEG + i] = v[u] * v[u];
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      if (lane < RG && ok[lane]) {  // in order, 16 LDS reads in flight
        const float* row = sq + lane * SEG;
        int i = 0;
        for (; i + 16 <= tl; i += 16) {
          float v[16];
#pragma unroll
          for (int u = 0; u < 16; u++) v[u] = row[i + u];
#pragma unroll
          for (int u = 0; u < 16; u++) xn = xn + v[u];
        }
        for (; i < tl; i++) xn = xn + row[i];
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
  }
  if (lane < RG && ok[lane]) {
    if (mybid == NONE) {
      mybid = 0;
      mybest = INFINITY;
    }
    labels[myp] = mybid;
    scores[myp] = ip ? -mybest : fmaxf(xn + mybest, 0.0f);
  }
}

template <bool VEC4>
__global__ __launch_bounds__(64) void k_exact1(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int n_direct, const uint32_t* __restrict__ list, uint32_t* __restrict__ small,
    const float* __restrict__ cents, const float* __restrict__ cnorm, int k, int ip,
    Cand* __restrict__ partial, uint32_t* __restrict__ tickets, uint32_t* __restrict__ labels,
    float* __restrict__ scores) {
  __shared__ __attribute__((aligned(16))) float ct[CJ * TDP];
  __shared__ __attribute__((aligned(16))) float xt[RG * TD];
  __shared__ uint32_t xid_s[RG];
  __shared__ int last_s;
  const int nrows = list ? (int)small[SW_FALLBACK_COUNT] : n_direct;
  if (list && blockIdx.x == 0 && threadIdx.x == 0) small[SW_FALLBACK_TOTAL] += (uint32_t)nrows;
  const int nch = (k + CJ - 1) / CJ;
  const int ngr = (nrows + RG - 1) / RG;
  const int ntd = (d + TD - 1) / TD;
  const int lane = threadIdx.x;
  const int c4 = lane % (TD / 4), r0 = lane / (TD / 4);  // this lane's float4 column, first row
  constexpr int RSTEP = WAVE / (TD / 4);                  // rows per load instruction
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
    const float* xp[XL4];
    bool xv[XL4];
#pragma unroll
    for (int u = 0; u < XL4; u++) {
      const uint32_t xid = xid_s[r0 + RSTEP * u];
      xv[u] = xid != NONE;
      xp[u] = x + (size_t)(xv[u] ? xid : 0) * d;
    }
    float4 cr[CL4], xr[XL4];
    auto gload = [&](int t0) {
      const int col = t0 + 4 * c4;
#pragma unroll
      for (int u = 0; u < CL4; u++)
        cr[u] = load_tile4<VEC4>(cents + (size_t)min(q * CJ + r0 + RSTEP * u, k - 1) * d, col, d);
#pragma unroll
      for (int u = 0; u < XL4; u++)
        xr[u] = load_tile4<VEC4>(xp[u], col, d, xv[u]);  // xp[u] is row 0 when invalid
    };
    float acc[RG];
#pragma unroll
    for (int r = 0; r < RG; r++) acc[r] = 0.f;
    gload(0);
    for (int tile = 0; tile < ntd; tile++) {
#pragma unroll
      for (int u = 0; u < CL4; u++)
        *reinterpret_cast<float4*>(&ct[(r0 + RSTEP * u) * TDP + 4 * c4]) = cr[u];
#pragma unroll
      for (int u = 0; u < XL4; u++)
        *reinterpret_cast<float4*>(&xt[(r0 + RSTEP * u) * TD + 4 * c4]) = xr[u];
      __syncthreads();
      const int t0 = tile * TD;
      if (tile + 1 < ntd) gload(t0 + TD);
      const int tl = min(TD, d - t0);
      const float* crow = &ct[lane * TDP];
      int tt = 0;
#pragma unroll 4
      for (; tt + 4 <= tl; tt += 4) {
        const float4 cv = *reinterpret_cast<const float4*>(crow + tt);
#pragma unroll
        for (int r = 0; r < RG; r++) {
          const float4 v = *reinterpret_cast<const float4*>(&xt[r * TD + tt]);
          acc[r] = fmaf(v.x, cv.x, acc[r]);
          acc[r] = fmaf(v.y, cv.y, acc[r]);
          acc[r] = fmaf(v.z, cv.z, acc[r]);
          acc[r] = fmaf(v.w, cv.w, acc[r]);
        }
      }
      for (; tt < tl; tt++) {
        const float cv = crow[tt];
#pragma unroll
        for (int r = 0; r < RG; r++) acc[r] = fmaf(xt[r * TD + tt], cv, acc[r]);
      }
      __syncthreads();
    }
    const int j = q * CJ + lane;
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
    // The group's ticket: the block that completes its last chunk finishes it.
    if (lane == 0) {
      __threadfence();
      last_s = atomicAdd(&tickets[g], 1u) == (uint32_t)(nch - 1);
    }
    __syncthreads();
    if (last_s) {
      __threadfence();
      finish_group(x, nx, d, ids, lo, list, small, nch, ip, partial, g, nrows, ct, labels, scores);
      if (lane == 0) tickets[g] = 0;
    }
    __syncthreads();
  }
}

// ------------------------------------------------- exact top-1, queued rows
// The check queues few rows (often one to eight per batch), so this scan is
// built for latency: many short items, each a single wave that copies its
// data to LDS in one burst and then runs one fma chain per lane.
//
// Item = (group of QR rows, chunk of QJ centroids), plus one norm item per
// group for L2. Lane (j = lane / QR, r = lane % QR) runs row r's chain against
// centroid j of the chunk. The dimensions go in phases of up to QPH: the
// phase's slice of the chunk's centroids and of the group's rows is copied to
// LDS by the DMA path (global_load_lds, 16 bytes per lane, all instructions in
// flight together), then the chains read it. LDS slots (16 bytes, 4 dims):
// centroids at u * QJ + j, rows at u * QR + r for dims 4u..4u+3 of the phase,
// so a read touches consecutive slots (no bank conflicts) and lanes sharing a
// centroid or a row read it by broadcast.
//
// Each item folds its chunk's winners into one 64-bit word per row with an
// atomic max of the complement of (ordered key << 32 | id << 1 | sign of a
// zero key): the smallest key wins, then the lower id (keys -0 and +0 are
// equal, as in the reference's comparison; the sign bit restores the winner's
// own zero), so the reduction is exact and independent of the item order. The
// item that takes a group's last ticket writes the group's labels and scores
// and leaves the words and the ticket at zero for the next launch.
constexpr int QR = 4, QJ = 16, QPH = 768;
constexpr int QU = QPH / 4;  // 4-dim slots per phase

__device__ __forceinline__ uint64_t pack_best(float key, uint32_t id) {
  uint32_t b = __float_as_uint(key), z = 0;
  if (key == 0.0f) {  // -0 and +0 compare equal: one code, the sign kept apart
    z = b >> 31;
    b = 0u;
  }
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ~(((uint64_t)o << 32) | ((uint64_t)id << 1) | z);
}

__device__ __forceinline__ bool unpack_best(uint64_t w, float& key, uint32_t& id) {
  if (w == 0) return false;
  const uint64_t v = ~w;
  const uint32_t o = (uint32_t)(v >> 32);
  uint32_t b = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  if (b == 0u && (v & 1u)) b = 0x80000000u;
  key = __uint_as_float(b);
  id = (uint32_t)((v >> 1) & 0x7fffffffu);
  return true;
}

__global__ __launch_bounds__(64) void k_queued1(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int n_direct, const uint32_t* __restrict__ list, uint32_t* __restrict__ small,
    const float* __restrict__ cents, const float* __restrict__ cnorm, int k, int ip,
    unsigned long long* __restrict__ best, uint32_t* __restrict__ tickets,
    float* __restrict__ xnq, uint32_t* __restrict__ labels, float* __restrict__ scores,
    uint32_t* __restrict__ tcnt, uint32_t* __restrict__ tcounts, size_t tlo, size_t tstride) {
  typedef float v4f __attribute__((ext_vector_type(4)));
  __shared__ v4f cs[QU * QJ];
  __shared__ v4f xs[QU * QR];
  __shared__ uint32_t xid_s[QR];
  // Queued rows (list: positions, count on the device), or a direct
  // selection of n_direct rows at positions lo, lo + 1, ...
  const int nrows = list ? (int)small[SW_FALLBACK_COUNT] : n_direct;
  if (list && blockIdx.x == 0 && threadIdx.x == 0) small[SW_FALLBACK_TOTAL] += (uint32_t)nrows;
  const int nch = (k + QJ - 1) / QJ;
  const int per = nch + (ip ? 0 : 1);  // items per group (the last one: |x|^2)
  const int ngr = (nrows + QR - 1) / QR;
  const int lane = threadIdx.x;
  const int j = lane / QR, r = lane % QR;
  for (int item = blockIdx.x; item < ngr * per; item += gridDim.x) {
    const int g = item / per, q = item - g * per;
    const bool norm = q == nch;
    if (lane < QR) {
      const int f = g * QR + lane;
      uint32_t xid = NONE;
      if (f < nrows) {
        const size_t p = list ? (size_t)list[f] : lo + (size_t)f;
        const size_t id = ids ? (size_t)ids[p] : p;
        if (id < nx)
          xid = (uint32_t)id;
        else
          small[SW_BAD_ID] = 1;
      }
      xid_s[lane] = xid;
    }
    __syncthreads();
    // This lane's DMA sources: rows (slot l of each row instruction covers
    // dims 4 * (16 i + l / QR) of row l % QR) and centroids (dims
    // 4 * (4 i + l / QJ) of centroid l % QJ).
    const uint32_t xr = xid_s[lane % QR];
    const float* xrow = x + (size_t)(xr == NONE ? 0u : xr) * d;
    const float* crow = cents + (size_t)min(q * QJ + lane % QJ, k - 1) * d;
    float acc = 0.f;
    for (int t0 = 0; t0 < d; t0 += QPH) {
      const int nu = min(QU, (d - t0) / 4);  // d % 4 == 0
      for (int i = 0; i < (nu + 15) / 16; i++) {
        const int col = min(t0 + 4 * (16 * i + lane / QR), d - 4);
        __builtin_amdgcn_global_load_lds(xrow + col, &xs[i * 64], 16, 0, 0);
      }
      if (!norm)
        for (int i = 0; i < (nu + 3) / 4; i++) {
          const int col = min(t0 + 4 * (4 * i + lane / QJ), d - 4);
          __builtin_amdgcn_global_load_lds(crow + col, &cs[i * 64], 16, 0, 0);
        }
      __syncthreads();  // waits for the copies
      if (norm) {  // |x|^2 of row r: sequential sum of rounded squares
#pragma unroll 8
        for (int u = 0; u < nu; u++) {
          const v4f v = xs[u * QR + r];
          acc = acc + v.x * v.x;
          acc = acc + v.y * v.y;
          acc = acc + v.z * v.z;
          acc = acc + v.w * v.w;
        }
      } else {
#pragma unroll 8
        for (int u = 0; u < nu; u++) {
          const v4f cv = cs[u * QJ + j];
          const v4f v = xs[u * QR + r];
          acc = fmaf(v.x, cv.x, acc);
          acc = fmaf(v.y, cv.y, acc);
          acc = fmaf(v.z, cv.z, acc);
          acc = fmaf(v.w, cv.w, acc);
        }
      }
      __syncthreads();  // the next phase's copies overwrite these slots
    }
    const int f = g * QR + r;
    const bool valid = f < nrows && xid_s[r] != NONE;
    if (norm) {
      if (j == 0 && valid) xnq[f] = acc;
    } else {
      const int cj = q * QJ + j;
      float kx = INFINITY;
      uint32_t id = NONE;
      if (valid && cj < k) {
        kx = ip ? -acc : cnorm[cj] - 2.0f * acc;
        id = (uint32_t)cj;
        if (!(kx < INFINITY)) id = NONE;  // NaN or +inf never wins
      }
      uint64_t w = id == NONE ? 0ull : pack_best(kx, id);
#pragma unroll
      for (int o = QR; o < WAVE; o <<= 1) {  // across the centroids of row r
        const uint64_t w2 = __shfl_xor(w, o, WAVE);
        w = w2 > w ? w2 : w;
      }
      if (j == 0 && w != 0) atomicMax(&best[f], (unsigned long long)w);
    }
    // The group's ticket: the item that completes it writes the rows.
    __shared__ int last_s;
    if (lane == 0) {
      __threadfence();
      last_s = atomicAdd(&tickets[g], 1u) == (uint32_t)(per - 1);
    }
    __syncthreads();
    if (last_s) {
      __threadfence();
      if (lane < QR && f < nrows) {
        const unsigned long long w = atomicExch(&best[f], 0ull);
        if (xid_s[r] != NONE) {
          float bk = INFINITY;
          uint32_t bid = 0;  // nothing wins: label 0 and the initial score
          unpack_best(w, bk, bid);
          const size_t p = list ? (size_t)list[f] : lo + (size_t)f;
          labels[p] = bid;
          scores[p] = ip ? -bk : fmaxf(xnq[f] + bk, 0.0f);
          if (tcnt) {  // the tally (few rows: one atomic each)
            atomicAdd(&tcnt[(size_t)bid * tstride + (p - tlo) / TALLY_CP], 1u);
            atomicAdd(&tcounts[bid], 1u);
          }
        }
      }
      if (lane == 0) tickets[g] = 0;
    }
    __syncthreads();
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

}  // namespace

// The latency-bound scan's items for n rows against k centroids.
size_t queued_items(size_t n, size_t k, bool ip) {
  return ((n + QR - 1) / QR) * ((k + QJ - 1) / QJ + (ip ? 0 : 1));
}

size_t exact1_scratch_bytes(emh_ctx* c, size_t n, size_t d, size_t k, bool ip, bool list) {
  auto r = [](size_t b) { return (b + 255) & ~size_t(255); };
  if ((list && d % 4 == 0) || (!list && queued_direct(c, n, d, k, ip))) {
    const size_t ngr = (n + QR - 1) / QR;
    return r(n * 8 + ngr * 4) + r(n * 4);
  }
  const size_t nch = (k + CJ - 1) / CJ, ngr = (n + RG - 1) / RG;
  return r(n * nch * sizeof(Cand)) + r(ngr * 4);
}

void launch_exact1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                   size_t lo, size_t n, const uint32_t* list, const float* cents,
                   const float* cnorm, size_t k, bool ip, uint32_t* labels, float* scores,
                   Arena* ar, const LabelTally* tally) {
  if (n == 0) return;
  EMH_ENSURE(!tally || (d % 4 == 0 && (list || queued_direct(c, n, d, k, ip))),
             "exact: a tally needs the queued-row scan");
  // Both kernels read row 0 in place of a row whose id is out of range.
  EMH_ENSURE(nx > 0, "top1: a selection of %zu rows over no data rows", n);
  // Queued rows (few), or a small direct selection: the latency-bound scan.
  // (k_exact1's tiles each wait a memory round trip: ~30 us at any size up
  // to a few thousand rows.)
  if ((list && d % 4 == 0) || (!list && queued_direct(c, n, d, k, ip))) {
    const size_t ngr = (n + QR - 1) / QR;
    const size_t per = (k + QJ - 1) / QJ + (ip ? 0 : 1);
    // Self-cleaning: the best words, then the tickets, all left at zero (a
    // fixed block is cleared on every call instead).
    char* z;
    float* xnq;
    if (ar) {
      z = (char*)ar->take(n * 8 + ngr * 4);
      launch_fill_u32(c, (uint32_t*)z, n * 2 + ngr, 0);
      xnq = (float*)ar->take(n * 4);
    } else {
      z = (char*)c->tickets.get_zeroed(n * 8 + ngr * 4, c->stream);
      xnq = (float*)c->knn_tmp.get(n * 4);
    }
    const unsigned g = (unsigned)std::min<size_t>(ngr * per, (size_t)2 * c->cus);
    hipLaunchKernelGGL(k_queued1, dim3(g), dim3(64), 0, c->stream, x, nx, (int)d, ids, lo,
                       (int)n, list, c->small, cents, cnorm, (int)k, ip ? 1 : 0,
                       (unsigned long long*)z,
                       (uint32_t*)(z + n * 8), xnq, labels, scores,
                       tally ? tally->cnt : nullptr, tally ? tally->counts : nullptr,
                       tally ? tally->lo : 0, tally ? tally->stride : 0);
    EMH_HIP(hipGetLastError());
    return;
  }
  const size_t nch = (k + CJ - 1) / CJ;
  const size_t ngr = (n + RG - 1) / RG;
  Cand* partial;
  uint32_t* tickets;
  if (ar) {
    partial = (Cand*)ar->take(n * nch * sizeof(Cand));
    tickets = (uint32_t*)ar->take(ngr * 4);
    launch_fill_u32(c, tickets, ngr, 0);
  } else {
    partial = (Cand*)c->knn_tmp.get(n * nch * sizeof(Cand));
    tickets = (uint32_t*)c->tickets.get_zeroed(ngr * 4, c->stream);
  }
  // Queued rows: the count lives on the device, so the grid covers the worst
  // case. Queued rows are few: a grid of 2 blocks per CU covers them, and
  // blocks past the device-side count exit at once.
  const size_t items = ngr * nch;
  const unsigned g = (unsigned)std::min<size_t>(items, (size_t)(list ? 2 : 8) * c->cus);
  if (d % 4 == 0)
    hipLaunchKernelGGL(k_exact1<true>, dim3(g), dim3(64), 0, c->stream, x, nx, (int)d, ids, lo,
                       (int)n, list, c->small, cents, cnorm, (int)k, ip ? 1 : 0, partial, tickets,
                       labels, scores);
  else
    hipLaunchKernelGGL(k_exact1<false>, dim3(g), dim3(64), 0, c->stream, x, nx, (int)d, ids, lo,
                       (int)n, list, c->small, cents, cnorm, (int)k, ip ? 1 : 0, partial, tickets,
                       labels, scores);
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
