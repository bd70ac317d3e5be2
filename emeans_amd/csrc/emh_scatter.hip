// scatter_add (core/cpu.rs:118-143, scatter_rows 337-375): per-label counts and
// sums of the selected rows, each sum added in selection order in f32 so the
// bits equal the CPU's. The order is a dependency chain per (cluster, column),
// so the work is split into a stable counting sort and ordered sums:
//   1. count:  labels -> counts (integer atomics; exact in any order); the
//              last workgroup to finish scans the counts into start offsets
//              and lists the clusters too large for the per-column path. For
//              k up to KCH the counts come from per-chunk LDS histograms of
//              CP positions, kept per chunk and added to the totals;
//   2. place:  each position's rank among the earlier positions of its label
//              (chunked: the sum of its label's earlier chunk histograms plus
//              a scan of its own chunk in LDS; else one wave per cluster
//              walking the labels with ballots), so each cluster's positions
//              land in order at its start offset;
//   3. sums (one launch, k_sums): clusters of up to SMALL rows: a
//              workgroup per cluster, a thread per four columns (d % 4 == 0;
//              else per column) adds the rows in order with SU4 (SU) row loads
//              in flight; larger clusters, beside them: a workgroup per
//              (cluster, 32-column strip); eight threads per column load the
//              next 128 rows into LDS while one lane per column adds the
//              current 128 in order, so a long chain waits on adds, not on
//              memory.
// HBM-bound: reads rows*d*4 bytes of rows (gathered by id) plus labels/ids,
// writes k*d*4 of sums (+ k*d*4 read/write of acc).

#include "emh_internal.h"

namespace emh {
namespace {

constexpr int WAVE = 64;
constexpr uint32_t NOROW = 0xffffffffu;
constexpr int SMALL = 128;  // largest cluster the per-column path takes
constexpr int SU = 32;      // row loads in flight per thread on that path
constexpr int BR = 128;     // rows per chunk on the large-cluster path
constexpr int BC = 32;      // columns per large-cluster workgroup
constexpr int BT = 256;     // threads per large-cluster workgroup (BT / BC per column)
constexpr int BIG_SLOTS = 32;  // large-cluster workgroup slots per strip

// Counts, then (last workgroup) exclusive scan into start[0..k] and the list
// of clusters with more than SMALL rows.
__global__ __launch_bounds__(256) void k_count(const uint32_t* __restrict__ labels, size_t lo,
                                               size_t hi, size_t k, uint32_t* __restrict__ counts,
                                               uint32_t* __restrict__ start,
                                               uint32_t* __restrict__ bigj,
                                               uint32_t* __restrict__ small) {
  __shared__ uint32_t part[256];
  __shared__ uint32_t nbig;
  __shared__ int last;
  const int tid = threadIdx.x;
  const size_t p = lo + (size_t)blockIdx.x * blockDim.x + tid;
  if (p < hi) {
    const uint32_t l = labels[p];
    if (l < k)
      atomicAdd(&counts[l], 1u);
    else
      small[SW_BAD_LABEL] = 1;
  }
  __threadfence();  // this workgroup's counts are visible before its ticket
  __syncthreads();
  if (tid == 0) {
    const uint32_t t = atomicAdd(&small[SW_TICKET], 1u);
    last = t == gridDim.x - 1;
    nbig = 0;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  // Thread t scans the run [t*per, (t+1)*per) of the counts.
  const size_t per = (k + 255) / 256;
  const size_t a = min(k, (size_t)tid * per), b = min(k, a + per);
  uint32_t s = 0;
  for (size_t j = a; j < b; j++)
    s += __hip_atomic_load(&counts[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  part[tid] = s;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {  // Hillis-Steele inclusive scan of the run totals
    const uint32_t add = tid >= o ? part[tid - o] : 0u;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  uint32_t run = part[tid] - s;
  for (size_t j = a; j < b; j++) {
    const uint32_t cj = __hip_atomic_load(&counts[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    start[j] = run;
    run += cj;
    if (cj > (uint32_t)SMALL) {
      const uint32_t i = atomicAdd(&nbig, 1u);
      bigj[3 * i] = (uint32_t)j;
      bigj[3 * i + 1] = run - cj;
      bigj[3 * i + 2] = cj;
    }
  }
  if (tid == 255) start[k] = part[255];
  __syncthreads();
  if (tid == 0) {
    small[SW_NBIG] = nbig;
    small[SW_TICKET] = 0;  // ready for the next call
  }
}

// ---- chunked count and placement (k <= KCH): positions in chunks of CP.
constexpr int CP = TALLY_CP;
constexpr int KCH = 8192;  // LDS histogram of one chunk
static_assert(CP == 256, "a chunk is one position per thread of a 256-thread block");

// Chunk c's label histogram (LDS atomics) goes to cnt[c][0..k) and is added
// to the totals counts[0..k) (zero on entry);
// the last workgroup to finish scans the totals into start[0..k] and lists
// the clusters above SMALL rows.
__global__ __launch_bounds__(256) void k_hist_total(const uint32_t* __restrict__ labels, size_t lo,
                                                    size_t hi, size_t k,
                                                    uint32_t* __restrict__ cnt,
                                                    uint32_t* __restrict__ counts,
                                                    uint32_t* __restrict__ start,
                                                    uint32_t* __restrict__ bigj,
                                                    uint32_t* __restrict__ small) {
  __shared__ uint32_t h[KCH];
  __shared__ uint32_t part[256];
  __shared__ uint32_t nbig;
  __shared__ int last;
  const int tid = threadIdx.x;
  const size_t c = blockIdx.x;
  for (size_t j = tid; j < k; j += 256) h[j] = 0;
  __syncthreads();
  const size_t p = lo + c * CP + tid;
  if (p < hi) {
    const uint32_t l = labels[p];
    if (l < k)
      atomicAdd(&h[l], 1u);
    else
      small[SW_BAD_LABEL] = 1;
  }
  __syncthreads();
  for (size_t j = tid; j < k; j += 256) {
    const uint32_t v = h[j];
    cnt[c * k + j] = v;
    if (v) atomicAdd(&counts[j], v);
  }
  __threadfence();  // this workgroup's counts are visible before its ticket
  __syncthreads();
  if (tid == 0) {
    const uint32_t t = atomicAdd(&small[SW_TICKET], 1u);
    last = t == gridDim.x - 1;
    nbig = 0;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  // Thread t scans the run [t*per, (t+1)*per) of the totals (per <= KCH / 256),
  // its loads all in flight at once and kept for the second pass.
  constexpr int PERMAX = KCH / 256;
  const size_t per = (k + 255) / 256;
  const size_t a = min(k, (size_t)tid * per), b = min(k, a + per);
  uint32_t tv[PERMAX];
#pragma unroll
  for (int u = 0; u < PERMAX; u++)
    tv[u] = a + u < b ? __hip_atomic_load(&counts[a + u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                      : 0u;
  uint32_t sacc = 0;
#pragma unroll
  for (int u = 0; u < PERMAX; u++) sacc += tv[u];
  part[tid] = sacc;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {  // Hillis-Steele inclusive scan of the run totals
    const uint32_t add = tid >= o ? part[tid - o] : 0u;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  uint32_t run = part[tid] - sacc;
#pragma unroll
  for (int u = 0; u < PERMAX; u++) {
    if (a + u >= b) break;
    start[a + u] = run;
    run += tv[u];
    if (tv[u] > (uint32_t)SMALL) {
      const uint32_t i = atomicAdd(&nbig, 1u);
      bigj[3 * i] = (uint32_t)(a + u);
      bigj[3 * i + 1] = run - tv[u];
      bigj[3 * i + 2] = tv[u];
    }
  }
  if (tid == 255) start[k] = part[255];
  __syncthreads();
  if (tid == 0) {
    small[SW_NBIG] = nbig;
    small[SW_TICKET] = 0;  // ready for the next call
  }
}

// Data row of position pos (NOROW, and the bad-id flag, when out of range).
__device__ __forceinline__ uint32_t row_of(const uint32_t* __restrict__ ids, size_t nx,
                                           uint32_t pos, uint32_t* __restrict__ small) {
  const size_t r = ids ? (size_t)ids[pos] : (size_t)pos;
  if (r >= nx) {  // a bad id adds nothing; reported at the next read
    small[SW_BAD_ID] = 1;
    return NOROW;
  }
  return (uint32_t)r;
}

// Position p of chunk c goes to rid[start[l] + (rows of label l in earlier
// chunks: the sum of the chunk histograms cnt[c'][l], c' < c, loads in flight
// together) + (rows of label l earlier in this chunk)], l = labels[p].
__global__ __launch_bounds__(256) void k_place_sum(const uint32_t* __restrict__ labels,
                                                    size_t lo, size_t hi, size_t k,
                                                    const uint32_t* __restrict__ start,
                                                    const uint32_t* __restrict__ cnt,
                                                    const uint32_t* __restrict__ ids, size_t nx,
                                                    uint32_t* __restrict__ small,
                                                    uint32_t* __restrict__ rid) {
  __shared__ __attribute__((aligned(16))) uint32_t lab[CP];
  const int tid = threadIdx.x;
  const size_t c = blockIdx.x;
  const size_t p = lo + c * CP + tid;
  const uint32_t l = p < hi ? labels[p] : 0xffffffffu;
  lab[tid] = l;
  __syncthreads();
  if (l >= k) return;
  uint32_t pre = 0;
  for (size_t c0 = 0; c0 < c; c0 += 64) {
    uint32_t v[64];
#pragma unroll
    for (int u = 0; u < 64; u++) v[u] = c0 + u < c ? cnt[(c0 + u) * k + l] : 0u;
#pragma unroll
    for (int u = 0; u < 64; u++) pre += v[u];
  }
  uint32_t rank = 0;
  const uint4* l4 = reinterpret_cast<const uint4*>(lab);
#pragma unroll 8
  for (int i4 = 0; i4 < CP / 4; i4++) {
    const uint4 q = l4[i4];
    const int i = 4 * i4;
    rank += (uint32_t)(i < tid && q.x == l) + (uint32_t)(i + 1 < tid && q.y == l) +
            (uint32_t)(i + 2 < tid && q.z == l) + (uint32_t)(i + 3 < tid && q.w == l);
  }
  rid[start[l] + pre + rank] = row_of(ids, nx, (uint32_t)p, small);
}

// k_place_sum for tallied labels (the top-1 call counted them: counts and the
// label-major chunk histograms cnt[label stride + chunk] are complete, and no
// k_hist_total ran; a label's earlier chunks are one contiguous run): every block
// scans the counts into start offsets in LDS itself, and block 0 also writes
// them to start[0..k] with the list of clusters above SMALL rows, for the
// sums that follow.
__global__ __launch_bounds__(256) void k_place_scan(const uint32_t* __restrict__ labels,
                                                     size_t lo, size_t hi, size_t k,
                                                     const uint32_t* __restrict__ counts,
                                                     const uint32_t* __restrict__ cnt,
                                                     size_t stride,
                                                     const uint32_t* __restrict__ ids, size_t nx,
                                                     uint32_t* __restrict__ small,
                                                     uint32_t* __restrict__ start,
                                                     uint32_t* __restrict__ bigj,
                                                     uint32_t* __restrict__ rid) {
  __shared__ uint32_t st[KCH];
  __shared__ uint32_t wsum[4];
  __shared__ __attribute__((aligned(16))) uint32_t lab[CP];
  __shared__ uint32_t nbig;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const size_t c = blockIdx.x;
  const size_t p = lo + c * CP + tid;
  // Thread t scans the run [t per, (t + 1) per) of the counts: its loads go
  // out first, beside the label's, ahead of the label's run.
  constexpr int PERMAX = KCH / 256;
  const size_t per = (k + 255) / 256;
  const size_t a = min(k, (size_t)tid * per), b = min(k, a + per);
  uint32_t tv[PERMAX];
#pragma unroll
  for (int u = 0; u < PERMAX; u++) tv[u] = a + u < b ? counts[a + u] : 0u;
  const uint32_t l = p < hi ? labels[p] : 0xffffffffu;
  // The position's row id, loaded beside the label; checked where it is used,
  // so that no wait on it comes before the run's loads.
  const uint32_t raw = p < hi ? (ids ? ids[p] : (uint32_t)p) : 0u;
  lab[tid] = l;
  // Rows of label l in earlier chunks: 16-byte loads of the label's run
  // (stride is a multiple of 4).
  // The loads are unconditional, clamped into the label's row (a load per
  // branch would wait before the next is issued), and masked after.
  uint32_t pre = 0;
  {
    const uint4* run4 = reinterpret_cast<const uint4*>(cnt + (size_t)(l < k ? l : 0u) * stride);
    const int n4 = l < k ? (int)((c + 3) >> 2) : 0, s4 = (int)(stride >> 2);
    for (int q0 = 0; q0 < n4; q0 += 16) {
      uint4 v[16];
#pragma unroll
      for (int u = 0; u < 16; u++) v[u] = run4[min(q0 + u, s4 - 1)];
#pragma unroll
      for (int u = 0; u < 16; u++) {
        const size_t e = 4 * (size_t)(q0 + u);
        pre += (e < c ? v[u].x : 0u) + (e + 1 < c ? v[u].y : 0u) + (e + 2 < c ? v[u].z : 0u) +
               (e + 3 < c ? v[u].w : 0u);
      }
    }
  }
  uint32_t sacc = 0;
#pragma unroll
  for (int u = 0; u < PERMAX; u++) sacc += tv[u];
  // Inclusive scan of the run totals: within each wave by shuffles, then
  // the earlier waves' totals.
  uint32_t inc = sacc;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = (uint32_t)__shfl_up((int)inc, o, 64);
    if (lane >= o) inc += t;
  }
  if (lane == 63) wsum[w] = inc;
  if (tid == 0) nbig = 0;
  __syncthreads();
  for (int i = 0; i < w; i++) inc += wsum[i];
  uint32_t run = inc - sacc;
#pragma unroll
  for (int u = 0; u < PERMAX; u++) {
    if (a + u >= b) break;
    st[a + u] = run;
    if (c == 0) {
      start[a + u] = run;
      if (tv[u] > (uint32_t)SMALL) {
        const uint32_t i = atomicAdd(&nbig, 1u);
        bigj[3 * i] = (uint32_t)(a + u);
        bigj[3 * i + 1] = run;
        bigj[3 * i + 2] = tv[u];
      }
    }
    run += tv[u];
  }
  __syncthreads();
  if (c == 0 && tid == 0) {
    start[k] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    small[SW_NBIG] = nbig;
  }
  if (l >= k) return;
  // Rows of label l earlier in the chunk: every position of the earlier
  // waves, then the lanes below this one in its own wave.
  uint32_t rank = 0;
  const uint4* l4 = reinterpret_cast<const uint4*>(lab);
  for (int i4 = 0; i4 < 16 * w; i4 += 8) {
    uint4 q[8];
#pragma unroll
    for (int u = 0; u < 8; u++) q[u] = l4[i4 + u];
#pragma unroll
    for (int u = 0; u < 8; u++)
      rank += (uint32_t)(q[u].x == l) + (uint32_t)(q[u].y == l) + (uint32_t)(q[u].z == l) +
              (uint32_t)(q[u].w == l);
  }
#pragma unroll 4
  for (int i4 = 16 * w; i4 < 16 * w + 16; i4++) {
    const uint4 q = l4[i4];
    const int i = 4 * i4;
    rank += (uint32_t)(i < tid && q.x == l) + (uint32_t)(i + 1 < tid && q.y == l) +
            (uint32_t)(i + 2 < tid && q.z == l) + (uint32_t)(i + 3 < tid && q.w == l);
  }
  uint32_t row = raw;
  if ((size_t)raw >= nx) {  // a bad id adds nothing; reported at the next read (as row_of)
    small[SW_BAD_ID] = 1;
    row = NOROW;
  }
  rid[st[l] + pre + rank] = row;
}

// Stable placement: wave j walks positions lo..hi in order; positions with
// label j go to rid[start[j] + rank], rank = number of earlier such positions.
// The block's waves share the labels, staged in LDS a segment at a time.
constexpr int SEG = 16384;
constexpr int PW = 4;  // waves (clusters) per block: k / 4 blocks spread over the CUs
__global__ __launch_bounds__(64 * PW) void k_place(const uint32_t* __restrict__ labels, size_t lo,
                                                size_t hi, size_t k,
                                                const uint32_t* __restrict__ start,
                                                const uint32_t* __restrict__ ids, size_t nx,
                                                uint32_t* __restrict__ small,
                                                uint32_t* __restrict__ rid) {
  __shared__ uint32_t lab[SEG];
  const int lane = threadIdx.x % WAVE;
  const size_t j = (size_t)blockIdx.x * PW + threadIdx.x / WAVE;
  uint32_t base = 0, end = 0;
  if (j < k) {
    base = start[j];
    end = start[j + 1];
  }
  for (size_t s0 = lo; s0 < hi; s0 += SEG) {
    const int len = (int)min((size_t)SEG, hi - s0);
    __syncthreads();
    for (int i0 = threadIdx.x; i0 < len; i0 += blockDim.x * 8) {  // 8 loads in flight
      uint32_t v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int i = i0 + (int)blockDim.x * u;
        v[u] = i < len ? labels[s0 + i] : 0u;
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int i = i0 + (int)blockDim.x * u;
        if (i < len) lab[i] = v[u];
      }
    }
    __syncthreads();
    for (int p0 = 0; p0 < len && base < end; p0 += 4 * WAVE) {
      uint32_t l[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int i = p0 + u * WAVE + lane;
        l[u] = i < len ? lab[i] : 0xffffffffu;
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const bool mine = l[u] == (uint32_t)j;
        const uint64_t m = __ballot(mine);
        if (mine) {
          const uint32_t rank = __builtin_amdgcn_mbcnt_hi(
              (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
          rid[base + rank] = row_of(ids, nx, (uint32_t)(s0 + p0 + u * WAVE + lane), small);
        }
        base += (uint32_t)__popcll(m);
      }
    }
  }
}

// Cluster j's sum of the rows rows[0..cnt) (in order; NOROW adds nothing)
// into sums[j] (and acc[j] += it), by the workgroup's 256 threads. rows is
// the cluster's run of the placement (global memory, read at uniform
// addresses: scalar loads, no staging). With VEC4 a thread adds four columns
// (16-byte loads, SU4 rows in flight), else one column (SU rows in flight).
constexpr int SU4 = 16;
template <bool VEC4>
__device__ __forceinline__ void sum_rows(const float* __restrict__ x, size_t d,
                                         const uint32_t* rows, uint32_t cnt, size_t j,
                                         float* __restrict__ sums, float* __restrict__ acc) {
  if (VEC4) {
    const size_t d4 = d / 4;
    for (size_t c4 = threadIdx.x; c4 < d4; c4 += blockDim.x) {
      float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
      for (uint32_t q = 0; q < cnt; q += SU4) {
        float4 v[SU4];
#pragma unroll
        for (int u = 0; u < SU4; u++) {
          const uint32_t r = q + u < cnt ? rows[q + u] : NOROW;
          v[u] = r != NOROW ? *reinterpret_cast<const float4*>(x + (size_t)r * d + 4 * c4)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < SU4; u++)
          if (q + u < cnt) {  // +0 for a bad row: s is never -0, so this adds nothing
            s.x = s.x + v[u].x;
            s.y = s.y + v[u].y;
            s.z = s.z + v[u].z;
            s.w = s.w + v[u].w;
          }
      }
      float4* so = reinterpret_cast<float4*>(sums + j * d) + c4;
      *so = s;
      if (acc) {
        float4* ao = reinterpret_cast<float4*>(acc + j * d) + c4;
        const float4 a0 = *ao;
        *ao = make_float4(a0.x + s.x, a0.y + s.y, a0.z + s.z, a0.w + s.w);
      }
    }
    return;
  }
  for (size_t col = threadIdx.x; col < d; col += blockDim.x) {
    float s = 0.0f;
    for (uint32_t q = 0; q < cnt; q += SU) {
      float v[SU];
#pragma unroll
      for (int u = 0; u < SU; u++) {
        const uint32_t r = q + u < cnt ? rows[q + u] : NOROW;
        v[u] = r != NOROW ? x[(size_t)r * d + col] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < SU; u++)
        if (q + u < cnt) s = s + v[u];  // +0 for a bad row: s is never -0, so this adds nothing
    }
    sums[j * d + col] = s;
    if (acc) acc[j * d + col] = acc[j * d + col] + s;
  }
}

// Clusters with more than SMALL rows (listed as (cluster, offset of its
// positions in rid, count) by the count kernels): workgroup = (listed
// cluster bi, strip of BC columns). Lane c < BC of wave 0 adds column c's
// rows in order, four per LDS read, from column-major chunks of BR rows
// (stride BRP) double-buffered in LDS; thread t loads rows RPT (t / BC) ..
// + RPT - 1 of each chunk in column t % BC. The loads run ahead of the adds
// in a software pipeline, so that the long chain of a large cluster waits on
// its adds rather than on memory: at step ch the values of chunk ch + 3 are
// loaded into one of three register sets (their row ids read from LDS), the
// values of chunk ch + 1 (loaded two steps before) go to LDS, and wave 0 adds
// chunk ch. Row ids come in blocks of IDB, loaded into registers one block
// ahead and stored to LDS four steps before their first use.
constexpr int BRP = BR + 4;          // column stride in LDS: 4-row accesses stay aligned
constexpr int RPT = BR * BC / BT;    // rows loaded per thread per chunk (16)
constexpr int IDB = 512;             // row ids per LDS block (four chunks)
constexpr int IDT = IDB / BT;        // ids loaded per thread per block
static_assert(IDB == 4 * BR && IDB % BT == 0 && RPT % 4 == 0, "pipeline shape");
__device__ __forceinline__ void sum_big(int bi, int strip, const float* __restrict__ x, size_t d,
                                        const uint32_t* __restrict__ rid,
                                        const uint32_t* __restrict__ bigj,
                                        float* __restrict__ sums, float* __restrict__ acc,
                                        float (*vals)[BC * BRP], uint32_t (*idl)[IDB]) {
  const uint32_t j = bigj[3 * bi], b = bigj[3 * bi + 1], cnt = bigj[3 * bi + 2];
  const int tid = threadIdx.x, c = tid % BC, g = tid / BC;
  const size_t col = (size_t)strip * BC + c;
  const bool colok = col < d;
  const float* xc = x + (colok ? col : 0);
  const uint32_t nch = (cnt + BR - 1) / BR;
  const uint32_t nblk = (cnt + IDB - 1) / IDB;
  uint32_t inext[IDT];
  // Loads are unconditional and nothing reads their results before the
  // step that needs them (ids past the cluster, and rows that add nothing,
  // are masked when stored), so that the compiler's waits come only where
  // the values are used.
  auto id_load = [&](uint32_t m) {
#pragma unroll
    for (int e = 0; e < IDT; e++) inext[e] = rid[b + min(m * IDB + tid + BT * e, cnt - 1)];
  };
  auto id_store = [&](uint32_t m) {
#pragma unroll
    for (int e = 0; e < IDT; e++) {
      const uint32_t i = m * IDB + tid + BT * e;
      idl[m & 1][tid + BT * e] = m < nblk && i < cnt ? inext[e] : NOROW;
    }
  };
  float v0[RPT], v1[RPT], v2[RPT];
  auto dload = [&](uint32_t ch, float (&v)[RPT]) -> uint32_t {  // returns the rows' mask
    const uint32_t* il = idl[(ch / 4) & 1] + (ch % 4) * BR + g * RPT;
    const bool live = ch < nch;
    uint32_t mk = 0;
#pragma unroll
    for (int u = 0; u < RPT; u++) {
      const uint32_t ri = il[u];
      const bool ok = live && ri != NOROW && colok;
      v[u] = xc[(size_t)(ok ? ri : 0u) * d];
      mk |= (uint32_t)ok << u;
    }
    return mk;
  };
  auto dstore = [&](uint32_t ch, const float (&v)[RPT], uint32_t mk) {
    if (ch >= nch) return;
    float* vb = vals[ch & 1] + c * BRP + g * RPT;
    auto m = [&](int u) { return (mk >> u) & 1u ? v[u] : 0.0f; };
#pragma unroll
    for (int u = 0; u < RPT; u += 4)
      *reinterpret_cast<float4*>(vb + u) = make_float4(m(u), m(u + 1), m(u + 2), m(u + 3));
  };
  float s = 0.0f;
  auto add = [&](uint32_t ch) {
    if (tid >= BC || ch >= nch) return;
    const uint32_t len = min((uint32_t)BR, cnt - ch * BR);
    const float* vc = vals[ch & 1] + tid * BRP;
    uint32_t i = 0;
    if (len >= 32) {  // the next 32 rows' LDS reads in flight while 32 are added
      float4 q[8], nq[8];
#pragma unroll
      for (int u = 0; u < 8; u++) q[u] = *reinterpret_cast<const float4*>(vc + 4 * u);
      for (; i + 32 <= len; i += 32) {
        const uint32_t in = i + 64 <= len ? i + 32 : i;  // the last group reloads itself
#pragma unroll
        for (int u = 0; u < 8; u++) nq[u] = *reinterpret_cast<const float4*>(vc + in + 4 * u);
#pragma unroll
        for (int u = 0; u < 8; u++) {
          s = s + q[u].x;
          s = s + q[u].y;
          s = s + q[u].z;
          s = s + q[u].w;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) q[u] = nq[u];
      }
    }
    for (; i < len; i++) s = s + vc[i];
  };
  // One step of the pipeline (see above); VL holds chunk ch + 3's loads,
  // VS chunk ch + 1's values.
  auto step = [&](uint32_t ch, float (&VL)[RPT], uint32_t& ML, const float (&VS)[RPT],
                  uint32_t MS) __attribute__((always_inline)) {
    ML = dload(ch + 3, VL);
    add(ch);
    __syncthreads();  // chunk ch - 1's buffer is free; chunk ch + 3's ids were read
    dstore(ch + 1, VS, MS);
    if (ch % 4 == 0) {  // block ch / 4 + 1's ids to LDS (its first chunk loads next step)
      id_store(ch / 4 + 1);
      id_load(ch / 4 + 2);
    }
    __syncthreads();
  };
  // Prologue: id block 0 in LDS, block 1 in registers; chunks 0-2 loaded,
  // chunk 0 stored.
  id_load(0);
  id_store(0);
  id_load(1);
  __syncthreads();
  uint32_t m0 = dload(0, v0), m1 = dload(1, v1), m2 = dload(2, v2);
  dstore(0, v0, m0);
  __syncthreads();
  for (uint32_t ch = 0; ch < nch; ch += 3) {
    step(ch, v0, m0, v1, m1);
    step(ch + 1, v1, m1, v2, m2);
    step(ch + 2, v2, m2, v0, m0);
  }
  if (tid < BC && colok) {
    sums[(size_t)j * d + col] = s;
    if (acc) acc[(size_t)j * d + col] = acc[(size_t)j * d + col] + s;
  }
}

// All the sums in one launch: workgroups [0, nbb) take (large cluster,
// strip) work (nbb = listed-cluster slots x strips; one past the clusters
// the count listed exits), the rest cluster j = blockIdx.x - nbb of up to
// SMALL rows. The large clusters' long in-order chains then run beside the
// small clusters' sums instead of after them.
template <bool VEC4>
__global__ __launch_bounds__(BT) void k_sums(const float* __restrict__ x, size_t nx, size_t d,
                                             const uint32_t* __restrict__ rid,
                                             const uint32_t* __restrict__ start, size_t k,
                                             const uint32_t* __restrict__ bigj, int strips,
                                             int nbb, float* __restrict__ sums,
                                             float* __restrict__ acc,
                                             uint32_t* __restrict__ small) {
  __shared__ __attribute__((aligned(16))) float vals[2][BC * BRP];
  __shared__ uint32_t idl[2][IDB];
  if ((int)blockIdx.x < nbb) {
    // Slot slot of nslots takes listed clusters slot, slot + nslots, ...
    const int slot = blockIdx.x / strips, strip = blockIdx.x % strips, nslots = nbb / strips;
    const int nbig = (int)small[SW_NBIG];
    for (int bi = slot; bi < nbig; bi += nslots)
      sum_big(bi, strip, x, d, rid, bigj, sums, acc, vals, idl);
    return;
  }
  const size_t j = blockIdx.x - nbb;
  const uint32_t b = start[j], cnt = start[j + 1] - b;
  if (cnt > (uint32_t)SMALL) return;  // a large cluster: done above
  sum_rows<VEC4>(x, d, rid + b, cnt, j, sums, acc);
}

}  // namespace

// The chunked path when the chunk histograms fit LDS and the last
// workgroup's per-label prefixes stay short; else per-cluster ballot walks.
static bool chunked(size_t n, size_t k) {
  const size_t nch = (n + CP - 1) / CP;
  return n > 0 && k <= (size_t)KCH && nch <= 256;
}

bool scatter_tallied(size_t n, size_t k) { return chunked(n, k); }

void launch_scatter_count(emh_ctx* c, size_t lo, size_t hi, const uint32_t* labels, size_t k,
                          uint32_t* counts, bool counts_zero) {
  const size_t n = hi > lo ? hi - lo : 0;
  uint32_t* start = (uint32_t*)c->start.get((k + 1) * 4);
  // Clusters above SMALL rows: at most n / (SMALL + 1) of them.
  const size_t maxbig = std::min(k, n / (SMALL + 1) + 1);
  uint32_t* bigj = (uint32_t*)c->bigj.get(maxbig * 12);
  if (chunked(n, k)) {
    const size_t nch = (n + CP - 1) / CP;
    uint32_t* cnt = (uint32_t*)c->chunkcnt.get(nch * k * 4);
    if (!counts_zero) launch_fill_u32(c, counts, k, 0);
    hipLaunchKernelGGL(k_hist_total, dim3((unsigned)nch), dim3(256), 0, c->stream, labels, lo,
                       hi, k, cnt, counts, start, bigj, c->small);
    EMH_HIP(hipGetLastError());
    return;
  }
  launch_fill_u32(c, counts, k, 0);
  if (n > 0) {
    hipLaunchKernelGGL(k_count, grid1(n, 256), dim3(256), 0, c->stream, labels, lo, hi, k, counts,
                       start, bigj, c->small);
    EMH_HIP(hipGetLastError());
  } else {
    launch_fill_u32(c, start, k + 1, 0);
    launch_fill_u32(c, c->small + SW_NBIG, 1, 0);
  }
}

void launch_scatter_sums(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                         size_t lo, size_t hi, const uint32_t* labels, size_t k, float* sums,
                         float* acc, const uint32_t* counts_tallied, const uint32_t* tally_cnt,
                         size_t tally_stride) {
  const size_t n = hi > lo ? hi - lo : 0;
  uint32_t* start = (uint32_t*)c->start.get((k + 1) * 4);
  uint32_t* rid = (uint32_t*)c->order.get(std::max<size_t>(n, 1) * 4);
  const size_t maxbig = std::min(k, n / (SMALL + 1) + 1);
  uint32_t* bigj = (uint32_t*)c->bigj.get(maxbig * 12);
  const int strips = (int)((d + BC - 1) / BC);
  if (counts_tallied) {
    EMH_ENSURE(chunked(n, k) && tally_cnt && tally_stride % 4 == 0 &&
                   tally_stride >= scatter_chunks(n),
               "scatter: tallied labels need the chunked path");
    hipLaunchKernelGGL(k_place_scan, dim3((unsigned)scatter_chunks(n)), dim3(256), 0, c->stream,
                       labels, lo, hi, k, counts_tallied, tally_cnt, tally_stride, ids, nx,
                       c->small, start, bigj, rid);
    EMH_HIP(hipGetLastError());
  } else if (chunked(n, k)) {
    const size_t nch = (n + CP - 1) / CP;
    const uint32_t* cnt = (const uint32_t*)c->chunkcnt.get(nch * k * 4);
    hipLaunchKernelGGL(k_place_sum, dim3((unsigned)nch), dim3(256), 0, c->stream, labels, lo, hi,
                       k, start, cnt, ids, nx, c->small, rid);
    EMH_HIP(hipGetLastError());
  } else if (n > 0) {
    hipLaunchKernelGGL(k_place, grid1(k, PW), dim3(64 * PW), 0, c->stream, labels, lo, hi, k,
                       start, ids, nx, c->small, rid);
    EMH_HIP(hipGetLastError());
  }
  // Workgroups for the large clusters: up to BIG_SLOTS slots of `strips`
  // each (a slot takes every BIG_SLOTS-th listed cluster), so that few
  // workgroups start only to find no cluster.
  const int nbb = n > (size_t)SMALL ? (int)(std::min(maxbig, (size_t)BIG_SLOTS) * strips) : 0;
  auto kern = d % 4 == 0 ? k_sums<true> : k_sums<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)(nbb + k)), dim3(BT), 0, c->stream, x, nx, d, rid, start,
                     k, bigj, strips, nbb, sums, acc, c->small);
  EMH_HIP(hipGetLastError());
}

void launch_scatter(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids, size_t lo,
                    size_t hi, const uint32_t* labels, size_t k, float* sums, uint32_t* counts,
                    float* acc) {
  launch_scatter_count(c, lo, hi, labels, k, counts, false);
  launch_scatter_sums(c, x, nx, d, ids, lo, hi, labels, k, sums, acc);
}

}  // namespace emh
