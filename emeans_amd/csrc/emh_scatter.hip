// scatter_add (core/cpu.rs:118-143, scatter_rows 337-375): per-label counts and
// sums of the selected rows, each sum added in selection order in f32 so the
// bits equal the CPU's. The order is a dependency chain per (cluster, column),
// so the work is split three ways:
//   1. count:  labels -> counts (integer atomics; exact in any order);
//   2. scan:   counts -> start offsets (one workgroup);
//   3. place:  a stable counting sort: one wave per cluster walks the labels in
//              selection order with wave ballots and writes the cluster's data
//              row ids, in order, at its start offset;
//   4. sum:    per (cluster, column strip), rows added in that order; the loads
//              of a run of rows are issued together so the chain waits on adds,
//              not on memory.
// HBM-bound: reads rows*d*4 bytes of rows (gathered by id) plus labels/ids,
// writes k*d*4 of sums (+ k*d*4 read/write of acc).

#include "emh_internal.h"

namespace emh {
namespace {

constexpr int WAVE = 64;

__global__ __launch_bounds__(256) void k_count(const uint32_t* __restrict__ labels, size_t lo,
                                               size_t hi, size_t k, uint32_t* __restrict__ counts,
                                               uint32_t* __restrict__ small) {
  size_t p = lo + (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= hi) return;
  uint32_t l = labels[p];
  if (l < k)
    atomicAdd(&counts[l], 1u);
  else
    small[SW_BAD_LABEL] = 1;
}

// Exclusive scan of counts[0..k) into start[0..k]; start[k] = total. One workgroup.
__global__ __launch_bounds__(1024) void k_scan(const uint32_t* __restrict__ counts, size_t k,
                                               uint32_t* __restrict__ start) {
  __shared__ uint32_t part[1024];
  __shared__ uint32_t carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (size_t b = 0; b < k; b += 1024) {
    size_t j = b + threadIdx.x;
    uint32_t v = j < k ? counts[j] : 0;
    part[threadIdx.x] = v;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {  // Hillis-Steele inclusive scan
      uint32_t add = threadIdx.x >= (unsigned)o ? part[threadIdx.x - o] : 0;
      __syncthreads();
      part[threadIdx.x] += add;
      __syncthreads();
    }
    if (j < k) start[j] = carry + part[threadIdx.x] - v;
    __syncthreads();
    if (threadIdx.x == 1023) carry += part[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) start[k] = carry;
}

// Stable placement: wave j walks positions lo..hi in order; rows with label j
// go to rid[start[j] + rank], rank = number of earlier such rows. The block's
// waves share the labels, staged in LDS a segment of SEG at a time.
constexpr int SEG = 16384;
constexpr int PW = 4;  // waves (clusters) per block: k / 4 blocks spread over the CUs
__global__ __launch_bounds__(64 * PW) void k_place(const uint32_t* __restrict__ labels,
                                                const uint32_t* __restrict__ ids, size_t nx,
                                                size_t lo, size_t hi, size_t k,
                                                const uint32_t* __restrict__ start,
                                                uint32_t* __restrict__ rid,
                                                uint32_t* __restrict__ small) {
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
          const size_t p = s0 + p0 + u * WAVE + lane;
          uint32_t r = ids ? ids[p] : (uint32_t)p;
          if (r >= nx) {  // a bad id adds nothing; reported at the next read
            small[SW_BAD_ID] = 1;
            r = 0xffffffffu;
          }
          rid[base + rank] = r;
        }
        base += (uint32_t)__popcll(m);
      }
    }
  }
}

// Ordered sums: thread = column of cluster blockIdx.x; rows in rid order.
constexpr int U = 16;  // rows whose loads are in flight together
__global__ __launch_bounds__(256) void k_sum(const float* __restrict__ x, size_t d,
                                             const uint32_t* __restrict__ rid,
                                             const uint32_t* __restrict__ start, size_t k,
                                             float* __restrict__ sums, float* __restrict__ acc) {
  size_t j = blockIdx.x;
  size_t col = (size_t)blockIdx.y * blockDim.x + threadIdx.x;
  if (col >= d) return;
  const uint32_t b = start[j], e = start[j + 1];
  float s = 0.0f;
  uint32_t q = b;
  for (; q + U <= e; q += U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      uint32_t r = rid[q + u];
      v[u] = r != 0xffffffffu ? x[(size_t)r * d + col] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; u++) s = s + v[u];
  }
  for (; q < e; q++) {
    uint32_t r = rid[q];
    if (r != 0xffffffffu) s = s + x[(size_t)r * d + col];
  }
  sums[j * d + col] = s;
  if (acc) acc[j * d + col] = acc[j * d + col] + s;
}

}  // namespace

void launch_scatter(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids, size_t lo,
                    size_t hi, const uint32_t* labels, size_t k, float* sums, uint32_t* counts,
                    float* acc) {
  size_t n = hi > lo ? hi - lo : 0;
  uint32_t* start = (uint32_t*)c->start.get((k + 1) * 4);
  uint32_t* rid = (uint32_t*)c->order.get(std::max<size_t>(n, 1) * 4);
  launch_fill_u32(c, counts, k, 0);
  if (n > 0) {
    hipLaunchKernelGGL(k_count, grid1(n, 256), dim3(256), 0, c->stream, labels, lo, hi, k, counts,
                       c->small);
    EMH_HIP(hipGetLastError());
  }
  hipLaunchKernelGGL(k_scan, dim3(1), dim3(1024), 0, c->stream, counts, k, start);
  EMH_HIP(hipGetLastError());
  if (n > 0) {
    hipLaunchKernelGGL(k_place, grid1(k, PW), dim3(64 * PW), 0, c->stream, labels, ids, nx, lo,
                       hi, k, start, rid, c->small);
    EMH_HIP(hipGetLastError());
  }
  dim3 g((unsigned)k, (unsigned)((d + 255) / 256));
  hipLaunchKernelGGL(k_sum, g, dim3(256), 0, c->stream, x, d, rid, start, k, sums, acc);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
