// The update of one small training batch (up to USB positions) in one launch:
// scatter_add (core/cpu.rs:118-143, scatter_rows 337-375) and the EMA step
// (cpu.rs:389-432), for labels the batch's top-1 call tallied. The separate
// path places every position in a cluster-sorted order (k_place_scan), adds
// the sums (k_sums) and moves the centroids (k_ema): three launches whose
// few, small workgroups spend their time waiting on memory, which on the
// small fits of the automatic-k sweeps (64- to 256-row batches, a hundred
// steps per fit) is most of a step. Here the workgroup of cluster j
//   - reads the batch's labels and row ids (every position at once: a batch
//     is at most USB) and keeps the positions with label j, in order, by
//     ballots: the cluster's rows in selection order;
//   - adds them in that order from +0 (a thread per four columns), as k_sums;
//   - moves the centroid from the sums in registers, as k_ema: the position,
//     then either the squared norm (one lane adds the rounded squares in
//     order) with the bf16 halves and the bound's maximum, or the spherical
//     readout (v / max|v| over its sqrt of the in-order sum of squares);
//   - updates the mass and the epoch's count, and clears its count and the
//     tally's chunk histograms for the next batch.
// Every add and rounding is the separate path's, so the bits are the same.
// No workgroup reads what another writes.

#include "emh_halves.h"
#include "emh_internal.h"

namespace emh {
namespace {

constexpr int UT = 256;                // most threads per workgroup (d <= 4 UT)
constexpr int USB = UPDATE_SMALL_BATCH;  // most positions per batch
constexpr int USU = 16;                // row loads in flight per thread
constexpr uint32_t NOROW = 0xffffffffu;
static_assert(USB % 64 == 0 && UPDATE_SMALL_MAX_D <= 4 * UT, "shape");

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// The mass half of the EMA step (as k_ema and k_mass_preview compute it).
__device__ __forceinline__ float ema_mass(float u, uint32_t cnt, float alpha, float decay,
                                          int replace, float* weight) {
  if (!replace) u = u * decay;
  *weight = 0.0f;
  if (cnt > 0) {
    const float count = (float)cnt;
    const float retained = replace ? 0.0f : u;
    const float step = alpha * count;
    const float mass = retained + step;
    *weight = step / mass;
    u = mass;
  }
  return u;
}

// One element of a moved row: sum s of its n = count rows, old value p.
__device__ __forceinline__ float ema_value(float s, float p, float count, float weight) {
  const float mean = s / count;
  if (weight == 1.0f) return mean;
  const float diff = mean - p;
  const float inc = weight * diff;
  return p + inc;
}

// s0 + v[0] + ... + v[len - 1] in order (one lane; v 16-byte aligned LDS), two
// groups of 16 values' reads alternating with the adds (as k_ema's chain).
__device__ __forceinline__ float ordered_sum(const float* v, int len) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  typedef const float __attribute__((address_space(3)))* lf;
  typedef const f4 __attribute__((address_space(3)))* lf4;
  uint32_t base = (uint32_t)(uintptr_t)v;
  asm volatile("" : "+v"(base));
  const lf lv = (lf)(uintptr_t)base;
  auto load = [&](f4 (&g)[4], int t) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 4; u++) g[u] = *(lf4)(lv + t + 4 * u);
  };
  auto add = [](float s, const f4 (&g)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
      s = s + g[u].x;
      s = s + g[u].y;
      s = s + g[u].z;
      s = s + g[u].w;
    }
    return s;
  };
  float s = 0.0f;
  const int len16 = len & ~15;
  int t = 0;
  if (len16 > 0) {
    f4 a[4], b[4];
    load(a, 0);
    for (; t + 32 <= len16; t += 32) {
      load(b, t + 16);
      s = add(s, a);
      load(a, min(t + 32, len16 - 16));  // the last step reloads a group it has
      s = add(s, b);
    }
    if (t < len16) {
      s = add(s, a);
      t += 16;
    }
  }
  for (; t < len; t++) s = s + lv[t];
  return s;
}

struct SmallLds {
  uint32_t lst[USB];                 // the cluster's rows in order
  float sq[UPDATE_SMALL_MAX_D];      // rounded squares of the new row (or of the readout's)
  float wmax[UT / 64];               // readout: each wave's max |v|
  uint32_t cnt;
  float weight, rnorm;
};

// Cluster j = blockIdx.x, a thread per four columns in whole waves.
__global__ __launch_bounds__(UT) void k_update_small(
    const float* __restrict__ x, size_t nx, size_t d, const uint32_t* __restrict__ ids,
    size_t lo, size_t hi, const uint32_t* __restrict__ labels, size_t k,
    uint32_t* __restrict__ counts, uint32_t* __restrict__ zero_words, size_t nzero,
    float* __restrict__ acc, float* __restrict__ pos, float* __restrict__ usage, float alpha,
    float decay, int replace, float* __restrict__ norms, char* __restrict__ csplit,
    uint32_t* __restrict__ cpart, float* __restrict__ readout, uint32_t* __restrict__ tally,
    uint32_t* __restrict__ small, int f16) {
  __shared__ __attribute__((aligned(16))) SmallLds L;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nw = (int)(blockDim.x >> 6);
  const size_t j = blockIdx.x;
  const int d4 = (int)(d / 4);
  const int n = (int)(hi - lo);
  // The next batch's tally starts from zero; the screen's words too.
  for (size_t i = (size_t)blockIdx.x * blockDim.x + tid; i < nzero;
       i += (size_t)gridDim.x * blockDim.x)
    zero_words[i] = 0;
  if (blockIdx.x == 0 && tid < 3) small[tid] = 0;
  if (tid == 0) {
    const uint32_t cnt = counts[j];
    counts[j] = 0;  // read above by this thread only
    tally[j] += cnt;
    float wgt;
    usage[j] = ema_mass(usage[j], cnt, alpha, decay, replace, &wgt);
    L.cnt = cnt;
    L.weight = wgt;
  }
  // The batch's labels and row ids, every position at once (wave 0).
  uint32_t lab[USB / 64], rw[USB / 64];
  if (w == 0) {
#pragma unroll
    for (int u = 0; u < USB / 64; u++) {
      const int i = 64 * u + lane;
      const size_t p = lo + (size_t)i;
      lab[u] = i < n ? labels[p] : NOROW;
      rw[u] = i < n ? (ids ? ids[p] : (uint32_t)p) : NOROW;
    }
  }
  __syncthreads();
  const uint32_t cnt = L.cnt;
  if (cnt == 0) {  // the row stays; so do its norm, halves and readout
    if (tid == 0 && cpart) cpart[2 * j] = cpart[2 * j + 1] = __float_as_uint(norms[j]);
    return;
  }
  float4 p = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (tid < d4) p = reinterpret_cast<const float4*>(pos + j * d)[tid];
  if (w == 0) {
    uint32_t r = 0;
    bool bad = false;  // a row id past the data adds nothing; reported at the next read
#pragma unroll
    for (int u = 0; u < USB / 64; u++) {
      const bool m = lab[u] == (uint32_t)j;
      const uint64_t b = __ballot(m);
      if (m) {
        const uint32_t i = r + lanes_below(b);
        const bool ok = (size_t)rw[u] < nx;
        bad |= !ok;
        if (i < (uint32_t)USB) L.lst[i] = ok ? rw[u] : NOROW;
      }
      r += (uint32_t)__popcll(b);
    }
    if (bad) small[SW_BAD_ID] = 1;
  }
  __syncthreads();
  // The rows in order from +0 (as k_sums), USU row loads in flight.
  const uint32_t nr = min(cnt, (uint32_t)USB);
  float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float tmx = 0.0f;  // readout: max |v| of this thread's values (fold from 0, fmaxf)
  if (tid < d4) {
    for (uint32_t q = 0; q < nr; q += USU) {
      float4 rv[USU];
#pragma unroll
      for (int u = 0; u < USU; u++) {
        const uint32_t r = q + u < nr ? L.lst[q + u] : NOROW;
        rv[u] = r != NOROW ? reinterpret_cast<const float4*>(x + (size_t)r * d)[tid]
                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
#pragma unroll
      for (int u = 0; u < USU; u++)
        if (q + u < nr) {  // +0 for a bad row: s is never -0, so this adds nothing
          s.x = s.x + rv[u].x;
          s.y = s.y + rv[u].y;
          s.z = s.z + rv[u].z;
          s.w = s.w + rv[u].w;
        }
    }
    if (acc) {
      float4* ao = reinterpret_cast<float4*>(acc + j * d) + tid;
      const float4 a0 = *ao;
      *ao = make_float4(a0.x + s.x, a0.y + s.y, a0.z + s.z, a0.w + s.w);
    }
    const float count = (float)cnt, wgt = L.weight;
    v.x = ema_value(s.x, p.x, count, wgt);
    v.y = ema_value(s.y, p.y, count, wgt);
    v.z = ema_value(s.z, p.z, count, wgt);
    v.w = ema_value(s.w, p.w, count, wgt);
    reinterpret_cast<float4*>(pos + j * d)[tid] = v;
    if (norms) {
      *reinterpret_cast<float4*>(L.sq + 4 * tid) =
          make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
    } else if (readout) {
      tmx = fmaxf(fmaxf(fmaxf(fmaxf(tmx, fabsf(v.x)), fabsf(v.y)), fabsf(v.z)), fabsf(v.w));
    }
  }
  // The halves, with the zero columns of the last slab.
  if (csplit && tid < (int)(((d + 31) & ~(size_t)31) / 4)) {
    uint2 h, l;
    split_quad(v, h, l, f16 != 0);  // zeros past d
    const size_t col = 4 * (size_t)tid;
    char* o = csplit + ((col >> 5) * k + j) * SLAB_BYTES + quad_hi_offset((int)(col & 31) >> 2);
    *reinterpret_cast<uint2*>(o) = h;
    *reinterpret_cast<uint2*>(o + 32) = l;
  }
  if (norms) {
    __syncthreads();
    if (tid == 0) {
      const float nrm = ordered_sum(L.sq, (int)d);
      norms[j] = nrm;
      if (cpart) cpart[2 * j] = cpart[2 * j + 1] = __float_as_uint(nrm);
    }
    return;
  }
  if (!readout) return;
  // The spherical readout (faiss normalize_into, as k_normalize_rows): v /
  // max|v|, then / sqrt of the in-order sum of the squares.
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) tmx = fmaxf(tmx, __shfl_xor(tmx, o, 64));
  if (lane == 0) L.wmax[w] = tmx;
  __syncthreads();
  float mx = L.wmax[0];
  for (int i = 1; i < nw; i++) mx = fmaxf(mx, L.wmax[i]);
  const float s1 = mx > 0.0f ? mx : 1.0f;
  float4 qv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (tid < d4) {
    qv = make_float4(v.x / s1, v.y / s1, v.z / s1, v.w / s1);
    *reinterpret_cast<float4*>(L.sq + 4 * tid) =
        make_float4(qv.x * qv.x, qv.y * qv.y, qv.z * qv.z, qv.w * qv.w);
  }
  __syncthreads();
  if (tid == 0) L.rnorm = sqrtf(ordered_sum(L.sq, (int)d));
  __syncthreads();
  const float nv = L.rnorm;
  const float s2 = nv > 0.0f ? nv : 1.0f;
  if (tid < d4)
    reinterpret_cast<float4*>(readout + j * d)[tid] =
        make_float4(qv.x / s2, qv.y / s2, qv.z / s2, qv.w / s2);
}

}  // namespace

bool update_small(size_t n, size_t d, bool spherical) {
  return n > 0 && n <= (size_t)USB && d % 4 == 0 && d <= UPDATE_SMALL_MAX_D &&
         (!spherical || d <= EMA_READOUT_MAX_D);
}

void launch_update_small(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                         size_t lo, size_t hi, const uint32_t* labels, size_t k, uint32_t* counts,
                         uint32_t* tcnt, size_t ntcnt, float* acc, float* pos, float* usage,
                         float alpha, float decay, int replace, float* norms, void* csplit,
                         uint32_t* cpart, float* readout, uint32_t* tally, bool f16) {
  const size_t n = hi > lo ? hi - lo : 0;
  EMH_ENSURE(update_small(n, d, readout != nullptr) && tally && (norms != nullptr) != (readout != nullptr) &&
                 (!csplit || (norms && cpart)),
             "update: shape outside the small-batch path");
  if (k == 0) return;
  const unsigned threads = (unsigned)std::max<size_t>(64, (d / 4 + 63) / 64 * 64);
  hipLaunchKernelGGL(k_update_small, dim3((unsigned)k), dim3(threads), 0, c->stream, x, nx, d, ids,
                     lo, hi, labels, k, counts, tcnt, tcnt ? ntcnt : 0, acc, pos, usage, alpha,
                     decay, replace, norms, (char*)csplit, cpart, readout, tally, c->small,
                     f16 ? 1 : 0);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
