// Exact per-batch ops of the device loop: row norms, faiss normalize_into,
// the EMA step and the revival split. Each follows the reference CPU backend's
// f32 operation order (crates/emeans-core/src/core/cpu.rs) so results are
// bit-equal; the library is built with -ffp-contract=off so that no multiply
// and add the reference keeps separate is fused, and with IEEE f32 divide and
// sqrt and f32 denormals kept.
//
// These ops are HBM/latency-bound: they touch k x d floats once. A row's
// squared norm is a sequential chain of d adds (the reference sums in order),
// so one wave owns a row: its lanes square the elements in parallel into LDS
// and one lane adds them in order.

#include "emh_halves.h"
#include "emh_internal.h"

namespace emh {
namespace {

constexpr int WAVE = 64;
constexpr int WAVES = 4;   // waves per workgroup
constexpr int CH = 1024;   // elements per LDS chunk of one row

__global__ __launch_bounds__(256) void k_fill_u32(uint32_t* p, size_t n, uint32_t v) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

constexpr int NU = CH / WAVE;  // values per lane in one chunk

__device__ __forceinline__ void ld8(float4* q, const float* v) {
#pragma unroll
  for (int u = 0; u < 8; u++) q[u] = *reinterpret_cast<const float4*>(v + 4 * u);
}
__device__ __forceinline__ float add8(float s, const float4* q) {
#pragma unroll
  for (int u = 0; u < 8; u++) {
    s = s + q[u].x;
    s = s + q[u].y;
    s = s + q[u].z;
    s = s + q[u].w;
  }
  return s;
}

// s + v[0] + v[1] + ... + v[len - 1] in order (one lane), v a CH-float LDS
// slice: the next 32 values are read while the current 32 are added (reads
// clamped into the slice, so none is conditional).
__device__ __forceinline__ float seq_add(const float* v, int len, float s) {
  float4 a[8], b[8];
  ld8(a, v);
  int t = 0;
  for (; t + 64 <= len; t += 64) {
    ld8(b, v + t + 32);
    s = add8(s, a);
    ld8(a, v + min(t + 64, CH - 32));
    s = add8(s, b);
  }
  if (t + 32 <= len) {
    s = add8(s, a);
    t += 32;
  }
  for (; t < len; t++) s = s + v[t];
  return s;
}

// One chunk (len <= CH values) of a row into registers, lane-strided: every
// load issued before any is used (indices clamped into the chunk; the lanes'
// values past len are not used).
__device__ __forceinline__ void ld_chunk(float* r, const float* row, int len, int lane) {
#pragma unroll
  for (int u = 0; u < NU; u++) r[u] = row[min(lane + WAVE * u, len - 1)];
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sequential sum of rounded squares of row r (assign.rs:150-155): the lanes of
// wave w square one chunk into sq; lane 0 adds the chunk in column order.
__device__ float seq_sq_sum(const float* row, size_t d, float* sq, int lane) {
  float s = 0.0f;
  for (size_t c0 = 0; c0 < d; c0 += CH) {
    const int len = (int)min((size_t)CH, d - c0);
    float v[NU];
    ld_chunk(v, row + c0, len, lane);
#pragma unroll
    for (int u = 0; u < NU; u++)
      if (lane + WAVE * u < len) sq[lane + WAVE * u] = v[u] * v[u];
    wave_sync_lds();
    if (lane == 0) s = seq_add(sq, len, s);
    wave_sync_lds();
  }
  return s;  // valid in lane 0
}

__global__ __launch_bounds__(256) void k_row_norms(const float* __restrict__ m, size_t rows,
                                                   size_t d, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) float sq[WAVES][CH];
  int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  size_t r = (size_t)blockIdx.x * WAVES + w;
  if (r >= rows) return;  // whole wave; no workgroup barrier below
  float s = seq_sq_sum(m + r * d, d, sq[w], lane);
  if (lane == 0) out[r] = s;
}

__device__ inline float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
  return v;
}

// faiss normalize_into (core/cpu.rs:219-230): divide by max |v| (if > 0), then
// by sqrt of the sequential sum of squares of the divided row (if > 0).
__global__ __launch_bounds__(256) void k_normalize_rows(const float* __restrict__ src,
                                                        size_t rows, size_t d,
                                                        float* __restrict__ dst) {
  __shared__ __attribute__((aligned(16))) float sq[WAVES][CH];
  int w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  size_t r = (size_t)blockIdx.x * WAVES + w;
  if (r >= rows) return;
  const float* row = src + r * d;
  float* out = dst + r * d;
  if (d <= (size_t)CH) {  // one chunk: the row stays in registers for all three passes
    const int len = (int)d;
    float v[NU];
    ld_chunk(v, row, len, lane);
    float mx = 0.0f;  // fold from 0 with max(|v|): NaN never wins (fmaxf)
#pragma unroll
    for (int u = 0; u < NU; u++) mx = fmaxf(mx, lane + WAVE * u < len ? fabsf(v[u]) : 0.0f);
    mx = wave_max(mx);
    const float s1 = mx > 0.0f ? mx : 1.0f;
#pragma unroll
    for (int u = 0; u < NU; u++) {
      v[u] = v[u] / s1;
      if (lane + WAVE * u < len) sq[w][lane + WAVE * u] = v[u] * v[u];
    }
    wave_sync_lds();
    float s = 0.0f;
    if (lane == 0) s = seq_add(sq[w], len, s);
    s = __shfl(s, 0, WAVE);
    const float norm = sqrtf(s);
    const float s2 = norm > 0.0f ? norm : 1.0f;
#pragma unroll
    for (int u = 0; u < NU; u++)
      if (lane + WAVE * u < len) out[lane + WAVE * u] = v[u] / s2;
    return;
  }
  float mx = 0.0f;
  for (size_t t = lane; t < d; t += WAVE) mx = fmaxf(mx, fabsf(row[t]));
  mx = wave_max(mx);
  const float s1 = mx > 0.0f ? mx : 1.0f;
  float s = 0.0f;
  for (size_t c0 = 0; c0 < d; c0 += CH) {
    const int len = (int)min((size_t)CH, d - c0);
    float v[NU];
    ld_chunk(v, row + c0, len, lane);
#pragma unroll
    for (int u = 0; u < NU; u++)
      if (lane + WAVE * u < len) {
        const float q = v[u] / s1;
        sq[w][lane + WAVE * u] = q * q;
      }
    wave_sync_lds();
    if (lane == 0) s = seq_add(sq[w], len, s);
    wave_sync_lds();
  }
  s = __shfl(s, 0, WAVE);
  const float norm = sqrtf(s);
  const float s2 = norm > 0.0f ? norm : 1.0f;
  for (size_t t = lane; t < d; t += WAVE) out[t] = (row[t] / s1) / s2;
}

// s0 + v[0] + v[1] + ... + v[len - 1] in order (one lane; v 16-byte aligned
// LDS): two groups of 16 values alternate, one group's reads in
// flight while the other's are added. The base address goes through a VGPR:
// when the compiler proves it uniform it addresses the LDS from scalar
// registers with one 4-byte read per value, issued after the previous
// group's adds, and the chain waits on every group's reads.
__device__ __forceinline__ float ordered_sum(const float* v, int len, float s0 = 0.0f) {
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
  float s = s0;
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

// EMA step (core/cpu.rs:389-432): all masses decay unless replace; each cluster
// with rows gets mass = retained + alpha n, w = alpha n / mass and
// c = (w == 1) ? s / n : c + w (s / n - c), two roundings, no FMA.
// The mass half of the EMA step; *weight = alpha n / mass for a cluster with
// rows (0 otherwise). One function for the EMA kernel and the mass preview, so
// both compute the same bits.
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

// With norms != nullptr, also the squared norm of every updated row (the next
// batch's L2 readout, assign.rs:150-155); rows without members keep theirs.
// With csplit (norms too), also the bf16 halves of every updated row in the
// split-operand layout of k rows (emh_halves.h), so the next batch's screen
// need not split the centroids again (rows without members keep theirs), and
// cpart[2 b] = cpart[2 b + 1] = the largest norms[] of block b's rows (f32
// bits; a NaN wins): the bound's centroid maxima, as k_halves leaves them.
// Workgroup = EC clusters: the 256 threads update the clusters' positions
// element by element, then lane c of the first wave adds cluster c's rounded
// squares in order from LDS (rows padded by four floats so the EC lanes read
// different banks with aligned 16-byte reads); the chains of EC clusters run
// side by side.
constexpr int EC = 4;
// LDS floats per cluster row of k_ema: seg values rounded up to a multiple of
// four, plus four (rows stay 16-byte aligned).
__host__ __device__ constexpr int ema_row(int seg) { return ((seg + 3) & ~3) + 4; }
constexpr int TPC = 256 / EC;  // threads per cluster in the update
constexpr int ECH = 1024;  // dimensions per LDS pass
static_assert(ECH == (int)EMA_READOUT_MAX_D, "the fused readout takes one pass");
constexpr int EU = 16;    // elements per thread whose loads are in flight together
__global__ __launch_bounds__(256) void k_ema(float* __restrict__ pos, float* __restrict__ usage,
                                             const float* __restrict__ sums,
                                             const uint32_t* counts, size_t k,
                                             size_t d, float alpha, float decay, int replace,
                                             float* __restrict__ norms,
                                             uint32_t* __restrict__ clear3,
                                             uint32_t* __restrict__ tally,
                                             uint32_t* zero_counts,  // counts itself, or null
                                             char* __restrict__ csplit,
                                             uint32_t* __restrict__ cpart,
                                             uint32_t* __restrict__ zero_words, size_t nzero,
                                             float* __restrict__ readout, int f16) {
  // EC rows of min(d, ECH) + 4 floats (norms, or readout): the rounded
  // squares; with csplit or readout, then as many for the values.
  extern __shared__ __attribute__((aligned(16))) float sq[];
  __shared__ float wgt[EC], cntf[EC];
  const int tid = threadIdx.x;
  const size_t j0 = (size_t)blockIdx.x * EC;
  const int nc = (int)min((size_t)EC, k - j0);
  if (clear3 && blockIdx.x == 0 && tid < 3) clear3[tid] = 0;
  for (size_t i = (size_t)blockIdx.x * 256 + tid; i < nzero; i += (size_t)gridDim.x * 256)
    zero_words[i] = 0;
  if (tid < nc) {
    const uint32_t cnt = counts[j0 + tid];
    if (zero_counts) zero_counts[j0 + tid] = 0;  // the same array: read above, this thread only
    if (tally) tally[j0 + tid] += cnt;
    float weight;
    usage[j0 + tid] = ema_mass(usage[j0 + tid], cnt, alpha, decay, replace, &weight);
    wgt[tid] = cnt > 0 ? weight : -1.0f;  // -1: no rows, position unchanged
    cntf[tid] = (float)cnt;
  }
  __syncthreads();
  const int seg = (int)min(d, (size_t)ECH), row = ema_row(seg);
  float* vs = sq + EC * row;
  // Thread layout of the update: TPC threads per cluster, thread q of cluster
  // c takes dimensions q, q + TPC, ...
  const int c = tid / TPC, q = tid % TPC;
  const float weight = c < nc ? wgt[c] : -1.0f;
  const float count = c < nc ? cntf[c] : 1.0f;
  float nrm = 0.0f;  // lane c < nc of wave 0: cluster c's chain
  float tmx = 0.0f;  // readout: max |v| of this thread's values (fold from 0, fmaxf)
  for (size_t c0 = 0; c0 < d; c0 += ECH) {
    const int len = (int)min((size_t)ECH, d - c0);
    if (weight >= 0.0f) {
      float* p = pos + (j0 + c) * d + c0;
      const float* s = sums + (j0 + c) * d + c0;
      for (int t0 = q; t0 < len; t0 += TPC * EU) {
        float sv[EU], pv[EU];
#pragma unroll
        for (int u = 0; u < EU; u++) {
          const int t = t0 + TPC * u;
          sv[u] = t < len ? s[t] : 0.0f;
          pv[u] = t < len ? p[t] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < EU; u++) {
          const int t = t0 + TPC * u;
          if (t >= len) continue;
          const float mean = sv[u] / count;
          float v;
          if (weight == 1.0f) {
            v = mean;
          } else {
            const float diff = mean - pv[u];
            const float inc = weight * diff;
            v = pv[u] + inc;
          }
          p[t] = v;
          if (norms) sq[c * row + t] = v * v;
          if (csplit || readout) vs[c * row + t] = v;
          if (readout) tmx = fmaxf(tmx, fabsf(v));
        }
      }
    }
    if (!norms) continue;
    __syncthreads();
    if (csplit && tid >= WAVE) {
      // Waves 1-3 write the halves of the pass's dimensions (c0 is a
      // multiple of 32; the last slab's dimensions past d are zero) while
      // lanes of wave 0 run the chains.
      const int nq = (((int)len + 31) & ~31) >> 2;  // quads in the pass
      for (int e = tid - WAVE; e < EC * nq; e += 256 - WAVE) {
        const int cc = e / nq, t = 4 * (e % nq);
        if (cc >= nc || wgt[cc] < 0.0f) continue;
        const float* vr = vs + cc * row;
        const float4 v4 = make_float4(t < len ? vr[t] : 0.0f, t + 1 < len ? vr[t + 1] : 0.0f,
                                      t + 2 < len ? vr[t + 2] : 0.0f,
                                      t + 3 < len ? vr[t + 3] : 0.0f);
        uint2 hi, lw;
        split_quad(v4, hi, lw, f16 != 0);
        const size_t col = c0 + (size_t)t;
        char* o = csplit + ((col >> 5) * k + j0 + cc) * SLAB_BYTES + quad_hi_offset((int)(col & 31) >> 2);
        *reinterpret_cast<uint2*>(o) = hi;
        *reinterpret_cast<uint2*>(o + 32) = lw;
      }
    }
    if (tid < nc && wgt[tid] >= 0.0f) nrm = ordered_sum(sq + tid * row, len, nrm);  // in order
    __syncthreads();
  }
  if (readout) {
    // The spherical readout (faiss normalize_into, as k_normalize_rows: v /
    // max|v|, then / sqrt of the in-order sum of the squares) of each moved
    // row; d <= ECH, and a cluster is one wave (TPC == WAVE). Rows that did
    // not move keep their readout.
    __shared__ float rnorm[EC];
    const float mx = wave_max(tmx);
    const float s1 = mx > 0.0f ? mx : 1.0f;
    const int len = (int)d;
    if (weight >= 0.0f)
      for (int t = q; t < len; t += TPC) {
        const float qv = vs[c * row + t] / s1;
        vs[c * row + t] = qv;
        sq[c * row + t] = qv * qv;
      }
    __syncthreads();
    if (tid < nc && wgt[tid] >= 0.0f) rnorm[tid] = sqrtf(ordered_sum(sq + tid * row, len));
    __syncthreads();
    if (weight >= 0.0f) {
      const float nv = rnorm[c];
      const float s2 = nv > 0.0f ? nv : 1.0f;
      for (int t = q; t < len; t += TPC) readout[(j0 + c) * d + t] = vs[c * row + t] / s2;
    }
  }
  if (norms && tid < nc && wgt[tid] >= 0.0f) norms[j0 + tid] = nrm;
  if (cpart && tid < WAVE) {
    uint32_t m = 0u;
    if (tid < nc) m = __float_as_uint(wgt[tid] >= 0.0f ? nrm : norms[j0 + tid]);
#pragma unroll
    for (int o = 1; o < EC; o <<= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, WAVE));
    if (tid == 0) {
      cpart[2 * blockIdx.x] = m;
      cpart[2 * blockIdx.x + 1] = m;
    }
  }
}

// The masses the EMA step will leave (for the host's revival check), without
// touching the state.
// With seq_out, the block that takes the last ticket then posts seq there
// (system scope, after every block's writes): a host polling pinned memory
// sees the results as soon as they land, with no event on the stream.
__global__ __launch_bounds__(256) void k_mass_preview(const float* __restrict__ usage,
                                                      const uint32_t* __restrict__ counts,
                                                      size_t k, float alpha, float decay,
                                                      int replace, float* __restrict__ out,
                                                      const uint32_t* __restrict__ small,
                                                      uint32_t* __restrict__ small_out,
                                                      uint32_t* __restrict__ ticket,
                                                      uint32_t* __restrict__ seq_out,
                                                      uint32_t seq) {
  const size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (small_out && j < (size_t)SW_WORDS) small_out[j] = small[j];
  if (j < k) {
    float weight;
    out[j] = ema_mass(usage[j], counts[j], alpha, decay, replace, &weight);
  }
  if (!seq_out) return;  // uniform
  __threadfence_system();
  __shared__ int last;
  if (threadIdx.x == 0) last = atomicAdd(ticket, 1u) == gridDim.x - 1;
  __syncthreads();
  if (last && threadIdx.x == 0) {
    *ticket = 0;
    __threadfence_system();
    __hip_atomic_store(seq_out, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Label histogram of positions [0, n) (labels >= k are not counted).
__global__ __launch_bounds__(256) void k_hist(const uint32_t* __restrict__ labels, size_t n,
                                              size_t k, uint32_t* __restrict__ counts) {
  const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const uint32_t l = labels[p];
  if (l < k) atomicAdd(&counts[l], 1u);
}

// Closing means (core/mod.rs:404-429): sums / (f32)count where the last pass
// gave the cluster rows, else the position.
__global__ __launch_bounds__(256) void k_closing(const float* __restrict__ pos,
                                                 const float* __restrict__ sums,
                                                 const uint32_t* __restrict__ counts, size_t d,
                                                 float* __restrict__ out) {
  const size_t j = blockIdx.y;
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= d) return;
  const uint32_t cnt = counts[j];
  out[j * d + t] = cnt > 0 ? sums[j * d + t] / (float)cnt : pos[j * d + t];
}

// out[order[p]] = lab[p] for p < rows: the last pass's labels by data row.
__global__ __launch_bounds__(256) void k_labels_by_row(const uint32_t* __restrict__ order,
                                                       const uint32_t* __restrict__ lab,
                                                       size_t rows, size_t n,
                                                       uint32_t* __restrict__ out) {
  const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= rows) return;
  const uint32_t r = order[p];
  if (r < n) out[r] = lab[p];
}

// flag = 1 when any of v[0..n) is NaN or infinite.
__global__ __launch_bounds__(256) void k_check_finite(const float* __restrict__ v, size_t n,
                                                      uint32_t* __restrict__ flag) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n && !isfinite(v[i])) *flag = 1;
}

__device__ inline float next_up(float x) {  // f32::next_up
  if (x != x || x == INFINITY) return x;
  uint32_t b = __float_as_uint(x);
  if ((b & 0x7fffffffu) == 0) return __uint_as_float(1u);
  return __uint_as_float(x > 0.0f ? b + 1 : b - 1);
}
__device__ inline float next_down(float x) {  // f32::next_down
  return -next_up(-x);
}

// Revival split (core/mod.rs:374-399): donor c (1 - off), child c (1 + off),
// off = +-1e-4 alternating by column parity; if donor == child element-wise the
// child's first element moves one ulp up (down if that overflows); half of the
// donor's mass each. One workgroup per pair, or one workgroup walking the plan
// in order when pairs share a centroid.
__global__ __launch_bounds__(256) void k_split(float* __restrict__ pos, float* __restrict__ usage,
                                               const uint32_t* __restrict__ pairs, int npairs,
                                               size_t d, int sequential) {
  __shared__ int diff;
  int q0 = sequential ? 0 : (int)blockIdx.x;
  int q1 = sequential ? npairs : q0 + 1;
  const float eps = 1e-4f;
  for (int q = q0; q < q1; q++) {
    uint32_t s = pairs[2 * q], t = pairs[2 * q + 1];
    if (threadIdx.x == 0) diff = 0;
    __syncthreads();
    float* cs = pos + (size_t)s * d;
    float* ct = pos + (size_t)t * d;
    bool mine = false;
    for (size_t i = threadIdx.x; i < d; i += blockDim.x) {
      float off = eps * ((i % 2 == 0) ? 1.0f : -1.0f);
      float c = cs[i];
      float lo = 1.0f - off, hi = 1.0f + off;
      float dn = c * lo, ch = c * hi;
      mine = mine || !(dn == ch);
    }
    if (mine) atomicOr(&diff, 1);
    __syncthreads();
    const bool same = diff == 0;
    float half = usage[s] / 2.0f;
    __syncthreads();
    for (size_t i = threadIdx.x; i < d; i += blockDim.x) {
      float off = eps * ((i % 2 == 0) ? 1.0f : -1.0f);
      float c = cs[i];
      float lo = 1.0f - off, hi = 1.0f + off;
      float dn = c * lo, ch = c * hi;
      if (i == 0 && same) {
        float up = next_up(ch);
        ch = isfinite(up) ? up : next_down(ch);
      }
      cs[i] = dn;
      ct[i] = ch;
    }
    if (threadIdx.x == 0) {
      usage[s] = half;
      usage[t] = half;
    }
    __syncthreads();
  }
}

// k_split over independent pairs (no row is both a donor and a dead
// cluster), d <= SPLIT_FUSED_MAX_D, leaving also what the next batch reads of
// the two rows it moves, as a full row_norms and halves pass would: norms[s]
// and norms[t] (k_row_norms' in-order chain of the rounded squares); with
// csplit their bf16 halves in the split layout of k rows; with cpart the pair
// cpart[2 q] = cpart[2 q + 1] = the larger of the two norms (f32 bits), which
// the caller appends to the bound's centroid partials. The partials of the
// blocks the two rows were in stay upper bounds: no other row changed.
// Workgroup q = pair q. LDS: the two rows' values, then their squares, each
// row ema_row(d) floats.
__global__ __launch_bounds__(256) void k_split_fused(float* __restrict__ pos,
                                                     float* __restrict__ usage,
                                                     const uint32_t* __restrict__ pairs, size_t d,
                                                     size_t k, float* __restrict__ norms,
                                                     char* __restrict__ csplit,
                                                     uint32_t* __restrict__ cpart, int f16) {
  extern __shared__ __attribute__((aligned(16))) float sl[];
  __shared__ int diff;
  __shared__ float nv[2];
  const int tid = threadIdx.x, q = blockIdx.x, len = (int)d, row = ema_row(len);
  float* vs = sl;
  float* sq = sl + 2 * row;
  const uint32_t s = pairs[2 * q], t = pairs[2 * q + 1];
  if (tid == 0) diff = 0;
  __syncthreads();
  float* cs = pos + (size_t)s * d;
  float* ct = pos + (size_t)t * d;
  const float eps = 1e-4f;
  bool mine = false;
  for (int i = tid; i < len; i += 256) {
    const float off = eps * ((i % 2 == 0) ? 1.0f : -1.0f);
    const float c = cs[i];
    const float lo = 1.0f - off, hi = 1.0f + off;
    mine = mine || !(c * lo == c * hi);
  }
  if (mine) atomicOr(&diff, 1);
  __syncthreads();
  const bool same = diff == 0;
  const float half = usage[s] / 2.0f;
  __syncthreads();  // every thread has read usage[s]
  for (int i = tid; i < len; i += 256) {
    const float off = eps * ((i % 2 == 0) ? 1.0f : -1.0f);
    const float c = cs[i];
    const float lo = 1.0f - off, hi = 1.0f + off;
    const float dn = c * lo;
    float ch = c * hi;
    if (i == 0 && same) {
      const float up = next_up(ch);
      ch = isfinite(up) ? up : next_down(ch);
    }
    cs[i] = dn;
    ct[i] = ch;
    vs[i] = dn;
    vs[row + i] = ch;
    sq[i] = dn * dn;
    sq[row + i] = ch * ch;
  }
  if (tid == 0) {
    usage[s] = half;
    usage[t] = half;
  }
  __syncthreads();
  if (csplit) {
    // Quads of the two rows (the last slab's dimensions past d are zero),
    // beside the chains of lanes 0 and 1.
    const int nq = ((len + 31) & ~31) >> 2;
    for (int e = tid; e < 2 * nq; e += 256) {
      const int r = e / nq, c4 = 4 * (e % nq);
      const float* vr = vs + r * row;
      const float4 v4 = make_float4(c4 < len ? vr[c4] : 0.0f, c4 + 1 < len ? vr[c4 + 1] : 0.0f,
                                    c4 + 2 < len ? vr[c4 + 2] : 0.0f,
                                    c4 + 3 < len ? vr[c4 + 3] : 0.0f);
      uint2 hv, lv;
      split_quad(v4, hv, lv, f16 != 0);
      char* o = csplit + ((size_t)(c4 >> 5) * k + (r ? t : s)) * SLAB_BYTES +
                quad_hi_offset((c4 & 31) >> 2);
      *reinterpret_cast<uint2*>(o) = hv;
      *reinterpret_cast<uint2*>(o + 32) = lv;
    }
  }
  if (tid < 2) {
    const float nrm = ordered_sum(sq + tid * row, len);
    norms[tid ? t : s] = nrm;
    nv[tid] = nrm;
  }
  if (cpart) {
    __syncthreads();
    if (tid == 0) {
      const uint32_t m = max(__float_as_uint(nv[0]), __float_as_uint(nv[1]));
      cpart[2 * q] = m;
      cpart[2 * q + 1] = m;
    }
  }
}

// out[i] = x[ids[i]] (m rows of d); an id >= nx gives a zero row.
__global__ __launch_bounds__(256) void k_gather_rows(const float* __restrict__ x, size_t nx,
                                                     size_t d, const uint32_t* __restrict__ ids,
                                                     size_t m, float* __restrict__ out) {
  size_t i = blockIdx.y;
  size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m || t >= d) return;
  size_t r = ids[i];
  out[i * d + t] = r < nx ? x[r * d + t] : 0.0f;
}

}  // namespace

void launch_gather_rows(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                        size_t m, float* out) {
  if (m == 0) return;
  dim3 g((unsigned)((d + 255) / 256), (unsigned)m);
  hipLaunchKernelGGL(k_gather_rows, g, dim3(256), 0, c->stream, x, nx, d, ids, m, out);
  EMH_HIP(hipGetLastError());
}

void launch_fill_u32(emh_ctx* c, uint32_t* p, size_t n, uint32_t v) {
  if (n == 0) return;
  hipLaunchKernelGGL(k_fill_u32, grid1(n, 256), dim3(256), 0, c->stream, p, n, v);
  EMH_HIP(hipGetLastError());
}

void launch_row_norms(emh_ctx* c, const float* m, size_t rows, size_t d, float* out) {
  if (rows == 0) return;
  hipLaunchKernelGGL(k_row_norms, grid1(rows, WAVES), dim3(256), 0, c->stream, m, rows, d, out);
  EMH_HIP(hipGetLastError());
}

void launch_normalize_rows(emh_ctx* c, const float* src, size_t rows, size_t d, float* dst) {
  if (rows == 0) return;
  hipLaunchKernelGGL(k_normalize_rows, grid1(rows, WAVES), dim3(256), 0, c->stream, src, rows, d,
                     dst);
  EMH_HIP(hipGetLastError());
}

void launch_ema(emh_ctx* c, float* pos, float* usage, const float* sums, const uint32_t* counts,
                size_t k, size_t d, float alpha, float decay, int replace, float* norms,
                bool clear_screen_words, uint32_t* tally, bool zero_counts, void* csplit,
                uint32_t* cpart, uint32_t* zero_words, size_t nzero, float* readout, bool f16) {
  if (k == 0) return;
  EMH_ENSURE(!csplit || (norms && cpart), "ema: the centroid halves need the norms and maxima");
  EMH_ENSURE(!readout || (!norms && !csplit && d <= (size_t)ECH),
             "ema: the fused readout is for spherical runs with d <= %d", ECH);
  const size_t lds = norms || readout ? (size_t)EC * ema_row((int)std::min(d, (size_t)ECH)) *
                                            sizeof(float) * (csplit || readout ? 2 : 1)
                                      : 0;
  hipLaunchKernelGGL(k_ema, grid1(k, EC), dim3(256), lds, c->stream, pos, usage, sums, counts, k,
                     d, alpha, decay, replace, norms, clear_screen_words ? c->small : nullptr,
                     tally, zero_counts ? const_cast<uint32_t*>(counts) : nullptr,
                     (char*)csplit, cpart, zero_words, zero_words ? nzero : 0, readout,
                     f16 ? 1 : 0);
  EMH_HIP(hipGetLastError());
}

size_t ema_blocks(size_t k) { return (k + EC - 1) / EC; }

void launch_mass_preview(emh_ctx* c, const float* usage, const uint32_t* counts, size_t k,
                         float alpha, float decay, int replace, float* out, uint32_t* small_out,
                         uint32_t* seq_out, uint32_t seq) {
  if (k == 0) return;
  uint32_t* ticket = seq_out ? (uint32_t*)c->preview_ticket.get_zeroed(4, c->stream) : nullptr;
  hipLaunchKernelGGL(k_mass_preview, grid1(std::max(k, (size_t)SW_WORDS), 256), dim3(256), 0,
                     c->stream, usage, counts, k, alpha, decay, replace, out, c->small, small_out,
                     ticket, seq_out, seq);
  EMH_HIP(hipGetLastError());
}

void launch_hist(emh_ctx* c, const uint32_t* labels, size_t n, size_t k, uint32_t* counts) {
  launch_fill_u32(c, counts, k, 0);
  if (n == 0) return;
  hipLaunchKernelGGL(k_hist, grid1(n, 256), dim3(256), 0, c->stream, labels, n, k, counts);
  EMH_HIP(hipGetLastError());
}

void launch_closing(emh_ctx* c, const float* pos, const float* sums, const uint32_t* counts,
                    size_t k, size_t d, float* out) {
  if (k == 0) return;
  dim3 g((unsigned)((d + 255) / 256), (unsigned)k);
  hipLaunchKernelGGL(k_closing, g, dim3(256), 0, c->stream, pos, sums, counts, d, out);
  EMH_HIP(hipGetLastError());
}

void launch_labels_by_row(emh_ctx* c, const uint32_t* order, const uint32_t* lab, size_t rows,
                          size_t n, uint32_t* out) {
  launch_fill_u32(c, out, n, 0xffffffffu);  // -1 for rows the pass did not see
  if (rows == 0) return;
  hipLaunchKernelGGL(k_labels_by_row, grid1(rows, 256), dim3(256), 0, c->stream, order, lab, rows,
                     n, out);
  EMH_HIP(hipGetLastError());
}

void launch_check_finite(emh_ctx* c, const float* v, size_t n, uint32_t* flag) {
  if (n == 0) return;
  hipLaunchKernelGGL(k_check_finite, grid1(n, 256), dim3(256), 0, c->stream, v, n, flag);
  EMH_HIP(hipGetLastError());
}

void launch_split_fused(emh_ctx* c, float* pos, float* usage, const uint32_t* pairs_dev,
                        size_t npairs, size_t d, size_t k, float* norms, void* csplit,
                        uint32_t* cpart, bool f16) {
  if (npairs == 0) return;
  EMH_ENSURE(d >= 1 && d <= SPLIT_FUSED_MAX_D && norms, "split_fused: shape out of range");
  const size_t lds = 4 * (size_t)ema_row((int)d) * sizeof(float);
  hipLaunchKernelGGL(k_split_fused, dim3((unsigned)npairs), dim3(256), lds, c->stream, pos, usage,
                     pairs_dev, d, k, norms, (char*)csplit, cpart, f16 ? 1 : 0);
  EMH_HIP(hipGetLastError());
}

void launch_split(emh_ctx* c, float* pos, float* usage, const uint32_t* pairs_dev, size_t npairs,
                  size_t d, bool independent) {
  if (npairs == 0) return;
  dim3 g(independent ? (unsigned)npairs : 1u);
  hipLaunchKernelGGL(k_split, g, dim3(256), 0, c->stream, pos, usage, pairs_dev, (int)npairs, d,
                     independent ? 0 : 1);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
