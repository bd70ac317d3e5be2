// The MFMA screen kernels of top-1 and top-k (see emh_screen.hip for the
// three-stage design and the error bound), shared by the translation units
// that instantiate them: emh_screen3.hip (the large-tile bf16 top-1 screen),
// emh_screen_t1_*.hip (the 128 x 128 top-1 screen, bf16 or f32 arithmetic) and
// emh_screen_kn_*.hip (the kNN screen). Each unit compiles only its own
// instantiations, so the build runs them in parallel.
#pragma once

#include "emh_select.h"

namespace emh {
namespace {

constexpr int BK = 32;       // dimensions per LDS slab
constexpr int TC = 128;      // centroids per tile (two 32-blocks per wave, two waves)
constexpr int RB = BK * 2;   // bf16 screen: bytes per LDS row of one half, four 16-byte chunks
constexpr int LDK = BK + 4;  // f32 screen: padded LDS row (floats), conflict-free b128 reads

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// Work item of block `bid` of `nb`: blocks are dealt round-robin to the 8 XCDs
// (consecutive ids land on different XCDs), so number each XCD's blocks
// consecutively. The centroid parts of one row tile then run on one XCD at
// about the same time and share its L2.
__device__ __forceinline__ uint32_t xcd_swizzle(uint32_t bid, uint32_t nb) {
  uint32_t xcd = bid & 7, q = bid >> 3;
  uint32_t m = nb >> 3, r = nb & 7;
  return xcd * m + min(xcd, r) + q;
}

// Four consecutive elements p[col..col+4) of a valid row, loaded from an
// address clamped into the row (no branches). Elements at or past d are
// garbage here and zeroed by mask4 when the slab is stored to LDS, so that
// nothing waits for the load before the MFMAs of the current slab. VEC4
// (d % 4 == 0, d >= 4) uses one 16-byte load.
template <bool VEC4>
__device__ __forceinline__ float4 load4(const float* p, int col, int d) {
  if (VEC4) return *reinterpret_cast<const float4*>(p + min(col, d - 4));
  return make_float4(p[min(col, d - 1)], p[min(col + 1, d - 1)], p[min(col + 2, d - 1)],
                     p[min(col + 3, d - 1)]);
}
__device__ __forceinline__ float4 mask4(float4 v, int col, int d) {
  return make_float4(col < d ? v.x : 0.f, col + 1 < d ? v.y : 0.f, col + 2 < d ? v.z : 0.f,
                     col + 3 < d ? v.w : 0.f);
}

// Byte offset of 16-byte chunk q (dimensions 8q..8q+7 of the slab) of LDS row r:
// rows of RB bytes, chunks XOR-swizzled by row so that the sixteen lanes of a
// b128 access served together (sixteen consecutive rows, one chunk) hit
// sixteen different 16-byte bank groups of the 64-bank LDS, and eight too
// for eight lanes; a thread quad's store (one row, four chunks) likewise.
__device__ __forceinline__ int chunk_at(int r, int q) {
  return r * RB + ((q ^ ((r >> 1) & 3) ^ ((r >> 3) & 1)) << 4);
}

// x ~ hi + lo with hi = bf16(x) and lo = bf16(x - hi), both rounded to nearest
// even (x - hi is exact in f32): |x - hi - lo| <= 2^-16 |x| for normal values,
// <= 2^-134 in the bf16 subnormal range.
__device__ __forceinline__ void split8(float4 a, float4 b, v8bf& hi, v8bf& lo) {
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const __bf16 h = (__bf16)v[e];
    hi[e] = h;
    lo[e] = (__bf16)(v[e] - (float)h);
  }
}

// ---------------------------------------------------------------- screen
// Block: 256 threads = 4 waves; wave w: wr = w & 1 (row half), wc = w >> 1
// (centroid half). Block tile: TR = 64*WN rows x TC centroids per tile;
// each wave owns 32*WN rows x 64 centroids = (2 x WN) 32x32 MFMA blocks,
// A = centroids (M), B = rows (N); lane l holds row n = l % 32 of each block,
// so a row's keys stay in two lanes of a wave. The screen sums the K
// dimension in any order. Two arithmetics:
//  BF3 (default): the bf16 MFMA (v_mfma_f32_32x32x16_bf16, f32 accumulation)
//    in three passes, x.c ~ xh.ch + xh.cl + xl.ch, each slab's rows and
//    centroids split into bf16 halves when staged in LDS; lane half h takes
//    chunk 2s + h (8 dimensions) of k-step s of each slab;
//  f32: v_mfma_f32_32x32x2_f32, lane half h takes dimensions
//    [16h, 16h + 16) of each slab, four per b128 LDS read.
// Slabs are double-buffered in LDS; the global loads of the next slab are
// issued before the MFMAs of the current one and stored to the other buffer
// after them.
template <int WN, int L, bool L2, bool KNN, bool VEC4, bool BF3>
__global__ __launch_bounds__(256, 2) void k_screen(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int nrows, const float* __restrict__ cents, const float* __restrict__ cnorm, int k,
    int tiles_per_part, int parts, int ntiles, Cand* __restrict__ cand,
    uint32_t* __restrict__ small, float* __restrict__ xnorm) {
  constexpr int TR = 64 * WN;
  constexpr int XI = TR / 64;  // 8-dimension chunks per thread per slab (rows)
  constexpr int CI = TC / 64;  // 8-dimension chunks per thread per slab (centroids)
  // Bytes of one slab buffer: bf16 xh, xl, ch, cl, or f32 x, c.
  constexpr int BUF = BF3 ? 2 * (TR + TC) * RB : (TR + TC) * LDK * 4;
  // One LDS block: the slabs (double-buffered), reused for the final merge.
  __shared__ __attribute__((aligned(16))) char smem[2 * BUF];
  __shared__ float Ns[2][TC];
  auto xh_at = [&](int buf) { return smem + buf * BUF; };
  auto xl_at = [&](int buf) { return smem + buf * BUF + TR * RB; };
  auto ch_at = [&](int buf) { return smem + buf * BUF + 2 * TR * RB; };
  auto cl_at = [&](int buf) { return smem + buf * BUF + 2 * TR * RB + TC * RB; };
  auto xf_at = [&](int buf) { return reinterpret_cast<float*>(smem + buf * BUF); };
  auto cf_at = [&](int buf) { return reinterpret_cast<float*>(smem + buf * BUF + TR * LDK * 4); };

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w & 1, wc = w >> 1;
  const int li = lane & 31, h = lane >> 5;
  const uint32_t wi = xcd_swizzle(blockIdx.x, gridDim.x);
  const int rt = (int)(wi / (uint32_t)parts), part = (int)(wi % (uint32_t)parts);
  const int t0 = part * tiles_per_part;
  const int t1 = min(ntiles, t0 + tiles_per_part);
  if (t0 >= t1) return;
  const int row0 = rt * TR;

  // Loads: thread tid stages chunk q = tid & 3 (8 dimensions) of rows
  // (tid >> 2) + 64u of the slab. Rows past the selection (or with a bad id)
  // read data row 0; their lists are never written.
  const int q8 = tid & 3, r4 = tid >> 2;
  const float* xp[XI];
#pragma unroll
  for (int u = 0; u < XI; u++) {
    int r = row0 + r4 + 64 * u;
    size_t xid = 0;
    if (r < nrows) {
      size_t p = lo + (size_t)r;
      xid = ids ? (size_t)ids[p] : p;
      if (xid >= nx) xid = 0;
    }
    xp[u] = x + xid * (size_t)d;
  }

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
  float4 xr[XI][2], cr[CI][2];
  float nreg = 0.f;
  bool nvalid = false;

  // Load cursor (tile lt, slab ls) runs one step ahead of the compute cursor.
  int lt = t0, ls = 0;
  const float* cp[CI];  // centroid rows of tile lt (ids past k read centroid k-1)
  auto set_tile = [&](int tile) {
#pragma unroll
    for (int u = 0; u < CI; u++) {
      int j = min(tile * TC + r4 + 64 * u, k - 1);
      cp[u] = cents + (size_t)j * d;
    }
  };
  // The error bound's inputs, gathered on the way: max |c_j|^2 over the
  // centroids (each row's squares summed in any order; by the blocks of row
  // tile 0), and max cnorm[j]. Compared as f32 bit patterns: a NaN or negative
  // value wins and sends every row of the call to the exact scan.
  float csq[CI];
#pragma unroll
  for (int u = 0; u < CI; u++) csq[u] = 0.f;
  uint32_t cmax_bits = 0, cnmax_bits = 0;
  // Each row's |x|^2 in any order (for the verify's bound), summed while the
  // first tile streams the rows through; written by the blocks of part 0.
  float xsq[XI];
#pragma unroll
  for (int u = 0; u < XI; u++) xsq[u] = 0.f;
  auto gload = [&]() {
    const int col = ls * BK + 8 * q8;
#pragma unroll
    for (int u = 0; u < XI; u++) {
      xr[u][0] = load4<VEC4>(xp[u], col, d);
      xr[u][1] = load4<VEC4>(xp[u], col + 4, d);
    }
#pragma unroll
    for (int u = 0; u < CI; u++) {
      cr[u][0] = load4<VEC4>(cp[u], col, d);
      cr[u][1] = load4<VEC4>(cp[u], col + 4, d);
    }
    if (ls == 0 && tid < TC) {
      int j = lt * TC + tid;
      nvalid = j < k;
      nreg = L2 ? cnorm[min(j, k - 1)] : 0.f;
    }
  };
  auto sq8 = [](const float4 (&v)[2]) {
    return v[0].x * v[0].x + v[0].y * v[0].y + v[0].z * v[0].z + v[0].w * v[0].w +
           v[1].x * v[1].x + v[1].y * v[1].y + v[1].z * v[1].z + v[1].w * v[1].w;
  };
  // Stores the slab loaded by gload (masked past d), split into bf16 halves;
  // the first use of the loaded registers, so the loads overlap the MFMAs
  // issued in between. The mask and the norm sums are block-uniform branches:
  // only a final partial slab is masked; only part 0 sums its rows' squares
  // (during its first tile), and only row tile 0 the centroids' (its parts
  // together cover every centroid tile).
  auto lstore = [&](int buf) {
    const int col = ls * BK + 8 * q8;
    if (ls == nslabs - 1 && d % BK != 0) {
#pragma unroll
      for (int u = 0; u < XI; u++) {
        xr[u][0] = mask4(xr[u][0], col, d);
        xr[u][1] = mask4(xr[u][1], col + 4, d);
      }
#pragma unroll
      for (int u = 0; u < CI; u++) {
        cr[u][0] = mask4(cr[u][0], col, d);
        cr[u][1] = mask4(cr[u][1], col + 4, d);
      }
    }
    if constexpr (BF3) {
#pragma unroll
      for (int u = 0; u < XI; u++) {
        v8bf hi, lo8;
        split8(xr[u][0], xr[u][1], hi, lo8);
        const int at = chunk_at(r4 + 64 * u, q8);
        *reinterpret_cast<v8bf*>(xh_at(buf) + at) = hi;
        *reinterpret_cast<v8bf*>(xl_at(buf) + at) = lo8;
      }
#pragma unroll
      for (int u = 0; u < CI; u++) {
        v8bf hi, lo8;
        split8(cr[u][0], cr[u][1], hi, lo8);
        const int at = chunk_at(r4 + 64 * u, q8);
        *reinterpret_cast<v8bf*>(ch_at(buf) + at) = hi;
        *reinterpret_cast<v8bf*>(cl_at(buf) + at) = lo8;
      }
    } else {
#pragma unroll
      for (int u = 0; u < XI; u++) {
        float* dst = xf_at(buf) + (r4 + 64 * u) * LDK + 8 * q8;
        *reinterpret_cast<float4*>(dst) = xr[u][0];
        *reinterpret_cast<float4*>(dst + 4) = xr[u][1];
      }
#pragma unroll
      for (int u = 0; u < CI; u++) {
        float* dst = cf_at(buf) + (r4 + 64 * u) * LDK + 8 * q8;
        *reinterpret_cast<float4*>(dst) = cr[u][0];
        *reinterpret_cast<float4*>(dst + 4) = cr[u][1];
      }
    }
    if (part == 0 && lt == t0) {
#pragma unroll
      for (int u = 0; u < XI; u++) xsq[u] += sq8(xr[u]);
    }
    if (rt == 0) {
#pragma unroll
      for (int u = 0; u < CI; u++) csq[u] += sq8(cr[u]);
    }
    if (ls == 0 && tid < TC) {
      Ns[lt & 1][tid] = nvalid ? nreg : INFINITY;
      if (L2 && nvalid) cnmax_bits = max(cnmax_bits, __float_as_uint(nreg));
    }
  };
  auto advance = [&]() {
    if (++ls == nslabs) {
      // Tile lt fully loaded: its rows' squared norms (4 lanes per row).
      if (rt == 0) {
#pragma unroll
        for (int u = 0; u < CI; u++) {
          float s = csq[u];
          s += __shfl_xor(s, 1, 64);
          s += __shfl_xor(s, 2, 64);
          cmax_bits = max(cmax_bits, __float_as_uint(s));
          csq[u] = 0.f;
        }
      }
      if (part == 0 && lt == t0) {
#pragma unroll
        for (int u = 0; u < XI; u++) {
          float s = xsq[u];
          s += __shfl_xor(s, 1, 64);
          s += __shfl_xor(s, 2, 64);
          const int r = row0 + r4 + 64 * u;
          if (q8 == 0 && r < nrows) xnorm[r] = s;
        }
      }
      ls = 0;
      ++lt;
      if (lt < t1) set_tile(lt);
    }
  };

  set_tile(lt);
  gload();
  lstore(0);
  advance();
  __syncthreads();
  int ct = t0, cs_ = 0;  // compute cursor
  for (int st = 0; st < nsteps; st++) {
    const int buf = st & 1;
    const bool more = st + 1 < nsteps;
    if (more) gload();
    if constexpr (BF3) {
      const char* chs = ch_at(buf);
      const char* cls = cl_at(buf);
      const char* xhs = xh_at(buf);
      const char* xls = xl_at(buf);
#pragma unroll
      for (int s2 = 0; s2 < BK / 16; s2++) {
        const int q = 2 * s2 + h;
        v8bf ah[2], al[2], bh[WN], bl[WN];
#pragma unroll
        for (int a = 0; a < 2; a++) {
          const int at = chunk_at(wc * 64 + a * 32 + li, q);
          ah[a] = *reinterpret_cast<const v8bf*>(chs + at);
          al[a] = *reinterpret_cast<const v8bf*>(cls + at);
        }
#pragma unroll
        for (int y = 0; y < WN; y++) {
          const int at = chunk_at(wr * 32 * WN + y * 32 + li, q);
          bh[y] = *reinterpret_cast<const v8bf*>(xhs + at);
          bl[y] = *reinterpret_cast<const v8bf*>(xls + at);
        }
#pragma unroll
        for (int y = 0; y < WN; y++)
#pragma unroll
          for (int a = 0; a < 2; a++)
            acc[a][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[a], bh[y], acc[a][y], 0, 0, 0);
#pragma unroll
        for (int y = 0; y < WN; y++)
#pragma unroll
          for (int a = 0; a < 2; a++)
            acc[a][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[a], bl[y], acc[a][y], 0, 0, 0);
#pragma unroll
        for (int y = 0; y < WN; y++)
#pragma unroll
          for (int a = 0; a < 2; a++)
            acc[a][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[a], bh[y], acc[a][y], 0, 0, 0);
      }
    } else {
      const float* cs = cf_at(buf);
      const float* xs = xf_at(buf);
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
    }
    if (cs_ == nslabs - 1) {
      // Tile done: fold its keys into the per-row lists.
      const int tile = ct;
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
            float key = L2 ? fmaf(-2.0f, v, nn) : nn - v;  // one rounding: within E
            if (KNN && gj == qrow[y]) key = INFINITY;
            // Skipped by the whole wave when no lane's key beats its list's
            // last entry (the common case once the lists have filled).
            if (__ballot(key < lkey[y][L - 1]) != 0ull) insert_nb<L>(lkey[y], lid[y], key, gj);
            acc[a][y][r] = 0.f;
          }
        }
      }
    }
    if (++cs_ == nslabs) {
      cs_ = 0;
      ++ct;
    }
    if (more) {
      lstore(buf ^ 1);  // after this slab's MFMAs: the loads had all of them to land
      advance();
    }
    __syncthreads();
  }

  // Bound inputs: one atomic per block.
  __shared__ uint32_t red[8];
  {
    uint32_t a = cmax_bits, b = cnmax_bits;
    for (int o = 32; o > 0; o >>= 1) {
      a = max(a, (uint32_t)__shfl_xor((int)a, o, 64));
      b = max(b, (uint32_t)__shfl_xor((int)b, o, 64));
    }
    if (lane == 0) {
      red[w] = a;
      red[4 + w] = b;
    }
  }
  // Merge the four partial lists of each row (two lane halves x two waves).
  Cand* M = reinterpret_cast<Cand*>(smem);  // [TR][4][L]
  static_assert(TR * 4 * L * 8 <= 2 * BUF, "merge space");
  __syncthreads();
  if (tid == 0) {
    atomicMax(&small[SW_CMAX2], max(max(red[0], red[1]), max(red[2], red[3])));
    if (L2) atomicMax(&small[SW_CNMAX], max(max(red[4], red[5]), max(red[6], red[7])));
  }
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
    Cand* out = cand + ((size_t)(row0 + row) * parts + part) * L;  // [row][part][L]
#pragma unroll
    for (int e = 0; e < L; e++) out[e] = Cand{mk[e], mi[e]};
  }
}

// ------------------------------------------------- screen, large tiles
// The bf16 three-pass screen for top-1 when d % 4 == 0, on bigger tiles: with
// 64 x 64 per wave the slab stores and operand reads need ~0.9 KB of LDS
// traffic per MFMA, about what the LDS can serve while the MFMA pipe runs, so
// the pipe idled. Here a block is 8 waves (512 threads, one block per CU, two
// waves per SIMD) over TR3 = 256 rows x TC3 = 256 centroids per tile; wave w
// owns rows 64 (w & 3) .. + 64 (two 32-row B blocks) and centroids
// 128 (w >> 2) .. + 128 (four 32-centroid A blocks): 24 MFMAs per 12 b128
// operand reads per k-step, a third fewer LDS bytes per MFMA. The 128
// accumulator registers per lane sit in AGPRs. Staging, split, bound inputs,
// epilogue and merge are those of k_screen (one chunk quad per row per slab,
// 4 threads per row, two rows per thread for each operand).
constexpr int TR3 = 256, TC3 = 256;

template <int L, bool L2, bool TAG>
__global__ __launch_bounds__(512, 1) void k_screen3(
    const float* __restrict__ x, size_t nx, int d, const uint32_t* __restrict__ ids, size_t lo,
    int nrows, const float* __restrict__ cents, const float* __restrict__ cnorm, int k,
    int tiles_per_part, int parts, int ntiles, Cand* __restrict__ cand,
    uint32_t* __restrict__ small, float* __restrict__ xnorm) {
  constexpr int WA = 4, WN = 2;       // A (centroid) and B (row) 32-blocks per wave
  constexpr int BUF = 2 * (TR3 + TC3) * RB;  // xh, xl, ch, cl of one slab: 64 KB
  __shared__ __attribute__((aligned(16))) char smem[2 * BUF];
  __shared__ float Ns[2][TC3];
  auto xh_at = [&](int buf) { return smem + buf * BUF; };
  auto xl_at = [&](int buf) { return smem + buf * BUF + TR3 * RB; };
  auto ch_at = [&](int buf) { return smem + buf * BUF + 2 * TR3 * RB; };
  auto cl_at = [&](int buf) { return smem + buf * BUF + 2 * TR3 * RB + TC3 * RB; };

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wr = w & 3, wc = w >> 2;
  const int li = lane & 31, h = lane >> 5;
  const uint32_t wi = xcd_swizzle(blockIdx.x, gridDim.x);
  const int rt = (int)(wi / (uint32_t)parts), part = (int)(wi % (uint32_t)parts);
  const int t0 = part * tiles_per_part;
  const int t1 = min(ntiles, t0 + tiles_per_part);
  if (t0 >= t1) return;
  const int row0 = rt * TR3;

  // Staging: thread tid takes chunk q8 = tid & 3 of rows r4 + 128u (u < 2) of
  // both operands. Rows past the selection (or with a bad id) read data row 0;
  // their lists are never written.
  const int q8 = tid & 3, r4 = tid >> 2;
  const float* xp[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    int r = row0 + r4 + 128 * u;
    size_t xid = 0;
    if (r < nrows) {
      size_t p = lo + (size_t)r;
      xid = ids ? (size_t)ids[p] : p;
      if (xid >= nx) xid = 0;
    }
    xp[u] = x + xid * (size_t)d;
  }

  float lkey[WN][L];
  uint32_t lid[WN][L];
#pragma unroll
  for (int y = 0; y < WN; y++)
#pragma unroll
    for (int e = 0; e < L; e++) {
      lkey[y][e] = INFINITY;
      lid[y][e] = NONE;
    }

  v16f acc[WA][WN];
#pragma unroll
  for (int a = 0; a < WA; a++)
#pragma unroll
    for (int y = 0; y < WN; y++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[a][y][r] = 0.f;

  const int nslabs = (d + BK - 1) / BK;
  const int nsteps = (t1 - t0) * nslabs;
  float4 xr[2][2], cr[2][2];
  float nreg = 0.f;
  bool nvalid = false;
  int lt = t0, ls = 0;  // load cursor, one step ahead of the compute cursor
  const float* cp[2];
  auto set_tile = [&](int tile) {
#pragma unroll
    for (int u = 0; u < 2; u++) cp[u] = cents + (size_t)min(tile * TC3 + r4 + 128 * u, k - 1) * d;
  };
  float csq[2] = {0.f, 0.f}, xsq[2] = {0.f, 0.f};
  uint32_t cmax_bits = 0, cnmax_bits = 0;
  auto gload = [&]() {
    const int col = ls * BK + 8 * q8;
#pragma unroll
    for (int u = 0; u < 2; u++) {
      xr[u][0] = load4<true>(xp[u], col, d);
      xr[u][1] = load4<true>(xp[u], col + 4, d);
      cr[u][0] = load4<true>(cp[u], col, d);
      cr[u][1] = load4<true>(cp[u], col + 4, d);
    }
    if (ls == 0 && tid < TC3) {
      int j = lt * TC3 + tid;
      nvalid = j < k;
      nreg = L2 ? cnorm[min(j, k - 1)] : 0.f;
    }
  };
  auto sq8 = [](const float4 (&v)[2]) {
    return v[0].x * v[0].x + v[0].y * v[0].y + v[0].z * v[0].z + v[0].w * v[0].w +
           v[1].x * v[1].x + v[1].y * v[1].y + v[1].z * v[1].z + v[1].w * v[1].w;
  };
  auto lstore = [&](int buf) {
    const int col = ls * BK + 8 * q8;
    if (ls == nslabs - 1 && d % BK != 0) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        xr[u][0] = mask4(xr[u][0], col, d);
        xr[u][1] = mask4(xr[u][1], col + 4, d);
        cr[u][0] = mask4(cr[u][0], col, d);
        cr[u][1] = mask4(cr[u][1], col + 4, d);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int at = chunk_at(r4 + 128 * u, q8);
      v8bf hi, lo8;
      split8(xr[u][0], xr[u][1], hi, lo8);
      *reinterpret_cast<v8bf*>(xh_at(buf) + at) = hi;
      *reinterpret_cast<v8bf*>(xl_at(buf) + at) = lo8;
      split8(cr[u][0], cr[u][1], hi, lo8);
      *reinterpret_cast<v8bf*>(ch_at(buf) + at) = hi;
      *reinterpret_cast<v8bf*>(cl_at(buf) + at) = lo8;
    }
    if (part == 0 && lt == t0) {
#pragma unroll
      for (int u = 0; u < 2; u++) xsq[u] += sq8(xr[u]);
    }
    if (rt == 0) {
#pragma unroll
      for (int u = 0; u < 2; u++) csq[u] += sq8(cr[u]);
    }
    if (ls == 0 && tid < TC3) {
      Ns[lt & 1][tid] = nvalid ? nreg : INFINITY;
      if (L2 && nvalid) cnmax_bits = max(cnmax_bits, __float_as_uint(nreg));
    }
  };
  auto advance = [&]() {
    if (++ls == nslabs) {
      if (rt == 0) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
          float s = csq[u];
          s += __shfl_xor(s, 1, 64);
          s += __shfl_xor(s, 2, 64);
          cmax_bits = max(cmax_bits, __float_as_uint(s));
          csq[u] = 0.f;
        }
      }
      if (part == 0 && lt == t0) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
          float s = xsq[u];
          s += __shfl_xor(s, 1, 64);
          s += __shfl_xor(s, 2, 64);
          const int r = row0 + r4 + 128 * u;
          if (q8 == 0 && r < nrows) xnorm[r] = s;
        }
      }
      ls = 0;
      ++lt;
      if (lt < t1) set_tile(lt);
    }
  };

  set_tile(lt);
  gload();
  lstore(0);
  advance();
  __syncthreads();
  int ct = t0, cs_ = 0;
  for (int st = 0; st < nsteps; st++) {
    const int buf = st & 1;
    const bool more = st + 1 < nsteps;
    if (more) gload();
    const char* chs = ch_at(buf);
    const char* cls = cl_at(buf);
    const char* xhs = xh_at(buf);
    const char* xls = xl_at(buf);
#pragma unroll
    for (int s2 = 0; s2 < BK / 16; s2++) {
      const int q = 2 * s2 + h;
      v8bf bh[WN], bl[WN];
#pragma unroll
      for (int y = 0; y < WN; y++) {
        const int at = chunk_at(wr * 64 + y * 32 + li, q);
        bh[y] = *reinterpret_cast<const v8bf*>(xhs + at);
        bl[y] = *reinterpret_cast<const v8bf*>(xls + at);
      }
#pragma unroll
      for (int a = 0; a < WA; a++) {
        const int at = chunk_at(wc * 128 + a * 32 + li, q);
        const v8bf ah = *reinterpret_cast<const v8bf*>(chs + at);
        const v8bf al = *reinterpret_cast<const v8bf*>(cls + at);
#pragma unroll
        for (int y = 0; y < WN; y++)
          acc[a][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh[y], acc[a][y], 0, 0, 0);
#pragma unroll
        for (int y = 0; y < WN; y++)
          acc[a][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl[y], acc[a][y], 0, 0, 0);
#pragma unroll
        for (int y = 0; y < WN; y++)
          acc[a][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh[y], acc[a][y], 0, 0, 0);
      }
    }
    if (!TAG && cs_ == nslabs - 1) {
      // Tile done: fold its keys into the per-row lists.
      const int tile = ct;
      const float* ns = Ns[tile & 1];
#pragma unroll
      for (int a = 0; a < WA; a++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          // 32x32 accumulator layout: element (m, n) with n = lane % 32,
          // m = 8 (r / 4) + 4 (lane / 32) + r % 4.
          const int ci = wc * 128 + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          const uint32_t gj = (uint32_t)(tile * TC3 + ci);
          const float nn = ns[ci];
#pragma unroll
          for (int y = 0; y < WN; y++) {
            float v = acc[a][y][r];
            float key = L2 ? fmaf(-2.0f, v, nn) : nn - v;  // one rounding: within E
            if (__ballot(key < lkey[y][L - 1]) != 0ull) insert_nb<L>(lkey[y], lid[y], key, gj);
            acc[a][y][r] = 0.f;
          }
        }
      }
    }
    if (TAG && cs_ == nslabs - 1) {
      // Tile done, the part's only one. Each key carries its lane-local
      // column tag 16 a + r in its low 6 mantissa bits (the bound covers the
      // change), so that an insert of bare floats keeps the tile's L smallest
      // per row; the tags then give the ids.
      const int tile = ct;
      const float* ns = Ns[tile & 1];
      float tk[WN][L];
#pragma unroll
      for (int y = 0; y < WN; y++)
#pragma unroll
        for (int e = 0; e < L; e++) tk[y][e] = INFINITY;
#pragma unroll
      for (int a = 0; a < WA; a++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          // 32x32 accumulator layout: element (m, n) with n = lane % 32,
          // m = 8 (r / 4) + 4 (lane / 32) + r % 4.
          const int ci = wc * 128 + a * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          const float nn = ns[ci];
#pragma unroll
          for (int y = 0; y < WN; y++) {
            const float v = acc[a][y][r];
            float key = L2 ? fmaf(-2.0f, v, nn) : nn - v;  // one rounding: within E
            // NaN -> +inf (never a candidate), -inf -> -FLT_MAX (keeps its tag);
            // a tagged +inf is a NaN, which the compare below never takes.
            key = fmaxf(fminf(key, INFINITY), -3.4028235e38f);
            const float tagged =
                __uint_as_float((__float_as_uint(key) & ~63u) | (uint32_t)(16 * a + r));
            if (__ballot(tagged < tk[y][L - 1]) != 0ull)
              insert_key<L>(tk[y], tagged < tk[y][L - 1] ? tagged : INFINITY);
            acc[a][y][r] = 0.f;
          }
        }
      }
#pragma unroll
      for (int y = 0; y < WN; y++) {
#pragma unroll
        for (int e = 0; e < L; e++) {
          const float kv = tk[y][e];
          const uint32_t tg = __float_as_uint(kv) & 63u;
          const int ci = wc * 128 + (int)(tg >> 4) * 32 + 8 * (int)((tg & 15u) >> 2) + 4 * h +
                         (int)(tg & 3u);
          const uint32_t gj = kv < INFINITY ? (uint32_t)(tile * TC3 + ci) : NONE;
          if (__ballot(kv < lkey[y][L - 1]) != 0ull) insert_nb<L>(lkey[y], lid[y], kv, gj);
        }
      }
    }
    if (++cs_ == nslabs) {
      cs_ = 0;
      ++ct;
    }
    if (more) {
      lstore(buf ^ 1);
      advance();
    }
    __syncthreads();
  }

  // Bound inputs: one atomic per block.
  __shared__ uint32_t red[16];
  {
    uint32_t a = cmax_bits, b = cnmax_bits;
    for (int o = 32; o > 0; o >>= 1) {
      a = max(a, (uint32_t)__shfl_xor((int)a, o, 64));
      b = max(b, (uint32_t)__shfl_xor((int)b, o, 64));
    }
    if (lane == 0) {
      red[w] = a;
      red[8 + w] = b;
    }
  }
  // Merge the four partial lists of each row (two lane halves x two centroid waves).
  Cand* M = reinterpret_cast<Cand*>(smem);  // [TR3][4][L]
  static_assert(TR3 * 4 * L * 8 <= 2 * BUF, "merge space");
  __syncthreads();
  if (tid == 0) {
    uint32_t a = 0, b = 0;
    for (int i = 0; i < 8; i++) {
      a = max(a, red[i]);
      b = max(b, red[8 + i]);
    }
    atomicMax(&small[SW_CMAX2], a);
    if (L2) atomicMax(&small[SW_CNMAX], b);
  }
#pragma unroll
  for (int y = 0; y < WN; y++) {
    const int row = wr * 64 + y * 32 + li;
    const int contrib = wc * 2 + h;
#pragma unroll
    for (int e = 0; e < L; e++) M[(row * 4 + contrib) * L + e] = Cand{lkey[y][e], lid[y][e]};
  }
  __syncthreads();
  for (int row = tid; row < TR3; row += 512) {
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
    Cand* out = cand + ((size_t)(row0 + row) * parts + part) * L;  // [row][part][L]
#pragma unroll
    for (int e = 0; e < L; e++) out[e] = Cand{mk[e], mi[e]};
  }
}

}  // namespace

// Launch geometry and operands of one screen launch.
struct ScreenArgs {
  unsigned blocks;
  const float* x;
  size_t nx, d;
  const uint32_t* ids;
  size_t lo, n;
  const float* cents;
  const float* cnorm;
  size_t k;
  int tpp, parts, ntiles;
  Cand* cand;
  float* xnorm;
};

// The large-tile bf16 top-1 screen (emh_screen3.hip): d % 4 == 0; tagged keys
// when every part is one tile.
void launch_screen3(emh_ctx* c, const ScreenArgs& a, bool ip, bool tagged);

// Operands of the large-tile screen over split rows and centroids (emh_screen4.hip):
// xs, cs hold d32 = ceil(d / 32) slabs of 128 bytes per row, slab-major (slab
// j of row r at j * slab stride + 128 r); xn the rows' |x|^2.
struct Screen4Args {
  unsigned blocks;
  const void* xs;
  size_t xslab;
  const float* xn;
  size_t nx, d;
  const uint32_t* ids;
  size_t lo, n;
  const void* cs;
  size_t cslab;
  const float* cnorm;
  size_t k;
  int tpp, parts, ntiles;
  Cand* cand;
  float* xnorm;
  const uint32_t* part;  // the centroid split's per-block maxima (launch_halves' part)
  int nparts;
  bool f16;  // both operands in fp16 halves: the two-pass screen (else bf16, three passes)
};
void launch_screen4(emh_ctx* c, const Screen4Args& a, bool ip);
// The 128 x 128 top-1 screen (emh_screen_t1_{bf3,f32}.hip) and the kNN screen
// (emh_screen_kn_{bf3,f32}_{self,any}.hip), in bf16 three-pass or f32 MFMA arithmetic.
void launch_screen_t1_bf3(emh_ctx* c, const ScreenArgs& a, bool ip);
void launch_screen_t1_f32(emh_ctx* c, const ScreenArgs& a, bool ip);
void launch_screen_kn_bf3_self(emh_ctx* c, const ScreenArgs& a);
void launch_screen_kn_bf3_any(emh_ctx* c, const ScreenArgs& a);
void launch_screen_kn_f32_self(emh_ctx* c, const ScreenArgs& a);
void launch_screen_kn_f32_any(emh_ctx* c, const ScreenArgs& a);

}  // namespace emh
