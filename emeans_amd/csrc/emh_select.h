// Device helpers shared by the MFMA screen (emh_screen.hip), its check
// (emh_rescore.hip) and the exact scans (emh_verify.hip) of top-1 and top-k,
// and their launchers.
#pragma once

#include "emh_internal.h"

namespace emh {

constexpr uint32_t NONE = 0xffffffffu;
constexpr int L1 = 6;    // top-1: the smallest screen keys each part keeps
constexpr int L1S = 5;   // ... with the sorted insert (parts of several 256-centroid tiles)
constexpr int L1F = 10;  // ... on the fp16 two-pass screen (its bound admits more near-ties)
constexpr int C1 = 16;   // top-1: most candidates a row sends to the exact chains
constexpr int LK = 24;   // top-k list: kk <= 16 plus 7 spare + the bound
constexpr int KMAX = 16;  // largest kk of the screened top-k (emeans-core/src/knn.rs:16)
constexpr int MAX_PARTS = 8;  // centroid parts per row tile: lists per row the verify merges

// A screen candidate: key (smaller is better: -dot for IP, |c|^2 - 2 dot for L2) and id.
struct Cand {
  float key;
  uint32_t id;
};

// Insert (v, j) into an ascending list of L keys that keeps the L smallest.
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

// The same insertion without a branch: every slot takes its new value at once
// from the comparisons c[e] = v < key[e] of the old list. For a sorted list,
// slot e becomes key[e - 1] if v < key[e - 1], else min(v, key[e]), which is
// med3(key[e - 1], v, key[e]). v is first mapped to +inf when it is NaN or
// +inf, so such a key leaves the list unchanged; equal keys stay after the
// ones already in the list.
// Insert v into an ascending list of L keys that keeps the L smallest (no
// ids; v and the keys are numbers or +inf, never NaN). Branch-free.
template <int L>
__device__ __forceinline__ void insert_key(float (&key)[L], float v) {
#pragma unroll
  for (int e = L - 1; e > 0; e--) key[e] = __builtin_amdgcn_fmed3f(key[e - 1], v, key[e]);
  key[0] = fminf(v, key[0]);
}

template <int L>
__device__ __forceinline__ void insert_nb(float (&key)[L], uint32_t (&id)[L], float v,
                                          uint32_t j) {
  v = fminf(v, INFINITY);  // NaN -> +inf
  bool c[L];
#pragma unroll
  for (int e = 0; e < L; e++) c[e] = v < key[e];
#pragma unroll
  for (int e = L - 1; e > 0; e--) {
    key[e] = __builtin_amdgcn_fmed3f(key[e - 1], v, key[e]);
    id[e] = c[e - 1] ? id[e - 1] : (c[e] ? j : id[e]);
  }
  key[0] = fminf(v, key[0]);
  id[0] = c[0] ? j : id[0];
}

// The screens' arithmetic, as the bound follows it.
enum BoundKind : int {
  BOUND_F32 = 0,         // f32 MFMA screen
  BOUND_BF16 = 1,        // bf16 three-pass screen
  BOUND_BF16_TAGGED = 2, // the same with tagged keys (k_screen4, k_screen3 one tile per part)
  BOUND_F16_TAGGED = 3,  // fp16 two-pass screen with tagged keys (k_screen4 on fp16 halves)
};

// Screen error bound E on |key' - key| for one row (see emh_screen.hip):
// xn and cmax2 are squared norms summed in any order (relative error <= gamma_d,
// absorbed by the (1 + g) factors); cnmax bounds the given centroid norms.
// Terms of |dot' - dot|, with S >= sum_t |x_t c_t|:
//   the check's fma chain: gamma_d S;
//   f32 screen: the MFMA's sum in any order, taken at 2 gamma_d S, with a
//   denormal-flush floor of d 2^-124, and 2^-126 sqrt(d) (|x| + cmax) for
//   elements below 2^-126 that the MFMA may take as zero;
//   bf16 screen: the split (x ~ xh + xl, c ~ ch + cl, the xl.cl product
//   dropped): <= 3.05 * 2^-16 S, plus 2^-133 per element in the bf16
//   subnormal range, <= 2^-133 sqrt(d) (|x| + cmax) for the three products;
//   fp16 screen (xh.ch + xl.ch, fp16 halves as emh_halves.h states, products
//   exact in f32): per element |x||c - ch| + |ch||x - xh - xl| <=
//   (2^-11 + 2^-22 (1 + 2^-11)) |x c| + 2^-25 (1.0011) (|x| + |c|) + 2^-50,
//   so <= 4.89e-4 S + 2.9836e-8 sqrt(d) (|x| + cmax) + d 2^-50; valid while
//   every element is below 65520 in magnitude, which |x| <= 32768 and
//   cmax <= 32768 ensure: beyond that the bound is NaN (the exact scan);
//   the MFMA accumulation: M MFMAs in a chain (6 ceil(d / 32) bf16, 4 ceil(d
//   / 32) fp16), each within 16 u (|C| + sum |p|) (v_mfma_f32_32x32x16_bf16
//   and _f16 round each product to a grid relative to the largest term, then
//   round the sum once; measured <= 5.9 u for both, with exponents spread
//   over 2^-20 .. 2^20 and f16 subnormal inputs), so <= gamma(16 M) * 1.02 S
//   (the passes' |products| sum to <= 1.02 S); underflow: (3d + M) 2^-124.
// With edot_out, also the bound's dot term (unscaled, before the L2 key and
// tag allowances): the part that rests on the split and the MFMA model.
__device__ __forceinline__ float screen_bound(float xn, float cmax2, float cnmax, int d, bool l2,
                                              int kind, float* edot_out = nullptr) {
  const float u = 5.9604645e-08f;  // 2^-24
  const float du = (float)d * u;
  const float g = du / (1.0f - du);
  // A square or a partial sum in the subnormal range loses at most 2^-150, so
  // the true squared norm is at most the computed one plus d 2^-149 (a row or
  // centroid whose |.|^2 underflows still gets a bound that covers its dots).
  const float uf = (float)d * 1.4012985e-45f;  // d 2^-149
  const float xa = sqrtf(xn + uf) * (1.0f + g), ca = sqrtf(cmax2 + uf) * (1.0f + g);
  const float S = xa * ca;
  float edot;
  if (kind == BOUND_F16_TAGGED) {
    const float m = (float)(4 * ((d + 31) / 32));  // MFMAs per dot
    const float mu = 16.0f * m * u;
    const float gm = mu / (1.0f - mu);
    edot = (g + 1.02f * gm + 4.8900e-4f) * S                  // 2^-11 + 2^-22 (1 + 2^-11)
           + 2.9836e-8f * sqrtf((float)d) * (xa + ca)         // 2^-25 (1.0011)
           + (float)d * 8.8818e-16f                           // d 2^-50
           + (float)(3 * d + (int)m) * 4.7019774e-38f;        // 2^-124
    if (!(xa <= 32768.0f && ca <= 32768.0f)) edot = __builtin_nanf("");
  } else if (kind != BOUND_F32) {
    const float m = (float)(6 * ((d + 31) / 32));  // MFMAs per dot
    const float mu = 16.0f * m * u;
    const float gm = mu / (1.0f - mu);
    edot = (g + 1.02f * gm + 4.6539e-5f) * S            // 3.05 * 2^-16
           + 9.1835e-41f * sqrtf((float)d) * (xa + ca)   // 2^-133
           + (float)(3 * d + (int)m) * 4.7019774e-38f;   // 2^-124
  } else {
    edot = 3.0f * g * S + (float)d * 4.7019774e-38f   // + d 2^-124
           + 1.1754944e-38f * sqrtf((float)d) * (xa + ca);  // inputs below 2^-126 taken as 0
  }
  if (edot_out) *edot_out = edot;
  float e = l2 ? 2.0f * edot + 2.0f * u * (cnmax + 2.0f * S) : edot;
  // Tagged keys (the single-tile large-tile screens) carry a 6-bit column tag
  // in their low mantissa bits: |tagged - key| <= 63 ulp < 2^-17 |key|, with
  // |key| <= S (IP) or cnmax + 2S (L2), plus 63 subnormal ulps (< 2^-143).
  if (kind == BOUND_BF16_TAGGED || kind == BOUND_F16_TAGGED)
    e += 7.63e-6f * (l2 ? cnmax + 2.0f * S : S) + 8.9e-44f;
  return e * 1.125f;
}

// IEEE total order of f32 as a signed integer (f32::total_cmp).
__device__ __forceinline__ int32_t total_key(float v) {
  int32_t b = __float_as_int(v);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

// Merge a row's parts' lists (parts x L entries, laid out [part][L]) into one
// ascending list of L.
template <int L>
__device__ __forceinline__ void merge_parts(const Cand* c, int parts, float (&key)[L],
                                            uint32_t (&id)[L]) {
#pragma unroll
  for (int e = 0; e < L; e++) {
    key[e] = INFINITY;
    id[e] = NONE;
  }
  for (int q = 0; q < parts * L; q++) {
    const Cand v = c[q];
    if (v.id != NONE) insert<L>(key, id, v.key, v.id);
  }
}

// ---- emh_rescore.hip: merge, bound and re-score the screen's lists; xnorm[r]
// is row lo + r's |x|^2 summed in any order (the bound's input); bound: the
// screen's arithmetic (BoundKind).
void launch_verify1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                    size_t lo, size_t n, const float* cents, const float* cnorm, size_t k, bool ip,
                    const Cand* cand, int parts, const float* xnorm, uint32_t* labels,
                    float* scores, uint32_t* fb, int bound, const LabelTally* tally = nullptr,
                    int L = L1);
// The kNN screen over split operands (emh_screen4kn.hip): whether it takes a
// call, and the call's screen (candidate lists [m][parts][LK] and the queries'
// |q|^2, in the context's scratch); returns the parts.
bool screen4kn_fits(emh_ctx* c, size_t m, size_t n, size_t d);
int screen4kn(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
              size_t kk, bool exclude_self, Cand** cand, float** xnorm);
void launch_verifyk(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                    size_t kk, const Cand* cand, int parts, const float* xnorm, uint32_t* ids,
                    float* sims, uint32_t* fb);
// Re-score every entry of the screen's lists (rows lo..lo+n, parts x L
// entries each, laid out [row][part][L]) with the check's exact key and fill
// rep's pair count, pairs beyond the bound and max |screen key - exact key| / E
// (E from the row's |x|^2 and the call's bound words; bound as in
// launch_verify1). Waits for the result.
void launch_margin(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                   size_t lo, size_t n, const float* cents, const float* cnorm, bool ip,
                   const Cand* cand, int parts, int L, const float* xnorm, int bound,
                   emh_screen_report* rep);
// ---- emh_verify.hip: the exact scans
// Exact scan of rows `list[0..*count)` (list != nullptr) or positions lo..lo+n.
// ar: take the scratch from this fixed block (see Arena) instead of the context's buffers.
void launch_exact1(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids,
                   size_t lo, size_t n, const uint32_t* list, const float* cents,
                   const float* cnorm, size_t k, bool ip, uint32_t* labels, float* scores,
                   Arena* ar = nullptr, const LabelTally* tally = nullptr);
// Fixed-block bytes launch_exact1 takes for n rows (an upper bound).
size_t exact1_scratch_bytes(emh_ctx* c, size_t n, size_t d, size_t k, bool ip, bool list);
// The latency-bound scan's (k_queued1's) items for n rows against k centroids.
size_t queued_items(size_t n, size_t k, bool ip);
// Whether a direct selection of n rows takes the latency-bound scan instead
// of k_exact1: d % 4 == 0 and at most QUEUED_DIRECT of its items (and the
// context's exact_below not 0, which keeps k_exact1 for every selection).
inline bool queued_direct(emh_ctx* c, size_t n, size_t d, size_t k, bool ip) {
  return d % 4 == 0 && c->exact_below > 0 && queued_items(n, k, ip) <= QUEUED_DIRECT;
}
void launch_exactk(emh_ctx* c, const float* q, size_t m, const float* data, size_t n, size_t d,
                   size_t kk, bool exclude_self, const uint32_t* fb, uint32_t* ids, float* sims);

}  // namespace emh
