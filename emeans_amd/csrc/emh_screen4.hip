// Instantiations of the split-operand large-tile screen (k_screen4) and the
// kernel that splits rows into bf16 halves (k_halves).
#include <algorithm>

#include "emh_screen4.h"

namespace emh {

void launch_screen4(emh_ctx* c, const Screen4Args& a, bool ip) {
  // The kernel addresses a slab's rows with 32-bit byte offsets (128 per row)
  // and keeps one tile per part.
  EMH_ENSURE(a.nx < (1u << 25) && a.k < (1u << 25), "screen: more than 2^25 rows or centroids");
  EMH_ENSURE(a.tpp == 1 && a.parts == a.ntiles, "screen: one tile per part");
  auto kern = ip ? k_screen4<L1, false, 8> : k_screen4<L1, true, 8>;
  hipLaunchKernelGGL(kern, dim3(a.blocks), dim3(512), 0, c->stream, (const char*)a.xs, a.xslab,
                     a.xn, a.nx, (int)a.d, a.ids, a.lo, (int)a.n, (const char*)a.cs, a.cslab,
                     a.cnorm, (int)a.k, a.tpp, a.parts, a.ntiles, a.cand, a.xnorm, a.part,
                     a.nparts, c->small);
  EMH_HIP(hipGetLastError());
}

void launch_halves(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids, size_t lo,
                   size_t n, void* out, float* norm, const float* cnorm, uint32_t* part) {
  if (n == 0) return;
  EMH_ENSURE(d >= 1 && n < (1u << 31), "halves: shape out of range");
  auto kern = d % 4 == 0 ? k_halves<true> : k_halves<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)halves_blocks(n)), dim3(256), 0, c->stream, x, nx,
                     (int)d, ids, lo, n, (char*)out, norm, cnorm, part);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
