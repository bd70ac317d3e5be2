// Instantiations of the split-operand large-tile screen (k_screen4: fp16
// two-pass or bf16 three-pass) and the kernel that splits rows into halves
// (k_halves).
#include <algorithm>

#include "emh_screen4.h"

namespace emh {

void launch_screen4(emh_ctx* c, const Screen4Args& a, bool ip) {
  // The kernel addresses a slab's rows with 32-bit byte offsets (128 per row)
  // and keeps one tile per part.
  EMH_ENSURE(a.nx < (1u << 25) && a.k < (1u << 25), "screen: more than 2^25 rows or centroids");
  EMH_ENSURE(a.tpp == 1 && a.parts == a.ntiles, "screen: one tile per part");
  auto kern = a.f16 ? (ip ? k_screen4<L1F, false, 8, true> : k_screen4<L1F, true, 8, true>)
                    : (ip ? k_screen4<L1, false, 8, false> : k_screen4<L1, true, 8, false>);
  hipLaunchKernelGGL(kern, dim3(a.blocks), dim3(512), 0, c->stream, (const char*)a.xs, a.xslab,
                     a.xn, a.nx, (int)a.d, a.ids, a.lo, (int)a.n, (const char*)a.cs, a.cslab,
                     a.cnorm, (int)a.k, a.tpp, a.parts, a.ntiles, a.cand, a.xnorm, a.part,
                     a.nparts, c->small);
  EMH_HIP(hipGetLastError());
}

namespace {
// out[0], out[1] = the largest part[2 i], part[2 i + 1] over i < nparts.
__global__ __launch_bounds__(256) void k_part_max(const uint32_t* __restrict__ part, size_t nparts,
                                                  uint32_t* __restrict__ out) {
  __shared__ uint32_t w[2][4];
  const int tid = threadIdx.x;
  uint32_t ma = 0, mb = 0;
  for (size_t i0 = 0; i0 < nparts; i0 += 256 * PMB) {
    uint2 v[PMB];
#pragma unroll
    for (int u = 0; u < PMB; u++) {
      const size_t i = i0 + 256 * (size_t)u + tid;
      v[u] = i < nparts ? reinterpret_cast<const uint2*>(part)[i] : make_uint2(0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < PMB; u++) {
      ma = max(ma, v[u].x);
      mb = max(mb, v[u].y);
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    ma = max(ma, (uint32_t)__shfl_xor((int)ma, o, 64));
    mb = max(mb, (uint32_t)__shfl_xor((int)mb, o, 64));
  }
  if ((tid & 63) == 0) {
    w[0][tid >> 6] = ma;
    w[1][tid >> 6] = mb;
  }
  __syncthreads();
  if (tid == 0) {
    out[0] = max(max(w[0][0], w[0][1]), max(w[0][2], w[0][3]));
    out[1] = max(max(w[1][0], w[1][1]), max(w[1][2], w[1][3]));
  }
}
}  // namespace

void launch_part_max(emh_ctx* c, const uint32_t* part, size_t nparts, uint32_t* out) {
  hipLaunchKernelGGL(k_part_max, dim3(1), dim3(256), 0, c->stream, part, nparts, out);
  EMH_HIP(hipGetLastError());
}

void launch_halves(emh_ctx* c, const float* x, size_t nx, size_t d, const uint32_t* ids, size_t lo,
                   size_t n, void* out, float* norm, const float* cnorm, uint32_t* part,
                   bool f16) {
  if (n == 0) return;
  EMH_ENSURE(d >= 1 && n < (1u << 31), "halves: shape out of range");
  auto kern = d % 4 == 0 ? k_halves<true> : k_halves<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)halves_blocks(n)), dim3(256), 0, c->stream, x, nx,
                     (int)d, ids, lo, n, (char*)out, norm, cnorm, part, f16 ? 1 : 0);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
