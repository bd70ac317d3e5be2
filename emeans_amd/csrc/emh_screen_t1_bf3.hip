// Instantiations of the 128 x 128 top-1 screen (k_screen, two 32-row blocks per wave, L1 lists)
// in bf16 three-pass MFMA arithmetic.
#include "emh_screen_kern.h"

namespace emh {

void launch_screen_t1_bf3(emh_ctx* c, const ScreenArgs& a, bool ip) {
  auto kern = a.d % 4 == 0 ? (ip ? k_screen<2, L1, false, false, true, true> : k_screen<2, L1, true, false, true, true>)
                           : (ip ? k_screen<2, L1, false, false, false, true> : k_screen<2, L1, true, false, false, true>);
  hipLaunchKernelGGL(kern, dim3(a.blocks), dim3(256), 0, c->stream, a.x, a.nx, (int)a.d, a.ids,
                     a.lo, (int)a.n, a.cents, a.cnorm, (int)a.k, a.tpp, a.parts, a.ntiles, a.cand,
                     c->small, a.xnorm);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
