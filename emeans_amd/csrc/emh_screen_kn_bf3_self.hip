// Instantiations of the kNN screen (k_screen, one 32-row block per wave, LK
// lists) in bf16 three-pass MFMA arithmetic, with exclude_self.
#include "emh_screen_kern.h"

namespace emh {

void launch_screen_kn_bf3_self(emh_ctx* c, const ScreenArgs& a) {
  auto kern = a.d % 4 == 0 ? k_screen<1, LK, false, true, true, true>
                           : k_screen<1, LK, false, true, false, true>;
  hipLaunchKernelGGL(kern, dim3(a.blocks), dim3(256), 0, c->stream, a.x, a.nx, (int)a.d, a.ids,
                     a.lo, (int)a.n, a.cents, a.cnorm, (int)a.k, a.tpp, a.parts, a.ntiles, a.cand,
                     c->small, a.xnorm);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
