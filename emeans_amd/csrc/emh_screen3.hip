// Instantiations of the large-tile bf16 top-1 screen (k_screen3).
#include "emh_screen_kern.h"

namespace emh {

void launch_screen3(emh_ctx* c, const ScreenArgs& a, bool ip, bool tagged) {
  auto kern = ip ? (tagged ? k_screen3<L1, false, true> : k_screen3<L1S, false, false>)
                 : (tagged ? k_screen3<L1, true, true> : k_screen3<L1S, true, false>);
  hipLaunchKernelGGL(kern, dim3(a.blocks), dim3(512), 0, c->stream, a.x, a.nx, (int)a.d, a.ids,
                     a.lo, (int)a.n, a.cents, a.cnorm, (int)a.k, a.tpp, a.parts, a.ntiles, a.cand,
                     c->small, a.xnorm);
  EMH_HIP(hipGetLastError());
}

}  // namespace emh
