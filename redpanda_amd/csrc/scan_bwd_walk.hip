// The scan backward's tile-walking (MULTI) instantiations for the 16-lane
// shapes (kernel in scan_bwd_kernel.h): a workgroup walks io.tpw adjacent
// 16-channel tiles, whose dB / dC partials add into one block.  A
// translation unit of its own, compiled in parallel with the others.

#include "scan_bwd_kernel.h"

namespace rp {

template <int S, int NPL, class GK, bool FAST>
static hipError_t launch_bwd_walk_t(const ScanParams& p, const BwdIO& io, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)io.ntg * io.nbg));
  hipLaunchKernelGGL((scan_bwd_kernel<S, NPL, GK, FAST, true>), grid, dim3(kThreads), 0, st, p,
                     io);
  return hipGetLastError();
}

hipError_t launch_scan_bwd_walk(int S, int NPL, int gk, bool fast, const ScanParams& p,
                                const BwdIO& io, hipStream_t st) {
#define RP_CASE(SS, NN)                                                              \
  if (S == SS && NN == NPL)                                                          \
    return with_gate_kind_scan<SS, NN>(gk, [&](auto g) {                                      \
      return fast ? launch_bwd_walk_t<SS, NN, decltype(g), true>(p, io, st)          \
                  : launch_bwd_walk_t<SS, NN, decltype(g), false>(p, io, st);        \
    });
  // the 16-lane shapes of RP_FOR_EACH_SHAPE
  RP_CASE(16, 3) RP_CASE(16, 4) RP_CASE(16, 5) RP_CASE(16, 6) RP_CASE(16, 8)
#undef RP_CASE
  return hipErrorInvalidValue;
}

}  // namespace rp
