// Whole-tile (FAST) instantiations of the scan backward (kernel in
// scan_bwd_kernel.h): a translation unit of their own, compiled in parallel
// with the general ones in scan_bwd.hip.

#include "scan_bwd_kernel.h"

namespace rp {

template <int S, int NPL, class GK>
static hipError_t launch_bwd_fast_t(const ScanParams& p, const BwdIO& io, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)io.ntg * io.nbg));
  hipLaunchKernelGGL((scan_bwd_kernel<S, NPL, GK, true, false>), grid, dim3(kThreads), 0, st, p,
                     io);
  return hipGetLastError();
}

hipError_t launch_scan_bwd_fast(int S, int NPL, int gk, const ScanParams& p, const BwdIO& io,
                                hipStream_t st) {
  if (io.tpw > 1) return launch_scan_bwd_walk(S, NPL, gk, true, p, io, st);
#define RP_CASE(SS, NN)                                                              \
  if (S == SS && NN == NPL)                                                          \
    return with_gate_kind_scan<SS, NN>(gk, [&](auto g) {                                      \
      return launch_bwd_fast_t<SS, NN, decltype(g)>(p, io, st);                      \
    });
  RP_FOR_EACH_SHAPE(RP_CASE)
#undef RP_CASE
  return hipErrorInvalidValue;
}

}  // namespace rp
