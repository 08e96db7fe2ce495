// The step tile kernel's instantiations for d_state below S * NPL (pad
// states; step_tile.h), in a translation unit of their own so that they
// compile beside step.hip's.

#include "step_tile.h"

namespace rp {

hipError_t launch_step_tile_pad(int S, int NPL, int gk, const StepParams& p, hipStream_t st) {
#define RP_CASE(SS, NN) \
  if (S == SS && NN == NPL) return launch_step_tile<SS, NN, true>(gk, p, st);
  RP_FOR_EACH_SHAPE(RP_CASE)
#undef RP_CASE
  return hipErrorInvalidValue;
}

}  // namespace rp
