// softplus(x) of the dt projection (engine/mamba.py:300, F.softplus with
// beta 1, threshold 20, fp32) as a standalone pass, with the bits that the
// scan and step kernels compute on load (softplus_of).  The host uses it
// where it builds a rank-1 beta row [softplus(x) u | B] itself, so that the
// row matches the full beta that the kernels write.  One element per lane,
// a grid-stride loop over n.

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

__global__ __launch_bounds__(kThreads) void softplus_kernel(const float* x, float* out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
    out[i] = softplus_of(x[i]);
}

hipError_t launch_softplus(const float* x, float* out, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int64_t blocks = (n + kThreads - 1) / kThreads;
  const dim3 grid((unsigned)(blocks < 8192 ? blocks : 8192));
  hipLaunchKernelGGL(softplus_kernel, grid, dim3(kThreads), 0, st, x, out, n);
  return hipGetLastError();
}

}  // namespace rp
