// Residual add + RMSNorm of the batched step's residual stream, fused
// (engine/mamba.py:82-89 RMSNorm, :592-597 the pre-norm residual loop of
// Mamba.step): per row
//     x'  = x + add                      (fp32; add in its storage dtype)
//     out = (x' * rsqrt(mean(x'^2) + eps)) * w
// in torch's op order (x'^2 rounded, the mean as the sum times the fp32
// reciprocal of d, as torch's mean computes it).  Forward only: the
// inference loop of step(); training keeps torch's ops and their autograd.
//
// Layout: one wave per row (lanes stride the row, so every access is
// coalesced), a butterfly for the sum of squares; a workgroup's 4 waves
// take consecutive rows.

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_kernel(RmsNormParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * kWaves + threadIdx.x / kWave;
  if (row >= p.rows) return;
  const float invd = 1.f / (float)p.d;
  const float* x = p.x + row * p.xsr;
  float ss = 0.f;
  for (int i = lane; i < p.d; i += kWave) {
    float v = x[i];
    if (p.add != nullptr) {
      v = v + load_in(p.add, row * p.asr + i, p.dt_add);
      p.x_out[row * p.d + i] = v;
    }
    ss += v * v;
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) ss += __shfl_xor(ss, m);
  const float r = rsqrtf(ss * invd + p.eps);
  for (int i = lane; i < p.d; i += kWave) {
    float v = x[i];
    if (p.add != nullptr) v = v + load_in(p.add, row * p.asr + i, p.dt_add);
    p.out[row * p.d + i] = (v * r) * p.w[i];
  }
}

hipError_t launch_rmsnorm_fwd(const RmsNormParams& p, hipStream_t st) {
  if (p.rows == 0 || p.d == 0) return hipSuccess;
  const int64_t blocks = (p.rows + kWaves - 1) / kWaves;
  hipLaunchKernelGGL(rmsnorm_fwd_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

}  // namespace rp
