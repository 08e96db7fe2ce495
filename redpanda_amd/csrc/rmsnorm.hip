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
// take consecutive rows.  Rows up to 1024 features are held in registers.

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

// VPL > 0: the row (d <= 64 VPL) stays in registers between the sum of
// squares and the scaling, so x and add are read once; VPL == 0 reads them
// twice (any d).
template <int VPL>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_kernel(RmsNormParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * kWaves + threadIdx.x / kWave;
  if (row >= p.rows) return;
  const float invd = 1.f / (float)p.d;
  const float* x = p.x + row * p.xsr;
  float ss = 0.f;
  if constexpr (VPL > 0) {
    float v[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int i = lane + k * kWave;
      v[k] = i < p.d ? x[i] : 0.f;
    }
    if (p.add != nullptr) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const int i = lane + k * kWave;
        if (i < p.d) {
          v[k] = v[k] + load_in(p.add, row * p.asr + i, p.dt_add);
          p.x_out[row * p.d + i] = v[k];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < VPL; ++k) ss += v[k] * v[k];
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) ss += __shfl_xor(ss, m);
    const float r = rsqrtf(ss * invd + p.eps);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int i = lane + k * kWave;
      if (i < p.d) p.out[row * p.d + i] = (v[k] * r) * p.w[i];
    }
  } else {
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
}

hipError_t launch_rmsnorm_fwd(const RmsNormParams& p, hipStream_t st) {
  if (p.rows == 0 || p.d == 0) return hipSuccess;
  const dim3 grid((unsigned)((p.rows + kWaves - 1) / kWaves));
  if (p.d <= 4 * kWave)
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<4>, grid, dim3(kThreads), 0, st, p);
  else if (p.d <= 8 * kWave)
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<8>, grid, dim3(kThreads), 0, st, p);
  else if (p.d <= 16 * kWave)
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<16>, grid, dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(rmsnorm_fwd_kernel<0>, grid, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

}  // namespace rp
