// The SSM input prologue, fused: BCNorm on the B and C projections and the
// MIMO contraction over p (engine/mamba.py:89 RMSNorm, :297-300 BCNorm and
// view, :336-337 sum over p):
//     r   = rsqrt(mean_j x_j^2 + eps)           (j over the N*P features)
//     Bc[n] = sum_p (x[n,p] * r) * w[n,p]       (fp32; p in order)
// for x = B_raw and C_raw of every token, or the plain p-sum when the
// layer has no BCNorm.  The backward is autograd's of the same ops:
//     gxr_j = g_n w_j,   grad_r = sum_j gxr_j x_j
//     gm    = (-0.5 grad_r) r^3,   dx_j = round(gxr_j r) + round((gm / K) 2 x_j)
// (1/K as the fp32 reciprocal, as torch's mean and its backward use it)
//     dw_j  = sum over tokens of g_n (x_j r)     (fixed-order float64 partials)
// with rounding to x's storage dtype where torch's ops round.
//
// Layout: one wave per token and part (B or C); lane l takes states l and
// l + 64 (N <= 128) and their P <= 8 consecutive features.  A workgroup's 4
// waves walk a contiguous range of tokens; the backward's dw partials are
// combined across the 4 waves in LDS and written per workgroup, then summed
// by a second kernel in a fixed order.

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

namespace {

__device__ __forceinline__ float round_dt(float v, int dtype) {
  if (dtype == RP_F32) return v;
  if (dtype == RP_BF16) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7f800000u) != 0x7f800000u) b += 0x7fffu + ((b >> 16) & 1u);
    return __uint_as_float(b & 0xffff0000u);
  }
  return static_cast<float>(static_cast<_Float16>(v));
}

__device__ __forceinline__ void store_dt(void* p, int64_t i, float v, int dtype) {
  if (dtype == RP_F32) {
    static_cast<float*>(p)[i] = v;
  } else if (dtype == RP_BF16) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(__float_as_uint(round_dt(v, RP_BF16)) >> 16);
  } else {
    static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
  }
}

// The token range of a workgroup and the token stride of its waves.
__device__ __forceinline__ void token_range(const BcNormParams& p, int64_t& t0, int64_t& t1) {
  t0 = (int64_t)blockIdx.x * p.tokens_per_group;
  t1 = min(p.T, t0 + p.tokens_per_group);
}

}  // namespace

// Forward: x (T rows, row stride xs) -> out (T, N) fp32.
template <int SL>
__global__ __launch_bounds__(kThreads) void bcnorm_fwd_kernel(BcNormParams p) {
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int K = p.N * p.P;
  const float invK = 1.f / (float)K;
  int64_t t0, t1;
  token_range(p, t0, t1);
  float wt[2][SL][kBcMaxP];
#pragma unroll
  for (int part = 0; part < 2; ++part)
#pragma unroll
    for (int s = 0; s < SL; ++s) {
      const int n = lane + s * kWave;
#pragma unroll
      for (int q = 0; q < kBcMaxP; ++q)
        wt[part][s][q] = (p.normalize && n < p.N && q < p.P) ? p.w[part][n * p.P + q] : 1.f;
    }
  for (int64_t t = t0 + w; t < t1; t += kWaves) {
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      float acc[SL];
      bcnorm_token<SL>(p.x[part], t * p.xs[part], p.dt_x, lane, p.N, p.P, p.normalize, p.eps, invK,
                       wt[part], acc);
#pragma unroll
      for (int s = 0; s < SL; ++s) {
        const int n = lane + s * kWave;
        if (n < p.N) p.out[part][t * p.N + n] = acc[s];
      }
    }
  }
}

// Backward: g (T, N) fp32 per part -> dx (T, N*P) in x's dtype, dw partials.
template <int SL>
__global__ __launch_bounds__(kThreads) void bcnorm_bwd_kernel(BcNormParams p, BcNormGrad gr) {
  __shared__ double sW[2][kWaves][kBcMaxP * kWave * SL];
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int K = p.N * p.P;
  const float invK = 1.f / (float)K;
  int64_t t0, t1;
  token_range(p, t0, t1);
  float wt[2][SL][kBcMaxP];
  double dw[2][SL][kBcMaxP];
#pragma unroll
  for (int part = 0; part < 2; ++part)
#pragma unroll
    for (int s = 0; s < SL; ++s) {
      const int n = lane + s * kWave;
#pragma unroll
      for (int q = 0; q < kBcMaxP; ++q) {
        wt[part][s][q] = (p.normalize && n < p.N && q < p.P) ? p.w[part][n * p.P + q] : 1.f;
        dw[part][s][q] = 0.0;
      }
    }
  for (int64_t t = t0 + w; t < t1; t += kWaves) {
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const void* x = p.x[part];
      float v[SL][kBcMaxP], g[SL];
      float ss = 0.f, gr_r = 0.f;
#pragma unroll
      for (int s = 0; s < SL; ++s) {
        const int n = lane + s * kWave;
        g[s] = n < p.N ? gr.g[part][t * p.N + n] : 0.f;
#pragma unroll
        for (int q = 0; q < kBcMaxP; ++q) {
          v[s][q] = (n < p.N && q < p.P) ? load_in(x, t * p.xs[part] + n * p.P + q, p.dt_x) : 0.f;
          ss += v[s][q] * v[s][q];
          gr_r += (g[s] * wt[part][s][q]) * v[s][q];
        }
      }
      float r = 1.f, gx2 = 0.f;
      if (p.normalize) {
        r = rsqrtf(wave_sum(ss) * invK + p.eps);
        const float gm = (-0.5f * wave_sum(gr_r)) * ((r * r) * r);
        gx2 = gm * invK;  // torch divides by the element count as a product with 1/K
      }
#pragma unroll
      for (int s = 0; s < SL; ++s) {
        const int n = lane + s * kWave;
        if (n >= p.N) continue;
#pragma unroll
        for (int q = 0; q < kBcMaxP; ++q) {
          if (q >= p.P) break;
          float dx;
          if (p.normalize) {
            const float gxr = g[s] * wt[part][s][q];
            dx = round_dt(round_dt(gxr * r, p.dt_x) + round_dt(gx2 * (2.f * v[s][q]), p.dt_x),
                          p.dt_x);
            dw[part][s][q] += (double)(g[s] * (v[s][q] * r));
          } else {
            dx = g[s];
          }
          store_dt(gr.dx[part], t * K + n * p.P + q, dx, p.dt_x);
        }
      }
    }
  }
  if (!p.normalize) return;
  // dw: waves' partials combined in a fixed order, one row per workgroup
#pragma unroll
  for (int part = 0; part < 2; ++part)
#pragma unroll
    for (int s = 0; s < SL; ++s)
#pragma unroll
      for (int q = 0; q < kBcMaxP; ++q) sW[part][w][(s * kWave + lane) * kBcMaxP + q] = dw[part][s][q];
  __syncthreads();
  for (int i = threadIdx.x; i < 2 * K; i += kThreads) {
    const int part = i / K, j = i % K;
    const int n = j / p.P, q = j % p.P;
    const int slot = n * kBcMaxP + q;  // lane n % 64 of slot n / 64 stored it
    const double a = ((sW[part][0][slot] + sW[part][1][slot]) + sW[part][2][slot]) + sW[part][3][slot];
    gr.part[((int64_t)blockIdx.x * 2 + part) * K + j] = a;
  }
}

// dw[part][j] = sum over workgroups of the partials: one wave per weight,
// lane l summing rows l, l + 64, ... (4 running sums so the loads overlap),
// then a butterfly across lanes; a fixed order for a given shape.
__global__ __launch_bounds__(kThreads) void bcnorm_reduce_kernel(const double* part, float* dwB,
                                                                 float* dwC, int K, int groups) {
  const int lane = threadIdx.x % kWave;
  const int i = blockIdx.x * kWaves + threadIdx.x / kWave;
  if (i >= 2 * K) return;
  const int pt = i / K, j = i % K;
  double a[4] = {0.0, 0.0, 0.0, 0.0};
  int g = lane;
  for (; g + 3 * kWave < groups; g += 4 * kWave) {
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] += part[((int64_t)(g + q * kWave) * 2 + pt) * K + j];
  }
  for (; g < groups; g += kWave) a[0] += part[((int64_t)g * 2 + pt) * K + j];
  double v = (a[0] + a[1]) + (a[2] + a[3]);
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) v += __shfl_xor(v, m);
  if (lane == 0) (pt == 0 ? dwB : dwC)[j] = (float)v;
}

hipError_t launch_bcnorm_fwd(const BcNormParams& p, hipStream_t st) {
  if (p.groups == 0) return hipSuccess;
  if (p.N > kWave) {
    hipLaunchKernelGGL(bcnorm_fwd_kernel<2>, dim3(p.groups), dim3(kThreads), 0, st, p);
  } else {
    hipLaunchKernelGGL(bcnorm_fwd_kernel<1>, dim3(p.groups), dim3(kThreads), 0, st, p);
  }
  return hipGetLastError();
}

hipError_t launch_bcnorm_bwd(const BcNormParams& p, const BcNormGrad& g, hipStream_t st) {
  if (p.groups > 0) {
    if (p.N > kWave) {
      hipLaunchKernelGGL(bcnorm_bwd_kernel<2>, dim3(p.groups), dim3(kThreads), 0, st, p, g);
    } else {
      hipLaunchKernelGGL(bcnorm_bwd_kernel<1>, dim3(p.groups), dim3(kThreads), 0, st, p, g);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (!p.normalize) return hipSuccess;
  const int K = p.N * p.P;
  hipLaunchKernelGGL(bcnorm_reduce_kernel, dim3((unsigned)((2 * K + kWaves - 1) / kWaves)),
                     dim3(kThreads), 0, st, (const double*)g.part, g.dw[0], g.dw[1], K, p.groups);
  return hipGetLastError();
}

}  // namespace rp
