// Fused O(1) recurrent step of the SSM core for a batch of rollouts, gfx950.
//
// Replaces the ~20 small torch ops of Mamba3Block.step between the input
// projections and out_proj (engine/mamba.py:466-494): gates, the trapezoid
// blend, the state update and the y = h.C + u*D readout, in one pass that
// reads (h, beta) once and writes (h', beta') once.  This is the HBM-bound
// half of the hot path (16 bytes of state traffic per state element).
//
// The lane layout and the per-state arithmetic are the scan kernel's own
// (fwd_update / reduce_states in rp_device.h), so a cached state advanced by
// this kernel matches the scan bit for bit.  beta' is stored as
// 2 * ((dt*u)/2 * B) = (dt*u) * B exactly, the association of the
// reference's dBu_t (engine/mamba.py:481).

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

template <int S, int NPL, class GK>
__global__ __launch_bounds__(kThreads) void step_kernel(StepParams p) {
  using Sh = Shape<S, NPL>;
  constexpr int DT = Sh::kDT, CB = Sh::kCB;
  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int dl = lane / S, s = lane % S;
  const int tile = blockIdx.x % p.ntiles, r = blockIdx.x / p.ntiles;
  const int c = tile * CB + wave * DT + dl;
  const bool cvalid = c < p.D;
  const bool has_imag = p.Ai != nullptr;

  __shared__ float2 sTab[16];  // cos, sin of 2 pi k / 16
  fill_sincos_table(sTab, tid);
  GateRegs<NPL> gp;
  float h[NPL], hbp[NPL], Bs[NPL], Cs[NPL];
  float dt = 0.f, uu = 0.f;
  if (cvalid) {
    dt = p.delta[(int64_t)r * p.dsr + c];
    uu = p.u[(int64_t)r * p.usr + c];
  }
  const int64_t sbase = ((int64_t)r * p.D + c) * p.N;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int n = j * S + s;
    h[j] = 0.f;
    hbp[j] = 0.f;
    Bs[j] = 0.f;
    Cs[j] = 0.f;
    if (n < p.N) {
      Bs[j] = p.Bc[(int64_t)r * p.bsr + n];
      Cs[j] = p.Cc[(int64_t)r * p.csr + n];
    }
    if (cvalid && n < p.N && p.h_in != nullptr) {
      h[j] = p.h_in[sbase + n];
      hbp[j] = 0.5f * p.beta_in[sbase + n];
    }
  }
  load_gate_regs<S, NPL>(gp, p.Ar, p.Ai, p.Tk, c, s, p.N, p.NR, p.NT, cvalid);
  __syncthreads();  // the sin/cos table
  const float hd = 0.5f * fmul(dt, uu);
  float y = fwd_update<S, NPL, GK>(h, hbp, gp, sTab, dt, hd, Bs, Cs, s, p.NR, has_imag);
  y = reduce_states<S>(y);
  if (cvalid) {
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int n = j * S + s;
      if (n < p.N) {
        p.h_out[sbase + n] = h[j];
        p.beta_out[sbase + n] = 2.f * hbp[j];
      }
    }
    if (s == 0) p.y[(int64_t)r * p.D + c] = y + fmul(uu, p.Dskip[c]);
  }
}

template <int S, int NPL, class GK>
static hipError_t launch_step_t(const StepParams& p, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)p.ntiles * p.R));
  hipLaunchKernelGGL((step_kernel<S, NPL, GK>), grid, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

__global__ void fill_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// Zero fill as a kernel (not a memset node), so it is safe under graph capture.
hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

hipError_t launch_step(int S, int NPL, bool spec, const StepParams& p, hipStream_t st) {
#define RP_CASE(SS, NN)                                                    \
  if (S == SS && NN == NPL)                                                \
    return spec ? launch_step_t<SS, NN, GateKind<NN - 1, 1>>(p, st)        \
                : launch_step_t<SS, NN, GateKind<0, 2>>(p, st);
  RP_FOR_EACH_SHAPE(RP_CASE)
#undef RP_CASE
  return hipErrorInvalidValue;
}

}  // namespace rp
