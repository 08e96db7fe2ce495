// Fused O(1) recurrent step of the SSM core for a batch of rollouts, gfx950.
//
// Replaces the ~20 small torch ops of Mamba3Block.step between the input
// projections and out_proj (engine/mamba.py:466-494): gates, the trapezoid
// blend, the state update and the y = h.C + u*D readout, in one pass that
// reads (h, beta) once and writes (h', beta') once.  This is the HBM-bound
// half of the hot path (16 bytes of state traffic per state element).
//
// Two kernels, bitwise the same as each other and as the scan:
//   * step_tile_kernel (step_tile.h; the rollout path: d_state a multiple of
//     4 up to 128, with pad states only in the last slot; step_pad.hip
//     instantiates it for d_state below the lane shape's S*NPL, e.g. 28,
//     36, 44-60, 68-76, 84-92, 116-124): a workgroup owns 256 / SPL channels
//     and walks a few rollouts.  Per rollout, the (channels x d_state) blocks of
//     h and beta move with coalesced streaming 16-byte loads and stores
//     through LDS, where SPL threads per channel (1 up to d_state 20, then
//     one per 4 slices) update its states; the gate parameters stay in
//     registers and the B / C rows in LDS for all the workgroup's rollouts.
//     (Moving each channel's 80 contiguous bytes per thread instead costs
//     ~15% of the bandwidth.)
//   * step_kernel: the scan's lane layout (S lanes per channel), for any
//     other shape.
// Both run the scan's per-state arithmetic (gate_of / fwd_update in
// rp_device.h); the tile kernel sums y over a channel's states in the same
// order as the scan's lanes + DPP butterfly (per-slice FMA chains, then a
// balanced pairwise tree), so a cached state advanced by either kernel
// matches the scan bit for bit.  beta' is stored as 2 * ((dt*u)/2 * B) =
// (dt*u) * B exactly, the association of the reference's dBu_t
// (engine/mamba.py:481).

#include "rp_device.h"
#include "rp_launch.h"
#include "step_tile.h"

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

  __shared__ float2 sCos[kTab];  // (m, b (-sin a)) records of the gate table
  fill_cos_lin(sCos, tid);
  GateRegs<NPL> gp;
  float h[NPL], hbp[NPL], Bs[NPL], Cs[NPL];
  float dt = 0.f, uu = 0.f;
  if (cvalid) {
    dt = p.delta[(int64_t)r * p.dsr + c];
    if (p.dsp) dt = softplus_of(dt);
    uu = p.u[(int64_t)r * p.usr + c];
  }
  const int64_t sbase = ((int64_t)r * p.D + c) * p.N;  // output state
  const int64_t ibase = (int64_t)r * p.ssr + (int64_t)c * p.N;  // input state
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
      h[j] = p.h_in[ibase + n];
      // beta_prev / 2: full form, or rank-1 (dt*u)_prev / 2 * B_prev
      hbp[j] = p.rank1 ? fmul(0.5f * p.beta_in[(int64_t)r * p.bssr + c],
                              p.beta_in[(int64_t)r * p.bssr + p.D + n])
                       : 0.5f * p.beta_in[ibase + n];
    }
  }
  load_gate_regs<S, NPL>(gp, p.Ar, p.Ai, p.Tk, c, s, p.N, p.NR, p.NT, cvalid);
  __syncthreads();  // the gate table
  const float hd = 0.5f * fmul(dt, uu);
  float y = fwd_update<S, NPL, GK>(h, hbp, gp, sCos, dt, hd, Bs, Cs, s, p.NR, has_imag);
  y = reduce_states<S>(y);
  if (cvalid) {
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int n = j * S + s;
      if (n < p.N) {
        p.h_out[sbase + n] = h[j];
        if (!p.rank1) p.beta_out[sbase + n] = 2.f * hbp[j];
      }
    }
    if (s == 0) {
      float yv = y + fmul(uu, p.Dskip[c]);
      if (p.z != nullptr) yv = silu_gate(yv, load_in(p.z, (int64_t)r * p.zsr + c, p.dt_z), p.dt_z);
      p.y[(int64_t)r * p.D + c] = yv;
      if (p.rank1) p.beta_out[(int64_t)r * (p.D + p.N) + c] = fmul(dt, uu);
    }
  }
  // rank-1: the rollout's B row, written once (by its first channel tile)
  if (p.rank1 && tile == 0 && tid < p.N)
    p.beta_out[(int64_t)r * (p.D + p.N) + p.D + tid] = p.Bc[(int64_t)r * p.bsr + tid];
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

hipError_t launch_step(int S, int NPL, int gk, bool tile, const StepParams& p, hipStream_t st) {
  if (tile && p.N != S * NPL) return launch_step_tile_pad(S, NPL, gk, p, st);
  if (tile) {
#define RP_CASE(SS, NN) \
    if (S == SS && NN == NPL) return launch_step_tile<SS, NN, false>(gk, p, st);
    RP_FOR_EACH_SHAPE(RP_CASE)
#undef RP_CASE
    return hipErrorInvalidValue;
  }
#define RP_CASE(SS, NN)                                                    \
  if (S == SS && NN == NPL)                                                \
    return with_gate_kind<NN>(gk, [&](auto g) {                            \
      return launch_step_t<SS, NN, decltype(g)>(p, st);                    \
    });
  RP_FOR_EACH_SHAPE(RP_CASE)
#undef RP_CASE
  return hipErrorInvalidValue;
}

}  // namespace rp
