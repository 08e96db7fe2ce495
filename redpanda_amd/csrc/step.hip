// Fused O(1) recurrent step of the SSM core for a batch of rollouts, gfx950.
//
// Replaces the ~20 small torch ops of Mamba3Block.step between the input
// projections and out_proj (engine/mamba.py:466-494): gates, the trapezoid
// blend, the state update and the y = h.C + u*D readout, in one pass that
// reads (h, beta) once and writes (h', beta') once.  This is the HBM-bound
// half of the hot path (16 bytes of state traffic per state element).
//
// Two kernels, bitwise the same as each other and as the scan:
//   * step_tile_kernel (the rollout path: d_state == S*NPL, a multiple of 4,
//     <= 40): one thread per channel holding all of the channel's states,
//     read and written as aligned 16-byte vectors; a workgroup owns 256
//     channels and walks a group of rollouts, keeping the gate parameters in
//     registers.  B and C are wave-uniform.
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

  __shared__ float2 sTab[kTab];  // cos, sin of 2 pi k / kTab
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

// Balanced pairwise sum of the S per-slice partials: the association of
// reduce_states<S> (every DPP stage adds two subtrees; fp addition is
// commutative, so operand order within a stage does not change the bits).
template <int S>
__device__ __forceinline__ float tree_sum(const float (&v)[S]) {
  if constexpr (S == 1) {
    return v[0];
  } else {
    float lo[S / 2], hi[S / 2];
#pragma unroll
    for (int i = 0; i < S / 2; ++i) {
      lo[i] = v[i];
      hi[i] = v[S / 2 + i];
    }
    return tree_sum<S / 2>(lo) + tree_sum<S / 2>(hi);
  }
}

template <int S, int NPL, class GK>
__global__ __launch_bounds__(kThreads) void step_tile_kernel(StepParams p) {
  constexpr int NP = S * NPL;
  constexpr int NV = NP / 4;            // float4s per channel at N == NP
  constexpr int TCH = kStepTile;
  __shared__ float2 sTab[kTab];           // cos, sin of 2 pi k / kTab
  __shared__ float2 sGate[NP][TCH];     // (pah, wh) of every channel's states
  __shared__ float sBC[2][2 * NP];       // B, C rows of the current / next rollout
  const int tid = threadIdx.x;
  const int tile = blockIdx.x % p.ctiles, rg = blockIdx.x / p.ctiles;
  const int c = tile * TCH + tid;
  const bool cvalid = c < p.D;
  const bool has_imag = p.Ai != nullptr;
  const int N = p.N;                    // N == NP (checked by the host)
  fill_sincos_table(sTab, tid);
  // gate parameters live in LDS (conflict-free [state][thread] layout), so
  // the registers hold the rollout's states only
#pragma unroll
  for (int n = 0; n < NP; ++n) {
    float a, w;
    load_gate_params(p.Ar, p.Ai, p.Tk, c, n, N, p.NR, p.NT, cvalid, a, w);
    sGate[n][tid] = make_float2(a, w);
  }
  const float dsk = cvalid ? p.Dskip[c] : 0.f;

  const int r_lo = rg * p.ri;
  const int r_hi = min(p.R, r_lo + p.ri);
  // Software pipeline over the workgroup's rollouts: everything rollout r+1
  // needs (its state vectors, dt and u, and its B / C rows, staged through a
  // double-buffered LDS row) is requested before rollout r is computed, so
  // every wave keeps a rollout of loads in flight.  The channel's states are
  // NP contiguous floats: NV aligned 16-byte vectors.
  float4 hv[NV], bv[NV], hn[NV], bn[NV];
  auto load_state = [&](int r, float4 (&h4)[NV], float4 (&b4)[NV]) {
    const int64_t base = ((int64_t)r * p.D + c) * NP;
    if (p.h_in != nullptr && cvalid) {
      const float4* hi4 = reinterpret_cast<const float4*>(p.h_in + base);
      const float4* bi4 = reinterpret_cast<const float4*>(p.beta_in + base);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        h4[v] = hi4[v];
        b4[v] = bi4[v];
      }
    } else {
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        h4[v] = make_float4(0.f, 0.f, 0.f, 0.f);
        b4[v] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  // B / C of a rollout: thread t < 2*NP loads element t (B then C)
  auto load_bc = [&](int r) -> float {
    if (tid < 2 * NP) {
      const int n = tid % NP;
      return tid < NP ? p.Bc[(int64_t)r * p.bsr + n] : p.Cc[(int64_t)r * p.csr + n];
    }
    return 0.f;
  };
  auto load_du = [&](int r, float& d, float& u) {
    d = cvalid ? p.delta[(int64_t)r * p.dsr + c] : 0.f;
    u = cvalid ? p.u[(int64_t)r * p.usr + c] : 0.f;
  };
  float dtc = 0.f, uc = 0.f, dtn = 0.f, un = 0.f;
  if (r_lo < r_hi) {
    load_state(r_lo, hv, bv);
    load_du(r_lo, dtc, uc);
    const float bc0 = load_bc(r_lo);
    if (tid < 2 * NP) sBC[0][tid] = bc0;
  }
  __syncthreads();  // the sin/cos table and the first B / C row
  for (int r = r_lo; r < r_hi; ++r) {
    const int buf = (r - r_lo) & 1;
    float bcn = 0.f;
    if (r + 1 < r_hi) {
      load_state(r + 1, hn, bn);
      load_du(r + 1, dtn, un);
      bcn = load_bc(r + 1);
    }
    const float hd = 0.5f * fmul(dtc, uc);
    float ys[S];
#pragma unroll
    for (int q = 0; q < S; ++q) ys[q] = 0.f;
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      const int j = n / S, q = n % S;
      float& hs = (&hv[n / 4].x)[n % 4];
      float& bs = (&bv[n / 4].x)[n % 4];
      const float Bn = sBC[buf][n];
      const float Cn = sBC[buf][NP + n];
      const float hbp = 0.5f * bs;
      float unused;
      const float2 gw = sGate[n][tid];
      const float g = gate_of<S, GK, false>(j, q, p.NR, has_imag, dtc, gw.x, gw.y, sTab, unused);
      const float hb = fmul(hd, Bn);
      const float sm = hs + hbp;
      hs = ffma(g, sm, hb);
      bs = 2.f * hb;
      ys[q] = ffma(hs, Cn, ys[q]);
    }
    if (cvalid) {
      p.y[(int64_t)r * p.D + c] = tree_sum<S>(ys) + fmul(uc, dsk);
      const int64_t base = ((int64_t)r * p.D + c) * NP;
      float4* ho4 = reinterpret_cast<float4*>(p.h_out + base);
      float4* bo4 = reinterpret_cast<float4*>(p.beta_out + base);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        ho4[v] = hv[v];
        bo4[v] = bv[v];
      }
    }
    if (tid < 2 * NP) sBC[buf ^ 1][tid] = bcn;
    __syncthreads();  // next B / C row visible; this row no longer read
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      hv[v] = hn[v];
      bv[v] = bn[v];
    }
    dtc = dtn;
    uc = un;
  }
}

template <int S, int NPL, class GK>
static hipError_t launch_step_tile_t(const StepParams& p, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)p.ctiles * p.rgroups));
  hipLaunchKernelGGL((step_tile_kernel<S, NPL, GK>), grid, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <int S, int NPL>
static hipError_t launch_step_tile(int gk, const StepParams& p, hipStream_t st) {
  if constexpr (S * NPL <= 40) {
    return with_gate_kind<NPL>(gk, [&](auto g) {
      return launch_step_tile_t<S, NPL, decltype(g)>(p, st);
    });
  } else {
    return hipErrorInvalidValue;
  }
}

hipError_t launch_step(int S, int NPL, int gk, bool tile, const StepParams& p, hipStream_t st) {
  if (tile) {
#define RP_CASE(SS, NN) \
    if (S == SS && NN == NPL) return launch_step_tile<SS, NN>(gk, p, st);
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
