// Forward trapezoidal selective scan (causal or bidirectional) for gfx950.
//
// Replaces the reference's _fwd_kernel (engine/triton_scan.py:44-98) and its
// two-launch bidirectional wrapper (engine/mamba.py:254-260).  One workgroup
// = 4 waves = CB channels of one batch row; each lane carries NPL states of
// one channel in VGPRs and walks the sequence serially.  Per block of 32
// steps (16 above 40 states) the workgroup stages dt, (dt*u)/2, B and C into
// LDS (converted to fp32 once), then every wave runs the recurrence out of
// LDS and leaves the block's y in LDS, written out coalesced once per block.
// In bidirectional mode the same workgroup runs the reversed direction next
// and accumulates into y, so inputs are read from HBM once per direction and
// there are no flip copies.
//
// Optional outputs: per-chunk state checkpoints for the backward, and the
// final state (h, beta) that step() continues from.

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

template <int S, int NPL, class GK>
__global__ __launch_bounds__(kThreads) void scan_fwd_kernel(ScanParams p, FwdOut o) {
  using Sh = Shape<S, NPL>;
  // steps staged per block: fewer for large states, whose B / C rows
  // dominate the LDS (occupancy)
  constexpr int DT = Sh::kDT, CB = Sh::kCB, NP = Sh::kNP, TB = NP > 40 ? kFwdTB / 2 : kFwdTB;
  __shared__ float2 sDH[TB][CB];   // (dt, (dt*u)/2) per step and channel
  __shared__ float sB[TB][NP];     // per step, layout [s*NPL + j] -> state j*S + s
  __shared__ float sC[TB][NP];
  __shared__ float sY[TB][CB];     // the block's y, written out channel-contiguous
  __shared__ float2 sCos[kTab];      // (m, b (-sin a)) records of the gate table

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int dl = lane / S, s = lane % S;
  const int cl = wave * DT + dl;
  const int tile = blockIdx.x % p.ntiles, b = blockIdx.x / p.ntiles;
  const int c = tile * CB + cl;
  const bool cvalid = c < p.D;
  const bool has_imag = p.Ai != nullptr;
  const int L = p.L;

  GateRegs<NPL> gp;  // loads issued first, so the table copy overlaps them
  load_gate_regs<S, NPL>(gp, p.Ar, p.Ai, p.Tk, c, s, p.N, p.NR, p.NT, cvalid);
  fill_cos_lin(sCos, tid);  // first read after the staging barrier below

  const int nblk = (L + TB - 1) / TB;
  for (int dir = 0; dir < p.ndir; ++dir) {
    // sm = h + hb of the previous step (of the initial state h0, beta0 / 2)
    float sm[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int n = j * S + s;
      sm[j] = 0.f;
      if (dir == 0 && p.h0 != nullptr && cvalid && n < p.N) {
        const int64_t idx = ((int64_t)b * p.D + c) * p.N + n;
        sm[j] = p.h0[idx] + 0.5f * p.beta0[idx];
      }
    }
    // y of the block starting at step i0 (cnt steps) from sY: coalesced, and
    // the reverse direction adds to what the forward direction stored
    auto write_y = [&](int i0, int cnt) {
      for (int e = tid; e < cnt * CB; e += kThreads) {
        const int r = e / CB, ci = e % CB;
        const int c2 = tile * CB + ci;
        if (c2 < p.D) {
          const int i = i0 + r;
          const int t = dir ? (L - 1 - i) : i;
          float* yp = o.y + ((int64_t)b * L + t) * p.D + c2;
          *yp = dir == 0 ? sY[r][ci] : *yp + sY[r][ci];
        }
      }
    };
    for (int bi = 0; bi < nblk; ++bi) {
      const int i0 = bi * TB;
      const int cnt = min(TB, L - i0);
      __syncthreads();
      if (bi > 0) write_y(i0 - TB, TB);
      for (int e = tid; e < TB * CB; e += kThreads) {
        const int r = e / CB, ci = e % CB;
        const int c2 = tile * CB + ci;
        float dt = 0.f, hd = 0.f;
        if (r < cnt && c2 < p.D) {
          const int i = i0 + r;
          const int t = dir ? (L - 1 - i) : i;
          const int64_t di = ((int64_t)b * L + t) * p.D + c2;
          if (dir == 1 && o.dcache != nullptr) {
            dt = o.dcache[di];  // cached by this workgroup's forward direction
          } else {
            dt = load_in(p.delta, (int64_t)b * p.dsb + (int64_t)t * p.dsl + c2, p.dt_delta);
            if (p.dsp) dt = softplus_of(dt);
            if (o.dcache != nullptr) o.dcache[di] = dt;
          }
          const float uu = load_in(p.u, (int64_t)b * p.usb + (int64_t)t * p.usl + c2, p.dt_u);
          hd = 0.5f * fmul(dt, uu);
        }
        sDH[r][ci] = make_float2(dt, hd);
      }
      for (int e = tid; e < TB * NP; e += kThreads) {
        const int r = e / NP, k = e % NP;
        const int n = (k % NPL) * S + (k / NPL);
        float bv = 0.f, cv = 0.f;
        if (r < cnt && n < p.N) {
          const int i = i0 + r;
          const int t = dir ? (L - 1 - i) : i;
          bv = load_in(p.Bc, (int64_t)b * p.bsb + (int64_t)t * p.bsl + n, p.dt_B);
          cv = load_in(p.Cc, (int64_t)b * p.csb + (int64_t)t * p.csl + n, p.dt_C);
        }
        sB[r][k] = bv;
        sC[r][k] = cv;
      }
      __syncthreads();
      for (int r = 0; r < cnt; ++r) {
        const int i = i0 + r;
        const float2 dh = sDH[r][cl];
        float h[NPL], hb[NPL];
        float y = fwd_update_carried<S, NPL, GK>(sm, h, hb, gp, sCos, dh.x, dh.y, &sB[r][s * NPL],
                                                 &sC[r][s * NPL], s, p.NR, has_imag);
        // the channel's S lanes hold the same total and store the same value
        sY[r][cl] = reduce_states<S>(y);
        if (o.ckpt != nullptr && ((i + 1) % kCkptK) == 0 && i + 1 < L) {
          // state entering chunk (i+1)/K, in a coalesced [tile][wave][j][lane] record
          const int64_t rec =
              ((int64_t)(dir * p.B + b) * p.nck + ((i + 1) / kCkptK - 1)) * p.ntiles + tile;
          float* dst = o.ckpt + (rec * kWaves + wave) * (NPL * kWave) + lane;
#pragma unroll
          for (int j = 0; j < NPL; ++j) dst[j * kWave] = h[j];
        }
        if (dir == 0 && i == L - 1 && o.h_last != nullptr && cvalid) {
          // the final state (h, beta) that step() continues from
#pragma unroll
          for (int j = 0; j < NPL; ++j) {
            const int n = j * S + s;
            if (n < p.N) {
              const int64_t idx = ((int64_t)b * p.D + c) * p.N + n;
              o.h_last[idx] = h[j];
              o.beta_last[idx] = 2.f * hb[j];
            }
          }
        }
      }
    }
    if (nblk > 0) {
      __syncthreads();
      write_y((nblk - 1) * TB, L - (nblk - 1) * TB);
    }
  }
}

template <int S, int NPL, class GK>
static hipError_t launch_fwd_t(const ScanParams& p, const FwdOut& o, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)p.ntiles * p.B));
  hipLaunchKernelGGL((scan_fwd_kernel<S, NPL, GK>), grid, dim3(kThreads), 0, st, p, o);
  return hipGetLastError();
}

hipError_t launch_scan_fwd(int S, int NPL, int gk, const ScanParams& p, const FwdOut& o,
                           hipStream_t st) {
#define RP_CASE(SS, NN)                                                              \
  if (S == SS && NN == NPL)                                                          \
    return with_gate_kind<NN>(gk, [&](auto g) {                                      \
      return launch_fwd_t<SS, NN, decltype(g)>(p, o, st);                            \
    });
  RP_FOR_EACH_SHAPE(RP_CASE)
#undef RP_CASE
  return hipErrorInvalidValue;
}

}  // namespace rp
