// Analytic reverse-scan backward of the trapezoidal selective scan, gfx950.
//
// Replaces the reference's _bwd_kernel (engine/triton_scan.py:100-241) and
// the Python-side partial sums / float atomics around it (:239-241, :313-315).
//
// Recurrence (per channel, per state; hb_t = beta_t / 2, s_{t-1} = h_{t-1}
// + hb_{t-1}, forward h_t = g_t s_{t-1} + hb_t):
//     q_t    = dy_t C_t + g_{t+1} q_{t+1}
//     dg_t   = q_t s_{t-1}
//     dhb_t  = q_t + g_{t+1} q_{t+1}               (= 2 dbeta_t)
//     dB_t  += dhb_t hdu_t          dC_t += dy_t h_t        (sums over channels)
//     dhdu_t = sum_n dhb_t B_t      -> ddt += u/2 dhdu, du = dt/2 dhdu
//     rot:   dAr += dg dt g,   dAi -= dg dt e sin,   ddt += dg (Ar g - Ai e sin)
//     track: dTk += dg
//
// Work split: one workgroup = CB channels x a group of `bg` batch rows, both
// directions.  The forward stored the state entering every kCkptK-step chunk;
// the backward walks chunks in reverse, recomputes the chunk's K steps into
// registers (keeping s_{t-1}, the gate and e*sin, so the adjoint evaluates
// no transcendental), then runs the adjoint over them.  The recompute calls
// the forward's gate code (with the sine added), so it rebuilds the forward's
// states exactly.
//
// Reductions, all in a fixed order (run-to-run deterministic, no atomics):
//   * over a channel's states (ddt, du): in-lane FMA chain + DPP butterfly;
//   * over channels (dB, dC): DPP row rotations inside each 16-lane row, the
//     row partials staged in LDS, then a 16-way sum per output, per tile;
//     the per-tile partials are summed in float64 by a second kernel;
//   * parameter gradients (dA, dTk): 8-step fp32 chunk sums accumulated in
//     float64 per lane over the batch group, then float64 across groups.

#include <type_traits>

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

template <int S, int NPL, class GK>
__global__ __launch_bounds__(kThreads, NPL <= 5 ? 2 : 1) void scan_bwd_kernel(ScanParams p, BwdIO io) {
  using Sh = Shape<S, NPL>;
  constexpr int DT = Sh::kDT, CB = Sh::kCB, NP = Sh::kNP, TB = kBwdTB, K = kCkptK;
  constexpr int KR = NP <= 40 ? K : K / 2;  // steps per channel-sum fold
  constexpr int NRW = kWaves * 4;           // 16-lane rows per workgroup
  static_assert(TB % K == 0 && K % KR == 0, "time block must hold whole chunks");
  // row 0 = the step just before the block (its (dt*u)/2 and B seed the
  // trapezoid carry at the first chunk's entry); rows 1..TB = the block
  __shared__ float4 sCh[TB + 1][CB];        // (dt, (dt*u)/2, u, dy)
  __shared__ float sB[TB + 1][NP];
  __shared__ float sC[TB + 1][NP];
  __shared__ float sRed[KR][2][NRW][NP];    // per-row channel sums of dB, dC
  __shared__ float2 sDD[TB][CB];            // (d_delta, d_u) of the block
  __shared__ float2 sTab[16];               // cos, sin of 2 pi k / 16

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int dl = lane / S, s = lane % S;
  const int cl = wave * DT + dl;
  const int wrow = wave * 4 + lane / 16;    // row index within the workgroup
  const bool row_leader = (lane % 16) < S;  // first channel of its row
  const int tile = blockIdx.x % p.ntiles, bgi = blockIdx.x / p.ntiles;
  const int c = tile * CB + cl;
  const bool cvalid = c < p.D;
  const bool has_imag = p.Ai != nullptr;
  const int L = p.L;

  fill_sincos_table(sTab, tid);  // first read after the staging barrier below
  GateRegs<NPL> gp;
  load_gate_regs<S, NPL>(gp, p.Ar, p.Ai, p.Tk, c, s, p.N, p.NR, p.NT, cvalid);
  double dpa[NPL], dpb[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    dpa[j] = 0.0;
    dpb[j] = 0.0;
  }

  const int b_lo = bgi * io.bg;
  const int b_hi = min(p.B, b_lo + io.bg);
  const int nblk = (L + TB - 1) / TB;

  for (int b = b_lo; b < b_hi; ++b) {
    for (int dir = 0; dir < p.ndir; ++dir) {
      // gq: the g_{t+1} q_{t+1} term of q_t;  gr: the term of dhb_t.  They are
      // equal except at the last step, where an outside consumer of the final
      // state contributes dh_last to q and 2*dbeta_last to dhb.
      float gq[NPL], gr[NPL];
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const int n = j * S + s;
        gq[j] = 0.f;
        gr[j] = 0.f;
        if (dir == 0 && cvalid && n < p.N) {
          const int64_t idx = ((int64_t)b * p.D + c) * p.N + n;
          if (io.dh_last != nullptr) gq[j] = io.dh_last[idx];
          if (io.dbeta_last != nullptr) gr[j] = 2.f * io.dbeta_last[idx];
        }
      }

      for (int bi = nblk - 1; bi >= 0; --bi) {
        const int i0 = bi * TB;
        const int cnt = min(TB, L - i0);
        __syncthreads();
        for (int e = tid; e < (TB + 1) * CB; e += kThreads) {
          const int r = e / CB, ci = e % CB;
          const int c2 = tile * CB + ci;
          const int i = i0 + r - 1;
          float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
          if (r <= cnt && i >= 0 && c2 < p.D) {
            const int t = dir ? (L - 1 - i) : i;
            const float dt = load_in(p.delta, (int64_t)b * p.dsb + (int64_t)t * p.dsl + c2, p.dt_delta);
            const float uu = load_in(p.u, (int64_t)b * p.usb + (int64_t)t * p.usl + c2, p.dt_u);
            v.x = dt;
            v.y = 0.5f * fmul(dt, uu);
            v.z = uu;
            v.w = io.dy[((int64_t)b * L + t) * p.D + c2];
          }
          sCh[r][ci] = v;
        }
        for (int e = tid; e < (TB + 1) * NP; e += kThreads) {
          const int r = e / NP, k = e % NP;
          const int n = (k % NPL) * S + (k / NPL);
          const int i = i0 + r - 1;
          float bv = 0.f, cv = 0.f;
          if (r <= cnt && i >= 0 && n < p.N) {
            const int t = dir ? (L - 1 - i) : i;
            bv = load_in(p.Bc, (int64_t)b * p.bsb + (int64_t)t * p.bsl + n, p.dt_B);
            cv = load_in(p.Cc, (int64_t)b * p.csb + (int64_t)t * p.csl + n, p.dt_C);
          }
          sB[r][k] = bv;
          sC[r][k] = cv;
        }
        __syncthreads();

        const int nchunk = (cnt + K - 1) / K;
        for (int kc = nchunk - 1; kc >= 0; --kc) {
          const int m0 = kc * K;
          const int kcnt = min(K, cnt - m0);
          const int chunk = (i0 + m0) / K;
          // state entering the chunk: h from the forward's checkpoint, hb
          // recomputed from the step before (row m0 of the stage)
          float hc[NPL], hbp[NPL];
          if (chunk == 0) {
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
              const int n = j * S + s;
              hc[j] = 0.f;
              hbp[j] = 0.f;
              if (dir == 0 && p.h0 != nullptr && cvalid && n < p.N) {
                const int64_t idx = ((int64_t)b * p.D + c) * p.N + n;
                hc[j] = p.h0[idx];
                hbp[j] = 0.5f * p.beta0[idx];
              }
            }
          } else {
            const int64_t rec = ((int64_t)(dir * p.B + b) * p.nck + (chunk - 1)) * p.ntiles + tile;
            const float* src = io.ckpt + (rec * kWaves + wave) * (NPL * kWave) + lane;
            const float hdp = sCh[m0][cl].y;
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
              hc[j] = src[j * kWave];
              hbp[j] = fmul(hdp, sB[m0][s * NPL + j]);
            }
          }
          // The chunk body, instantiated twice: FULL (all K steps present, the
          // common case; straight-line code) and a guarded tail for a last
          // chunk shorter than K.
          auto chunk_body = [&](auto full_tag) {
            constexpr bool FULL = decltype(full_tag)::value;
            // recompute the chunk: s_{t-1}, g_t and e*sin for every step
            float SP[K][NPL], G[K][NPL], ES[K][NPL];
#pragma unroll
            for (int m = 0; m < K; ++m) {
              if (FULL || m < kcnt) {
                const int row = m0 + m + 1;
                const float dt = sCh[row][cl].x;
                const float hd = sCh[row][cl].y;
#pragma unroll
                for (int j = 0; j < NPL; ++j) {
                  float es;
                  const float g = gate_of<S, GK, true>(j, s, p.NR, has_imag, dt, gp.pah[j],
                                                       gp.wh[j], sTab, es);
                  const float hb = fmul(hd, sB[row][s * NPL + j]);
                  const float sm = hc[j] + hbp[j];
                  SP[m][j] = sm;
                  G[m][j] = g;
                  ES[m][j] = es;
                  hc[j] = ffma(g, sm, hb);
                  hbp[j] = hb;
                }
              }
            }
            // adjoint over the chunk, last step first.  Parameter gradients
            // sum into chunk-local fp32 accumulators, then into float64.
            float cpa[NPL], cpb[NPL];
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
              cpa[j] = 0.f;
              cpb[j] = 0.f;
            }
#pragma unroll
            for (int m = K - 1; m >= 0; --m) {
              if (FULL || m < kcnt) {
                const int row = m0 + m + 1;
                const float4 ch = sCh[row][cl];
                const float dt = ch.x, hd = ch.y, uu = ch.z, dy = ch.w;
                float ddA = 0.f, ddB = 0.f, sBc = 0.f;
#pragma unroll
                for (int j = 0; j < NPL; ++j) {
                  const float Bv = sB[row][s * NPL + j];
                  const float Cv = sC[row][s * NPL + j];
                  const float g = G[m][j];
                  const float hb = fmul(hd, Bv);
                  const float ht = ffma(g, SP[m][j], hb);
                  const float q = ffma(dy, Cv, gq[j]);
                  const float dhb = q + gr[j];
                  sBc = ffma(dhb, Bv, sBc);
                  const float dg = fmul(q, SP[m][j]);
                  if (is_rot<S, GK>(j, s, p.NR)) {
                    const float t1 = fmul(dg, g);
                    const float t2 = fmul(dg, ES[m][j]);
                    cpa[j] = ffma(t1, dt, cpa[j]);
                    cpb[j] = ffma(t2, dt, cpb[j]);
                    ddA = ffma(gp.pah[j], t1, ddA);  // Ar log2(e) dg g
                    ddB = ffma(gp.wh[j], t2, ddB);   // Ai 16/(2 pi) dg e sin
                  } else {
                    cpa[j] = cpa[j] + dg;
                  }
                  gq[j] = fmul(g, q);
                  gr[j] = gq[j];
                  const float xB = reduce_row<S>(fmul(dhb, hd));
                  const float xC = reduce_row<S>(fmul(dy, ht));
                  if (row_leader) {
                    sRed[m % KR][0][wrow][s * NPL + j] = xB;
                    sRed[m % KR][1][wrow][s * NPL + j] = xC;
                  }
                }
                ddA = reduce_states<S>(ddA);
                ddB = reduce_states<S>(ddB);
                sBc = reduce_states<S>(sBc);
                if (s == 0) {
                  const float ddt = ffma(kLn2, ddA, -fmul(kPi8, ddB)) + fmul(0.5f * uu, sBc);
                  const float dut = fmul(0.5f * dt, sBc);
                  sDD[m0 + m][cl] = make_float2(ddt, dut);
                }
              }
              if (m % KR == 0) {
                // fold the 16 row partials of steps [m, m + KR) into this
                // tile's global dB / dC partials
                __syncthreads();
                for (int e = tid; e < KR * 2 * p.N; e += kThreads) {
                  const int rr = e / (2 * p.N);
                  const int rem = e % (2 * p.N);
                  const int which = rem / p.N, n = rem % p.N;
                  if (m + rr < kcnt) {
                    const int k = (n % S) * NPL + n / S;
                    float v = sRed[rr][which][0][k];
#pragma unroll
                    for (int w = 1; w < NRW; ++w) v = v + sRed[rr][which][w][k];
                    const int i = i0 + m0 + m + rr;
                    const int t = dir ? (L - 1 - i) : i;
                    float* dst = io.part_bc +
                                 (((int64_t)which * p.ntiles + tile) * p.B + b) * ((int64_t)L * p.N) +
                                 (int64_t)t * p.N + n;
                    if (dir == 0)
                      *dst = v;
                    else
                      *dst = *dst + v;
                  }
                }
                __syncthreads();
              }
            }
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
              dpa[j] += (double)cpa[j];
              dpb[j] += (double)cpb[j];
            }
          };
          if (kcnt == K)
            chunk_body(std::true_type{});
          else
            chunk_body(std::false_type{});
        }
        // the block's (d_delta, d_u) rows, written channel-contiguous
        for (int e = tid; e < cnt * CB; e += kThreads) {
          const int r = e / CB, ci = e % CB;
          const int c2 = tile * CB + ci;
          if (c2 < p.D) {
            const int i = i0 + r;
            const int t = dir ? (L - 1 - i) : i;
            const float2 v = sDD[r][ci];
            const int64_t idx = ((int64_t)b * L + t) * p.D + c2;
            if (dir == 0) {
              io.d_delta[idx] = v.x;
              io.d_u[idx] = v.y;
            } else {
              io.d_delta[idx] = io.d_delta[idx] + v.x;
              io.d_u[idx] = io.d_u[idx] + v.y;
            }
          }
        }
      }
      // after the sweep gq = g_0 q_0: the gradient of the initial state, since
      // h_0 = g_0 (h0 + beta0/2) + hb_0
      if (dir == 0 && io.d_h0 != nullptr && cvalid) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          const int n = j * S + s;
          if (n < p.N) {
            const int64_t idx = ((int64_t)b * p.D + c) * p.N + n;
            io.d_h0[idx] = gq[j];
            io.d_beta0[idx] = 0.5f * gq[j];
          }
        }
      }
    }
  }
  // per-batch-group parameter-gradient partials (float64)
  if (cvalid) {
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int n = j * S + s;
      if (n < p.N) {
        const int64_t base = ((int64_t)bgi * 2) * p.D * p.N;
        io.part_par[base + (int64_t)c * p.N + n] = dpa[j];
        io.part_par[base + (int64_t)p.D * p.N + (int64_t)c * p.N + n] = dpb[j];
      }
    }
  }
}

// dB / dC: sum the per-tile partials in a fixed order (fp64 accumulator).
__global__ void bwd_reduce_bc(const float* __restrict__ part, float* __restrict__ dB,
                              float* __restrict__ dC, int64_t per, int ntiles) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= 2 * per) return;
  const int which = e >= per;
  const int64_t k = which ? e - per : e;
  double acc = 0.0;
  for (int g = 0; g < ntiles; ++g) acc += part[((int64_t)which * ntiles + g) * per + k];
  (which ? dC : dB)[k] = (float)acc;
}

// dA_real / dA_imag / dtrack: sum the per-batch-group float64 partials.
__global__ void bwd_reduce_par(const double* __restrict__ part, float* __restrict__ dAr,
                               float* __restrict__ dAi, float* __restrict__ dTk, int D, int N,
                               int NR, int nbg) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t DN = (int64_t)D * N;
  if (e >= DN) return;
  const int c = (int)(e / N), n = (int)(e % N);
  double a = 0.0, bsum = 0.0;
  for (int g = 0; g < nbg; ++g) {
    a += part[(int64_t)g * 2 * DN + e];
    bsum += part[(int64_t)g * 2 * DN + DN + e];
  }
  if (n < NR) {
    dAr[(int64_t)c * NR + n] = (float)a;
    if (dAi != nullptr) dAi[(int64_t)c * NR + n] = (float)(-bsum);
  } else {
    dTk[(int64_t)c * (N - NR) + (n - NR)] = (float)a;
  }
}

template <int S, int NPL, class GK>
static hipError_t launch_bwd_t(const ScanParams& p, const BwdIO& io, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)p.ntiles * io.nbg));
  hipLaunchKernelGGL((scan_bwd_kernel<S, NPL, GK>), grid, dim3(kThreads), 0, st, p, io);
  return hipGetLastError();
}

hipError_t launch_scan_bwd(int S, int NPL, bool spec, const ScanParams& p, const BwdIO& io,
                           hipStream_t st) {
#define RP_CASE(SS, NN)                                                          \
  if (S == SS && NN == NPL)                                                      \
    return spec ? launch_bwd_t<SS, NN, GateKind<NN - 1, 1>>(p, io, st)           \
                : launch_bwd_t<SS, NN, GateKind<0, 2>>(p, io, st);
  RP_FOR_EACH_SHAPE(RP_CASE)
#undef RP_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_finalize(const ScanParams& p, const BwdIO& io, float* d_Bc, float* d_Cc,
                               float* d_Ar, float* d_Ai, float* d_Tk, hipStream_t st) {
  const int64_t per = (int64_t)p.B * p.L * p.N;
  if (per > 0) {
    const int64_t n = 2 * per;
    hipLaunchKernelGGL(bwd_reduce_bc, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       (const float*)io.part_bc, d_Bc, d_Cc, per, p.ntiles);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int64_t dn = (int64_t)p.D * p.N;
  if (dn > 0) {
    hipLaunchKernelGGL(bwd_reduce_par, dim3((unsigned)((dn + 255) / 256)), dim3(256), 0, st,
                       (const double*)io.part_par, d_Ar, d_Ai, d_Tk, p.D, p.N, p.NR, io.nbg);
    return hipGetLastError();
  }
  return hipSuccess;
}

}  // namespace rp
