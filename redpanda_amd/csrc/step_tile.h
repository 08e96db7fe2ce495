// The step tile kernel (the rollout path of rp_step), shared by step.hip
// (d_state == S * NPL) and step_pad.hip (d_state a multiple of 4 below
// S * NPL: pad states).  See step.hip for the two step kernels and how they
// match the scan.
#pragma once

#include <type_traits>

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

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

// Streaming 16-byte loads and stores that bypass cache retention (the state
// is read once and written once per launch).
__device__ __forceinline__ float4 load_stream(const float4* p) {
  float4 v;
  v.x = __builtin_nontemporal_load(&p->x);
  v.y = __builtin_nontemporal_load(&p->y);
  v.z = __builtin_nontemporal_load(&p->z);
  v.w = __builtin_nontemporal_load(&p->w);
  return v;
}
__device__ __forceinline__ void store_stream(float4* p, float4 v) {
  __builtin_nontemporal_store(v.x, &p->x);
  __builtin_nontemporal_store(v.y, &p->y);
  __builtin_nontemporal_store(v.z, &p->z);
  __builtin_nontemporal_store(v.w, &p->w);
}

// FULLD: D is a multiple of the workgroup's channels (no channel guard).
// DSP: delta holds x and the step uses softplus(x).
// RANK1: beta travels as rows [dt*u | B] (D + N floats per rollout); only
// h moves through the LDS block, and beta_prev = (dt*u)_prev * B_prev.
// SHARED (whole tiles only): every rollout starts from the one input state
// (ssr == 0).  Its blocks are read with plain loads, which L2 keeps for the
// other rollouts, where a rollout's own block is read once with streaming
// loads: from a shared state 1.65x faster (4096 rollouts: 144 against
// 237 us); for per-rollout states plain loads were 3-7 % slower.
// PAD: d_state N (a multiple of 4) below S * NPL.  A channel's row in memory
// and in the LDS block is N floats; the slots' states n >= N are pad states,
// held as the lane-layout kernel and the scan hold them (zero state, zero
// B / C, zero beta_prev), so that y's sum over the slices keeps its bits.
template <int S, int NPL, class GK, bool FULLD, bool DSP, bool RANK1, bool SHARED, bool PAD>
__global__ __launch_bounds__(kThreads) void step_tile_kernel(StepParams p) {
  static_assert(FULLD || !SHARED, "the shared-state instantiation is for whole tiles");
  constexpr int NP = S * NPL;
  constexpr int NV = NP / 4;            // float4s per channel at N == NP
  // SPL threads per channel: from 8 slices up (d_state 24-40, 44-96) a
  // channel's states split between S / 4 adjacent lanes, 4 slices each (one
  // float4 per slot), so that the gate parameters and the states of a thread
  // fit the registers of several waves per SIMD (one thread per channel took
  // 256 VGPRs, one wave per SIMD, at d_state 32 all rotational); at 6 and 8
  // slots of 16 (d_state 81-96, 97-128) between S / 2 lanes, 2 slices each
  // (one float2 per slot)
  constexpr int SPL = step_tile_split(S, NPL);
  constexpr int SS = S / SPL;           // slices per thread
  constexpr int NPT = NP / SPL;         // states per thread
  constexpr int NVT = NPL;              // vectors per thread: one per slot
  using V = std::conditional_t<SS == 2, float2, float4>;
  static_assert(SS == 4 || (SS == 2 && SPL > 1), "a thread holds one float4 or float2 per slot");
  static_assert(SPL <= 8, "the y combine covers up to eight threads per channel");
  static_assert(!PAD || SPL > 1, "a one-thread channel (S == 4) has no pad float4s");
  constexpr int VPC = NP / SS;          // vectors per channel at N == NP
  constexpr int TCH = kThreads / SPL;   // channels per workgroup
  constexpr int NBLK = TCH * NV;      // float4s of a block at N == NP
  constexpr int NB = (NBLK + kThreads - 1) / kThreads;  // float4s per thread when staging it (at most)
  constexpr bool WHOLE = NBLK % kThreads == 0;  // whole passes of the workgroup; else the last is bounded
  constexpr int NBC = RANK1 ? 3 : 2;    // rows staged per rollout: B, C (and B_prev)
  constexpr int RIM = step_tile_ri_max(S, NPL, RANK1);  // rollouts per workgroup, at most
  __shared__ float2 sCos[kTab];           // (m, b (-sin a)) records of the gate table
  __shared__ float sBC[RIM][NBC * NP];    // B, C (B_prev) rows of the workgroup's rollouts
  // the (h, beta) block of one rollout: TCH channels x N states each, as in
  // memory ([channel][state]), so float4 k holds channel k / NVM
  // Rank-1 rows with pad states: B_prev is read for every state, then
  // selected (below); with 2 slices per thread (every vector tested at run
  // time) the store-back of a vector past its row goes to a slot of its
  // thread behind the block (kThreads float2s), so that no LDS access sits
  // behind a branch.  The sink not for the generic gate kind (no slot known
  // rotational at compile time), whose registers it would take past three
  // waves per SIMD, nor for full beta blocks, which move twice the bytes per
  // update and gain nothing.
  constexpr bool SINK = RANK1 && PAD && SS == 2 && GK::kRJ > 0;
  constexpr int SINKV = SINK ? kThreads / 2 : 0;  // float4s of the sink
  __shared__ float4 sH[TCH * NV + SINKV], sBt[TCH * NV];
  const int tid = threadIdx.x;
  const int tile = blockIdx.x % p.ctiles, rg = blockIdx.x / p.ctiles;
  const int c0 = tile * TCH;
  const int cl = tid / SPL, half = tid % SPL;  // channel in the tile, slice half
  const int c = c0 + cl;
  const bool cvalid = FULLD || c < p.D;
  const int cld = cvalid ? c : p.D - 1;  // loads stay in bounds; only valid channels store
  const int N = p.N;                    // N == NP, or with PAD N < NP (checked by the host)
  const int NVM = PAD ? N / 4 : NV;     // float4s per channel row
  const int VPM = PAD ? N / SS : VPC;   // vectors (V) per channel row
  // whether the thread's vector of slot v lies in the row; a thread's vector
  // of slot v is the channel's vector v * SPL + half.  With 4 slices per
  // thread pad states only ever fill part of the last slot (N > S * (NPL -
  // 1)), so only that vector is tested at run time; with 2, every one is
  const bool last_in = !PAD || (NPL - 1) * SPL + (tid % SPL) < VPM;
  auto in_row = [&](int v) {
    if constexpr (SS == 2) return !PAD || v * SPL + (tid % SPL) < VPM;
    return v < NVT - 1 || last_in;
  };
  // float4s of the block
  const int nvalid = (FULLD && !PAD) ? NBLK : (FULLD ? TCH : min(TCH, p.D - c0)) * NVM;
  const bool has_imag = p.Ai != nullptr;
  const int r_lo = rg * p.ri;
  const int nr = min(p.R, r_lo + p.ri) - r_lo;  // <= RIM (checked by the host)
  // The prologue issues every load (B / C rows, gate parameters, D) before
  // it stores anything, so their latencies overlap.  The B / C rows of all
  // the workgroup's rollouts are staged once, pad states as zeros.
  constexpr int BCPT = (RIM * NBC * NP + kThreads - 1) / kThreads;
  float bc[BCPT];
#pragma unroll
  for (int k = 0; k < BCPT; ++k) {
    const int e = tid + k * kThreads;
    const int rr = e / (NBC * NP), q = e % (NBC * NP);
    const int col = q % NP;
    const int64_t r = r_lo + rr;
    bc[k] = 0.f;
    if (e < nr * NBC * NP && !(p.bn_fused && q < 2 * NP) && (!PAD || col < N)) {
      if (q < NP)
        bc[k] = p.Bc[r * p.bsr + q];
      else if (q < 2 * NP)
        bc[k] = p.Cc[r * p.csr + (q - NP)];
      else if (p.beta_in != nullptr)  // B_prev: the tail of the rank-1 row
        bc[k] = p.beta_in[r * p.bssr + p.D + (q - 2 * NP)];
    }
  }
  // state i of this thread: slot i / SS, slice half * SS + i % SS
  auto st_n = [&](int i) { return (i / SS) * S + half * SS + i % SS; };
  // the thread's gate parameters stay in registers for all its rollouts
  GateRaw graw[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i)
    graw[i] = gate_param_load(p.Ar, p.Ai, p.Tk, cld, st_n(i), N, p.NR, p.NT, true);
  const float dsk = p.Dskip[cld];
  if (p.bn_fused) {
    // the B and C rows of the workgroup's rollout from the raw projections:
    // BCNorm + p-sum, one wave per row (bcnorm_token, the BCNorm kernel's
    // arithmetic, zero for the pad states); its loads are issued behind the
    // prologue's
    const int lane = tid % kWave, wv = tid / kWave;
    const float invK = 1.f / (float)(N * p.bn_P);
    for (int pr = wv; pr < nr * 2; pr += kWaves) {
      const int rr = pr >> 1, part = pr & 1;
      float wt[1][kBcMaxP];
#pragma unroll
      for (int q = 0; q < kBcMaxP; ++q)
        wt[0][q] = (p.bn_normalize && lane < N && q < p.bn_P) ? p.bn_w[part][lane * p.bn_P + q] : 1.f;
      float acc[1];
      bcnorm_token<1>(p.bn_x[part], (int64_t)(r_lo + rr) * p.bn_xs[part], p.bn_dt, lane, N,
                      p.bn_P, p.bn_normalize != 0, p.bn_eps, invK, wt, acc);
      if constexpr (PAD) {
        if (lane < NP) sBC[rr][part * NP + lane] = lane < N ? acc[0] : 0.f;
      } else {
        if (lane < N) sBC[rr][part * NP + lane] = acc[0];
      }
    }
  }
  fill_cos_lin(sCos, tid);
#pragma unroll
  for (int k = 0; k < BCPT; ++k) {
    const int e = tid + k * kThreads;
    if (e < nr * NBC * NP && !(p.bn_fused && e % (NBC * NP) < 2 * NP))
      sBC[e / (NBC * NP)][e % (NBC * NP)] = bc[k];
  }
  float pah[NPT], wh[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) gate_param_finish(st_n(i), N, p.NR, true, graw[i], pah[i], wh[i]);

  // Per rollout: the block's (h, beta) arrive with coalesced streaming loads
  // (thread t moves float4s t, t+256, ...) into LDS; each thread updates its
  // states of its channel there; coalesced streaming stores write the block
  // back.
  // Every input is in LDS or registers before the first store, so h_out and
  // beta_out may alias h_in and beta_in (per-rollout states).
  for (int rr = 0; rr < nr; ++rr) {
    const int64_t r = r_lo + rr;
    const int64_t blk = (r * p.D + c0) * NVM;  // float4 offset of the output block
    float dt = p.delta[r * p.dsr + cld];
    if constexpr (DSP) dt = softplus_of(dt);
    const float uu = p.u[r * p.usr + cld];
    // the gate branch, when y leaves gated
    const float zz = p.z != nullptr ? load_in(p.z, r * p.zsr + cld, p.dt_z) : 0.f;
    // rank-1: the channel's (dt*u)_prev, halved as the scan halves dt*u
    float hdp = 0.f;
    if (p.h_in != nullptr) {
      if constexpr (RANK1) hdp = 0.5f * p.beta_in[r * p.bssr + cld];
      // input block: the rollout's own, or the one shared state (ssr == 0)
      const int64_t iblk = r * (p.ssr / 4) + (int64_t)c0 * NVM;
      const float4* hi4 = reinterpret_cast<const float4*>(p.h_in) + iblk;
      const float4* bi4 = reinterpret_cast<const float4*>(p.beta_in) + iblk;
      float4 hl[NB], bl[NB];
#pragma unroll
      for (int m = 0; m < NB; ++m) {
        const int k = tid + m * kThreads;
        if ((FULLD && !PAD && WHOLE) || k < nvalid) {
          hl[m] = SHARED ? hi4[k] : load_stream(hi4 + k);
          if constexpr (!RANK1) bl[m] = SHARED ? bi4[k] : load_stream(bi4 + k);
        }
      }
#pragma unroll
      for (int m = 0; m < NB; ++m) {
        const int k = tid + m * kThreads;
        if ((FULLD && !PAD && WHOLE) || k < nvalid) {
          sH[k] = hl[m];
          if constexpr (!RANK1) sBt[k] = bl[m];
        }
      }
    } else {
#pragma unroll
      for (int m = 0; m < NB; ++m) {
        if (WHOLE || tid + m * kThreads < NBLK) {
          sH[tid + m * kThreads] = make_float4(0.f, 0.f, 0.f, 0.f);
          if constexpr (!RANK1) sBt[tid + m * kThreads] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
    __syncthreads();  // the block (and, the first time, the table and B / C rows)
    // the thread's vector v: the channel's vector v * SPL + half; with PAD,
    // beyond the row (pad states) zeros
    V* const sHv = reinterpret_cast<V*>(sH);
    V* const sBv = reinterpret_cast<V*>(sBt);
    V h4[NVT], b4[NVT];
#pragma unroll
    for (int v = 0; v < NVT; ++v) {
      // read as values, then selected (an index past the row stays inside
      // the block's LDS); a select of the two places would load through a
      // generic pointer
      const bool row = in_row(v);
      const int k = cl * VPM + v * SPL + half;
      h4[v] = sHv[k];
      if (!row) h4[v] = V{};
      if constexpr (!RANK1) {
        b4[v] = sBv[k];
        if (!row) b4[v] = V{};
      }
    }
    const float* Bs = sBC[rr];
    const float* Cs = sBC[rr] + NP;
    const float* Bp = sBC[rr] + (NBC - 1) * NP;  // B_prev (rank-1 only)
    const float hd = 0.5f * fmul(dt, uu);
    float ys[SS];
#pragma unroll
    for (int q = 0; q < SS; ++q) ys[q] = 0.f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int j = i / SS, ql = i % SS;
      const int n = st_n(i);
      float& hs = (&h4[i / SS].x)[i % SS];
      float& bs = (&b4[i / SS].x)[i % SS];
      // beta_prev / 2: from the full form, or (dt*u)_prev / 2 * B_prev, the
      // same bits as the product the full form stored (zero for a pad state)
      float hbp;
      if constexpr (RANK1 && PAD) {
        // (a pad state's index stays in the row's LDS; its B_prev is 0)
        const float bpn = fmul(hdp, Bp[n]);
        hbp = in_row(j) ? bpn : 0.f;
      } else {
        hbp = RANK1 ? (in_row(j) ? fmul(hdp, Bp[n]) : 0.f) : 0.5f * bs;
      }
      const float g = gate_of<S, GK>(j, half * SS + ql, p.NR, has_imag, dt, pah[i], wh[i], sCos);
      const float hb = fmul(hd, Bs[n]);
      hs = ffma(g, hs, ffma(g, hbp, hb));  // fwd_update's form and rounding
      if constexpr (!RANK1) bs = 2.f * hb;
      ys[ql] = ffma(hs, Cs[n], ys[ql]);
    }
    // the channel's y: the balanced tree over its S slices, whose subtrees of
    // 4 slices are the threads' trees when split, combined pairwise as the
    // tree pairs them (fp addition commutes, so every lane of the channel
    // gets the same bits)
    float ysum = tree_sum<SS>(ys);
    if constexpr (SPL >= 2) ysum = ysum + __shfl_xor(ysum, 1);
    if constexpr (SPL >= 4) ysum = ysum + __shfl_xor(ysum, 2);
    if constexpr (SPL >= 8) ysum = ysum + __shfl_xor(ysum, 4);
    if (cvalid && half == 0) {
      float yv = ysum + fmul(uu, dsk);
      if (p.z != nullptr) yv = silu_gate(yv, zz, p.dt_z);
      p.y[r * p.D + c] = yv;
      if constexpr (RANK1) p.beta_out[r * (p.D + N) + c] = fmul(dt, uu);
    }
    if constexpr (RANK1) {
      if (tile == 0 && tid < N) p.beta_out[r * (p.D + N) + p.D + tid] = Bs[tid];
    }
#pragma unroll
    for (int v = 0; v < NVT; ++v) {
      if constexpr (SINK) {
        const int k = in_row(v) ? cl * VPM + v * SPL + half : TCH * NV * 2 + tid;
        sHv[k] = h4[v];
      } else if (in_row(v)) {
        sHv[cl * VPM + v * SPL + half] = h4[v];
        if constexpr (!RANK1) sBv[cl * VPM + v * SPL + half] = b4[v];
      }
    }
    __syncthreads();  // the updated block
    float4* ho4 = reinterpret_cast<float4*>(p.h_out) + blk;
    float4* bo4 = reinterpret_cast<float4*>(p.beta_out) + blk;
#pragma unroll
    for (int m = 0; m < NB; ++m) {
      const int k = tid + m * kThreads;
      if ((FULLD && !PAD && WHOLE) || k < nvalid) {
        store_stream(ho4 + k, sH[k]);
        if constexpr (!RANK1) store_stream(bo4 + k, sBt[k]);
      }
    }
    __syncthreads();  // the block's LDS is free for the next rollout
  }
}

template <int S, int NPL, class GK, bool DSP, bool RANK1, bool PAD>
hipError_t launch_step_tile_d(const StepParams& p, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)p.ctiles * p.rgroups));
  const int tch = kThreads / step_tile_split(S, NPL);
  if (p.D % tch == 0 && p.ssr == 0)
    hipLaunchKernelGGL((step_tile_kernel<S, NPL, GK, true, DSP, RANK1, true, PAD>), grid,
                       dim3(kThreads), 0, st, p);
  else if (p.D % tch == 0)
    hipLaunchKernelGGL((step_tile_kernel<S, NPL, GK, true, DSP, RANK1, false, PAD>), grid,
                       dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL((step_tile_kernel<S, NPL, GK, false, DSP, RANK1, false, PAD>), grid,
                       dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <int S, int NPL, class GK, bool PAD>
hipError_t launch_step_tile_t(const StepParams& p, hipStream_t st) {
  if (p.rank1)
    return p.dsp ? launch_step_tile_d<S, NPL, GK, true, true, PAD>(p, st)
                 : launch_step_tile_d<S, NPL, GK, false, true, PAD>(p, st);
  return p.dsp ? launch_step_tile_d<S, NPL, GK, true, false, PAD>(p, st)
               : launch_step_tile_d<S, NPL, GK, false, false, PAD>(p, st);
}

// The tile kernel for shape (S, NPL), with or without pad states; without,
// also the all-rotational gate kind (no slot decided at run time) and, on
// all_gate_shape, the all-real one.
template <int S, int NPL, bool PAD>
hipError_t launch_step_tile(int gk, const StepParams& p, hipStream_t st) {
  if constexpr (step_tile_shape(S, NPL) && (!PAD || step_tile_split(S, NPL) > 1)) {
    if constexpr (!PAD) {
      if (gk == kGateRotAll) return launch_step_tile_t<S, NPL, GateKind<NPL, 1, NPL>, PAD>(p, st);
      if constexpr (all_gate_shape(S, NPL)) {
        if (gk == kGateRealAll)
          return launch_step_tile_t<S, NPL, GateKind<NPL, 0, NPL>, PAD>(p, st);
      }
    }
    return with_gate_kind<NPL>(gk, [&](auto g) {
      return launch_step_tile_t<S, NPL, decltype(g), PAD>(p, st);
    });
  } else {
    return hipErrorInvalidValue;
  }
}

}  // namespace rp
