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
// q_t is formed as fma(g_{t+1}, q_{t+1}, dy_t C_t) and dhb_t as 2 q_t - dy_t
// C_t: one rounding per step at q's magnitude (fwd_update in rp_device.h has
// the forward's counterpart and the reason).  The chunk recompute keeps the
// form h_t = g_t s_{t-1} + hb_t, since dg needs s_{t-1} anyway; it restarts
// from the forward's checkpoint every kCkptK steps, so its states stay
// within an ulp or two of the forward's and its roundings do not accumulate.
//
// Work split: one workgroup = CB channels x a group of `bg` batch rows, both
// directions.  The forward stored the state entering every kCkptK-step chunk;
// the backward walks chunks in reverse, recomputes the chunk's K steps into
// registers (keeping s_{t-1}, the gate and e*sin, so the adjoint evaluates
// no transcendental), then runs the adjoint over them.  The recompute
// evaluates the forward's gate expansion from (m, b sin) table records,
// which also give the sine (one 8-byte table read; the forward's records
// would need a second read for it); each gate matches the forward's to
// within an ulp and every chunk restarts from the forward's checkpoint.
//
// Streaming: the per-step inputs (dt, (dt*u)/2, u, dy per channel; B, C per
// state) of a chunk and of the step before it sit in one of two LDS slots.
// While chunk c is computed from its slot, the inputs of chunk c-1 are loaded
// into registers and written to the other slot after the compute, so
// global-memory latency hides behind a whole chunk; the checkpoint entering
// the next chunk and every value a read-modify-write needs (reverse
// direction) are likewise loaded a chunk ahead.  The chunk code is
// instantiated per slot, so every LDS address is a compile-time offset.
//
// Reductions, all in a fixed order (run-to-run deterministic; no address is
// updated by more than one thread):
//   * over a channel's states (ddt, du): in-lane FMA chain, then the S lanes'
//     partials summed pairwise from LDS where the chunk's outputs are written;
//   * over channels (dB, dC): DPP row rotations inside each 16-lane row, the
//     row partials staged in LDS, then a balanced 16-way sum per output, per tile;
//     the per-tile partials are summed in float64 by a second kernel;
//   * parameter gradients (dA, dTk): fp32 sums over up to 16 chunks (64
//     steps) accumulated in float64 per lane over the batch group (above 40
//     states per channel, in the group's global partials by atomic adds that
//     only that lane makes), then float64 across groups.

#pragma once

#include <type_traits>

#include "rp_device.h"
#include "rp_launch.h"

namespace rp {

// Chunks whose parameter-gradient terms are summed in fp32 before they are
// added into the float64 sums (64 steps).
constexpr int kParChunks = 16;

// FAST: the instantiation for launches with no initial state, no final-state
// gradients and every channel of every tile present, whose arrays span less
// than 4 GiB each (bwd_fast in scan_bwd.hip).  Every global address of the chunk loop
// is then a wave-uniform base pointer plus a 32-bit byte offset, taken per
// batch-row sweep and moved by a uniform multiple of the chunk index: one
// full-rate add per staged element, where the general form multiplies 64-bit
// indices per element and chunk.  Both instantiations compute the same
// values in the same order.
// One channel tile's backward over the workgroup's batch rows: tile `tile`,
// the tpass-th of the io.tpw adjacent tiles the workgroup walks (tile group
// tgrp), batch group bgi.  The tiles of a group share one dB / dC partial
// block: the first writes it, the others add onto it (as the reverse
// direction adds onto the forward direction's), in tile order.
template <int S, int NPL, class GK, bool FAST, bool MULTI>
__device__ __forceinline__ void scan_bwd_tile(const ScanParams& p, const BwdIO& io, int tile,
                                              int tpass, int tgrp, int bgi) {
  using Sh = Shape<S, NPL>;
  // ALT: the entry state is prefetched into two buffers that alternate with
  // the LDS slot (the chunk in slot SL enters from buffer SL and loads the
  // next chunk's entry into the other), and a chunk takes its entry before
  // it issues its own loads.  Loads complete in issue order, so a wait for a
  // single prefetch buffer, copied after the chunk's loads were issued, had
  // to wait for those loads too.  The second buffer costs registers: only
  // instantiations with room take it (without spills).
  constexpr bool ALT = NPL <= 3 || (NPL == 4 && S >= 8) ||
                       (NPL == 5 && S == 8 && GK::kRJ == NPL - 1 && GK::kTJ == NPL - 1);
  constexpr int DT = Sh::kDT, CB = Sh::kCB, NP = Sh::kNP, K = kCkptK;
  // Steps per channel-sum fold: one fold (two barriers) per chunk up to 40
  // states and for 16 lanes x 5 slots with the last slot tracking in every
  // lane (N 65-80 with 64 rotational states, the long-sequence shape:
  // measured 1.7 % faster), two folds elsewhere above 40 states (a whole
  // chunk's row partials spilled registers there and measured 3-5 % slower).
  // Above 40 states a whole chunk's row partials take the LDS that the
  // per-thread float64 parameter sums would: those then go to their global
  // per-batch-group partials instead (the same additions in the same order).
  constexpr bool FOLD_CHUNK = S * NPL <= 40 || (S == 16 && NPL == 5 && GK::kImag == 1 &&
                                                GK::kRJ == NPL - 1 && GK::kTJ == NPL - 1);
  constexpr int KR = FOLD_CHUNK ? K : K / 2;
  // ONEBAR (FAST, one fold per chunk, up to 40 states): the row partials
  // and the (d_delta, d_u) sit in one of two buffers by the chunk's slot, so
  // no wave can overwrite a buffer before every wave has folded it (the next
  // writer of a buffer is two chunks on, past the next chunk's barrier) and
  // a chunk ends without the second barrier.  The second buffers take the
  // LDS of the per-thread float64 parameter sums, which then go to their
  // global partials (the same additions in the same order).
  constexpr bool ONEBAR = FAST && FOLD_CHUNK && S * NPL <= 40;
  constexpr int NB = ONEBAR ? 2 : 1;  // row-partial and (d_delta, d_u) buffers
  // staging of the next chunk's inputs after the recompute (one barrier per
  // chunk, fewer than 40 states) instead of at the chunk's end
  constexpr bool EARLY_STAGE = ONEBAR && S * NPL < 40;
  constexpr bool PAR_GLOBAL = (S * NPL > 40 && FOLD_CHUNK) || ONEBAR;
  constexpr int NFOLD = K / KR;             // folds per chunk
  constexpr int NRW = kWaves * 4;           // 16-lane rows per workgroup
  // row partials of one output are contiguous (4 x 16-byte reads); the
  // padding to 20 spreads the writers of a row over distinct banks
  constexpr int RWP = NRW + 4;
  static_assert(NRW == 16, "the fold sums 16 row partials");
  constexpr int FPT = (KR * 2 * NP + kThreads - 1) / kThreads;  // fold outputs per thread
  constexpr int KS = K + 1;  // staged steps per chunk: the step before it, then its K steps
  constexpr int CPT = (KS * CB + kThreads - 1) / kThreads;      // staged channel-steps per thread
  constexpr int SPT = (KS * NP + kThreads - 1) / kThreads;      // staged state-steps per thread
  constexpr int DPT = (K * CB + kThreads - 1) / kThreads;       // d_delta / d_u outputs per thread
  // keep each step's h_t from the recompute (up to 40 states per channel;
  // larger shapes recompute it in the adjoint to stay within registers)
  constexpr bool KEEP_HT = NP <= 40;
  static_assert(K % KR == 0, "a chunk holds whole folds");
  __shared__ float4 sCh[2][KS][CB];       // input slots: (dt, (dt*u)/2, u/2, dy)
  __shared__ float sB[2][KS][NP];
  __shared__ float sC[2][KS][NP];
  __shared__ __align__(16) float sRed[NB][KR][2][NP][RWP];  // per-row channel sums of dB, dC
  // per lane: its (d gate / d dt, dhb . B) sums over its states of each
  // chunk step, summed over the channel's S lanes where the chunk's
  // (d_delta, d_u) are written.  Channel-contiguous per lane slice s; the
  // row of a slice padded to CB + 16/S so that 16 lanes' writes (16/S
  // channels x S slices) meet 32 distinct banks.
  constexpr int DDP = CB + 16 / S;
  __shared__ float2 sDD[NB][K][S][DDP];
  __shared__ float2 sCS[kTab];              // (m, b sin) records of the gate table
  // per-thread float64 sums of the parameter gradients over the batch group
  // (dA_real or dtrack, dA_imag), kept in LDS to spare registers (in their
  // global partials when PAR_GLOBAL)
  __shared__ double sPar[PAR_GLOBAL ? 1 : 2][PAR_GLOBAL ? 1 : NPL][PAR_GLOBAL ? 1 : kThreads];

  // MULTI (a walk over several tiles): the thread index through an opaque
  // copy, so that what derives from it is computed per tile instead of
  // hoisted out of the walk and held in registers across it
  int tid = threadIdx.x;
  if constexpr (MULTI) asm volatile("" : "+v"(tid));
  const int wave = tid / kWave, lane = tid % kWave;
  const int dl = lane / S, s = lane % S;
  const int cl = wave * DT + dl;
  const int wrow = wave * 4 + lane / 16;  // row index within the workgroup
  const int c = tile * CB + cl;
  const bool cvalid = FAST || c < p.D;
  const bool has_imag = p.Ai != nullptr;
  const int L = p.L;

  GateRegs<NPL> gp;  // loads issued first, so the table copy overlaps them
  load_gate_regs<S, NPL>(gp, p.Ar, p.Ai, p.Tk, c, s, p.N, p.NR, p.NT, cvalid);
  // first read after the staging barrier below (the table stays from the
  // workgroup's first tile on)
  if (tpass == 0) fill_sincos_pairs(sCS, tid);
  // pam: the coefficient of the ddt sum over rotational states, zero for a
  // tracking state (only read for slots whose kind is decided at run time)
  float pam[NPL];
  // this thread's entry for state slot j of the per-batch-group partials
  // (dA_real or dtrack; dA_imag is one D*N block further)
  auto par_at = [&](int j) { return ((int64_t)bgi * 2) * p.D * p.N + (int64_t)c * p.N + j * S + s; };
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    pam[j] = is_rot<S, GK>(j, s, p.NR) ? gp.pah[j] : 0.f;
    if constexpr (PAR_GLOBAL) {
      if (cvalid && j * S + s < p.N) {
        io.part_par[par_at(j)] = 0.0;
        io.part_par[par_at(j) + (int64_t)p.D * p.N] = 0.0;
      }
    } else {
      sPar[0][j][tid] = 0.0;
      sPar[1][j][tid] = 0.0;
    }
  }

  // time index of forward-order step i in this direction
  auto tix = [&](int dir, int i) { return dir ? (L - 1 - i) : i; };
  // Inputs of chunk ch (rows 1..K) and of the step before it (row 0) as
  // stored: loaded into registers (stage_load), then converted into an LDS
  // slot (stage_store).  Steps and channels beyond the data load as zeros.
  uint32_t rdt[CPT], ru[CPT], rb[SPT], rc[SPT];
  float rdy[CPT];
  // delta as staged: the input itself, or with softplus the forward's cache
  // of softplus(x) (fp32, contiguous)
  const bool cached = p.dsp != 0;
  const void* dsrc = cached ? static_cast<const void*>(io.dcache) : p.delta;
  const int64_t d_sb = cached ? (int64_t)L * p.D : p.dsb;
  const int64_t d_sl = cached ? (int64_t)p.D : p.dsl;
  const int d_dt = cached ? RP_F32 : p.dt_delta;
  // FAST: this thread's byte offsets for the sweep (b, dir) as they would be
  // at chunk 0, and the wave-uniform byte step per chunk: the offset at chunk
  // ch is o + ch * step (mod 2^32; the elements a lane loads or stores lie in
  // their arrays, whose spans fit in 32 bits).  oF is relative to the
  // sweep's (tile group, b) block of the dB / dC partials, pbc.
  uint32_t oDT[CPT], oU[CPT], oDY[CPT], oB[SPT], oC[SPT], oF[NFOLD][FPT], oD[DPT];
  uint32_t stDT = 0, stU = 0, stDY = 0, stB = 0, stC = 0, stF = 0;
  float* pbc = io.part_bc;
  // FAST: fold output k of this thread as LDS float index * 8 + its row
  // within the fold, or -1 beyond the fold's outputs
  int fInfo[FPT];
  // FAST: fold output of this thread in round k; the last, partial round
  // runs on the last waves (the d_delta / d_u outputs run on the first)
  constexpr int FREM = KR * 2 * NP - (FPT - 1) * kThreads;  // outputs in the last round
  auto fold_e = [&](int k) {
    if (k < FPT - 1) return tid + k * kThreads;
    return tid < kThreads - FREM ? -1 : tid + k * kThreads - (kThreads - FREM);
  };
  if constexpr (FAST) {
#pragma unroll
    for (int k = 0; k < FPT; ++k) {
      const int e = fold_e(k);
      fInfo[k] = -1;
      if (e >= 0 && e < KR * 2 * p.N) {
        const int rr = e / (2 * p.N), rem = e % (2 * p.N);
        const int which = rem / p.N, n = rem % p.N;
        const int kk = (n % S) * NPL + n / S;
        fInfo[k] = (((rr * 2 + which) * NP + kk) * RWP) * 8 + rr;
      }
    }
  }
  auto fast_sweep = [&](int b, int dir) {
    const int64_t sg = dir ? -1 : 1;  // time steps per forward-order step
    const int64_t t0 = dir ? L - 1 : 0;
    const int64_t es_d = d_dt == RP_F32 ? 4 : 2, es_u = p.dt_u == RP_F32 ? 4 : 2;
    const int64_t es_b = p.dt_B == RP_F32 ? 4 : 2, es_c = p.dt_C == RP_F32 ? 4 : 2;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int e = tid + k * kThreads;
      const int64_t t = t0 + sg * (e / CB - 1), c2 = tile * CB + e % CB;
      oDT[k] = (uint32_t)((b * d_sb + t * d_sl + c2) * es_d);
      oU[k] = (uint32_t)((b * p.usb + t * p.usl + c2) * es_u);
      oDY[k] = (uint32_t)((((int64_t)b * L + t) * p.D + c2) * 4);
    }
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int e = tid + k * kThreads;
      const int kk = e % NP;
      const int64_t t = t0 + sg * (e / NP - 1), n = (kk % NPL) * S + kk / NPL;
      oB[k] = (uint32_t)((b * p.bsb + t * p.bsl + n) * es_b);
      oC[k] = (uint32_t)((b * p.csb + t * p.csl + n) * es_c);
    }
    const int64_t half = (int64_t)io.ntg * p.B * L * p.N;  // the dC half of the partials
#pragma unroll
    for (int f = 0; f < NFOLD; ++f) {
#pragma unroll
      for (int k = 0; k < FPT; ++k) {
        const int e = fold_e(k);
        const int rr = e / (2 * p.N), rem = e % (2 * p.N);
        const int64_t t = t0 + sg * (f * KR + rr);
        oF[f][k] = (uint32_t)(((rem / p.N) * half + t * p.N + rem % p.N) * 4);
      }
    }
#pragma unroll
    for (int k = 0; k < DPT; ++k) {
      const int e = tid + k * kThreads;
      const int64_t t = t0 + sg * (e / CB), c2 = tile * CB + e % CB;
      oD[k] = (uint32_t)((((int64_t)b * L + t) * p.D + c2) * 4);
    }
    stDT = (uint32_t)(sg * K * d_sl * es_d);
    stU = (uint32_t)(sg * K * p.usl * es_u);
    stDY = (uint32_t)(sg * K * p.D * 4);
    stB = (uint32_t)(sg * K * p.bsl * es_b);
    stC = (uint32_t)(sg * K * p.csl * es_c);
    stF = (uint32_t)(sg * K * p.N * 4);
    pbc = io.part_bc + ((int64_t)tgrp * p.B + b) * L * p.N;
  };
  // FAST: the storage codes of (delta as staged, u, B and C) as one of the
  // common combinations, fixed at compile time in the staging code, so that
  // a staging branches once on them instead of once per element (-1: codes
  // read at run time)
  const int tcombo =
      !FAST ? -1
      : (d_dt == RP_BF16 && p.dt_u == RP_BF16 && p.dt_B == RP_BF16 && p.dt_C == RP_BF16) ? 0
      : (d_dt == RP_F32 && p.dt_u == RP_F32 && p.dt_B == RP_F32 && p.dt_C == RP_F32)     ? 1
      : (d_dt == RP_F32 && p.dt_u == RP_BF16 && p.dt_B == RP_F32 && p.dt_C == RP_F32)    ? 2
      : (d_dt == RP_F32 && p.dt_u == RP_F16 && p.dt_B == RP_F32 && p.dt_C == RP_F32)     ? 3
      : (d_dt == RP_F16 && p.dt_u == RP_F16 && p.dt_B == RP_F16 && p.dt_C == RP_F16)     ? 4
                                                                                          : -1;
  using TBF = std::integral_constant<int, RP_BF16>;
  using TF32 = std::integral_constant<int, RP_F32>;
  using TF16 = std::integral_constant<int, RP_F16>;
  using TRT = std::integral_constant<int, -1>;
  auto with_types = [&](auto f) {
    switch (tcombo) {
      case 0: f(TBF{}, TBF{}, TBF{}); break;
      case 1: f(TF32{}, TF32{}, TF32{}); break;
      case 2: f(TF32{}, TBF{}, TF32{}); break;
      case 3: f(TF32{}, TF16{}, TF32{}); break;
      case 4: f(TF16{}, TF16{}, TF16{}); break;
      default: f(TRT{}, TRT{}, TRT{}); break;
    }
  };
  // an element as stored (type IT, or the run-time code rt when IT is -1),
  // and its value
  auto load_t = [&](auto it_tag, const void* base, uint32_t off, int rt) -> uint32_t {
    constexpr int IT = decltype(it_tag)::value;
    if constexpr (IT < 0)
      return load_raw_byte(base, off, rt);
    else
      return load_byte<RawOf<IT>>(base, off);
  };
  auto cvt_t = [&](auto it_tag, uint32_t v, int rt) -> float {
    constexpr int IT = decltype(it_tag)::value;
    if constexpr (IT < 0)
      return cvt_raw(v, rt);
    else
      return cvt_raw(v, IT);
  };
  auto stage_load = [&](int b, int dir, int ch) {
    if constexpr (FAST) {
      const uint32_t cu = (uint32_t)ch;
      with_types([&](auto tdt, auto tu, auto ts) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
          const int e = tid + k * kThreads;
          const int i = ch * K + e / CB - 1;
          rdt[k] = 0u;
          ru[k] = 0u;
          rdy[k] = 0.f;
          if (e < KS * CB && (unsigned)i < (unsigned)L) {
            rdt[k] = load_t(tdt, dsrc, oDT[k] + cu * stDT, d_dt);
            ru[k] = load_t(tu, p.u, oU[k] + cu * stU, p.dt_u);
            rdy[k] = load_byte<float>(io.dy, oDY[k] + cu * stDY);
          }
        }
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
          const int e = tid + k * kThreads;
          const int kk = e % NP;
          const int i = ch * K + e / NP - 1;
          rb[k] = 0u;
          rc[k] = 0u;
          if (e < KS * NP && (kk % NPL) * S + kk / NPL < p.N && (unsigned)i < (unsigned)L) {
            rb[k] = load_t(ts, p.Bc, oB[k] + cu * stB, p.dt_B);
            rc[k] = load_t(ts, p.Cc, oC[k] + cu * stC, p.dt_C);
          }
        }
      });
      return;
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int e = tid + k * kThreads;
      const int r = e / CB, ci = e % CB;
      const int i = ch * K + r - 1, c2 = tile * CB + ci;
      rdt[k] = 0u;
      ru[k] = 0u;
      rdy[k] = 0.f;
      if (e < KS * CB && i >= 0 && i < L && c2 < p.D) {
        const int t = tix(dir, i);
        rdt[k] = load_raw(dsrc, (int64_t)b * d_sb + (int64_t)t * d_sl + c2, d_dt);
        ru[k] = load_raw(p.u, (int64_t)b * p.usb + (int64_t)t * p.usl + c2, p.dt_u);
        rdy[k] = io.dy[((int64_t)b * L + t) * p.D + c2];
      }
    }
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int e = tid + k * kThreads;
      const int r = e / NP, kk = e % NP;
      const int n = (kk % NPL) * S + (kk / NPL);
      const int i = ch * K + r - 1;
      rb[k] = 0u;
      rc[k] = 0u;
      if (e < KS * NP && i >= 0 && i < L && n < p.N) {
        const int t = tix(dir, i);
        rb[k] = load_raw(p.Bc, (int64_t)b * p.bsb + (int64_t)t * p.bsl + n, p.dt_B);
        rc[k] = load_raw(p.Cc, (int64_t)b * p.csb + (int64_t)t * p.csl + n, p.dt_C);
      }
    }
  };
  auto stage_store = [&](auto slot_tag) {
    constexpr int SL = decltype(slot_tag)::value;
    if constexpr (FAST) {
      with_types([&](auto tdt, auto tu, auto ts) {
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
          const int e = tid + k * kThreads;
          if (e < KS * CB) {
            const float dt = cvt_t(tdt, rdt[k], d_dt);
            const float uu = cvt_t(tu, ru[k], p.dt_u);
            sCh[SL][e / CB][e % CB] = make_float4(dt, 0.5f * fmul(dt, uu), 0.5f * uu, rdy[k]);
          }
        }
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
          const int e = tid + k * kThreads;
          if (e < KS * NP) {
            sB[SL][e / NP][e % NP] = cvt_t(ts, rb[k], p.dt_B);
            sC[SL][e / NP][e % NP] = cvt_t(ts, rc[k], p.dt_C);
          }
        }
      });
      return;
    }
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int e = tid + k * kThreads;
      if (e < KS * CB) {
        const float dt = cvt_raw(rdt[k], d_dt);
        const float uu = cvt_raw(ru[k], p.dt_u);
        sCh[SL][e / CB][e % CB] = make_float4(dt, 0.5f * fmul(dt, uu), 0.5f * uu, rdy[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int e = tid + k * kThreads;
      if (e < KS * NP) {
        sB[SL][e / NP][e % NP] = cvt_raw(rb[k], p.dt_B);
        sC[SL][e / NP][e % NP] = cvt_raw(rc[k], p.dt_C);
      }
    }
  };
  using Slot0 = std::integral_constant<int, 0>;
  using Slot1 = std::integral_constant<int, 1>;
  // h entering chunk `chunk` of this lane's states: the forward's checkpoint,
  // or for chunk 0 the initial state (zero unless h0 is given, causal only)
  auto load_entry_h = [&](int chunk, int b, int dir, float (&dst)[NPL]) {
    if constexpr (FAST) {
      // no initial state: zero entering chunk 0
      if (chunk == 0) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) dst[j] = 0.f;
      } else {
        const int64_t rec = ((int64_t)(dir * p.B + b) * p.nck + (chunk - 1)) * p.ntiles + tile;
        const float* src =
            io.ckpt + (rec * kWaves + __builtin_amdgcn_readfirstlane(wave)) * (NPL * kWave);
#pragma unroll
        for (int j = 0; j < NPL; ++j) dst[j] = load_at<float>(src, (uint32_t)(lane + j * kWave));
      }
      return;
    }
    if (chunk == 0) {
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const int n = j * S + s;
        dst[j] = 0.f;
        if (dir == 0 && p.h0 != nullptr && cvalid && n < p.N)
          dst[j] = p.h0[((int64_t)b * p.D + c) * p.N + n];
      }
    } else {
      const int64_t rec = ((int64_t)(dir * p.B + b) * p.nck + (chunk - 1)) * p.ntiles + tile;
      const float* src = io.ckpt + (rec * kWaves + wave) * (NPL * kWave) + lane;
#pragma unroll
      for (int j = 0; j < NPL; ++j) dst[j] = src[j * kWave];
    }
  };
  // The (which, t, n) partial of tile group tgrp, batch row b that fold output e
  // of the fold starting at chunk step mf writes; null when beyond the chunk.
  auto fold_dst = [&](int e, int b, int dir, int i0, int mf, int kcnt) -> float* {
    const int rr = e / (2 * p.N);
    if (e >= KR * 2 * p.N || mf + rr >= kcnt) return nullptr;
    const int rem = e % (2 * p.N);
    const int which = rem / p.N, n = rem % p.N;
    const int t = tix(dir, i0 + mf + rr);
    return io.part_bc + (((int64_t)which * io.ntg + tgrp) * p.B + b) * ((int64_t)L * p.N) +
           (int64_t)t * p.N + n;
  };
  // The d_delta / d_u element of chunk step e / CB, channel e % CB; -1 when
  // beyond the chunk or the channels.
  auto dd_index = [&](int e, int b, int dir, int i0, int kcnt) -> int64_t {
    const int r = e / CB, c2 = tile * CB + e % CB;
    if (e >= K * CB || r >= kcnt || c2 >= p.D) return -1;
    return ((int64_t)b * L + tix(dir, i0 + r)) * p.D + c2;
  };
  // (d_delta, d_u) of one chunk step and channel from its S lanes' partial
  // sums (d gate / d dt, dhb . B) in sDD: the sums over the lanes in the
  // order of reduce_states (pairwise, adjacent halves), then
  //     d_delta = dga + u/2 * sBc,   d_u = dt/2 * sBc   (hb = (dt*u)/2 * B)
  auto dd_of = [&](int buf, int r, int cc, float dt, float uh) -> float2 {
    float2 v[S];
#pragma unroll
    for (int i = 0; i < S; ++i) v[i] = sDD[buf][r][i][cc];
#pragma unroll
    for (int w = 1; w < S; w *= 2)
#pragma unroll
      for (int i = 0; i < S; i += 2 * w) v[i] = make_float2(v[i].x + v[i + w].x, v[i].y + v[i + w].y);
    return make_float2(v[0].x + fmul(uh, v[0].y), fmul(0.5f * dt, v[0].y));
  };
  // whether this direction's d_delta store is the last one (the gradient
  // is then complete and, with softplus, taken through it)
  auto dd_final = [&](int dir) { return dir == p.ndir - 1; };

  const int b_lo = bgi * io.bg;
  const int b_hi = min(p.B, b_lo + io.bg);
  const int nct = (L + K - 1) / K;  // chunks per sweep

  for (int b = b_lo; b < b_hi; ++b) {
    for (int dir = 0; dir < p.ndir; ++dir) {
      // qn, gn: q and g of the step processed before (the next in the
      // recurrence's time order), so that q_t = fma(g_{t+1}, q_{t+1}, dy_t C_t)
      // rounds once at q's magnitude (see fwd_update in rp_device.h), and
      // dhb_t = q_t + g_{t+1} q_{t+1} = 2 q_t - dy_t C_t.  An outside consumer
      // of the final state (general instantiation, causal) contributes
      // dh_last to the last step's q (as qn with gn = 1) and 2 * dbeta_last
      // to its dhb (gr, used at that step only: fin).
      float qn[NPL], gn[NPL], gr[NPL];
      bool fin = false;
      // dB / dC partials added onto the block's values: the reverse
      // direction, and every sweep of the group's later tiles
      const bool add_bc = dir == 1 || tpass > 0;
      if constexpr (FAST) fast_sweep(b, dir);
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const int n = j * S + s;
        qn[j] = 0.f;
        gn[j] = 0.f;
        gr[j] = 0.f;
        if (!FAST && dir == 0 && cvalid && n < p.N) {
          const int64_t idx = ((int64_t)b * p.D + c) * p.N + n;
          if (io.dh_last != nullptr) {
            qn[j] = io.dh_last[idx];
            gn[j] = 1.f;
          }
          if (io.dbeta_last != nullptr) gr[j] = 2.f * io.dbeta_last[idx];
        }
      }
      if constexpr (!FAST) fin = dir == 0 && (io.dh_last != nullptr || io.dbeta_last != nullptr);
      // parameter-gradient sums over up to kParChunks chunks (fp32), added
      // into the float64 per-thread sums every kParChunks chunks and at the
      // end of the sweep; cpt: the tracking-state sum of a slot decided at
      // run time
      float cpa[NPL], cpb[NPL], cpt[NPL];
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        cpa[j] = 0.f;
        cpb[j] = 0.f;
        cpt[j] = 0.f;
      }
      // the entry state of the next chunk to process, loaded one chunk ahead
      // (with ALT, into the buffer of that chunk's LDS slot)
      float hE[ALT ? 2 : 1][NPL];
      if (nct > 0) {
        if (ALT && (nct - 1) % 2 == 1)
          load_entry_h(nct - 1, b, dir, hE[ALT ? 1 : 0]);
        else
          load_entry_h(nct - 1, b, dir, hE[0]);
        // stage the sweep's first chunk (the slots are free: the previous
        // sweep ended with a barrier)
        stage_load(b, dir, nct - 1);
        if ((nct - 1) % 2 == 0)
          stage_store(Slot0{});
        else
          stage_store(Slot1{});
        __syncthreads();
        // the first entry state waited for here too, so that on entering the
        // chunk loop no load is pending into its registers (the loop's waits
        // are placed for both ways in)
#pragma unroll
        for (int a = 0; a < (ALT ? 2 : 1); ++a)
#pragma unroll
          for (int j = 0; j < NPL; ++j) asm volatile("" : "+v"(hE[a][j]));
      }

      // one chunk, its slot and whether it is whole fixed at compile time
      auto one_chunk = [&](const int ch, auto full_arg, auto slot_arg) {
        const int i0 = ch * K;
        const int kcnt = min(K, L - i0);
        float prev[NFOLD][FPT], pdd[DPT][2];
        float hc[NPL], hbp[NPL];
        // loads a chunk ahead: the inputs of chunk ch-1, the partials the
        // reverse direction adds to (dB / dC and d_delta / d_u; dB / dC also
        // from the tile group's second tile on), and the state entering
        // chunk ch-1 (into `next`)
        auto issue_loads = [&](float (&next)[NPL]) {
          if (ch >= 1) stage_load(b, dir, ch - 1);
#pragma unroll
          for (int f = 0; f < NFOLD; ++f) {
#pragma unroll
            for (int k = 0; k < FPT; ++k) {
              prev[f][k] = 0.f;
              if constexpr (FAST) {
                if (add_bc && fInfo[k] >= 0 && f * KR + (fInfo[k] & 7) < kcnt)
                  prev[f][k] = load_byte<float>(pbc, oF[f][k] + (uint32_t)ch * stF);
              } else if (add_bc) {
                const float* src = fold_dst(tid + k * kThreads, b, dir, i0, f * KR, kcnt);
                if (src != nullptr) prev[f][k] = *src;
              }
            }
          }
#pragma unroll
          for (int k = 0; k < DPT; ++k) {
            pdd[k][0] = 0.f;
            pdd[k][1] = 0.f;
            if constexpr (FAST) {
              const int e = tid + k * kThreads;
              if (dir == 1 && e < K * CB && e / CB < kcnt) {
                const uint32_t o = oD[k] + (uint32_t)ch * stDY;
                pdd[k][0] = load_byte<float>(io.pd_delta, o);
                pdd[k][1] = load_byte<float>(io.pd_u, o);
              }
            } else if (dir == 1) {
              const int64_t idx = dd_index(tid + k * kThreads, b, dir, i0, kcnt);
              if (idx >= 0) {
                pdd[k][0] = io.pd_delta[idx];
                pdd[k][1] = io.pd_u[idx];
              }
            }
          }
          if (ch > 0) load_entry_h(ch - 1, b, dir, next);
        };
        // The entry state into hc, waited for here: its loads were issued a
        // chunk earlier and have completed.  The opaque use keeps the wait
        // before this chunk's own loads; at a later first use it would also
        // wait for those (loads complete in issue order).
        auto take_entry = [&](const float (&src)[NPL]) {
#pragma unroll
          for (int j = 0; j < NPL; ++j) {
            hc[j] = src[j];
            asm volatile("" : "+v"(hc[j]));
          }
        };
        if constexpr (!ALT) {
          // the entry state is copied out of the one prefetch buffer, which
          // then receives the next chunk's
          take_entry(hE[0]);
          issue_loads(hE[0]);
        }
        // The chunk body, instantiated for FULL (all K steps present, the
        // common case; straight-line code) or a guarded tail for a last chunk
        // shorter than K, and for the LDS slot SL that holds the chunk.
        auto chunk_body = [&](auto full_tag, auto slot_tag) {
          constexpr bool FULL = decltype(full_tag)::value;
          constexpr int SL = decltype(slot_tag)::value;
          if constexpr (ALT) {
            // the entry state, taken before this chunk issues its loads
            take_entry(hE[SL]);
            issue_loads(hE[1 - SL]);
          }
          // hb entering the chunk: from the step before (row 0 of the slot;
          // zero before the first step) or, for chunk 0 of a causal scan from
          // a given state, from beta0
          if (ch == 0) {
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
              const int n = j * S + s;
              hbp[j] = 0.f;
              if (!FAST && dir == 0 && p.h0 != nullptr && cvalid && n < p.N)
                hbp[j] = 0.5f * p.beta0[((int64_t)b * p.D + c) * p.N + n];
            }
          } else {
            const float hdp = sCh[SL][0][cl].y;
#pragma unroll
            for (int j = 0; j < NPL; ++j) hbp[j] = fmul(hdp, sB[SL][0][s * NPL + j]);
          }
          // recompute the chunk: s_{t-1}, g_t, e*sin and h_t for every step
          float SP[K][NPL], G[K][NPL], ES[K][NPL], HT[KEEP_HT ? K : 1][NPL];
#pragma unroll
          for (int m = 0; m < K; ++m) {
            if (FULL || m < kcnt) {
              const float dt = sCh[SL][m + 1][cl].x;
              const float hd = sCh[SL][m + 1][cl].y;
              // start every state's exponential and table read, then finish
              GatePartCS part[NPL];
#pragma unroll
              for (int j = 0; j < NPL; ++j)
                part[j] = gate_issue_cs<S, GK>(j, p.NR, has_imag, dt, gp.pah[j], gp.wh[j], sCS);
#pragma unroll
              for (int j = 0; j < NPL; ++j) {
                float es;
                const float g = gate_finish_cs<S, GK>(j, s, p.NR, has_imag, part[j], gp.pah[j], es);
                const float hb = fmul(hd, sB[SL][m + 1][s * NPL + j]);
                const float sm = hc[j] + hbp[j];
                SP[m][j] = sm;
                G[m][j] = g;
                ES[m][j] = es;
                hc[j] = ffma(g, sm, hb);
                if constexpr (KEEP_HT) HT[m][j] = hc[j];
                hbp[j] = hb;
              }
            }
          }
          // EARLY_STAGE: the inputs of chunk ch-1 into the other slot here,
          // which no wave reads after the previous chunk's barrier (the loads
          // have had the recompute to arrive, and the LDS writes stay off the
          // barrier's path): 4 % faster at N 16-32; at 40 states and in the
          // two-barrier instantiations the chunk's end measured 0.5 % faster
          if (EARLY_STAGE && ch >= 1) stage_store(std::integral_constant<int, 1 - SL>{});
          // adjoint over the chunk, last step first.  Parameter gradients
          // sum into chunk-local fp32 accumulators, then into float64.
#pragma unroll
          for (int m = K - 1; m >= 0; --m) {
            if (FULL || m < kcnt) {
              const float4 chv = sCh[SL][m + 1][cl];
              const float dt = chv.x, hd = chv.y, dy = chv.w;
              float ddA = 0.f, ddB = 0.f, sBc = 0.f;
#pragma unroll
              for (int j = 0; j < NPL; ++j) {
                const float Bv = sB[SL][m + 1][s * NPL + j];
                const float Cv = sC[SL][m + 1][s * NPL + j];
                const float g = G[m][j];
                float ht;
                if constexpr (KEEP_HT)
                  ht = HT[m][j];
                else
                  ht = ffma(g, SP[m][j], fmul(hd, Bv));
                const float dyc = fmul(dy, Cv);
                const float q = ffma(gn[j], qn[j], dyc);
                float dhb = ffma(2.f, q, -dyc);
                if constexpr (!FAST) {
                  if (fin) dhb = q + gr[j];
                }
                sBc = ffma(dhb, Bv, sBc);
                const float dg = fmul(q, SP[m][j]);
                if (j >= GK::kTJ) {  // tracking in every lane
                  cpa[j] = cpa[j] + dg;
                } else {
                  // rotational (for a slot decided at run time, a tracking
                  // lane has pam = wh = es = 0 and sums dg into cpt)
                  const float t1 = fmul(dg, g);
                  const float t2 = fmul(dg, ES[m][j]);
                  cpa[j] = ffma(t1, dt, cpa[j]);
                  cpb[j] = ffma(t2, dt, cpb[j]);
                  if (j >= GK::kRJ) cpt[j] = cpt[j] + dg;
                  ddA = ffma(j < GK::kRJ ? gp.pah[j] : pam[j], t1, ddA);  // Ar log2(e) dg g
                  ddB = ffma(gp.wh[j], t2, ddB);                          // Ai 256/(2 pi) dg e sin
                }
                qn[j] = q;
                gn[j] = g;
                // every lane of the row holds the row's total for its slice
                // s, so the lanes sharing s store the same value
                sRed[ONEBAR ? SL : 0][m % KR][0][s * NPL + j][wrow] = reduce_row<S>(fmul(dhb, hd));
                sRed[ONEBAR ? SL : 0][m % KR][1][s * NPL + j][wrow] = reduce_row<S>(fmul(dy, ht));
              }
              // d(gate)/d(dt) and sBc summed over the lane's states; their
              // sums over the channel's lanes are taken from sDD at the
              // chunk's end
              sDD[ONEBAR ? SL : 0][m][s][cl] = make_float2(ffma(kLn2, ddA, -fmul(kRadPerStep, ddB)), sBc);
              if constexpr (!FAST) fin = false;
            }
            if (m % KR == 0) {
              // dt and (dt*u)/2 of each (d_delta, d_u) element this thread
              // writes, read while the slot is still this chunk's (with
              // ONEBAR, another wave may restage it after the barrier)
              float fdt[DPT], fuh[DPT], fsp[DPT];
              if (m == 0) {
#pragma unroll
                for (int k = 0; k < DPT; ++k) {
                  const int e = tid + k * kThreads;
                  const int ee = e < K * CB ? e : 0;
                  const float4 v = sCh[SL][ee / CB + 1][ee % CB];
                  fdt[k] = v.x;
                  fuh[k] = v.z;
                }
              }
              // with softplus, the factor -expm1(-delta) of each d_delta
              // element; the empty volatile statement keeps this a branch
              // (executed for every launch if the compiler selected it)
              if (m == 0 && p.dsp && dd_final(dir)) {
                asm volatile("");
#pragma unroll
                for (int k = 0; k < DPT; ++k) fsp[k] = -expm1f(-fdt[k]);
              }
              // the inputs of chunk ch-1 into the other slot (EARLY_STAGE: above)
              if (!EARLY_STAGE && m == 0 && ch >= 1) stage_store(std::integral_constant<int, 1 - SL>{});
              // fold the 16 row partials of steps [m, m + KR) into this
              // tile's global dB / dC partials
              __syncthreads();
              // The reverse direction's prior values, waited for here (their
              // loads were issued at the chunk's start).  Stores count with
              // the loads in the same in-order counter, so a wait placed at a
              // later first use would also wait for the stores issued before
              // it, one memory round trip per store.
              // Likewise the next chunk's entry state: the loop's register
              // copies at its back edge would otherwise wait for these stores.
              if (m == 0) {
#pragma unroll
                for (int f = 0; f < NFOLD; ++f)
#pragma unroll
                  for (int k = 0; k < FPT; ++k) asm volatile("" : "+v"(prev[f][k]));
#pragma unroll
                for (int k = 0; k < DPT; ++k) asm volatile("" : "+v"(pdd[k][0]), "+v"(pdd[k][1]));
#pragma unroll
                for (int a = 0; a < (ALT ? 2 : 1); ++a)
#pragma unroll
                  for (int j = 0; j < NPL; ++j) asm volatile("" : "+v"(hE[a][j]));
              }
#pragma unroll
              for (int k = 0; k < FPT; ++k) {
                if constexpr (FAST) {
                  if (fInfo[k] >= 0 && (FULL || m + (fInfo[k] & 7) < kcnt)) {
                    const float4* rp =
                        reinterpret_cast<const float4*>(&sRed[ONEBAR ? SL : 0][0][0][0][0] + (fInfo[k] >> 3));
                    const float4 a0 = rp[0], a1 = rp[1], a2 = rp[2], a3 = rp[3];
                    const float v = (((a0.x + a0.y) + (a0.z + a0.w)) + ((a1.x + a1.y) + (a1.z + a1.w))) +
                                    (((a2.x + a2.y) + (a2.z + a2.w)) + ((a3.x + a3.y) + (a3.z + a3.w)));
                    store_byte<float>(pbc, oF[m / KR][k] + (uint32_t)ch * stF,
                                      add_bc ? prev[m / KR][k] + v : v);
                  }
                  continue;
                }
                const int e = tid + k * kThreads;
                float* dst = fold_dst(e, b, dir, i0, m, kcnt);
                if (dst != nullptr) {
                  const int rem = e % (2 * p.N);
                  const int which = rem / p.N, n = rem % p.N;
                  const int kk = (n % S) * NPL + n / S;
                  const float4* rp = reinterpret_cast<const float4*>(&sRed[0][e / (2 * p.N)][which][kk][0]);
                  const float4 a0 = rp[0], a1 = rp[1], a2 = rp[2], a3 = rp[3];
                  const float v = (((a0.x + a0.y) + (a0.z + a0.w)) + ((a1.x + a1.y) + (a1.z + a1.w))) +
                                  (((a2.x + a2.y) + (a2.z + a2.w)) + ((a3.x + a3.y) + (a3.z + a3.w)));
                  *dst = add_bc ? prev[m / KR][k] + v : v;
                }
              }
              if (m == 0) {
                // the chunk's (d_delta, d_u), channel-contiguous
#pragma unroll
                for (int k = 0; k < DPT; ++k) {
                  const int e = tid + k * kThreads;
                  if constexpr (FAST) {
                    if (e < K * CB && (FULL || e / CB < kcnt)) {
                      const uint32_t o = oD[k] + (uint32_t)ch * stDY;
                      const float2 v = dd_of(ONEBAR ? SL : 0, e / CB, e % CB, fdt[k], fuh[k]);
                      float dd = dir == 0 ? v.x : pdd[k][0] + v.x;
                      if (p.dsp && dd_final(dir)) dd = fmul(dd, fsp[k]);
                      const float du = dir == 0 ? v.y : pdd[k][1] + v.y;
                      if (dd_final(dir)) {
                        store_grad(io.d_delta, o, dd, io.dt_dd);
                        store_grad(io.d_u, o, du, io.dt_du);
                      } else {
                        store_byte<float>(io.pd_delta, o, dd);
                        store_byte<float>(io.pd_u, o, du);
                      }
                    }
                    continue;
                  }
                  const int64_t idx = dd_index(e, b, dir, i0, kcnt);
                  if (idx >= 0) {
                    const float2 v = dd_of(0, e / CB, e % CB, fdt[k], fuh[k]);
                    float dd = dir == 0 ? v.x : pdd[k][0] + v.x;
                    // with softplus, the complete gradient is taken through it
                    if (p.dsp && dd_final(dir)) dd = fmul(dd, fsp[k]);
                    const float du = dir == 0 ? v.y : pdd[k][1] + v.y;
                    if (dd_final(dir)) {
                      store_grad_at(io.d_delta, idx, dd, io.dt_dd);
                      store_grad_at(io.d_u, idx, du, io.dt_du);
                    } else {
                      io.pd_delta[idx] = dd;
                      io.pd_u[idx] = du;
                    }
                  }
                }
              }
              if constexpr (!ONEBAR) __syncthreads();
            }
          }
          if (ch % kParChunks == 0) {
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
              const float a = (j >= GK::kRJ && j < GK::kTJ && !is_rot<S, GK>(j, s, p.NR)) ? cpt[j]
                                                                                          : cpa[j];
              if constexpr (PAR_GLOBAL) {
                // float64 atomic adds whose result is not used: nothing waits
                // on a load.  Only this thread updates these entries, and its
                // accesses to one address execute in program order, so the
                // sums are the same, in the same order, as a load-add-store
                // (bitwise-identical results; the reduction kernel reads them
                // after this kernel ends).
                if (cvalid && j * S + s < p.N) {
                  unsafeAtomicAdd(&io.part_par[par_at(j)], (double)a);
                  if (j < GK::kTJ)
                    unsafeAtomicAdd(&io.part_par[par_at(j) + (int64_t)p.D * p.N], (double)cpb[j]);
                }
              } else {
                sPar[0][j][tid] += (double)a;
                if (j < GK::kTJ) sPar[1][j][tid] += (double)cpb[j];
              }
              cpa[j] = 0.f;
              cpb[j] = 0.f;
              cpt[j] = 0.f;
            }
          }
        };
        chunk_body(full_arg, slot_arg);
      };
      // The chunk walk.  FAST: unrolled by the two slots, so that every
      // prefetch buffer keeps one register assignment around the loop (a
      // join of the two slot bodies at the back edge needs register copies,
      // and a copy's wait for a loaded value also waits for the stores issued
      // before it).  Only the walk's first chunk can be shorter than K.  The
      // general instantiation keeps one body per iteration (compile time).
      if constexpr (!FAST) {
        for (int ch = nct - 1; ch >= 0; --ch) {
          const bool full = L - ch * K >= K;
          if (full && ch % 2 == 0)
            one_chunk(ch, std::true_type{}, Slot0{});
          else if (full)
            one_chunk(ch, std::true_type{}, Slot1{});
          else if (ch % 2 == 0)
            one_chunk(ch, std::false_type{}, Slot0{});
          else
            one_chunk(ch, std::false_type{}, Slot1{});
        }
      } else {
        int ch = nct - 1;
        if (ch >= 0 && L - ch * K < K) {
          if (ch % 2 == 0)
            one_chunk(ch, std::false_type{}, Slot0{});
          else
            one_chunk(ch, std::false_type{}, Slot1{});
          --ch;
        }
        if (ch >= 0 && ch % 2 == 0) {
          one_chunk(ch, std::true_type{}, Slot0{});
          --ch;
        }
        for (; ch >= 1; ch -= 2) {
          one_chunk(ch, std::true_type{}, Slot1{});
          one_chunk(ch - 1, std::true_type{}, Slot0{});
        }
      }
      // after the sweep (qn, gn) = (q_0, g_0), and g_0 q_0 is the gradient of
      // the initial state, since h_0 = g_0 (h0 + beta0/2) + hb_0
      if (!FAST && dir == 0 && io.d_h0 != nullptr && cvalid) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          const int n = j * S + s;
          if (n < p.N) {
            const int64_t idx = ((int64_t)b * p.D + c) * p.N + n;
            const float gq = fmul(gn[j], qn[j]);
            io.d_h0[idx] = gq;
            io.d_beta0[idx] = 0.5f * gq;
          }
        }
      }
    }
  }
  // per-batch-group parameter-gradient partials (float64)
  if constexpr (!PAR_GLOBAL) {
    if (cvalid) {
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const int n = j * S + s;
        if (n < p.N) {
          const int64_t base = ((int64_t)bgi * 2) * p.D * p.N;
          io.part_par[base + (int64_t)c * p.N + n] = sPar[0][j][tid];
          io.part_par[base + (int64_t)p.D * p.N + (int64_t)c * p.N + n] = sPar[1][j][tid];
        }
      }
    }
  }
}

// The backward kernel: workgroup = tile group x batch group.  MULTI: it
// walks the group's io.tpw adjacent channel tiles in turn (fewer dB / dC
// partials to write and reduce where tiles are narrow: 16 channels at 16
// lanes); otherwise one tile (io.tpw == 1), without the loop, whose
// hoisting would cost registers.
template <int S, int NPL, class GK, bool FAST, bool MULTI>
__global__ __launch_bounds__(kThreads, NPL <= 5 ? 2 : 1) void scan_bwd_kernel(ScanParams p, BwdIO io) {
  const int tgrp = blockIdx.x % io.ntg, bgi = blockIdx.x / io.ntg;
  if constexpr (MULTI) {
    for (int tp = 0; tp < io.tpw; ++tp) {
      const int tile = tgrp * io.tpw + tp;
      if (tile >= p.ntiles) break;
      scan_bwd_tile<S, NPL, GK, FAST, true>(p, io, tile, tp, tgrp, bgi);
    }
  } else {
    scan_bwd_tile<S, NPL, GK, FAST, false>(p, io, tgrp, 0, tgrp, bgi);
  }
}

// The whole-tile (FAST) launches, instantiated in scan_bwd_fast.hip.
hipError_t launch_scan_bwd_fast(int S, int NPL, int gk, const ScanParams& p, const BwdIO& io,
                                hipStream_t st);
// The tile-walking (MULTI) launches of the 16-lane shapes, whole-tile or
// general, instantiated in scan_bwd_walk.hip.
hipError_t launch_scan_bwd_walk(int S, int NPL, int gk, bool fast, const ScanParams& p,
                                const BwdIO& io, hipStream_t st);

}  // namespace rp
