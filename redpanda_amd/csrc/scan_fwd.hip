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

// Steps staged per block: fewer for large states, whose B / C rows dominate
// the LDS (occupancy).
template <int S, int NPL>
constexpr int fwd_tb() { return S * NPL > 40 ? kFwdTB / 2 : kFwdTB; }

// Workgroups per CU that the kernel's LDS allows (160 KB per CU), at most 7:
// the register budget the compiler is held to, so that VGPRs do not limit
// the occupancy below what the LDS gives (7 leaves the recurrence of every
// shape its registers).
template <int S, int NPL, int REC = 8>
constexpr int fwd_occupancy_rec() {
  constexpr int TB = fwd_tb<S, NPL>(), CB = kWaves * (kWave / S), NP = S * NPL;
  constexpr int lds = TB * CB * 12 + 2 * TB * NP * 4 + kTab * REC;
  return 163840 / lds < 7 ? 163840 / lds : 7;
}
// The gate table's records carry their two expansion coefficients (16
// bytes: two VALU operations fewer per rotational state-step) where that
// leaves the occupancy as it is with 8-byte records.
template <int S, int NPL>
constexpr bool fwd_wide_rec() {
  return fwd_occupancy_rec<S, NPL, 16>() == fwd_occupancy_rec<S, NPL, 8>();
}
template <int S, int NPL>
constexpr int fwd_occupancy() {
  return fwd_occupancy_rec<S, NPL, fwd_wide_rec<S, NPL>() ? 16 : 8>();
}

// MODEL: the instantiation for the model's launches, whose full blocks take
// the fast staging with delta as the dt projection x (the scan uses
// softplus(x), kept in the delta cache by the first direction and read back
// by the second), delta and u in bf16 or fp16 (autocast) and B, C in fp32
// (the fused BCNorm's output).  A separate instantiation: the other kernel's
// fast staging keeps its registers.
template <int S, int NPL, class GK, bool MODEL>
__global__ __launch_bounds__(kThreads, (fwd_occupancy<S, NPL>())) void scan_fwd_kernel(ScanParams p,
                                                                                          FwdOut o) {
  using Sh = Shape<S, NPL>;
  constexpr int DT = Sh::kDT, CB = Sh::kCB, NP = Sh::kNP, TB = fwd_tb<S, NPL>();
  __shared__ float2 sDH[TB][CB];   // (dt, (dt*u)/2) per step and channel
  __shared__ float sB[TB][NP];     // per step, layout [s*NPL + j] -> state j*S + s
  __shared__ float sC[TB][NP];
  __shared__ float sY[TB][CB];     // the block's y, written out channel-contiguous
  // (m, b (-sin a)) records of the gate table, with their coefficients when wide
  __shared__ std::conditional_t<fwd_wide_rec<S, NPL>(), float4, float2> sCos[kTab];

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
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // wave index, scalar
  // Full blocks (all TB steps, every channel of the tile present) whose four
  // streamed inputs share one storage type take the fast staging: rows are
  // wave-uniform, so an address is a scalar row base plus the lane's fixed
  // 32-bit offset, and each part issues all its loads before converting any.
  // Channel rows: a wave instruction covers RW rows of CW channels (lane =
  // rh * CW + ci0), NHC instructions per row, QC passes per wave.
  constexpr int CW = CB < kWave ? CB : kWave, RW = kWave / CW, NHC = CB / CW;
  constexpr int QC = TB / (kWaves * RW);
  static_assert(QC * kWaves * RW == TB, "a block is whole passes of channel rows");
  // State rows: one row per wave instruction, lane = LDS column kk (NH
  // instructions per row), QB rows per wave.
  constexpr int NH = (NP + kWave - 1) / kWave, QB = TB / kWaves;
  static_assert(QB * kWaves == TB, "a block is whole passes of state rows");
  const bool tile_full = (tile + 1) * CB <= p.D;
  const bool one_type = p.dt_delta == p.dt_u && p.dt_u == p.dt_B && p.dt_B == p.dt_C;
  constexpr int64_t kOffMax = 1ll << 29;  // lane offsets stay 32-bit byte offsets
  const bool offs_fit = (int64_t)RW * (p.dsl + p.usl + p.D) + CB < kOffMax && p.N < kOffMax;
  // The lane's place in the fast paths' row layouts, recomputed from an opaque
  // copy of the lane index at every use: otherwise the compiler keeps the
  // derived per-lane addresses live through the recurrence (registers).
  auto lane_fresh = [&]() {
    int l = lane;
    asm volatile("" : "+v"(l));
    return l;
  };
  // Likewise the batch row and tile as scalars: the 64-bit row bases derived
  // from them are recomputed per block instead of held in scalar registers.
  auto row_tile_fresh = [&](int& bo, int& to) {
    bo = b;
    to = tile;
    asm volatile("" : "+s"(bo), "+s"(to));
  };
  for (int dir = 0; dir < p.ndir; ++dir) {
    // the state h and the previous step's hb (the initial state h0, beta0 / 2)
    float h[NPL], hb[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int n = j * S + s;
      h[j] = 0.f;
      hb[j] = 0.f;
      if (dir == 0 && p.h0 != nullptr && cvalid && n < p.N) {
        const int64_t idx = ((int64_t)b * p.D + c) * p.N + n;
        h[j] = p.h0[idx];
        hb[j] = 0.5f * p.beta0[idx];
      }
    }
    // the lane's channel-row slot (rh, ci0), its row within a pass in time
    // order, and its offsets into delta, u and the (B, L, D) arrays (y, the
    // delta cache)
    struct ChanLane {
      int rh, ci0;
      uint32_t od, ou, oy;
    };
    auto chan_lane = [&]() {
      const int l = lane_fresh();
      ChanLane cl;
      cl.rh = l / CW;
      cl.ci0 = l % CW;
      const int rl = dir ? RW - 1 - cl.rh : cl.rh;
      cl.od = rl * (uint32_t)p.dsl + cl.ci0;
      cl.ou = rl * (uint32_t)p.usl + cl.ci0;
      cl.oy = rl * (uint32_t)p.D + cl.ci0;
      return cl;
    };
    // earliest time of the RW channel rows from block row rb
    auto pass_t = [&](int i0, int rb) { return dir ? L - i0 - rb - RW : i0 + rb; };
    // y of the block starting at step i0 (cnt steps) from sY: coalesced, and
    // the reverse direction adds to what the forward direction stored
    auto write_y = [&](int i0, int cnt) {
      if (cnt == TB && tile_full && offs_fit) {
        const ChanLane ln = chan_lane();
        const int rh = ln.rh, ci0 = ln.ci0;
        const uint32_t oy = ln.oy;
        int bo, to;
        row_tile_fresh(bo, to);
        float prev[QC][NHC];
        if (dir == 1) {
#pragma unroll
          for (int q = 0; q < QC; ++q)
#pragma unroll
            for (int h = 0; h < NHC; ++h)
              prev[q][h] = load_at<float>(
                  o.y + ((int64_t)bo * L + pass_t(i0, (wv + kWaves * q) * RW)) * p.D + to * CB + h * CW, oy);
        }
#pragma unroll
        for (int q = 0; q < QC; ++q) {
          const int rb = (wv + kWaves * q) * RW;
#pragma unroll
          for (int h = 0; h < NHC; ++h) {
            const float v = sY[rb + rh][h * CW + ci0];
            store_at(o.y + ((int64_t)bo * L + pass_t(i0, rb)) * p.D + to * CB + h * CW, oy,
                     dir == 0 ? v : prev[q][h] + v);
          }
        }
        return;
      }
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
    // fast staging of a full block: ITC the storage code of delta and u, ITS
    // that of B and C; DSP: delta holds x and the scan uses softplus(x),
    // cached in o.dcache (when given) by the first direction and read back
    // by the second (the generic staging's order of operations).  Row bases
    // advance by a signed stride per pass (passes are kWaves * RW channel
    // rows or kWaves state rows apart in the block).
    auto stage_fast = [&](auto itc_tag, auto its_tag, auto dsp_tag, int i0) {
      constexpr int ITC = decltype(itc_tag)::value, ITS = decltype(its_tag)::value;
      constexpr bool DSP = decltype(dsp_tag)::value;
      using Raw = RawOf<ITC>;
      using RawS = RawOf<ITS>;
      const ChanLane ln = chan_lane();
      const int rh = ln.rh, ci0 = ln.ci0;
      const uint32_t od = ln.od, ou = ln.ou, oy = ln.oy;
      int bo, to;
      row_tile_fresh(bo, to);
      const int dtq = dir ? -kWaves * RW : kWaves * RW;  // time step between passes
      const int64_t tq0 = pass_t(i0, wv * RW);
      const Raw* drow = static_cast<const Raw*>(p.delta) + (int64_t)bo * p.dsb + tq0 * p.dsl + to * CB;
      const Raw* urow = static_cast<const Raw*>(p.u) + (int64_t)bo * p.usb + tq0 * p.usl + to * CB;
      // the delta cache's rows (y's layout); with DSP, the second direction
      // reads softplus(x) from it
      float* crow = DSP && o.dcache != nullptr ? o.dcache + ((int64_t)bo * L + tq0) * p.D + to * CB
                                               : nullptr;
      const bool from_cache = DSP && dir == 1 && crow != nullptr;
      const int64_t dstep = dtq * p.dsl, ustep = dtq * p.usl, cstep = (int64_t)dtq * p.D;
      __builtin_amdgcn_sched_barrier(0);
      // delta as stored, or (DSP) the cached fp32 bits
      typename std::conditional<DSP, uint32_t, Raw>::type rd[QC][NHC];
      Raw ru[QC][NHC];
      if (from_cache) {
        const float* cr = crow;
#pragma unroll
        for (int q = 0; q < QC; ++q) {
#pragma unroll
          for (int h = 0; h < NHC; ++h) {
            rd[q][h] = load_at<uint32_t>(cr + h * CW, oy);
            ru[q][h] = load_at<Raw>(urow + h * CW, ou);
          }
          cr += cstep;
          urow += ustep;
        }
      } else {
#pragma unroll
        for (int q = 0; q < QC; ++q) {
#pragma unroll
          for (int h = 0; h < NHC; ++h) {
            rd[q][h] = load_at<Raw>(drow + h * CW, od);
            ru[q][h] = load_at<Raw>(urow + h * CW, ou);
          }
          drow += dstep;
          urow += ustep;
        }
      }
#pragma unroll
      for (int q = 0; q < QC; ++q) {
        const int rb = (wv + kWaves * q) * RW;
#pragma unroll
        for (int h = 0; h < NHC; ++h) {
          float dt;
          if constexpr (DSP) {
            if (from_cache) {
              dt = __uint_as_float(rd[q][h]);
            } else {
              dt = softplus_of(cvt_raw(rd[q][h], ITC));
              if (crow != nullptr) store_at(crow + q * cstep + h * CW, oy, dt);
            }
          } else {
            dt = cvt_raw(rd[q][h], ITC);
          }
          sDH[rb + rh][h * CW + ci0] = make_float2(dt, 0.5f * fmul(dt, cvt_raw(ru[q][h], ITC)));
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // the state of each of the lane's LDS columns, clamped into the row for
      // the load; columns past NP and pad states stage zeros
      const int l = lane_fresh();
      uint32_t nld[NH];
      bool nval[NH];
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const int kk = l + h * kWave;
        const int n = kk < NP ? (kk % NPL) * S + kk / NPL : 0;
        nld[h] = (uint32_t)min(n, p.N - 1);
        nval[h] = kk < NP && n < p.N;
      }
      const int dts = dir ? -kWaves : kWaves;  // time step between state rows of a wave
      const int64_t ts0 = dir ? L - 1 - i0 - wv : i0 + wv;
      const RawS* brow = static_cast<const RawS*>(p.Bc) + (int64_t)bo * p.bsb + ts0 * p.bsl;
      const RawS* cbrow = static_cast<const RawS*>(p.Cc) + (int64_t)bo * p.csb + ts0 * p.csl;
      const int64_t bstep = dts * p.bsl, cbstep = dts * p.csl;
      // in groups of QG state rows: at most 2 * QG * NH loads in flight, so
      // the staging stays within the register budget of the recurrence
      constexpr int QG = QB < 4 ? QB : 4;
      static_assert(QB % QG == 0, "whole groups of state rows");
#pragma unroll
      for (int q0 = 0; q0 < QB; q0 += QG) {
        __builtin_amdgcn_sched_barrier(0);
        RawS rbv[QG][NH], rcv[QG][NH];
#pragma unroll
        for (int q = 0; q < QG; ++q) {
#pragma unroll
          for (int h = 0; h < NH; ++h) {
            rbv[q][h] = load_at<RawS>(brow, nld[h]);
            rcv[q][h] = load_at<RawS>(cbrow, nld[h]);
          }
          brow += bstep;
          cbrow += cbstep;
        }
#pragma unroll
        for (int q = 0; q < QG; ++q) {
          const int r = wv + kWaves * (q0 + q);
#pragma unroll
          for (int h = 0; h < NH; ++h) {
            const int kk = l + h * kWave;
            if (NH * kWave == NP || kk < NP) {
              sB[r][kk] = nval[h] ? cvt_raw(rbv[q][h], ITS) : 0.f;
              sC[r][kk] = nval[h] ? cvt_raw(rcv[q][h], ITS) : 0.f;
            }
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int bi = 0; bi < nblk; ++bi) {
      const int i0 = bi * TB;
      const int cnt = min(TB, L - i0);
      __syncthreads();
      if (bi > 0) write_y(i0 - TB, TB);
      using BF16 = std::integral_constant<int, RP_BF16>;
      using F32 = std::integral_constant<int, RP_F32>;
      using F16 = std::integral_constant<int, RP_F16>;
      if (MODEL && cnt == TB && tile_full && offs_fit) {
        // (the host launches MODEL only for its storage types, with softplus)
        if (p.dt_u == RP_BF16)
          stage_fast(BF16{}, F32{}, std::true_type{}, i0);
        else
          stage_fast(F16{}, F32{}, std::true_type{}, i0);
      } else if (!MODEL && cnt == TB && tile_full && one_type && offs_fit && !p.dsp &&
                 o.dcache == nullptr) {
        if (p.dt_B == RP_BF16)
          stage_fast(BF16{}, BF16{}, std::false_type{}, i0);
        else if (p.dt_B == RP_F32)
          stage_fast(F32{}, F32{}, std::false_type{}, i0);
        else
          stage_fast(F16{}, F16{}, std::false_type{}, i0);
      } else {
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
      }
      __syncthreads();
      // one step of the block (row r); i0 is a multiple of kCkptK, so the
      // checkpoint steps are the rows r with (r + 1) % kCkptK == 0
      auto step = [&](int r) {
        const int i = i0 + r;
        const float2 dh = sDH[r][cl];
        float y = fwd_update<S, NPL, GK>(h, hb, gp, sCos, dh.x, dh.y, &sB[r][s * NPL],
                                         &sC[r][s * NPL], s, p.NR, has_imag);
        // the channel's S lanes hold the same total and store the same value
        sY[r][cl] = reduce_states<S>(y);
        if (o.ckpt != nullptr && ((r + 1) % kCkptK) == 0 && i + 1 < L) {
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
      };
      static_assert(TB % kCkptK == 0, "blocks start on checkpoint boundaries");
      if (cnt == TB) {
        // a full block in groups of kCkptK steps: LDS offsets and the
        // checkpoint test are compile-time within a group
        for (int r0 = 0; r0 < TB; r0 += kCkptK) {
#pragma unroll
          for (int k = 0; k < kCkptK; ++k) step(r0 + k);
        }
      } else {
        for (int r = 0; r < cnt; ++r) step(r);
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
  // the model's launches: softplus, delta and u in bf16 or fp16, B and C in fp32
  const bool model = p.dsp && p.dt_delta == p.dt_u && (p.dt_u == RP_BF16 || p.dt_u == RP_F16) &&
                     p.dt_B == RP_F32 && p.dt_C == RP_F32;
  if (model)
    hipLaunchKernelGGL((scan_fwd_kernel<S, NPL, GK, true>), grid, dim3(kThreads), 0, st, p, o);
  else
    hipLaunchKernelGGL((scan_fwd_kernel<S, NPL, GK, false>), grid, dim3(kThreads), 0, st, p, o);
  return hipGetLastError();
}

hipError_t launch_scan_fwd(int S, int NPL, int gk, const ScanParams& p, const FwdOut& o,
                           hipStream_t st) {
#define RP_CASE(SS, NN)                                                              \
  if (S == SS && NN == NPL)                                                          \
    return with_gate_kind_scan<SS, NN>(gk, [&](auto g) {                                      \
      return launch_fwd_t<SS, NN, decltype(g)>(p, o, st);                            \
    });
  RP_FOR_EACH_SHAPE(RP_CASE)
#undef RP_CASE
  return hipErrorInvalidValue;
}

}  // namespace rp
