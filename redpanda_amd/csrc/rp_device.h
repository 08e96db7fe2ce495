// Device-side building blocks shared by the scan, backward and step kernels.
//
// Lane layout (all kernels).  A wave64 owns DT = 64/S channels; S adjacent
// lanes share one channel and split its N states between them:
//     lane = dl * S + s,   channel = tile*CB + wave*DT + dl,
//     lane (dl, s) holds states n = j*S + s for j in [0, NPL).
// A workgroup is 4 waves (256 threads) and covers CB = 4*DT channels.
// Interleaving the states this way keeps the rotational / tracking split
// (n < NR vs n >= NR) uniform across the wave for every j but at most one,
// so gate selection is a scalar branch.  The sum over a channel's states is
// an in-lane FMA chain over j followed by a DPP butterfly over the S lanes;
// the step kernel uses the very same functions, so step == scan bit for bit.
//
// Gate arithmetic (rot_gate below).  exp uses the transcendental unit
// (v_exp_f32 is good to 0.8 ulp and unbiased); cos / sin do not: measured on
// gfx950, v_cos_f32 / v_sin_f32 are off by up to ~2 ulp with a bias of
// +-0.3..0.6 ulp that depends on the angle (-0.6 ulp near cos = 1).  A gate
// close to 1 carries state over tens of steps, so a biased gate turns into a
// relative drift of the state of ~(steps x bias) and a visible error in the
// gradients that sum over steps.  The rotational gate is therefore
// evaluated to ~1 ulp without systematic bias:
//     exp(dt*Ar)  = 2^(dt (pah + pal)), pah + pal = Ar log2(e) to 2^-48;
//     cos / sin   of the angle in 1/16 revolutions w = dt (wh + wl), where
//                   wh + wl = 16 Ai / (2 pi) to 2^-48, reduced exactly to a
//                   16-entry table and |x| <= pi/16, where short Taylor
//                   polynomials are accurate to < 1e-9.
// The forward, the step and the backward's recompute share the code, so the
// backward recomputes exactly the gates the forward used.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "redpanda_hip.h"
#include "rp_launch.h"

namespace rp {

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kTwoPi = 6.28318530717958647692f;
constexpr double kInv2PiD = 0.15915494309189533577;

template <int S, int NPL>
struct Shape {
  static constexpr int kS = S;
  static constexpr int kNPL = NPL;
  static constexpr int kDT = kWave / S;        // channels per wave
  static constexpr int kCB = kWaves * kDT;     // channels per workgroup
  static constexpr int kNP = S * NPL;          // padded states per channel
  static_assert(S == 2 || S == 4 || S == 8 || S == 16, "S must be a power of two <= 16");
};

// Streamed-input load with on-the-fly conversion to fp32 (uniform dtype).
__device__ __forceinline__ float load_in(const void* p, int64_t i, int dtype) {
  if (dtype == RP_F32) return static_cast<const float*>(p)[i];
  if (dtype == RP_BF16) {
    const uint32_t bits = static_cast<const uint16_t*>(p)[i];
    return __uint_as_float(bits << 16);
  }
  return static_cast<float>(static_cast<const _Float16*>(p)[i]);
}

__device__ __forceinline__ float fmul(float a, float b) { return a * b; }
__device__ __forceinline__ float ffma(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// exp2 on the transcendental unit (v_exp_f32).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// cos / sin of 2 pi k / 16, k = 0..15 (filled into LDS once per workgroup).
__device__ __forceinline__ void sincos_table_entry(int k, float& c, float& s) {
  constexpr float kC1 = 0.923879532511286756f, kC2 = 0.707106781186547524f,
                  kC3 = 0.382683432365089772f;
  const float cq[4] = {1.f, kC1, kC2, kC3};  // cos of 0, 1/16, 2/16, 3/16 rev
  const int q = (k >> 2) & 3, r = k & 3;
  const float c0 = cq[r];
  const float s0 = (r == 0) ? 0.f : cq[(4 - r) & 3];
  c = (q == 0) ? c0 : (q == 1) ? -s0 : (q == 2) ? -c0 : s0;
  s = (q == 0) ? s0 : (q == 1) ? c0 : (q == 2) ? -s0 : -c0;
}

__device__ __forceinline__ void fill_sincos_table(float2* tab, int tid) {
  if (tid < 16) {
    float c, s;
    sincos_table_entry(tid, c, s);
    tab[tid] = make_float2(c, s);
  }
}

// Per-state gate parameters held in registers.  Rotational states:
//   pah + pal = A_real * log2(e)      (fp32 pair, |pal| <= ulp(pah)/2)
//   wh  + wl  = 16 A_imag / (2 pi)    (the angle in 1/16 revolutions),
//   wlr = wl * pi / 8                 (the low part in radians)
// so the per-step products dt*pah and dt*wh round once per step, at random,
// as the reference's fl(dt*A) does, and no constant per-state rounding of
// log2(e) or 1/(2 pi) biases a gate over time.  Tracking states carry
// pah = tanh(theta); pad states carry zeros.
__device__ __forceinline__ void load_gate_params(const float* Ar, const float* Ai, const float* Tk,
                                                 int c, int n, int N, int NR, int NT, bool valid,
                                                 float& pah, float& pal, float& wh, float& wlr) {
  pah = 0.f;
  pal = 0.f;
  wh = 0.f;
  wlr = 0.f;
  if (!valid) return;
  if (n < NR) {
    const double P = (double)Ar[(int64_t)c * NR + n] * 1.4426950408889634074;
    pah = (float)P;
    pal = (float)(P - (double)pah);
    if (Ai != nullptr) {
      const double W = (double)Ai[(int64_t)c * NR + n] * (16.0 * kInv2PiD);
      wh = (float)W;
      wlr = (float)((W - (double)wh) * 0.39269908169872415481);  // * pi / 8
    }
  } else if (n < N) {
    pah = Tk[(int64_t)c * NT + (n - NR)];
  }
}

constexpr float kPi8 = 0.39269908169872415481f;  // pi / 8: radians per table step
constexpr float kRint = 12582912.f;               // 1.5 * 2^23: x + kRint rounds x to an integer

// Rotational gate g = 2^(dt (pah + pal)) cos(pi/8 dt (wh + wl)); with WITH_SIN
// also es = 2^(...) sin(...) for the backward.  The angle is reduced exactly
// to k + rr (k an integer, |rr| <= 1/2, in 1/16 revolutions) by the
// round-to-integer addition; cos / sin of the 16 table angles come from LDS
// and those of the remainder (|x| <= pi/16) from Taylor polynomials whose
// truncation error is below 1e-9.  The cos path is the same code in both
// instantiations, so g is bitwise the same.
template <bool WITH_SIN>
__device__ __forceinline__ float rot_gate(float dt, float pah, float pal, float wh, float wlr,
                                          bool has_imag, const float2* tab, float& es) {
  const float e = exp2_hw(ffma(dt, pal, fmul(dt, pah)));
  if (!has_imag) {
    es = 0.f;
    return e;
  }
  const float w = fmul(dt, wh);
  const float t = w + kRint;
  const float kf = t - kRint;                    // rint(w), exact
  const float rr = w - kf;                       // exact
  const float xr = ffma(rr, kPi8, fmul(dt, wlr));
  const float x2 = fmul(xr, xr);
  const float cm1 = fmul(x2, ffma(x2, ffma(x2, -1.f / 720.f, 1.f / 24.f), -0.5f));  // cos - 1
  const float sx = ffma(fmul(xr, x2), ffma(x2, 1.f / 120.f, -1.f / 6.f), xr);        // sin
  const float2 cs = tab[__float_as_int(t) & 15];
  const float cv = ffma(-cs.y, sx, ffma(cs.x, cm1, cs.x));
  if (WITH_SIN) {
    const float sv = ffma(cs.x, sx, ffma(cs.y, cm1, cs.y));
    es = fmul(e, sv);
  } else {
    es = 0.f;
  }
  return fmul(e, cv);
}

// Gate of state j for lane slice s: rotational if n < NR, else the tracking
// gate pah = tanh(theta) (pad states beyond N carry 0 and B = C = 0).
template <int S, bool WITH_SIN>
__device__ __forceinline__ float gate_of(int j, int s, int NR, bool has_imag, float dt, float pah,
                                         float pal, float wh, float wlr, const float2* tab,
                                         float& es) {
  if (j * S >= NR) {
    es = 0.f;
    return pah;
  }
  const float gr = rot_gate<WITH_SIN>(dt, pah, pal, wh, wlr, has_imag, tab, es);
  if ((j + 1) * S <= NR || j * S + s < NR) return gr;
  es = 0.f;
  return pah;
}

// Per-lane gate parameters of NPL states.
template <int NPL>
struct GateRegs {
  float pah[NPL], pal[NPL], wh[NPL], wlr[NPL];
};

template <int S, int NPL>
__device__ __forceinline__ void load_gate_regs(GateRegs<NPL>& gp, const float* Ar, const float* Ai,
                                               const float* Tk, int c, int s, int N, int NR,
                                               int NT, bool valid) {
#pragma unroll
  for (int j = 0; j < NPL; ++j)
    load_gate_params(Ar, Ai, Tk, c, j * S + s, N, NR, NT, valid, gp.pah[j], gp.pal[j], gp.wh[j],
                     gp.wlr[j]);
}

// One recurrence step for the lane's NPL states; returns the lane's partial
//     y = sum_j h_j C_j     (FMA chain in j order).
// hdu = (dt*u)/2, so hb = hdu*B_n equals beta_t/2 exactly; hbp holds the
// previous step's hb.  Shared verbatim by the scan and step kernels.
template <int S, int NPL>
__device__ __forceinline__ float fwd_update(float (&h)[NPL], float (&hbp)[NPL],
                                            const GateRegs<NPL>& gp, const float2* tab, float dt,
                                            float hdu, const float* __restrict__ Bs,
                                            const float* __restrict__ Cs, int s, int NR,
                                            bool has_imag) {
  float y = 0.f;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    float unused;
    const float g = gate_of<S, false>(j, s, NR, has_imag, dt, gp.pah[j], gp.pal[j], gp.wh[j],
                                      gp.wlr[j], tab, unused);
    const float hb = fmul(hdu, Bs[j]);
    const float sm = h[j] + hbp[j];
    h[j] = ffma(g, sm, hb);
    hbp[j] = hb;
    y = ffma(h[j], Cs[j], y);
  }
  return y;
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over the S adjacent lanes of one channel; every one of those lanes ends
// with the bitwise-identical total (each butterfly stage is commutative).
template <int S>
__device__ __forceinline__ float reduce_states(float v) {
  if (S >= 2) v = v + dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  if (S >= 4) v = v + dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  if (S >= 8) v = v + dpp<0x141>(v);  // row_half_mirror
  if (S >= 16) v = v + dpp<0x140>(v); // row_mirror
  return v;
}

// Sum over the channels of one 16-lane row that share slice s (lanes
// s, s+S, ... of the row), with DPP row rotations on the VALU.  Every lane
// of the row ends with the total of its slice; the order of the additions is
// fixed, so the result is deterministic.
template <int S>
__device__ __forceinline__ float reduce_row(float v) {
  static_assert(S == 2 || S == 4 || S == 8 || S == 16, "S must divide a 16-lane row");
  if (S <= 8) v = v + dpp<0x128>(v);  // row_ror:8
  if (S <= 4) v = v + dpp<0x124>(v);  // row_ror:4
  if (S <= 2) v = v + dpp<0x122>(v);  // row_ror:2
  return v;
}

}  // namespace rp
