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
// (v_exp_f32: 0.8 ulp, unbiased); cos / sin do not: measured on gfx950,
// v_cos_f32 / v_sin_f32 are off by up to ~2 ulp with a bias of +-0.3..0.6 ulp
// that depends on the angle (-0.6 ulp near cos = 1).  Any error that repeats
// at every step is a fixed relative error per step, so a gate close to 1,
// which carries state over M ~ 1/(1-|g|) steps, turns it into a relative
// drift of ~M x that error in the state and in every gradient summed over
// steps.  The rotational cos / sin are therefore evaluated from an exact
// angle reduction: the angle in 1/256 revolutions splits into a table index
// plus a remainder |x| <= pi/256, where cos x - 1 = -x^2/2 and
// sin x = x - x^3/6 are accurate to 1e-9 absolute.  The table records are
// sign-folded around the nearest of +-1 (gen_sincos_table.py): a record holds
// m = b (1 - |cos|), b = +-1 the sign of m, so the kernels form
// w = cos / b - 1 and the gate as (b e)(1 + w) with one rounding.  |m| is
// small where |cos| is close to 1, so the error that a table entry repeats
// at every step that reads it stays below 0.02 ulp of the gate there (a
// table of rounded cosines repeats up to 0.5 ulp, which drifted the A
// gradients of long-memory states to ~2x the reference's distance from
// float64).  The gate is then accurate to ~0.6 ulp of 1 in absolute terms,
// which is what the state update h = g s + hb needs for any |g|.
// (Rounding Ar*log2(e) and 256*Ai/(2 pi) once per state is harmless by
// contrast: its error scales with dt*A, so it stays ~1 ulp of the state over
// any memory length.)
// The forward and the step share the gate code, so the step continues the
// scan bit for bit; the backward evaluates the same expansion from its own
// records (it also needs the sine), to within an ulp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "redpanda_hip.h"
#include "rp_launch.h"
#include "rp_sincos_table.h"

namespace rp {

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kTwoPi = 6.28318530717958647692f;

template <int S, int NPL>
struct Shape {
  static constexpr int kS = S;
  static constexpr int kNPL = NPL;
  static constexpr int kDT = kWave / S;        // channels per wave
  static constexpr int kCB = kWaves * kDT;     // channels per workgroup
  static constexpr int kNP = S * NPL;          // padded states per channel
  static_assert(S == 2 || S == 4 || S == 8 || S == 16, "S must be a power of two <= 16");
};

// Streamed-input element as stored (fp32 bits, or a bf16 / fp16 pattern in
// the low half), and its fp32 value; split so that a load can be issued well
// before its value is needed.
__device__ __forceinline__ uint32_t load_raw(const void* p, int64_t i, int dtype) {
  if (dtype == RP_F32) return __float_as_uint(static_cast<const float*>(p)[i]);
  return static_cast<const uint16_t*>(p)[i];
}

__device__ __forceinline__ float cvt_raw(uint32_t v, int dtype) {
  if (dtype == RP_F32) return __uint_as_float(v);
  if (dtype == RP_BF16) return __uint_as_float(v << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v)));
}

// Streamed-input load with on-the-fly conversion to fp32 (uniform dtype).
__device__ __forceinline__ float load_in(const void* p, int64_t i, int dtype) {
  return cvt_raw(load_raw(p, i, dtype), dtype);
}

// Features per state of the MIMO projections (P <= kBcMaxP).
constexpr int kBcMaxP = 8;

// Sum over a wave's 64 lanes (xor butterfly; every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

// BCNorm + p-sum of one token (engine/mamba.py:89 RMSNorm, :297-300,
// :336-337) for the states n = lane + 64 s of a wave:
//     acc[s] = sum_p (x[n,p] r) w[n,p]   (p in order),
//     r = rsqrt(mean of x^2 over the N*P features + eps),
// or the plain p-sum when not normalising.  x holds the token's features at
// row + n * P + p, in storage dtype dt.  One wave per token, every lane
// taking part; wt: the lane's weights (1 beyond N or P).  The BCNorm kernel
// and the step kernel's fused prologue both use it, so they give the same
// bits.
template <int SL>
__device__ __forceinline__ void bcnorm_token(const void* x, int64_t row, int dt, int lane, int N,
                                             int P, bool normalize, float eps, float invK,
                                             const float (&wt)[SL][kBcMaxP], float (&acc)[SL]) {
  float v[SL][kBcMaxP];
  float ss = 0.f;
#pragma unroll
  for (int s = 0; s < SL; ++s) {
    const int n = lane + s * kWave;
#pragma unroll
    for (int q = 0; q < kBcMaxP; ++q) {
      v[s][q] = (n < N && q < P) ? load_in(x, row + n * P + q, dt) : 0.f;
      ss += v[s][q] * v[s][q];
    }
  }
  float r = 1.f;
  if (normalize) r = rsqrtf(wave_sum(ss) * invK + eps);
#pragma unroll
  for (int s = 0; s < SL; ++s) {
    float a = 0.f;
#pragma unroll
    for (int q = 0; q < kBcMaxP; ++q) {
      if (q >= P) break;
      const float y = normalize ? (v[s][q] * r) * wt[s][q] : v[s][q];
      a = q == 0 ? y : a + y;
    }
    acc[s] = a;
  }
}

// The raw element type of storage code IT, as load_raw returns it widened.
template <int IT>
using RawOf = typename std::conditional<IT == RP_F32, uint32_t, uint16_t>::type;

// Element i of a row given by a wave-uniform pointer, i a 32-bit lane offset:
// the address form of a global access with a scalar base and a 32-bit vector
// offset, so the lane's part costs no 64-bit arithmetic.
template <class T>
__device__ __forceinline__ T load_at(const void* row, uint32_t i) {
  return *reinterpret_cast<const T*>(static_cast<const char*>(row) + i * (uint32_t)sizeof(T));
}
template <class T>
__device__ __forceinline__ void store_at(void* row, uint32_t i, T v) {
  *reinterpret_cast<T*>(static_cast<char*>(row) + i * (uint32_t)sizeof(T)) = v;
}
// The same with the lane's part given in bytes.
template <class T>
__device__ __forceinline__ T load_byte(const void* base, uint32_t off) {
  return *reinterpret_cast<const T*>(static_cast<const char*>(base) + off);
}
template <class T>
__device__ __forceinline__ void store_byte(void* base, uint32_t off, T v) {
  *reinterpret_cast<T*>(static_cast<char*>(base) + off) = v;
}
// A streamed-input element as stored (load_raw's result) at a byte offset.
__device__ __forceinline__ uint32_t load_raw_byte(const void* base, uint32_t off, int dtype) {
  if (dtype == RP_F32) return load_byte<uint32_t>(base, off);
  return load_byte<uint16_t>(base, off);
}

__device__ __forceinline__ float fmul(float a, float b) { return a * b; }

// delta = softplus(x) for the dt projection (engine/mamba.py:300, F.softplus
// with beta 1, threshold 20, in fp32), as max(x, 0) + log1p(t), t = exp(-|x|)
// in (0, 1].  log1p from the series log1p(t) = 2 atanh(s) = 2 (s + s^3/3 +
// s^5/5 + ...), s = t / (2 + t) <= 1/3 (Abramowitz & Stegun 4.1.27): the
// terms through s^15 leave a truncation below 3e-9 relative.  s from the
// reciprocal with one Newton step against the exact denominator (2 + t
// rounds to d, and t - (d - 2) is its rounding error, exact).  About 30 VALU
// where log1pf's double-float evaluation takes about 110; within 2.8 ulp of
// the exact value (log1pf(expf(x)) in fp32 is within 2.7: the rounding of
// exp's result dominates both).  Explicit FMAs and no contraction: every
// kernel rounds it the same way.
__device__ __forceinline__ float softplus_of(float x) {
#pragma clang fp contract(off)
  const float t = expf(-fabsf(x));
  const float d = 2.f + t;
  const float dlo = t - (d - 2.f);
  const float r = __builtin_amdgcn_rcpf(d);
  const float s0 = t * r;
  float e = __builtin_fmaf(-s0, d, t);
  e = __builtin_fmaf(-s0, dlo, e);
  const float s = __builtin_fmaf(e, r, s0);
  const float s2 = s * s;
  float q = 1.f / 15.f;
  q = __builtin_fmaf(q, s2, 1.f / 13.f);
  q = __builtin_fmaf(q, s2, 1.f / 11.f);
  q = __builtin_fmaf(q, s2, 1.f / 9.f);
  q = __builtin_fmaf(q, s2, 1.f / 7.f);
  q = __builtin_fmaf(q, s2, 1.f / 5.f);
  q = __builtin_fmaf(q, s2, 1.f / 3.f);
  const float l = __builtin_fmaf(2.f * (s * s2), q, 2.f * s);
  const float v = fmaxf(x, 0.f) + l;
  return x > 20.f ? x : v;
}

// fp32 -> the value a storage dtype holds (round to nearest even, as torch
// converts); inf and nan pass through.
__device__ __forceinline__ float round_storage(float v, int dtype) {
  if (dtype == RP_F32) return v;
  if (dtype == RP_BF16) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7f800000u) != 0x7f800000u) b += 0x7fffu + ((b >> 16) & 1u);
    return __uint_as_float(b & 0xffff0000u);
  }
  return static_cast<float>(static_cast<_Float16>(v));
}

// A gradient element in its storage dtype at the byte offset o of its fp32
// layout (o / 2 for a 16-bit one), rounded to nearest even as torch converts.
__device__ __forceinline__ void store_grad(void* base, uint32_t o, float v, int dtype) {
  if (dtype == RP_F32)
    store_byte<float>(base, o, v);
  else if (dtype == RP_BF16)
    store_byte<uint16_t>(base, o >> 1, (uint16_t)(__float_as_uint(round_storage(v, RP_BF16)) >> 16));
  else
    store_byte<_Float16>(base, o >> 1, static_cast<_Float16>(v));
}
// The same at element index i.
__device__ __forceinline__ void store_grad_at(void* base, int64_t i, float v, int dtype) {
  if (dtype == RP_F32)
    static_cast<float*>(base)[i] = v;
  else if (dtype == RP_BF16)
    static_cast<uint16_t*>(base)[i] = (uint16_t)(__float_as_uint(round_storage(v, RP_BF16)) >> 16);
  else
    static_cast<_Float16*>(base)[i] = static_cast<_Float16>(v);
}

// y * silu(z) as torch computes it: silu(z) = z / (1 + exp(-z)) rounded to
// z's storage dtype, then the product in fp32.
__device__ __forceinline__ float silu_gate(float y, float z, int dtype_z) {
  return y * round_storage(z / (1.f + expf(-z)), dtype_z);
}
// The same derivative from delta = softplus(x) itself: sigmoid(x) =
// 1 - exp(-delta), as -expm1(-delta) (accurate for small delta; 1 above the
// threshold, where delta = x > 20).
__device__ __forceinline__ float softplus_grad_from_delta(float g, float delta) {
  return fmul(g, -expm1f(-delta));
}
__device__ __forceinline__ float ffma(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// exp2 on the transcendental unit (v_exp_f32).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// The gate tables copied into LDS once per workgroup (read after the
// workgroup's next barrier): the sign-folded records (m, b (-sin a))
// (forward and step) or (m, b sin) (backward) of the kTab table angles
// 2 pi k / kTab.
__device__ __forceinline__ void fill_cos_lin(float2* ctab, int tid) {
  for (int k = tid; k < kTab; k += kThreads) ctab[k] = kCosLin[k];
}
// the forward's records with their two expansion coefficients (16 bytes)
__device__ __forceinline__ float2 cos_lin_coefs(float2 rec);
__device__ __forceinline__ void fill_cos_lin(float4* ctab, int tid) {
  for (int k = tid; k < kTab; k += kThreads) {
    const float2 rec = kCosLin[k], pc = cos_lin_coefs(rec);
    ctab[k] = make_float4(rec.x, rec.y, pc.x, pc.y);
  }
}
__device__ __forceinline__ void fill_sincos_pairs(float2* cstab, int tid) {
  for (int k = tid; k < kTab; k += kThreads) cstab[k] = kSinCos[k];
}

// Per-state gate parameters held in registers: pah = fl(A_real log2(e)) and
// wh = fl(256 A_imag / (2 pi)) (the angle rate in 1/256 revolutions) for
// rotational states; pah = tanh(theta) for tracking states; zeros for pad.
// In two phases, so that a caller issues the loads of all its states before
// the first value is needed: gate_param_load fetches without lane-divergent
// control flow (every lane loads from a valid address: Ar is non-null when
// NR > 0 and Tk when NT > 0), gate_param_finish selects and converts.
struct GateRaw {
  float ar, ai, tk;
};

__device__ __forceinline__ GateRaw gate_param_load(const float* Ar, const float* Ai,
                                                   const float* Tk, int c, int n, int N, int NR,
                                                   int NT, bool valid) {
  const bool rot = valid && n < NR;
  const bool trk = valid && n >= NR && n < N;
  const int64_t ir = rot ? (int64_t)c * NR + n : 0;
  const int64_t it = trk ? (int64_t)c * NT + (n - NR) : 0;
  GateRaw g{0.f, 0.f, 0.f};
  if (NR > 0) {
    g.ar = Ar[ir];
    if (Ai != nullptr) g.ai = Ai[ir];
  }
  if (NT > 0) g.tk = Tk[it];
  return g;
}

__device__ __forceinline__ void gate_param_finish(int n, int N, int NR, bool valid,
                                                  const GateRaw& g, float& pah, float& wh) {
  // x * K with K split as kHi + kLo: one rounding of the extended product
  constexpr float kL2eHi = 1.4426950216293335f, kL2eLo = 1.925963033500011e-08f;  // log2(e)
  constexpr float kWHi = 40.7436637878418f, kWLo = 1.6436833902844228e-06f;  // 256/(2 pi)
  const bool rot = valid && n < NR;
  const bool trk = valid && n >= NR && n < N;
  const float pr = ffma(g.ar, kL2eHi, fmul(g.ar, kL2eLo));
  const float wr = ffma(g.ai, kWHi, fmul(g.ai, kWLo));
  pah = rot ? pr : (trk ? g.tk : 0.f);
  wh = rot ? wr : 0.f;
}

constexpr float kRadPerStep = 0.02454369328916073f;  // 2 pi / 256: radians per table step
constexpr float kRint = 12582912.f;  // 1.5 * 2^23: x + kRint rounds x to an integer
// With a = 2 pi / 256 and |r| <= 1/2:  cos(a r) - 1 = kC2 r^2  (truncation
// < 9.5e-10),  sin(a r) = r (kS1 + kS3 r^2)  (truncation < 2.4e-12)
constexpr float kC2 = -0.0003011964145116508f;
constexpr float kS1 = 0.02454369328916073f, kS3 = -2.464157432768843e-06f;

// How a kernel instantiation knows the rotational / tracking split:
//   RJ   leading state slots j < RJ are rotational in every lane (compile
//        time);
//   TJ   trailing slots j >= TJ are tracking (or padding) in every lane
//        (compile time); slots RJ <= j < TJ are decided at run time from NR;
//   IMAG 1: complex rotational gates, 0: real decay gates, 2: decided at
//        run time from has_imag.
// Specialised and generic instantiations run the same arithmetic, so their
// results are bitwise equal.
template <int RJ, int IMAG, int TJ>
struct GateKind {
  static constexpr int kRJ = RJ;
  static constexpr int kImag = IMAG;
  static constexpr int kTJ = TJ;
};

// Rotational gate g = 2^(dt pah) cos(a dt wh), a = 2 pi / 256.  The exact
// product dt*wh (an FMA with the round-to-integer constant, then one with
// -k) splits into an integer k, the table index, and a remainder |r| <= 1/2
// rounded once.  The split needs |dt wh| < 2^22, i.e. |dt A_imag| < 1e5.
// Returns the table index (low kTabBits of the rounded value).
__device__ __forceinline__ int angle_split(float dt, float wh, float& r) {
  const float t = ffma(dt, wh, kRint);
  const float kf = t - kRint;  // rint(dt wh), exact
  r = ffma(dt, wh, -kf);
  return __float_as_int(t) & (kTab - 1);
}

// Two flavours of the same expansion, in two phases each so that a caller
// can start the exponentials and table reads of several states before
// finishing any of them (issue, then finish):
//   * the forward and the step: w = cos/b - 1 as the cubic in r from the
//     index's record (m, b (-s a)) (one 8-byte table read; the two higher
//     coefficients one operation each, then three FMAs);
//   * the backward: w and also b sin from the index's record (m, b s) (one
//     8-byte read; the two expansions share r^2, cos(a r) - 1 and sin(a r)).
//     Its gate is the forward's to within an ulp (the same expansion,
//     rounded differently).
// Both return the gate as (b e)(1 + w), b e = e with the sign bit of m.
// R: the forward's table record, (m, b (-s a)) as float2, or as float4 with
// the expansion's two record-only coefficients (p3, p2) appended (taken at
// the table's fill by the same operations, so the gate is bitwise the same)
template <class R>
struct GatePart {
  float e;  // 2^(dt pah)
  float r;  // angle remainder, |r| <= 1/2 (table steps)
  R cr;     // the table angle's record
};

struct GatePartCS {
  float e;
  float r;
  float2 cs;  // (m, b s) of the table angle
};

// e (>= 0) with the sign bit of m: b e for a sign-folded record.
__device__ __forceinline__ float signed_by(float e, float m) {
  return __uint_as_float(__float_as_uint(e) | (__float_as_uint(m) & 0x80000000u));
}

// cos(a (k + r)) / b - 1 = -|m| + r (t + r ((1 - |m|) kC2 + r t kA3)),
// t = b (-s a), kA3 = -a^2/6: the coefficients (p3, p2) = (t kA3,
// (1 - |m|) kC2) of the record (m, t)
__device__ __forceinline__ float2 cos_lin_coefs(float2 rec) {
  constexpr float kA3 = -1.0039880779102944e-4f;
  return make_float2(fmul(rec.y, kA3), ffma(-fabsf(rec.x), kC2, kC2));
}

template <class R>
__device__ __forceinline__ GatePart<R> rot_gate_issue(float dt, float pah, float wh, bool imag,
                                                      const R* ctab) {
  GatePart<R> g;
  g.e = exp2_hw(fmul(dt, pah));
  if (!imag) {
    g.r = 0.f;
    g.cr = R{};
    return g;
  }
  g.cr = ctab[angle_split(dt, wh, g.r)];
  return g;
}

template <class R>
__device__ __forceinline__ float rot_gate_finish(const GatePart<R>& g, bool imag) {
  if (!imag) return g.e;
  const float r = g.r, am = fabsf(g.cr.x);
  float2 pc;  // (p3, p2)
  if constexpr (std::is_same<R, float4>::value)
    pc = make_float2(g.cr.z, g.cr.w);
  else
    pc = cos_lin_coefs(g.cr);
  const float w = ffma(r, ffma(r, ffma(r, pc.x, pc.y), g.cr.y), -am);
  const float be = signed_by(g.e, g.cr.x);
  return ffma(be, w, be);
}

__device__ __forceinline__ GatePartCS rot_gate_issue_cs(float dt, float pah, float wh, bool imag,
                                                        const float2* cstab) {
  GatePartCS g;
  g.e = exp2_hw(fmul(dt, pah));
  if (!imag) {
    g.r = 0.f;
    g.cs = make_float2(0.f, 0.f);
    return g;
  }
  g.cs = cstab[angle_split(dt, wh, g.r)];
  return g;
}

__device__ __forceinline__ float rot_gate_finish_cs(const GatePartCS& g, bool imag, float& es) {
  if (!imag) {
    es = 0.f;
    return g.e;
  }
  const float r = g.r, am = fabsf(g.cs.x), sb = g.cs.y;  // |m|, b sin
  const float r2 = fmul(r, r);
  const float cm1 = fmul(r2, kC2);                 // cos(a r) - 1
  const float sx = fmul(r, ffma(r2, kS3, kS1));    // sin(a r)
  // cos / b - 1 = cm1 - |m| (1 + cm1) - (b s) sin(a r)
  const float w = ffma(-sb, sx, ffma(-am, cm1, cm1 - am));
  // sin / b = (b s)(1 + cm1) + (1 - |m|) sin(a r)
  const float v = ffma(sb, cm1, sb) + ffma(-am, sx, sx);
  const float be = signed_by(g.e, g.cs.x);
  es = fmul(be, v);
  return ffma(be, w, be);
}

// Whether state slot j of lane slice s is rotational (n = j*S + s < NR).
template <int S, class GK>
__device__ __forceinline__ bool is_rot(int j, int s, int NR) {
  if (j >= GK::kTJ) return false;
  if (j < GK::kRJ) return true;
  if (j * S >= NR) return false;
  return (j + 1) * S <= NR || j * S + s < NR;
}

// Host side: calls f(GK{}) with the GateKind instantiation of gate code gk.
// (kGateRotAll takes the RotLead instantiation here, kGateRealAll the
// Generic one: the same values; the launchers that instantiate them test for
// them first.)
template <int NPL, class F>
hipError_t with_gate_kind(int gk, F&& f) {
  if (gk == kGateRotTrack) return f(GateKind<NPL - 1, 1, NPL - 1>{});
  if (gk == kGateRotLead || gk == kGateRotAll) return f(GateKind<NPL - 1, 1, NPL>{});
  return f(GateKind<0, 2, NPL>{});
}

// The scan launchers' dispatch: with_gate_kind, plus the all-rotational and
// all-real instantiations on the shapes of all_gate_shape.
template <int S, int NPL, class F>
hipError_t with_gate_kind_scan(int gk, F&& f) {
  if constexpr (all_gate_shape(S, NPL)) {
    if (gk == kGateRotAll) return f(GateKind<NPL, 1, NPL>{});
    if (gk == kGateRealAll) return f(GateKind<NPL, 0, NPL>{});
  }
  return with_gate_kind<NPL>(gk, f);
}

template <class GK>
__device__ __forceinline__ bool imag_of(bool has_imag) {
  return GK::kImag == 2 ? has_imag : GK::kImag == 1;
}

// Gate of state slot j for lane slice s (forward flavour): rotational if
// n < NR, else the tracking gate pah = tanh(theta) (pad states beyond N
// carry 0 and B = C = 0).
template <int S, class GK, class R>
__device__ __forceinline__ float gate_of(int j, int s, int NR, bool has_imag, float dt, float pah,
                                         float wh, const R* ctab) {
  if (j >= GK::kTJ) return pah;
  const bool imag = imag_of<GK>(has_imag);
  if (j < GK::kRJ) return rot_gate_finish(rot_gate_issue(dt, pah, wh, imag, ctab), imag);
  if (j * S >= NR) return pah;
  const float gr = rot_gate_finish(rot_gate_issue(dt, pah, wh, imag, ctab), imag);
  if ((j + 1) * S <= NR || j * S + s < NR) return gr;
  return pah;
}

// The backward flavour of gate_of (with es), in two phases: gate_issue_cs
// starts the rotational part of slot j, gate_finish_cs returns the gate.
template <int S, class GK>
__device__ __forceinline__ GatePartCS gate_issue_cs(int j, int NR, bool has_imag, float dt,
                                                    float pah, float wh, const float2* cstab) {
  if (j >= GK::kTJ || (j >= GK::kRJ && j * S >= NR)) return GatePartCS{0.f, 0.f, {1.f, 0.f}};
  return rot_gate_issue_cs(dt, pah, wh, imag_of<GK>(has_imag), cstab);
}

template <int S, class GK>
__device__ __forceinline__ float gate_finish_cs(int j, int s, int NR, bool has_imag,
                                                const GatePartCS& part, float pah, float& es) {
  if (j >= GK::kTJ) {
    es = 0.f;
    return pah;
  }
  if (j < GK::kRJ) return rot_gate_finish_cs(part, imag_of<GK>(has_imag), es);
  if (j * S >= NR) {
    es = 0.f;
    return pah;
  }
  const float gr = rot_gate_finish_cs(part, imag_of<GK>(has_imag), es);
  if ((j + 1) * S <= NR || j * S + s < NR) return gr;
  es = 0.f;
  return pah;
}

// Per-lane gate parameters of NPL states.
template <int NPL>
struct GateRegs {
  float pah[NPL], wh[NPL];
};

template <int S, int NPL>
__device__ __forceinline__ void load_gate_regs(GateRegs<NPL>& gp, const float* Ar, const float* Ai,
                                               const float* Tk, int c, int s, int N, int NR,
                                               int NT, bool valid) {
  GateRaw g[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) g[j] = gate_param_load(Ar, Ai, Tk, c, j * S + s, N, NR, NT, valid);
#pragma unroll
  for (int j = 0; j < NPL; ++j) gate_param_finish(j * S + s, N, NR, valid, g[j], gp.pah[j], gp.wh[j]);
}

// One recurrence step for the lane's NPL states; returns the lane's partial
//     y = sum_j h_j C_j     (FMA chain in j order).
// hdu = (dt*u)/2, so hb = hdu*B_n equals beta_t/2 exactly; hbp holds the
// previous step's hb.  Shared verbatim by the scan and step kernels.
//
// The update is h_t = g h_{t-1} + (g hb_{t-1} + hb_t): the trapezoid's two
// input terms are combined first (one rounding at their own, small
// magnitude), then one FMA with the state.  A state with a long memory
// (|g| near 1) is much larger than its per-step input, so each step then
// rounds once at the state's magnitude, where the form g (h + hb) + hb
// rounds twice (the sum, then the FMA).  Those roundings accumulate over the
// memory (about 1 / (1 - |g|) steps); a CPU emulation of the kernels'
// operations at the long-sequence shape (L = 2048, tracking gates up to
// 0.9993) put the tracking-gate gradient 2.5e-6 from float64 with the
// two-rounding forms and 2.5e-7 with these (the adjoint takes the same
// form, scan_bwd_kernel.h), against 1.2e-6 for the reference's fp32 scan.
template <int S, int NPL, class GK, class R>
__device__ __forceinline__ float fwd_update(float (&h)[NPL], float (&hbp)[NPL],
                                            const GateRegs<NPL>& gp, const R* ctab, float dt,
                                            float hdu, const float* __restrict__ Bs,
                                            const float* __restrict__ Cs, int s, int NR,
                                            bool has_imag) {
  float y = 0.f;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const float g = gate_of<S, GK>(j, s, NR, has_imag, dt, gp.pah[j], gp.wh[j], ctab);
    const float hb = fmul(hdu, Bs[j]);
    h[j] = ffma(g, h[j], ffma(g, hbp[j], hb));
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
