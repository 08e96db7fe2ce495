// Launchers and reduction kernels of the scan backward, and its general
// (non-FAST) instantiations; the kernel itself is in scan_bwd_kernel.h and its
// whole-tile instantiations in scan_bwd_fast.hip (separate translation units
// so that the two compile in parallel).

#include "scan_bwd_kernel.h"

namespace rp {

// dB / dC: sum the per-tile-group partials in a fixed order (fp64 accumulator).
// The loads do not depend on the sum, so the unrolled loop keeps 8 of them in
// flight while the additions stay in tile order.  bwd_reduce_bc4 sums four
// adjacent elements per thread with 16-byte loads (the same additions in the
// same order), for (B*L*N) a multiple of 4 and 16-byte aligned partials,
// dB and dC.
__global__ void bwd_reduce_bc4(const float4* __restrict__ part, float4* __restrict__ dB,
                               float4* __restrict__ dC, int64_t per4, int ntiles) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= 2 * per4) return;
  const int which = e >= per4;
  const int64_t k = which ? e - per4 : e;
  const float4* src = part + (int64_t)which * ntiles * per4 + k;
  double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
#pragma unroll 8
  for (int g = 0; g < ntiles; ++g) {
    const float4 v = src[(int64_t)g * per4];
    a0 += v.x;
    a1 += v.y;
    a2 += v.z;
    a3 += v.w;
  }
  (which ? dC : dB)[k] = make_float4((float)a0, (float)a1, (float)a2, (float)a3);
}

__global__ void bwd_reduce_bc(const float* __restrict__ part, float* __restrict__ dB,
                              float* __restrict__ dC, int64_t per, int ntiles) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= 2 * per) return;
  const int which = e >= per;
  const int64_t k = which ? e - per : e;
  const float* src = part + (int64_t)which * ntiles * per + k;
  double acc = 0.0;
#pragma unroll 8
  for (int g = 0; g < ntiles; ++g) acc += src[(int64_t)g * per];
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
#pragma unroll 8
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

// Whether a launch takes the FAST instantiation: no initial state and no
// final-state gradients, every tile's channels present, and every array the
// chunk loop addresses spanning less than 4 GiB (its byte offsets then fit
// in 32 bits).
static bool bwd_fast(const ScanParams& p, const BwdIO& io, int CB) {
  if (p.h0 != nullptr || io.dh_last != nullptr || io.dbeta_last != nullptr || io.d_h0 != nullptr)
    return false;
  if (p.D % CB != 0) return false;
  const int64_t lim = (int64_t)1 << 32;
  auto es = [](int dt) { return (int64_t)(dt == RP_F32 ? 4 : 2); };
  // one past the last byte of a (B, L, inner) array with strides sb, sl
  auto span = [&](int64_t sb, int64_t sl, int64_t inner, int64_t e) {
    return ((p.B - 1) * sb + (p.L - 1) * sl + inner) * e;
  };
  const bool cached = p.dsp != 0;
  const int64_t dspan = cached ? (int64_t)p.B * p.L * p.D * 4 : span(p.dsb, p.dsl, p.D, es(p.dt_delta));
  const int64_t half = (int64_t)p.ntiles * p.B * p.L * p.N;
  return dspan < lim && span(p.usb, p.usl, p.D, es(p.dt_u)) < lim &&
         span(p.bsb, p.bsl, p.N, es(p.dt_B)) < lim && span(p.csb, p.csl, p.N, es(p.dt_C)) < lim &&
         (int64_t)p.B * p.L * p.D * 4 < lim && (half + (int64_t)p.L * p.N) * 4 < lim;
}

template <int S, int NPL, class GK>
static hipError_t launch_bwd_t(const ScanParams& p, const BwdIO& io, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)io.ntg * io.nbg));
  hipLaunchKernelGGL((scan_bwd_kernel<S, NPL, GK, false, false>), grid, dim3(kThreads), 0, st, p,
                     io);
  return hipGetLastError();
}

hipError_t launch_scan_bwd(int S, int NPL, int gk, const ScanParams& p, const BwdIO& io,
                           hipStream_t st) {
  if (S > 0 && bwd_fast(p, io, kWaves * (kWave / S))) return launch_scan_bwd_fast(S, NPL, gk, p, io, st);
  if (io.tpw > 1) return launch_scan_bwd_walk(S, NPL, gk, false, p, io, st);
#define RP_CASE(SS, NN)                                                              \
  if (S == SS && NN == NPL)                                                          \
    return with_gate_kind_scan<SS, NN>(gk, [&](auto g) {                                      \
      return launch_bwd_t<SS, NN, decltype(g)>(p, io, st);                           \
    });
  RP_FOR_EACH_SHAPE(RP_CASE)
#undef RP_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_finalize(const ScanParams& p, const BwdIO& io, float* d_Bc, float* d_Cc,
                               float* d_Ar, float* d_Ai, float* d_Tk, hipStream_t st) {
  const int64_t per = (int64_t)p.B * p.L * p.N;
  auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  if (per > 0 && per % 4 == 0 && al16(io.part_bc) && al16(d_Bc) && al16(d_Cc)) {
    const int64_t n = 2 * (per / 4);
    hipLaunchKernelGGL(bwd_reduce_bc4, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       (const float4*)io.part_bc, (float4*)d_Bc, (float4*)d_Cc, per / 4, io.ntg);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  } else if (per > 0) {
    const int64_t n = 2 * per;
    hipLaunchKernelGGL(bwd_reduce_bc, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       (const float*)io.part_bc, d_Bc, d_Cc, per, io.ntg);
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
