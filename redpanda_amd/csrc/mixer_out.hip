// The mixer's output gate around the scan, fused: out = (y + k u D) silu(z).
//
// Replaces the elementwise torch ops that follow the scan in
// Mamba3Block.forward (engine/mamba.py:262-265 and :350 / :375): the D-skip
// (added once per direction, k = 1 causal / 2 bidirectional) and the
// y * silu(z) gate, and their backward, each as one pass over (B, L, D).
//
// Rounding follows torch's own ops in order, so fp32 inputs reproduce the
// eager result: y + u*D (+ u*D), silu(z) = z / (1 + exp(-z)) rounded to z's
// dtype, then the product in fp32 -- stored in fp32, or rounded to the
// autocast dtype the next projection casts it to (its gradient then arrives
// in that dtype too).  Backward (autograd of the same graph):
//     s = silu(z) (rounded),   dyk = dout * s,   ds = round_z(dout * yk)
//     dz = round_z(ds * sig (1 + z (1 - sig))),  sig = 1 / (1 + exp(-z))
//     dy = dyk (the scan's upstream gradient)
//     du = round_u(dyk * D) [+ round_u(dyk * D)]  (one term per skip)
//     dD = k * sum_{b,t} dyk * u    (fixed-order float64 partials, then fp32)
// Layout: each lane owns 8 consecutive channels (16-byte loads and stores of
// every operand); a workgroup takes a row group of one 512-channel tile, its
// 4 waves a quarter of the rows each.  Shapes whose rows are not 16-byte
// aligned use a scalar kernel (one thread per channel, a workgroup per row
// group).  The backward's dD partials are per row group, summed by a second
// kernel in a fixed order.

#include "rp_device.h"
#include "rp_launch.h"

#include <type_traits>

namespace rp {

// fp32 -> storage dtype, round to nearest even (torch's conversions).
__device__ __forceinline__ float round_to(float v, int dtype) {
  if (dtype == RP_F32) return v;
  if (dtype == RP_BF16) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7f800000u) != 0x7f800000u) b += 0x7fffu + ((b >> 16) & 1u);  // not inf / nan
    return __uint_as_float(b & 0xffff0000u);
  }
  return static_cast<float>(static_cast<_Float16>(v));
}

__device__ __forceinline__ void store_as(void* p, int64_t i, float v, int dtype) {
  if (dtype == RP_F32) {
    static_cast<float*>(p)[i] = v;
  } else if (dtype == RP_BF16) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(__float_as_uint(round_to(v, RP_BF16)) >> 16);
  } else {
    static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
  }
}

// Row r = b * L + t of a (B, L, D) tensor with batch / time strides; the
// workgroup's rows are walked with a branch-free cursor so that loads of
// consecutive rows can be issued together.
struct RowCursor {
  int b, t;
  __device__ __forceinline__ RowCursor(int64_t r, int L) : b((int)(r / L)), t((int)(r % L)) {}
  __device__ __forceinline__ int64_t at(int64_t sb, int64_t sl) const { return b * sb + t * sl; }
  __device__ __forceinline__ void next(int L) {
    ++t;
    const bool wrap = t == L;
    b += wrap ? 1 : 0;
    t = wrap ? 0 : t;
  }
};

__global__ __launch_bounds__(kThreads) void mixer_out_fwd_kernel(MixerOutParams p) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= p.D) return;
  const float dk = p.Dskip[c];
  const int64_t r_lo = (int64_t)blockIdx.y * p.rows_per_unit;
  const int64_t r_hi = min(p.rows, r_lo + p.rows_per_unit);
  RowCursor cur(r_lo, p.L);
#pragma unroll 4
  for (int64_t r = r_lo; r < r_hi; ++r) {
    const float u = load_in(p.u, cur.at(p.usb, p.usl) + c, p.dt_u);
    const float z = load_in(p.z, cur.at(p.zsb, p.zsl) + c, p.dt_z);
    cur.next(p.L);
    float yk = p.y[r * p.D + c] + u * dk;
    if (p.k_skip == 2) yk = yk + u * dk;
    const float s = round_to(z / (1.f + expf(-z)), p.dt_z);
    store_as(p.out, r * p.D + c, yk * s, p.dt_out);
  }
}

__global__ __launch_bounds__(kThreads) void mixer_out_bwd_kernel(MixerOutParams p, MixerOutGrad g) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= p.D) return;
  const float dk = p.Dskip[c];
  const int64_t r_lo = (int64_t)blockIdx.y * p.rows_per_unit;
  const int64_t r_hi = min(p.rows, r_lo + p.rows_per_unit);
  RowCursor cur(r_lo, p.L);
  double acc = 0.0;  // sum of dyk * u over the group's rows
#pragma unroll 4
  for (int64_t r = r_lo; r < r_hi; ++r) {
    const float u = load_in(p.u, cur.at(p.usb, p.usl) + c, p.dt_u);
    const float z = load_in(p.z, cur.at(p.zsb, p.zsl) + c, p.dt_z);
    cur.next(p.L);
    const int64_t i = r * p.D + c;
    const float dout = load_in(g.dout, i, p.dt_out);
    float yk = p.y[i] + u * dk;
    if (p.k_skip == 2) yk = yk + u * dk;
    const float e = expf(-z);
    const float sig = 1.f / (1.f + e);
    const float s = round_to(z / (1.f + e), p.dt_z);
    const float dyk = dout * s;
    const float ds = round_to(dout * yk, p.dt_z);
    const float dz = ds * sig * (1.f + z * (1.f - sig));
    g.dy[i] = dyk;
    store_as(g.dz, i, dz, p.dt_z);
    const float du1 = round_to(dyk * dk, p.dt_u);
    store_as(g.du, i, p.k_skip == 2 ? round_to(du1 + du1, p.dt_u) : du1, p.dt_u);
    acc += (double)(dyk * u);
  }
  g.part[(int64_t)blockIdx.y * p.D + c] = acc;
}

// ── vector path: 8 channels per lane ──

template <int DT>
__device__ __forceinline__ void load8(const void* p, int64_t i, float (&v)[kMixVec]) {
  if constexpr (DT == RP_F32) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 a = q[0], b = q[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = cvt_raw(ws[k] & 0xffffu, DT);
      v[2 * k + 1] = cvt_raw(ws[k] >> 16, DT);
    }
  }
}

__device__ __forceinline__ void load8f(const float* p, int64_t i, float (&v)[kMixVec]) {
  load8<RP_F32>(p, i, v);
}

// storage bits of an fp32 value already rounded to the storage dtype
template <int DT>
__device__ __forceinline__ uint32_t bits16(float v) {
  if constexpr (DT == RP_BF16) return __float_as_uint(round_to(v, RP_BF16)) >> 16;
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

template <int DT>
__device__ __forceinline__ void store8(void* p, int64_t i, const float (&v)[kMixVec]) {
  if constexpr (DT == RP_F32) {
    float4* q = reinterpret_cast<float4*>(static_cast<float*>(p) + i);
    q[0] = make_float4(v[0], v[1], v[2], v[3]);
    q[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint4 w;
    w.x = bits16<DT>(v[0]) | (bits16<DT>(v[1]) << 16);
    w.y = bits16<DT>(v[2]) | (bits16<DT>(v[3]) << 16);
    w.z = bits16<DT>(v[4]) | (bits16<DT>(v[5]) << 16);
    w.w = bits16<DT>(v[6]) | (bits16<DT>(v[7]) << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) = w;
  }
}

// The same for a dtype known only at run time (uniform across the launch).
__device__ __forceinline__ void load8_rt(const void* p, int64_t i, float (&v)[kMixVec], int dt) {
  if (dt == RP_F32)
    load8<RP_F32>(p, i, v);
  else if (dt == RP_BF16)
    load8<RP_BF16>(p, i, v);
  else
    load8<RP_F16>(p, i, v);
}

__device__ __forceinline__ void store8_rt(void* p, int64_t i, const float (&v)[kMixVec], int dt) {
  if (dt == RP_F32)
    store8<RP_F32>(p, i, v);
  else if (dt == RP_BF16)
    store8<RP_BF16>(p, i, v);
  else
    store8<RP_F16>(p, i, v);
}

// Lane's first channel and its wave's rows: a workgroup takes row group
// blockIdx.y (rows_per_unit rows) of one 512-channel tile, each wave a
// quarter of the group.  False when the lane has no channels; the row range
// may be empty.
__device__ __forceinline__ bool vec_slot(const MixerOutParams& p, int& c0, int64_t& r_lo,
                                         int64_t& r_hi) {
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  c0 = (blockIdx.x * kWave + lane) * kMixVec;
  const int64_t g_lo = (int64_t)blockIdx.y * p.rows_per_unit;
  const int64_t g_hi = min(p.rows, g_lo + p.rows_per_unit);
  const int64_t per_wave = (p.rows_per_unit + kWaves - 1) / kWaves;
  r_lo = min(g_hi, g_lo + w * per_wave);
  r_hi = min(g_hi, r_lo + per_wave);
  return c0 < p.D;
}

template <int DU, int DZ>
__global__ __launch_bounds__(kThreads) void mixer_out_fwd_vec_kernel(MixerOutParams p) {
  int c0;
  int64_t r_lo, r_hi;
  if (!vec_slot(p, c0, r_lo, r_hi)) return;
  float dk[kMixVec];
  load8f(p.Dskip, c0, dk);
  RowCursor cur(r_lo, p.L);
#pragma unroll 2
  for (int64_t r = r_lo; r < r_hi; ++r) {
    float u[kMixVec], z[kMixVec], y[kMixVec], o[kMixVec];
    load8<DU>(p.u, cur.at(p.usb, p.usl) + c0, u);
    load8<DZ>(p.z, cur.at(p.zsb, p.zsl) + c0, z);
    load8f(p.y, r * p.D + c0, y);
    cur.next(p.L);
#pragma unroll
    for (int k = 0; k < kMixVec; ++k) {
      float yk = y[k] + u[k] * dk[k];
      if (p.k_skip == 2) yk = yk + u[k] * dk[k];
      const float s = round_to(z[k] / (1.f + expf(-z[k])), DZ);
      o[k] = yk * s;
    }
    store8_rt(p.out, r * p.D + c0, o, p.dt_out);
  }
}

template <int DU, int DZ>
__global__ __launch_bounds__(kThreads) void mixer_out_bwd_vec_kernel(MixerOutParams p,
                                                                     MixerOutGrad g) {
  // per-wave dD partials of the workgroup's 512 channels, summed across
  // waves in a fixed order at the end
  __shared__ double sAcc[kWaves][kMixTile];
  int c0;
  int64_t r_lo, r_hi;
  const bool active = vec_slot(p, c0, r_lo, r_hi);
  double acc[kMixVec];
#pragma unroll
  for (int k = 0; k < kMixVec; ++k) acc[k] = 0.0;
  float dk[kMixVec];
  if (active) load8f(p.Dskip, c0, dk);
  RowCursor cur(r_lo, p.L);
#pragma unroll 2
  for (int64_t r = r_lo; active && r < r_hi; ++r) {
    float u[kMixVec], z[kMixVec], y[kMixVec], dout[kMixVec];
    load8<DU>(p.u, cur.at(p.usb, p.usl) + c0, u);
    load8<DZ>(p.z, cur.at(p.zsb, p.zsl) + c0, z);
    const int64_t i = r * p.D + c0;
    load8f(p.y, i, y);
    load8_rt(g.dout, i, dout, p.dt_out);
    cur.next(p.L);
    float dy[kMixVec], du[kMixVec], dz[kMixVec];
#pragma unroll
    for (int k = 0; k < kMixVec; ++k) {
      float yk = y[k] + u[k] * dk[k];
      if (p.k_skip == 2) yk = yk + u[k] * dk[k];
      const float e = expf(-z[k]);
      const float sig = 1.f / (1.f + e);
      const float s = round_to(z[k] / (1.f + e), DZ);
      const float dyk = dout[k] * s;
      const float ds = round_to(dout[k] * yk, DZ);
      dz[k] = ds * sig * (1.f + z[k] * (1.f - sig));
      dy[k] = dyk;
      const float du1 = round_to(dyk * dk[k], DU);
      du[k] = p.k_skip == 2 ? round_to(du1 + du1, DU) : du1;
      acc[k] += (double)(dyk * u[k]);
    }
    store8<RP_F32>(g.dy, i, dy);
    store8<DU>(g.du, i, du);
    store8<DZ>(g.dz, i, dz);
  }
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
#pragma unroll
  for (int k = 0; k < kMixVec; ++k) sAcc[w][lane * kMixVec + k] = acc[k];
  __syncthreads();
  // thread t: channels t and t + 256 of the tile
#pragma unroll
  for (int h = 0; h < kMixTile / kThreads; ++h) {
    const int j = threadIdx.x + h * kThreads;
    const int c = blockIdx.x * kMixTile + j;
    if (c < p.D)
      g.part[(int64_t)blockIdx.y * p.D + c] = ((sAcc[0][j] + sAcc[1][j]) + sAcc[2][j]) + sAcc[3][j];
  }
}

// Instantiation for the (u, z) storage dtypes.
#define RP_MIX_CASE(DU_, DZ_) \
  if (du == DU_ && dz == DZ_) return f(std::integral_constant<int, DU_>{}, std::integral_constant<int, DZ_>{})

template <typename F>
hipError_t with_mix_dtypes(int du, int dz, F&& f) {
  RP_MIX_CASE(RP_F32, RP_F32);
  RP_MIX_CASE(RP_F32, RP_BF16);
  RP_MIX_CASE(RP_F32, RP_F16);
  RP_MIX_CASE(RP_BF16, RP_F32);
  RP_MIX_CASE(RP_BF16, RP_BF16);
  RP_MIX_CASE(RP_BF16, RP_F16);
  RP_MIX_CASE(RP_F16, RP_F32);
  RP_MIX_CASE(RP_F16, RP_BF16);
  RP_MIX_CASE(RP_F16, RP_F16);
  return hipErrorInvalidValue;
}
#undef RP_MIX_CASE

// dD[c] = k * sum over row groups of the partials: wave w of a workgroup
// sums groups w, w + 4, ... for 64 channels (8 running sums, so that the
// loads overlap), then the waves' sums are added in a fixed order.
__global__ __launch_bounds__(kThreads) void mixer_out_reduce_kernel(const double* part, float* dD,
                                                                    int D, int units, int k) {
  __shared__ double sSum[kWaves][kWave];
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int c = blockIdx.x * kWave + lane;
  double a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (c < D) {
    int i = w;
    for (; i + 7 * kWaves < units; i += 8 * kWaves) {
#pragma unroll
      for (int q = 0; q < 8; ++q) a[q] += part[(int64_t)(i + q * kWaves) * D + c];
    }
    for (; i < units; i += kWaves) a[0] += part[(int64_t)i * D + c];
  }
  sSum[w][lane] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  __syncthreads();
  if (w == 0 && c < D) {
    const float s = (float)(((sSum[0][lane] + sSum[1][lane]) + sSum[2][lane]) + sSum[3][lane]);
    dD[c] = k == 2 ? s + s : s;
  }
}

hipError_t launch_mixer_out_fwd(const MixerOutParams& p, hipStream_t st) {
  if (p.vec) {
    dim3 grid((unsigned)((p.D + kMixTile - 1) / kMixTile), (unsigned)p.units);
    return with_mix_dtypes(p.dt_u, p.dt_z, [&](auto du, auto dz) {
      hipLaunchKernelGGL((mixer_out_fwd_vec_kernel<decltype(du)::value, decltype(dz)::value>),
                         grid, dim3(kThreads), 0, st, p);
      return hipGetLastError();
    });
  }
  dim3 grid((unsigned)((p.D + kThreads - 1) / kThreads), (unsigned)p.units);
  hipLaunchKernelGGL(mixer_out_fwd_kernel, grid, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_mixer_out_bwd(const MixerOutParams& p, const MixerOutGrad& g, hipStream_t st) {
  if (p.units > 0) {
    hipError_t e;
    if (p.vec) {
      dim3 grid((unsigned)((p.D + kMixTile - 1) / kMixTile), (unsigned)p.units);
      e = with_mix_dtypes(p.dt_u, p.dt_z, [&](auto du, auto dz) {
        hipLaunchKernelGGL((mixer_out_bwd_vec_kernel<decltype(du)::value, decltype(dz)::value>),
                           grid, dim3(kThreads), 0, st, p, g);
        return hipGetLastError();
      });
    } else {
      dim3 grid((unsigned)((p.D + kThreads - 1) / kThreads), (unsigned)p.units);
      hipLaunchKernelGGL(mixer_out_bwd_kernel, grid, dim3(kThreads), 0, st, p, g);
      e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(mixer_out_reduce_kernel, dim3((unsigned)((p.D + kWave - 1) / kWave)),
                     dim3(kThreads), 0, st, (const double*)g.part, g.dD, p.D, p.units, p.k_skip);
  return hipGetLastError();
}

}  // namespace rp
