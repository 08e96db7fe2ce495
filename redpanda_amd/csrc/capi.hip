// extern "C" boundary of libredpanda_hip: argument validation, workspace
// sizing, shape selection and launches.  No allocation, no blocking, no
// exceptions; failures return a negative status and set a thread-local
// message (rp_last_error).

#include <algorithm>
#include <atomic>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "redpanda_hip.h"
#include "rp_launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int fail_hip(hipError_t e, const char* what) {
  return fail(RP_ERR_LAUNCH, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

constexpr int64_t kI32Max = 0x7fffffff;

bool aligned(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Whether byte ranges [a, a + na) and [b, b + nb) intersect.
bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + (uintptr_t)nb && y < x + (uintptr_t)na;
}

int64_t elem_size(int dtype) { return dtype == RP_F32 ? 4 : 2; }

int64_t round_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// Lanes-per-channel override for tuning (RP_LANES_PER_CHANNEL=4, 8 or 16;
// a size the override cannot hold falls through to the next larger split).
int lanes_override() {
  static int v = [] {
    const char* s = getenv("RP_LANES_PER_CHANNEL");
    if (s == nullptr) return 0;
    const int x = atoi(s);
    return (x == 4 || x == 8 || x == 16) ? x : 0;
  }();
  return v;
}

// Rollouts per step workgroup (RP_STEP_RI overrides; 0 = automatic).
int step_ri_override() {
  static int v = [] {
    const char* s = getenv("RP_STEP_RI");
    const int x = s ? atoi(s) : 0;
    return (x >= 1 && x <= rp::kStepRiMax) ? x : 0;
  }();
  return v;
}

// Tiles per backward workgroup forced by RP_BWD_TPW (1-8, for measurements);
// 0: the plan's own choice.
int bwd_tpw_override() {
  static int v = [] {
    const char* s = getenv("RP_BWD_TPW");
    const int x = s ? atoi(s) : 0;
    return (x >= 1 && x <= 8) ? x : 0;
  }();
  return v;
}

struct Plan {
  int S, NPL, CB, ntiles, nck, ndir, bg, nbg, tpw, ntg;
  int gk;     // gate kind: rotational / tracking split fixed at compile time
  int64_t ckpt_bytes, part_bc_bytes, part_par_bytes;
  int64_t pd_bytes;    // the first direction's fp32 (d_delta, d_u) sums, when the outputs are 16-bit
  int64_t dcache_off;  // byte offset of the softplus(x) cache in the workspace, or -1
};

int scan_validate(const rp_scan_args* a) {
  if (a == nullptr) return fail(RP_ERR_INVALID, "scan args: NULL");
  if (a->B < 0 || a->L < 0 || a->D < 0 || a->NR < 0 || a->NT < 0)
    return fail(RP_ERR_INVALID, "scan args: negative size (B=%lld L=%lld D=%lld NR=%lld NT=%lld)",
                (long long)a->B, (long long)a->L, (long long)a->D, (long long)a->NR,
                (long long)a->NT);
  if (a->N != a->NR + a->NT)
    return fail(RP_ERR_INVALID, "scan args: N=%lld must equal NR+NT=%lld", (long long)a->N,
                (long long)(a->NR + a->NT));
  if (a->N < 1 || a->N > RP_MAX_STATE)
    return fail(RP_ERR_UNSUPPORTED, "scan args: N=%lld outside [1, %d]", (long long)a->N,
                RP_MAX_STATE);
  if (a->B > kI32Max || a->L > kI32Max || a->D > kI32Max)
    return fail(RP_ERR_UNSUPPORTED, "scan args: B, L, D must each fit in int32");
  const int codes[4] = {a->dtype_delta, a->dtype_u, a->dtype_B, a->dtype_C};
  for (int code : codes)
    if (code != RP_F32 && code != RP_BF16 && code != RP_F16)
      return fail(RP_ERR_INVALID, "scan args: unknown dtype code %d", code);
  if (a->delta_softplus != 0 && a->delta_softplus != 1)
    return fail(RP_ERR_INVALID, "scan args: delta_softplus must be 0 or 1");
  if (a->bidirectional != 0 && a->bidirectional != 1)
    return fail(RP_ERR_INVALID, "scan args: bidirectional must be 0 or 1");
  if (a->grad_in_storage != 0 && a->grad_in_storage != 1)
    return fail(RP_ERR_INVALID, "scan args: grad_in_storage must be 0 or 1");
  const int64_t work = a->B * a->L;
  if (work > 0 && a->D > 0) {
    if (!a->delta || !a->u || !a->Bc || !a->Cc)
      return fail(RP_ERR_INVALID, "scan args: NULL delta/u/Bc/Cc");
    if (!aligned(a->delta, elem_size(a->dtype_delta)) || !aligned(a->u, elem_size(a->dtype_u)) ||
        !aligned(a->Bc, elem_size(a->dtype_B)) || !aligned(a->Cc, elem_size(a->dtype_C)))
      return fail(RP_ERR_INVALID, "scan args: misaligned input pointer");
    if (a->delta_sb < 0 || a->delta_sl < 0 || a->u_sb < 0 || a->u_sl < 0 || a->Bc_sb < 0 ||
        a->Bc_sl < 0 || a->Cc_sb < 0 || a->Cc_sl < 0)
      return fail(RP_ERR_INVALID, "scan args: negative stride");
  }
  if (a->D > 0) {
    if (a->NR > 0 && (!a->A_real || !aligned(a->A_real, 4)))
      return fail(RP_ERR_INVALID, "scan args: NR>0 needs a 4-byte aligned A_real");
    if (a->NR > 0 && a->A_imag && !aligned(a->A_imag, 4))
      return fail(RP_ERR_INVALID, "scan args: misaligned A_imag");
    if (a->NR == 0 && a->A_imag)
      return fail(RP_ERR_INVALID, "scan args: A_imag given without rotational states");
    if (a->NT > 0 && (!a->track || !aligned(a->track, 4)))
      return fail(RP_ERR_INVALID, "scan args: NT>0 needs a 4-byte aligned track");
  }
  if ((a->h0 == nullptr) != (a->beta0 == nullptr))
    return fail(RP_ERR_INVALID, "scan args: h0 and beta0 go together");
  if (a->h0 != nullptr) {
    if (a->bidirectional)
      return fail(RP_ERR_INVALID, "scan args: an initial state needs a causal scan");
    if (a->L < 1) return fail(RP_ERR_INVALID, "scan args: an initial state needs L >= 1");
    if (!aligned(a->h0, 4) || !aligned(a->beta0, 4))
      return fail(RP_ERR_INVALID, "scan args: misaligned initial state");
  }
  return RP_OK;
}

Plan make_plan(const rp_scan_args* a) {
  Plan pl{};
  int S = 0, NPL = 0;
  rp::choose_shape((int)a->N, &S, &NPL);
  pl.S = S;
  pl.NPL = NPL;
  pl.CB = rp::kWaves * (rp::kWave / S);
  pl.gk = rp::gate_code_all(a->A_imag != nullptr, a->NR, a->N, S, NPL);
  pl.ntiles = (int)((a->D + pl.CB - 1) / pl.CB);
  const int64_t nchunks = (a->L + rp::kCkptK - 1) / rp::kCkptK;
  pl.nck = (int)(nchunks > 0 ? nchunks - 1 : 0);
  pl.ndir = a->bidirectional ? 2 : 1;
  // batch rows per backward workgroup: enough workgroups to fill 256 CUs
  // several times over, while amortising the parameter-gradient partials
  int64_t bg = (a->B * (int64_t)pl.ntiles) / 3072;
  if (bg < 1) bg = 1;
  if (bg > 8) bg = 8;
  pl.bg = (int)bg;
  pl.nbg = (int)((a->B + bg - 1) / bg);
  // adjacent channel tiles per backward workgroup: where a tile is 16
  // channels (16 lanes per channel), a workgroup walks 4 (or 2) tiles in
  // turn and their dB / dC partials add up in one block, so the partials
  // and the reduction's reads shrink by that factor, as long as the grid
  // keeps at least 1024 workgroups
  pl.tpw = 1;
  if (S == 16) {
    for (int t : {4, 2}) {
      if (pl.ntiles % t == 0 && (int64_t)(pl.ntiles / t) * pl.nbg >= 1024) {
        pl.tpw = t;
        break;
      }
    }
  }
  if (bwd_tpw_override() > 0 && S == 16) pl.tpw = bwd_tpw_override();
  pl.ntg = (pl.ntiles + pl.tpw - 1) / pl.tpw;
  pl.ckpt_bytes = (int64_t)pl.ndir * a->B * pl.nck * pl.ntiles * rp::kThreads * NPL * 4;
  // with softplus the forward also keeps delta = softplus(x) for the
  // backward, which then stages it as stored
  pl.dcache_off = -1;
  if (a->delta_softplus && a->B * a->L * a->D > 0) {
    pl.dcache_off = round_up(pl.ckpt_bytes, 256);
    pl.ckpt_bytes = pl.dcache_off + a->B * a->L * a->D * 4;
  }
  pl.part_bc_bytes = round_up(2 * (int64_t)pl.ntg * a->B * a->L * a->N * 4, 256);
  pl.part_par_bytes = round_up((int64_t)pl.nbg * 2 * a->D * a->N * 8, 256);
  pl.pd_bytes = 0;
  if (a->grad_in_storage && pl.ndir == 2 && (a->dtype_delta != RP_F32 || a->dtype_u != RP_F32))
    pl.pd_bytes = round_up(2 * a->B * a->L * a->D * 4, 256);
  return pl;
}

rp::ScanParams scan_params(const rp_scan_args* a, const Plan& pl) {
  rp::ScanParams p{};
  p.delta = a->delta;
  p.u = a->u;
  p.Bc = a->Bc;
  p.Cc = a->Cc;
  p.dsb = a->delta_sb;
  p.dsl = a->delta_sl;
  p.usb = a->u_sb;
  p.usl = a->u_sl;
  p.bsb = a->Bc_sb;
  p.bsl = a->Bc_sl;
  p.csb = a->Cc_sb;
  p.csl = a->Cc_sl;
  p.Ar = a->NR > 0 ? a->A_real : nullptr;
  p.Ai = a->NR > 0 ? a->A_imag : nullptr;
  p.Tk = a->NT > 0 ? a->track : nullptr;
  p.h0 = a->h0;
  p.beta0 = a->beta0;
  p.B = (int)a->B;
  p.L = (int)a->L;
  p.D = (int)a->D;
  p.N = (int)a->N;
  p.NR = (int)a->NR;
  p.NT = (int)a->NT;
  p.dt_delta = a->dtype_delta;
  p.dsp = a->delta_softplus;
  p.dt_u = a->dtype_u;
  p.dt_B = a->dtype_B;
  p.dt_C = a->dtype_C;
  p.ndir = pl.ndir;
  p.ntiles = pl.ntiles;
  p.nck = pl.nck;
  return p;
}

}  // namespace

namespace rp {

bool choose_shape(int N, int* S, int* NPL) {
  // lanes per channel grow with the state size so that a lane holds at most
  // a handful of states (the backward keeps K steps of three per-state
  // values in registers); 16-lane rows keep every channel inside one row
  static const int npl4[] = {1, 2, 3, 4, 5};
  static const int npl8[] = {3, 4, 5};
  static const int npl16[] = {3, 4, 5, 6, 8};
  const int force = lanes_override();
  if ((force == 0 && N <= 20) || force == 4) {
    for (int v : npl4)
      if (4 * v >= N) {
        *S = 4;
        *NPL = v;
        return true;
      }
  }
  if ((force == 0 && N <= 40) || force == 8) {
    for (int v : npl8)
      if (8 * v >= N) {
        *S = 8;
        *NPL = v;
        return true;
      }
  }
  for (int v : npl16)
    if (16 * v >= N) {
      *S = 16;
      *NPL = v;
      return true;
    }
  return false;
}

}  // namespace rp

extern "C" {

int rp_abi_version(void) { return RP_ABI_VERSION; }

const char* rp_last_error(void) { return g_err; }

int rp_scan_check(const rp_scan_args* a) { return scan_validate(a); }

int64_t rp_scan_ckpt_bytes(const rp_scan_args* a) {
  if (scan_validate(a) != RP_OK) return -1;
  return make_plan(a).ckpt_bytes;
}

int64_t rp_scan_bwd_work_bytes(const rp_scan_args* a) {
  if (scan_validate(a) != RP_OK) return -1;
  const Plan pl = make_plan(a);
  return pl.part_bc_bytes + pl.part_par_bytes + pl.pd_bytes;
}

int rp_scan_fwd(const rp_scan_args* a, const rp_scan_fwd_out* out, void* stream) {
  int st = scan_validate(a);
  if (st != RP_OK) return st;
  if (out == nullptr) return fail(RP_ERR_INVALID, "scan fwd: NULL output block");
  const int64_t work = a->B * a->L * a->D;
  if (work > 0 && (!out->y || !aligned(out->y, 4)))
    return fail(RP_ERR_INVALID, "scan fwd: NULL or misaligned y");
  if ((out->h_last == nullptr) != (out->beta_last == nullptr))
    return fail(RP_ERR_INVALID, "scan fwd: h_last and beta_last go together");
  if (out->h_last && a->bidirectional)
    return fail(RP_ERR_INVALID, "scan fwd: the final state exists for causal scans only");
  const Plan pl = make_plan(a);
  if (out->ckpt && pl.ckpt_bytes > 0 && !aligned(out->ckpt, 256))
    return fail(RP_ERR_INVALID, "scan fwd: checkpoint workspace must be 256-byte aligned");
  if (a->B == 0 || a->D == 0) return RP_OK;
  if (a->L == 0) {
    if (out->h_last) {
      const int64_t ne = a->B * a->D * a->N;
      hipError_t e = rp::launch_fill_zero(out->h_last, ne, (hipStream_t)stream);
      if (e == hipSuccess) e = rp::launch_fill_zero(out->beta_last, ne, (hipStream_t)stream);
      if (e != hipSuccess) return fail_hip(e, "scan fwd: zero final state");
    }
    return RP_OK;
  }
  if ((int64_t)pl.ntiles * a->B > kI32Max)
    return fail(RP_ERR_UNSUPPORTED, "scan fwd: grid too large");
  const rp::ScanParams p = scan_params(a, pl);
  float* ck = pl.ckpt_bytes > 0 ? out->ckpt : nullptr;
  float* dc = (ck != nullptr && pl.dcache_off >= 0)
                  ? reinterpret_cast<float*>(reinterpret_cast<char*>(ck) + pl.dcache_off)
                  : nullptr;
  rp::FwdOut o{out->y, ck, out->h_last, out->beta_last, dc};
  hipError_t e = rp::launch_scan_fwd(pl.S, pl.NPL, pl.gk, p, o, (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "scan fwd launch");
  return RP_OK;
}

}  // extern "C"

// Scratch of rp_scan_bwd_noalloc: one static device array, each GPU holding
// its own copy at its own address for as long as the process runs.  Host code
// uses the array only to look that address up (hipGetSymbolAddress, once per
// device); everything else goes through the looked-up device pointer.
static __device__ __align__(256) unsigned char scratch[RP_SCAN_BWD_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The device address of `scratch` on the device that `stream` runs on.
int scratch_for_stream(hipStream_t stream, void** out) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return fail_hip(e, "scan bwd noalloc: hipGetDevice");
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sd = 0;
    e = hipStreamGetDevice(stream, &sd);
    if (e != hipSuccess) return fail_hip(e, "scan bwd noalloc: hipStreamGetDevice");
    dev = (int)sd;
  }
  if (dev < 0 || dev >= kMaxDevices)
    return fail(RP_ERR_UNSUPPORTED, "scan bwd noalloc: device %d beyond %d", dev, kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      // with the stream's device current, as the lookup is per device
      if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
        return fail_hip(e, "scan bwd noalloc: hipSetDevice");
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      hipError_t e2 = dev != cur ? hipSetDevice(cur) : hipSuccess;
      if (e != hipSuccess) return fail_hip(e, "scan bwd noalloc: hipGetSymbolAddress(scratch)");
      if (e2 != hipSuccess) return fail_hip(e2, "scan bwd noalloc: hipSetDevice (restore)");
      if (p == nullptr) return fail(RP_ERR_LAUNCH, "scan bwd noalloc: scratch has no address");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return RP_OK;
}

// rp_scan_bwd with its scratch given: the caller's workspace (use_io_work)
// or the static scratch of rp_scan_bwd_noalloc.
int scan_bwd_impl(const rp_scan_args* a, const rp_scan_bwd_io* io, void* stream,
                  bool use_io_work) {
  int st = scan_validate(a);
  if (st != RP_OK) return st;
  if (io == nullptr) return fail(RP_ERR_INVALID, "scan bwd: NULL io block");
  const Plan pl = make_plan(a);
  const int64_t need = pl.part_bc_bytes + pl.part_par_bytes + pl.pd_bytes;
  const int64_t work = a->B * a->L * a->D;
  const int dt_dd = a->grad_in_storage ? a->dtype_delta : RP_F32;
  const int dt_du = a->grad_in_storage ? a->dtype_u : RP_F32;
  if (work > 0) {
    if (!io->dy || !io->d_delta || !io->d_u)
      return fail(RP_ERR_INVALID, "scan bwd: NULL dy / d_delta / d_u");
    if (!aligned(io->d_delta, elem_size(dt_dd)) || !aligned(io->d_u, elem_size(dt_du)))
      return fail(RP_ERR_INVALID, "scan bwd: misaligned d_delta / d_u");
    if (pl.ckpt_bytes > 0 && (!io->ckpt || !aligned(io->ckpt, 256)))
      return fail(RP_ERR_INVALID,
                  "scan bwd: 256-byte aligned checkpoint workspace required for L=%lld",
                  (long long)a->L);
  }
  if (a->B * a->L > 0 && (!io->d_Bc || !io->d_Cc))
    return fail(RP_ERR_INVALID, "scan bwd: NULL d_Bc / d_Cc");
  if (a->D > 0) {
    if (a->NR > 0 && !io->d_A_real) return fail(RP_ERR_INVALID, "scan bwd: NULL d_A_real");
    if (a->NR > 0 && a->A_imag && !io->d_A_imag)
      return fail(RP_ERR_INVALID, "scan bwd: NULL d_A_imag");
    if (a->NT > 0 && !io->d_track) return fail(RP_ERR_INVALID, "scan bwd: NULL d_track");
  }
  if ((io->d_h0 == nullptr) != (io->d_beta0 == nullptr))
    return fail(RP_ERR_INVALID, "scan bwd: d_h0 and d_beta0 go together");
  if (io->d_h0 && !a->h0)
    return fail(RP_ERR_INVALID, "scan bwd: d_h0 needs an initial state h0");
  if ((io->dh_last || io->dbeta_last) && a->bidirectional)
    return fail(RP_ERR_INVALID, "scan bwd: final-state gradients exist for causal scans only");
  void* scr = nullptr;
  if (use_io_work) {
    if (need > 0 && (io->work == nullptr || io->work_bytes < need || !aligned(io->work, 256)))
      return fail(RP_ERR_WORKSPACE, "scan bwd: workspace needs %lld bytes (256-aligned), got %lld",
                  (long long)need, (long long)io->work_bytes);
    scr = io->work;
  } else if (need > 0) {
    if (need > RP_SCAN_BWD_SCRATCH_BYTES)
      return fail(RP_ERR_WORKSPACE,
                  "scan bwd noalloc: this shape needs %lld bytes of scratch, the static scratch "
                  "holds %lld; use rp_scan_bwd with a workspace of rp_scan_bwd_work_bytes()",
                  (long long)need, (long long)RP_SCAN_BWD_SCRATCH_BYTES);
    st = scratch_for_stream((hipStream_t)stream, &scr);
    if (st != RP_OK) return st;
  }
  if (a->D == 0) return RP_OK;
  if ((int64_t)pl.ntg * pl.nbg > kI32Max)
    return fail(RP_ERR_UNSUPPORTED, "scan bwd: grid too large");
  const rp::ScanParams p = scan_params(a, pl);
  rp::BwdIO b{};
  b.dy = io->dy;
  b.ckpt = io->ckpt;
  b.dcache = pl.dcache_off >= 0
                 ? reinterpret_cast<const float*>(reinterpret_cast<const char*>(io->ckpt) +
                                                  pl.dcache_off)
                 : nullptr;
  b.dh_last = io->dh_last;
  b.dbeta_last = io->dbeta_last;
  b.d_h0 = io->d_h0;
  b.d_beta0 = io->d_beta0;
  b.d_delta = io->d_delta;
  b.d_u = io->d_u;
  b.dt_dd = dt_dd;
  b.dt_du = dt_du;
  b.part_bc = static_cast<float*>(scr);
  b.part_par = reinterpret_cast<double*>(static_cast<char*>(scr) + pl.part_bc_bytes);
  if (pl.pd_bytes > 0) {
    // the first direction's sums in the workspace, behind the partials
    b.pd_delta = reinterpret_cast<float*>(static_cast<char*>(scr) + pl.part_bc_bytes +
                                          pl.part_par_bytes);
    b.pd_u = b.pd_delta + a->B * a->L * a->D;
  } else {
    b.pd_delta = static_cast<float*>(io->d_delta);
    b.pd_u = static_cast<float*>(io->d_u);
  }
  b.bg = pl.bg;
  b.nbg = pl.nbg;
  b.tpw = pl.tpw;
  b.ntg = pl.ntg;
  hipStream_t s = (hipStream_t)stream;
  if (a->B > 0) {
    hipError_t e = rp::launch_scan_bwd(pl.S, pl.NPL, pl.gk, p, b, s);
    if (e != hipSuccess) return fail_hip(e, "scan bwd launch");
  }
  hipError_t e = rp::launch_bwd_finalize(p, b, io->d_Bc, io->d_Cc,
                                         a->NR > 0 ? io->d_A_real : nullptr,
                                         (a->NR > 0 && a->A_imag) ? io->d_A_imag : nullptr,
                                         a->NT > 0 ? io->d_track : nullptr, s);
  if (e != hipSuccess) return fail_hip(e, "scan bwd finalize launch");
  return RP_OK;
}

}  // namespace

extern "C" {

int rp_scan_bwd(const rp_scan_args* a, const rp_scan_bwd_io* io, void* stream) {
  return scan_bwd_impl(a, io, stream, true);
}

int rp_scan_bwd_noalloc(const rp_scan_args* a, const rp_scan_bwd_io* io, void* stream) {
  return scan_bwd_impl(a, io, stream, false);
}

int rp_step_check(const rp_step_args* a) {
  if (a == nullptr) return fail(RP_ERR_INVALID, "step args: NULL");
  if (a->R < 0 || a->D < 0 || a->NR < 0 || a->NT < 0)
    return fail(RP_ERR_INVALID, "step args: negative size");
  if (a->N != a->NR + a->NT) return fail(RP_ERR_INVALID, "step args: N must equal NR+NT");
  if (a->N < 1 || a->N > RP_MAX_STATE)
    return fail(RP_ERR_UNSUPPORTED, "step args: N=%lld outside [1, %d]", (long long)a->N,
                RP_MAX_STATE);
  if (a->R > kI32Max || a->D > kI32Max)
    return fail(RP_ERR_UNSUPPORTED, "step args: R and D must fit in int32");
  if (a->R == 0 || a->D == 0) return RP_OK;
  if (!a->delta || !a->u || !a->Bc || !a->Cc || !a->Dskip || !a->h_out || !a->beta_out || !a->y)
    return fail(RP_ERR_INVALID, "step args: NULL required pointer");
  if ((a->h_in == nullptr) != (a->beta_in == nullptr))
    return fail(RP_ERR_INVALID, "step args: h_in and beta_in go together");
  if ((a->broadcast_state != 0 && a->broadcast_state != 1) ||
      (a->delta_softplus != 0 && a->delta_softplus != 1) ||
      (a->beta_rank1 != 0 && a->beta_rank1 != 1) || a->reserved != 0)
    return fail(RP_ERR_INVALID,
                "step args: broadcast_state, delta_softplus and beta_rank1 must be 0 or 1, "
                "reserved 0");
  if (a->broadcast_state && a->h_in == nullptr)
    return fail(RP_ERR_INVALID, "step args: broadcast_state needs h_in / beta_in");
  {
    // bytes of the input and output h and beta blocks
    const int64_t rows_in = a->broadcast_state ? 1 : a->R;
    const int64_t h_in_b = rows_in * a->D * a->N * 4, h_out_b = a->R * a->D * a->N * 4;
    const int64_t bw = a->beta_rank1 ? a->D + a->N : a->D * a->N;
    const int64_t b_in_b = rows_in * bw * 4, b_out_b = a->R * bw * 4;
    if (a->broadcast_state) {
      // every rollout reads the one input state while others write theirs
      if (overlaps(a->h_in, h_in_b, a->h_out, h_out_b) ||
          overlaps(a->h_in, h_in_b, a->beta_out, b_out_b) ||
          overlaps(a->beta_in, b_in_b, a->h_out, h_out_b) ||
          overlaps(a->beta_in, b_in_b, a->beta_out, b_out_b))
        return fail(RP_ERR_INVALID, "step args: a broadcast input state overlaps an output");
    }
    // a rank-1 row's B part is read by every channel tile of the rollout
    if (a->beta_rank1 && a->h_in && overlaps(a->beta_in, b_in_b, a->beta_out, b_out_b))
      return fail(RP_ERR_INVALID, "step args: rank-1 beta_out must not overlap beta_in");
  }
  if (a->reserved2 != 0) return fail(RP_ERR_INVALID, "step args: reserved2 must be 0");
  if (a->z != nullptr) {
    if (a->dtype_z != RP_F32 && a->dtype_z != RP_BF16 && a->dtype_z != RP_F16)
      return fail(RP_ERR_INVALID, "step args: unknown dtype code %d for z", a->dtype_z);
    if (a->z_sr < a->D || !aligned(a->z, elem_size(a->dtype_z)))
      return fail(RP_ERR_INVALID, "step args: z row stride shorter than D or z misaligned");
  }
  if (a->NR > 0 && !a->A_real) return fail(RP_ERR_INVALID, "step args: NR>0 needs A_real");
  if (a->NR == 0 && a->A_imag) return fail(RP_ERR_INVALID, "step args: A_imag without NR");
  if (a->NT > 0 && !a->track) return fail(RP_ERR_INVALID, "step args: NT>0 needs track");
  if (a->delta_sr < a->D || a->u_sr < a->D || a->Bc_sr < a->N || a->Cc_sr < a->N)
    return fail(RP_ERR_INVALID, "step args: row stride shorter than the row");
  const void* ptrs[] = {a->delta, a->u, a->Bc, a->Cc, a->h_in, a->beta_in, a->A_real,
                        a->A_imag, a->track, a->Dskip, a->h_out, a->beta_out, a->y};
  for (const void* q : ptrs)
    if (q && !aligned(q, 4)) return fail(RP_ERR_INVALID, "step args: misaligned pointer");
  return RP_OK;
}

}  // extern "C"

namespace {

// rp_step, and with bn the B / C rows from the raw projections: computed in
// the tile kernel's prologue when it takes one rollout per workgroup (small
// batches, where a launch saved is worth most), else by the BCNorm kernel
// into bn->Bc / bn->Cc (= a->Bc / a->Cc) ahead of the step.
int step_impl(const rp_step_args* a, const rp_bcnorm_args* bn, void* stream) {
  int st = rp_step_check(a);
  if (st != RP_OK) return st;
  if (bn != nullptr) {
    st = rp_bcnorm_check(bn);
    if (st != RP_OK) return st;
    if (bn->T != a->R || bn->N != a->N)
      return fail(RP_ERR_INVALID, "step bcnorm: T must be R and N the step's d_state");
    if (bn->Bc != a->Bc || bn->Cc != a->Cc || a->Bc_sr != a->N || a->Cc_sr != a->N)
      return fail(RP_ERR_INVALID, "step bcnorm: a->Bc / a->Cc must be bn->Bc / bn->Cc, row stride N");
  }
  if (a->R == 0 || a->D == 0) return RP_OK;
  int S = 0, NPL = 0;
  rp::choose_shape((int)a->N, &S, &NPL);
  const int CB = rp::kWaves * (rp::kWave / S);
  rp::StepParams p{};
  p.R = (int)a->R;
  p.D = (int)a->D;
  p.N = (int)a->N;
  p.NR = (int)a->NR;
  p.NT = (int)a->NT;
  p.delta = a->delta;
  p.dsr = a->delta_sr;
  p.u = a->u;
  p.usr = a->u_sr;
  p.Bc = a->Bc;
  p.bsr = a->Bc_sr;
  p.Cc = a->Cc;
  p.csr = a->Cc_sr;
  p.h_in = a->h_in;
  p.beta_in = a->beta_in;
  p.ssr = a->broadcast_state ? 0 : a->D * a->N;
  p.dsp = a->delta_softplus;
  p.rank1 = a->beta_rank1;
  p.bssr = a->broadcast_state ? 0 : a->D + a->N;
  p.z = a->z;
  p.zsr = a->z_sr;
  p.dt_z = a->dtype_z;
  p.Ar = a->NR > 0 ? a->A_real : nullptr;
  p.Ai = a->NR > 0 ? a->A_imag : nullptr;
  p.Tk = a->NT > 0 ? a->track : nullptr;
  p.Dskip = a->Dskip;
  p.h_out = a->h_out;
  p.beta_out = a->beta_out;
  p.y = a->y;
  p.ntiles = (int)((a->D + CB - 1) / CB);
  if ((int64_t)p.ntiles * a->R > kI32Max)
    return fail(RP_ERR_UNSUPPORTED, "step: grid too large");

  // the tile kernel moves each channel's (h, beta) as 16-byte vectors (with
  // pad states when N is below the shape's S * NPL)
  // (pad states only in the last slot, or anywhere with two slices per
  // thread, whose vectors are checked one by one)
  const bool tile = a->N % 4 == 0 && rp::step_tile_shape(S, NPL) &&
                    (a->N == S * NPL || a->N > S * (NPL - 1) ||
                     rp::step_tile_split(S, NPL) * 2 == S) &&
                    aligned(a->h_out, 16) &&
                    (a->h_in == nullptr || aligned(a->h_in, 16)) &&
                    (a->beta_rank1 || (aligned(a->beta_out, 16) &&
                                       (a->h_in == nullptr || aligned(a->beta_in, 16))));
  if (tile) {
    const int tch = rp::kStepTile / rp::step_tile_split(S, NPL);
    p.ctiles = (int)((a->D + tch - 1) / tch);
    // rollouts per workgroup: a few amortise the workgroup's prologue (gate
    // parameters, B / C rows) while keeping many workgroups in flight;
    // measured at 4096 rollouts x 1024 channels, d_state 20: 4 per workgroup
    // (4096 workgroups) beat 1..3 and 6..32 with the full beta; with rank-1
    // rows (half the bytes per rollout) 8 beat 1..4 and 16.  Below those
    // caps the count aims at about 512 workgroups, so that fewer rollouts
    // still amortise the prologue: at 512 rollouts, 4 per workgroup (512
    // workgroups) take 42 us full / 27 us rank-1, where 1 per workgroup
    // (2048) took 55 / 47 us
    const int64_t ri_max = a->beta_rank1 ? 8 : 4;
    int64_t ri = step_ri_override();
    if (ri == 0) {
      ri = (a->R * (int64_t)p.ctiles) / 512;
      if (ri < 1) ri = 1;
      if (ri > ri_max) ri = ri_max;
    }
    if (ri > rp::step_tile_ri_max(S, NPL, a->beta_rank1 != 0))
      return fail(RP_ERR_UNSUPPORTED, "step: rollouts per workgroup");
    p.ri = (int)ri;
    p.rgroups = (int)((a->R + ri - 1) / ri);
    if ((int64_t)p.ctiles * p.rgroups > kI32Max)
      return fail(RP_ERR_UNSUPPORTED, "step: grid too large");
  }
  // the tile kernel's all-rotational gate kind: no slot's split decided at
  // run time (the default configurations: d_state 32 and 64, no tracking);
  // the lane-layout kernel takes RotLead for it
  const int gk_launch = rp::gate_code_all(a->A_imag != nullptr, a->NR, a->N, S, NPL);
  // (the prologue's BCNorm takes a state per lane: d_state <= 64)
  if (bn != nullptr && tile && p.ri == 1 && a->N <= rp::kWave) {
    p.bn_fused = 1;
    p.bn_x[0] = bn->B_raw;
    p.bn_x[1] = bn->C_raw;
    p.bn_xs[0] = bn->B_sr;
    p.bn_xs[1] = bn->C_sr;
    p.bn_dt = bn->dtype_x;
    p.bn_w[0] = bn->wB;
    p.bn_w[1] = bn->wC;
    p.bn_P = (int)bn->P;
    p.bn_normalize = bn->normalize;
    p.bn_eps = bn->eps;
  } else if (bn != nullptr) {
    st = rp_bcnorm_fwd(bn, stream);
    if (st != RP_OK) return st;
  }
  hipError_t e = rp::launch_step(S, NPL, gk_launch, tile, p, (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "step launch");
  return RP_OK;
}

}  // namespace

extern "C" {

int rp_step(const rp_step_args* a, void* stream) { return step_impl(a, nullptr, stream); }

int rp_step_bcnorm(const rp_step_args* a, const rp_bcnorm_args* bn, void* stream) {
  if (bn == nullptr) return fail(RP_ERR_INVALID, "step bcnorm: NULL bcnorm args");
  return step_impl(a, bn, stream);
}

}  // extern "C"

// ── mixer output gate ──

namespace {

struct MixPlan {
  int64_t rows, rows_per_unit;
  int units, vec;
};

// Row units (each with its own dD partial): enough workgroups, with the
// channel tiles, to fill the chip a few times over.  A fixed function of the
// shape and path, so dD sums the same partials in the same order every call.
MixPlan mixer_plan(const rp_mixer_out_args* a, bool vec, int workgroups) {
  MixPlan m{};
  m.vec = vec ? 1 : 0;
  m.rows = a->B * a->L;
  if (m.rows == 0 || a->D == 0) return m;
  const int64_t tile = vec ? rp::kMixTile : rp::kThreads;
  const int64_t ctiles = (a->D + tile - 1) / tile;
  int64_t units = (workgroups + ctiles - 1) / ctiles;
  units = units < 1 ? 1 : (units > m.rows ? m.rows : units);
  m.rows_per_unit = (m.rows + units - 1) / units;
  m.units = (int)((m.rows + m.rows_per_unit - 1) / m.rows_per_unit);
  return m;
}

// Whether every row of every operand starts on 16 bytes, so that a lane can
// move 8 channels of each with one or two 16-byte accesses.
bool mixer_vec_ok(const rp_mixer_out_args* a, const rp_mixer_out_grad* g) {
  if (a->D % rp::kMixVec != 0) return false;
  const int64_t qu = 16 / elem_size(a->dtype_u), qz = 16 / elem_size(a->dtype_z);
  if (a->u_sb % qu || a->u_sl % qu || a->z_sb % qz || a->z_sl % qz) return false;
  const void* ptrs[] = {a->y, a->u, a->z, a->Dskip, a->out};
  for (const void* q : ptrs)
    if (q && !aligned(q, 16)) return false;
  if (g != nullptr) {
    const void* gp[] = {g->dout, g->dy, g->du, g->dz};
    for (const void* q : gp)
      if (!aligned(q, 16)) return false;
  }
  return true;
}

rp::MixerOutParams mixer_params(const rp_mixer_out_args* a, const MixPlan& m) {
  rp::MixerOutParams p{};
  p.rows = m.rows;
  p.L = (int)a->L;
  p.D = (int)a->D;
  p.k_skip = a->k_skip;
  p.dt_u = a->dtype_u;
  p.dt_z = a->dtype_z;
  p.y = a->y;
  p.u = a->u;
  p.usb = a->u_sb;
  p.usl = a->u_sl;
  p.z = a->z;
  p.zsb = a->z_sb;
  p.zsl = a->z_sl;
  p.Dskip = a->Dskip;
  p.out = a->out;
  p.dt_out = a->dtype_out;
  p.rows_per_unit = m.rows_per_unit;
  p.units = m.units;
  p.vec = m.vec;
  return p;
}

// Byte span of a (B, L, D) view with the given strides (elements) and size.
int64_t span_bytes(const rp_mixer_out_args* a, int64_t sb, int64_t sl, int64_t es) {
  return ((a->B - 1) * sb + (a->L - 1) * sl + a->D) * es;
}

}  // namespace

extern "C" {

int rp_mixer_out_check(const rp_mixer_out_args* a) {
  if (a == nullptr) return fail(RP_ERR_INVALID, "mixer out args: NULL");
  if (a->B < 0 || a->L < 0 || a->D < 0)
    return fail(RP_ERR_INVALID, "mixer out args: negative size");
  if (a->B > kI32Max || a->L > kI32Max || a->D > kI32Max)
    return fail(RP_ERR_UNSUPPORTED, "mixer out args: B, L, D must each fit in int32");
  if (a->k_skip != 1 && a->k_skip != 2)
    return fail(RP_ERR_INVALID, "mixer out args: k_skip must be 1 or 2");
  const int codes[3] = {a->dtype_u, a->dtype_z, a->dtype_out};
  for (int code : codes)
    if (code != RP_F32 && code != RP_BF16 && code != RP_F16)
      return fail(RP_ERR_INVALID, "mixer out args: unknown dtype code %d", code);
  if (a->B * a->L == 0 || a->D == 0) return RP_OK;
  if (!a->y || !a->u || !a->z || !a->Dskip)
    return fail(RP_ERR_INVALID, "mixer out args: NULL y/u/z/Dskip");
  if (!aligned(a->y, 4) || !aligned(a->Dskip, 4) || !aligned(a->out, elem_size(a->dtype_out)) ||
      !aligned(a->u, elem_size(a->dtype_u)) || !aligned(a->z, elem_size(a->dtype_z)))
    return fail(RP_ERR_INVALID, "mixer out args: misaligned pointer");
  if (a->u_sb < 0 || a->u_sl < 0 || a->z_sb < 0 || a->z_sl < 0)
    return fail(RP_ERR_INVALID, "mixer out args: negative stride");
  // out is written once per element after that element's inputs are read:
  // it may be y itself (fp32), but must not overlap u or z
  if (a->out == nullptr) return RP_OK;  // the backward reads no out
  const int64_t dense = a->B * a->L * a->D * 4;
  const int64_t out_b = a->B * a->L * a->D * elem_size(a->dtype_out);
  if (overlaps(a->out, out_b, a->u, span_bytes(a, a->u_sb, a->u_sl, elem_size(a->dtype_u))) ||
      overlaps(a->out, out_b, a->z, span_bytes(a, a->z_sb, a->z_sl, elem_size(a->dtype_z))))
    return fail(RP_ERR_INVALID, "mixer out args: out overlaps u or z");
  if (!(a->out == a->y && a->dtype_out == RP_F32) && overlaps(a->out, out_b, a->y, dense))
    return fail(RP_ERR_INVALID, "mixer out args: out partly overlaps y");
  return RP_OK;
}

int64_t rp_mixer_out_work_bytes(const rp_mixer_out_args* a) {
  if (rp_mixer_out_check(a) != RP_OK) return -1;
  // enough for either path (the backward picks one from its pointers too)
  const int64_t units = std::max(mixer_plan(a, true, rp::kMixerBwdWorkgroups).units,
                                 mixer_plan(a, false, rp::kMixerBwdWorkgroups).units);
  return round_up(units * a->D * (int64_t)sizeof(double), 256);
}

int rp_mixer_out_fwd(const rp_mixer_out_args* a, void* stream) {
  int st = rp_mixer_out_check(a);
  if (st != RP_OK) return st;
  const MixPlan m = mixer_plan(a, mixer_vec_ok(a, nullptr), rp::kMixerFwdWorkgroups);
  if (m.units == 0) return RP_OK;
  if (a->out == nullptr) return fail(RP_ERR_INVALID, "mixer out fwd: NULL out");
  hipError_t e = rp::launch_mixer_out_fwd(mixer_params(a, m), (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "mixer out fwd launch");
  return RP_OK;
}

int rp_mixer_out_bwd(const rp_mixer_out_args* a, const rp_mixer_out_grad* g, void* stream) {
  int st = rp_mixer_out_check(a);
  if (st != RP_OK) return st;
  if (g == nullptr) return fail(RP_ERR_INVALID, "mixer out grad: NULL");
  if (a->D == 0) return RP_OK;
  if (!g->dD || !aligned(g->dD, 4)) return fail(RP_ERR_INVALID, "mixer out grad: NULL or misaligned dD");
  rp::MixerOutGrad mg{};
  mg.dD = g->dD;
  if (a->B * a->L == 0) {
    const MixPlan m = mixer_plan(a, false, rp::kMixerBwdWorkgroups);
    // no rows: dD is a sum over nothing (written by a kernel, so that the
    // call stays capturable)
    hipError_t e = rp::launch_mixer_out_bwd(mixer_params(a, m), mg, (hipStream_t)stream);
    if (e != hipSuccess) return fail_hip(e, "mixer out bwd launch");
    return RP_OK;
  }
  if (!g->dout || !g->dy || !g->du || !g->dz)
    return fail(RP_ERR_INVALID, "mixer out grad: NULL dout/dy/du/dz");
  if (!aligned(g->dout, elem_size(a->dtype_out)) || !aligned(g->dy, 4) ||
      !aligned(g->du, elem_size(a->dtype_u)) ||
      !aligned(g->dz, elem_size(a->dtype_z)))
    return fail(RP_ERR_INVALID, "mixer out grad: misaligned pointer");
  const int64_t n = a->B * a->L * a->D;
  const int64_t ubytes = span_bytes(a, a->u_sb, a->u_sl, elem_size(a->dtype_u));
  const int64_t zbytes = span_bytes(a, a->z_sb, a->z_sl, elem_size(a->dtype_z));
  struct Span { const void* p; int64_t n; };
  // outputs: disjoint from each other and from every input (dy may be dout itself)
  const Span outs[4] = {{g->dy, n * 4}, {g->du, n * elem_size(a->dtype_u)},
                        {g->dz, n * elem_size(a->dtype_z)}, {g->dD, a->D * 4}};
  const Span ins[5] = {{a->y, n * 4}, {a->u, ubytes}, {a->z, zbytes}, {a->Dskip, a->D * 4},
                       {g->dout, n * elem_size(a->dtype_out)}};
  for (int i = 0; i < 4; ++i) {
    for (int j = i + 1; j < 4; ++j)
      if (overlaps(outs[i].p, outs[i].n, outs[j].p, outs[j].n))
        return fail(RP_ERR_INVALID, "mixer out grad: outputs overlap");
    for (int j = 0; j < 5; ++j) {
      if (i == 0 && j == 4 && g->dy == g->dout && a->dtype_out == RP_F32) continue;
      if (overlaps(outs[i].p, outs[i].n, ins[j].p, ins[j].n))
        return fail(RP_ERR_INVALID, "mixer out grad: an output overlaps an input");
    }
  }
  const MixPlan m = mixer_plan(a, mixer_vec_ok(a, g), rp::kMixerBwdWorkgroups);
  const int64_t need = rp_mixer_out_work_bytes(a);
  if (g->work == nullptr || g->work_bytes < need || !aligned(g->work, 256))
    return fail(RP_ERR_WORKSPACE, "mixer out bwd: workspace needs %lld bytes (256-aligned), got %lld",
                (long long)need, (long long)g->work_bytes);
  mg.dout = g->dout;
  mg.dy = g->dy;
  mg.du = g->du;
  mg.dz = g->dz;
  mg.part = static_cast<double*>(g->work);
  hipError_t e = rp::launch_mixer_out_bwd(mixer_params(a, m), mg, (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "mixer out bwd launch");
  return RP_OK;
}

}  // extern "C"

// ── BCNorm + p-sum ──

namespace {

rp::BcNormParams bcnorm_params(const rp_bcnorm_args* a) {
  rp::BcNormParams p{};
  p.T = a->T;
  p.N = (int)a->N;
  p.P = (int)a->P;
  p.dt_x = a->dtype_x;
  p.normalize = a->normalize;
  p.eps = a->eps;
  p.x[0] = a->B_raw;
  p.x[1] = a->C_raw;
  p.xs[0] = a->B_sr;
  p.xs[1] = a->C_sr;
  p.w[0] = a->wB;
  p.w[1] = a->wC;
  p.out[0] = a->Bc;
  p.out[1] = a->Cc;
  if (a->T > 0) {
    int64_t tpg = (a->T + rp::kBcNormWorkgroups - 1) / rp::kBcNormWorkgroups;
    tpg = tpg < rp::kWaves ? rp::kWaves : tpg;
    p.tokens_per_group = tpg;
    p.groups = (int)((a->T + tpg - 1) / tpg);
  }
  return p;
}

}  // namespace

extern "C" {

int rp_bcnorm_check(const rp_bcnorm_args* a) {
  if (a == nullptr) return fail(RP_ERR_INVALID, "bcnorm args: NULL");
  if (a->T < 0 || a->N < 1 || a->P < 1)
    return fail(RP_ERR_INVALID, "bcnorm args: T >= 0, N >= 1, P >= 1 required");
  if (a->N > RP_MAX_STATE || a->P > 8)
    return fail(RP_ERR_UNSUPPORTED, "bcnorm args: N=%lld P=%lld beyond N <= %d, P <= 8",
                (long long)a->N, (long long)a->P, RP_MAX_STATE);
  if (a->dtype_x != RP_F32 && a->dtype_x != RP_BF16 && a->dtype_x != RP_F16)
    return fail(RP_ERR_INVALID, "bcnorm args: unknown dtype code %d", a->dtype_x);
  if ((a->normalize != 0 && a->normalize != 1) || a->reserved != 0)
    return fail(RP_ERR_INVALID, "bcnorm args: normalize must be 0 or 1, reserved 0");
  if (a->normalize && !(a->eps >= 0.f))
    return fail(RP_ERR_INVALID, "bcnorm args: eps must be >= 0");
  if (a->normalize && (!a->wB || !a->wC || !aligned(a->wB, 4) || !aligned(a->wC, 4)))
    return fail(RP_ERR_INVALID, "bcnorm args: normalize needs 4-byte aligned wB, wC");
  if (a->T == 0) return RP_OK;
  const int64_t K = a->N * a->P;
  if (!a->B_raw || !a->C_raw) return fail(RP_ERR_INVALID, "bcnorm args: NULL B_raw/C_raw");
  if (!aligned(a->B_raw, elem_size(a->dtype_x)) || !aligned(a->C_raw, elem_size(a->dtype_x)) ||
      (a->Bc && !aligned(a->Bc, 4)) || (a->Cc && !aligned(a->Cc, 4)))
    return fail(RP_ERR_INVALID, "bcnorm args: misaligned pointer");
  if (a->B_sr < K || a->C_sr < K)
    return fail(RP_ERR_INVALID, "bcnorm args: row stride shorter than N*P");
  return RP_OK;
}

int64_t rp_bcnorm_work_bytes(const rp_bcnorm_args* a) {
  if (rp_bcnorm_check(a) != RP_OK) return -1;
  const rp::BcNormParams p = bcnorm_params(a);
  return round_up((int64_t)p.groups * 2 * a->N * a->P * (int64_t)sizeof(double), 256);
}

int rp_bcnorm_fwd(const rp_bcnorm_args* a, void* stream) {
  int st = rp_bcnorm_check(a);
  if (st != RP_OK) return st;
  if (a->T == 0) return RP_OK;
  if (!a->Bc || !a->Cc) return fail(RP_ERR_INVALID, "bcnorm fwd: NULL Bc/Cc");
  const int64_t in_b = ((a->T - 1) * a->B_sr + a->N * a->P) * elem_size(a->dtype_x);
  const int64_t in_c = ((a->T - 1) * a->C_sr + a->N * a->P) * elem_size(a->dtype_x);
  const int64_t ob = a->T * a->N * 4;
  if (overlaps(a->Bc, ob, a->Cc, ob) || overlaps(a->Bc, ob, a->B_raw, in_b) ||
      overlaps(a->Bc, ob, a->C_raw, in_c) || overlaps(a->Cc, ob, a->B_raw, in_b) ||
      overlaps(a->Cc, ob, a->C_raw, in_c))
    return fail(RP_ERR_INVALID, "bcnorm fwd: outputs overlap each other or the inputs");
  hipError_t e = rp::launch_bcnorm_fwd(bcnorm_params(a), (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "bcnorm fwd launch");
  return RP_OK;
}

int rp_bcnorm_bwd(const rp_bcnorm_args* a, const rp_bcnorm_grad* g, void* stream) {
  int st = rp_bcnorm_check(a);
  if (st != RP_OK) return st;
  if (g == nullptr) return fail(RP_ERR_INVALID, "bcnorm grad: NULL");
  if (a->normalize && (!g->dwB || !g->dwC || !aligned(g->dwB, 4) || !aligned(g->dwC, 4)))
    return fail(RP_ERR_INVALID, "bcnorm grad: normalize needs 4-byte aligned dwB, dwC");
  const rp::BcNormParams p = bcnorm_params(a);
  rp::BcNormGrad bg{};
  bg.dw[0] = g->dwB;
  bg.dw[1] = g->dwC;
  if (a->T > 0) {
    const int64_t K = a->N * a->P, es = elem_size(a->dtype_x);
    if (!g->dBc || !g->dCc || !g->dB_raw || !g->dC_raw)
      return fail(RP_ERR_INVALID, "bcnorm grad: NULL dBc/dCc/dB_raw/dC_raw");
    if (!aligned(g->dBc, 4) || !aligned(g->dCc, 4) || !aligned(g->dB_raw, es) ||
        !aligned(g->dC_raw, es))
      return fail(RP_ERR_INVALID, "bcnorm grad: misaligned pointer");
    const int64_t nx = a->T * K * es;
    if (overlaps(g->dB_raw, nx, g->dC_raw, nx))
      return fail(RP_ERR_INVALID, "bcnorm grad: dB_raw and dC_raw overlap");
    const int64_t in_b = ((a->T - 1) * a->B_sr + K) * es, in_c = ((a->T - 1) * a->C_sr + K) * es;
    const int64_t gb = a->T * a->N * 4;
    const void* outs[2] = {g->dB_raw, g->dC_raw};
    for (const void* o : outs)
      if (overlaps(o, nx, a->B_raw, in_b) || overlaps(o, nx, a->C_raw, in_c) ||
          overlaps(o, nx, g->dBc, gb) || overlaps(o, nx, g->dCc, gb))
        return fail(RP_ERR_INVALID, "bcnorm grad: an output overlaps an input");
    bg.g[0] = g->dBc;
    bg.g[1] = g->dCc;
    bg.dx[0] = g->dB_raw;
    bg.dx[1] = g->dC_raw;
  }
  const int64_t need = rp_bcnorm_work_bytes(a);
  if (a->normalize && need > 0 &&
      (g->work == nullptr || g->work_bytes < need || !aligned(g->work, 256)))
    return fail(RP_ERR_WORKSPACE, "bcnorm bwd: workspace needs %lld bytes (256-aligned), got %lld",
                (long long)need, (long long)g->work_bytes);
  bg.part = static_cast<double*>(g->work);
  hipError_t e = rp::launch_bcnorm_bwd(p, bg, (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "bcnorm bwd launch");
  return RP_OK;
}

int rp_rmsnorm_check(const rp_rmsnorm_args* a) {
  if (a == nullptr) return fail(RP_ERR_INVALID, "rmsnorm args: NULL");
  if (a->rows < 0 || a->d < 0) return fail(RP_ERR_INVALID, "rmsnorm args: negative size");
  if (a->d > kI32Max) return fail(RP_ERR_UNSUPPORTED, "rmsnorm args: d must fit in int32");
  if (!(a->eps >= 0.f)) return fail(RP_ERR_INVALID, "rmsnorm args: eps must be >= 0");
  if (a->rows * a->d == 0) return RP_OK;
  if (!a->x || !a->w || !a->out) return fail(RP_ERR_INVALID, "rmsnorm args: NULL x / w / out");
  if (a->x_sr < a->d) return fail(RP_ERR_INVALID, "rmsnorm args: x row stride shorter than d");
  if (!aligned(a->x, 4) || !aligned(a->w, 4) || !aligned(a->out, 4))
    return fail(RP_ERR_INVALID, "rmsnorm args: misaligned pointer");
  const int64_t n = a->rows * a->d * 4;
  const int64_t xb = ((a->rows - 1) * a->x_sr + a->d) * 4;
  if (a->add != nullptr) {
    if (a->dtype_add != RP_F32 && a->dtype_add != RP_BF16 && a->dtype_add != RP_F16)
      return fail(RP_ERR_INVALID, "rmsnorm args: unknown dtype code %d", a->dtype_add);
    if (a->add_sr < a->d || !aligned(a->add, elem_size(a->dtype_add)))
      return fail(RP_ERR_INVALID, "rmsnorm args: add row stride shorter than d or misaligned");
    if (!a->x_out || !aligned(a->x_out, 4))
      return fail(RP_ERR_INVALID, "rmsnorm args: add needs a 4-byte aligned x_out");
    const int64_t ab = ((a->rows - 1) * a->add_sr + a->d) * elem_size(a->dtype_add);
    if (overlaps(a->x_out, n, a->x, xb) || overlaps(a->x_out, n, a->add, ab) ||
        overlaps(a->x_out, n, a->out, n) || overlaps(a->out, n, a->add, ab))
      return fail(RP_ERR_INVALID, "rmsnorm args: an output overlaps another buffer");
  }
  if (overlaps(a->out, n, a->x, xb))
    return fail(RP_ERR_INVALID, "rmsnorm args: out overlaps x");
  return RP_OK;
}

int rp_rmsnorm_fwd(const rp_rmsnorm_args* a, void* stream) {
  int st = rp_rmsnorm_check(a);
  if (st != RP_OK) return st;
  rp::RmsNormParams p{};
  p.rows = a->rows;
  p.d = (int)a->d;
  p.dt_add = a->dtype_add;
  p.eps = a->eps;
  p.x = a->x;
  p.xsr = a->x_sr;
  p.add = a->add;
  p.asr = a->add_sr;
  p.w = a->w;
  p.x_out = a->x_out;
  p.out = a->out;
  hipError_t e = rp::launch_rmsnorm_fwd(p, (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "rmsnorm launch");
  return RP_OK;
}

int rp_softplus(const float* x, float* out, int64_t n, void* stream) {
  if (n < 0) return fail(RP_ERR_INVALID, "softplus: n < 0");
  if (n > 0 && (x == nullptr || out == nullptr)) return fail(RP_ERR_INVALID, "softplus: NULL buffer");
  if (n > 0 && (!aligned(x, 4) || !aligned(out, 4)))
    return fail(RP_ERR_INVALID, "softplus: misaligned buffer");
  hipError_t e = rp::launch_softplus(x, out, n, (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "softplus launch");
  return RP_OK;
}

int rp_ply_topk_check(const rp_ply_topk_args* a) {
  if (a == nullptr) return fail(RP_ERR_INVALID, "ply topk args: NULL");
  if (a->R < 0 || a->V < 1) return fail(RP_ERR_INVALID, "ply topk args: R < 0 or V < 1");
  if (a->V > kI32Max / 2) return fail(RP_ERR_UNSUPPORTED, "ply topk args: V must fit in int32");
  if (a->k < 1 || a->k > rp::kPlyMaxK)
    return fail(RP_ERR_UNSUPPORTED, "ply topk args: k=%d outside [1, %d]", a->k, rp::kPlyMaxK);
  if (a->dtype_logits != RP_F32 && a->dtype_logits != RP_BF16 && a->dtype_logits != RP_F16)
    return fail(RP_ERR_INVALID, "ply topk args: unknown dtype code %d", a->dtype_logits);
  if (a->out_sr < 2 * (int64_t)a->k + 1)
    return fail(RP_ERR_INVALID, "ply topk args: out row stride below 2k + 1");
  if (a->R == 0) return RP_OK;
  if (!a->logits || !a->out) return fail(RP_ERR_INVALID, "ply topk args: NULL logits / out");
  if (a->logits_sr < a->V) return fail(RP_ERR_INVALID, "ply topk args: logits row stride below V");
  const int64_t es = elem_size(a->dtype_logits);
  if (!aligned(a->logits, es) || !aligned(a->out, 4) || (a->values && !aligned(a->values, 4)))
    return fail(RP_ERR_INVALID, "ply topk args: misaligned pointer");
  const int64_t ob = ((a->R - 1) * a->out_sr + 2 * a->k + 1) * 4;
  const int64_t lb = ((a->R - 1) * a->logits_sr + a->V) * es;
  if (overlaps(a->out, ob, a->logits, lb) || (a->values && overlaps(a->out, ob, a->values, a->R * 4)))
    return fail(RP_ERR_INVALID, "ply topk args: out overlaps an input");
  return RP_OK;
}

int rp_ply_topk(const rp_ply_topk_args* a, void* stream) {
  int st = rp_ply_topk_check(a);
  if (st != RP_OK) return st;
  rp::PlyTopkParams p{};
  p.R = a->R;
  p.V = (int)a->V;
  p.k = a->k;
  p.dt = a->dtype_logits;
  p.logits = a->logits;
  p.lsr = a->logits_sr;
  p.values = a->values;
  p.out = a->out;
  p.osr = a->out_sr;
  hipError_t e = rp::launch_ply_topk(p, (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "ply topk launch");
  return RP_OK;
}

int rp_ply_gather_check(const rp_ply_gather_args* a) {
  if (a == nullptr) return fail(RP_ERR_INVALID, "ply gather args: NULL");
  if (a->R < 0 || a->M < 0 || a->V < 1)
    return fail(RP_ERR_INVALID, "ply gather args: R or M negative, or V < 1");
  if (a->V > kI32Max) return fail(RP_ERR_UNSUPPORTED, "ply gather args: V must fit in int32");
  if (a->dtype_logits != RP_F32 && a->dtype_logits != RP_BF16 && a->dtype_logits != RP_F16)
    return fail(RP_ERR_INVALID, "ply gather args: unknown dtype code %d", a->dtype_logits);
  if (a->reserved != 0) return fail(RP_ERR_INVALID, "ply gather args: reserved must be 0");
  if (a->R * a->M == 0) return RP_OK;
  if (!a->logits || !a->tokens || !a->out)
    return fail(RP_ERR_INVALID, "ply gather args: NULL logits / tokens / out");
  if (a->logits_sr < a->V || a->tokens_sr < a->M || a->out_sr < a->M)
    return fail(RP_ERR_INVALID, "ply gather args: a row stride below its row length");
  const int64_t es = elem_size(a->dtype_logits);
  if (!aligned(a->logits, es) || !aligned(a->tokens, 4) || !aligned(a->out, 4))
    return fail(RP_ERR_INVALID, "ply gather args: misaligned pointer");
  const int64_t ob = ((a->R - 1) * a->out_sr + a->M) * 4;
  if (overlaps(a->out, ob, a->logits, ((a->R - 1) * a->logits_sr + a->V) * es) ||
      overlaps(a->out, ob, a->tokens, ((a->R - 1) * a->tokens_sr + a->M) * 4))
    return fail(RP_ERR_INVALID, "ply gather args: out overlaps an input");
  return RP_OK;
}

int rp_ply_gather(const rp_ply_gather_args* a, void* stream) {
  int st = rp_ply_gather_check(a);
  if (st != RP_OK) return st;
  rp::PlyGatherParams p{};
  p.R = a->R;
  p.M = a->M;
  p.V = (int)a->V;
  p.dt = a->dtype_logits;
  p.logits = a->logits;
  p.lsr = a->logits_sr;
  p.tokens = a->tokens;
  p.tsr = a->tokens_sr;
  p.out = a->out;
  p.osr = a->out_sr;
  hipError_t e = rp::launch_ply_gather(p, (hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "ply gather launch");
  return RP_OK;
}

}  // extern "C"
