// Kernel parameter blocks and host-side launchers (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rp {

constexpr int kWave = 64;
constexpr int kWaves = 4;  // waves per workgroup
constexpr int kThreads = kWave * kWaves;

// Time steps staged in LDS per block by the forward kernel, and the
// checkpoint interval (the chunk) of the backward's recompute.
constexpr int kFwdTB = 32;
constexpr int kCkptK = 4;

struct ScanParams {
  const void* delta;
  const void* u;
  const void* Bc;
  const void* Cc;
  int64_t dsb, dsl, usb, usl, bsb, bsl, csb, csl;
  const float* Ar;
  const float* Ai;
  const float* Tk;
  const float* h0;     // (B, D, N) initial state or null (zero)
  const float* beta0;
  int B, L, D, N, NR, NT;
  int dt_delta, dt_u, dt_B, dt_C;
  int dsp;       // 1: delta holds x and the scan uses softplus(x)
  int ndir;      // 1 causal, 2 bidirectional
  int ntiles;    // ceil(D / CB)
  int nck;       // stored checkpoints per (dir, b): ceil(L / K) - 1
};

struct FwdOut {
  float* y;
  float* ckpt;
  float* h_last;
  float* beta_last;
  float* dcache;  // (B, L, D) softplus(x) for the backward, or null
};

struct BwdIO {
  const float* dy;
  const float* ckpt;
  const float* dh_last;     // (B, D, N) or null: gradient of the final h
  const float* dbeta_last;  // (B, D, N) or null: gradient of the final beta
  void* d_delta;     // (B, L, D) in dt_dd: written by the last direction
  void* d_u;         // (B, L, D) in dt_du
  float* pd_delta;   // (B, L, D) fp32: the first direction's sums, which the
  float* pd_u;       //   second reads back (d_delta / d_u themselves when fp32)
  int dt_dd, dt_du;  // storage codes of d_delta / d_u (RP_F32 unless asked)
  float* d_h0;       // (B, D, N) or null
  float* d_beta0;
  const float* dcache;  // (B, L, D) delta = softplus(x) cached by the forward (dsp only)
  float* part_bc;    // [2][ntg][B][L][N]     per-tile-group dB / dC partial sums
  double* part_par;  // [nbg][2][D][N]        per-batch-group dA partial sums
  int bg;           // batch rows per workgroup
  int nbg;          // ceil(B / bg)
  int tpw;          // adjacent channel tiles per workgroup (a tile group)
  int ntg;          // ceil(ntiles / tpw)
};

struct StepParams {
  int R, D, N, NR, NT;
  const float* delta;
  int64_t dsr;
  const float* u;
  int64_t usr;
  const float* Bc;
  int64_t bsr;
  const float* Cc;
  int64_t csr;
  const float* h_in;
  const float* beta_in;
  int64_t ssr;  // elements between consecutive rollouts' input states (0: one shared state)
  int dsp;      // 1: delta holds x and the step uses softplus(x)
  int rank1;    // 1: beta as rows [dt*u | B] of D + N floats
  const void* z;  // (R, D) gate branch or null: y = y * silu(z)
  int64_t zsr;
  int dt_z;
  int64_t bssr; // rank-1 input rows: elements between rollouts (0: one shared row)
  const float* Ar;
  const float* Ai;
  const float* Tk;
  const float* Dskip;
  float* h_out;
  float* beta_out;
  float* y;
  int ntiles;   // lane-layout kernel: channel tiles of CB
  int ctiles;   // tile kernel: channel tiles of kStepTile / step_tile_split(S, NPL)
  int ri;       // tile kernel: rollouts per workgroup
  int rgroups;  // tile kernel: ceil(R / ri)
  // tile kernel, one rollout per workgroup: the B / C rows computed in the
  // prologue from the raw projections (BCNorm + p-sum) instead of read
  int bn_fused;
  const void* bn_x[2];    // B_raw, C_raw rows (R, N * bn_P), row strides bn_xs
  int64_t bn_xs[2];
  int bn_dt;              // their storage dtype
  const float* bn_w[2];   // (N * bn_P,) norm weights
  int bn_P;
  int bn_normalize;
  float bn_eps;
};

// The mixer output gate out = (y + k u D) silu(z) over rows = B * L.
// Rows are split into row groups (units) of rows_per_unit consecutive rows,
// one workgroup per group and channel tile, each with its own dD partial.
struct MixerOutParams {
  int64_t rows;            // B * L
  int L, D;
  int k_skip;              // 1 or 2 D-skips
  int dt_u, dt_z;
  const float* y;          // (rows, D) fp32
  const void* u;
  int64_t usb, usl;
  const void* z;
  int64_t zsb, zsl;
  const float* Dskip;      // (D,)
  void* out;               // (rows, D) in dt_out
  int dt_out;              // dtype of out (and of the backward's dout)
  int64_t rows_per_unit;
  int units;
  int vec;                 // 1: 16-byte vectors of 8 channels per lane
};

struct MixerOutGrad {
  const void* dout;   // (rows, D) in dt_out
  float* dy;          // (rows, D) fp32
  void* du;           // (rows, D) in u's dtype
  void* dz;           // (rows, D) in z's dtype
  float* dD;          // (D,)
  double* part;       // (units, D) workspace; unused when there are no rows
};

// Workgroups a mixer-output launch aims for (channel tiles x row groups):
// the forward streams with a few per CU; the backward (about 130 VGPRs on
// the vector path, 3 workgroups per CU) with one resident round.
constexpr int kMixerFwdWorkgroups = 1024;
constexpr int kMixerBwdWorkgroups = 768;
// Channels per lane on the vector path, and per workgroup column tile.
constexpr int kMixVec = 8;
constexpr int kMixTile = kWave * kMixVec;

hipError_t launch_mixer_out_fwd(const MixerOutParams& p, hipStream_t st);
hipError_t launch_mixer_out_bwd(const MixerOutParams& p, const MixerOutGrad& g, hipStream_t st);

// BCNorm + MIMO p-sum of the B and C projections (part 0: B, part 1: C).
struct BcNormParams {
  int64_t T;               // tokens
  int N, P;                // states, MIMO channels (K = N * P features)
  int dt_x;                // storage dtype of both projections
  int normalize;           // 1: RMSNorm before the p-sum
  float eps;
  const void* x[2];        // (T, K), row strides xs, inner stride 1
  int64_t xs[2];
  const float* w[2];       // (K,) norm weights
  float* out[2];           // (T, N) fp32
  int64_t tokens_per_group;
  int groups;              // workgroups (token ranges)
};

struct BcNormGrad {
  const float* g[2];       // (T, N) fp32
  void* dx[2];             // (T, K) contiguous, dt_x
  float* dw[2];            // (K,)
  double* part;            // (groups, 2, K) workspace
};

// Workgroups a BCNorm launch aims for.
constexpr int kBcNormWorkgroups = 1024;

hipError_t launch_bcnorm_fwd(const BcNormParams& p, hipStream_t st);
hipError_t launch_bcnorm_bwd(const BcNormParams& p, const BcNormGrad& g, hipStream_t st);

// Residual add + RMSNorm of rows (forward only).
struct RmsNormParams {
  int64_t rows;
  int d;
  int dt_add;
  float eps;
  const float* x;   // (rows, d), row stride xsr
  int64_t xsr;
  const void* add;  // (rows, d) or null, row stride asr
  int64_t asr;
  const float* w;   // (d,)
  float* x_out;     // (rows, d) contiguous: x + add (with add only)
  float* out;       // (rows, d) contiguous
};

hipError_t launch_rmsnorm_fwd(const RmsNormParams& p, hipStream_t st);
hipError_t launch_softplus(const float* x, float* out, int64_t n, hipStream_t st);

// Channels (one per thread) of the step tile kernel's workgroup, and the
// most rollouts one of its workgroups walks.
constexpr int kStepTile = kThreads;
// Threads per channel of the step tile kernel for S state slices: S / 4 from
// 8 slices up (d_state 24-40 and 48-80), each thread taking 4 slices (one
// float4 per slot); the tile then holds kStepTile / (S / 4) channels.
// From 5 slots of 16 slices up (d_state 65-128), and at 5 slots of 8
// (d_state 33-40), S / 2 threads of 2 slices each (one float2 per slot),
// halving a thread's states.
constexpr int step_tile_split(int S, int NPL) {
  return ((S == 16 && NPL >= 5) || (S == 8 && NPL == 5)) ? S / 2 : S >= 8 ? S / 4 : 1;
}
// Whether the step tile kernel takes the shape (S, NPL): d_state a multiple
// of 4 up to S * NPL; below S * NPL the host also asks for pad states only
// in the last slot (above S * (NPL - 1)), except where a thread holds 2
// slices (float2 per slot), which takes any pad pattern.
constexpr bool step_tile_shape(int S, int NPL) {
  return S * NPL <= 40 || S == 16;
}
constexpr int kStepRiMax = 16;
// The most rollouts a step tile workgroup walks: above 80 states the B / C
// rows of fewer rollouts stay in LDS, so that two workgroups fit a CU beside
// the (h, beta) blocks (the host's automatic choice never exceeds these).
constexpr int step_tile_ri_max(int S, int NPL, bool rank1) {
  return S * NPL > 80 ? (rank1 ? 8 : 4) : kStepRiMax;
}

// Chosen lane split for a state dimension N: S lanes per channel holding NPL
// states each.  Returns false when N is beyond the compiled shapes.
bool choose_shape(int N, int* S, int* NPL);

// Gate kind of a launch: how much of the rotational / tracking split of the
// state slots is fixed at compile time.  Every kind gives bitwise the same
// results; the specialised ones drop run-time selects and dead gate code.
enum GateCode {
  kGateGeneric = 0,   // every slot decided at run time
  kGateRotLead = 1,   // complex gates, slots j < NPL-1 rotational (NR >= S*(NPL-1))
  kGateRotTrack = 2,  // complex gates, slots j < NPL-1 rotational, slot NPL-1
                      // tracking or padding (NR == S*(NPL-1))
  kGateRotAll = 3,    // complex gates, every slot rotational (NR == N == S*NPL):
                      // instantiated for the step tile kernel and the scan
                      // kernels of all_gate_shape; elsewhere RotLead
  kGateRealAll = 4,   // real decay (no A_imag), every slot decaying (NR == N ==
                      // S*NPL): instantiated for all_gate_shape; elsewhere
                      // Generic
};

// The lane shapes whose kernels also take the all-rotational and all-real
// gate kinds: 4 slots of 4, 8 or 16 lanes, d_state 16, 32 and 64 (the
// reference's default d_state 32 and 64, and its CPU configuration's real
// d_state 16).
constexpr bool all_gate_shape(int S, int NPL) {
  return NPL == 4 && (S == 4 || S == 8 || S == 16);
}

inline int gate_code(bool has_imag, int64_t NR, int S, int NPL) {
  if (!has_imag || NR < (int64_t)S * (NPL - 1)) return kGateGeneric;
  return NR == (int64_t)S * (NPL - 1) ? kGateRotTrack : kGateRotLead;
}
// The gate kind with the all-rotational and all-real cases (every state
// rotational or decaying, no pad slot) told apart.
inline int gate_code_all(bool has_imag, int64_t NR, int64_t N, int S, int NPL) {
  if (NR == N && N == (int64_t)S * NPL) return has_imag ? kGateRotAll : kGateRealAll;
  return gate_code(has_imag, NR, S, NPL);
}

hipError_t launch_scan_fwd(int S, int NPL, int gk, const ScanParams& p, const FwdOut& o,
                           hipStream_t st);
hipError_t launch_scan_bwd(int S, int NPL, int gk, const ScanParams& p, const BwdIO& io,
                           hipStream_t st);
hipError_t launch_bwd_finalize(const ScanParams& p, const BwdIO& io, float* d_Bc, float* d_Cc,
                               float* d_Ar, float* d_Ai, float* d_Tk, hipStream_t st);
// `tile`: the tile kernel (N % 4 == 0, step_tile_shape, 16-byte aligned
// state pointers; N below S*NPL takes its pad-state instantiation,
// launch_step_tile_pad); otherwise the lane-layout kernel.  Bitwise the same.
hipError_t launch_step(int S, int NPL, int gk, bool tile, const StepParams& p, hipStream_t st);
hipError_t launch_step_tile_pad(int S, int NPL, int gk, const StepParams& p, hipStream_t st);
hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t st);

// Rollout-ply boundary (ply.hip).
constexpr int kPlyMaxK = 16;

struct PlyTopkParams {
  int64_t R;
  int V, k, dt;
  const void* logits;
  int64_t lsr;           // logits row stride (elements)
  const float* values;   // (R,) or null
  void* out;             // (R, osr) 32-bit words: value, k logits, k ids
  int64_t osr;
};

struct PlyGatherParams {
  int64_t R, M;
  int V, dt;
  const void* logits;
  int64_t lsr;
  const int32_t* tokens;  // (R, M), row stride tsr
  int64_t tsr;
  float* out;             // (R, M), row stride osr
  int64_t osr;
};

hipError_t launch_ply_topk(const PlyTopkParams& p, hipStream_t st);
hipError_t launch_ply_gather(const PlyGatherParams& p, hipStream_t st);

}  // namespace rp

// Compiled (S, NPL) shapes: S lanes per channel, NPL states per lane.
// d_state <= 20 uses 4 lanes per channel, <= 40 uses 8, <= 128 uses 16.
#define RP_FOR_EACH_SHAPE(X) \
  X(4, 1) X(4, 2) X(4, 3) X(4, 4) X(4, 5) \
  X(8, 3) X(8, 4) X(8, 5) \
  X(16, 3) X(16, 4) X(16, 5) X(16, 6) X(16, 8)
