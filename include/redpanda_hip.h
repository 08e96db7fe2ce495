/*
 * redpanda_hip.h — C ABI of the MI355X (gfx950) kernels for ChessMamba's
 * hot path: the Mamba-3 exponential-trapezoidal selective scan (forward,
 * bidirectional forward, analytic reverse-scan backward) and the batched
 * O(1) recurrent step.
 *
 * Plain C: device pointers, element counts and strides, a hipStream_t passed
 * as void*.  The library never allocates or frees device memory; every buffer
 * (outputs and workspace) is caller-allocated, as the reference allocates its
 * outputs and scratch with torch (engine/triton_scan.py:260-262, :293-300).
 * All entry points are asynchronous on the given stream and return 0 or a
 * negative status; rp_last_error() describes the last failure of the calling
 * thread.  Nothing blocks, nothing aborts, no exceptions cross the ABI.
 *
 * Recurrence (one channel d, state index n; NR rotational + NT tracking):
 *   g_t[n]    = exp(dt_t Ar[d,n]) cos(dt_t Ai[d,n])   n <  NR
 *             = Tk[d,n-NR]  (= tanh theta)            n >= NR
 *   beta_t[n] = dt_t u_t B_t[n]
 *   h_t       = g_t h_{t-1} + beta_t/2 + g_t beta_{t-1}/2
 *   y_t       = sum_n h_t[n] C_t[n]           (scan: no D-skip; step: + u D)
 */
#ifndef REDPANDA_HIP_H
#define REDPANDA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RP_ABI_VERSION 13

/* element type codes of the streamed scan inputs (delta, u, Bc, Cc); each
 * tensor carries its own code, as autocast hands over mixed dtypes */
enum { RP_F32 = 0, RP_BF16 = 1, RP_F16 = 2 };

/* status codes */
enum {
  RP_OK = 0,
  RP_ERR_INVALID = -1,      /* bad shape, stride, pointer or dtype   */
  RP_ERR_UNSUPPORTED = -2,  /* a size beyond the compiled limits     */
  RP_ERR_LAUNCH = -3,       /* hipGetLastError after a launch        */
  RP_ERR_WORKSPACE = -4     /* workspace missing or too small        */
};

/* Largest supported state dimension N = NR + NT. */
#define RP_MAX_STATE 128

/*
 * Scan arguments.  delta, u: (B, L, D); Bc, Cc: (B, L, N) — B and C already
 * contracted over the MIMO dimension p (engine/mamba.py:336-337).  Strides
 * are in elements for the batch and time dimensions; the innermost (channel
 * or state) stride must be 1.  A_real, A_imag: (D, NR) fp32 row-major, or
 * NULL; A_imag NULL means a real decay gate exp(dt Ar).  track: (D, NT) fp32
 * tanh(theta) gates, or NULL when NT == 0.  h0, beta0: NULL (zero state, as
 * the reference's scan always starts), or (B, D, N) fp32 contiguous state to
 * continue from — the cache format of step() (causal scans, L >= 1).
 * delta_softplus = 1: delta holds the dt projection x and the scan runs on
 * softplus(x) as engine/mamba.py:300 computes it (F.softplus, beta 1,
 * threshold 20, fp32); rp_scan_bwd's d_delta is then the gradient of x.
 * grad_in_storage = 1: rp_scan_bwd writes d_delta and d_u in delta's and
 * u's storage dtypes (rounded to nearest even, as torch converts its fp32
 * result), instead of fp32: autograd returns input gradients in the input's
 * dtype, and the conversion passes over (B, L, D) then disappear.  A
 * bidirectional scan then also keeps its first direction's fp32 partial
 * sums in the backward's workspace (rp_scan_bwd_work_bytes counts them).
 */
typedef struct rp_scan_args {
  int64_t B, L, D, N, NR, NT;
  int32_t dtype_delta, dtype_u, dtype_B, dtype_C;  /* RP_F32 / RP_BF16 / RP_F16 */
  int32_t bidirectional;   /* 0: causal; 1: y = S(x) + flip(S(flip(x)))     */
  int32_t delta_softplus;  /* 0: delta as given; 1: see below               */
  const void* delta;  int64_t delta_sb, delta_sl;
  const void* u;      int64_t u_sb, u_sl;
  const void* Bc;     int64_t Bc_sb, Bc_sl;
  const void* Cc;     int64_t Cc_sb, Cc_sl;
  const float* A_real;
  const float* A_imag;
  const float* track;
  const float* h0;
  const float* beta0;
  int32_t grad_in_storage;  /* 0: fp32 d_delta / d_u; 1: see above           */
} rp_scan_args;

/*
 * Forward outputs.  y: (B, L, D) fp32 contiguous, WITHOUT the u*D skip
 * (the caller adds it, as engine/mamba.py:350 does).  ckpt: NULL for
 * inference, else rp_scan_ckpt_bytes() of 256-byte aligned workspace that
 * rp_scan_bwd reads (with delta_softplus it also keeps softplus(x)).
 * h_last, beta_last: NULL, or (B, D, N) fp32 contiguous to receive the final
 * recurrent state (h_{L-1}, beta_{L-1}) that rp_step continues from
 * (engine/mamba.py:377-379); causal scans only.
 */
typedef struct rp_scan_fwd_out {
  float* y;
  float* ckpt;
  float* h_last;
  float* beta_last;
} rp_scan_fwd_out;

/*
 * Backward.  dy: (B, L, D) fp32 contiguous upstream gradient of y.  ckpt:
 * the workspace the matching forward filled.  Outputs, contiguous, fp32
 * (d_delta and d_u in delta's and u's dtypes with grad_in_storage):
 * d_delta, d_u (B, L, D); d_Bc, d_Cc (B, L, N); d_A_real, d_A_imag (D, NR)
 * (d_A_imag ignored when A_imag is NULL); d_track (D, NT).  work:
 * rp_scan_bwd_work_bytes() of scratch.  dh_last, dbeta_last: NULL, or
 * (B, D, N) fp32 gradients of the final state returned by a causal forward
 * (training through prime_cache + step, engine/search_mamba.py:252-273).
 * d_h0, d_beta0: NULL, or (B, D, N) fp32 outputs receiving the gradient of
 * the initial state h0 / beta0 (requires h0).  Deterministic: every sum
 * runs in a fixed order (the float atomic adds some shapes use each update
 * an address that no other thread touches).  work must be ordinary device
 * memory (hipMalloc, or a tensor of torch's caching allocator): those
 * float64 atomic adds run on the device's own atomic units, which HIP does
 * not guarantee for host-mapped, managed or fine-grained allocations.
 */
typedef struct rp_scan_bwd_io {
  const float* dy;
  const float* ckpt;
  const float* dh_last;
  const float* dbeta_last;
  void* d_delta;   /* fp32, or delta's dtype with grad_in_storage */
  void* d_u;       /* fp32, or u's dtype with grad_in_storage     */
  float* d_Bc;
  float* d_Cc;
  float* d_A_real;
  float* d_A_imag;
  float* d_track;
  float* d_h0;
  float* d_beta0;
  void* work;
  int64_t work_bytes;
} rp_scan_bwd_io;

/*
 * Step arguments (one token per rollout, engine/mamba.py:466-498).
 * delta, u: (R, D) fp32 with row stride; Bc, Cc: (R, N) fp32 with row
 * stride; h_in, beta_in: (R, D, N) fp32 contiguous, or both NULL for a fresh
 * (zero) state; Dskip: (D,) fp32.  Outputs: h_out, beta_out (R, D, N) fp32
 * contiguous (may alias h_in / beta_in for an in-place update); y: (R, D)
 * fp32 contiguous = sum_n h_out C + u D.  beta_out = (dt u) B exactly as the
 * reference stores dBu_t.
 * broadcast_state = 1: h_in and beta_in hold ONE (D, N) state that every
 * rollout continues from -- a batch-1 cache fanned out to R rollouts without
 * the copies of engine/search_mamba.py:177-187 (expand().contiguous()); the
 * outputs must then not overlap the inputs.  0: the (R, D, N) layout above.
 * z: with the gate branch given, y is returned already gated, y * silu(z)
 * (the out_proj input of engine/mamba.py:497), silu rounded to z's dtype as
 * torch rounds it.
 * beta_rank1 = 1: beta is carried by its rank-1 factors, since beta =
 * (dt u) outer B: beta_in / beta_out are (R, D + N) fp32 rows [dt*u | B]
 * (one (D + N) row with broadcast_state), and the step forms beta_prev =
 * (dt*u)_prev * B_prev with the multiply that produced the full form, so the
 * results are the same bits at half the state traffic.  beta_out must not
 * overlap beta_in (a rollout's B row is read by all its channel tiles).
 */
typedef struct rp_step_args {
  int64_t R, D, N, NR, NT;
  const float* delta;  int64_t delta_sr;
  const float* u;      int64_t u_sr;
  const float* Bc;     int64_t Bc_sr;
  const float* Cc;     int64_t Cc_sr;
  const float* h_in;
  const float* beta_in;
  const float* A_real;
  const float* A_imag;
  const float* track;
  const float* Dskip;
  float* h_out;
  float* beta_out;
  float* y;
  int32_t broadcast_state;  /* 0 or 1, see above */
  int32_t delta_softplus;   /* 0 or 1: delta holds x, the step uses softplus(x) */
  int32_t beta_rank1;       /* 0 or 1, see above */
  int32_t reserved;         /* must be 0 */
  const void* z;  int64_t z_sr;  /* NULL, or the (R, D) gate branch: y = y * silu(z) */
  int32_t dtype_z;          /* RP_F32 / RP_BF16 / RP_F16 */
  int32_t reserved2;        /* must be 0 */
} rp_step_args;

/*
 * The mixer's output gate around the scan (engine/mamba.py:262-265, with the
 * D-skip of :350 / :375): out = (y + k u D) * silu(z), k = 1 for a causal
 * layer, 2 for a bidirectional one (the skip is added once per direction).
 * y: (B, L, D) fp32 contiguous (the scan output); u, z: (B, L, D) with batch
 * and time strides, inner stride 1, each RP_F32 / RP_BF16 / RP_F16; Dskip:
 * (D,) fp32; out: (B, L, D) contiguous in dtype_out (may be y itself when
 * fp32; unused, and may be NULL, for the backward).  silu(z) is rounded to
 * z's dtype before the product, as torch's ops on those dtypes do; a 16-bit
 * dtype_out rounds the fp32 result as the autocast cast before out_proj
 * does.
 */
typedef struct rp_mixer_out_args {
  int64_t B, L, D;
  int32_t k_skip;          /* 1 or 2 */
  int32_t dtype_u, dtype_z;
  int32_t dtype_out;       /* of out and the backward's dout (RP_F32 = 0 by default) */
  const float* y;
  const void* u;  int64_t u_sb, u_sl;
  const void* z;  int64_t z_sb, z_sl;
  const float* Dskip;
  void* out;
} rp_mixer_out_args;

/*
 * Its backward given dout (B, L, D) contiguous in dtype_out: dy (fp32, the scan's
 * upstream gradient), du (u's dtype, the skip's share only), dz (z's dtype),
 * all (B, L, D) contiguous; dD (D,) fp32 (deterministic sums).  work:
 * rp_mixer_out_work_bytes() of scratch.
 */
typedef struct rp_mixer_out_grad {
  const void* dout;        /* in dtype_out */
  float* dy;
  void* du;
  void* dz;
  float* dD;
  void* work;
  int64_t work_bytes;
} rp_mixer_out_grad;

/* Validate mixer-output arguments on the host without launching anything. */
int rp_mixer_out_check(const rp_mixer_out_args* a);

/* Bytes of scratch rp_mixer_out_bwd needs. */
int64_t rp_mixer_out_work_bytes(const rp_mixer_out_args* a);

/* out = (y + k u D) * silu(z); replaces the elementwise ops after the scan
 * in Mamba3Block.forward (engine/mamba.py:262-265, :350). */
int rp_mixer_out_fwd(const rp_mixer_out_args* a, void* stream);

/* The autograd of those ops in one pass (plus a small dD reduction). */
int rp_mixer_out_bwd(const rp_mixer_out_args* a, const rp_mixer_out_grad* g, void* stream);

/*
 * The SSM input prologue (engine/mamba.py:297-300 BCNorm, :89 RMSNorm,
 * :336-337 contraction over p): per token, Bc[n] = sum_p RMSNorm(B_raw)[n,p]
 * and the same for C, or the plain sums over p when normalize = 0.
 * B_raw, C_raw: (T, N*P) with row strides B_sr, C_sr (elements), inner
 * stride 1, one dtype for both (RP_F32 / RP_BF16 / RP_F16; they are views
 * of one x_proj output); wB, wC: (N*P,) fp32 norm weights; Bc, Cc: (T, N)
 * fp32 contiguous.  1 <= N <= RP_MAX_STATE, 1 <= P <= 8.
 */
typedef struct rp_bcnorm_args {
  int64_t T, N, P;
  int32_t dtype_x;
  int32_t normalize;       /* 0 or 1 */
  float eps;
  int32_t reserved;        /* must be 0 */
  const void* B_raw;  int64_t B_sr;
  const void* C_raw;  int64_t C_sr;
  const float* wB;
  const float* wC;
  float* Bc;
  float* Cc;
} rp_bcnorm_args;

/*
 * Its backward given dBc, dCc (T, N) fp32: dB_raw, dC_raw (T, N*P)
 * contiguous in dtype_x; dwB, dwC (N*P,) fp32 (deterministic sums; unused
 * when normalize = 0).  work: rp_bcnorm_work_bytes() of scratch.
 */
typedef struct rp_bcnorm_grad {
  const float* dBc;
  const float* dCc;
  void* dB_raw;
  void* dC_raw;
  float* dwB;
  float* dwC;
  void* work;
  int64_t work_bytes;
} rp_bcnorm_grad;

/* Validate BCNorm arguments on the host without launching anything. */
int rp_bcnorm_check(const rp_bcnorm_args* a);

/* Bytes of scratch rp_bcnorm_bwd needs. */
int64_t rp_bcnorm_work_bytes(const rp_bcnorm_args* a);

/* Bc, Cc from the raw projections; replaces Mamba3Block._ssm_proj's BCNorm
 * and the B/C sums of _selective_scan_trapezoidal (engine/mamba.py:297-300,
 * :336-337) and of step (:470-471). */
int rp_bcnorm_fwd(const rp_bcnorm_args* a, void* stream);

/* The autograd of those ops in one pass (plus a small dw reduction). */
int rp_bcnorm_bwd(const rp_bcnorm_args* a, const rp_bcnorm_grad* g, void* stream);

/*
 * Residual add + RMSNorm of the batched step's residual stream
 * (engine/mamba.py:82-89, :592-597): x' = x + add (when add is given,
 * written to x_out), out = (x' * rsqrt(mean(x'^2) + eps)) * w, per row.
 * x: (rows, d) fp32 with row stride x_sr; add: NULL or (rows, d) in
 * dtype_add with row stride add_sr; w: (d,) fp32; x_out, out: (rows, d)
 * fp32 contiguous.  Forward only (inference); outputs must not overlap the
 * inputs.
 */
typedef struct rp_rmsnorm_args {
  int64_t rows, d;
  int32_t dtype_add;
  float eps;
  const float* x;    int64_t x_sr;
  const void* add;   int64_t add_sr;
  const float* w;
  float* x_out;
  float* out;
} rp_rmsnorm_args;

/* Validate RMSNorm arguments on the host without launching anything. */
int rp_rmsnorm_check(const rp_rmsnorm_args* a);

/* The residual add and the next RMSNorm of Mamba.step's layer loop in one
 * pass; replaces x + out and RMSNorm's five elementwise and reduction ops. */
int rp_rmsnorm_fwd(const rp_rmsnorm_args* a, void* stream);

/* softplus(x) of n fp32 values (engine/mamba.py:300: F.softplus of the dt
 * projection, beta 1, threshold 20), with the same bits as the scan's and
 * the step's softplus on load (delta_softplus): for a caller that builds a
 * rank-1 beta row [softplus(x) u | B] itself (engine/mamba.py:480-481) and
 * needs it to match the full beta the kernels write.  out may equal x. */
int rp_softplus(const float* x, float* out, int64_t n, void* stream);

/*
 * Host boundary of one lockstep rollout ply.  The reference moves each
 * rollout's continuation row (engine/mars_search.py:262, _select_move's
 * cont_logits.float().cpu()), the logits of its legal moves (:475,
 * _select_fc_move) and the ply's values (:446, :556, vals.cpu().tolist())
 * to the host one rollout at a time; these reduce and pack them on the
 * device, so that one device-to-host copy per ply carries the ply.
 *
 * rp_ply_topk: per rollout r, the k largest logits of row r (IEEE total
 * order, so a positive NaN ranks above +inf; equal logits by ascending token
 * id) and the rollout's value, as row r of `out` in 32-bit words:
 *     word 0          values[r] (fp32; 0 when values is NULL)
 *     words 1 .. k    the logits, fp32, largest first (-inf past V)
 *     words k+1 .. 2k their token ids, int32 (-1 past V)
 * logits: (R, V) in dtype_logits with row stride logits_sr (elements);
 * values: NULL or (R,) fp32; out: (R, out_sr) words, out_sr >= 2k + 1.
 * 1 <= k <= 16.  This is _select_move's candidate list (np.argpartition over
 * the row, then sorted by logit) for every rollout at once.
 */
typedef struct rp_ply_topk_args {
  int64_t R, V;
  int32_t k, dtype_logits;
  const void* logits;  int64_t logits_sr;
  const float* values;
  void* out;           int64_t out_sr;
} rp_ply_topk_args;

/* Validate rp_ply_topk arguments on the host without launching anything. */
int rp_ply_topk_check(const rp_ply_topk_args* a);

/* Top-k continuation candidates and values of a ply, packed per rollout. */
int rp_ply_topk(const rp_ply_topk_args* a, void* stream);

/*
 * rp_ply_gather: out[r, j] = logits[r, tokens[r, j]] as fp32 for j < M, and
 * -inf for ids outside [0, V) (padding): _select_fc_move's gather of the
 * legal moves' logits (engine/mars_search.py:475) for all rollouts at once.
 * tokens: (R, M) int32 with row stride tokens_sr; out: (R, M) fp32 with row
 * stride out_sr; logits as in rp_ply_topk.
 */
typedef struct rp_ply_gather_args {
  int64_t R, V, M;
  int32_t dtype_logits, reserved;
  const void* logits;     int64_t logits_sr;
  const int32_t* tokens;  int64_t tokens_sr;
  float* out;             int64_t out_sr;
} rp_ply_gather_args;

/* Validate rp_ply_gather arguments on the host without launching anything. */
int rp_ply_gather_check(const rp_ply_gather_args* a);

/* The legal moves' logits of every rollout of a ply. */
int rp_ply_gather(const rp_ply_gather_args* a, void* stream);

/* ABI version this library was built with (RP_ABI_VERSION). */
int rp_abi_version(void);

/* Message for the last non-zero status returned on this thread. */
const char* rp_last_error(void);

/* Validate scan arguments on the host without launching anything. */
int rp_scan_check(const rp_scan_args* a);

/* Bytes of checkpoint workspace rp_scan_fwd writes for a later backward. */
int64_t rp_scan_ckpt_bytes(const rp_scan_args* a);

/* Bytes of scratch rp_scan_bwd needs. */
int64_t rp_scan_bwd_work_bytes(const rp_scan_args* a);

/*
 * Forward scan; replaces _TrapezoidalScanFn.forward / _fwd_kernel
 * (engine/triton_scan.py:247-281, :44-98) and, with bidirectional = 1, the
 * two-pass bidirectional branch of Mamba3Block.forward
 * (engine/mamba.py:254-260, minus the D-skip).
 */
int rp_scan_fwd(const rp_scan_args* a, const rp_scan_fwd_out* out, void* stream);

/*
 * Analytic backward; replaces _TrapezoidalScanFn.backward / _bwd_kernel
 * (engine/triton_scan.py:283-315, :100-241) including the dBp/dCp partial
 * sums and the dA atomics, here as deterministic two-stage reductions.
 */
int rp_scan_bwd(const rp_scan_args* a, const rp_scan_bwd_io* io, void* stream);

/*
 * rp_scan_bwd without a caller workspace: the same kernels, with their
 * scratch (the dB / dC partials per tile group and the per-batch-group parameter
 * gradient partials) in a static device array of RP_SCAN_BWD_SCRATCH_BYTES
 * that the library holds on every GPU it runs on until the process ends.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It allocates nothing and frees nothing; io->work and
 * io->work_bytes are ignored.  A shape whose rp_scan_bwd_work_bytes()
 * exceeds the scratch is refused with RP_ERR_WORKSPACE (for example the
 * Eval-Mamba layer, d_inner 1536 and d_state 40 at L = 64, fits up to about
 * 50 batch rows).  Every call on one GPU shares that GPU's scratch, which
 * keeps the last call's contents: calls that overlap on one GPU (concurrent
 * streams, host threads, parallel graph branches) race and must be
 * serialised.  Every partial is written before it is read, so nothing needs
 * clearing between calls.  The scratch is looked up on the stream's device
 * on the first call there; that first call may itself be made under HIP
 * graph capture (the launches are captured, the lookup is not a stream
 * operation).
 */
#define RP_SCAN_BWD_SCRATCH_BYTES (64ll << 20)
int rp_scan_bwd_noalloc(const rp_scan_args* a, const rp_scan_bwd_io* io, void* stream);

/* Validate step arguments on the host without launching anything. */
int rp_step_check(const rp_step_args* a);

/*
 * Fused O(1) step of the SSM core; replaces the ~20 torch ops of
 * Mamba3Block.step between the projections (engine/mamba.py:466-494).
 */
int rp_step(const rp_step_args* a, void* stream);

/*
 * The step with its B / C rows taken from the raw x_proj projections: the
 * BCNorm + p-sum of rp_bcnorm_fwd (engine/mamba.py:297-300, :336-337)
 * followed by rp_step (engine/mamba.py:466-494), the same values as those
 * two calls.  bn->T must be a->R, bn->N the step's d_state, and a->Bc /
 * a->Cc must be bn->Bc / bn->Cc with row stride N: with one rollout per
 * workgroup (small batches) the step kernel computes the rows in its
 * prologue and leaves those buffers unwritten, otherwise rp_bcnorm_fwd
 * writes them ahead of the step.  One launch fewer per layer where launches
 * dominate (a Mamba.step ply at MARS's batch sizes).
 */
int rp_step_bcnorm(const rp_step_args* a, const rp_bcnorm_args* bn, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* REDPANDA_HIP_H */
