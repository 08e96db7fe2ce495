"""Fused O(1) recurrent step of the SSM core (one token for a batch of rollouts).

`hip_step` replaces the torch ops of Mamba3Block.step between the input
projections and out_proj (engine/mamba.py:466-494) with one kernel that reads
the (h, beta) state once and writes the new state once.  The new state is a
pair of fresh tensors, as in the reference (callers clone / cat / expand cached
states, engine/mars_search.py:222-224, engine/search_mamba.py:177-187), unless
`out` passes preallocated (possibly aliasing) buffers.

A state that is an expanded view of one (D, N) state -- a batch-1 cache
fanned out to R rollouts, as SearchMamba._expand_cache returns it -- is read
in place by every rollout (no copies).

Compact states: beta_t = (dt_t u_t) outer B_t is rank-1, so a cache may carry
it as rows [dt*u | B] of D + N floats (`(h, bp)` with bp (R, D + N)) instead
of (R, D, N).  The step then moves half the bytes and returns the same
format; results are the same bits as with the full form, since beta_prev is
formed by the multiply that produced it.  `compact_beta` builds such a row
from a step's inputs; `full_beta` expands one back.
"""

import ctypes

import torch

from redpanda_amd import _lib
from redpanda_amd.bcnorm import _rows as _bn_rows, make_bcnorm_args


# (the conversions are skipped where a tensor already qualifies: at the
# batch sizes MARS runs, a step is bound by the host's per-op cost)
def _f32c(t):
    """fp32 contiguous (only the data pointer is used: no autograd)."""
    if t.dtype is torch.float32 and t.is_contiguous():
        return t
    return t.detach().to(torch.float32).contiguous()


def _rows(t):
    if t.dtype is not torch.float32:
        t = t.to(torch.float32)
    return t if t.stride(-1) == 1 else t.contiguous()


def is_compact(beta):
    """Whether a cached beta is in the rank-1 row form (R, D + N)."""
    return beta.dim() == 2


def compact_beta(dtu, Bc):
    """Rank-1 rows [dt*u | B] (fp32, (R, D + N)) of beta = (dt*u) outer B."""
    return torch.cat([dtu.to(torch.float32), Bc.to(torch.float32)], dim=-1)


class _Softplus(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        xf = x.detach().to(torch.float32).contiguous()
        out = torch.empty_like(xf)
        lib = _lib.load()
        _lib.check(lib.rp_softplus(xf.data_ptr(), out.data_ptr(), xf.numel(),
                                   _lib.stream_of(xf.device)), lib)
        ctx.save_for_backward(xf)
        ctx.in_dtype = x.dtype
        return out

    @staticmethod
    def backward(ctx, g):
        # torch's softplus backward: g z / (z + 1), z = exp(x); g above 20
        (xf,) = ctx.saved_tensors
        z = torch.exp(xf)
        return torch.where(xf > 20.0, g, g * z / (z + 1.0)).to(ctx.in_dtype)


def hip_softplus(x):
    """fp32 softplus(x) of the dt projection (engine/mamba.py:300) with the
    bits the scan and step kernels compute on load (delta_softplus), for
    rank-1 beta rows built on the host; differentiable (d/dx = sigmoid(x))."""
    if not x.is_cuda:
        raise RuntimeError("hip_softplus: x must be on a ROCm device")
    return _Softplus.apply(x)


def full_beta(bp, D):
    """The (R, D, N) beta of rank-1 rows bp (R, D + N): (dt*u)[:, :, None] * B[:, None, :]."""
    return bp[..., :D, None] * bp[..., None, D:]


def _state_pair(h, b, R, D, N):
    """(h, beta, broadcast, rank1) for the kernel: per-rollout contiguous
    states, or one shared state when both are stride-0 expansions of one;
    beta full (R, D, N) or in rank-1 rows (R, D + N)."""
    rank1 = is_compact(b)
    bshape = (R, D + N) if rank1 else (R, D, N)
    if h.shape != (R, D, N) or b.shape != bshape:
        raise ValueError(f"step: state must be h {(R, D, N)} and beta {bshape}")
    if h.dtype is not torch.float32:
        h = h.to(torch.float32)
    if b.dtype is not torch.float32:
        b = b.to(torch.float32)
    if R > 1 and h.stride(0) == 0 and b.stride(0) == 0 and h[0].is_contiguous() and \
            b[0].is_contiguous():
        return h, b, 1, rank1
    return h.contiguous(), b.contiguous(), 0, rank1


def hip_step(delta, u, Bc, Cc, A_real, A_imag, track, Dskip, state=None, out=None,
             delta_softplus=False, compact=False, z=None, bcnorm=None):
    """One step for R rollouts.

    delta, u: (R, D); Bc, Cc: (R, N) (contracted over p); A_real/A_imag:
    (D, NR) or None; track: (D, NT) or None; Dskip: (D,); state: (h, beta)
    fp32 (R, D, N) (or an expansion of one (1, D, N) state) or None for a
    fresh state.  Returns (y (R, D) incl. u*D, (h_new, beta_new)).  With
    delta_softplus, `delta` is the dt projection x and the step uses
    F.softplus(x) (engine/mamba.py:300).  beta in rank-1 rows (R, D + N)
    returns rank-1 rows; with no state, `compact` chooses the form returned.
    With the gate branch z (R, D) given, y is returned gated: y * silu(z)
    (silu rounded to z's dtype, as torch computes it).  out: None, or the
    (y, h_new, beta_new) buffers to write (y may be None): fp32 contiguous,
    h_new (R, D, N), beta_new in the form of the state; h_new may be the
    input h itself (updated in place), a rank-1 beta_new may not overlap
    the input rows.  bcnorm: None, or (B_raw, C_raw, wB, wC, P, eps,
    normalize), the raw x_proj projections (R, N * P) and BCNorm's weights
    (engine/mamba.py:297-300), with Bc and Cc None: the step then takes
    BCNorm + the p-sum itself (rp_step_bcnorm; the values of
    hip_bcnorm_psum's rows), inside the step kernel at small batches.
    """
    lib = _lib.load()
    R, D = u.shape
    bn_args = None
    if bcnorm is not None:
        if Bc is not None or Cc is not None:
            raise ValueError("step: give either Bc, Cc or bcnorm")
        B_raw, C_raw, wB, wC, P, eps, normalize = bcnorm
        if B_raw.shape != C_raw.shape or B_raw.shape[0] != R or B_raw.shape[-1] % P:
            raise ValueError(f"step: bcnorm projections must be (R, N * P) = ({R}, N * {P})")
        Bx, Cx = _bn_rows(B_raw), _bn_rows(C_raw)
        if Cx.dtype != Bx.dtype:
            Cx = Cx.to(Bx.dtype)
        wBc = _f32c(wB) if normalize else None
        wCc = _f32c(wC) if normalize else None
        Nb = Bx.shape[-1] // P
        Bc = torch.empty((R, Nb), dtype=torch.float32, device=u.device)
        Cc = torch.empty((R, Nb), dtype=torch.float32, device=u.device)
        bn_args = make_bcnorm_args(Bx, Cx, wBc, wCc, Nb, P, eps, normalize, Bc, Cc)
    N = Bc.shape[-1]
    NR = 0 if A_real is None else A_real.shape[-1]
    NT = 0 if track is None else track.shape[-1]
    if NR + NT != N:
        raise ValueError(f"step: n_rot ({NR}) + n_track ({NT}) != d_state ({N})")
    if delta.shape != (R, D) or Bc.shape != (R, N) or Cc.shape != (R, N):
        raise ValueError("step: delta/u must be (R, D) and B/C (R, N)")
    dev = u.device
    delta, u, Bc, Cc = (_rows(t) for t in (delta, u, Bc, Cc))
    Ar = None if A_real is None else _f32c(A_real)
    Ai = None if A_imag is None else _f32c(A_imag)
    Tk = None if track is None else _f32c(track)
    Dk = _f32c(Dskip)
    h_in = beta_in = None
    broadcast = 0
    rank1 = bool(compact)
    if state is not None:
        h_in, beta_in, broadcast, rank1 = _state_pair(state[0], state[1], R, D, N)
    bshape = (R, D + N) if rank1 else (R, D, N)
    if out is None:
        h_out = torch.empty((R, D, N), dtype=torch.float32, device=dev)
        beta_out = torch.empty(bshape, dtype=torch.float32, device=dev)
        y = torch.empty((R, D), dtype=torch.float32, device=dev)
    else:
        y, h_out, beta_out = out
        if y is None:
            y = torch.empty((R, D), dtype=torch.float32, device=dev)
        for name, t, shp in (("y", y, (R, D)), ("h", h_out, (R, D, N)), ("beta", beta_out, bshape)):
            if (t.shape != shp or t.dtype != torch.float32 or t.device != dev or
                    not t.is_contiguous()):
                raise ValueError(f"step: out {name} must be a contiguous fp32 {shp} tensor on {dev}")
    a = _lib.StepArgs()
    a.R, a.D, a.N, a.NR, a.NT = R, D, N, NR, NT
    a.delta, a.delta_sr = delta.data_ptr(), delta.stride(0)
    a.u, a.u_sr = u.data_ptr(), u.stride(0)
    a.Bc, a.Bc_sr = Bc.data_ptr(), Bc.stride(0)
    a.Cc, a.Cc_sr = Cc.data_ptr(), Cc.stride(0)
    a.h_in, a.beta_in = _lib.ptr(h_in), _lib.ptr(beta_in)
    a.A_real, a.A_imag, a.track = _lib.ptr(Ar), _lib.ptr(Ai), _lib.ptr(Tk)
    a.Dskip = Dk.data_ptr()
    a.h_out, a.beta_out, a.y = h_out.data_ptr(), beta_out.data_ptr(), y.data_ptr()
    a.broadcast_state = broadcast
    a.delta_softplus = 1 if delta_softplus else 0
    a.beta_rank1 = 1 if rank1 else 0
    if z is not None:
        if z.shape != (R, D) or not z.is_cuda:
            raise ValueError(f"step: z must be a (R, D) = {(R, D)} device tensor")
        if z.stride(-1) != 1:
            z = z.contiguous()
        a.z, a.z_sr = z.data_ptr(), z.stride(0)
        try:
            a.dtype_z = _lib.DTYPE_CODES[z.dtype]
        except KeyError:
            raise TypeError(f"step: unsupported dtype {z.dtype} for z") from None
    if bn_args is None:
        _lib.check(lib.rp_step(ctypes.byref(a), _lib.stream_of(dev)), lib)
    else:
        _lib.check(lib.rp_step_bcnorm(ctypes.byref(a), ctypes.byref(bn_args), _lib.stream_of(dev)),
                   lib)
    return y, (h_out, beta_out)
