"""Autograd-aware entry points of the HIP trapezoidal selective scan.

`hip_trapezoidal_scan` keeps the signature and contract of the reference's
`triton_trapezoidal_scan` (engine/triton_scan.py:318-337): contracted B/C,
y returned in fp32 WITHOUT the u*D skip, gradients returned in each input's
dtype (:313-315).  It adds a `bidirectional` keyword for the fused
two-direction forward, and `hip_scan_with_state` returns the final recurrent
state (the reference's return_state path, engine/mamba.py:377-379) with a
backward that accepts gradients of that state.
"""

import ctypes

import torch

from redpanda_amd import _lib

HAS_HIP = False
try:  # availability flag, like the reference's HAS_TRITON (engine/triton_scan.py:30-37)
    import os as _os
    HAS_HIP = torch.cuda.is_available() and _os.path.exists(_lib.LIB_PATH)
except Exception:  # pragma: no cover
    HAS_HIP = False


def _inner_contig(t):
    return t if t.stride(-1) == 1 else t.contiguous()


def _param(t):
    return None if t is None else t.detach().to(torch.float32).contiguous()


def _code(t):
    try:
        return _lib.DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"redpanda_amd scan: unsupported dtype {t.dtype}") from None


def make_scan_args(delta, u, Bc, Cc, Ar, Ai, Tk, bidirectional, h0=None, beta0=None,
                   delta_softplus=False):
    """ScanArgs for device tensors (delta/u (B,L,D), Bc/Cc (B,L,N); optional
    (B,D,N) fp32 contiguous initial state h0, beta0).  delta_softplus: delta
    holds the dt projection x and the kernels use softplus(x)."""
    B, L, D = u.shape
    N = Bc.shape[-1]
    NR = 0 if Ar is None else Ar.shape[-1]
    NT = 0 if Tk is None else Tk.shape[-1]
    a = _lib.ScanArgs()
    a.B, a.L, a.D, a.N, a.NR, a.NT = B, L, D, N, NR, NT
    a.dtype_delta, a.dtype_u, a.dtype_B, a.dtype_C = _code(delta), _code(u), _code(Bc), _code(Cc)
    a.bidirectional = 1 if bidirectional else 0
    a.delta_softplus = 1 if delta_softplus else 0
    a.delta, a.delta_sb, a.delta_sl = delta.data_ptr(), delta.stride(0), delta.stride(1)
    a.u, a.u_sb, a.u_sl = u.data_ptr(), u.stride(0), u.stride(1)
    a.Bc, a.Bc_sb, a.Bc_sl = Bc.data_ptr(), Bc.stride(0), Bc.stride(1)
    a.Cc, a.Cc_sb, a.Cc_sl = Cc.data_ptr(), Cc.stride(0), Cc.stride(1)
    a.A_real, a.A_imag, a.track = _lib.ptr(Ar), _lib.ptr(Ai), _lib.ptr(Tk)
    a.h0, a.beta0 = _lib.ptr(h0), _lib.ptr(beta0)
    return a


def _check_shapes(delta, u, Bc, Cc, Ar, Ai, Tk):
    if u.dim() != 3 or delta.shape != u.shape:
        raise ValueError(f"scan: delta {tuple(delta.shape)} and u {tuple(u.shape)} must be (B, L, D)")
    B, L, D = u.shape
    if Bc.dim() != 3 or Bc.shape[:2] != (B, L) or Cc.shape != Bc.shape:
        raise ValueError(f"scan: B/C {tuple(Bc.shape)} / {tuple(Cc.shape)} must be (B, L, N)")
    N = Bc.shape[-1]
    NR = 0 if Ar is None else Ar.shape[-1]
    NT = 0 if Tk is None else Tk.shape[-1]
    if Ar is not None and Ar.shape != (D, NR):
        raise ValueError(f"scan: A_real {tuple(Ar.shape)} must be (D, n_rot)")
    if Ai is not None and (Ar is None or Ai.shape != Ar.shape):
        raise ValueError("scan: A_imag needs A_real of the same shape")
    if Tk is not None and Tk.shape != (D, NT):
        raise ValueError(f"scan: track {tuple(Tk.shape)} must be (D, n_track)")
    if NR + NT != N:
        raise ValueError(f"scan: n_rot ({NR}) + n_track ({NT}) != d_state ({N})")
    if not 1 <= N <= _lib.MAX_STATE:
        raise ValueError(f"scan: d_state {N} outside [1, {_lib.MAX_STATE}]")
    for t in (delta, u, Bc, Cc):
        if not t.is_cuda:
            raise RuntimeError("redpanda_amd scan: inputs must be ROCm device tensors")


class _HipScan(torch.autograd.Function):
    """y = S(x) (or S(x) + flip(S(flip(x)))), optionally from an initial state
    (h0, beta0) and optionally returning the final state (h_last, beta_last)."""

    @staticmethod
    def forward(ctx, delta, u, Bc, Cc, Ar, Ai, Tk, h0, beta0, bidirectional, with_state,
                delta_softplus=False):
        lib = _lib.load()
        delta, u, Bc, Cc = (_inner_contig(t) for t in (delta, u, Bc, Cc))
        Arc, Aic, Tkc = _param(Ar), _param(Ai), _param(Tk)
        h0c, b0c = _param(h0), _param(beta0)
        B, L, D = u.shape
        N = Bc.shape[-1]
        dev = u.device
        args = make_scan_args(delta, u, Bc, Cc, Arc, Aic, Tkc, bidirectional, h0c, b0c,
                              delta_softplus)
        y = torch.empty((B, L, D), dtype=torch.float32, device=dev)
        need_grad = any(ctx.needs_input_grad[:9])
        ckpt = None
        if need_grad:
            nbytes = lib.rp_scan_ckpt_bytes(ctypes.byref(args))
            _lib.check(0 if nbytes >= 0 else -1, lib)
            ckpt = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=dev)
        h_last = beta_last = None
        if with_state:
            h_last = torch.empty((B, D, N), dtype=torch.float32, device=dev)
            beta_last = torch.empty((B, D, N), dtype=torch.float32, device=dev)
        out = _lib.ScanFwdOut(y.data_ptr(), _lib.ptr(ckpt), _lib.ptr(h_last), _lib.ptr(beta_last))
        _lib.check(lib.rp_scan_fwd(ctypes.byref(args), ctypes.byref(out), _lib.stream_of(dev)), lib)
        ctx.bidirectional = bidirectional
        ctx.with_state = with_state
        ctx.delta_softplus = delta_softplus
        ctx.in_dtypes = tuple(None if t is None else t.dtype
                              for t in (delta, u, Bc, Cc, Ar, Ai, Tk, h0, beta0))
        if need_grad:
            ctx.save_for_backward(delta, u, Bc, Cc, Arc, Aic, Tkc, h0c, b0c, ckpt)
        if with_state:
            return y, h_last, beta_last
        return y

    @staticmethod
    def backward(ctx, dy, dh_last=None, dbeta_last=None):
        lib = _lib.load()
        delta, u, Bc, Cc, Arc, Aic, Tkc, h0c, b0c, ckpt = ctx.saved_tensors
        B, L, D = u.shape
        N = Bc.shape[-1]
        dev = u.device
        args = make_scan_args(delta, u, Bc, Cc, Arc, Aic, Tkc, ctx.bidirectional, h0c, b0c,
                              ctx.delta_softplus)
        f32 = dict(dtype=torch.float32, device=dev)
        dy = torch.zeros((B, L, D), **f32) if dy is None else dy.to(torch.float32).contiguous()
        if dh_last is not None:
            dh_last = dh_last.to(torch.float32).contiguous()
        if dbeta_last is not None:
            dbeta_last = dbeta_last.to(torch.float32).contiguous()
        # d_delta and d_u leave the kernel in delta's and u's dtypes (rounded as
        # torch converts), so 16-bit inputs need no conversion pass
        if delta.dtype != torch.float32 or u.dtype != torch.float32:
            args.grad_in_storage = 1
        d_delta = torch.empty((B, L, D), dtype=delta.dtype, device=dev)
        d_u = torch.empty((B, L, D), dtype=u.dtype, device=dev)
        d_B = torch.empty((B, L, N), **f32)
        d_C = torch.empty((B, L, N), **f32)
        d_Ar = torch.empty_like(Arc) if Arc is not None else None
        d_Ai = torch.empty_like(Aic) if Aic is not None else None
        d_Tk = torch.empty_like(Tkc) if Tkc is not None else None
        d_h0 = torch.empty((B, D, N), **f32) if h0c is not None else None
        d_b0 = torch.empty((B, D, N), **f32) if h0c is not None else None
        wbytes = lib.rp_scan_bwd_work_bytes(ctypes.byref(args))
        _lib.check(0 if wbytes >= 0 else -1, lib)
        work = torch.empty(max(wbytes, 256), dtype=torch.uint8, device=dev)
        io = _lib.ScanBwdIO(dy=dy.data_ptr(), ckpt=_lib.ptr(ckpt), dh_last=_lib.ptr(dh_last),
                            dbeta_last=_lib.ptr(dbeta_last), d_delta=d_delta.data_ptr(),
                            d_u=d_u.data_ptr(), d_Bc=d_B.data_ptr(), d_Cc=d_C.data_ptr(),
                            d_A_real=_lib.ptr(d_Ar), d_A_imag=_lib.ptr(d_Ai),
                            d_track=_lib.ptr(d_Tk), d_h0=_lib.ptr(d_h0), d_beta0=_lib.ptr(d_b0),
                            work=work.data_ptr(), work_bytes=work.numel())
        _lib.check(lib.rp_scan_bwd(ctypes.byref(args), ctypes.byref(io), _lib.stream_of(dev)), lib)
        grads = [d_delta, d_u, d_B, d_C, d_Ar, d_Ai, d_Tk, d_h0, d_b0]
        out = []
        for g, dt, need in zip(grads, ctx.in_dtypes, ctx.needs_input_grad[:9]):
            out.append(g.to(dt) if (g is not None and need) else None)
        return (*out, None, None, None)


def hip_trapezoidal_scan(delta, u, B_contracted, C_contracted, A_real, A_imag, track,
                         n_rot, n_state, bidirectional=False, delta_softplus=False):
    """Drop-in for the reference's triton_trapezoidal_scan (engine/triton_scan.py:318-337).

    delta, u: (B, L, D); B_contracted, C_contracted: (B, L, N); A_real,
    A_imag: (D, n_rot) or None; track: (D, n_state - n_rot) tanh gates or
    None.  Returns y (B, L, D) fp32 without the u*D skip.  With
    bidirectional=True returns S(x) + flip(S(flip(x))) from one fused launch.
    With delta_softplus=True, `delta` is the dt projection x and the scan runs
    on F.softplus(x) (engine/mamba.py:300), differentiable in x.
    """
    if A_real is not None and A_real.shape[-1] != n_rot:
        raise ValueError(f"scan: A_real has {A_real.shape[-1]} states, n_rot={n_rot}")
    if track is None and n_state != n_rot:
        raise ValueError("scan: track gates missing for the tracking states")
    if A_real is None and n_rot != 0:
        raise ValueError("scan: n_rot > 0 needs A_real")
    _check_shapes(delta, u, B_contracted, C_contracted, A_real, A_imag, track)
    if B_contracted.shape[-1] != n_state:
        raise ValueError(f"scan: B_contracted has {B_contracted.shape[-1]} states, n_state={n_state}")
    return _HipScan.apply(delta, u, B_contracted, C_contracted, A_real, A_imag, track,
                          None, None, bool(bidirectional), False, bool(delta_softplus))


def hip_scan_with_state(delta, u, B_contracted, C_contracted, A_real, A_imag, track,
                        state=None, delta_softplus=False):
    """Causal scan continuing from `state` = (h0, beta0) (or the zero state)
    and returning (y, (h_last, beta_last)): the return_state path of the
    reference (engine/mamba.py:377-379) on the HIP kernel.  Differentiable in
    every input, the initial state and both outputs.  h_last, beta_last are
    exactly the cache step() continues from."""
    _check_shapes(delta, u, B_contracted, C_contracted, A_real, A_imag, track)
    h0 = beta0 = None
    if state is not None:
        h0, beta0 = state
        B, L, D = u.shape
        N = B_contracted.shape[-1]
        if h0.shape != (B, D, N) or beta0.shape != (B, D, N):
            raise ValueError(f"scan: initial state must be (B, D, N) = {(B, D, N)}")
        if L < 1:
            raise ValueError("scan: an initial state needs L >= 1")
    y, h, beta = _HipScan.apply(delta, u, B_contracted, C_contracted, A_real, A_imag, track,
                                h0, beta0, False, True, bool(delta_softplus))
    return y, (h, beta)


# Names the reference's callers import (engine/mamba.py:344).
HAS_TRITON = HAS_HIP
triton_trapezoidal_scan = hip_trapezoidal_scan
