"""The SSM input prologue on the HIP kernel: BCNorm and the MIMO p-sum.

Replaces, per token, RMSNorm on the B and C projections and their sum over
the p MIMO channels (engine/mamba.py:297-300, :89 and :336-337): one pass
forward and one backward instead of the dozen elementwise and reduction
kernels autograd runs for those ops.  Outputs are fp32, as torch's sum
returns them under autocast; gradients come back in the projections' dtype.
"""

import ctypes

import torch

from redpanda_amd import _lib


def _code(t):
    try:
        return _lib.DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"redpanda_amd bcnorm: unsupported dtype {t.dtype}") from None


def _rows(x):
    """(T, K) view with one row stride and inner stride 1, copying only if
    the leading dimensions cannot be flattened into one stride."""
    x2 = x.reshape(-1, x.shape[-1]) if x.dim() != 2 else x
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def make_bcnorm_args(Bx, Cx, wB, wC, N, P, eps, normalize, Bc=None, Cc=None):
    a = _lib.BcNormArgs()
    a.T, a.N, a.P = Bx.shape[0], N, P
    a.dtype_x, a.normalize, a.eps, a.reserved = _code(Bx), 1 if normalize else 0, float(eps), 0
    a.B_raw, a.B_sr = Bx.data_ptr(), Bx.stride(0)
    a.C_raw, a.C_sr = Cx.data_ptr(), Cx.stride(0)
    a.wB, a.wC = _lib.ptr(wB), _lib.ptr(wC)
    a.Bc, a.Cc = _lib.ptr(Bc), _lib.ptr(Cc)
    return a


class _HipBcNorm(torch.autograd.Function):

    @staticmethod
    def forward(ctx, B_raw, C_raw, wB, wC, P, eps, normalize):
        lib = _lib.load()
        lead = B_raw.shape[:-1]
        K = B_raw.shape[-1]
        N = K // P
        Bx, Cx = _rows(B_raw), _rows(C_raw)
        if Cx.dtype != Bx.dtype:
            Cx = Cx.to(Bx.dtype)
        wBc = wB.detach().to(torch.float32).contiguous() if normalize else None
        wCc = wC.detach().to(torch.float32).contiguous() if normalize else None
        dev = Bx.device
        Bc = torch.empty((Bx.shape[0], N), dtype=torch.float32, device=dev)
        Cc = torch.empty((Bx.shape[0], N), dtype=torch.float32, device=dev)
        a = make_bcnorm_args(Bx, Cx, wBc, wCc, N, P, eps, normalize, Bc, Cc)
        _lib.check(lib.rp_bcnorm_fwd(ctypes.byref(a), _lib.stream_of(dev)), lib)
        ctx.meta = (lead, N, P, eps, normalize, B_raw.dtype, C_raw.dtype,
                    None if wB is None else wB.dtype, None if wC is None else wC.dtype)
        ctx.save_for_backward(Bx, Cx, wBc, wCc)
        return Bc.view(*lead, N), Cc.view(*lead, N)

    @staticmethod
    def backward(ctx, dBc, dCc):
        lib = _lib.load()
        lead, N, P, eps, normalize, bdt, cdt, wbdt, wcdt = ctx.meta
        Bx, Cx, wBc, wCc = ctx.saved_tensors
        dev = Bx.device
        T, K = Bx.shape
        f32 = dict(dtype=torch.float32, device=dev)
        dBc = torch.zeros((T, N), **f32) if dBc is None else dBc.reshape(T, N).to(torch.float32).contiguous()
        dCc = torch.zeros((T, N), **f32) if dCc is None else dCc.reshape(T, N).to(torch.float32).contiguous()
        a = make_bcnorm_args(Bx, Cx, wBc, wCc, N, P, eps, normalize)
        dBx = torch.empty((T, K), dtype=Bx.dtype, device=dev)
        dCx = torch.empty((T, K), dtype=Bx.dtype, device=dev)
        dwB = torch.empty(K, **f32) if normalize else None
        dwC = torch.empty(K, **f32) if normalize else None
        wb = lib.rp_bcnorm_work_bytes(ctypes.byref(a))
        _lib.check(0 if wb >= 0 else -1, lib)
        work = torch.empty(max(wb, 256), dtype=torch.uint8, device=dev)
        g = _lib.BcNormGrad(dBc=dBc.data_ptr(), dCc=dCc.data_ptr(), dB_raw=dBx.data_ptr(),
                            dC_raw=dCx.data_ptr(), dwB=_lib.ptr(dwB), dwC=_lib.ptr(dwC),
                            work=work.data_ptr(), work_bytes=work.numel())
        _lib.check(lib.rp_bcnorm_bwd(ctypes.byref(a), ctypes.byref(g), _lib.stream_of(dev)), lib)
        need = ctx.needs_input_grad
        dB = dBx.view(*lead, K).to(bdt) if need[0] else None
        dC = dCx.view(*lead, K).to(cdt) if need[1] else None
        gwB = dwB.to(wbdt) if (normalize and need[2]) else None
        gwC = dwC.to(wcdt) if (normalize and need[3]) else None
        return dB, dC, gwB, gwC, None, None, None


def hip_bcnorm_psum(B_raw, C_raw, wB, wC, P, eps=1e-5, normalize=True):
    """(Bc, Cc): RMSNorm(B_raw) and RMSNorm(C_raw) (weights wB, wC; eps)
    summed over the P MIMO channels of each state, fp32 (..., N).

    B_raw, C_raw: (..., N*P) projections (fp32 / bf16 / fp16, inner stride
    1; views of one x_proj output are read in place).  normalize=False is
    the layer without BCNorm: plain sums over p (wB, wC unused)."""
    K = B_raw.shape[-1]
    if C_raw.shape != B_raw.shape:
        raise ValueError(f"bcnorm: B_raw {tuple(B_raw.shape)} and C_raw {tuple(C_raw.shape)} differ")
    if P < 1 or K % P:
        raise ValueError(f"bcnorm: feature size {K} is not a multiple of P={P}")
    if normalize and (wB is None or wC is None or wB.shape != (K,) or wC.shape != (K,)):
        raise ValueError(f"bcnorm: norm weights must be ({K},)")
    for t in (B_raw, C_raw):
        if not t.is_cuda:
            raise RuntimeError("redpanda_amd bcnorm: inputs must be ROCm device tensors")
    return _HipBcNorm.apply(B_raw, C_raw, wB if normalize else None, wC if normalize else None,
                            int(P), float(eps), bool(normalize))
