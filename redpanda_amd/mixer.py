"""The mixer's output gate on the HIP kernel: out = (y + k u D) * silu(z).

Replaces the elementwise ops between the scan and out_proj in
Mamba3Block.forward (engine/mamba.py:262-265, with the D-skip of :350 /
:375): the skip u * D added once per scan direction (k = 1 causal, 2
bidirectional) and the y * silu(z) gate.  Forward and backward are one pass
each over (B, L, D) instead of the five to nine elementwise kernels autograd
runs for those ops.  Rounding follows those ops: silu(z) is rounded to z's
dtype before the product, gradients come back in each input's dtype.
"""

import ctypes

import torch

from redpanda_amd import _lib


def _code(t):
    try:
        return _lib.DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"redpanda_amd mixer out: unsupported dtype {t.dtype}") from None


def _inner_contig(t):
    return t if t.stride(-1) == 1 else t.contiguous()


def make_mixer_args(y, u, z, Dskip, k_skip, out, dtype_out=None):
    B, L, D = u.shape
    a = _lib.MixerOutArgs()
    a.B, a.L, a.D = B, L, D
    a.k_skip, a.dtype_u, a.dtype_z = k_skip, _code(u), _code(z)
    if dtype_out is not None:
        a.dtype_out = _lib.DTYPE_CODES[dtype_out]
    else:
        a.dtype_out = _lib.RP_F32 if out is None else _code(out)
    a.y = y.data_ptr()
    a.u, a.u_sb, a.u_sl = u.data_ptr(), u.stride(0), u.stride(1)
    a.z, a.z_sb, a.z_sl = z.data_ptr(), z.stride(0), z.stride(1)
    a.Dskip = Dskip.data_ptr()
    a.out = _lib.ptr(out)
    return a


class _HipMixerOut(torch.autograd.Function):

    @staticmethod
    def forward(ctx, y, u, z, Dskip, k_skip, out_dtype):
        lib = _lib.load()
        y = y.to(torch.float32).contiguous()
        u, z = _inner_contig(u), _inner_contig(z)
        Dc = Dskip.detach().to(torch.float32).contiguous()
        out = torch.empty(u.shape, dtype=out_dtype, device=u.device)
        a = make_mixer_args(y, u, z, Dc, k_skip, out)
        ctx.out_dtype = out_dtype
        _lib.check(lib.rp_mixer_out_fwd(ctypes.byref(a), _lib.stream_of(u.device)), lib)
        ctx.k_skip = k_skip
        ctx.dtypes = (y.dtype, u.dtype, z.dtype, Dskip.dtype)
        if any(ctx.needs_input_grad[:4]):
            ctx.save_for_backward(y, u, z, Dc)
        return out

    @staticmethod
    def backward(ctx, dout):
        lib = _lib.load()
        y, u, z, Dc = ctx.saved_tensors
        dev = u.device
        dout = dout.to(ctx.out_dtype).contiguous()
        a = make_mixer_args(y, u, z, Dc, ctx.k_skip, None, dtype_out=ctx.out_dtype)
        dy = torch.empty(u.shape, dtype=torch.float32, device=dev)
        du = torch.empty(u.shape, dtype=u.dtype, device=dev)
        dz = torch.empty(z.shape, dtype=z.dtype, device=dev)
        dD = torch.empty(Dc.shape, dtype=torch.float32, device=dev)
        wbytes = lib.rp_mixer_out_work_bytes(ctypes.byref(a))
        _lib.check(0 if wbytes >= 0 else -1, lib)
        work = torch.empty(max(wbytes, 256), dtype=torch.uint8, device=dev)
        g = _lib.MixerOutGrad(dout=dout.data_ptr(), dy=dy.data_ptr(), du=du.data_ptr(),
                              dz=dz.data_ptr(), dD=dD.data_ptr(), work=work.data_ptr(),
                              work_bytes=work.numel())
        _lib.check(lib.rp_mixer_out_bwd(ctypes.byref(a), ctypes.byref(g), _lib.stream_of(dev)), lib)
        need = ctx.needs_input_grad
        grads = (dy, du, dz, dD.to(ctx.dtypes[3]))
        return (*(gr if need[i] else None for i, gr in enumerate(grads)), None, None)


def hip_mixer_out(y, u, z, Dskip, k_skip=1, out_dtype=torch.float32):
    """(y + k_skip * u * Dskip) * silu(z), (B, L, D) in out_dtype: fp32, or
    the autocast dtype of the projection it feeds (the fp32 result rounded
    as autocast's cast rounds it; its gradient then arrives in that dtype).

    y: the scan output (B, L, D) (fp32; without the skip); u: the scan input
    and z: the gate branch, (B, L, D) each, fp32 / bf16 / fp16, inner stride
    1 (other strides free: z may be a chunk of the in_proj output); Dskip:
    (D,).  k_skip = 2 for a bidirectional layer, whose skip is added once per
    direction (engine/mamba.py:255-258, :350)."""
    if u.dim() != 3 or y.shape != u.shape or z.shape != u.shape:
        raise ValueError(f"mixer out: y {tuple(y.shape)}, u {tuple(u.shape)}, z {tuple(z.shape)} "
                         "must all be (B, L, D)")
    if Dskip.shape != (u.shape[-1],):
        raise ValueError(f"mixer out: D {tuple(Dskip.shape)} must be ({u.shape[-1]},)")
    if k_skip not in (1, 2):
        raise ValueError("mixer out: k_skip must be 1 or 2")
    if out_dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"mixer out: unsupported output dtype {out_dtype}")
    for t in (y, u, z, Dskip):
        if not t.is_cuda:
            raise RuntimeError("redpanda_amd mixer out: inputs must be ROCm device tensors")
    return _HipMixerOut.apply(y, u, z, Dskip, int(k_skip), out_dtype)
