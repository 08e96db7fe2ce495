"""Residual add + RMSNorm of the batched step's residual stream, on the HIP
kernel (engine/mamba.py:82-89 RMSNorm; the pre-norm loop of Mamba.step,
:592-597).  Forward only: used by the inference loop of Mamba.step when no
autograd graph is being recorded; training keeps torch's ops.
"""

import ctypes

import torch

from redpanda_amd import _lib


def hip_add_rmsnorm(x, add, w, eps):
    """(x + add, RMSNorm(x + add) * w) for fp32 rows x (R, d); add: None or
    (R, d) in fp32 / bf16 / fp16 (x itself is normalised then, and returned
    as the first element).  Torch's op order: (x' * rsqrt(mean(x'^2) + eps))
    * w, the mean as the sum times the fp32 reciprocal of d."""
    if x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda:
        raise ValueError("add_rmsnorm: x must be a (R, d) fp32 device tensor")
    R, d = x.shape
    if w.shape != (d,):
        raise ValueError(f"add_rmsnorm: weight {tuple(w.shape)} must be ({d},)")
    lib = _lib.load()
    if x.stride(-1) != 1:
        x = x.contiguous()
    wc = w  # only its data pointer is used
    if w.dtype is not torch.float32 or not w.is_contiguous():
        wc = w.detach().to(torch.float32).contiguous()
    a = _lib.RmsNormArgs()
    a.rows, a.d, a.eps = R, d, float(eps)
    a.x, a.x_sr = x.data_ptr(), x.stride(0)
    a.w = wc.data_ptr()
    out = torch.empty((R, d), dtype=torch.float32, device=x.device)
    a.out = out.data_ptr()
    x_new = x
    if add is not None:
        if add.shape != (R, d):
            raise ValueError(f"add_rmsnorm: add {tuple(add.shape)} must be {(R, d)}")
        if add.stride(-1) != 1:
            add = add.contiguous()
        try:
            a.dtype_add = _lib.DTYPE_CODES[add.dtype]
        except KeyError:
            raise TypeError(f"add_rmsnorm: unsupported dtype {add.dtype}") from None
        a.add, a.add_sr = add.data_ptr(), add.stride(0)
        x_new = torch.empty((R, d), dtype=torch.float32, device=x.device)
        a.x_out = x_new.data_ptr()
    _lib.check(lib.rp_rmsnorm_fwd(ctypes.byref(a), _lib.stream_of(x.device)), lib)
    return x_new, out
