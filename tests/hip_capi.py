"""Direct C-ABI calls for the GPU parity tests (fp32 outputs, no autograd).

The product's autograd wrapper returns gradients in each input's dtype, as the
reference does; parity of the kernels themselves is measured on the fp32
buffers the C ABI writes, whatever the storage dtype of the inputs.
"""

import ctypes

import torch

from redpanda_amd import _lib
from redpanda_amd.scan import make_scan_args


def _dev(t):
    return None if t is None else t.to("cuda").contiguous()


def scan_fwd(c, bidirectional=False, with_ckpt=False, with_state=False, h0=None, beta0=None,
             softplus=False):
    lib = _lib.load()
    delta, u, Bc, Cc = (_dev(c[k]) for k in ("delta", "u", "Bc", "Cc"))
    Ar, Ai, Tk = (_dev(None if c[k] is None else c[k].float()) for k in ("Ar", "Ai", "Tk"))
    h0, beta0 = _dev(h0), _dev(beta0)
    B, L, D = u.shape
    N = Bc.shape[-1]
    a = make_scan_args(delta, u, Bc, Cc, Ar, Ai, Tk, bidirectional, h0=h0, beta0=beta0,
                       delta_softplus=softplus)
    y = torch.empty((B, L, D), dtype=torch.float32, device="cuda")
    ckpt = None
    if with_ckpt:
        nb = lib.rp_scan_ckpt_bytes(ctypes.byref(a))
        assert nb >= 0
        ckpt = torch.empty(max(nb // 4, 1), dtype=torch.float32, device="cuda")
    h = b = None
    if with_state:
        h = torch.empty((B, D, N), dtype=torch.float32, device="cuda")
        b = torch.empty((B, D, N), dtype=torch.float32, device="cuda")
    out = _lib.ScanFwdOut(y.data_ptr(), _lib.ptr(ckpt), _lib.ptr(h), _lib.ptr(b))
    _lib.check(lib.rp_scan_fwd(ctypes.byref(a), ctypes.byref(out), _lib.stream_of("cuda")), lib)
    keep = (delta, u, Bc, Cc, Ar, Ai, Tk, h0, beta0)
    return y, ckpt, (h, b), (a, keep)


def scan_fwd_bwd(c, bidirectional=False, dh_last=None, dbeta_last=None, h0=None, beta0=None,
                 softplus=False, grad_in_storage=False):
    """Forward with checkpoints, then backward with upstream c['dy'] -> fp32 grads
    (with an initial state h0, beta0 also its gradients, as grads 'h0' and 'beta0';
    with grad_in_storage, d_delta and d_u in delta's and u's dtypes)."""
    lib = _lib.load()
    y, ckpt, _, (a, keep) = scan_fwd(c, bidirectional, with_ckpt=True, h0=h0, beta0=beta0,
                                     softplus=softplus)
    delta, u, Bc, Cc, Ar, Ai, Tk, h0d, _ = keep
    B, L, D = u.shape
    N = Bc.shape[-1]
    f32 = dict(dtype=torch.float32, device="cuda")
    dy = _dev(c["dy"].float())
    a.grad_in_storage = 1 if grad_in_storage else 0
    gdt = (delta.dtype, u.dtype) if grad_in_storage else (torch.float32, torch.float32)
    g = {"delta": torch.empty((B, L, D), dtype=gdt[0], device="cuda"),
         "u": torch.empty((B, L, D), dtype=gdt[1], device="cuda"),
         "Bc": torch.empty((B, L, N), **f32), "Cc": torch.empty((B, L, N), **f32),
         "Ar": None if Ar is None else torch.empty_like(Ar),
         "Ai": None if Ai is None else torch.empty_like(Ai),
         "Tk": None if Tk is None else torch.empty_like(Tk)}
    if h0d is not None:
        g["h0"] = torch.empty_like(h0d)
        g["beta0"] = torch.empty_like(h0d)
    wb = lib.rp_scan_bwd_work_bytes(ctypes.byref(a))
    work = torch.empty(max(wb, 256), dtype=torch.uint8, device="cuda")
    dh = _dev(dh_last)
    db = _dev(dbeta_last)
    io = _lib.ScanBwdIO(dy=dy.data_ptr(), ckpt=_lib.ptr(ckpt), dh_last=_lib.ptr(dh),
                        dbeta_last=_lib.ptr(db), d_delta=g["delta"].data_ptr(),
                        d_u=g["u"].data_ptr(), d_Bc=g["Bc"].data_ptr(), d_Cc=g["Cc"].data_ptr(),
                        d_A_real=_lib.ptr(g["Ar"]), d_A_imag=_lib.ptr(g["Ai"]),
                        d_track=_lib.ptr(g["Tk"]), d_h0=_lib.ptr(g.get("h0")),
                        d_beta0=_lib.ptr(g.get("beta0")), work=work.data_ptr(),
                        work_bytes=work.numel())
    _lib.check(lib.rp_scan_bwd(ctypes.byref(a), ctypes.byref(io), _lib.stream_of("cuda")), lib)
    torch.cuda.synchronize()
    return y.cpu(), {k: (None if v is None else v.cpu()) for k, v in g.items()}
