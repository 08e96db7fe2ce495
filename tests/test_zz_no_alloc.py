"""rp_scan_bwd_noalloc, the allocation-free scan backward: the same kernels as
rp_scan_bwd with their scratch in the library's static device array.  Its
results must equal rp_scan_bwd's bit for bit, also on a second call that
finds the first call's partials still in the scratch, and a shape beyond the
scratch must be refused on the host."""

import ctypes
import math

import pytest
import torch
import torch.nn.functional as F

from redpanda_amd import _lib
from tests import hip_capi

pytestmark = pytest.mark.gpu


def _case(seed, B, L, D, NR, NT):
    gen = torch.Generator().manual_seed(seed)
    N = NR + NT
    c = dict(u=torch.randn(B, L, D, generator=gen),
             delta=F.softplus(torch.randn(B, L, D, generator=gen) * 0.5 - 2.0),
             Bc=torch.randn(B, L, N, generator=gen), Cc=torch.randn(B, L, N, generator=gen),
             Ar=-torch.exp(torch.rand(D, NR, generator=gen) * 3.0),
             Ai=(torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi,
             Tk=torch.tanh(torch.randn(D, NT, generator=gen) * 1.5) if NT else None,
             dy=torch.randn(B, L, D, generator=gen))
    return c


def _backward(entry, c, bidirectional, in_storage=False):
    """Forward with checkpoints, then the backward through `entry`; every
    output the caller owns is allocated here, the scratch only by
    rp_scan_bwd (a workspace) or not at all (rp_scan_bwd_noalloc).
    in_storage: d_delta / d_u in the inputs' dtypes (grad_in_storage)."""
    lib = _lib.load()
    _, ckpt, _, (a, keep) = hip_capi.scan_fwd(c, bidirectional, with_ckpt=True)
    delta, u, Bc, Cc, Ar, Ai, Tk = keep[:7]
    a.grad_in_storage = 1 if in_storage else 0
    B, L, D = u.shape
    N = Bc.shape[-1]
    f32 = dict(dtype=torch.float32, device="cuda")
    dy = c["dy"].to("cuda").contiguous()
    g = {"delta": torch.full((B, L, D), float("nan"), dtype=delta.dtype if in_storage
                             else torch.float32, device="cuda"),
         "u": torch.full((B, L, D), float("nan"), dtype=u.dtype if in_storage else torch.float32,
                         device="cuda"),
         "Bc": torch.full((B, L, N), float("nan"), **f32),
         "Cc": torch.full((B, L, N), float("nan"), **f32),
         "Ar": torch.full_like(Ar, float("nan")), "Ai": torch.full_like(Ai, float("nan")),
         "Tk": None if Tk is None else torch.full_like(Tk, float("nan"))}
    work = None
    if entry == "rp_scan_bwd":
        work = torch.empty(max(lib.rp_scan_bwd_work_bytes(ctypes.byref(a)), 256),
                           dtype=torch.uint8, device="cuda")
    io = _lib.ScanBwdIO(dy=dy.data_ptr(), ckpt=_lib.ptr(ckpt), d_delta=g["delta"].data_ptr(),
                        d_u=g["u"].data_ptr(), d_Bc=g["Bc"].data_ptr(), d_Cc=g["Cc"].data_ptr(),
                        d_A_real=_lib.ptr(g["Ar"]), d_A_imag=_lib.ptr(g["Ai"]),
                        d_track=_lib.ptr(g["Tk"]), work=_lib.ptr(work),
                        work_bytes=0 if work is None else work.numel())
    _lib.check(getattr(lib, entry)(ctypes.byref(a), ctypes.byref(io), _lib.stream_of("cuda")),
               lib)
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in g.items() if v is not None}


def _same_bits(x, y):
    bits = lambda t: t.view(torch.int16 if t.element_size() == 2 else torch.int32)
    return all(x[k].dtype == y[k].dtype and torch.equal(bits(x[k]), bits(y[k])) for k in x)


def test_noalloc_equals_workspace_entry_twice(gpu_lib):
    """Two calls in a row, the second smaller: bit for bit rp_scan_bwd's."""
    cases = [(_case(71, B=6, L=64, D=256, NR=32, NT=8), True),
             (_case(72, B=2, L=33, D=96, NR=12, NT=4), False)]
    for c, bidir in cases:
        print(f"case B={c['u'].shape[0]} L={c['u'].shape[1]} D={c['u'].shape[2]} "
              f"bidir={bidir}", flush=True)
        free = _backward("rp_scan_bwd_noalloc", c, bidir)
        ref = _backward("rp_scan_bwd", c, bidir)
        assert all(torch.isfinite(v).all() for v in free.values())
        assert _same_bits(free, ref)


def test_noalloc_gradients_in_storage_dtype(gpu_lib):
    """bf16 inputs with grad_in_storage: d_delta / d_u leave in bf16, and a
    bidirectional scan keeps its first direction's fp32 sums in the static
    scratch; two calls in a row, the second smaller, bit for bit
    rp_scan_bwd's."""
    to16 = lambda c: {k: (v.bfloat16() if k in ("delta", "u", "Bc", "Cc") else v)
                      for k, v in c.items()}
    for c, bidir in ((to16(_case(73, B=4, L=64, D=256, NR=32, NT=8)), True),
                     (to16(_case(74, B=2, L=40, D=96, NR=12, NT=4)), True)):
        print(f"case B={c['u'].shape[0]} L={c['u'].shape[1]} D={c['u'].shape[2]} bf16 "
              f"bidir={bidir}", flush=True)
        free = _backward("rp_scan_bwd_noalloc", c, bidir, in_storage=True)
        ref = _backward("rp_scan_bwd", c, bidir, in_storage=True)
        assert free["delta"].dtype == torch.bfloat16 and free["u"].dtype == torch.bfloat16
        assert all(torch.isfinite(v).all() for v in free.values())
        assert _same_bits(free, ref)


def test_noalloc_refuses_a_shape_beyond_the_scratch(gpu_lib):
    """The Eval-Mamba layer at batch 256 needs ~315 MB of scratch: refused on
    the host with RP_ERR_WORKSPACE before anything is launched."""
    lib = _lib.load()
    t = torch.zeros(64, device="cuda")
    p = t.data_ptr()
    a = _lib.ScanArgs()
    a.B, a.L, a.D, a.N, a.NR, a.NT = 256, 64, 1536, 40, 32, 8
    a.dtype_delta = a.dtype_u = a.dtype_B = a.dtype_C = _lib.RP_F32
    a.bidirectional = 1
    a.delta, a.delta_sb, a.delta_sl = p, 64 * 1536, 1536
    a.u, a.u_sb, a.u_sl = p, 64 * 1536, 1536
    a.Bc, a.Bc_sb, a.Bc_sl = p, 64 * 40, 40
    a.Cc, a.Cc_sb, a.Cc_sl = p, 64 * 40, 40
    a.A_real, a.A_imag, a.track = p, p, p
    need = lib.rp_scan_bwd_work_bytes(ctypes.byref(a))
    assert need > (64 << 20)
    io = _lib.ScanBwdIO(dy=p, ckpt=p, d_delta=p, d_u=p, d_Bc=p, d_Cc=p, d_A_real=p, d_A_imag=p,
                        d_track=p)
    st = lib.rp_scan_bwd_noalloc(ctypes.byref(a), ctypes.byref(io), _lib.stream_of("cuda"))
    assert st == -4
    assert b"static scratch holds" in lib.rp_last_error()


def test_noalloc_first_call_under_graph_capture(gpu_lib):
    """The first call of a process, captured into a HIP graph (the use the
    entry point is for), replayed four times with other allocation-free
    calls between the replays: bit for bit rp_scan_bwd's every time.  A
    child process, so the captured call is the process's first (the one that
    looks the scratch up)."""
    import os
    import subprocess
    import sys
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_graph_capture.py")
    r = subprocess.run([sys.executable, "-u", script], capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    assert r.returncode == 0, r.stderr[-3000:]
    assert r.stdout.strip().endswith("ok")
