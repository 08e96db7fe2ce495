"""GPU parity of the fused mixer output gate, out = (y + k u D) * silu(z).

The reference runs these as torch elementwise ops (engine/mamba.py:262-265,
D-skip at :350 and once per direction at :255-258), so the reference here
is those same ops on the same GPU with the same inputs, forward and
autograd.  In fp32 every output is the same sequence of IEEE operations as
torch's kernels (checked here to 1e-6 relative, element-wise), dD is a sum
in another order (1e-6 of the sum of magnitudes).  With bf16 / fp16 u and z,
silu(z) and the gradients of u and z are rounded to those dtypes as
autocast's ops do; a one-ulp difference of the fp32 exp before that rounding
may flip it, so those compare to one storage ulp.
"""

import ctypes

import pytest
import torch
import torch.nn.functional as F

from redpanda_amd import _lib
from redpanda_amd.mixer import hip_mixer_out, make_mixer_args

pytestmark = pytest.mark.gpu
dev = "cuda"

ULP = {torch.float32: 2.0 ** -23, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}


def eager(y, u, z, D, k):
    """The reference's op sequence."""
    yk = y + u * D
    if k == 2:
        yk = yk + u * D
    return yk * F.silu(z)


def _inputs(B, L, D, dt=torch.float32, seed=0, z_view=True):
    g = torch.Generator(device=dev).manual_seed(seed)
    y = torch.randn(B, L, D, device=dev, generator=g)
    u = torch.randn(B, L, D, device=dev, generator=g).to(dt)
    if z_view:
        # z as the second half of an in_proj output (time stride 2D)
        xz = torch.randn(B, L, 2 * D, device=dev, generator=g).to(dt) * 3
        z = xz.chunk(2, dim=-1)[1]
    else:
        z = (torch.randn(B, L, D, device=dev, generator=g) * 3).to(dt)
    Dp = torch.randn(D, device=dev, generator=g)
    return y, u, z, Dp


def _close(a, b, rtol, what, scale=None):
    """|a - b| <= rtol * (|b| + scale) element-wise (scale: the magnitude of
    the terms that cancel in b, where they do)."""
    a, b = a.detach().float(), b.detach().float()
    ref = b.abs() if scale is None else b.abs() + scale.detach().float()
    err = ((a - b).abs() / (ref + 1e-30)).where(ref != 0, (a - b).abs())
    assert float(err.max()) <= rtol, f"{what}: max rel err {float(err.max()):.3e} > {rtol:.1e}"


def _dz_scale(dout, y, u, z, D, k):
    """Magnitude of the terms of dz = ds sig (1 + z (1 - sig)), which cancel
    where silu' vanishes (z near -1.28)."""
    z = z.float()
    sig = torch.sigmoid(z)
    yk = y + k * u.float() * D
    return (dout * yk).abs() * sig * (1 + z.abs() * (1 - sig))


# d_inner % 8 == 0 with 16-byte aligned rows takes the 8-channel vector
# path; 300 and 1001 take the scalar one
SHAPES = [(2, 64, 256), (3, 17, 320), (1, 1, 1000), (5, 33, 64), (16, 64, 1024),
          (2, 9, 300), (1, 3, 1001)]


@pytest.mark.parametrize("k", [1, 2])
@pytest.mark.parametrize("shape", SHAPES)
def test_forward_fp32(gpu_lib, shape, k):
    y, u, z, Dp = _inputs(*shape, seed=sum(shape) + k)
    out = hip_mixer_out(y, u, z, Dp, k)
    ref = eager(y, u, z, Dp, k)
    torch.cuda.synchronize()
    _close(out, ref, 1e-6, "out")
    print(f"[mixer fwd] {shape} k={k} bitwise fraction "
          f"{float((out == ref).float().mean()):.6f}", flush=True)


@pytest.mark.parametrize("k", [1, 2])
@pytest.mark.parametrize("shape", SHAPES)
def test_backward_fp32(gpu_lib, shape, k):
    y, u, z, Dp = _inputs(*shape, seed=3 * sum(shape) + k)
    ins = [t.detach().clone().requires_grad_() for t in (y, u, z, Dp)]
    hip_mixer_out(*ins, k).backward(torch.ones_like(y) * 0.5 + y.detach().sin())
    refs = [t.detach().clone().requires_grad_() for t in (y, u, z, Dp)]
    eager(*refs, k).backward(torch.ones_like(y) * 0.5 + y.detach().sin())
    torch.cuda.synchronize()
    dout = torch.ones_like(y) * 0.5 + y.sin()
    _close(ins[0].grad, refs[0].grad, 1e-6, "dy")
    _close(ins[1].grad, refs[1].grad, 1e-6, "du")
    _close(ins[2].grad, refs[2].grad, 1e-6, "dz", _dz_scale(dout, y, u, z, Dp, k))
    # dD: sums over B*L rows in another order; bound by the sum of |terms|
    dyk = (0.5 + y.sin()) * F.silu(z)
    scale = (dyk * u).abs().sum(dim=(0, 1)) * k
    err = (ins[3].grad - refs[3].grad).abs()
    assert float((err / (scale + 1e-30)).max()) <= 1e-6, "dD"


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k", [1, 2])
def test_low_precision_inputs(gpu_lib, dt, k):
    B, L, D = 4, 48, 384
    y, u, z, Dp = _inputs(B, L, D, dt, seed=11 + k)
    ins = [y.clone().requires_grad_(), u.clone().requires_grad_(), z.clone().requires_grad_(),
           Dp.clone().requires_grad_()]
    out = hip_mixer_out(*ins, k)
    dout = torch.randn(B, L, D, device=dev)
    out.backward(dout)
    refs = [y.clone().requires_grad_(), u.clone().requires_grad_(), z.clone().requires_grad_(),
            Dp.clone().requires_grad_()]
    ref = eager(*refs, k)
    ref.backward(dout)
    torch.cuda.synchronize()
    assert out.dtype == ref.dtype == torch.float32
    assert ins[1].grad.dtype == dt and ins[2].grad.dtype == dt
    # silu(z) is rounded to dt by both: one storage ulp of slack for it
    tol = 2 * ULP[dt]
    _close(out, ref, tol, "out")
    _close(ins[0].grad, refs[0].grad, tol, "dy")
    _close(ins[1].grad, refs[1].grad, 2 * tol, "du")
    # dz: ds is rounded to dt before the product, then the product is rounded
    _close(ins[2].grad, refs[2].grad, 3 * tol, "dz", _dz_scale(dout, y, u, z, Dp, k))
    dyk = dout * F.silu(z.float()).to(dt).float()
    scale = (dyk * u.float()).abs().sum(dim=(0, 1)) * k
    err = (ins[3].grad - refs[3].grad).abs()
    assert float((err / (scale + 1e-30)).max()) <= tol


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_unaligned_views_take_scalar_path(gpu_lib, dt):
    """u and z as views starting one element into a wider tensor (rows no
    longer 16-byte aligned): same results as the torch ops."""
    B, L, D = 3, 20, 512
    g = torch.Generator(device=dev).manual_seed(21)
    y = torch.randn(B, L, D, device=dev, generator=g)
    u = torch.randn(B, L, D + 1, device=dev, generator=g).to(dt)[..., 1:]
    z = (torch.randn(B, L, 2 * D + 1, device=dev, generator=g) * 3).to(dt)[..., 1 + D:]
    Dp = torch.randn(D, device=dev, generator=g)
    ins = [t.clone().requires_grad_() if t.is_contiguous() else t.detach().requires_grad_()
           for t in (y, u, z, Dp)]
    out = hip_mixer_out(*ins, 2)
    out.backward(y)
    refs = [t.detach().clone().requires_grad_() for t in (y, u, z, Dp)]
    ref = eager(*refs, 2)
    ref.backward(y)
    torch.cuda.synchronize()
    tol = 1e-6 if dt == torch.float32 else 2 * ULP[dt]
    _close(out, ref, tol, "out")
    _close(ins[1].grad, refs[1].grad, 2 * tol, "du")
    _close(ins[2].grad, refs[2].grad, 3 * tol, "dz", _dz_scale(y, y, u, z, Dp, 2))


def test_empty_rows_give_zero_dD(gpu_lib):
    y, u, z, Dp = _inputs(2, 0, 300)
    ins = [t.clone().requires_grad_() for t in (y, u, z, Dp)]
    out = hip_mixer_out(*ins, 2)
    assert out.shape == (2, 0, 300)
    out.sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(ins[3].grad, torch.zeros_like(Dp))


def test_dD_deterministic(gpu_lib):
    y, u, z, Dp = _inputs(8, 64, 512, seed=5)
    grads = []
    for _ in range(2):
        Dg = Dp.clone().requires_grad_()
        hip_mixer_out(y, u, z, Dg, 2).backward(y)
        grads.append(Dg.grad)
    torch.cuda.synchronize()
    assert torch.equal(grads[0], grads[1])


def test_in_place_over_y(gpu_lib):
    """The C ABI allows out == y (each element read before it is written)."""
    lib = _lib.load()
    y, u, z, Dp = _inputs(3, 40, 768, seed=9)
    ref = eager(y, u, z, Dp, 1)
    yy = y.clone()
    a = make_mixer_args(yy, u, z, Dp, 1, yy)
    _lib.check(lib.rp_mixer_out_fwd(ctypes.byref(a), _lib.stream_of(dev)), lib)
    torch.cuda.synchronize()
    _close(yy, ref, 1e-6, "out in place")


def test_block_forward_uses_fused_gate(gpu_lib):
    """Mamba3Block.forward (fused prologue and gate) against the block's
    scan with the eager prologue and gate, causal and bidirectional, output
    and parameter gradients (norm-wise per tensor)."""
    from redpanda_amd import mamba as hm

    for bi in (False, True):
        torch.manual_seed(0)
        cfg = hm.MambaConfig(d_model=128, n_layer=1, d_state=40, n_track_state=8,
                             bidirectional=bi)
        blk = hm.Mamba3Block(cfg).to(dev)
        x = torch.randn(3, 24, 128, device=dev)

        def eager_block(x):
            xb, z = blk.in_proj(x).chunk(2, dim=-1)
            xb = F.silu(xb)
            delta, B, C = blk._ssm_proj(xb)
            Ar, Ai = blk._compute_A()
            y = blk._selective_scan_trapezoidal(xb, delta, Ar, Ai, B, C, blk.D,
                                                bidirectional=bi)
            return blk.out_proj(y * F.silu(z))

        out = blk(x)
        out.square().sum().backward()
        g_fused = {k: p.grad.clone() for k, p in blk.named_parameters()}
        blk.zero_grad()
        ref = eager_block(x)
        ref.square().sum().backward()
        torch.cuda.synchronize()
        # norm-wise: the block's B/C prologue is fused too, so the scan's
        # inputs differ from the eager block's in the last bits
        d = ((out - ref).abs().max() / ref.abs().max()).detach()
        assert float(d) <= 1e-5, f"block out bi={bi}: {float(d):.2e}"
        for k, p in blk.named_parameters():
            d = (g_fused[k] - p.grad).abs().max() / (p.grad.abs().max() + 1e-30)
            assert float(d) <= 1e-5, f"grad {k} bi={bi}: {float(d):.2e}"


@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [512, 300])
def test_autocast_dtype_output(gpu_lib, odt, D):
    """Output in out_proj's autocast dtype: the same bits as torch's fp32
    result cast to it; its (16-bit) gradient gives the same gradients as the
    fp32 output with that gradient upcast, as autocast's cast backward does."""
    y, u, z, Dp = _inputs(3, 21, D, torch.bfloat16, seed=D)
    a16 = [t.clone().requires_grad_() for t in (y, u, z, Dp)]
    out16 = hip_mixer_out(*a16, 2, out_dtype=odt)
    ref = eager(y, u, z, Dp, 2)
    assert out16.dtype == odt and torch.equal(out16, ref.to(odt))
    g = torch.randn(3, 21, D, device=dev).to(odt)
    out16.backward(g)
    a32 = [t.clone().requires_grad_() for t in (y, u, z, Dp)]
    hip_mixer_out(*a32, 2).backward(g.float())
    torch.cuda.synchronize()
    for p16, p32 in zip(a16, a32):
        assert torch.equal(p16.grad, p32.grad)
