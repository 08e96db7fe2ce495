"""GPU parity of the fused SSM input prologue: BCNorm + MIMO p-sum.

The reference's ops (engine/mamba.py:89 RMSNorm, :297-300, :336-337) run by
torch on the same GPU and inputs are the reference: forward and autograd.
The kernel reduces over the N*P features and over tokens in its own fixed
order, so fp32 results are compared to a few ulp of the terms' magnitude:
outputs 1e-6 relative (norm-wise), gradients of the projections 1e-6
relative to the magnitude of the two terms that make them, weight gradients
1e-6 of the sum of |terms|.  bf16 projections (autocast's x_proj output)
round the projection gradients to bf16 as autograd does: one bf16 ulp.
"""

import ctypes

import pytest
import torch

from redpanda_amd import _lib
from redpanda_amd.bcnorm import hip_bcnorm_psum, make_bcnorm_args

pytestmark = pytest.mark.gpu
dev = "cuda"


def rmsnorm(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def eager(Braw, Craw, wB, wC, P, eps, normalize):
    lead = Braw.shape[:-1]
    N = Braw.shape[-1] // P
    if normalize:
        Braw, Craw = rmsnorm(Braw, wB, eps), rmsnorm(Craw, wC, eps)
    return Braw.view(*lead, N, P).sum(-1), Craw.view(*lead, N, P).sum(-1)


def _inputs(lead, N, P, dt, seed, dt_rank=7):
    g = torch.Generator(device=dev).manual_seed(seed)
    K = N * P
    # the projections as views of one x_proj output (dt_rank + 2 N P features)
    x = (torch.randn(*lead, dt_rank + 2 * K, device=dev, generator=g) * 2).to(dt)
    _, Braw, Craw = x.split([dt_rank, K, K], dim=-1)
    wB = 1 + 0.3 * torch.randn(K, device=dev, generator=g)
    wC = 1 + 0.3 * torch.randn(K, device=dev, generator=g)
    return Braw, Craw, wB, wC


def nrel(a, b):
    a, b = a.detach().float(), b.detach().float()
    return float((a - b).abs().max() / (b.abs().max() + 1e-30))


CASES = [((2, 64), 40, 4), ((3, 17), 20, 4), ((5,), 1, 1), ((2, 9), 64, 2), ((1, 33), 65, 3),
         ((2, 5), 128, 8), ((256,), 16, 4)]


@pytest.mark.parametrize("normalize", [True, False])
@pytest.mark.parametrize("lead,N,P", CASES)
def test_fp32_forward_backward(gpu_lib, lead, N, P, normalize):
    Braw, Craw, wB, wC = _inputs(lead, N, P, torch.float32, seed=N * 10 + P)
    leaves = [t.detach().clone().requires_grad_() for t in (Braw, Craw, wB, wC)]
    Bc, Cc = hip_bcnorm_psum(*leaves, P, 1e-5, normalize)
    g = torch.Generator(device=dev).manual_seed(3)
    gB = torch.randn(Bc.shape, device=dev, generator=g)
    gC = torch.randn(Cc.shape, device=dev, generator=g)
    (Bc * gB + Cc * gC).sum().backward()
    refs = [t.detach().clone().requires_grad_() for t in (Braw, Craw, wB, wC)]
    rB, rC = eager(*refs, P, 1e-5, normalize)
    (rB * gB + rC * gC).sum().backward()
    torch.cuda.synchronize()
    assert Bc.shape == (*lead, N) and Bc.dtype == torch.float32
    assert nrel(Bc, rB) <= 1e-6 and nrel(Cc, rC) <= 1e-6
    assert nrel(leaves[0].grad, refs[0].grad) <= 1e-6
    assert nrel(leaves[1].grad, refs[1].grad) <= 1e-6
    if normalize:
        assert nrel(leaves[2].grad, refs[2].grad) <= 1e-6
        assert nrel(leaves[3].grad, refs[3].grad) <= 1e-6
    else:
        assert leaves[2].grad is None and leaves[3].grad is None


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_low_precision_projections(gpu_lib, dt):
    """Autocast's x_proj output: projections in dt, sums and norms in fp32."""
    lead, N, P = (4, 64), 40, 4
    Braw, Craw, wB, wC = _inputs(lead, N, P, dt, seed=17)
    leaves = [t.detach().clone().requires_grad_() for t in (Braw, Craw, wB, wC)]
    Bc, Cc = hip_bcnorm_psum(*leaves, P, 1e-5, True)
    gB = torch.randn(Bc.shape, device=dev)
    (Bc * gB + Cc).sum().backward()
    refs = [t.detach().clone().requires_grad_() for t in (Braw, Craw, wB, wC)]
    with torch.autocast("cuda", dtype=torch.bfloat16 if dt == torch.bfloat16 else torch.float16):
        rB, rC = eager(*refs, P, 1e-5, True)
    assert rB.dtype == torch.float32
    (rB * gB + rC).sum().backward()
    torch.cuda.synchronize()
    assert leaves[0].grad.dtype == dt
    assert nrel(Bc, rB) <= 1e-6 and nrel(Cc, rC) <= 1e-6
    ulp = 2.0 ** -8 if dt == torch.bfloat16 else 2.0 ** -11
    assert nrel(leaves[0].grad, refs[0].grad) <= 2 * ulp
    assert nrel(leaves[1].grad, refs[1].grad) <= 2 * ulp
    assert nrel(leaves[2].grad, refs[2].grad) <= 1e-5
    assert nrel(leaves[3].grad, refs[3].grad) <= 1e-5


def test_no_tokens(gpu_lib):
    Braw, Craw, wB, wC = _inputs((0,), 40, 4, torch.float32, seed=1)
    leaves = [t.detach().clone().requires_grad_() for t in (Braw, Craw, wB, wC)]
    Bc, Cc = hip_bcnorm_psum(*leaves, 4)
    assert Bc.shape == (0, 40)
    (Bc.sum() + Cc.sum()).backward()
    torch.cuda.synchronize()
    assert torch.equal(leaves[2].grad, torch.zeros_like(wB))


def test_weight_grads_deterministic(gpu_lib):
    Braw, Craw, wB, wC = _inputs((64, 64), 40, 4, torch.bfloat16, seed=2)
    out = []
    for _ in range(2):
        w = [wB.clone().requires_grad_(), wC.clone().requires_grad_()]
        Bc, Cc = hip_bcnorm_psum(Braw, Craw, w[0], w[1], 4)
        (Bc.square().sum() + Cc.sum()).backward()
        out.append((w[0].grad, w[1].grad))
    torch.cuda.synchronize()
    assert torch.equal(out[0][0], out[1][0]) and torch.equal(out[0][1], out[1][1])


def test_views_read_in_place(gpu_lib):
    """The C ABI reads the projections with their row stride (no copies)."""
    lib = _lib.load()
    Braw, Craw, wB, wC = _inputs((6, 10), 20, 4, torch.float32, seed=4)
    Bx, Cx = Braw.reshape(-1, 80), Craw.reshape(-1, 80)
    assert Bx.stride(0) == 7 + 160 and Bx.data_ptr() != Braw.contiguous().data_ptr()
    Bc = torch.empty(60, 20, device=dev)
    Cc = torch.empty(60, 20, device=dev)
    a = make_bcnorm_args(Bx, Cx, wB, wC, 20, 4, 1e-5, True, Bc, Cc)
    _lib.check(lib.rp_bcnorm_fwd(ctypes.byref(a), _lib.stream_of(dev)), lib)
    rB, rC = eager(Braw, Craw, wB, wC, 4, 1e-5, True)
    torch.cuda.synchronize()
    assert nrel(Bc, rB.reshape(60, 20)) <= 1e-6 and nrel(Cc, rC.reshape(60, 20)) <= 1e-6
