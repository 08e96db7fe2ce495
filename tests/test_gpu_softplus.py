"""GPU parity of softplus(dt) fused into the scan and step kernels.

The reference computes delta = F.softplus(dt_proj(dt_raw)) (engine/mamba.py:
300; beta 1, threshold 20, in fp32 under autocast) and hands delta to the
scan.  Here the kernels read the projection x and apply softplus on load;
the backward returns the gradient of x.  The reference below is torch's
F.softplus on the same GPU, composed with the same HIP scan, so the
comparison isolates the fusion: forward and step to 1e-6 (they agree bit
for bit where the kernel's softplus rounds as torch's does), gradients of
x and of every other input to 1e-6, norm-wise per tensor.
"""

import pytest
import torch
import torch.nn.functional as F

from redpanda_amd.scan import hip_scan_with_state, hip_trapezoidal_scan
from redpanda_amd.step import hip_softplus, hip_step

pytestmark = pytest.mark.gpu
dev = "cuda"


def nrel(a, b):
    a, b = a.detach().float(), b.detach().float()
    return float((a - b).abs().max() / (b.abs().max() + 1e-30))


def _inputs(B, L, D, NR, NT, seed, dt=torch.float32):
    g = torch.Generator(device=dev).manual_seed(seed)
    N = NR + NT
    # dt projections around softplus' knee, a few beyond its threshold (20)
    x = torch.randn(B, L, D, device=dev, generator=g) * 2 - 3
    x.view(-1)[:: 97] = 20.5
    x.view(-1)[1:: 89] = -30.0
    x = x.to(dt)
    u = torch.randn(B, L, D, device=dev, generator=g).to(dt)
    Bc = torch.randn(B, L, N, device=dev, generator=g)
    Cc = torch.randn(B, L, N, device=dev, generator=g)
    Ar = -torch.exp(torch.rand(D, NR, device=dev, generator=g) * 2 - 1) if NR else None
    Ai = (torch.rand(D, NR, device=dev, generator=g) * 2 - 1) * 3 if NR else None
    Tk = torch.tanh(torch.randn(D, NT, device=dev, generator=g)) if NT else None
    return x, u, Bc, Cc, Ar, Ai, Tk


def _leaves(ts):
    return [None if t is None else t.detach().clone().requires_grad_() for t in ts]


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 64, 96, 32, 8), (3, 19, 40, 16, 4), (1, 1, 64, 8, 0)])
def test_scan_softplus_matches_torch_softplus(gpu_lib, shape, dt, bidirectional):
    B, L, D, NR, NT = shape
    ins = _inputs(*shape, seed=sum(shape), dt=dt)
    dy = torch.randn(B, L, D, device=dev)
    a = _leaves(ins)
    y = hip_trapezoidal_scan(*a, NR, NR + NT, bidirectional=bidirectional, delta_softplus=True)
    y.backward(dy)
    r = _leaves(ins)
    delta = F.softplus(r[0].float())   # autocast runs softplus in fp32
    yr = hip_trapezoidal_scan(delta, *r[1:], NR, NR + NT, bidirectional=bidirectional)
    yr.backward(dy)
    torch.cuda.synchronize()
    assert nrel(y, yr) <= 1e-6
    print(f"[softplus scan] {shape} {dt} bi={bidirectional} y bitwise "
          f"{float((y == yr).float().mean()):.6f}", flush=True)
    assert a[0].grad.dtype == dt
    for name, ga, gr in zip(("x", "u", "Bc", "Cc", "Ar", "Ai", "Tk"), a, r):
        if ga is None:
            continue
        tol = 1e-6 if dt == torch.float32 or name not in ("x", "u") else 2.0 ** -8
        assert nrel(ga.grad, gr.grad) <= tol, name


def test_scan_with_state_softplus(gpu_lib):
    B, L, D, NR, NT = 2, 21, 64, 16, 4
    ins = _inputs(B, L, D, NR, NT, seed=5)
    N = NR + NT
    g = torch.Generator(device=dev).manual_seed(6)
    h0 = torch.randn(B, D, N, device=dev, generator=g)
    b0 = torch.randn(B, D, N, device=dev, generator=g)
    a = _leaves(ins + (h0, b0))
    y, (h, beta) = hip_scan_with_state(*a[:7], state=(a[7], a[8]), delta_softplus=True)
    (y.sum() + h.square().sum() + beta.sum()).backward()
    r = _leaves(ins + (h0, b0))
    yr, (hr, br) = hip_scan_with_state(F.softplus(r[0]), *r[1:7], state=(r[7], r[8]))
    (yr.sum() + hr.square().sum() + br.sum()).backward()
    torch.cuda.synchronize()
    assert nrel(y, yr) <= 1e-6 and nrel(h, hr) <= 1e-6 and nrel(beta, br) <= 1e-6
    for ga, gr in zip(a, r):
        if ga is not None:
            assert nrel(ga.grad, gr.grad) <= 1e-6


@pytest.mark.parametrize("R,D,NR,NT", [(300, 256, 16, 4), (7, 96, 32, 8)])
def test_step_softplus(gpu_lib, R, D, NR, NT):
    x, u, Bc, Cc, Ar, Ai, Tk = _inputs(1, R, D, NR, NT, seed=R)
    x, u, Bc, Cc = x[0], u[0], Bc[0], Cc[0]
    N = NR + NT
    g = torch.Generator(device=dev).manual_seed(1)
    st = (torch.randn(R, D, N, device=dev, generator=g), torch.randn(R, D, N, device=dev, generator=g))
    Dk = torch.randn(D, device=dev, generator=g)
    y, (h, b) = hip_step(x, u, Bc, Cc, Ar, Ai, Tk, Dk, st, delta_softplus=True)
    yr, (hr, br) = hip_step(F.softplus(x), u, Bc, Cc, Ar, Ai, Tk, Dk, st)
    torch.cuda.synchronize()
    assert nrel(y, yr) <= 1e-6 and nrel(h, hr) <= 1e-6 and nrel(b, br) <= 1e-6
    print(f"[softplus step] R={R} D={D} h bitwise {float((h == hr).float().mean()):.6f}",
          flush=True)


@pytest.mark.parametrize("bidirectional", [False, True])
def test_inference_forward_equals_training_forward(gpu_lib, bidirectional):
    """Without checkpoints (no autograd) every direction applies softplus on
    load; with them the forward direction caches softplus(x) and the reverse
    direction reads the cache: the same bits either way."""
    B, L, D, NR, NT = 3, 37, 160, 32, 8
    ins = _inputs(B, L, D, NR, NT, seed=41, dt=torch.bfloat16)
    with torch.no_grad():
        y_inf = hip_trapezoidal_scan(*ins, NR, NR + NT, bidirectional=bidirectional,
                                     delta_softplus=True)
    a = _leaves(ins)
    y_tr = hip_trapezoidal_scan(*a, NR, NR + NT, bidirectional=bidirectional,
                                delta_softplus=True)
    torch.cuda.synchronize()
    assert torch.equal(y_inf, y_tr.detach())


def _ulp_err(v, ref64):
    """|v - ref| in units of the fp32 spacing at ref (float64 arithmetic)."""
    import numpy as np
    r32 = ref64.astype(np.float32)
    return np.abs(v.astype(np.float64) - ref64) / np.spacing(np.abs(r32))


def test_softplus_bits_against_float64(gpu_lib):
    """The kernels' softplus itself, read out exactly: one step from a fresh
    state with u = 1, B = C = 1 on the first state (0 on the others) and no
    skip term gives h = (delta * u / 2) B and y = C h = delta / 2
    (engine/mamba.py:481-494 with h = beta_prev = 0), so 2y is the kernel's
    delta bit for bit.  Against float64's log1p(exp(x)): within 3 ulp
    (fp32's log1pf(expf(x)) is within 2.7: the rounding of exp's result
    dominates both), and x itself above the threshold 20."""
    import numpy as np
    R, D, NT = 64, 1024, 4
    g = torch.Generator().manual_seed(77)
    x = torch.cat([torch.rand(R * D // 2, generator=g) * 100 - 80,      # (-80, 20)
                   torch.randn(R * D // 4, generator=g) * 2,            # the knee
                   torch.randn(R * D // 4, generator=g) * 1e-3])
    x[:8] = torch.tensor([20.0, 20.000002, 19.999998, 0.0, -0.0, 25.0, -80.0, 1e-30])
    x = x.view(R, D).to(dev)
    u = torch.ones(R, D, device=dev)
    bc = torch.zeros(R, NT, device=dev)
    bc[:, 0] = 1.0
    Tk = torch.full((D, NT), 0.5, device=dev)
    Dk = torch.zeros(D, device=dev)
    y, _ = hip_step(x, u, bc, bc.clone(), None, None, Tk, Dk, None, delta_softplus=True)
    torch.cuda.synchronize()
    delta = (2.0 * y).cpu().numpy().astype(np.float32)
    xs = x.cpu().numpy()
    xd = xs.astype(np.float64)
    above = xs > 20.0
    ref = np.where(above, xd, np.log1p(np.exp(np.minimum(xd, 20.0))))
    assert np.array_equal(delta[above], xs[above])
    # the standalone pass (rank-1 beta rows built on the host) has the same bits
    assert np.array_equal(hip_softplus(x).cpu().numpy(), delta)
    err = _ulp_err(delta[~above], ref[~above])
    err_torch = _ulp_err(F.softplus(x).cpu().numpy(), ref)[~above]
    print(f"[softplus bits] max {err.max():.2f} ulp (torch fp32 {err_torch.max():.2f}), "
          f"mean {err.mean():.3f} ({err_torch.mean():.3f}), equal to torch "
          f"{float((delta == F.softplus(x).cpu().numpy()).mean()):.4f}", flush=True)
    assert err.max() <= 3.0
