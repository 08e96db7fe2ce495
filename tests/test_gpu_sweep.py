"""Seeded shape sweeps of the fused kernels around the scan and step against
torch's ops (the reference's expressions) on the same GPU: odd sizes,
strided and offset views, and every storage-dtype combination the C ABI
accepts.  Each case is small; tolerances as in the per-kernel tests.
"""

import os
import random

import pytest
import torch
import torch.nn.functional as F

from redpanda_amd.bcnorm import hip_bcnorm_psum
from redpanda_amd.mixer import hip_mixer_out
from redpanda_amd.norm import hip_add_rmsnorm
from redpanda_amd.step import compact_beta, full_beta, hip_step

pytestmark = pytest.mark.gpu
dev = "cuda"
DTS = [torch.float32, torch.bfloat16, torch.float16]
ULP = {torch.float32: 2.0 ** -23, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
# RP_SWEEP_SCALE=k draws k times as many cases (new seeds; the first ones unchanged)
SCALE = int(os.environ.get("RP_SWEEP_SCALE", "1"))


def nrel(a, b):
    a, b = a.detach().float(), b.detach().float()
    return float((a - b).abs().max() / (b.abs().max() + 1e-30)) if b.numel() else 0.0


def _view(shape, dt, g, pad, scale=1.0):
    """A (..., D) view with `pad` extra leading elements per row."""
    *lead, D = shape
    base = (torch.randn(*lead, D + pad, device=dev, generator=g) * scale).to(dt)
    return base[..., pad:]


@pytest.mark.parametrize("case", range(12 * SCALE))
def test_mixer_sweep(gpu_lib, case):
    rng = random.Random(100 + case)
    g = torch.Generator(device=dev).manual_seed(case)
    B, L, D = rng.randint(1, 4), rng.randint(1, 40), rng.choice([8, 64, 200, 264, 513, 1024])
    du, dz, k = rng.choice(DTS), rng.choice(DTS), rng.choice([1, 2])
    y = torch.randn(B, L, D, device=dev, generator=g)
    u = _view((B, L, D), du, g, rng.choice([0, 8, 1]))
    z = _view((B, L, D), dz, g, rng.choice([0, D, 3]), scale=3)
    Dp = torch.randn(D, device=dev, generator=g)
    a = [t.detach().clone().requires_grad_() if t.is_contiguous() else t.detach().requires_grad_()
         for t in (y, u, z, Dp)]
    out = hip_mixer_out(*a, k)
    dout = torch.randn(B, L, D, device=dev, generator=g)
    out.backward(dout)
    r = [t.detach().clone().requires_grad_() for t in (y, u, z, Dp)]
    yk = r[0] + r[1] * r[3]
    if k == 2:
        yk = yk + r[1] * r[3]
    ref = yk * F.silu(r[2])
    ref.backward(dout)
    torch.cuda.synchronize()
    tol = 4 * max(ULP[du], ULP[dz], 1e-6 / 4)
    assert nrel(out, ref) <= tol
    assert nrel(a[0].grad, r[0].grad) <= tol
    assert nrel(a[1].grad, r[1].grad) <= 2 * tol
    assert nrel(a[3].grad, r[3].grad) <= tol


@pytest.mark.parametrize("case", range(10 * SCALE))
def test_bcnorm_sweep(gpu_lib, case):
    rng = random.Random(200 + case)
    g = torch.Generator(device=dev).manual_seed(case)
    N, P = rng.randint(1, 128), rng.randint(1, 8)
    T, dt, norm = rng.randint(0, 300), rng.choice(DTS), rng.random() < 0.8
    K = N * P
    x = (torch.randn(T, 3 + 2 * K, device=dev, generator=g) * 2).to(dt)
    Bx, Cx = x[:, 3:3 + K], x[:, 3 + K:]
    wB = 1 + 0.1 * torch.randn(K, device=dev, generator=g)
    wC = 1 + 0.1 * torch.randn(K, device=dev, generator=g)
    a = [Bx.detach().requires_grad_(), Cx.detach().requires_grad_(), wB.clone().requires_grad_(),
         wC.clone().requires_grad_()]
    Bc, Cc = hip_bcnorm_psum(*a, P, 1e-5, norm)
    gB = torch.randn(T, N, device=dev, generator=g)
    (Bc * gB + Cc).sum().backward()
    r = [t.detach().float().requires_grad_() for t in (Bx, Cx)] + \
        [t.clone().requires_grad_() for t in (wB, wC)]

    def ref_norm(v, w):
        if norm:
            v = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-5) * w
        return v.view(T, N, P).sum(-1)

    rB, rC = ref_norm(r[0], r[2]), ref_norm(r[1], r[3])
    (rB * gB + rC).sum().backward()
    torch.cuda.synchronize()
    assert nrel(Bc, rB) <= 1e-6 and nrel(Cc, rC) <= 1e-6
    tol = 4 * max(ULP[dt], 1e-6 / 4)
    if T:
        assert nrel(a[0].grad, r[0].grad) <= tol and nrel(a[1].grad, r[1].grad) <= tol
        if norm:
            assert nrel(a[2].grad, r[2].grad) <= 1e-5 and nrel(a[3].grad, r[3].grad) <= 1e-5


@pytest.mark.parametrize("case", range(8 * SCALE))
def test_rmsnorm_sweep(gpu_lib, case):
    rng = random.Random(300 + case)
    g = torch.Generator(device=dev).manual_seed(case)
    R, d = rng.randint(1, 500), rng.choice([1, 63, 64, 65, 257, 512, 1024, 1100])
    x = _view((R, d), torch.float32, g, rng.choice([0, 5]), scale=2)
    add = None if rng.random() < 0.3 else _view((R, d), rng.choice(DTS), g, rng.choice([0, 7]))
    w = 1 + 0.1 * torch.randn(d, device=dev, generator=g)
    xn, out = hip_add_rmsnorm(x, add, w, 1e-5)
    xr = x if add is None else x + add
    ref = xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + 1e-5) * w
    torch.cuda.synchronize()
    assert torch.equal(xn, xr) and nrel(out, ref) <= 1e-6


@pytest.mark.parametrize("case", range(8 * SCALE))
def test_step_sweep(gpu_lib, case):
    """Gated, softplus-on-load steps in both beta forms against the full-form
    step and torch's gate, across kernel choices (d_state 4..72)."""
    rng = random.Random(400 + case)
    g = torch.Generator(device=dev).manual_seed(case)
    NR, NT = rng.choice([(4, 0), (12, 4), (16, 4), (32, 8), (36, 4), (64, 8), (6, 2), (32, 0),
                         (48, 16), (40, 8)])
    N, R, D = NR + NT, rng.randint(1, 300), rng.choice([32, 100, 256, 300, 1024])
    x = torch.randn(R, D, device=dev, generator=g) - 2
    u = torch.randn(R, D, device=dev, generator=g)
    Bc = torch.randn(R, N, device=dev, generator=g)
    Cc = torch.randn(R, N, device=dev, generator=g)
    Ar = -torch.exp(torch.rand(D, NR, device=dev, generator=g))
    Ai = torch.rand(D, NR, device=dev, generator=g) * 3
    Tk = torch.tanh(torch.randn(D, NT, device=dev, generator=g)) if NT else None
    Dk = torch.randn(D, device=dev, generator=g)
    zdt = rng.choice(DTS)
    z = _view((R, D), zdt, g, rng.choice([0, D]), scale=3)
    h = torch.randn(R, D, N, device=dev, generator=g)
    bp = compact_beta(torch.rand(R, D, device=dev, generator=g) * 0.3,
                      torch.randn(R, N, device=dev, generator=g))
    st_full = (h, full_beta(bp, D).contiguous())
    y0, (h0, b0) = hip_step(x, u, Bc, Cc, Ar, Ai, Tk, Dk, st_full, delta_softplus=True)
    y1, (h1, b1) = hip_step(x, u, Bc, Cc, Ar, Ai, Tk, Dk, (h, bp), delta_softplus=True, z=z)
    torch.cuda.synchronize()
    assert torch.equal(h1, h0) and torch.equal(full_beta(b1, D), b0)
    assert torch.equal(y1, y0 * F.silu(z))


@pytest.mark.parametrize("case", range(16 * SCALE))
def test_step_scan_sweep(gpu_lib, case):
    """One step from a cached state against a length-1 scan from the same
    state, bit for bit (y, h, beta), over d_state 1..128 with random
    rotational / tracking splits, rollout and channel counts: every step
    kernel choice (lane layout; tile with 1, 2 or 4 threads per channel, pad
    states, each gate kind)."""
    from redpanda_amd.scan import hip_scan_with_state
    rng = random.Random(900 + case)
    g = torch.Generator(device=dev).manual_seed(900 + case)
    N = rng.choice([rng.randint(1, 128), 4 * rng.randint(1, 32)])
    NR = rng.choice([N, 0, rng.randint(0, N)])
    NT = N - NR
    cplx = NR > 0 and rng.random() < 0.85
    R, D = rng.randint(1, 600), rng.choice([16, 64, 100, 256, 512])
    dt = F.softplus(torch.randn(R, D, device=dev, generator=g) * 0.5 - 2.0)
    u = torch.randn(R, D, device=dev, generator=g)
    Bc = torch.randn(R, N, device=dev, generator=g)
    Cc = torch.randn(R, N, device=dev, generator=g)
    Ar = -torch.exp(torch.rand(D, NR, device=dev, generator=g) * 3) if NR else None
    Ai = (torch.rand(D, NR, device=dev, generator=g) * 2 - 1) * 3 if cplx else None
    Tk = torch.tanh(torch.randn(D, NT, device=dev, generator=g)) if NT else None
    h = torch.randn(R, D, N, device=dev, generator=g)
    b = torch.randn(R, D, N, device=dev, generator=g) * 0.3
    print(f"[step scan sweep {case}] R={R} D={D} N={N} NR={NR} NT={NT} complex={cplx}", flush=True)
    with torch.no_grad():
        y_s, (h_s, b_s) = hip_scan_with_state(dt[:, None], u[:, None], Bc[:, None], Cc[:, None],
                                              Ar, Ai, Tk, state=(h, b))
        y_t, (h_t, b_t) = hip_step(dt, u, Bc, Cc, Ar, Ai, Tk, torch.zeros(D, device=dev), (h, b))
    torch.cuda.synchronize()
    assert torch.equal(y_t, y_s[:, 0]) and torch.equal(h_t, h_s) and torch.equal(b_t, b_s)


@pytest.mark.parametrize("case", range(8 * SCALE))
def test_step_bcnorm_sweep(gpu_lib, case):
    """The step from raw B / C projections (BCNorm + p-sum inside the step, or
    the BCNorm kernel first, as the batch decides) equals hip_bcnorm_psum
    followed by the step, bit for bit: d_state 4..72, P 1..8, 1..700 rollouts,
    every projection dtype, strided projection views, with and without the
    norm, both beta forms."""
    rng = random.Random(500 + case)
    g = torch.Generator(device=dev).manual_seed(50 + case)
    NR, NT = rng.choice([(4, 0), (12, 4), (16, 4), (32, 8), (36, 4), (64, 8), (6, 2)])
    N, R, D = NR + NT, rng.choice([1, 3, 64, 200, 700]), rng.choice([32, 100, 256, 1024])
    P, dt, norm = rng.choice([1, 2, 4, 8]), rng.choice(DTS), rng.random() < 0.8
    off = rng.choice([0, 3, 32])
    X = (torch.randn(R, off + 2 * N * P + 5, device=dev, generator=g) * 2).to(dt)
    B_raw, C_raw = X[:, off:off + N * P], X[:, off + N * P:off + 2 * N * P]
    wB = torch.rand(N * P, device=dev, generator=g) + 0.5
    wC = torch.rand(N * P, device=dev, generator=g) + 0.5
    x = torch.randn(R, D, device=dev, generator=g) - 2
    u = torch.randn(R, D, device=dev, generator=g)
    Ar = -torch.exp(torch.rand(D, NR, device=dev, generator=g))
    Ai = torch.rand(D, NR, device=dev, generator=g) * 3
    Tk = torch.tanh(torch.randn(D, NT, device=dev, generator=g)) if NT else None
    Dk = torch.randn(D, device=dev, generator=g)
    h = torch.randn(R, D, N, device=dev, generator=g)
    if rng.random() < 0.5:
        beta = compact_beta(torch.rand(R, D, device=dev, generator=g) * 0.3,
                            torch.randn(R, N, device=dev, generator=g))
    else:
        beta = torch.randn(R, D, N, device=dev, generator=g)
    with torch.no_grad():
        Bc, Cc = hip_bcnorm_psum(B_raw, C_raw, wB, wC, P, 1e-5, normalize=norm)
        y0, (h0, b0) = hip_step(x, u, Bc, Cc, Ar, Ai, Tk, Dk, (h, beta), delta_softplus=True)
        y1, (h1, b1) = hip_step(x, u, None, None, Ar, Ai, Tk, Dk, (h, beta), delta_softplus=True,
                                bcnorm=(B_raw, C_raw, wB, wC, P, 1e-5, norm))
    torch.cuda.synchronize()
    same = lambda a, b: torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert same(y1, y0) and same(h1, h0) and same(b1, b0)
