"""GPU parity of the fused step kernel: against the reference's step
(golden fixture and oracle), step == scan (bit-exact, same arithmetic),
batched == singles, and K-step chains (engine/mars_diagnostics.py:94-164)."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import scan_ref
from tests.conftest import load_golden

pytestmark = pytest.mark.gpu
dev = "cuda"


def _step():
    from redpanda_amd.step import hip_step
    return hip_step


def rel(a, b):
    return scan_ref.rel_err(a.detach().cpu(), b.detach().cpu())


def make_step_case(seed, R, D, NR, NT, complex_=True):
    gen = torch.Generator().manual_seed(seed)
    N = NR + NT
    dt = F.softplus(torch.randn(R, D, generator=gen) * 0.5 - 2.0)
    u = torch.randn(R, D, generator=gen)
    Bc = torch.randn(R, N, generator=gen)
    Cc = torch.randn(R, N, generator=gen)
    Ar = -torch.exp(torch.rand(D, NR, generator=gen) * 3.0) if NR else None
    Ai = (torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi if (NR and complex_) else None
    Tk = torch.tanh(torch.randn(D, NT, generator=gen) * 1.5) if NT else None
    Dk = torch.randn(D, generator=gen)
    h = torch.randn(R, D, N, generator=gen)
    b = torch.randn(R, D, N, generator=gen) * 0.3
    return dict(delta=dt, u=u, Bc=Bc, Cc=Cc, Ar=Ar, Ai=Ai, Tk=Tk, D=Dk, h=h, beta=b)


def to(t):
    return None if t is None else t.to(dev)


@pytest.mark.parametrize("NR,NT,cplx", [(16, 4, True), (12, 4, True), (8, 0, False), (0, 5, True),
                                        (32, 8, True), (64, 8, True), (32, 0, True),
                                        (40, 8, True), (48, 16, True), (64, 16, False),
                                        (20, 4, True), (72, 8, True), (20, 8, True),
                                        (40, 4, True), (56, 4, False), (80, 16, True),
                                        (120, 8, True), (100, 16, True), (16, 0, False),
                                        (64, 0, False), (32, 0, False)])
@pytest.mark.parametrize("fresh", [False, True])
def test_step_matches_reference_step(gpu_lib, NR, NT, cplx, fresh):
    hip_step = _step()
    c = make_step_case(10 + NR + NT, R=5, D=70, NR=NR, NT=NT, complex_=cplx)
    state = None if fresh else (c["h"], c["beta"])
    y_ref, (h_ref, b_ref) = scan_ref.step_core_ref(c["delta"], c["u"], c["Bc"], c["Cc"], c["Ar"],
                                                   c["Ai"], c["Tk"], c["D"], state)
    st = None if fresh else (to(c["h"]), to(c["beta"]))
    y, (h, b) = hip_step(to(c["delta"]), to(c["u"]), to(c["Bc"]), to(c["Cc"]), to(c["Ar"]),
                         to(c["Ai"]), to(c["Tk"]), to(c["D"]), st)
    eh, eb, ey = rel(h, h_ref), rel(b, b_ref), rel(y, y_ref)
    print(f"NR={NR} NT={NT} fresh={fresh}: h {eh:.1e} beta {eb:.1e} y {ey:.1e}")
    assert eh <= 1e-6 and ey <= 1e-6
    assert torch.equal(b.cpu(), b_ref), "beta = (dt*u)*B is computed exactly as the reference"


def test_step_matches_golden_block_step(gpu_lib):
    """The SSM core of the reference's Mamba3Block.step on its own fixture."""
    g = load_golden("step_rot_trk")
    from oracle import model_ref
    cfg = model_ref.MambaConfig(vocab_size=64, n_layer=1, d_model=8, d_state=12,
                                n_track_state=4, mimo_p=2)
    blk = model_ref.Mamba3Block(cfg).eval()
    blk.load_state_dict({k[3:]: v for k, v in g.items() if k.startswith("sd.")})
    hip_step = _step()
    with torch.no_grad():
        xb, z = blk.in_proj(g["x"]).chunk(2, dim=-1)
        xb = F.silu(xb)
        delta, Bm, Cm = blk._ssm_proj(xb)
        Ar, Ai = blk._compute_A()
        y, (h, b) = hip_step(to(delta), to(xb), to(Bm.sum(-1)), to(Cm.sum(-1)), to(Ar), to(Ai),
                             to(blk._track_gate()), to(blk.D), (to(g["h0"]), to(g["beta0"])))
        out = blk.out_proj(y.cpu() * F.silu(z))
    assert rel(h, g["h"]) <= 1e-6
    assert rel(b, g["beta"]) <= 1e-6
    assert rel(out, g["out"]) <= 1e-5


@pytest.mark.parametrize("NR,NT,L", [(12, 4, 37), (32, 8, 64), (16, 4, 20), (64, 8, 19),
                                     (32, 0, 40), (40, 8, 11), (48, 16, 23), (64, 16, 9),
                                     (20, 8, 30), (52, 8, 17)])
def test_step_equals_scan_bitwise(gpu_lib, NR, NT, L):
    """Stepping token by token reproduces the scan's y and final state bit for bit."""
    from redpanda_amd.scan import hip_scan_with_state
    hip_step = _step()
    gen = torch.Generator().manual_seed(NR * 100 + L)
    B, D = 3, 72
    N = NR + NT
    dt = F.softplus(torch.randn(B, L, D, generator=gen) * 0.5 - 2.0).to(dev)
    u = torch.randn(B, L, D, generator=gen).to(dev)
    Bc = torch.randn(B, L, N, generator=gen).to(dev)
    Cc = torch.randn(B, L, N, generator=gen).to(dev)
    Ar = (-torch.exp(torch.rand(D, NR, generator=gen) * 3.0)).to(dev)
    Ai = ((torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi).to(dev)
    Tk = torch.tanh(torch.randn(D, NT, generator=gen) * 1.5).to(dev)
    Dz = torch.zeros(D, device=dev)
    with torch.no_grad():
        y_scan, (h_scan, b_scan) = hip_scan_with_state(dt, u, Bc, Cc, Ar, Ai, Tk)
        state, ys = None, []
        for t in range(L):
            yt, state = hip_step(dt[:, t], u[:, t], Bc[:, t], Cc[:, t], Ar, Ai, Tk, Dz, state)
            ys.append(yt)
    assert torch.equal(torch.stack(ys, 1), y_scan)
    assert torch.equal(state[0], h_scan)
    assert torch.equal(state[1], b_scan)


@pytest.mark.parametrize("NR,NT", [(16, 4), (12, 8), (28, 8), (32, 0), (20, 4), (48, 16), (64, 16),
                                   (72, 8), (20, 8), (36, 8), (52, 8), (64, 8), (68, 8),
                                   (76, 8), (80, 16), (100, 16), (112, 16), (128, 0), (90, 14)])
def test_step_equals_scan_many_rollouts(gpu_lib, NR, NT):
    """Thousands of rollouts over whole 256-channel tiles (several rollouts
    per workgroup, a short last group): still the scan's bits."""
    from redpanda_amd.scan import hip_scan_with_state
    hip_step = _step()
    gen = torch.Generator().manual_seed(7 * NR + NT)
    B, L, D = 2101, 3, 512
    N = NR + NT
    dt = F.softplus(torch.randn(B, L, D, generator=gen) * 0.5 - 2.0).to(dev)
    u = torch.randn(B, L, D, generator=gen).to(dev)
    Bc = torch.randn(B, L, N, generator=gen).to(dev)
    Cc = torch.randn(B, L, N, generator=gen).to(dev)
    Ar = (-torch.exp(torch.rand(D, NR, generator=gen) * 3.0)).to(dev)
    Ai = ((torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi).to(dev)
    Tk = torch.tanh(torch.randn(D, NT, generator=gen) * 1.5).to(dev)
    Dz = torch.zeros(D, device=dev)
    with torch.no_grad():
        y_scan, (h_scan, b_scan) = hip_scan_with_state(dt, u, Bc, Cc, Ar, Ai, Tk)
        state, ys = None, []
        for t in range(L):
            yt, state = hip_step(dt[:, t], u[:, t], Bc[:, t], Cc[:, t], Ar, Ai, Tk, Dz, state)
            ys.append(yt)
    assert torch.equal(torch.stack(ys, 1), y_scan)
    assert torch.equal(state[0], h_scan)
    assert torch.equal(state[1], b_scan)


def test_scan_prefix_then_step_continues(gpu_lib):
    """scan([0, s)) state + steps over [s, L) == scan([0, L)) (bitwise)."""
    from redpanda_amd.scan import hip_scan_with_state
    hip_step = _step()
    gen = torch.Generator().manual_seed(77)
    B, L, D, NR, NT, s = 2, 30, 64, 16, 4, 11
    N = NR + NT
    dt = F.softplus(torch.randn(B, L, D, generator=gen) * 0.5 - 2.0).to(dev)
    u = torch.randn(B, L, D, generator=gen).to(dev)
    Bc = torch.randn(B, L, N, generator=gen).to(dev)
    Cc = torch.randn(B, L, N, generator=gen).to(dev)
    Ar = (-torch.exp(torch.rand(D, NR, generator=gen) * 3.0)).to(dev)
    Ai = ((torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi).to(dev)
    Tk = torch.tanh(torch.randn(D, NT, generator=gen)).to(dev)
    Dz = torch.zeros(D, device=dev)
    with torch.no_grad():
        y_full, _ = hip_scan_with_state(dt, u, Bc, Cc, Ar, Ai, Tk)
        _, state = hip_scan_with_state(dt[:, :s].contiguous(), u[:, :s].contiguous(),
                                       Bc[:, :s].contiguous(), Cc[:, :s].contiguous(), Ar, Ai, Tk)
        for t in range(s, L):
            yt, state = hip_step(dt[:, t], u[:, t], Bc[:, t], Cc[:, t], Ar, Ai, Tk, Dz, state)
            assert torch.equal(yt, y_full[:, t]), t


def test_batched_equals_singles_and_chains(gpu_lib):
    """(a) one batched step == N single steps; (b) a K-step batched chain == K
    single chains (engine/mars_diagnostics.py:110-143)."""
    hip_step = _step()
    c = make_step_case(42, R=6, D=96, NR=16, NT=4)
    p = [to(c[k]) for k in ("Ar", "Ai", "Tk", "D")]
    gen = torch.Generator().manual_seed(3)
    K = 8
    dts = F.softplus(torch.randn(K, 6, 96, generator=gen) * 0.5 - 2).to(dev)
    us = torch.randn(K, 6, 96, generator=gen).to(dev)
    Bs = torch.randn(K, 6, 20, generator=gen).to(dev)
    Cs = torch.randn(K, 6, 20, generator=gen).to(dev)
    st = (to(c["h"]), to(c["beta"]))
    with torch.no_grad():
        yb, _ = hip_step(dts[0], us[0], Bs[0], Cs[0], *p, st)
        for i in range(6):
            yi, _ = hip_step(dts[0, i:i + 1], us[0, i:i + 1], Bs[0, i:i + 1], Cs[0, i:i + 1], *p,
                             (st[0][i:i + 1].clone(), st[1][i:i + 1].clone()))
            assert torch.equal(yi[0], yb[i])
        chain = st
        for k in range(K):
            yk, chain = hip_step(dts[k], us[k], Bs[k], Cs[k], *p, chain)
        for i in range(6):
            si = (st[0][i:i + 1].clone(), st[1][i:i + 1].clone())
            for k in range(K):
                yi, si = hip_step(dts[k, i:i + 1], us[k, i:i + 1], Bs[k, i:i + 1],
                                  Cs[k, i:i + 1], *p, si)
            assert torch.equal(yi[0], yk[i])
            assert torch.equal(si[0][0], chain[0][i])


@pytest.mark.parametrize("R,D,NR,NT", [(300, 512, 16, 4), (37, 100, 12, 8), (64, 256, 20, 5),
                                     (300, 512, 32, 0), (50, 256, 64, 16), (40, 128, 40, 4),
                                     (33, 256, 24, 4)])
def test_broadcast_state_equals_copies(gpu_lib, R, D, NR, NT):
    """A (1, D, N) state expanded to R rollouts (a stride-0 view, read in
    place) steps exactly like its materialised copies."""
    hip_step = _step()
    c = make_step_case(5 * R + NT, R=R, D=D, NR=NR, NT=NT)
    p = [to(c[k]) for k in ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk", "D")]
    h1, b1 = to(c["h"][:1]), to(c["beta"][:1])
    hv, bv = h1.expand(R, -1, -1), b1.expand(R, -1, -1)
    assert hv.stride(0) == 0
    with torch.no_grad():
        y_v, (h_v, b_v) = hip_step(*p, (hv, bv))
        y_c, (h_c, b_c) = hip_step(*p, (hv.contiguous(), bv.contiguous()))
    assert torch.equal(y_v, y_c) and torch.equal(h_v, h_c) and torch.equal(b_v, b_c)
    assert torch.equal(h1, to(c["h"][:1]))  # the shared input is untouched


def test_in_place_state_update(gpu_lib):
    hip_step = _step()
    c = make_step_case(43, R=4, D=64, NR=16, NT=4)
    p = [to(c[k]) for k in ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk", "D")]
    h, b = to(c["h"]), to(c["beta"])
    with torch.no_grad():
        y1, (h1, b1) = hip_step(*p, (h.clone(), b.clone()))
        y2 = torch.empty_like(y1)
        hip_step(*p, (h, b), out=(y2, h, b))
    assert torch.equal(y1, y2) and torch.equal(h1, h) and torch.equal(b1, b)


@pytest.mark.parametrize("R,D,NR,NT,P,norm,dt,form", [
    (8, 256, 16, 4, 2, True, torch.float32, "full"),        # one rollout per workgroup: fused
    (5, 300, 12, 8, 2, True, torch.bfloat16, "rank1"),      # partial channel tile, fused
    (3, 512, 32, 8, 4, True, torch.float16, "shared"),      # a broadcast state, fused
    (16, 128, 16, 0, 8, False, torch.float32, "full"),      # plain p-sum, fused
    (700, 1024, 16, 4, 2, True, torch.float32, "full"),     # several rollouts per workgroup
    (700, 1024, 16, 4, 2, True, torch.bfloat16, "rank1"),
    (6, 96, 12, 6, 2, True, torch.float32, "full"),         # d_state 18: the lane kernel
    (4, 256, 20, 8, 2, True, torch.float32, "rank1"),       # d_state 28: pad states, fused
    (3, 192, 52, 8, 2, True, torch.bfloat16, "shared"),     # d_state 60: pad states, fused
    (600, 512, 36, 8, 2, True, torch.float32, "full"),      # d_state 44: pad states, BCNorm first
])
def test_step_bcnorm_equals_bcnorm_then_step(gpu_lib, R, D, NR, NT, P, norm, dt, form):
    """rp_step_bcnorm (BCNorm + p-sum of the raw x_proj projections inside the
    step where it takes one rollout per workgroup, else the BCNorm kernel
    first) gives the bits of hip_bcnorm_psum followed by rp_step: y, h and
    beta, in every cache form, with softplus on load and the output gate."""
    from redpanda_amd.bcnorm import hip_bcnorm_psum
    from redpanda_amd.step import compact_beta
    hip_step = _step()
    N = NR + NT
    g = torch.Generator(device=dev).manual_seed(R * 7 + D + N)
    X = (torch.randn(R, 24 + 2 * N * P, device=dev, generator=g) * 2).to(dt)  # an x_proj output
    B_raw, C_raw = X[:, 24:24 + N * P], X[:, 24 + N * P:]
    wB = torch.rand(N * P, device=dev, generator=g) + 0.5
    wC = torch.rand(N * P, device=dev, generator=g) + 0.5
    x = torch.randn(R, D, device=dev, generator=g) - 2.0
    u = torch.randn(R, D, device=dev, generator=g)
    z = torch.randn(R, D, device=dev, generator=g).to(torch.bfloat16)
    Ar = -torch.exp(torch.rand(D, NR, device=dev, generator=g) * 2) if NR else None
    Ai = (torch.rand(D, NR, device=dev, generator=g) * 2 - 1) * 3 if NR else None
    Tk = torch.tanh(torch.randn(D, NT, device=dev, generator=g)) if NT else None
    Dk = torch.randn(D, device=dev, generator=g)
    h = torch.randn(1 if form == "shared" else R, D, N, device=dev, generator=g)
    if form == "rank1":
        beta = compact_beta(torch.randn(R, D, device=dev, generator=g),
                            torch.randn(R, N, device=dev, generator=g))
    else:
        beta = torch.randn(h.shape, device=dev, generator=g)
    if form == "shared":
        h, beta = h.expand(R, D, N), beta.expand(R, D, N)
    eps = 1e-5
    with torch.no_grad():
        Bc, Cc = hip_bcnorm_psum(B_raw, C_raw, wB, wC, P, eps, normalize=norm)
        y0, (h0, b0) = hip_step(x, u, Bc, Cc, Ar, Ai, Tk, Dk, (h, beta), delta_softplus=True, z=z)
        y1, (h1, b1) = hip_step(x, u, None, None, Ar, Ai, Tk, Dk, (h, beta), delta_softplus=True,
                                z=z, bcnorm=(B_raw, C_raw, wB, wC, P, eps, norm))
    torch.cuda.synchronize()
    same = lambda a, b: torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert same(y1, y0) and same(h1, h0) and same(b1, b0)
