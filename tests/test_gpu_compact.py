"""GPU tests of the rank-1 (compact) cache: beta carried as rows [dt*u | B].

beta_t = (dt_t u_t) outer B_t is rank-1 (engine/mamba.py:480-481), so a
cache can hold D + N floats per rollout instead of D * N.  The step forms
beta_prev with the multiply that produced the full form, so every result --
y, h and the beta the full form would hold -- is required to be the same
bits as the full-form path, for the tile kernel and the lane-layout kernel,
per-rollout and broadcast states, chains of steps, and whole models primed
with prime_cache(compact=True).
"""

import pytest
import torch
import torch.nn.functional as F

from redpanda_amd.step import compact_beta, full_beta, hip_step

pytestmark = pytest.mark.gpu
dev = "cuda"


def _inputs(R, D, NR, NT, seed, softplus=False):
    g = torch.Generator(device=dev).manual_seed(seed)
    N = NR + NT
    x = torch.randn(R, D, device=dev, generator=g) * 0.5 - 2.5
    dt = x if softplus else F.softplus(x)
    u = torch.randn(R, D, device=dev, generator=g)
    Bc = torch.randn(R, N, device=dev, generator=g)
    Cc = torch.randn(R, N, device=dev, generator=g)
    Ar = -torch.exp(torch.rand(D, NR, device=dev, generator=g) * 2 - 1) if NR else None
    Ai = (torch.rand(D, NR, device=dev, generator=g) * 2 - 1) * 3 if NR else None
    Tk = torch.tanh(torch.randn(D, NT, device=dev, generator=g)) if NT else None
    Dk = torch.randn(D, device=dev, generator=g)
    return dt, u, Bc, Cc, Ar, Ai, Tk, Dk


def _rank1_state(R, D, N, seed):
    """A state whose beta is rank-1, in both forms (as a previous step left it)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    h = torch.randn(R, D, N, device=dev, generator=g)
    dtu = torch.rand(R, D, device=dev, generator=g) * 0.2
    B = torch.randn(R, N, device=dev, generator=g)
    bp = compact_beta(dtu, B)
    return h, bp, full_beta(bp, D).contiguous()


# (R, D, NR, NT): tile kernel (d_state % 4 == 0 up to 128; from d_state 24
# each channel split over S / 4 threads; pad states at d_state 28, 44, 72,
# 116), partial channel tiles, and the lane-layout kernel (d_state 6, 90,
# and 108, whose pads would span two slots)
SHAPES = [(300, 1024, 16, 4), (37, 200, 32, 8), (9, 96, 64, 8), (11, 130, 4, 2),
          (65, 384, 48, 16), (7, 100, 24, 8), (20, 192, 72, 8), (33, 256, 20, 8),
          (70, 512, 36, 8), (5, 64, 80, 10), (40, 256, 112, 16), (9, 70, 100, 16),
          (6, 128, 100, 8),
          # pad states at 8 slots of 16 with compile-time rotational slots
          # (the branch-free rank-1 path), a run-time split there, and a
          # partial tile; 6 slots (2 slices per thread); 4-slice pad shapes
          (33, 256, 112, 0), (17, 128, 116, 8), (9, 96, 90, 14), (6, 100, 120, 8),
          (12, 256, 80, 4), (7, 64, 88, 4), (5, 256, 96, 0), (11, 256, 64, 8),
          (13, 256, 24, 4),
          # 5 slots of 16 (2 slices per thread, the block's last staging pass
          # bounded): pad states in a middle slot, a partial tile
          (10, 96, 56, 16), (3, 40, 60, 8), (8, 256, 72, 0),
          # 5 slots of 8 (2 slices per thread over 4 lanes, 64-channel tile)
          (9, 128, 28, 8), (5, 100, 24, 12), (6, 64, 40, 0)]


@pytest.mark.parametrize("R,D,NR,NT", SHAPES)
def test_rank1_step_equals_full(gpu_lib, R, D, NR, NT):
    N = NR + NT
    ins = _inputs(R, D, NR, NT, seed=R + D)
    h, bp, bfull = _rank1_state(R, D, N, seed=1)
    y1, (h1, bp1) = hip_step(*ins, state=(h, bp))
    y0, (h0, b0) = hip_step(*ins, state=(h, bfull))
    torch.cuda.synchronize()
    assert bp1.shape == (R, D + N)
    assert torch.equal(y1, y0) and torch.equal(h1, h0)
    assert torch.equal(full_beta(bp1, D), b0)
    dt, u, Bc = ins[0], ins[1], ins[2]
    assert torch.equal(bp1, compact_beta(dt * u, Bc))


@pytest.mark.parametrize("R,D,NR,NT", [(64, 512, 16, 4), (5, 72, 64, 8)])
def test_rank1_broadcast_and_chain(gpu_lib, R, D, NR, NT):
    """A batch-1 rank-1 cache expanded to R rows (stride 0), then 5 steps
    with softplus on load, against the full form."""
    N = NR + NT
    h, bp, bfull = _rank1_state(1, D, N, seed=2)
    st1 = (h.expand(R, D, N), bp.expand(R, D + N))
    st0 = (h.expand(R, D, N), bfull.expand(R, D, N))
    for k in range(5):
        ins = _inputs(R, D, NR, NT, seed=10 + k, softplus=True)
        y1, st1 = hip_step(*ins, state=st1, delta_softplus=True)
        y0, st0 = hip_step(*ins, state=st0, delta_softplus=True)
        assert torch.equal(y1, y0), k
    torch.cuda.synchronize()
    assert torch.equal(st1[0], st0[0]) and torch.equal(full_beta(st1[1], D), st0[1])


def test_rank1_fresh_state(gpu_lib):
    ins = _inputs(40, 256, 16, 4, seed=3)
    y1, (h1, bp1) = hip_step(*ins, state=None, compact=True)
    y0, (h0, b0) = hip_step(*ins, state=None)
    torch.cuda.synchronize()
    assert torch.equal(y1, y0) and torch.equal(h1, h0) and torch.equal(full_beta(bp1, 256), b0)


def _model(seed=0):
    from redpanda_amd import mamba as hm
    torch.manual_seed(seed)
    cfg = hm.MambaConfig(d_model=128, n_layer=3, d_state=20, n_track_state=4, vocab_size=300)
    return hm.Mamba(cfg).to(dev).eval()


def test_model_compact_cache_equals_full(gpu_lib):
    """prime_cache(compact=True) + steps give the same bits as the full cache,
    and the cache survives the MARS operations (clone, cat, expand)."""
    m = _model()
    ids = torch.randint(0, 300, (3, 17), device=dev)
    with torch.no_grad():
        hA, cA = m.prime_cache(ids)
        hB, cB = m.prime_cache(ids, compact=True)
        assert torch.equal(hA, hB)
        for (h0, b0), (h1, b1) in zip(cA, cB):
            assert b1.shape == (3, 256 + 20)
            assert torch.equal(h0, h1) and torch.equal(full_beta(b1, 256), b0)
        cB = [(h.clone(), b.clone()) for h, b in cB]                      # _clone_cache
        cB = [(torch.cat([h, h[:1]]), torch.cat([b, b[:1]])) for h, b in cB]  # grow the batch
        cA = [(torch.cat([h, h[:1]]), torch.cat([b, b[:1]])) for h, b in cA]
        for t in range(4):
            tok = torch.randint(0, 300, (4,), device=dev)
            xA, cA = m.step(token_id=tok, cache=cA)
            xB, cB = m.step(token_id=tok, cache=cB)
            assert torch.equal(xA, xB), t
    torch.cuda.synchronize()


def test_training_through_compact_step(gpu_lib):
    """Under autograd a compact state runs the L=1 scan from its full form:
    gradients match the full-form path."""
    m = _model(1).train()
    ids = torch.randint(0, 300, (2, 9), device=dev)
    toks = torch.randint(0, 300, (2, 3), device=dev)

    def run(compact):
        m.zero_grad()
        _, cache = m.prime_cache(ids, compact=compact)
        loss = 0
        for t in range(toks.shape[1]):
            x, cache = m.step(token_id=toks[:, t], cache=cache)
            loss = loss + x.square().mean()
        loss.backward()
        return float(loss.detach()), {k: p.grad.clone() for k, p in m.named_parameters()
                                      if p.grad is not None}

    l0, g0 = run(False)
    l1, g1 = run(True)
    torch.cuda.synchronize()
    assert abs(l0 - l1) <= 1e-6 * abs(l0)
    for k in g0:
        d = (g0[k] - g1[k]).abs().max() / (g0[k].abs().max() + 1e-30)
        assert float(d) <= 1e-6, k


@pytest.mark.parametrize("zdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("R,D,NR,NT", SHAPES)
def test_gated_step_equals_torch_gate(gpu_lib, R, D, NR, NT, zdt):
    """y * silu(z) applied by the step kernel (z a strided chunk, fp32 or
    bf16) is the same bits as torch's gate on the kernel's y, for both beta
    forms."""
    N = NR + NT
    ins = _inputs(R, D, NR, NT, seed=R * 3 + D)
    g = torch.Generator(device=dev).manual_seed(8)
    xz = (torch.randn(R, 2 * D, device=dev, generator=g) * 3).to(zdt)
    z = xz.chunk(2, dim=-1)[1]
    h, bp, bfull = _rank1_state(R, D, N, seed=4)
    for st in ((h, bfull), (h, bp)):
        yg, (hg, bg) = hip_step(*ins, state=st, z=z)
        y0, (h0, b0) = hip_step(*ins, state=st)
        torch.cuda.synchronize()
        assert torch.equal(yg, y0 * F.silu(z)), st[1].dim()
        assert torch.equal(hg, h0) and torch.equal(bg, b0)
