"""GPU parity of the drop-in backbone (redpanda_amd.mamba / search_mamba).

Two kinds of reference:
  * the golden fixtures: the reference's own modules run on the CPU
    (tests/golden/make_golden.py), compared across devices;
  * the oracle's restatement of the reference modules (oracle/model_ref.py)
    run on the same GPU with the same weights, so the projections and norms
    use the same GPU GEMMs and only the SSM core differs.  This is the
    comparison the fp32 bars apply to: forward <= 1e-5, gradients <= 1e-6
    (norm-wise max|a-b|/max|b| per tensor), falling back to "no further from a
    float64 run than the reference is" where the reference's own fp32 error
    exceeds the bar.
"""

import math

import pytest
import torch

from oracle import model_ref, scan_ref
from tests.conftest import load_golden

pytestmark = pytest.mark.gpu
dev = "cuda"
FWD_TOL = 1e-5
GRAD_TOL = 1e-6


def rel(a, b):
    return scan_ref.rel_err(a.detach().cpu(), b.detach().cpu())


def _hip():
    from redpanda_amd import mamba as hm
    return hm


def _pair(cfg_kw, seed=0, perturb=True):
    """(hip model, oracle model) on the GPU with identical weights."""
    hm = _hip()
    torch.manual_seed(seed)
    ref = model_ref.Mamba(model_ref.MambaConfig(**cfg_kw))
    if perturb:
        # move A / theta off their structured init so every lane matters, while
        # keeping Re(A) = -exp(log_mag) cos(phase) < 0 (|phase| < pi/2): a
        # positive real part makes exp(dt Re A) > 1 and the scan grow without
        # bound, which no fp32 implementation reproduces
        gen = torch.Generator().manual_seed(seed + 1)
        with torch.no_grad():
            for layer in ref.layers:
                mx = layer["mixer"]
                if hasattr(mx, "A_phase"):
                    mx.A_phase.copy_((torch.rand(mx.A_phase.shape, generator=gen) * 2 - 1) * 1.4)
                    mx.A_log_mag.copy_(torch.rand(mx.A_log_mag.shape, generator=gen) * 3.0 - 1.0)
                if hasattr(mx, "A_log"):
                    mx.A_log.copy_(torch.rand(mx.A_log.shape, generator=gen) * 3.0 - 1.0)
                if hasattr(mx, "track_theta"):
                    mx.track_theta.copy_(torch.randn(mx.track_theta.shape, generator=gen) * 1.5)
    hip = hm.Mamba(hm.MambaConfig(**cfg_kw))
    hip.load_state_dict(ref.state_dict())
    return hip.to(dev), ref.to(dev)


def _grads(m):
    return {k: p.grad for k, p in m.named_parameters() if p.grad is not None}


# Where the reference's own fp32 result is further than the bar from float64
# (12 stacked layers put it ~2e-5 away), no implementation that is not
# bitwise identical to it can be within the bar of it; the test then asks
# for the same accuracy: no further from float64 than the reference, up to
# the scatter of a max-norm error estimate (ACCURACY_SLACK: across kernel
# revisions the HIP/reference ratio of that distance has ranged over
# 0.6..1.6 on the 12-layer case, tensor by tensor).
ACCURACY_SLACK = 2.0


def within_bar(e_hip_ref, e_hip_64, e_ref_64, tol):
    return e_hip_ref <= tol or e_hip_64 <= max(tol, ACCURACY_SLACK * e_ref_64)


def _compare_train_step(cfg_kw, B, L, seed, tag):
    hip, ref = _pair(cfg_kw, seed)
    ref64 = model_ref.Mamba(model_ref.MambaConfig(**cfg_kw)).to(dev).double()
    ref64.load_state_dict(ref.state_dict())
    gen = torch.Generator().manual_seed(seed + 7)
    ids = torch.randint(0, cfg_kw["vocab_size"], (B, L), generator=gen).to(dev)
    # upstream gradient dout ~ N(0, 1): a loss whose gradient is not a
    # cancellation residue (mean(norm_f(x)^2) is nearly constant in x)
    dout = torch.randn(B, L, cfg_kw["d_model"], generator=gen).to(dev)
    outs = {}
    for name, m in (("hip", hip), ("ref", ref), ("f64", ref64)):
        m.train()
        y = m(ids)
        (y * dout.to(y.dtype)).sum().backward()
        outs[name] = (y.detach(), _grads(m))
    (yh, gh), (yr, gr), (y64, g64) = outs["hip"], outs["ref"], outs["f64"]
    rep = {"y": (rel(yh, yr), rel(yh, y64), rel(yr, y64))}
    for k in gr:
        rep[k] = (rel(gh[k], gr[k]), rel(gh[k], g64[k]), rel(gr[k], g64[k]))
    worst = max(rep.items(), key=lambda kv: kv[1][0])
    print(tag, "y (hip-ref, hip-f64, ref-f64) = (%.1e %.1e %.1e)" % rep["y"],
          f"worst grad {worst[0]} {worst[1][0]:.1e} "
          f"(hip-f64 {worst[1][1]:.1e}, ref-f64 {worst[1][2]:.1e})", flush=True)
    for k, v in rep.items():
        if k != "y":
            print(f"   {k}: %.1e %.1e %.1e" % v)
    assert within_bar(*rep.pop("y"), FWD_TOL), tag
    for k, v in rep.items():
        assert within_bar(*v, GRAD_TOL), f"{tag}: {k} (hip-ref, hip-f64, ref-f64) = {v}"


@pytest.mark.parametrize("bidir", [False, True])
def test_small_model_train_step_matches_reference(gpu_lib, bidir):
    cfg = dict(d_model=32, n_layer=2, d_state=12, n_track_state=4, mimo_p=2, vocab_size=500,
               bidirectional=bidir)
    _compare_train_step(cfg, B=3, L=70, seed=1, tag=f"small bidir={bidir}")


def test_real_decay_model_matches_reference(gpu_lib):
    cfg = dict(d_model=48, n_layer=2, d_state=16, n_track_state=0, mimo_p=2, vocab_size=500,
               use_complex=False, bidirectional=True)
    _compare_train_step(cfg, B=3, L=33, seed=2, tag="real decay")


def test_eval_mamba_12_layers_end_to_end(gpu_lib):
    """The Eval-Mamba training shape end to end over 12 stacked bidirectional
    layers (d_model 768, d_inner 1536, d_state 40 = 32 rotational + 8
    tracking, mimo_p 4), at a reduced batch of 8 boards x 64 tokens."""
    cfg = dict(d_model=768, n_layer=12, d_state=40, n_track_state=8, mimo_p=4, vocab_size=512,
               bidirectional=True)
    _compare_train_step(cfg, B=8, L=64, seed=3, tag="eval-mamba 12L")


def _f64_arbiter(g, bidir):
    """The oracle's restatement of the fixture model in float64 on the CPU:
    the arbiter for cross-device comparisons (fixture weights put half the
    rotational gates above 1, so the fp32 results carry amplified rounding)."""
    cfg = model_ref.MambaConfig(d_model=16, n_layer=2, d_state=12, n_track_state=4, mimo_p=2,
                                vocab_size=64, bidirectional=bidir)
    m = model_ref.Mamba(cfg).double()
    m.load_state_dict({k[3:]: v.double() if v.is_floating_point() else v
                       for k, v in g.items() if k.startswith("sd.")})
    m.train()
    y = m(g["ids"])
    y.pow(2).mean().backward()
    return y.detach(), {k: p.grad for k, p in m.named_parameters() if p.grad is not None}


XDEV_TOL = 1e-5  # GPU GEMMs vs the fixture's CPU GEMMs


def fixture_grad_ok(e_hip_ref, e_hip_64, e_ref_64):
    """Sanity bound for gradients of the model fixtures.  Their losses are
    near-cancellations (mean(norm_f(x)^2) is almost constant in x; the mean
    of LayerNorm-ed logits likewise) and half their rotational gates exceed
    1, so the gradients are rounding residues at the 1e-5 level in any fp32
    implementation; the fixture itself is up to 1e-5 from float64.  This
    catches a wrong sign or a dropped term (O(1) errors); the gradient
    parity claim rests on the well-conditioned same-device tests above."""
    return e_hip_ref <= XDEV_TOL or e_hip_64 <= 10.0 * max(XDEV_TOL, e_ref_64)


@pytest.mark.parametrize("bidir", [False, True])
def test_golden_model_fixture(gpu_lib, bidir):
    """The reference's own CPU outputs and gradients.  Cross-device (GEMMs on
    the GPU vs the CPU): each tensor is within 1e-5 of the fixture, or no
    further from the float64 arbiter than the fixture itself is."""
    hm = _hip()
    g = load_golden(f"model_bi{int(bidir)}")
    cfg = hm.MambaConfig(d_model=16, n_layer=2, d_state=12, n_track_state=4, mimo_p=2,
                         vocab_size=64, bidirectional=bidir)
    m = hm.Mamba(cfg)
    sd = {k[3:]: v for k, v in g.items() if k.startswith("sd.")}
    assert sorted(sd) == sorted(m.state_dict())
    m.load_state_dict(sd)
    m.to(dev).train()
    ids = g["ids"].to(dev)
    y = m(ids)
    y.pow(2).mean().backward()
    y64, g64 = _f64_arbiter(g, bidir)
    checks = [("y", y, g["y_train"], y64)]
    checks += [(k, p.grad, g["grad." + k], g64[k]) for k, p in m.named_parameters()
               if "grad." + k in g]
    k, a, ref, r64 = checks.pop(0)
    assert within_bar(rel(a, ref), rel(a, r64), rel(ref, r64), XDEV_TOL), "y"
    for k, a, ref, r64 in checks:
        e = (rel(a, ref), rel(a, r64), rel(ref, r64))
        assert fixture_grad_ok(*e), f"{k}: (hip-ref, hip-f64, ref-f64) = {e}"
    m.eval()
    with torch.no_grad():
        assert rel(m(ids), g["y_eval"]) <= XDEV_TOL
        if not bidir:
            cache, outs = None, []
            for t in range(ids.shape[1]):
                hdn, cache = m.step(token_id=ids[:, t], cache=cache)
                outs.append(hdn)
            assert rel(torch.stack(outs, 1), g["y_step"]) <= XDEV_TOL
            fin, pc = m.prime_cache(ids[:, :20])
            assert rel(fin, g["prime_final"]) <= XDEV_TOL
            for i, (h, b) in enumerate(pc):
                assert rel(h, g[f"prime_h{i}"]) <= XDEV_TOL
                assert rel(b, g[f"prime_beta{i}"]) <= XDEV_TOL
            nxt, _ = m.step(token_id=ids[:, 20], cache=pc)
            assert rel(nxt, g["prime_next"]) <= XDEV_TOL


def test_model_step_equals_forward(gpu_lib):
    """engine/test_v3.py:44-62 at a BASELINE step shape: stepping token by
    token reproduces the full causal forward (1e-6), and prime_cache + step
    continues it."""
    cfg = dict(d_model=128, n_layer=3, d_state=20, n_track_state=4, mimo_p=2, vocab_size=512)
    hip, _ = _pair(cfg, seed=4)
    hip.eval()
    gen = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 512, (6, 32), generator=gen).to(dev)
    with torch.no_grad():
        full = hip(ids)
        cache, outs = None, []
        for t in range(ids.shape[1]):
            hdn, cache = hip.step(token_id=ids[:, t], cache=cache)
            outs.append(hdn)
        e_step = rel(torch.stack(outs, 1), full)
        fin, pc = hip.prime_cache(ids[:, :20])
        e_prime = rel(fin, full[:, 19])
        nxt, _ = hip.step(token_id=ids[:, 20], cache=pc)
        e_next = rel(nxt, full[:, 20])
    print(f"step vs forward {e_step:.1e}; prime {e_prime:.1e}; continue {e_next:.1e}")
    assert e_step <= 1e-6 and e_prime <= 1e-6 and e_next <= 1e-6


@pytest.mark.parametrize("compact", [False, True])
def test_search_shape_plies_equal_forward(gpu_lib, compact):
    """The batched-step workload at its model shape (8 causal layers, d_model
    512, d_state 16 + 4, mimo_p 2) on a row subset: 32 plies of step() with
    input_embed reproduce Mamba.forward(input_embeds=(R, 32, 512)) (1e-6),
    with the reference's cache format and with rank-1 beta rows."""
    cfg = dict(d_model=512, n_layer=8, d_state=20, n_track_state=4, mimo_p=2, vocab_size=64)
    hip, _ = _pair(cfg, seed=6)
    hip.eval()
    gen = torch.Generator().manual_seed(7)
    emb = torch.randn(12, 32, 512, generator=gen).to(dev)
    with torch.no_grad():
        full = hip(None, input_embeds=emb)
        cache, outs = None, []
        for t in range(emb.shape[1]):
            hdn, cache = hip.step(input_embed=emb[:, t], cache=cache, compact=compact)
            assert all(c[1].dim() == (2 if compact else 3) for c in cache)
            outs.append(hdn)
        e = rel(torch.stack(outs, 1), full)
    print(f"32 plies vs forward (compact={compact}): {e:.1e}")
    assert e <= 1e-6


def test_step_under_autograd_matches_reference(gpu_lib):
    """Training through step() (SearchMamba.dynamics_rollout pattern): prime
    on a prefix, step T moves with autograd on, gradients of every parameter
    against the oracle on the same GPU (fp32 bars, float64 arbiter)."""
    cfg = dict(d_model=32, n_layer=2, d_state=12, n_track_state=4, mimo_p=2, vocab_size=200)
    hip, ref = _pair(cfg, seed=6)
    ref64 = model_ref.Mamba(model_ref.MambaConfig(**cfg)).to(dev).double()
    ref64.load_state_dict(ref.state_dict())
    gen = torch.Generator().manual_seed(8)
    board = torch.randint(0, 200, (3, 15), generator=gen).to(dev)
    moves = torch.randint(0, 200, (3, 5), generator=gen).to(dev)
    proj = torch.randn(5, 3, 32, generator=gen).to(dev)
    res = {}
    for name, m in (("hip", hip), ("ref", ref), ("f64", ref64)):
        m.train()
        _, cache = m.prime_cache(board)
        loss = 0.0
        for t in range(moves.shape[1]):
            h, cache = m.step(token_id=moves[:, t], cache=cache)
            loss = loss + (h * proj[t].to(h.dtype)).sum()
        loss.backward()
        res[name] = (loss.detach(), _grads(m))
    (lh, gh), (lr, gr), (l64, g64) = res["hip"], res["ref"], res["f64"]
    assert within_bar(rel(lh, lr), rel(lh, l64), rel(lr, l64), FWD_TOL)
    for k in gr:
        e = (rel(gh[k], gr[k]), rel(gh[k], g64[k]), rel(gr[k], g64[k]))
        assert within_bar(*e, GRAD_TOL), f"{k}: (hip-ref, hip-f64, ref-f64) = {e}"


def _search_pair(g):
    """The HIP SearchMamba on the GPU and a float64 arbiter on the CPU: the
    same heads over the oracle's restated backbone."""
    from redpanda_amd.search_mamba import SearchMamba, SearchMambaConfig
    kw = dict(d_model=16, n_layer=2, d_state=8, n_track_state=2, mimo_p=2, vocab_size=64)
    sd = {k[3:]: v for k, v in g.items() if k.startswith("sd.")}
    sm = SearchMamba(SearchMambaConfig(**kw), vocab_size=64, eval_dim=12)
    sm.load_state_dict(sd)
    arb = SearchMamba(SearchMambaConfig(**kw), vocab_size=64, eval_dim=12)
    arb.backbone = model_ref.Mamba(model_ref.MambaConfig(**kw))
    arb.load_state_dict(sd)
    return sm.to(dev), arb.double()


def test_search_mamba_golden(gpu_lib):
    """SearchMamba on the reference's fixture: dynamics_rollout values and
    gradients, prime_board, eval_step, _expand_cache + batched step, and the
    fast (prime + step) vs slow (full scan) line evaluation.  Cross-device,
    so each tensor is within 1e-5 of the fixture or no further from the
    float64 arbiter than the fixture is."""
    g = load_golden("search")
    sm, arb = _search_pair(g)
    sm.train()
    arb.train()
    board, moves = g["board"], g["moves"]
    v, c, f = sm.dynamics_rollout(board.to(dev), moves.to(dev))
    v64, c64, f64 = arb.dynamics_rollout(board, moves)
    (v.pow(2).mean() + c.mean() + f.pow(2).mean()).backward()
    (v64.pow(2).mean() + c64.mean() + f64.pow(2).mean()).backward()
    checks = [("dyn_v", v, g["dyn_v"], v64), ("dyn_c", c, g["dyn_c"], c64),
              ("dyn_f", f, g["dyn_f"], f64)]
    g64 = dict(arb.named_parameters())
    checks += [(k, p.grad, g["grad." + k], g64[k].grad) for k, p in sm.named_parameters()
               if "grad." + k in g]
    for k, a, ref, r64 in checks[:3]:
        assert within_bar(rel(a, ref), rel(a, r64), rel(ref, r64), XDEV_TOL), k
    for k, a, ref, r64 in checks[3:]:
        e = (rel(a, ref), rel(a, r64), rel(ref, r64))
        assert fixture_grad_ok(*e), f"{k}: (hip-ref, hip-f64, ref-f64) = {e}"
    sm.eval()
    with torch.no_grad():
        b0 = board[0].to(dev)
        fin, cache = sm.prime_board(b0)
        assert rel(fin, g["prime_final"]) <= XDEV_TOL
        val, cont, cache2 = sm.eval_step(cache, int(moves[0, 0]))
        ev = float(g["eval_value"][0])
        assert abs(val - ev) <= XDEV_TOL * max(1.0, abs(ev))
        assert rel(cont, g["eval_cont"]) <= XDEV_TOL
        exp = sm._expand_cache(cache2, 4)
        hB, _ = sm.backbone.step(token_id=moves[:, 1].repeat(2)[:4].to(dev), cache=exp)
        assert rel(hB, g["expand_step"]) <= XDEV_TOL
        assert rel(sm.evaluate_lines_fast(b0, moves.to(dev)), g["lines_fast"]) <= XDEV_TOL
        assert rel(sm.evaluate_lines(b0, moves.to(dev)), g["lines_slow"]) <= XDEV_TOL


def test_cpu_tensors_are_refused(gpu_lib):
    """No silent CPU path: the SSM core needs device tensors."""
    hm = _hip()
    m = hm.Mamba(hm.MambaConfig(d_model=16, n_layer=1, d_state=8, n_track_state=2, mimo_p=2,
                                vocab_size=64))
    with pytest.raises(RuntimeError, match="ROCm device"):
        m(torch.zeros(1, 4, dtype=torch.long))
