"""StepGraph: a fixed-size batched step() captured into HIP graphs.

Every replay is compared bit for bit with the eager Mamba.step on the same
inputs and state (the same kernels in the same order), over several plies
with the program's own eager work and synchronisations between replays; also
after loading a primed cache, and after in-place parameter updates (which
the replays must follow)."""

import pytest
import torch

from tests.test_gpu_model import _pair

pytestmark = pytest.mark.gpu
dev = "cuda"
CFG = dict(d_model=128, n_layer=4, d_state=20, n_track_state=4, mimo_p=2, vocab_size=256)


def _same(a, b):
    return torch.equal(a.view(torch.int32), b.view(torch.int32))


def _eager(model, inputs, embed, compact, cache=None):
    outs = []
    with torch.no_grad():
        for x in inputs:
            kw = {"input_embed": x} if embed else {"token_id": x}
            h, cache = model.step(cache=cache, compact=compact, **kw)
            outs.append((h.clone(), [(a.clone(), b.clone()) for a, b in cache]))
    return outs


@pytest.mark.parametrize("R", [1, 7, 64])
@pytest.mark.parametrize("compact", [False, True], ids=["full", "rank1"])
@pytest.mark.parametrize("embed", [False, True], ids=["tokens", "embed"])
def test_step_graph_replays_equal_eager_step(gpu_lib, R, compact, embed):
    from redpanda_amd.step_graph import StepGraph
    model, _ = _pair(CFG, seed=11)
    model.eval()
    gen = torch.Generator().manual_seed(12)
    T = 6
    if embed:
        inputs = [torch.randn(R, CFG["d_model"], generator=gen).to(dev) for _ in range(T)]
    else:
        inputs = [torch.randint(0, CFG["vocab_size"], (R,), generator=gen).to(dev)
                  for _ in range(T)]
    ref = _eager(model, inputs, embed, compact)
    sg = StepGraph(model, R, compact=compact, embed=embed)
    for rnd in range(2):  # the graphs replayed again after a reset
        sg.reset()
        for t, x in enumerate(inputs):
            kw = {"input_embed": x} if embed else {"token_id": x}
            h, cache = sg(**kw)
            # eager work between replays, then a synchronisation
            junk = torch.randn(4096, device=dev).sum()
            torch.cuda.synchronize()
            assert _same(h, ref[t][0]), f"round {rnd} ply {t}: hidden"
            for i, ((a, b), (ra, rb)) in enumerate(zip(cache, ref[t][1])):
                assert _same(a, ra) and _same(b, rb), f"round {rnd} ply {t} layer {i}: state"
            del junk


def test_step_graph_continues_a_primed_cache(gpu_lib):
    """prime_cache + load + replays == prime_cache + eager steps."""
    from redpanda_amd.step_graph import StepGraph
    model, _ = _pair(CFG, seed=13)
    model.eval()
    R = 9
    gen = torch.Generator().manual_seed(14)
    board = torch.randint(0, CFG["vocab_size"], (R, 20), generator=gen).to(dev)
    moves = [torch.randint(0, CFG["vocab_size"], (R,), generator=gen).to(dev) for _ in range(4)]
    for compact in (False, True):
        with torch.no_grad():
            _, pc = model.prime_cache(board, compact=compact)
        ref = _eager(model, moves, False, compact, cache=pc)
        sg = StepGraph(model, R, compact=compact)
        sg.load(pc)
        for t, m in enumerate(moves):
            h, cache = sg(token_id=m)
            assert _same(h, ref[t][0]), f"compact={compact} ply {t}"
            for (a, b), (ra, rb) in zip(cache, ref[t][1]):
                assert _same(a, ra) and _same(b, rb)


def test_step_graph_follows_in_place_parameter_updates(gpu_lib):
    """The graphs read the parameters in place: after an in-place update of
    the gate parameters and a projection, replays equal the eager step of
    the updated model."""
    from redpanda_amd.step_graph import StepGraph
    model, _ = _pair(CFG, seed=15)
    model.eval()
    R = 5
    gen = torch.Generator().manual_seed(16)
    moves = [torch.randint(0, CFG["vocab_size"], (R,), generator=gen).to(dev) for _ in range(3)]
    sg = StepGraph(model, R)
    with torch.no_grad():
        for layer in model.layers:
            mx = layer["mixer"]
            mx.A_log_mag.add_(0.05)
            mx.track_theta.mul_(0.9)
            mx.in_proj.weight.mul_(1.01)
    ref = _eager(model, moves, False, False)
    sg.reset()
    for t, m in enumerate(moves):
        h, _ = sg(token_id=m)
        assert _same(h, ref[t][0]), f"ply {t}"


def test_training_through_step_captured_into_graphs(gpu_lib):
    """SearchMamba.dynamics_rollout forward + backward (prime_cache, then
    differentiable steps: the L=1 scans from the cache, BCNorm, the fused
    gate) captured with torch.cuda.make_graphed_callables: every replay's
    gradients equal the eager ones bit for bit."""
    from redpanda_amd.search_mamba import SearchMamba, SearchMambaConfig
    torch.manual_seed(17)
    cfg = SearchMambaConfig(d_model=64, n_layer=2, d_state=12, n_track_state=4, mimo_p=2,
                            vocab_size=128)
    sm = SearchMamba(cfg, vocab_size=128, eval_dim=32).to(dev).train()
    gen = torch.Generator().manual_seed(18)
    board = torch.randint(0, 128, (6, 20), generator=gen).to(dev)
    moves = torch.randint(0, 128, (6, 4), generator=gen).to(dev)

    class Rollout(torch.nn.Module):
        def __init__(self, m):
            super().__init__()
            self.m = m

        def forward(self, b, mv):
            return self.m.dynamics_rollout(b, mv)

    roll = Rollout(sm)

    def run(fn):
        sm.zero_grad(set_to_none=True)
        v, c, f = fn(board, moves)
        (v.sum() + c.mean() + f.pow(2).mean()).backward()
        return {k: p.grad.clone() for k, p in sm.named_parameters() if p.grad is not None}

    ref = run(roll)
    graphed = torch.cuda.make_graphed_callables(roll, (board, moves), allow_unused_input=True)
    for rep in range(3):
        g = run(graphed)
        torch.randn(1000, device=dev).sum()
        torch.cuda.synchronize()
        assert sorted(g) == sorted(ref)
        for k in ref:
            assert _same(g[k], ref[k]), f"replay {rep}: {k}"
