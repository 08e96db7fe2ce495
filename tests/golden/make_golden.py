"""Write the golden fixtures under tests/golden/ by importing the reference.

Run once, in the build container only (the reference tree is not present on
the GPU hosts):    python tests/golden/make_golden.py

What only an import can pin, and therefore what these fixtures record:
  * the exact fp32 output of the reference's own PyTorch scan path (its
    Hillis-Steele association, engine/mamba.py:104-136, :318-423) and of its
    autograd gradients, on small seeded inputs;
  * the reference's O(1) step (engine/mamba.py:427-498);
  * the reference's module construction (state_dict keys, seeded init) and
    the forward / step / prime_cache / gradient behaviour of small
    Mamba (engine/mamba.py:503-620) and SearchMamba
    (engine/search_mamba.py:39-291) models.
Every fixture is data: inputs and expected outputs, as float32/int64 arrays.
"""

import json
import math
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

REF_ENGINE = "/root/reference/redpanda/engine"
OUT = os.path.dirname(os.path.abspath(__file__))


def _np(t):
    return t.detach().cpu().numpy()


def scan_cases():
    """(name, cfg kwargs, L list, bidir)."""
    return [
        ("rot_trk", dict(d_model=8, d_state=12, n_track_state=4, mimo_p=2), [1, 31, 32, 33, 70]),
        ("rot_only", dict(d_model=8, d_state=16, n_track_state=0, mimo_p=2), [33, 70]),
        ("real_decay", dict(d_model=8, d_state=8, n_track_state=0, mimo_p=1, use_complex=False), [33]),
        ("trk_heavy", dict(d_model=8, d_state=6, n_track_state=5, mimo_p=2), [40]),
    ]


def make_scan(M, rng_seed=1234):
    out = {}
    gen = torch.Generator().manual_seed(rng_seed)
    for name, kw, lens in scan_cases():
        cfg = M.MambaConfig(vocab_size=64, n_layer=1, **kw)
        torch.manual_seed(7)
        blk = M.Mamba3Block(cfg)
        D, N, NR, NT, p = cfg.d_inner, cfg.d_state, cfg.n_rot_state, cfg.n_track_state, cfg.mimo_p
        with torch.no_grad():
            if NT:
                blk.track_theta.copy_(torch.randn(D, NT, generator=gen) * 1.5)
            blk.D.copy_(torch.randn(D, generator=gen) * 0.5 + 1.0)
        for L in lens:
            for bidir in (False, True):
                key = f"scan_{name}_L{L}_bi{int(bidir)}"
                Bsz = 2
                u = torch.randn(Bsz, L, D, generator=gen)
                delta = F.softplus(torch.randn(Bsz, L, D, generator=gen) * 0.5 - 2.0)
                Bm = torch.randn(Bsz, L, N, p, generator=gen)
                Cm = torch.randn(Bsz, L, N, p, generator=gen)
                if NR:
                    Ar = -torch.exp(torch.rand(D, NR, generator=gen) * 2.0)
                    Ai = (torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi if cfg.use_complex else None
                else:
                    Ar = Ai = None
                dout = torch.randn(Bsz, L, D, generator=gen)
                rec = {"u": u, "delta": delta, "B": Bm, "C": Cm, "dout": dout,
                       "Dskip": blk.D.detach().clone()}
                if Ar is not None:
                    rec["A_real"] = Ar
                if Ai is not None:
                    rec["A_imag"] = Ai
                if NT:
                    rec["theta"] = blk.track_theta.detach().clone()
                leaves = {k: v.clone().requires_grad_(True) for k, v in
                          [("u", u), ("delta", delta), ("B", Bm), ("C", Cm)]}
                if Ar is not None:
                    leaves["A_real"] = Ar.clone().requires_grad_(True)
                if Ai is not None:
                    leaves["A_imag"] = Ai.clone().requires_grad_(True)
                blk.train()
                blk.zero_grad(set_to_none=True)
                args = (leaves["u"], leaves["delta"], leaves.get("A_real"), leaves.get("A_imag"),
                        leaves["B"], leaves["C"], blk.D)
                y = blk._selective_scan_trapezoidal(*args)
                if bidir:
                    y = y + blk._selective_scan_trapezoidal(
                        leaves["u"].flip(1), leaves["delta"].flip(1), leaves.get("A_real"),
                        leaves.get("A_imag"), leaves["B"].flip(1), leaves["C"].flip(1),
                        blk.D).flip(1)
                (y * dout).sum().backward()
                rec["y"] = y.detach()
                for k, v in leaves.items():
                    rec["grad_" + k] = v.grad
                if NT:
                    rec["grad_theta"] = blk.track_theta.grad
                rec["grad_Dskip"] = blk.D.grad
                if not bidir:
                    blk.eval()
                    with torch.no_grad():
                        y2, (h, bl) = blk._selective_scan_trapezoidal(
                            u, delta, Ar, Ai, Bm, Cm, blk.D, return_state=True)
                    rec["state_h"] = h
                    rec["state_beta"] = bl
                    rec["y_eval"] = y2
                out[key] = {k: _np(v) for k, v in rec.items()}
    return out


def make_step(M, rng_seed=99):
    out = {}
    gen = torch.Generator().manual_seed(rng_seed)
    for name, kw in [("rot_trk", dict(d_model=8, d_state=12, n_track_state=4, mimo_p=2)),
                     ("real", dict(d_model=8, d_state=8, mimo_p=2, use_complex=False))]:
        cfg = M.MambaConfig(vocab_size=64, n_layer=1, **kw)
        torch.manual_seed(11)
        blk = M.Mamba3Block(cfg).eval()
        with torch.no_grad():
            if cfg.use_complex:
                blk.A_phase.copy_((torch.rand(blk.A_phase.shape, generator=gen) * 2 - 1) * math.pi)
                blk.A_log_mag.copy_(torch.rand(blk.A_log_mag.shape, generator=gen) * 2.0)
            if cfg.n_track_state:
                blk.track_theta.copy_(torch.randn(blk.track_theta.shape, generator=gen) * 1.5)
            for p in (blk.in_proj.weight, blk.x_proj.weight, blk.out_proj.weight):
                p.copy_(torch.randn(p.shape, generator=gen) * 0.3)
        sd = {k: v.detach().clone() for k, v in blk.state_dict().items()}
        Bsz, D, N = 3, cfg.d_inner, cfg.d_state
        x = torch.randn(Bsz, cfg.d_model, generator=gen)
        h0 = torch.randn(Bsz, D, N, generator=gen)
        b0 = torch.randn(Bsz, D, N, generator=gen) * 0.1
        with torch.no_grad():
            o1, (h1, bt1) = blk.step(x, None)
            o2, (h2, bt2) = blk.step(x, (h0, b0))
        rec = {"x": x, "h0": h0, "beta0": b0, "out_none": o1, "h_none": h1, "beta_none": bt1,
               "out": o2, "h": h2, "beta": bt2}
        rec.update({"sd." + k: v for k, v in sd.items()})
        out[f"step_{name}"] = {k: _np(v) for k, v in rec.items()}
    return out


def make_model(M, rng_seed=5):
    out = {}
    for bidir in (False, True):
        torch.manual_seed(rng_seed)
        cfg = M.MambaConfig(d_model=16, n_layer=2, d_state=12, n_track_state=4, mimo_p=2,
                            vocab_size=64, bidirectional=bidir)
        m = M.Mamba(cfg)
        gen = torch.Generator().manual_seed(rng_seed + 1)
        with torch.no_grad():  # move A off its degenerate init so rot lanes matter
            for layer in m.layers:
                mx = layer["mixer"]
                mx.A_phase.copy_((torch.rand(mx.A_phase.shape, generator=gen) * 2 - 1) * math.pi)
                mx.A_log_mag.copy_(torch.rand(mx.A_log_mag.shape, generator=gen) * 2.0)
                mx.track_theta.copy_(torch.randn(mx.track_theta.shape, generator=gen) * 1.5)
        ids = torch.randint(0, cfg.vocab_size, (2, 37), generator=gen)
        rec = {"ids": ids}
        m.train()
        y = m(ids)
        y.pow(2).mean().backward()
        rec["y_train"] = y.detach()
        for k, p in m.named_parameters():
            if p.grad is not None:
                rec["grad." + k] = p.grad
        m.zero_grad(set_to_none=True)
        m.eval()
        with torch.no_grad():
            rec["y_eval"] = m(ids)
            if not bidir:
                cache = None
                outs = []
                for t in range(ids.shape[1]):
                    hdn, cache = m.step(token_id=ids[:, t], cache=cache)
                    outs.append(hdn)
                rec["y_step"] = torch.stack(outs, 1)
                fin, pc = m.prime_cache(ids[:, :20])
                rec["prime_final"] = fin
                for i, (h, b) in enumerate(pc):
                    rec[f"prime_h{i}"] = h
                    rec[f"prime_beta{i}"] = b
                nxt, _ = m.step(token_id=ids[:, 20], cache=pc)
                rec["prime_next"] = nxt
        rec.update({"sd." + k: v for k, v in m.state_dict().items()})
        out[f"model_bi{int(bidir)}"] = {k: _np(v) for k, v in rec.items()}
    return out


def make_search(M, S, rng_seed=21):
    torch.manual_seed(rng_seed)
    cfg = S.SearchMambaConfig(d_model=16, n_layer=2, d_state=8, n_track_state=2, mimo_p=2,
                              vocab_size=64)
    sm = S.SearchMamba(cfg, vocab_size=64, eval_dim=12)
    gen = torch.Generator().manual_seed(rng_seed + 1)
    board = torch.randint(1, 64, (3, 15), generator=gen)
    moves = torch.randint(1, 64, (3, 4), generator=gen)
    rec = {"board": board, "moves": moves}
    sm.train()
    v, c, f = sm.dynamics_rollout(board, moves)
    (v.pow(2).mean() + c.mean() + f.pow(2).mean()).backward()
    rec.update({"dyn_v": v.detach(), "dyn_c": c.detach(), "dyn_f": f.detach()})
    for k, p in sm.named_parameters():
        if p.grad is not None:
            rec["grad." + k] = p.grad
    sm.zero_grad(set_to_none=True)
    sm.eval()
    with torch.no_grad():
        fin, cache = sm.prime_board(board[0])
        val, cont, cache2 = sm.eval_step(cache, int(moves[0, 0]))
        rec["prime_final"] = fin
        rec["eval_value"] = torch.tensor([val])
        rec["eval_cont"] = cont
        exp = sm._expand_cache(cache2, 4)
        hB, _ = sm.backbone.step(token_id=moves[:, 1].repeat(2)[:4], cache=exp)
        rec["expand_step"] = hB
        rec["lines_fast"] = sm.evaluate_lines_fast(board[0], moves)
        rec["lines_slow"] = sm.evaluate_lines(board[0], moves)
    rec.update({"sd." + k: v for k, v in sm.state_dict().items()})
    cfgd = {k: getattr(cfg, k) for k in ("d_model", "n_layer", "d_state", "expand", "mimo_p",
                                          "n_track_state", "vocab_size", "d_inner", "dt_rank")}
    return {"search": {k: _np(v) for k, v in rec.items()}}, cfgd


def main():
    sys.path.insert(0, REF_ENGINE)
    import mamba as M  # noqa: E402  (reference module, this container only)
    import search_mamba as S  # noqa: E402
    fixtures = {}
    fixtures.update(make_scan(M))
    fixtures.update(make_step(M))
    fixtures.update(make_model(M))
    srch, search_cfg = make_search(M, S)
    fixtures.update(srch)
    manifest = {"torch": torch.__version__, "cases": {}, "search_cfg": search_cfg}
    for name, rec in fixtures.items():
        np.savez_compressed(os.path.join(OUT, name + ".npz"), **rec)
        manifest["cases"][name] = sorted(rec.keys())
    with open(os.path.join(OUT, "manifest.json"), "w") as fh:
        json.dump(manifest, fh, indent=1, sort_keys=True)
    print(f"wrote {len(fixtures)} fixtures to {OUT}")


if __name__ == "__main__":
    main()
