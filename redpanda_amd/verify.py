"""Self-verification gate of the HIP scan path.

`verify(device, thorough, verbose)` has the role and signature of the
reference's gate (engine/triton_scan.py:342-398, called by
engine/train.py:708-716 before training with the fused scan): it builds
small Mamba models over the reference's configuration x length x direction
matrix, runs forward + backward through the HIP kernels, and raises
AssertionError on any mismatch.

The checker is an independent float64 evaluation of the same model from the
same parameters (functional torch ops, a sequential float64 recurrence for
the scan), on the same device.  Two criteria must hold:
  * the reference gate's own: forward max-abs < 2e-3, and per parameter
    max|dgrad| / max(max|grad|, 1) < 2e-3, under the loss mean(y^2);
  * a norm-wise one that a real defect cannot hide under: forward and every
    parameter gradient within 1e-4 of float64 (max|a-b| / max|b|) under a
    well-conditioned loss (a fixed random projection of y).
The float64 code here only checks; it never produces results for callers.
"""

import torch
import torch.nn.functional as F

from redpanda_amd.mamba import Mamba, MambaConfig

REF_GATE_TOL = 2e-3     # engine/triton_scan.py:375-384
NORM_TOL = 1e-4


def _rms64(x, w, eps=1e-5):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _scan64(u, delta, Ar, Ai, Bc, Cc, Tk, reverse=False):
    """Sequential float64 trapezoidal recurrence on contracted B/C (no skip)."""
    batch, L, d = u.shape
    n = Bc.shape[-1]
    h = torch.zeros(batch, d, n, dtype=u.dtype, device=u.device)
    bp = torch.zeros_like(h)
    ys = [None] * L
    for t in (range(L - 1, -1, -1) if reverse else range(L)):
        parts = []
        if Ar is not None:
            g = torch.exp(delta[:, t].unsqueeze(-1) * Ar)
            if Ai is not None:
                g = g * torch.cos(delta[:, t].unsqueeze(-1) * Ai)
            parts.append(g)
        if Tk is not None:
            parts.append(Tk.expand(batch, d, -1))
        g = torch.cat(parts, -1) if len(parts) > 1 else parts[0]
        beta = (delta[:, t] * u[:, t]).unsqueeze(-1) * Bc[:, t].unsqueeze(1)
        h = g * h + 0.5 * beta + 0.5 * g * bp
        bp = beta
        ys[t] = (h * Cc[:, t].unsqueeze(1)).sum(-1)
    return torch.stack(ys, 1)


def _mixer64(mx, x, p):
    """Float64 Mamba3Block.forward from the block's parameters (dict p)."""
    cfg = mx.config
    xb, z = F.linear(x, p["in_proj.weight"], p.get("in_proj.bias")).chunk(2, dim=-1)
    xb = F.silu(xb)
    n, mp = cfg.d_state, cfg.mimo_p
    dt_raw, B_raw, C_raw = F.linear(xb, p["x_proj.weight"], p["x_proj.bias"]).split(
        [cfg.dt_rank, n * mp, n * mp], dim=-1)
    if cfg.use_bcnorm:
        B_raw = _rms64(B_raw, p["b_norm.weight"])
        C_raw = _rms64(C_raw, p["c_norm.weight"])
    delta = F.softplus(F.linear(dt_raw, p["dt_proj.weight"], p["dt_proj.bias"]))
    lead = xb.shape[:-1]
    Bc = B_raw.view(*lead, n, mp).sum(-1)
    Cc = C_raw.view(*lead, n, mp).sum(-1)
    Ar = Ai = Tk = None
    if cfg.n_rot_state > 0:
        if cfg.use_complex:
            mag = -torch.exp(p["A_log_mag"])
            Ar, Ai = mag * torch.cos(p["A_phase"]), mag * torch.sin(p["A_phase"])
        else:
            Ar = -torch.exp(p["A_log"])
    if cfg.n_track_state > 0:
        Tk = torch.tanh(p["track_theta"])
    y = _scan64(xb, delta, Ar, Ai, Bc, Cc, Tk) + xb * p["D"]
    if cfg.bidirectional:
        y = y + _scan64(xb, delta, Ar, Ai, Bc, Cc, Tk, reverse=True) + xb * p["D"]
    return F.linear(y * F.silu(z), p["out_proj.weight"], p.get("out_proj.bias"))


def _model64(model, ids, params):
    x = F.embedding(ids, params["embedding.weight"])
    for i, layer in enumerate(model.layers):
        pre = f"layers.{i}."
        blk = {k[len(pre) + 6:]: v for k, v in params.items() if k.startswith(pre + "mixer.")}
        x = x + _mixer64(layer["mixer"], _rms64(x, params[pre + "norm.weight"]), blk)
    return _rms64(x, params["norm_f.weight"])


def gate_errors(y, y64, grads, grads64):
    """(reference-gate forward error, reference-gate grad error, norm-wise
    forward error, worst norm-wise grad error, its parameter name)."""
    fd = (y.double() - y64).abs().max().item()
    gd = 0.0
    for k, g64 in grads64.items():
        den = max(g64.abs().max().item(), 1.0)
        gd = max(gd, (grads[k].double() - g64).abs().max().item() / den)
    den = y64.abs().max().item() or 1.0
    fn = fd / den
    gn, gk = 0.0, ""
    for k, g64 in grads64.items():
        e = (grads[k].double() - g64).abs().max().item() / (g64.abs().max().item() or 1.0)
        if e > gn:
            gn, gk = e, k
    return fd, gd, fn, gn, gk


def check_gate(errs, where=""):
    """Raise AssertionError unless both criteria hold."""
    fd, gd, fn, gn, gk = errs
    assert fd < REF_GATE_TOL, f"forward mismatch {fd:.2e} {where}"
    assert gd < REF_GATE_TOL, f"grad mismatch {gd:.2e} {where}"
    assert fn < NORM_TOL, f"forward mismatch (norm-wise) {fn:.2e} {where}"
    assert gn < NORM_TOL, f"grad mismatch (norm-wise) {gn:.2e} in {gk} {where}"


def _run_case(kw, L, bidir, device, seed):
    torch.manual_seed(seed)
    vocab = 500
    cfg = MambaConfig(vocab_size=vocab, bidirectional=bidir, use_triton_scan=True, **kw)
    model = Mamba(cfg).to(device)
    with torch.no_grad():  # spread A and theta off their structured init
        gen = torch.Generator(device="cpu").manual_seed(seed + 1)
        for layer in model.layers:
            mx = layer["mixer"]
            if hasattr(mx, "A_phase"):
                mx.A_phase.copy_(((torch.rand(mx.A_phase.shape, generator=gen) * 2 - 1) * 1.4).to(device))
            if hasattr(mx, "track_theta"):
                mx.track_theta.copy_((torch.randn(mx.track_theta.shape, generator=gen) * 1.5).to(device))
    model.train()
    ids = torch.randint(0, vocab, (3, L), device=device)
    proj = torch.randn(3, L, cfg.d_model, device=device)
    params64 = {k: v.detach().double().requires_grad_(True) for k, v in model.named_parameters()}
    out = []
    for loss_fn in (lambda y: y.pow(2).mean(), lambda y: (y * proj.to(y.dtype)).sum()):
        model.zero_grad(set_to_none=True)
        y = model(ids)
        loss_fn(y).backward()
        grads = {k: p.grad for k, p in model.named_parameters() if p.grad is not None}
        for v in params64.values():
            v.grad = None
        y64 = _model64(model, ids, params64)
        loss_fn(y64).backward()
        grads64 = {k: v.grad for k, v in params64.items() if v.grad is not None and k in grads}
        out.append(gate_errors(y.detach(), y64.detach(), grads, grads64))
    return out


def verify(device="cuda", thorough=True, verbose=True):
    """Compare the HIP scan path with float64 over the reference gate's
    matrix; raise AssertionError on any mismatch, return True otherwise."""
    if not torch.cuda.is_available():
        raise AssertionError("redpanda_amd.verify: no ROCm GPU visible")
    cfgs = [dict(d_model=32, n_layer=2, d_state=12, n_track_state=4, mimo_p=2),
            dict(d_model=48, n_layer=2, d_state=16, n_track_state=0, mimo_p=2)]
    if thorough:
        cfgs.append(dict(d_model=512, n_layer=2, d_state=64, n_track_state=16, mimo_p=4))
    lens = (1, 31, 32, 33, 70, 107, 160) if thorough else (33, 70)
    for kw in cfgs:
        for bidir in (False, True):
            for L in lens:
                (e_ref, e_norm) = _run_case(kw, L, bidir, device, seed=L)
                where = f"cfg={kw} L={L} bidir={bidir}"
                check_gate((e_ref[0], e_ref[1], e_norm[2], e_norm[3], e_norm[4]), where)
                if verbose:
                    print(f"  ok cfg(d={kw['d_model']},N={kw['d_state']},trk={kw['n_track_state']}) "
                          f"L={L} bidir={int(bidir)} | fwd {e_ref[0]:.1e} grad {e_ref[1]:.1e} "
                          f"| norm-wise fwd {e_norm[2]:.1e} grad {e_norm[3]:.1e}", flush=True)
    if verbose:
        print("HIP SCAN VERIFIED: forward + gradients match float64.")
    return True


__all__ = ["verify", "check_gate", "gate_errors", "REF_GATE_TOL", "NORM_TOL"]
