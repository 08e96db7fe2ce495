"""Seeded shape sweep of the scan through the product's autograd entry
(hip_trapezoidal_scan), against the oracle in fp32 (the reference's chunk
loop, engine/mamba.py:360-373) and float64 (the sequential recurrence and its
hand-derived adjoint).

Each case draws its shape (batch, length across chunk and block boundaries,
channels across tile boundaries, state count across the 4 / 8 / 16-lane
layouts, the rotational / tracking split, real decay or the cos-modulated
gate), the direction mode, softplus on load, the storage dtype of
(delta, u) and of (B, C), and the memory layout of each input as the model
hands them over: contiguous, a column slice of a wider row (the in_proj /
x_proj outputs), or a batch-time transposed view.

Bars: y within 1e-5 and fp32 gradients within 1e-6 of the fp32 oracle, or no
further from float64 than the oracle is (the same criterion as the other
scan tests); gradients returned in a 16-bit storage dtype within one unit of
that dtype's rounding, norm-wise.
"""

import math
import os
import random

import pytest
import torch
import torch.nn.functional as F

from oracle import scan_ref

pytestmark = pytest.mark.gpu
dev = "cuda"
FWD_TOL = 1e-5
GRAD_TOL = 1e-6
ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
DTS = [torch.float32, torch.bfloat16, torch.float16]
# RP_SWEEP_SCALE=k draws k times as many cases (new seeds; the first ones unchanged)
SCALE = int(os.environ.get("RP_SWEEP_SCALE", "1"))


def rel(a, b):
    return scan_ref.rel_err(a.detach().cpu(), b.detach().cpu())


def within_bar(e_hip_ref, e_hip_64, e_ref_64, tol):
    return e_hip_ref <= tol or e_hip_64 <= max(tol, e_ref_64)


def _draw(case):
    rng = random.Random(7000 + case)
    B = rng.randint(1, 3)
    L = rng.choice([1, 3, 4, 5, 16, 17, 31, 33, 64, 65, 129])
    D = rng.choice([1, 5, 31, 32, 33, 64, 65, 100, 160])
    N = rng.choice([1, 3, 8, 16, 17, 20, 24, 33, 40, 41, 64, 72, 100, 128])
    NR = rng.choice([0, N, rng.randint(0, N)])
    NT = N - NR
    cplx = NR > 0 and rng.random() < 0.8
    return dict(B=B, L=L, D=D, N=N, NR=NR, NT=NT, cplx=cplx, bidir=rng.random() < 0.5,
                softplus=rng.random() < 0.4, dt_in=rng.choice(DTS), dt_bc=rng.choice(DTS),
                layouts=[rng.choice(["contig", "pad", "tb"]) for _ in range(4)],
                ar_hi=rng.choice([1.0, 3.0]))


def _inputs(s, case):
    g = torch.Generator().manual_seed(9000 + case)
    B, L, D, N, NR, NT = s["B"], s["L"], s["D"], s["N"], s["NR"], s["NT"]
    if s["softplus"]:
        delta = torch.randn(B, L, D, generator=g) * 1.5 - 2.5  # the dt projection x
    else:
        delta = F.softplus(torch.randn(B, L, D, generator=g) * 0.5 - 2.0)
    u = torch.randn(B, L, D, generator=g)
    Bc = torch.randn(B, L, N, generator=g)
    Cc = torch.randn(B, L, N, generator=g)
    Bc = Bc / Bc.pow(2).mean(-1, keepdim=True).sqrt()
    Cc = Cc / Cc.pow(2).mean(-1, keepdim=True).sqrt()
    Ar = -torch.exp(torch.rand(D, NR, generator=g) * s["ar_hi"]) if NR else None
    Ai = (torch.rand(D, NR, generator=g) * 2 - 1) * math.pi if s["cplx"] else None
    Tk = torch.tanh(torch.randn(D, NT, generator=g) * 1.5) if NT else None
    dy = torch.randn(B, L, D, generator=g)
    # stored values: what both sides compute from
    delta, u = delta.to(s["dt_in"]), u.to(s["dt_in"])
    Bc, Cc = Bc.to(s["dt_bc"]), Cc.to(s["dt_bc"])
    return delta, u, Bc, Cc, Ar, Ai, Tk, dy


def _placed(t, layout, pad_seed):
    """(leaf, view): the device view in the given layout and the leaf that
    owns its storage (the view's gradient is read back from the leaf)."""
    Bn, L, X = t.shape
    if layout == "contig":
        leaf = t.to(dev).clone().requires_grad_(True)
        return leaf, leaf
    if layout == "pad":
        off = 1 + pad_seed % 5
        big = torch.zeros(Bn, L, X + off + 3, dtype=t.dtype)
        big[..., off:off + X] = t
        leaf = big.to(dev).requires_grad_(True)
        return leaf, leaf[..., off:off + X]
    leaf = t.transpose(0, 1).contiguous().to(dev).requires_grad_(True)  # (L, B, X)
    return leaf, leaf.transpose(0, 1)


def _grad_of(leaf, layout, X, pad_seed):
    g = leaf.grad
    if layout == "contig":
        return g
    if layout == "pad":
        off = 1 + pad_seed % 5
        return g[..., off:off + X]
    return g.transpose(0, 1)


def _oracle32(delta, u, Bc, Cc, Ar, Ai, Tk, dy, N, bidir, softplus):
    f = lambda t: None if t is None else t.float().clone().requires_grad_(True)
    lv = [f(t) for t in (delta, u, Bc, Cc, Ar, Ai, Tk)]
    x, uu, b, c, ar, ai, tk = lv
    dl = F.softplus(x) if softplus else x
    y, _ = scan_ref.contracted_scan_ref(dl, uu, b, c, ar, ai, tk, N)
    if bidir:
        yr, _ = scan_ref.contracted_scan_ref(dl.flip(1), uu.flip(1), b.flip(1), c.flip(1),
                                             ar, ai, tk, N)
        y = y + yr.flip(1)
    (y * dy).sum().backward()
    return y.detach(), [None if t is None else t.grad for t in lv]


def _oracle64(delta, u, Bc, Cc, Ar, Ai, Tk, dy, bidir, softplus):
    d = lambda t: None if t is None else t.double()
    x, uu, b, c, ar, ai, tk = (d(t) for t in (delta, u, Bc, Cc, Ar, Ai, Tk))
    dl = F.softplus(x) if softplus else x
    args = (dl, uu, b, c, ar, ai, tk)
    y, _, _ = scan_ref.scan_sequential(*args)
    gr = scan_ref.scan_adjoint(*args, dy.double())
    if bidir:
        y = y + scan_ref.scan_sequential(*args, reverse=True)[0]
        g2 = scan_ref.scan_adjoint(*args, dy.double(), reverse=True)
        gr = {k: (None if v is None else v + g2[k]) for k, v in gr.items()}
    names = ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk")
    out = [gr[k] for k in names]
    if softplus and out[0] is not None:
        out[0] = out[0] * torch.sigmoid(x)
    return y, out


@pytest.mark.parametrize("case", range(16 * SCALE))
def test_scan_shape_sweep(gpu_lib, case):
    from redpanda_amd.scan import hip_trapezoidal_scan
    s = _draw(case)
    delta, u, Bc, Cc, Ar, Ai, Tk, dy = _inputs(s, case)
    print(f"[scan sweep {case}] {s}", flush=True)
    placed = [_placed(t, lay, case + i) for i, (t, lay) in
              enumerate(zip((delta, u, Bc, Cc), s["layouts"]))]
    prm = [None if t is None else t.to(dev).clone().requires_grad_(True) for t in (Ar, Ai, Tk)]
    y = hip_trapezoidal_scan(*[v for _, v in placed], *prm, s["NR"], s["N"],
                             bidirectional=s["bidir"], delta_softplus=s["softplus"])
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    hip_g = [_grad_of(leaf, lay, t.shape[-1], case + i) for i, ((leaf, _), lay, t) in
             enumerate(zip(placed, s["layouts"], (delta, u, Bc, Cc)))]
    hip_g += [None if p is None else p.grad for p in prm]
    y32, g32 = _oracle32(delta, u, Bc, Cc, Ar, Ai, Tk, dy, s["N"], s["bidir"], s["softplus"])
    y64, g64 = _oracle64(delta, u, Bc, Cc, Ar, Ai, Tk, dy, s["bidir"], s["softplus"])
    ey = (rel(y, y32), rel(y, y64), rel(y32, y64))
    assert y.dtype == torch.float32
    assert within_bar(*ey, FWD_TOL), f"y {ey}"
    report = {"y": ey}
    names = ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk")
    stored = (s["dt_in"], s["dt_in"], s["dt_bc"], s["dt_bc"]) + (torch.float32,) * 3
    for name, hg, r32, r64, dt in zip(names, hip_g, g32, g64, stored):
        if r32 is None:
            assert hg is None, name
            continue
        assert hg.dtype == dt, f"{name}: gradient dtype {hg.dtype}, input {dt}"
        e = (rel(hg, r32), rel(hg, r64), rel(r32, r64))
        report[name] = e
        if dt == torch.float32:
            assert within_bar(*e, GRAD_TOL), f"{name} (hip-ref, hip-f64, ref-f64) = {e}"
        else:
            assert e[0] <= ULP[dt], f"{name} ({dt}) hip-ref {e[0]:.3e}"
    print(" ".join("%s[%.1e %.1e %.1e]" % (k, *v) for k, v in report.items()),
          "(hip-ref hip-f64 ref-f64)", flush=True)
