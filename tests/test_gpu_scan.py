"""GPU parity of the HIP scan (forward, bidirectional, backward, final state)
against the oracle and the reference's own fp32 outputs (golden fixtures).

Metric everywhere: norm-wise relative error max|a - b| / max|b| per tensor.
Bars (fp32): forward <= 1e-5 and gradients <= 1e-6 against the reference's
fp32 path.  Both implementations are also measured against float64; where
the reference's own fp32 error exceeds the bar (long sequences: its
Hillis-Steele products drift), the HIP result must instead be at least as
close to float64 as the reference is (`within_bar`).
Kernel parity goes through the C ABI (tests/hip_capi.py) so gradients are
compared in fp32 whatever the storage dtype of the inputs.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import scan_ref
from tests.conftest import golden_names, load_golden
from tests import hip_capi

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-5
GRAD_TOL = 1e-6
dev = "cuda"


def _scan():
    from redpanda_amd.scan import hip_trapezoidal_scan, hip_scan_with_state
    return hip_trapezoidal_scan, hip_scan_with_state


def rel(a, b):
    return scan_ref.rel_err(a.detach().cpu(), b.detach().cpu())


# ─── golden fixtures: the reference's fp32 outputs and gradients ────────────

@pytest.mark.parametrize("name", golden_names("scan_"))
def test_golden_forward_and_grads(gpu_lib, name):
    scan, _ = _scan()
    g = load_golden(name)
    bidir = name.endswith("bi1")
    leaves = {k: g[k].to(dev).requires_grad_(True) for k in ("u", "delta", "B", "C", "Dskip")}
    Ar = g["A_real"].to(dev).requires_grad_(True) if "A_real" in g else None
    Ai = g["A_imag"].to(dev).requires_grad_(True) if "A_imag" in g else None
    th = g["theta"].to(dev).requires_grad_(True) if "theta" in g else None
    N = g["B"].shape[2]
    NR = 0 if Ar is None else Ar.shape[-1]
    Tk = torch.tanh(th) if th is not None else None
    Bc, Cc = leaves["B"].sum(-1), leaves["C"].sum(-1)
    u, D = leaves["u"], leaves["Dskip"]
    y = scan(leaves["delta"], u, Bc, Cc, Ar, Ai, Tk, NR, N, bidirectional=bidir)
    y = y + u * D
    if bidir:
        y = y + u * D
    e_fwd = rel(y, g["y"])
    (y * g["dout"].to(dev)).sum().backward()
    errs = {"y": e_fwd}
    for k in ("u", "delta", "B", "C", "Dskip"):
        errs[k] = rel(leaves[k].grad, g["grad_" + k])
    if Ar is not None:
        errs["A_real"] = rel(Ar.grad, g["grad_A_real"])
    if Ai is not None:
        errs["A_imag"] = rel(Ai.grad, g["grad_A_imag"])
    if th is not None:
        errs["theta"] = rel(th.grad, g["grad_theta"])
    print(name, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs.pop("y") <= FWD_TOL
    for k, v in errs.items():
        assert v <= GRAD_TOL, f"{name}: grad {k} rel err {v:.3e}"


@pytest.mark.parametrize("name", [n for n in golden_names("scan_") if n.endswith("bi0")])
def test_golden_final_state(gpu_lib, name):
    _, scan_state = _scan()
    g = load_golden(name)
    Ar = g.get("A_real")
    Ai = g.get("A_imag")
    Tk = torch.tanh(g["theta"]) if "theta" in g else None
    to = lambda t: None if t is None else t.to(dev)
    y, (h, b) = scan_state(g["delta"].to(dev), g["u"].to(dev), g["B"].sum(-1).to(dev),
                           g["C"].sum(-1).to(dev), to(Ar), to(Ai), to(Tk))
    y = y + g["u"].to(dev) * g["Dskip"].to(dev)
    assert rel(y, g["y_eval"]) <= FWD_TOL
    assert rel(h, g["state_h"]) <= FWD_TOL
    assert rel(b, g["state_beta"]) <= FWD_TOL


# ─── synthetic cases: shapes, edge lengths, dtypes ──────────────────────────

def make_case(seed, B, L, D, NR, NT, complex_=True, dtype=torch.float32, ar_hi=3.0):
    """BASELINE-style inputs: dt = softplus(N(-2, .5)), x ~ N(0,1), RMS-normalised
    B/C, Ar = -exp(U(0, ar_hi)), Ai = U(-pi, pi), Tk = tanh(N(0, 1.5))."""
    gen = torch.Generator().manual_seed(seed)
    N = NR + NT
    u = torch.randn(B, L, D, generator=gen)
    dt = F.softplus(torch.randn(B, L, D, generator=gen) * 0.5 - 2.0)
    Bc = torch.randn(B, L, N, generator=gen)
    Cc = torch.randn(B, L, N, generator=gen)
    Bc = Bc / Bc.pow(2).mean(-1, keepdim=True).sqrt()
    Cc = Cc / Cc.pow(2).mean(-1, keepdim=True).sqrt()
    Ar = -torch.exp(torch.rand(D, NR, generator=gen) * ar_hi) if NR else None
    Ai = (torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi if (NR and complex_) else None
    Tk = torch.tanh(torch.randn(D, NT, generator=gen) * 1.5) if NT else None
    dy = torch.randn(B, L, D, generator=gen)
    # storage dtype (bf16 / fp16): the oracle consumes the same rounded values
    u, dt, Bc, Cc = (t.to(dtype) for t in (u, dt, Bc, Cc))
    return dict(delta=dt, u=u, Bc=Bc, Cc=Cc, Ar=Ar, Ai=Ai, Tk=Tk, dy=dy, N=N, NR=NR)


def oracle_fp32(c, bidirectional=False):
    f = lambda t: None if t is None else t.float()
    args = [f(c[k]) for k in ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk")]
    leaves = [a.clone().requires_grad_(True) if a is not None else None for a in args]
    dl, uu, Bc, Cc, Ar, Ai, Tk = leaves
    y, _ = scan_ref.contracted_scan_ref(dl, uu, Bc, Cc, Ar, Ai, Tk, c["N"])
    if bidirectional:
        yr, _ = scan_ref.contracted_scan_ref(dl.flip(1), uu.flip(1), Bc.flip(1), Cc.flip(1),
                                             Ar, Ai, Tk, c["N"])
        y = y + yr.flip(1)
    (y * c["dy"]).sum().backward()
    grads = {k: (t.grad if t is not None else None)
             for k, t in zip(("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk"), leaves)}
    return y.detach(), grads


def oracle_fp64(c, bidirectional=False):
    args = [c[k] for k in ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk")]
    y, _, _ = scan_ref.scan_sequential(*args)
    grads = scan_ref.scan_adjoint(*args, c["dy"])
    if bidirectional:
        yr, _, _ = scan_ref.scan_sequential(*args, reverse=True)
        y = y + yr
        gr = scan_ref.scan_adjoint(*args, c["dy"], reverse=True)
        grads = {k: (None if v is None else v + gr[k]) for k, v in grads.items()}
    return y, grads


def hip_run(c, bidirectional=False):
    return hip_capi.scan_fwd_bwd(c, bidirectional)


def within_bar(e_hip_ref, e_hip_64, e_ref_64, tol):
    """Pass at `tol` against the reference, or, where the reference's own fp32
    error already exceeds `tol`, be no further from float64 than it is."""
    return e_hip_ref <= tol or e_hip_64 <= max(tol, e_ref_64)


def compare(c, bidirectional, tag, grad_tol=GRAD_TOL, record=None):
    y, g = hip_run(c, bidirectional)
    y32, g32 = oracle_fp32(c, bidirectional)
    y64, g64 = oracle_fp64(c, bidirectional)
    rep = {"y": (rel(y, y32), rel(y, y64), rel(y32, y64))}
    for k in g:
        if g[k] is None:
            continue
        rep[k] = (rel(g[k], g32[k]), rel(g[k], g64[k]), rel(g32[k], g64[k]))
    print(tag, " ".join("%s[%.1e %.1e %.1e]" % (k, *v) for k, v in rep.items()),
          "(hip-ref hip-f64 ref-f64)", flush=True)
    if record is not None:
        g = {k: v for k, v in rep.items() if k != "y"}
        wk = max(g, key=lambda k: g[k][0])
        record("parity", f"scan {tag}: y hip-ref {rep['y'][0]:.1e} (hip-f64 {rep['y'][1]:.1e}, "
                         f"ref-f64 {rep['y'][2]:.1e}); worst grad hip-ref {g[wk][0]:.1e} ({wk}; "
                         f"hip-f64 {g[wk][1]:.1e}, ref-f64 {g[wk][2]:.1e})")
    assert within_bar(*rep.pop("y"), FWD_TOL), tag
    for k, v in rep.items():
        assert within_bar(*v, grad_tol), f"{tag}: grad {k} (hip-ref, hip-f64, ref-f64) = {v}"
    return rep


@pytest.mark.parametrize("L", [1, 7, 8, 9, 15, 16, 17, 31, 32, 33, 64, 65, 100])
def test_edge_lengths(gpu_lib, L):
    c = make_case(100 + L, B=2, L=L, D=40, NR=8, NT=4)
    compare(c, False, f"L={L}")


def test_empty_sequence(gpu_lib):
    """L = 0: nothing to scan, and every parameter gradient is zero."""
    c = make_case(99, B=2, L=0, D=40, NR=8, NT=4)
    for bidir in (False, True):
        y, g = hip_run(c, bidir)
        assert y.shape == (2, 0, 40)
        for k in ("Ar", "Ai", "Tk"):
            assert torch.count_nonzero(g[k]).item() == 0, k


@pytest.mark.parametrize("D", [1, 16, 63, 64, 65, 200])
def test_channel_counts(gpu_lib, D):
    c = make_case(200 + D, B=2, L=20, D=D, NR=12, NT=4)
    compare(c, True, f"D={D}")


@pytest.mark.parametrize("NR,NT,cplx", [(1, 0, True), (0, 3, True), (16, 0, False), (12, 4, True),
                                        (30, 10, True), (32, 8, True), (16, 4, True),
                                        (56, 8, True), (64, 8, True), (120, 8, True),
                                        (32, 0, True), (64, 0, True)])
def test_state_splits(gpu_lib, NR, NT, cplx):
    c = make_case(300 + NR * 7 + NT, B=2, L=40, D=48, NR=NR, NT=NT, complex_=cplx)
    compare(c, False, f"NR={NR} NT={NT} complex={cplx}")


@pytest.mark.parametrize("N", [16, 32, 64])
@pytest.mark.parametrize("bidir", [False, True])
@pytest.mark.parametrize("cplx", [True, False])
def test_all_rotational_whole_tiles(gpu_lib, N, bidir, cplx):
    """Every state rotational (complex) or decaying (real) at d_state 16, 32
    and 64 (the reference's default configurations and its CPU one) over
    whole channel tiles: the whole-tile kernels' all-rotational and all-real
    instantiations against the oracle."""
    c = make_case(700 + N, B=2, L=37, D=64, NR=N, NT=0, complex_=cplx)
    compare(c, bidir, f"all {'rotational' if cplx else 'real'} N={N} bidirectional={bidir}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_low_precision_storage(gpu_lib, dtype):
    c = make_case(400, B=2, L=64, D=96, NR=32, NT=8, dtype=dtype)
    compare(c, True, f"storage={dtype}")


def test_mixed_input_dtypes(gpu_lib):
    """autocast hands over bf16 u with fp32 delta/B/C: each is loaded as is."""
    c = make_case(401, B=2, L=33, D=64, NR=12, NT=4)
    c["u"] = c["u"].to(torch.bfloat16)
    compare(c, False, "mixed dtypes")


def test_eval_mamba_shape_reduced_batch(gpu_lib, record_property):
    """C2/C3 shape (D=1536, N=40 = 32 rot + 8 track, L=64, bf16 storage) at B=2."""
    c = make_case(1002, B=2, L=64, D=1536, NR=32, NT=8, dtype=torch.bfloat16)
    compare(c, True, "eval-mamba bidir B=2", record=record_property)


def test_long_sequence_reduced(gpu_lib, record_property):
    """C5 shape per channel (L=2048, N=72 = 64 rot + 8 track) at B=1, D=64."""
    c = make_case(1005, B=1, L=2048, D=64, NR=64, NT=8)
    compare(c, False, "long L=2048", record=record_property)


def test_autograd_wrapper_dtype_contract(gpu_lib):
    """Through autograd, y is fp32 and each gradient comes back in its input's
    dtype (engine/triton_scan.py:278-281, :313-315), equal to the fp32 kernel
    gradient rounded once."""
    scan, _ = _scan()
    c = make_case(402, B=2, L=40, D=64, NR=12, NT=4, dtype=torch.bfloat16)
    lv = {k: (None if c[k] is None else c[k].to(dev).requires_grad_(True))
          for k in ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk")}
    y = scan(lv["delta"], lv["u"], lv["Bc"], lv["Cc"], lv["Ar"], lv["Ai"], lv["Tk"], 12, 16)
    assert y.dtype == torch.float32
    (y * c["dy"].to(dev)).sum().backward()
    _, g = hip_run(c)
    for k, v in lv.items():
        if v is None:
            continue
        assert v.grad.dtype == v.dtype, k
        assert torch.equal(v.grad.cpu(), g[k].to(v.dtype)), k


def test_backward_is_deterministic(gpu_lib):
    c = make_case(500, B=3, L=50, D=130, NR=16, NT=4)
    _, g1 = hip_run(c, True)
    _, g2 = hip_run(c, True)
    for k in g1:
        if g1[k] is not None:
            assert torch.equal(g1[k], g2[k]), k


@pytest.mark.parametrize("NR,NT,D", [(12, 4, 128), (16, 4, 128), (32, 8, 64), (24, 9, 64),
                                     (40, 8, 48), (56, 8, 48), (64, 8, 48), (88, 8, 48),
                                     (120, 8, 48)])
@pytest.mark.parametrize("softplus", [False, True])
def test_whole_tile_backward_equals_general(gpu_lib, NR, NT, D, softplus):
    """The backward's whole-tile instantiation (no initial state, no final-state
    gradients, D a multiple of the tile) against its general one on the same
    causal scan, taken by passing an all-zero initial state and all-zero
    final-state gradients: every output bit for bit (L=37 ends in a partial
    chunk).  The state counts cover every lane split (4, 8 and 16 lanes per
    channel, 1 to 8 states per lane, padded slots) and so every way the
    channel-sum fold's outputs divide into rounds over the workgroup."""
    c = make_case(505, B=3, L=37, D=D, NR=NR, NT=NT)
    if softplus:
        c["delta"] = torch.randn(c["delta"].shape, generator=torch.Generator().manual_seed(5)) - 2
    N = NR + NT
    y1, g1 = hip_capi.scan_fwd_bwd(c, softplus=softplus)
    zero = torch.zeros(3, D, N)
    y2, g2 = hip_capi.scan_fwd_bwd(c, dh_last=zero, dbeta_last=zero, softplus=softplus)
    y3, g3 = hip_capi.scan_fwd_bwd(c, h0=zero, beta0=zero, softplus=softplus)
    assert torch.equal(y1, y2) and torch.equal(y1, y3)
    for k in g1:
        if g1[k] is not None:
            assert torch.equal(g1[k], g2[k]), f"final-state gradients, {k}"
            assert torch.equal(g1[k], g3[k]), f"initial state, {k}"


@pytest.mark.parametrize("D", [128, 120])
@pytest.mark.parametrize("bidir", [False, True])
def test_backward_tile_walk_matches_single_tile(gpu_lib, D, bidir):
    """At 16 lanes per channel (16-channel tiles) a large batch has each
    backward workgroup walk 4 adjacent channel tiles, whose dB / dC partials
    add into one block; a single batch row runs one tile per workgroup.  Rows
    are independent, so every checked row of the large batch has the
    single-row run's bits in y, d_delta and d_u (per-channel sums), and its
    dB / dC within about one fp32 rounding per tile (their partials are added
    in another order).  D=120 leaves a partial tile: the general
    instantiation walks too."""
    B, L, NR, NT = 1100, 9, 64, 8
    c = make_case(808, B=B, L=L, D=D, NR=NR, NT=NT)
    y, g = hip_capi.scan_fwd_bwd(c, bidir)
    for r in (0, 517, B - 1):
        cr = {k: (v[r:r + 1] if k in ("delta", "u", "Bc", "Cc", "dy") else v) for k, v in c.items()}
        yr, gr = hip_capi.scan_fwd_bwd(cr, bidir)
        assert torch.equal(y[r:r + 1], yr), r
        assert torch.equal(g["delta"][r:r + 1], gr["delta"]), r
        assert torch.equal(g["u"][r:r + 1], gr["u"]), r
        for k in ("Bc", "Cc"):
            e = rel(g[k][r:r + 1], gr[k])
            assert e <= 1e-6, f"row {r} d{k}: {e:.2e}"


@pytest.mark.parametrize("bidir", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,L,D,NR,NT,softplus", [
    (2, 37, 96, 32, 8, False),     # 8 lanes, whole tiles, a one-step last chunk
    (3, 64, 100, 12, 4, True),     # 4 lanes, a partial tile, softplus on load
    (2, 70, 64, 64, 8, False),     # 16 lanes
    (1100, 9, 128, 64, 8, False),  # 16 lanes, 4 channel tiles per workgroup
])
def test_gradients_in_storage_dtype(gpu_lib, B, L, D, NR, NT, softplus, dtype, bidir):
    """grad_in_storage: d_delta and d_u leave the backward in delta's and u's
    16-bit dtype, rounded to nearest even: bit for bit torch's conversion of
    the fp32 gradients that the default writes, every other output unchanged
    (a bidirectional scan keeps its first direction's sums in the workspace)."""
    c = make_case(900 + B + D, B=B, L=L, D=D, NR=NR, NT=NT, dtype=dtype)
    if softplus:  # the dt projection x, softplus(x) ~ dt
        c["delta"] = torch.log(torch.expm1(c["delta"].float())).to(dtype)
    y0, g0 = hip_capi.scan_fwd_bwd(c, bidir, softplus=softplus)
    y1, g1 = hip_capi.scan_fwd_bwd(c, bidir, softplus=softplus, grad_in_storage=True)
    assert torch.equal(y0, y1)
    assert g1["delta"].dtype == dtype and g1["u"].dtype == dtype
    assert torch.equal(g1["delta"], g0["delta"].to(dtype))
    assert torch.equal(g1["u"], g0["u"].to(dtype))
    for k in ("Bc", "Cc", "Ar", "Ai", "Tk"):
        assert (g0[k] is None and g1[k] is None) or torch.equal(g0[k], g1[k]), k


def test_gradients_in_storage_dtype_mixed(gpu_lib):
    """fp32 delta with bf16 u: d_delta stays fp32, d_u leaves in bf16."""
    c = make_case(931, B=2, L=50, D=96, NR=32, NT=8, dtype=torch.bfloat16)
    c["delta"] = c["delta"].float()
    y0, g0 = hip_capi.scan_fwd_bwd(c, True)
    y1, g1 = hip_capi.scan_fwd_bwd(c, True, grad_in_storage=True)
    assert g1["delta"].dtype == torch.float32 and g1["u"].dtype == torch.bfloat16
    assert torch.equal(g1["delta"], g0["delta"])
    assert torch.equal(g1["u"], g0["u"].to(torch.bfloat16))


def test_linearity_in_u(gpu_lib):
    scan, _ = _scan()
    c = make_case(501, B=2, L=40, D=64, NR=12, NT=4)
    to = lambda t: None if t is None else t.to(dev)
    y1 = scan(to(c["delta"]), to(c["u"]), to(c["Bc"]), to(c["Cc"]), to(c["Ar"]), to(c["Ai"]),
              to(c["Tk"]), 12, 16)
    y2 = scan(to(c["delta"]), to(c["u"] * -2.0), to(c["Bc"]), to(c["Cc"]), to(c["Ar"]),
              to(c["Ai"]), to(c["Tk"]), 12, 16)
    assert rel(y2, -2.0 * y1) <= 1e-6


def test_bidirectional_equals_forward_plus_flipped(gpu_lib):
    scan, _ = _scan()
    c = make_case(502, B=2, L=45, D=64, NR=12, NT=4)
    to = lambda t: None if t is None else t.to(dev)
    args = [to(c[k]) for k in ("delta", "u", "Bc", "Cc")]
    p = [to(c[k]) for k in ("Ar", "Ai", "Tk")]
    yb = scan(*args, *p, 12, 16, bidirectional=True)
    yf = scan(*args, *p, 12, 16)
    yr = scan(*[a.flip(1).contiguous() for a in args], *p, 12, 16).flip(1)
    assert torch.equal(yb, yf + yr)


def test_final_state_gradients(gpu_lib):
    """Gradient through (y, h_last, beta_last) matches float64 autograd."""
    _, scan_state = _scan()
    c = make_case(503, B=2, L=37, D=48, NR=12, NT=4)
    gen = torch.Generator().manual_seed(9)
    dh = torch.randn(2, 48, 16, generator=gen)
    db = torch.randn(2, 48, 16, generator=gen)
    names = ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk")
    lv = {k: c[k].to(dev).requires_grad_(True) for k in names}
    y, (h, b) = scan_state(*[lv[k] for k in names])
    ((y * c["dy"].to(dev)).sum() + (h * dh.to(dev)).sum() + (b * db.to(dev)).sum()).backward()
    lv64 = {k: c[k].double().requires_grad_(True) for k in names}
    y64, h64, b64 = scan_ref.scan_sequential(*[lv64[k] for k in names])
    ((y64 * c["dy"].double()).sum() + (h64 * dh.double()).sum() + (b64 * db.double()).sum()).backward()
    for k in names:
        e = rel(lv[k].grad, lv64[k].grad)
        assert e <= 2e-6, f"{k}: {e:.3e}"


# ─── whole-tile fast paths against the partial-tile path, bit for bit ───────

def _lanes_per_channel(N):
    return 4 if N <= 20 else (8 if N <= 40 else 16)


STORAGE = {
    # (delta / u storage, B / C storage, softplus on load); the last two take
    # the forward's instantiation for the model's launches
    "fp32": (torch.float32, torch.float32, False),
    "bf16": (torch.bfloat16, torch.bfloat16, False),
    "fp16": (torch.float16, torch.float16, False),
    "model-bf16": (torch.bfloat16, torch.float32, True),
    "model-fp16": (torch.float16, torch.float32, True),
}


@pytest.mark.parametrize("N,NT", [(20, 4), (40, 8), (72, 8), (32, 0), (64, 0)])
@pytest.mark.parametrize("storage", sorted(STORAGE))
@pytest.mark.parametrize("bidir", [False, True])
def test_whole_tile_paths_equal_partial_tile(gpu_lib, N, NT, storage, bidir):
    """Channels are independent, so a launch over D = CB channels (one whole
    tile: the forward's fast staging of full blocks, and the backward's
    whole-tile instantiation) and one over D = CB - 1 (a partial tile: the
    element-wise staging and the general backward) must give the first CB - 1
    channels the same bits: y; for causal scans the final state; d_delta,
    d_u and the parameter gradients, each a per-channel sum in a fixed order
    (dB / dC sum over channels and are left out).  L = 70 covers full blocks
    and a tail; storage types, directions and the softplus-on-load delta
    cache (read back by the reverse direction) as the kernels take them."""
    dt_in, dt_bc, softplus = STORAGE[storage]
    CB = 4 * (64 // _lanes_per_channel(N))
    c = make_case(600 + N, B=3, L=70, D=CB, NR=N - NT, NT=NT)
    if softplus:
        c["delta"] = torch.randn(c["delta"].shape, generator=torch.Generator().manual_seed(6)) - 2
    c["delta"], c["u"] = c["delta"].to(dt_in), c["u"].to(dt_in)
    c["Bc"], c["Cc"] = c["Bc"].to(dt_bc), c["Cc"].to(dt_bc)
    part = dict(c)
    for k in ("delta", "u", "dy"):
        part[k] = c[k][:, :, :CB - 1].contiguous()
    for k in ("Ar", "Ai", "Tk"):
        part[k] = None if c[k] is None else c[k][:CB - 1].contiguous()
    y1, g1 = hip_capi.scan_fwd_bwd(c, bidir, softplus=softplus)
    y2, g2 = hip_capi.scan_fwd_bwd(part, bidir, softplus=softplus)
    same = lambda a, b: torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert same(y1[:, :, :CB - 1].contiguous(), y2), "y"
    for k in ("delta", "u"):
        assert same(g1[k][:, :, :CB - 1].contiguous(), g2[k]), k
    for k in ("Ar", "Ai", "Tk"):
        if g1[k] is not None:
            assert same(g1[k][:CB - 1].contiguous(), g2[k]), k
    if not bidir:
        _, _, (h1, b1), keep1 = hip_capi.scan_fwd(c, with_state=True, softplus=softplus)
        _, _, (h2, b2), keep2 = hip_capi.scan_fwd(part, with_state=True, softplus=softplus)
        torch.cuda.synchronize()
        assert same(h1[:, :CB - 1].contiguous().cpu(), h2.cpu()), "h_last"
        assert same(b1[:, :CB - 1].contiguous().cpu(), b2.cpu()), "beta_last"
