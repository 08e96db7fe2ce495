"""Pin the CPU oracle (oracle/scan_ref.py, oracle/model_ref.py).

The oracle is only trusted after these pass:
  * golden fixtures: the fp32 restatement reproduces the reference's own
    PyTorch outputs and autograd gradients bit-for-bit (fixtures written by
    tests/golden/make_golden.py from the reference itself);
  * closed forms and invariants that a dropped term, a wrong sign, a wrong
    time index or a transposed operand would break;
  * the float64 sequential scan agrees with the fp32 restatement, and its
    hand-derived adjoint agrees with autograd and with finite differences.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import scan_ref
from oracle import model_ref
from tests.conftest import golden_names, load_golden


def _track(theta):
    return torch.tanh(theta)


def _scan_inputs(g):
    Ar = g.get("A_real")
    Ai = g.get("A_imag")
    Tk = _track(g["theta"]) if "theta" in g else None
    N = g["B"].shape[2]
    return Ar, Ai, Tk, N


# ─── golden fixtures (reference outputs) ────────────────────────────────────

@pytest.mark.parametrize("name", golden_names("scan_"))
def test_scan_matches_reference_bits(name):
    g = load_golden(name)
    Ar, Ai, Tk, N = _scan_inputs(g)
    bidir = name.endswith("bi1")
    leaves = {k: g[k].clone().requires_grad_(True) for k in ("u", "delta", "B", "C")}
    Arl = Ar.clone().requires_grad_(True) if Ar is not None else None
    Ail = Ai.clone().requires_grad_(True) if Ai is not None else None
    th = g["theta"].clone().requires_grad_(True) if "theta" in g else None
    Dl = g["Dskip"].clone().requires_grad_(True)
    # the reference evaluates tanh(theta) once per scan call (engine/mamba.py:338)
    tk = lambda: torch.tanh(th) if th is not None else None
    y = scan_ref.selective_scan_ref(leaves["u"], leaves["delta"], Arl, Ail, leaves["B"],
                                    leaves["C"], Dl, tk(), N, checkpoint=True)
    if bidir:
        y = y + scan_ref.selective_scan_ref(
            leaves["u"].flip(1), leaves["delta"].flip(1), Arl, Ail, leaves["B"].flip(1),
            leaves["C"].flip(1), Dl, tk(), N, checkpoint=True).flip(1)
    assert torch.equal(y.detach(), g["y"]), f"{name}: y differs by {(y - g['y']).abs().max()}"
    (y * g["dout"]).sum().backward()
    for k, v in leaves.items():
        assert torch.equal(v.grad, g["grad_" + k]), f"{name}: grad {k}"
    if Arl is not None:
        assert torch.equal(Arl.grad, g["grad_A_real"])
    if Ail is not None:
        assert torch.equal(Ail.grad, g["grad_A_imag"])
    if th is not None:
        assert torch.equal(th.grad, g["grad_theta"])
    assert torch.equal(Dl.grad, g["grad_Dskip"])
    if not bidir:
        y2, (h, b) = scan_ref.selective_scan_ref(g["u"], g["delta"], Ar, Ai, g["B"], g["C"],
                                                 g["Dskip"], Tk, N, return_state=True)
        assert torch.equal(y2, g["y_eval"])
        assert torch.equal(h, g["state_h"]) and torch.equal(b, g["state_beta"])


def _load_block(g, cfg):
    blk = model_ref.Mamba3Block(cfg).eval()
    sd = {k[3:]: v for k, v in g.items() if k.startswith("sd.")}
    blk.load_state_dict(sd)
    return blk


@pytest.mark.parametrize("name,kw", [
    ("step_rot_trk", dict(d_model=8, d_state=12, n_track_state=4, mimo_p=2)),
    ("step_real", dict(d_model=8, d_state=8, mimo_p=2, use_complex=False)),
])
def test_step_matches_reference_bits(name, kw):
    g = load_golden(name)
    cfg = model_ref.MambaConfig(vocab_size=64, n_layer=1, **kw)
    blk = _load_block(g, cfg)
    with torch.no_grad():
        o1, (h1, b1) = blk.step(g["x"], None)
        o2, (h2, b2) = blk.step(g["x"], (g["h0"], g["beta0"]))
    for a, k in [(o1, "out_none"), (h1, "h_none"), (b1, "beta_none"),
                 (o2, "out"), (h2, "h"), (b2, "beta")]:
        assert torch.equal(a, g[k]), f"{name}:{k} max diff {(a - g[k]).abs().max()}"


@pytest.mark.parametrize("bidir", [False, True])
def test_model_matches_reference_bits(bidir):
    g = load_golden(f"model_bi{int(bidir)}")
    cfg = model_ref.MambaConfig(d_model=16, n_layer=2, d_state=12, n_track_state=4, mimo_p=2,
                                vocab_size=64, bidirectional=bidir)
    m = model_ref.Mamba(cfg)
    sd = {k[3:]: v for k, v in g.items() if k.startswith("sd.")}
    assert sorted(sd) == sorted(m.state_dict()), "state_dict keys differ from the reference"
    m.load_state_dict(sd)
    m.train()
    y = m(g["ids"])
    assert torch.equal(y.detach(), g["y_train"])
    y.pow(2).mean().backward()
    for k, p in m.named_parameters():
        if "grad." + k in g:
            assert torch.equal(p.grad, g["grad." + k]), k
    m.eval()
    with torch.no_grad():
        assert torch.equal(m(g["ids"]), g["y_eval"])
        if not bidir:
            cache, outs = None, []
            for t in range(g["ids"].shape[1]):
                hdn, cache = m.step(token_id=g["ids"][:, t], cache=cache)
                outs.append(hdn)
            assert torch.equal(torch.stack(outs, 1), g["y_step"])
            fin, pc = m.prime_cache(g["ids"][:, :20])
            assert torch.equal(fin, g["prime_final"])
            for i, (h, b) in enumerate(pc):
                assert torch.equal(h, g[f"prime_h{i}"]) and torch.equal(b, g[f"prime_beta{i}"])
            nxt, _ = m.step(token_id=g["ids"][:, 20], cache=pc)
            assert torch.equal(nxt, g["prime_next"])


def test_seeded_init_matches_reference():
    """Same construction / RNG consumption order as engine/mamba.py:151-207, :508-532."""
    g = load_golden("model_bi0")
    torch.manual_seed(5)
    cfg = model_ref.MambaConfig(d_model=16, n_layer=2, d_state=12, n_track_state=4, mimo_p=2,
                                vocab_size=64)
    m = model_ref.Mamba(cfg)
    sd = m.state_dict()
    for k, v in sd.items():
        if k.endswith(("A_phase", "A_log_mag", "track_theta")):
            continue  # the fixture script overwrote these after init
        assert torch.equal(v, g["sd." + k]), k


# ─── fp64 sequential scan vs the fp32 restatement and closed forms ──────────

def _rand_case(seed, B=2, L=9, D=5, NR=3, NT=2, complex_=True):
    gen = torch.Generator().manual_seed(seed)
    N = NR + NT
    u = torch.randn(B, L, D, generator=gen, dtype=torch.float64)
    dt = F.softplus(torch.randn(B, L, D, generator=gen, dtype=torch.float64) * 0.5 - 1.0)
    Bc = torch.randn(B, L, N, generator=gen, dtype=torch.float64)
    Cc = torch.randn(B, L, N, generator=gen, dtype=torch.float64)
    Ar = -torch.exp(torch.rand(D, NR, generator=gen, dtype=torch.float64) * 2) if NR else None
    Ai = ((torch.rand(D, NR, generator=gen, dtype=torch.float64) * 2 - 1) * math.pi
          if (NR and complex_) else None)
    Tk = torch.tanh(torch.randn(D, NT, generator=gen, dtype=torch.float64)) if NT else None
    return dt, u, Bc, Cc, Ar, Ai, Tk


@pytest.mark.parametrize("L", [1, 7, 32, 33, 70])
def test_fp64_sequential_matches_fp32_restatement(L):
    dt, u, Bc, Cc, Ar, Ai, Tk = _rand_case(3, L=L)
    N = Bc.shape[-1]
    y64, h64, b64 = scan_ref.scan_sequential(dt, u, Bc, Cc, Ar, Ai, Tk)
    f = lambda t: None if t is None else t.float()
    y32, (h32, b32) = scan_ref.contracted_scan_ref(f(dt), f(u), f(Bc), f(Cc), f(Ar), f(Ai), f(Tk), N)
    assert scan_ref.rel_err(y32, y64) < 2e-6
    assert scan_ref.rel_err(h32, h64) < 2e-6
    assert scan_ref.rel_err(b32, b64) < 2e-6


def test_closed_form_length_one():
    """L = 1: y0 = 1/2 dt0 u0 sum_n B0 C0 (no previous token, g irrelevant)."""
    dt, u, Bc, Cc, Ar, Ai, Tk = _rand_case(4, L=1)
    y, h, b = scan_ref.scan_sequential(dt, u, Bc, Cc, Ar, Ai, Tk)
    expect = 0.5 * dt[:, 0] * u[:, 0] * (Bc[:, 0] * Cc[:, 0]).sum(-1).unsqueeze(-1)
    assert torch.allclose(y[:, 0], expect, rtol=1e-12, atol=1e-12)


def test_closed_form_unit_gate_is_trapezoid_sum():
    """g == 1 (Tk = 1 on every lane): h_t = sum_{s<t} beta_s + beta_t / 2."""
    dt, u, Bc, Cc, _, _, _ = _rand_case(5, L=11, NR=0, NT=4)
    D = u.shape[-1]
    Tk = torch.ones(D, 4, dtype=torch.float64)
    _, hL, _ = scan_ref.scan_sequential(dt, u, Bc, Cc, None, None, Tk)
    beta = (dt * u).unsqueeze(-1) * Bc.unsqueeze(2)        # (B, L, D, N)
    expect = beta[:, :-1].sum(1) + 0.5 * beta[:, -1]
    assert torch.allclose(hL, expect, rtol=1e-12, atol=1e-12)


def test_closed_form_zero_gate_is_half_beta():
    dt, u, Bc, Cc, _, _, _ = _rand_case(6, L=6, NR=0, NT=3)
    Tk = torch.zeros(u.shape[-1], 3, dtype=torch.float64)
    y, hL, bL = scan_ref.scan_sequential(dt, u, Bc, Cc, None, None, Tk)
    beta = (dt * u).unsqueeze(-1) * Bc.unsqueeze(2)
    assert torch.allclose(hL, 0.5 * beta[:, -1], atol=1e-14)
    assert torch.allclose(y, 0.5 * (beta * Cc.unsqueeze(2)).sum(-1), atol=1e-13)


def test_closed_form_constant_inputs_geometric_series():
    """Constant dt, u, B and a constant real gate g: h_t = b (1 + g) (1 - g^t)/(1 - g)/2 + b g^t / 2
    with b = dt u B; so h_t -> b (1 + g) / (2 (1 - g))."""
    B, L, D, N = 1, 25, 2, 3
    dt = torch.full((B, L, D), 0.3, dtype=torch.float64)
    u = torch.full((B, L, D), 1.7, dtype=torch.float64)
    Bc = torch.tensor([0.5, -1.0, 2.0], dtype=torch.float64).expand(B, L, N).clone()
    Cc = torch.ones(B, L, N, dtype=torch.float64)
    Ar = torch.full((D, N), -0.9, dtype=torch.float64)
    g = math.exp(0.3 * -0.9)
    _, hL, _ = scan_ref.scan_sequential(dt, u, Bc, Cc, Ar, None, None)
    b = 0.3 * 1.7 * Bc[0, 0]
    t = L - 1
    # h_0 = b/2 ; h_t = g h_{t-1} + b/2 + g b/2  ->  closed form
    expect = (b / 2) * g ** t + (b / 2) * (1 + g) * (1 - g ** t) / (1 - g)
    assert torch.allclose(hL[0, 0], expect, rtol=1e-12)


def test_closed_form_parity_flip():
    """Tk = -1: h_t = -h_{t-1} + beta_t/2 - beta_{t-1}/2; with beta constant, h alternates."""
    B, L, D, N = 1, 8, 1, 1
    dt = torch.full((B, L, D), 0.5, dtype=torch.float64)
    u = torch.full((B, L, D), 2.0, dtype=torch.float64)
    Bc = torch.ones(B, L, N, dtype=torch.float64)
    Cc = torch.ones(B, L, N, dtype=torch.float64)
    Tk = -torch.ones(D, N, dtype=torch.float64)
    y, _, _ = scan_ref.scan_sequential(dt, u, Bc, Cc, None, None, Tk)
    # beta = 1: h0 = 0.5, then h_t = -h_{t-1} + 0.5 - 0.5 = -h_{t-1}
    expect = torch.tensor([0.5 * (-1) ** t for t in range(L)], dtype=torch.float64)
    assert torch.allclose(y[0, :, 0], expect)


def test_rotation_gate_is_real_cosine():
    """A rotational lane with Ar = 0 has gate cos(dt Ai): a real, sign-changing gate."""
    B, L, D = 1, 5, 1
    dt = torch.full((B, L, D), 1.0, dtype=torch.float64)
    u = torch.zeros(B, L, D, dtype=torch.float64)
    u[0, 0, 0] = 2.0
    Bc = torch.ones(B, L, 1, dtype=torch.float64)
    Cc = torch.ones(B, L, 1, dtype=torch.float64)
    Ar = torch.zeros(D, 1, dtype=torch.float64)
    Ai = torch.full((D, 1), math.pi, dtype=torch.float64)  # g = cos(pi) = -1
    y, _, _ = scan_ref.scan_sequential(dt, u, Bc, Cc, Ar, Ai, None)
    # beta_0 = 2: h0 = 1 ; h1 = -1*1 + 0 + 0.5*(-1)*2 = -2 ; h2 = 2 ; ...
    assert torch.allclose(y[0, :, 0], torch.tensor([1.0, -2.0, 2.0, -2.0, 2.0], dtype=torch.float64))


def test_linearity_in_u():
    dt, u, Bc, Cc, Ar, Ai, Tk = _rand_case(7, L=13)
    y1, _, _ = scan_ref.scan_sequential(dt, u, Bc, Cc, Ar, Ai, Tk)
    y2, _, _ = scan_ref.scan_sequential(dt, -2.5 * u, Bc, Cc, Ar, Ai, Tk)
    assert torch.allclose(y2, -2.5 * y1, rtol=1e-12, atol=1e-12)


def test_chunk_split_carry_equivalence():
    """scan([0, s)) carried into scan([s, L)) equals scan([0, L))."""
    dt, u, Bc, Cc, Ar, Ai, Tk = _rand_case(8, L=20)
    yf, hf, bf = scan_ref.scan_sequential(dt, u, Bc, Cc, Ar, Ai, Tk)
    s = 7
    ya, ha, ba = scan_ref.scan_sequential(dt[:, :s], u[:, :s], Bc[:, :s], Cc[:, :s], Ar, Ai, Tk)
    yb, hb, bb = scan_ref.scan_sequential(dt[:, s:], u[:, s:], Bc[:, s:], Cc[:, s:], Ar, Ai, Tk,
                                          h0=ha, beta0=ba)
    assert torch.allclose(torch.cat([ya, yb], 1), yf, rtol=1e-12, atol=1e-12)
    assert torch.allclose(hb, hf, rtol=1e-12, atol=1e-12)


def test_reverse_equals_flip():
    dt, u, Bc, Cc, Ar, Ai, Tk = _rand_case(9, L=10)
    yr, _, _ = scan_ref.scan_sequential(dt, u, Bc, Cc, Ar, Ai, Tk, reverse=True)
    yf, _, _ = scan_ref.scan_sequential(dt.flip(1), u.flip(1), Bc.flip(1), Cc.flip(1), Ar, Ai, Tk)
    assert torch.allclose(yr, yf.flip(1), rtol=1e-13, atol=1e-13)


def test_step_core_equals_scan_step():
    """step_core_ref advanced L times equals the scan (engine/test_v3.py:44-56 pattern)."""
    dt, u, Bc, Cc, Ar, Ai, Tk = _rand_case(10, L=12)
    f = lambda t: None if t is None else t.float()
    N = Bc.shape[-1]
    y, _ = scan_ref.contracted_scan_ref(f(dt), f(u), f(Bc), f(Cc), f(Ar), f(Ai), f(Tk), N)
    state, outs = None, []
    Dz = torch.zeros(u.shape[-1])
    for t in range(u.shape[1]):
        yt, state = scan_ref.step_core_ref(f(dt[:, t]), f(u[:, t]), f(Bc[:, t]), f(Cc[:, t]),
                                           f(Ar), f(Ai), f(Tk), Dz, state)
        outs.append(yt)
    assert scan_ref.rel_err(torch.stack(outs, 1), y) < 1e-6


# ─── adjoint: autograd and finite differences ───────────────────────────────

@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("complex_", [True, False])
def test_adjoint_matches_autograd(reverse, complex_):
    dt, u, Bc, Cc, Ar, Ai, Tk = _rand_case(11, L=9, complex_=complex_)
    dy = torch.randn(u.shape, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    leaves = [t.clone().requires_grad_(True) if t is not None else None
              for t in (dt, u, Bc, Cc, Ar, Ai, Tk)]
    y, _, _ = scan_ref.scan_sequential(*leaves, reverse=reverse)
    (y * dy).sum().backward()
    adj = scan_ref.scan_adjoint(dt, u, Bc, Cc, Ar, Ai, Tk, dy, reverse=reverse)
    for name, leaf in zip(("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk"), leaves):
        if leaf is None:
            continue
        assert torch.allclose(adj[name], leaf.grad, rtol=1e-10, atol=1e-11), name


def test_gradcheck_finite_differences():
    dt, u, Bc, Cc, Ar, Ai, Tk = _rand_case(12, B=1, L=4, D=2, NR=2, NT=1)
    fn = lambda *a: scan_ref.scan_sequential(*a)[0]
    inputs = tuple(t.clone().requires_grad_(True) for t in (dt, u, Bc, Cc, Ar, Ai, Tk))
    assert torch.autograd.gradcheck(fn, inputs, eps=1e-6, atol=1e-7)


def test_planted_error_is_caught():
    """A dropped trapezoid term in the oracle must fail the closed-form check."""
    dt, u, Bc, Cc, _, _, _ = _rand_case(5, L=11, NR=0, NT=4)
    D = u.shape[-1]
    Tk = torch.ones(D, 4, dtype=torch.float64)
    beta = (dt * u).unsqueeze(-1) * Bc.unsqueeze(2)
    wrong = beta.sum(1)                              # forgot the 1/2 on the last token
    _, hL, _ = scan_ref.scan_sequential(dt, u, Bc, Cc, None, None, Tk)
    assert not torch.allclose(hL, wrong, rtol=1e-6)


# ─── rollout ply host reads (oracle/rollout_ref.py) ─────────────────────────

def test_rollout_candidates_match_reference_expression():
    """On tie-free rows the oracle's candidate list is exactly the reference's
    argpartition / argsort expression (engine/mars_search.py:262-265)."""
    import numpy as np
    from oracle import rollout_ref
    rng = np.random.default_rng(0)
    for V, k in [(8192, 8), (100, 8), (7, 8), (1, 1), (64, 16), (3000, 5)]:
        row = rng.standard_normal(V).astype(np.float32)
        ids, lns = rollout_ref.candidates(row, k)
        assert np.array_equal(ids, rollout_ref.candidates_reference_expr(row, k))
        assert np.array_equal(lns, row[ids])


def _numpy_order(row, k):
    """Brute force of numpy's order on a tiny row: NaN (either sign) above
    +inf, -0 equal to +0, equal values by ascending id."""
    import math
    key = lambda i: (0 if math.isnan(row[i]) else 1, 0.0 if math.isnan(row[i]) else -float(row[i]), i)
    return sorted(range(len(row)), key=key)[:min(k, len(row))]


def test_rollout_candidates_brute_force_and_ties():
    """Brute force on tiny rows with many ties, +-0, +-inf and NaNs of both
    signs: the list is the k largest in numpy's order, equal logits by
    ascending id; nothing outside beats anything inside.  A planted wrong
    order (ascending) fails the same check."""
    import numpy as np
    from oracle import rollout_ref
    rng = np.random.default_rng(1)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan], dtype=np.float32)
    neg_nan = np.array([0xffc00000], dtype=np.uint32).view(np.float32)[0]
    for _ in range(400):
        V = int(rng.integers(1, 9))
        k = int(rng.integers(1, 6))
        row = rng.integers(-2, 3, V).astype(np.float32)
        for i in range(V):
            if rng.random() < 0.3:
                row[i] = special[rng.integers(0, 5)] if rng.random() < 0.8 else neg_nan
        ids, lns = rollout_ref.candidates(row, k)
        assert _numpy_order(row, k) == list(ids)
        assert np.array_equal(lns.view(np.uint32), rollout_ref.canonical(row)[ids].view(np.uint32))
        rest = set(range(V)) - set(ids.tolist())
        ranks = {i: r for r, i in enumerate(_numpy_order(row, V))}
        assert all(ranks[j] > max(ranks[i] for i in ids) for j in rest)
        # a planted mistake (the k smallest, ascending) fails the same check
        wrong = list(reversed(_numpy_order(row, V)))[:min(k, V)]
        if len({(float(x) if x == x else "nan") for x in row}) > 1:
            assert wrong != list(ids)


def test_rollout_candidates_nan_against_reference_expr():
    """One NaN in an otherwise tie-free row: the reference's own expression
    (numpy's argpartition / argsort) puts it first, as candidates does."""
    import numpy as np
    from oracle import rollout_ref
    rng = np.random.default_rng(2)
    for V, k in [(300, 8), (40, 16), (9, 4)]:
        for sign in (1, -1):
            row = rng.standard_normal(V).astype(np.float32)
            j = int(rng.integers(0, V))
            row[j] = np.float32(np.nan) * sign
            ids, _ = rollout_ref.candidates(row, k)
            assert ids[0] == j
            assert np.array_equal(ids, rollout_ref.candidates_reference_expr(row, k))


def _draw_counts(select, logits, temp, n, seed):
    import numpy as np
    rng = np.random.default_rng(seed)
    row = np.asarray(logits, dtype=np.float32)
    counts = np.zeros(len(row), dtype=np.int64)
    for _ in range(n):
        counts[select(row, len(row), lambda t: True, temp, rng)] += 1
    return counts


def _softmax_ok(select, logits, temp, n=20000, seed=11):
    """Draw frequencies within 4.5 sigma of exp(l / T) / sum (computed here
    with math.exp, not the oracle's code)."""
    import math
    z = [math.exp(l / temp) for l in logits]
    p = [x / sum(z) for x in z]
    c = _draw_counts(select, logits, temp, n, seed)
    return all(abs(c[i] - n * p[i]) <= 4.5 * math.sqrt(n * p[i] * (1 - p[i])) + 1e-9
               for i in range(len(p)))


def test_rollout_select_draw_is_the_softmax():
    """The sampling branch of the walk (engine/mars_search.py:271-276),
    pinned by what the mathematics fixes: equal logits draw uniformly, a logit
    far above the rest is always drawn, frequencies match exp(l/T)/sum, and
    scaling logits and T by the same power of two changes no draw.  Planted
    mistakes (l*T for l/T, T ignored) fail."""
    import numpy as np
    from oracle import rollout_ref
    sel = rollout_ref.select_move
    assert _softmax_ok(sel, [1.0, 1.0, 1.0, 1.0], 0.7)
    assert _softmax_ok(sel, [2.0, 1.0, 0.5, -1.0], 0.8)
    assert _softmax_ok(sel, [0.3, -0.2, 0.1], 2.5)
    dominant = _draw_counts(sel, [10.0, 0.0, 0.0, 0.0], 0.1, 2000, 3)
    assert dominant[0] == 2000
    a = [sel(np.array([2.0, 1.0, 0.5, -1.0], np.float32), 4, lambda t: True, 0.8,
             np.random.default_rng(s)) for s in range(300)]
    b = [sel(np.array([8.0, 4.0, 2.0, -4.0], np.float32), 4, lambda t: True, 3.2,
             np.random.default_rng(s)) for s in range(300)]
    assert a == b

    def planted_product(row, k, is_legal, temp, rng):
        return sel(np.asarray(row) * temp * temp, k, is_legal, temp, rng)  # l*T

    def planted_no_temp(row, k, is_legal, temp, rng):
        return sel(row, k, is_legal, 1.0, rng)
    assert not _softmax_ok(planted_product, [2.0, 1.0, 0.5, -1.0], 0.8)
    assert not _softmax_ok(planted_no_temp, [2.0, 1.0, 0.5, -1.0], 0.3)


def test_rollout_gather_and_select_walk():
    import numpy as np
    from oracle import rollout_ref
    row = np.arange(10, dtype=np.float32) * 0.5
    assert np.array_equal(rollout_ref.gather_legal(row, [3, -1, 9, 10]),
                          np.array([1.5, -np.inf, 4.5, -np.inf], dtype=np.float32))
    # greedy: the first legal candidate, largest logit first
    assert rollout_ref.select_move(row, 4, lambda t: t % 2 == 0, 0.0, None) == 8
    assert rollout_ref.select_move(row, 4, lambda t: False, 0.0, None) is None
    # the draw: a softmax over the legal candidates, one rng.choice call
    a = rollout_ref.select_move(row, 4, lambda t: t != 9, 0.6, np.random.default_rng(5))
    lg = np.array([4.0, 3.5, 3.0]) / 0.6
    lg -= lg.max()
    pr = np.exp(lg) / np.exp(lg).sum()
    assert a == [8, 7, 6][int(np.random.default_rng(5).choice(3, p=pr))]
