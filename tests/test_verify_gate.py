"""The self-verification gate (redpanda_amd/verify.py; the reference's gate is
engine/triton_scan.py:342-398): its float64 checker agrees with the oracle,
its criteria refuse planted errors (CPU), and the HIP path passes it (GPU)."""

import math

import pytest
import torch

from oracle import scan_ref
from redpanda_amd import verify as gate


def _case(seed, B=2, L=9, D=5, NR=3, NT=2):
    g = torch.Generator().manual_seed(seed)
    N = NR + NT
    f = dict(dtype=torch.float64)
    u = torch.randn(B, L, D, generator=g, **f)
    dt = torch.nn.functional.softplus(torch.randn(B, L, D, generator=g, **f) - 1)
    Bc = torch.randn(B, L, N, generator=g, **f)
    Cc = torch.randn(B, L, N, generator=g, **f)
    Ar = -torch.exp(torch.rand(D, NR, generator=g, **f))
    Ai = (torch.rand(D, NR, generator=g, **f) * 2 - 1) * math.pi
    Tk = torch.tanh(torch.randn(D, NT, generator=g, **f))
    return u, dt, Ar, Ai, Bc, Cc, Tk


@pytest.mark.parametrize("reverse", [False, True])
def test_gate_checker_scan_matches_oracle(reverse):
    u, dt, Ar, Ai, Bc, Cc, Tk = _case(1)
    y = gate._scan64(u, dt, Ar, Ai, Bc, Cc, Tk, reverse=reverse)
    y_ref, _, _ = scan_ref.scan_sequential(dt, u, Bc, Cc, Ar, Ai, Tk, reverse=reverse)
    assert torch.allclose(y, y_ref, rtol=1e-13, atol=1e-13)


def _errs(y_err=0.0, g_err=0.0):
    y64 = torch.linspace(-2, 2, 50, dtype=torch.float64)
    g64 = {"w": torch.linspace(-1e-3, 3e-3, 20, dtype=torch.float64)}
    y = (y64 + y_err).float()
    grads = {"w": (g64["w"] + g_err).float()}
    return gate.gate_errors(y, y64, grads, g64)


def test_gate_accepts_fp32_rounding():
    gate.check_gate(_errs())


@pytest.mark.parametrize("y_err,g_err,needle", [
    (3e-3, 0.0, "forward mismatch"),        # the reference gate's forward bound
    (1e-3, 0.0, "norm-wise"),               # passes 2e-3 max-abs, not 1e-4 of |y|=2
    (0.0, 1e-6, "grad mismatch (norm-wise)"),  # tiny gradients: the clamped metric misses it
])
def test_gate_refuses_planted_errors(y_err, g_err, needle):
    with pytest.raises(AssertionError, match=needle.replace("(", r"\(").replace(")", r"\)")):
        gate.check_gate(_errs(y_err, g_err))


def _oracle_case(planted=None):
    """The gate's comparison run on the CPU with the oracle's fp32
    restatement of the reference model standing in for the product:
    (errors of the fp32 run, errors of the fp32 run with `planted` applied).
    planted: "trapezoid" drops the 1/2 g beta_prev term of every scan token
    (engine/mamba.py:409-412), "grad" scales one gradient by 1 + 3e-4."""
    from oracle import model_ref
    torch.manual_seed(4)
    cfg = model_ref.MambaConfig(d_model=16, n_layer=2, d_state=8, n_track_state=2, mimo_p=2,
                                vocab_size=64, bidirectional=True)
    m = model_ref.Mamba(cfg)
    with torch.no_grad():
        gen = torch.Generator().manual_seed(5)
        for layer in m.layers:
            layer["mixer"].A_phase.copy_((torch.rand(layer["mixer"].A_phase.shape, generator=gen) * 2 - 1) * 1.4)
    m.train()
    ids = torch.randint(0, 64, (2, 33), generator=torch.Generator().manual_seed(6))
    proj = torch.randn(2, 33, 16, generator=torch.Generator().manual_seed(7))
    params64 = {k: v.detach().double().requires_grad_(True) for k, v in m.named_parameters()}
    y64 = gate._model64(m, ids, params64)
    (y64 * proj.double()).sum().backward()
    g64 = {k: v.grad for k, v in params64.items()}

    def fp32_run():
        m.zero_grad(set_to_none=True)
        y = m(ids)
        (y * proj).sum().backward()
        return y.detach(), {k: p.grad.clone() for k, p in m.named_parameters()}

    y, grads = fp32_run()
    clean = gate.gate_errors(y, y64.detach(), grads, g64)
    if planted == "trapezoid":
        orig = scan_ref.scan_chunk_ref

        def dropped(delta_c, u_c, B_c, C_c, h, beta_prev, A_real, A_imag, track):
            # the planted mistake: tokens without the 1/2 g beta_{t-1} term
            gates = scan_ref.gate_tensor_ref(delta_c, A_real, A_imag, track)
            beta = torch.einsum("bld,bln->bldn", delta_c, B_c) * u_c.unsqueeze(-1)
            tokens = 0.5 * beta
            first = tokens[:, 0] + gates[:, 0] * h.to(gates.dtype)
            tokens = torch.cat([first.unsqueeze(1), tokens[:, 1:]], dim=1)
            hs = scan_ref.hillis_steele_scan(gates, tokens)
            return torch.einsum("bldn,bln->bld", hs, C_c), hs[:, -1], beta[:, -1]
        scan_ref.scan_chunk_ref = dropped
        try:
            y, grads = fp32_run()
        finally:
            scan_ref.scan_chunk_ref = orig
    elif planted == "grad":
        grads = dict(grads)
        grads["layers.0.mixer.A_phase"] = grads["layers.0.mixer.A_phase"] * (1 + 3e-4)
    return clean, gate.gate_errors(y, y64.detach(), grads, g64)


def test_gate_passes_the_reference_algorithm():
    """The reference's own fp32 algorithm (the oracle) passes the gate."""
    clean, _ = _oracle_case()
    gate.check_gate(clean)


@pytest.mark.parametrize("planted,needle", [("trapezoid", "mismatch"),
                                            ("grad", "grad mismatch \\(norm-wise\\)")])
def test_gate_refuses_a_planted_model_error(planted, needle):
    """A whole model's results with a planted mistake (a dropped trapezoid
    term in every scan; one parameter gradient 3e-4 off) are refused."""
    _, bad = _oracle_case(planted)
    with pytest.raises(AssertionError, match=needle):
        gate.check_gate(bad)


@pytest.mark.gpu
def test_hip_path_passes_the_gate(gpu_lib):
    assert gate.verify("cuda", thorough=False, verbose=True)


@pytest.mark.gpu
def test_hip_path_passes_the_thorough_gate(gpu_lib, record_property):
    """The reference gate's full matrix (engine/triton_scan.py:353-357):
    d_model 512 with d_state 64 of which 16 tracking and mimo_p 4 beside the
    two small configurations, L in {1, 31, 32, 33, 70, 107, 160}, both
    directions."""
    assert gate.verify("cuda", thorough=True, verbose=True)
    record_property("parity", "gate verify(thorough=True): 42 cases within 2e-3 (reference "
                              "criteria) and 1e-4 norm-wise of float64")
