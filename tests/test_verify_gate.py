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


@pytest.mark.gpu
def test_hip_path_passes_the_gate(gpu_lib):
    assert gate.verify("cuda", thorough=False, verbose=True)
