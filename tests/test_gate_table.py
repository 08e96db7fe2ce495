"""The rotational gate tables (redpanda_amd/csrc/rp_sincos_table.h) and the
expansions the kernels evaluate from them (rp_device.h rot_gate_finish and
rot_gate_finish_cs), checked on the CPU against float64 trigonometry.

The committed header must be exactly what gen_sincos_table.py writes; every
record must be the correctly rounded fp32 value of its sign-folded quantity;
the sign bit of m must carry b = sign(cos) for every entry, zeros included;
and the kernels' cubic in the remainder r, evaluated from a record with the
kernels' constants, must give cos (and, for the backward, sin) of the angle
to within the truncation and representation bounds.  A planted table that
rounds cos itself, the form the sign-folded records replaced, is refused by
the repeated-error bound near |cos| = 1.
"""

import importlib.util
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "redpanda_amd", "csrc")
T = 256
A = 2 * np.pi / T
ULP1 = 2.0 ** -24  # ulp of floats just below 1 (the gate's scale)


def _gen():
    spec = importlib.util.spec_from_file_location("gen_sincos_table",
                                                  os.path.join(CSRC, "gen_sincos_table.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _header_tables():
    """{name: (T, 2) float32} parsed from the committed header."""
    text = open(os.path.join(CSRC, "rp_sincos_table.h")).read()
    out = {}
    for name in ("kCosLin", "kSinCos"):
        body = text.split(f"{name}[kTab] = {{", 1)[1].split("};", 1)[0]
        vals = [float.fromhex(v) for v in re.findall(r"(-?0x[0-9a-fA-F.]+p[-+]\d+)f", body)]
        out[name] = np.array(vals, dtype=np.float64).astype(np.float32).reshape(T, 2)
    return out


def _constants():
    """The expansion constants as rp_device.h writes them."""
    text = open(os.path.join(CSRC, "rp_device.h")).read()
    get = lambda n: float(np.float32(re.search(rf"\b{n} = (-?[0-9.e+-]+)f", text).group(1)))
    return {n: get(n) for n in ("kC2", "kA3", "kS1", "kS3")}


def _exact():
    k = np.arange(T)
    c, s = np.cos(A * k), np.sin(A * k)
    for q in range(4):  # quadrant points exactly
        c[q * T // 4], s[q * T // 4] = [(1, 0), (0, 1), (-1, 0), (0, -1)][q]
    b = np.where(c >= 0, 1.0, -1.0)
    return c, s, b


def _correctly_rounded(rec, exact):
    """|rec - exact| <= half an fp32 ulp of exact (float64 stands in for the
    exact value: its own error is ~1e-16 relative)."""
    ex32 = exact.astype(np.float32)
    ulp = np.spacing(np.abs(ex32)).astype(np.float64)
    ulp = np.where(ex32 == 0, np.float64(np.finfo(np.float32).smallest_subnormal), ulp)
    return np.abs(rec.astype(np.float64) - exact) <= 0.5 * ulp * (1 + 1e-6) + 1e-300


def test_header_is_the_generators_output():
    fwd, bwd = _gen().records()
    tab = _header_tables()
    assert np.array_equal(tab["kCosLin"].view(np.uint32), fwd.view(np.uint32))
    assert np.array_equal(tab["kSinCos"].view(np.uint32), bwd.view(np.uint32))


def test_records_are_the_rounded_sign_folded_values():
    tab = _header_tables()
    c, s, b = _exact()
    m = tab["kCosLin"][:, 0]
    assert np.array_equal(tab["kSinCos"][:, 0].view(np.uint32), m.view(np.uint32))
    # b rides in the sign bit of m, for every entry (m is +0 at k = 0, -0 at k = 128)
    assert np.array_equal(np.signbit(m), b < 0)
    assert m[0] == 0 and not np.signbit(m[0]) and m[128] == 0 and np.signbit(m[128])
    assert _correctly_rounded(m, b * (1 - np.abs(c))).all()
    assert _correctly_rounded(tab["kCosLin"][:, 1], b * (-s * A)).all()
    assert _correctly_rounded(tab["kSinCos"][:, 1], b * s).all()


def _repeated_error_near_one(m_rec, c, b):
    """Worst representation error of the gate's constant term, in ulps of 1,
    over the entries with |cos| >= 0.99 (the long-memory gates)."""
    near = np.abs(c) >= 0.99
    err = np.abs(np.abs(m_rec.astype(np.float64)) - (1 - np.abs(c)))
    return float(err[near].max() / ULP1)


def test_repeated_error_near_unit_gates():
    """Below 0.02 ulp where |cos| >= 0.99; a table of rounded cosines (the
    form the sign-folded records replaced) repeats up to 0.5 ulp there and
    is refused."""
    c, s, b = _exact()
    m = _header_tables()["kCosLin"][:, 0]
    assert _repeated_error_near_one(m, c, b) < 0.02
    planted = (b - c.astype(np.float32).astype(np.float64)).astype(np.float32)
    assert _repeated_error_near_one(planted, c, b) > 0.1


def _cos_expansion(m, t, r, k):
    """rot_gate_finish's w = cos / b - 1 in float64 from the fp32 record."""
    am = np.abs(m)
    p3 = t * k["kA3"]
    p2 = -am * k["kC2"] + k["kC2"]
    return r * (r * (r * p3 + p2) + t) - am


def _cs_expansion(m, sb, r, k):
    """rot_gate_finish_cs's (w, v) = (cos / b - 1, sin / b) in float64."""
    am = np.abs(m)
    r2 = r * r
    cm1 = r2 * k["kC2"]
    sx = r * (r2 * k["kS3"] + k["kS1"])
    w = -sb * sx + (-am * cm1 + (cm1 - am))
    v = (sb * cm1 + sb) + (-am * sx + sx)
    return w, v


def _half_ulp(x):
    """Half an fp32 ulp of |x| (x held as fp32)."""
    return 0.5 * np.spacing(np.abs(np.asarray(x, dtype=np.float32))).astype(np.float64)


@pytest.mark.parametrize("flavour", ["forward", "backward"])
def test_expansion_gives_cos_and_sin(flavour):
    """Over every entry and remainders r in [-1/2, 1/2], b (1 + w) is cos(a (k
    + r)) and b v is sin(a (k + r)) to within the fp32 representation of the
    record's terms (half an ulp of |m| and of r times the slope) plus 2e-9
    (truncation below 1e-9, the constants' rounding the rest).  Where |cos|
    is close to 1, |m| is small and the bound is close to 2e-9: the accuracy
    the long-memory gates rely on."""
    tab = _header_tables()
    k = _constants()
    r = np.linspace(-0.5, 0.5, 41)[None, :]
    ang = A * (np.arange(T)[:, None] + r)
    rec = tab["kCosLin"] if flavour == "forward" else tab["kSinCos"]
    m = rec[:, 0].astype(np.float64)[:, None]
    sl = rec[:, 1].astype(np.float64)[:, None]
    sign = np.where(np.signbit(rec[:, 0]), -1.0, 1.0)[:, None]
    hm, hs = _half_ulp(rec[:, 0])[:, None], _half_ulp(rec[:, 1])[:, None]
    if flavour == "forward":
        w = _cos_expansion(m, sl, r, k)
        bound = hm + 0.5 * hs + 2e-9
    else:
        w, v = _cs_expansion(m, sl, r, k)
        # sin / b carries the slope's own rounding (b s) and |m| times sin(a r)
        assert (np.abs(sign * v - np.sin(ang)) <= hs + A * hm + 2e-9).all()
        bound = hm + A * 0.5 * hs + 2e-9
    err = np.abs(sign * (1 + w) - np.cos(ang))
    assert (err <= bound).all(), float((err / bound).max())
    # near the unit gates the bound is the tight one
    near = (np.abs(rec[:, 0]) <= 0.01)[:, None] & np.ones_like(err, dtype=bool)
    assert err[near].max() < 3e-9


def test_expansion_refuses_a_planted_coefficient():
    """A dropped cubic term (p3 = 0), a sign flip of the slope and the sine's
    cubic coefficient left out each break the bound."""
    tab = _header_tables()
    k = _constants()
    r = np.linspace(-0.5, 0.5, 41)[None, :]
    ang = A * (np.arange(T)[:, None] + r)
    rec = tab["kCosLin"]
    m = rec[:, 0].astype(np.float64)[:, None]
    t = rec[:, 1].astype(np.float64)[:, None]
    sign = np.where(np.signbit(rec[:, 0]), -1.0, 1.0)[:, None]
    hm, hs = _half_ulp(rec[:, 0])[:, None], _half_ulp(rec[:, 1])[:, None]
    over = lambda w: bool((np.abs(sign * (1 + w) - np.cos(ang)) > hm + 0.5 * hs + 2e-9).any())
    assert over(_cos_expansion(m, t, r, dict(k, kA3=0.0)))
    assert over(_cos_expansion(m, -t, r, k))
    rs = tab["kSinCos"]
    _, v = _cs_expansion(rs[:, 0].astype(np.float64)[:, None], rs[:, 1].astype(np.float64)[:, None], r,
                         dict(k, kS3=0.0))
    s_sign = np.where(np.signbit(rs[:, 0]), -1.0, 1.0)[:, None]
    bound = _half_ulp(rs[:, 1])[:, None] + A * _half_ulp(rs[:, 0])[:, None] + 2e-9
    assert (np.abs(s_sign * v - np.sin(ang)) > bound).any()
