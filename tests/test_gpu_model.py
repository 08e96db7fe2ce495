"""GPU parity of the drop-in backbone (redpanda_amd.mamba / search_mamba).

Three kinds of reference:
  * the golden fixtures: the reference's own modules run on the CPU
    (tests/golden/make_golden.py), compared across devices;
  * the oracle's restatement of the reference modules (oracle/model_ref.py)
    run on the same GPU with the same weights, so the projections and norms
    use the same GPU GEMMs and only the SSM core differs;
  * the same oracle in float64, the arbiter of accuracy.

The fp32 bars (forward <= 1e-5, gradients <= 1e-6, norm-wise
max|a-b|/max|b| per tensor) are checked layer by layer: every layer of a
model is fed the float64 run's input to that layer and the float64 run's
gradient of its output (both rounded to fp32), and the HIP layer's output,
input gradient and parameter gradients are compared with the reference
layer's on those same inputs.  A tensor passes if it is within the bar of
the reference, or, where the reference itself is further than the bar from
float64, if HIP's distance from float64 exceeds the reference's by no more
than the bar.

End to end over a whole model the bars are not meaningful: a 12-layer stack
puts any fp32 implementation ~2e-5 from float64, and which of two equally
accurate fp32 runs is closer on a given tensor is chance.  A control shows
it: the reference model with its scan evaluated exactly (float64) is, tensor
by tensor, up to ~2x further from float64 than the plain reference.  End to
end the tests therefore check accuracy in aggregate: the geometric mean over
all tensors of HIP's distance from float64, relative to the reference's, is
at most END_TO_END_GEO; the control's figures are printed beside HIP's.
"""

import contextlib
import math

import pytest
import torch

from oracle import model_ref, scan_ref
from tests.conftest import load_golden

pytestmark = pytest.mark.gpu
dev = "cuda"
FWD_TOL = 1e-5
GRAD_TOL = 1e-6
# autocast: one ulp of the autocast dtype, relative to a tensor's largest value
AMP_TOL = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}
# end to end: HIP no further from float64 than the reference, in aggregate,
# up to the scatter of that mean (+-0.02 over seeds at the 12-layer shape)
END_TO_END_GEO = 1.05
# end to end, per tensor: a guard against gross errors (a dropped term or a
# wrong sign shows up as a ratio of 10 and more).  Equally accurate fp32 runs
# scatter tensor by tensor: the exact-scan control (a reference model whose
# scan has no rounding error at all) measured up to 1.79x the plain
# reference's distance from float64 on the models tested here
END_TO_END_GUARD = 2.0


def rel(a, b):
    return scan_ref.rel_err(a.detach().float().cpu(), b.detach().float().cpu())


def _hip():
    from redpanda_amd import mamba as hm
    return hm


def _ref_state(cfg_kw, seed, perturb=True):
    """A reference model's state_dict.  With `perturb`, A / theta are moved
    off their structured init so every lane matters, keeping
    Re(A) = -exp(log_mag) cos(phase) < 0 (|phase| < pi/2): a positive real
    part makes exp(dt Re A) > 1 and the scan grow without bound, which no
    fp32 implementation reproduces."""
    torch.manual_seed(seed)
    ref = model_ref.Mamba(model_ref.MambaConfig(**cfg_kw))
    if perturb:
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
    return ref.state_dict()


def _pair(cfg_kw, seed=0, perturb=True, sd=None):
    """(hip model, oracle model) on the GPU with identical weights (a seeded
    reference init, or the given state_dict)."""
    hm = _hip()
    if sd is None:
        sd = _ref_state(cfg_kw, seed, perturb)
    ref = model_ref.Mamba(model_ref.MambaConfig(**cfg_kw))
    ref.load_state_dict(sd)
    hip = hm.Mamba(hm.MambaConfig(**cfg_kw))
    hip.load_state_dict(sd)
    return hip.to(dev), ref.to(dev)


def _f64(cfg_kw, sd):
    m = model_ref.Mamba(model_ref.MambaConfig(**cfg_kw)).to(dev).double()
    m.load_state_dict(sd)
    return m


def _grads(m):
    return {k: p.grad for k, p in m.named_parameters() if p.grad is not None}


def _inputs(cfg_kw, B, L, seed):
    gen = torch.Generator().manual_seed(seed + 7)
    ids = torch.randint(0, cfg_kw["vocab_size"], (B, L), generator=gen).to(dev)
    # upstream gradient dout ~ N(0, 1): a loss whose gradient is not a
    # cancellation residue (mean(norm_f(x)^2) is nearly constant in x)
    dout = torch.randn(B, L, cfg_kw["d_model"], generator=gen).to(dev)
    return ids, dout


def within_bar(e_hip_ref, e_hip_64, e_ref_64, tol):
    """Within `tol` of the reference, or no more than `tol` further from
    float64 than the reference is."""
    return e_hip_ref <= tol or e_hip_64 <= e_ref_64 + tol


def _amp(dtype):
    return torch.autocast("cuda", dtype=dtype) if dtype is not None else contextlib.nullcontext()


class _Fp32Scan:
    """The reference's GPU path under autocast: its scan kernel upcasts every
    input to fp32 (engine/triton_scan.py:251-254, :278-281), so the oracle's
    chunk scan runs with autocast off on fp32 copies of its inputs."""

    def __enter__(self):
        self.orig = model_ref.Mamba3Block._scan
        orig = self.orig

        def scan(blk, u, delta, A_real, A_imag, B, C, return_state=False):
            f = lambda t: None if t is None else t.float()
            with torch.autocast("cuda", enabled=False):
                return orig(blk, f(u), f(delta), f(A_real), f(A_imag), f(B), f(C), return_state)
        model_ref.Mamba3Block._scan = scan
        return self

    def __exit__(self, *exc):
        model_ref.Mamba3Block._scan = self.orig


class _ExactScan:
    """Control: the oracle model with its scan evaluated in float64 (inputs
    and outputs fp32), i.e. an fp32 model whose scan has no rounding error."""

    def __enter__(self):
        self.orig = model_ref.Mamba3Block._scan

        def scan(blk, u, delta, A_real, A_imag, B, C, return_state=False):
            cfg = blk.config
            d = lambda t: None if t is None else t.double()
            with torch.autocast("cuda", enabled=False):
                track = d(blk._track_gate()) if cfg.n_track_state > 0 else None
                return scan_ref.selective_scan_ref(d(u), d(delta), d(A_real), d(A_imag), d(B),
                                                   d(C), d(blk.D), track, cfg.d_state).float()
        model_ref.Mamba3Block._scan = scan
        return self

    def __exit__(self, *exc):
        model_ref.Mamba3Block._scan = self.orig


def _layer_trace(m64, ids, dout):
    """Each layer's mixer input and the gradient of its output in a float64
    training step of the whole model."""
    m64.train()
    m64.zero_grad(set_to_none=True)
    ins, outs = [], []
    x = m64.embedding(ids)
    for layer in m64.layers:
        xn = layer["norm"](x)
        ins.append(xn.detach())
        o = layer["mixer"](xn)
        o.retain_grad()
        outs.append(o)
        x = x + o
    (m64.norm_f(x) * dout.double()).sum().backward()
    return ins, [o.grad.detach() for o in outs]


def _layer_step(blk, x_in, g_out, dtype, amp):
    blk.train()
    blk.zero_grad(set_to_none=True)
    x = x_in.to(dtype).clone().requires_grad_(True)
    with _amp(amp):
        out = blk(x)
    (out.to(dtype) * g_out.to(dtype)).sum().backward()
    res = {"out": out.detach(), "x": x.grad.detach()}
    res.update({k: p.grad.detach().clone() for k, p in blk.named_parameters()
                if p.grad is not None})
    return res


def _teacher_forced(cfg_kw, B, L, seed, tag, record, amp=None, sd=None, ids=None,
                    anchor_control=False):
    """Layer-by-layer parity (see the module docstring): per tensor
    (hip-ref, hip-f64, ref-f64), within_bar with the fp32 bars, or one fp16
    ulp under fp16 autocast.  sd / ids: given weights and token ids instead
    of a seeded init and random ids.  anchor_control: the allowance is
    anchored at the larger of the reference's and the exact-scan control's
    distances from float64 (see test_golden_model_fixture_same_device)."""
    hip, ref = _pair(cfg_kw, seed, sd=sd)
    m64 = _f64(cfg_kw, ref.state_dict())
    rand_ids, dout = _inputs(cfg_kw, B, L, seed)
    ids = rand_ids if ids is None else ids.to(dev)
    ins, gouts = _layer_trace(m64, ids, dout)
    rows = []
    ctx = _Fp32Scan() if amp is not None else contextlib.nullcontext()
    with ctx:
        for i in range(len(ins)):
            xin, gin = ins[i].float(), gouts[i].float()
            rh = _layer_step(hip.layers[i]["mixer"], xin, gin, torch.float32, amp)
            rr = _layer_step(ref.layers[i]["mixer"], xin, gin, torch.float32, amp)
            r64 = _layer_step(m64.layers[i]["mixer"], xin, gin, torch.float64, None)
            with _ExactScan():
                rc = _layer_step(ref.layers[i]["mixer"], xin, gin, torch.float32, amp)
            for k in rr:
                tol = (AMP_TOL[amp] if amp is not None else (FWD_TOL if k == "out" else GRAD_TOL))
                rows.append((f"{i}.{k}", tol, rel(rh[k], rr[k]), rel(rh[k], r64[k]),
                             rel(rr[k], r64[k]), rel(rc[k], r64[k])))
    if anchor_control:
        bad = [r for r in rows if not within_bar(r[2], r[3], max(r[4], r[5]), r[1])]
    else:
        bad = [r for r in rows if not within_bar(*r[2:5], r[1])]
    worst = max(rows, key=lambda r: r[2] / r[1])
    excess = max(rows, key=lambda r: r[3] - r[4])
    geo = math.exp(sum(math.log(r[3] / r[4]) for r in rows) / len(rows))
    cgeo = math.exp(sum(math.log(r[5] / r[4]) for r in rows) / len(rows))
    line = (f"{tag} per layer: worst hip-ref {worst[2]:.1e} ({worst[0]}, bar {worst[1]:.0e}, "
            f"hip-f64 {worst[3]:.1e}, ref-f64 {worst[4]:.1e}); max hip-f64 minus ref-f64 "
            f"{excess[3] - excess[4]:+.1e} ({excess[0]}); geo-mean hip-f64/ref-f64 {geo:.2f} "
            f"(exact-scan control {cgeo:.2f}); {len(bad)}/{len(rows)} outside")
    print(line, flush=True)
    record("parity", line)
    assert not bad, f"{tag}: (tensor, bar, hip-ref, hip-f64, ref-f64) outside the bar: {bad[:6]}"


def _end_to_end(cfg_kw, B, L, seed, tag, record, amp=None, grad_checkpoint=False):
    """Whole-model accuracy against float64 (see the module docstring)."""
    hm = _hip()
    sd = _ref_state(cfg_kw, seed)
    ids, dout = _inputs(cfg_kw, B, L, seed)

    def step(m, amp_dtype):
        m.train()
        m.zero_grad(set_to_none=True)
        wide = torch.float64 if next(m.parameters()).dtype == torch.float64 else torch.float32
        with _amp(amp_dtype):
            y = m(ids)
            loss = (y.to(wide) * dout.to(wide)).sum()
        loss.backward()
        return y.detach(), _grads(m)

    y64, g64 = step(_f64(cfg_kw, sd), None)
    ref = model_ref.Mamba(model_ref.MambaConfig(**cfg_kw)).to(dev)
    ref.load_state_dict(sd)
    with (_Fp32Scan() if amp is not None else contextlib.nullcontext()):
        yr, gr = step(ref, amp)
    with _ExactScan():
        yc, gc = step(ref, amp)
    hip = hm.Mamba(hm.MambaConfig(**cfg_kw, grad_checkpoint=grad_checkpoint)).to(dev)
    hip.load_state_dict(sd)
    yh, gh = step(hip, amp)
    rows = [("y", rel(yh, yr), rel(yh, y64), rel(yr, y64), rel(yc, y64))]
    rows += [(k, rel(gh[k], gr[k]), rel(gh[k], g64[k]), rel(gr[k], g64[k]), rel(gc[k], g64[k]))
             for k in g64]
    ratio = [r[2] / r[3] for r in rows]
    cratio = [r[4] / r[3] for r in rows]
    geo = math.exp(sum(map(math.log, ratio)) / len(ratio))
    cgeo = math.exp(sum(map(math.log, cratio)) / len(cratio))
    worst = max(range(len(rows)), key=lambda i: ratio[i])
    wg = max(rows[1:], key=lambda r: r[1])
    line = (f"{tag} end to end: y hip-ref {rows[0][1]:.1e} (hip-f64 {rows[0][2]:.1e}, ref-f64 "
            f"{rows[0][3]:.1e}); worst grad hip-ref {wg[1]:.1e} ({wg[0]}; hip-f64 {wg[2]:.1e}, "
            f"ref-f64 {wg[3]:.1e}); hip-f64/ref-f64 geo-mean {geo:.2f} max {ratio[worst]:.2f} "
            f"({rows[worst][0]}); exact-scan control geo-mean {cgeo:.2f} max {max(cratio):.2f}")
    print(line, flush=True)
    record("parity", line)
    assert geo <= END_TO_END_GEO, line
    assert max(ratio) <= END_TO_END_GUARD, line
    if amp is None:
        assert within_bar(rows[0][1], rows[0][2], rows[0][3], FWD_TOL), line


SMALL = dict(d_model=32, n_layer=2, d_state=12, n_track_state=4, mimo_p=2, vocab_size=500)
REAL = dict(d_model=48, n_layer=2, d_state=16, n_track_state=0, mimo_p=2, vocab_size=500,
            use_complex=False, bidirectional=True)
# The Eval-Mamba training shape: 12 stacked bidirectional layers, d_model 768,
# d_inner 1536, d_state 40 = 32 rotational + 8 tracking, mimo_p 4, at a
# reduced batch of 8 boards x 64 tokens
EVAL12 = dict(d_model=768, n_layer=12, d_state=40, n_track_state=8, mimo_p=4, vocab_size=512,
              bidirectional=True)


@pytest.mark.parametrize("bidir", [False, True])
def test_small_model_layers_match_reference(gpu_lib, record_property, bidir):
    _teacher_forced(dict(SMALL, bidirectional=bidir), 3, 70, 1, f"small bidir={int(bidir)}",
                    record_property)


def test_real_decay_model_layers_match_reference(gpu_lib, record_property):
    _teacher_forced(REAL, 3, 33, 2, "real decay", record_property)


@pytest.mark.parametrize("bidir", [False, True])
def test_small_model_end_to_end_accuracy(gpu_lib, record_property, bidir):
    _end_to_end(dict(SMALL, bidirectional=bidir), 3, 70, 1, f"small bidir={int(bidir)}",
                record_property)


def test_real_decay_model_end_to_end_accuracy(gpu_lib, record_property):
    _end_to_end(REAL, 3, 33, 2, "real decay", record_property)


def test_eval_mamba_12_layers_per_layer(gpu_lib, record_property):
    """The C3 shape layer by layer: each of the 12 bidirectional layers
    within the fp32 bars of the reference layer on the same inputs."""
    _teacher_forced(EVAL12, 8, 64, 3, "eval-mamba 12L", record_property)


def test_eval_mamba_12_layers_end_to_end(gpu_lib, record_property):
    """The C3 shape end to end: 12 stacked layers, accuracy against float64
    no worse than the reference's in aggregate."""
    _end_to_end(EVAL12, 8, 64, 3, "eval-mamba 12L", record_property)


@pytest.mark.parametrize("amp", [None, torch.float16], ids=["fp32", "fp16-autocast"])
def test_grad_checkpoint_recompute_is_bitwise(gpu_lib, record_property, amp):
    """The reference trains with layer checkpointing and fp16 autocast on
    (engine/train.py:13, :103, :127; engine/mamba.py:544-553): backward
    re-runs every mixer.  The fused scan, BCNorm, softplus-on-load and the
    gate's autocast-dtype output must recompute exactly: outputs and every
    gradient equal bit for bit with checkpointing on and off."""
    hm = _hip()
    sd = _ref_state(EVAL12, 3)
    ids, dout = _inputs(EVAL12, 8, 64, 3)
    res = []
    for ck in (False, True):
        m = hm.Mamba(hm.MambaConfig(**EVAL12, grad_checkpoint=ck)).to(dev)
        m.load_state_dict(sd)
        m.train()
        with _amp(amp):
            y = m(ids)
            loss = (y.float() * dout).sum()
        loss.backward()
        res.append((y.detach(), _grads(m)))
    (y0, g0), (y1, g1) = res
    differ = [k for k in g0 if not torch.equal(g0[k], g1[k])]
    line = (f"grad checkpoint ({'fp32' if amp is None else str(amp)[6:] + ' autocast'}): y bitwise "
            f"{torch.equal(y0, y1)}, {len(g0) - len(differ)}/{len(g0)} gradients bitwise")
    record_property("parity", line)
    assert torch.equal(y0, y1) and not differ, line


def test_eval_mamba_fp16_autocast_matches_reference(gpu_lib, record_property):
    """The reference's training default: fp16 autocast with layer
    checkpointing.  Layer by layer within one fp16 ulp of the reference under
    the same autocast (its scan in fp32, as its kernel computes), and end to
    end no less accurate than it."""
    _teacher_forced(EVAL12, 8, 64, 3, "eval-mamba 12L fp16 autocast", record_property,
                    amp=torch.float16)
    _end_to_end(EVAL12, 8, 64, 3, "eval-mamba 12L fp16 autocast + grad checkpoint",
                record_property, amp=torch.float16, grad_checkpoint=True)


def test_eval_mamba_bf16_autocast_matches_reference(gpu_lib, record_property):
    """bf16 autocast, as the reference's trainers run with bf16=True
    (engine/train.py:112, :124-127; :523-525): layer by layer within one bf16
    ulp of the reference under the same autocast (its scan in fp32, as its
    kernel computes), and end to end no less accurate than it in aggregate,
    with layer checkpointing as in training."""
    _teacher_forced(EVAL12, 8, 64, 3, "eval-mamba 12L bf16 autocast", record_property,
                    amp=torch.bfloat16)
    _end_to_end(EVAL12, 8, 64, 3, "eval-mamba 12L bf16 autocast + grad checkpoint",
                record_property, amp=torch.bfloat16, grad_checkpoint=True)


def test_grad_checkpoint_recompute_is_bitwise_bf16(gpu_lib, record_property):
    """Layer checkpointing under bf16 autocast recomputes bit for bit."""
    test_grad_checkpoint_recompute_is_bitwise(gpu_lib, record_property, torch.bfloat16)


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


@pytest.mark.parametrize("bidir", [False, True])
def test_golden_model_fixture_same_device(gpu_lib, record_property, bidir):
    """The model fixtures' weights and ids (the reference's own seeded init,
    engine/mamba.py:503-532, whose rotational gates are half above 1: states
    that grow along the sequence) on one device, layer by layer: HIP against
    the oracle's restatement of the reference (pinned bit for bit to the
    fixture on the CPU, tests/test_oracle.py), float64 as the arbiter, the
    fp32 bars, with an N(0, 1) upstream gradient (the fixture's own loss,
    mean(norm_f(x)^2), is a near-cancellation whose gradients are rounding
    residues for any fp32 run).  This makes the cross-device fixture check
    above a parity check.  Layer by layer, because with growing states the
    first layer's gradients amplify whatever the later layers hand back: end
    to end its A gradients sit ~1e-6 from float64 for HIP and ~5e-8 for the
    reference by that sensitivity, while on the same inputs HIP's are closer
    to float64 than the reference's.  With growing states every fp32 run's
    gradients are several 1e-6 from float64, and how close the reference
    lands on a given tensor is partly chance: the exact-scan control (the
    same fp32 layer with its scan evaluated in float64, i.e. no scan error at
    all) lands up to 13x further than the reference on some.  So here the
    allowance is anchored at the larger of the reference's and the control's
    distances: HIP is within the bar of the reference, or no further from
    float64 than an error-free scan's fp32 layer plus the bar."""
    g = load_golden(f"model_bi{int(bidir)}")
    kw = dict(d_model=16, n_layer=2, d_state=12, n_track_state=4, mimo_p=2, vocab_size=64,
              bidirectional=bidir)
    sd = {k[3:]: v for k, v in g.items() if k.startswith("sd.")}
    B, L = g["ids"].shape
    _teacher_forced(kw, B, L, 19, f"model fixture bidir={int(bidir)} (reference init)",
                    record_property, sd=sd, ids=g["ids"], anchor_control=True)


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


def test_branch_scoring_cached_equals_full(gpu_lib):
    """score_branch (prime the board once, then O(1) steps through a line,
    engine/search_mamba.py:228-240) and evaluate_with_continuation (the board
    and every line through the full causal scan, :137-146) score the same
    lines: line values and continuation logits within 1e-5 of each other and
    of the float64 arbiter's, on the fixture's weights."""
    g = load_golden("search")
    sm, arb = _search_pair(g)
    sm.eval()
    arb.eval()
    board, moves = g["board"][0], g["moves"]
    with torch.no_grad():
        vals, conts = sm.evaluate_with_continuation(board.to(dev), moves.to(dev))
        v64, c64 = arb.evaluate_with_continuation(board, moves)
        _, cache = sm.prime_board(board.to(dev))
        for i in range(moves.shape[0]):
            q, cont = sm.score_branch(cache, [int(t) for t in moves[i]])
            assert abs(q - float(vals[i])) <= 1e-5 * max(1.0, abs(float(vals[i]))), i
            assert rel(cont, conts[i]) <= 1e-5, i
            assert abs(q - float(v64[i])) <= 1e-5 * max(1.0, abs(float(v64[i]))), i
            assert rel(cont, c64[i]) <= 1e-5, i
    assert rel(vals, v64) <= 1e-5 and rel(conts, c64) <= 1e-5


def test_block_ssm_entry_matches_reference(gpu_lib):
    """Mamba3Block.ssm (engine/mamba.py:303-316: projections, gates and the
    scan with the D skip), with and without the final state, against the
    oracle block's same composition; and Mamba.init_cache (:560-562)."""
    cfg = dict(d_model=32, n_layer=2, d_state=12, n_track_state=4, mimo_p=2, vocab_size=64)
    hip, ref = _pair(cfg, seed=21)
    hb, rb = hip.layers[1]["mixer"], ref.layers[1]["mixer"]
    gen = torch.Generator().manual_seed(22)
    u = torch.randn(3, 19, hb.config.d_inner, generator=gen).to(dev)
    with torch.no_grad():
        y = hb.ssm(u)
        y2, (h2, b2) = hb.ssm(u, return_state=True)
        delta, B, C = rb._ssm_proj(u)
        A_real, A_imag = rb._compute_A()
        yr = rb._scan(u, delta, A_real, A_imag, B, C)
        yr2, (hr, br) = rb._scan(u, delta, A_real, A_imag, B, C, return_state=True)
    assert rel(y, yr) <= 1e-5 and rel(y2, yr2) <= 1e-5
    assert rel(h2, hr) <= 1e-5 and rel(b2, br) <= 1e-5
    assert hip.init_cache(3, dev) == [None] * cfg["n_layer"]


def test_cpu_tensors_are_refused(gpu_lib):
    """No silent CPU path: the SSM core needs device tensors."""
    hm = _hip()
    m = hm.Mamba(hm.MambaConfig(d_model=16, n_layer=1, d_state=8, n_track_state=2, mimo_p=2,
                                vocab_size=64))
    with pytest.raises(RuntimeError, match="ROCm device"):
        m(torch.zeros(1, 4, dtype=torch.long))
