"""Throughput of the hot path on one MI355X: the trapezoidal selective scan
(bidirectional forward + analytic backward at the Eval-Mamba training shape)
and the batched O(1) step (4096 rollouts x 8 layers).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-step] [--no-long]
                    [--no-sweep] [--no-layer] [--no-mixer] [--no-rollout]

One "step" of the headline workload is one forward + backward of one
bidirectional scan layer over a batch of 256 boards x 64 tokens, d_inner 1536
(24 heads x 64), d_state 40 (32 rotational + 8 tanh-tracking), bf16-stored
inputs, fp32 arithmetic and fp32 gradients, through the product's autograd
entry (redpanda_amd.scan.hip_trapezoidal_scan).  Inputs are synthetic and
resident in HBM before the timed region.  Tokens are counted once per
forward + backward (both directions fused).

Besides the headline number the JSON line carries:
  roofline      the dominant kernel's algorithmic bytes / measured duration
                (HIP events on the launch stream) against 8 TB/s, and (the
                scan being VALU-bound) its vector-ALU issue rate against
                the VALU peak;
  kernels       the same for every kernel of the path;
  long_sequence tokens/s of a causal fwd + bwd at L=2048, d_state 72, with
                each kernel's HBM and VALU roofline (profiles/*_long.json);
  c1            the reference's CPU configuration (causal real-decay forward,
                B=8 L=64 D=256 N=16) on the GPU, beside its CPU baseline;
  step          rollout-steps/s of the fused step kernel over 8 layers;
  layer         tokens/s of a whole bidirectional Mamba3Block fwd + bwd, fused,
                beside the reference's layer with only its scan swapped;
  mixer_gate    the fused (y + 2 u D) silu(z) gate after the scan: kernel
                durations and bytes, and fwd + bwd against torch's ops;
  rollout_boundary  one ply's host transfers for 4096 rollouts through the
                pinned boundary (one upload, the top-k kernel, one download)
                beside the reference's per-rollout reads, sampled;
  cpu_baseline  the reference's CPU PyTorch path (the oracle's fp32
                restatement) on a bounded sample, on this host's cores;
                the step, layer, C1 and long-sequence blocks carry their
                own.
Only one GPU is used; --gpus above 1 exits with a message.
"""

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor figure
# vector-ALU issue peak: 256 CUs x 4 SIMDs x 2.4 GHz / 4 cycles per wave64
# fp32 instruction (16 lanes per SIMD), in wave-instructions per second
VALU_PEAK_IPS = 256 * 4 * 2.4e9 / 4

# Eval-Mamba training shape of one layer: batch 256, L=64 board tokens,
# d_model 768, expand 2 -> d_inner 1536 (24 heads x 64), d_state 32 complex
# plus 8 tanh-tracking channels.
SCAN_SHAPE = dict(B=256, L=64, D=1536, NR=32, NT=8)
# Search-Mamba batched step: 4096 rollouts, 8 causal layers, d_model 512
# (d_inner 1024 = 16 heads x 64), d_state 16 complex plus 4 tracking.
STEP_SHAPE = dict(R=4096, layers=8, D=1024, NR=16, NT=4)
# The step at the reference's default search-model core (SearchMambaConfig,
# engine/search_mamba.py:28-35: 12 layers, d_model 384 -> d_inner 768,
# d_state 32, no tracking states), 4096 rollouts.
STEP_SHAPE_DEFAULT = dict(R=4096, layers=12, D=768, NR=32, NT=0)
# The step kernel across state sizes (4096 rollouts, d_inner 1024, two
# layers alternating so that neither block stays in the caches): (rotational,
# tracking) splits from d_state 24 to 128, whole slots and pad states, the
# last slot's split fixed at compile time or decided at run time.
STEP_STATES = [(16, 8), (24, 4), (32, 0), (28, 8), (32, 8), (40, 4), (48, 0), (56, 4),
               (64, 0), (64, 8), (64, 16), (80, 4), (96, 0), (90, 14), (100, 8), (112, 0),
               (100, 16), (120, 8), (112, 16), (128, 0)]
# Long-sequence causal stress: batch 64, L=2048, d_inner 1024, d_state 64
# complex plus 8 tracking, fp32 inputs.
LONG_SHAPE = dict(B=64, L=2048, D=1024, NR=64, NT=8)
# Launch groups whose HBM bytes are reported as one figure: the scan
# backward with its two reductions (dB/dC tile partials, float64 parameter
# partials), and the mixer gate's backward with its dD reduction.  The names
# are the kernels' short names in the rocprofv3 counter summaries.
TRAFFIC_SUMS = {
    "scan_bwd_kernel+reductions": ("scan_bwd_kernel", "bwd_reduce_bc4", "bwd_reduce_par"),
    "mixer_out_bwd+reduction": ("mixer_out_bwd_vec_kernel", "mixer_out_reduce_kernel"),
}
# The reference's CPU configuration: one causal layer, batch 8, L=64, 8 heads
# x head_dim 32 (d_inner 256), d_state 16 real decay-only, forward only.
C1_SHAPE = dict(B=8, L=64, D=256, NR=16, NT=0)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-step", action="store_true", help="skip the step() workload")
    ap.add_argument("--no-long", action="store_true",
                    help="skip the long-sequence (L=2048) scan line")
    ap.add_argument("--no-layer", action="store_true", help="skip the whole-layer comparison")
    ap.add_argument("--no-mixer", action="store_true", help="skip the mixer-gate kernels")
    ap.add_argument("--no-rollout", action="store_true", help="skip the rollout-boundary ply")
    ap.add_argument("--no-step-states", action="store_true",
                    help="skip the step kernel across state sizes (d_state 24-128)")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the step sweep over rollout counts and the training-through-step "
                         "leg (their thousands of small launches swamp a kernel trace)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="approximate budget of the CPU baseline sample")
    ap.add_argument("--profile-pass", action="store_true",
                    help="counter pass: run each kernel of the path a few times at the bench "
                         "shapes plus one elementwise pass over 1 GiB (torch.neg: the reference "
                         "dispatch that scales FETCH_SIZE / WRITE_SIZE), then exit")
    ap.add_argument("--profile-pass-long", action="store_true",
                    help="the same counter pass for the long-sequence scan kernels only (their "
                         "dB / dC reduction shares its name with the Eval-shape one)")
    return ap.parse_args()


def scan_inputs(B, L, D, NR, NT, seed, device, dtype):
    """dt = softplus(N(-2, .5)); x, B, C ~ N(0, 1) with B/C RMS-normalised per
    token; Ar = -exp(U(0, 3)); Ai = U(-pi, pi); Tk = tanh(N(0, 1.5));
    dout ~ N(0, 1).  Generated on the CPU in fp32, stored in `dtype`."""
    import torch
    import torch.nn.functional as F
    gen = torch.Generator().manual_seed(seed)
    N = NR + NT
    u = torch.randn(B, L, D, generator=gen)
    dt = F.softplus(torch.randn(B, L, D, generator=gen) * 0.5 - 2.0)
    Bc = torch.randn(B, L, N, generator=gen)
    Cc = torch.randn(B, L, N, generator=gen)
    Bc = Bc / Bc.pow(2).mean(-1, keepdim=True).sqrt()
    Cc = Cc / Cc.pow(2).mean(-1, keepdim=True).sqrt()
    Ar = -torch.exp(torch.rand(D, NR, generator=gen) * 3.0)
    Ai = (torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi
    Tk = torch.tanh(torch.randn(D, NT, generator=gen) * 1.5)
    dy = torch.randn(B, L, D, generator=gen)
    st = [t.to(dtype).to(device) for t in (dt, u, Bc, Cc)]
    return dict(delta=st[0], u=st[1], Bc=st[2], Cc=st[3], Ar=Ar.to(device), Ai=Ai.to(device),
                Tk=Tk.to(device), dy=dy.to(device), N=N, NR=NR)


def scan_bytes(B, L, D, N, NR, NT, s_in, bidirectional):
    """Algorithmic HBM bytes of one forward and one backward launch.

    forward : read delta, u (s_in each per channel) and B, C (s_in per state),
              write y (fp32): T*(D*(2 s_in + 4) + 2 N s_in); parameters
              Ar, Ai (D x NR) and Tk (D x NT) in fp32.  Both directions of a
              bidirectional layer share one read of the inputs.
    backward: read delta, u, B, C (s_in) and dy (fp32), write d_delta, d_u,
              d_B, d_C (fp32): T*(D*(2 s_in + 4 + 8) + N*(2 s_in + 8));
              parameters read once and their gradients written once.
    """
    T = B * L
    par = (2 * D * NR + D * NT) * 4
    fwd = T * (D * (2 * s_in + 4) + 2 * N * s_in) + par
    bwd = T * (D * (2 * s_in + 12) + N * (2 * s_in + 8)) + 2 * par
    return fwd, bwd


def step_bytes(R, D, N, NR, NT):
    """Algorithmic HBM bytes of one fused step launch: read and write h and
    beta (fp32, 16 B per state element), read delta and u, write y (12 B per
    channel), read B and C (8 B per state), per rollout; plus parameters."""
    return R * (16 * D * N + 12 * D + 8 * N) + (2 * D * NR + D * NT + D) * 4


def step_bytes_rank1(R, D, N, NR, NT):
    """The same with beta in rank-1 rows [dt*u | B]: read and write h (8 B
    per state element) and the D + N floats of the row (8 B each), plus the
    per-channel and per-state inputs and y as above."""
    return R * (8 * D * N + 8 * (D + N) + 12 * D + 8 * N) + (2 * D * NR + D * NT + D) * 4


class EventTimer:
    """Average GPU duration of a launch sequence, with events on the stream
    the kernels are launched on (torch's current stream)."""

    def __init__(self, torch):
        self.torch = torch

    def time(self, fn, reps):
        torch = self.torch
        s = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            fn()
        e1.record(s)
        e1.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3  # seconds per call

    def time_cold(self, fn, reps, flush):
        """Average duration of single calls, each after `flush()` has
        displaced the last-level (Infinity) cache; the flush is outside the
        timed window."""
        torch = self.torch
        s = torch.cuda.current_stream()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
        for e0, e1 in ev:
            flush()
            e0.record(s)
            fn()
            e1.record(s)
        ev[-1][1].synchronize()
        return sum(e0.elapsed_time(e1) for e0, e1 in ev) / reps * 1e-3


def bench_scan(torch, args, dtype):
    from redpanda_amd import _lib
    from redpanda_amd.scan import hip_trapezoidal_scan, make_scan_args
    sh = SCAN_SHAPE
    B, L, D, NR, NT = sh["B"], sh["L"], sh["D"], sh["NR"], sh["NT"]
    N = NR + NT
    dev = torch.device("cuda:0")
    c = scan_inputs(B, L, D, NR, NT, 1003, dev, dtype)
    leaves = [c[k].requires_grad_(True) for k in ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk")]
    dy = c["dy"]

    def one_step():
        for t in leaves:
            t.grad = None
        y = hip_trapezoidal_scan(*leaves[:4], leaves[4], leaves[5], leaves[6], NR, N,
                                 bidirectional=True)
        y.backward(dy)

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tok_s = B * L * args.steps / elapsed

    # per-kernel durations through the C ABI with preallocated buffers
    lib = _lib.load()
    f32 = dict(dtype=torch.float32, device=dev)
    a = make_scan_args(c["delta"], c["u"], c["Bc"], c["Cc"], c["Ar"].detach(), c["Ai"].detach(),
                       c["Tk"].detach(), True)
    y = torch.empty((B, L, D), **f32)
    nck = lib.rp_scan_ckpt_bytes(ctypes.byref(a))
    ckpt = torch.empty(max(nck // 4, 1), **f32)
    out_ck = _lib.ScanFwdOut(y.data_ptr(), ckpt.data_ptr(), None, None)
    out_inf = _lib.ScanFwdOut(y.data_ptr(), None, None, None)
    g = [torch.empty((B, L, D), **f32), torch.empty((B, L, D), **f32),
         torch.empty((B, L, N), **f32), torch.empty((B, L, N), **f32),
         torch.empty((D, NR), **f32), torch.empty((D, NR), **f32), torch.empty((D, NT), **f32)]
    wb = lib.rp_scan_bwd_work_bytes(ctypes.byref(a))
    work = torch.empty(max(wb, 256), dtype=torch.uint8, device=dev)
    io = _lib.ScanBwdIO(dy=dy.data_ptr(), ckpt=ckpt.data_ptr(), d_delta=g[0].data_ptr(),
                        d_u=g[1].data_ptr(), d_Bc=g[2].data_ptr(), d_Cc=g[3].data_ptr(),
                        d_A_real=g[4].data_ptr(), d_A_imag=g[5].data_ptr(),
                        d_track=g[6].data_ptr(), work=work.data_ptr(), work_bytes=work.numel())
    stream = _lib.stream_of(dev)

    def fwd_train():
        _lib.check(lib.rp_scan_fwd(ctypes.byref(a), ctypes.byref(out_ck), stream), lib)

    def fwd_inf():
        _lib.check(lib.rp_scan_fwd(ctypes.byref(a), ctypes.byref(out_inf), stream), lib)

    def bwd():
        _lib.check(lib.rp_scan_bwd(ctypes.byref(a), ctypes.byref(io), stream), lib)

    timer = EventTimer(torch)
    reps = max(args.steps, 5)
    fwd_train()
    bwd()
    t_fwd = timer.time(fwd_train, reps)
    t_inf = timer.time(fwd_inf, reps)
    t_bwd = timer.time(bwd, reps)   # includes the two small reduction kernels
    s_in = 2 if dtype != torch.float32 else 4
    fb, bb = scan_bytes(B, L, D, N, NR, NT, s_in, True)
    kern = [
        {"kernel": "scan_fwd_kernel (bidirectional, checkpoints)", "seconds": t_fwd,
         "alg_bytes": fb, "GBps": fb / t_fwd / 1e9, "traffic_key": "scan_fwd_kernel"},
        {"kernel": "scan_fwd_kernel (bidirectional, inference)", "seconds": t_inf,
         "alg_bytes": fb, "GBps": fb / t_inf / 1e9, "traffic_key": None},
        {"kernel": "scan_bwd_kernel + reductions", "seconds": t_bwd,
         "alg_bytes": bb, "GBps": bb / t_bwd / 1e9, "traffic_key": "scan_bwd_kernel+reductions"},
    ]
    return dict(tok_s=tok_s, elapsed=elapsed, kernels=kern, t_fwd=t_fwd, t_bwd=t_bwd,
                t_inf=t_inf, fwd_bytes=fb, bwd_bytes=bb, T=B * L)


def bench_step(torch, args, layers=None, plies=32, keep=True, R=None, shape=None):
    from redpanda_amd import _lib
    sh = STEP_SHAPE if shape is None else shape
    R = sh["R"] if R is None else R
    D, NR, NT = sh["D"], sh["NR"], sh["NT"]
    layers = sh["layers"] if layers is None else layers
    N = NR + NT
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(1004)
    import torch.nn.functional as F
    lib = _lib.load()
    f32 = dict(dtype=torch.float32, device=dev)
    per_layer = []
    for _ in range(layers):
        dt = F.softplus(torch.randn(R, D, generator=gen) * 0.5 - 2.0).to(dev)
        u = torch.randn(R, D, generator=gen).to(dev)
        Bc = torch.randn(R, N, generator=gen)
        Cc = torch.randn(R, N, generator=gen)
        Bc = (Bc / Bc.pow(2).mean(-1, keepdim=True).sqrt()).to(dev)
        Cc = (Cc / Cc.pow(2).mean(-1, keepdim=True).sqrt()).to(dev)
        Ar = (-torch.exp(torch.rand(D, NR, generator=gen) * 3.0)).to(dev)
        Ai = ((torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi).to(dev)
        Tk = torch.tanh(torch.randn(D, NT, generator=gen) * 1.5).to(dev)
        Dk = torch.randn(D, generator=gen).to(dev)
        h = torch.zeros((R, D, N), **f32)
        beta = torch.zeros((R, D, N), **f32)
        y = torch.empty((R, D), **f32)
        a = _lib.StepArgs()
        a.R, a.D, a.N, a.NR, a.NT = R, D, N, NR, NT
        a.delta, a.delta_sr = dt.data_ptr(), D
        a.u, a.u_sr = u.data_ptr(), D
        a.Bc, a.Bc_sr = Bc.data_ptr(), N
        a.Cc, a.Cc_sr = Cc.data_ptr(), N
        a.h_in, a.beta_in = h.data_ptr(), beta.data_ptr()
        a.A_real, a.A_imag, a.track = Ar.data_ptr(), Ai.data_ptr(), Tk.data_ptr()
        a.Dskip = Dk.data_ptr()
        a.h_out, a.beta_out, a.y = h.data_ptr(), beta.data_ptr(), y.data_ptr()  # in place
        per_layer.append((a, (dt, u, Bc, Cc, Ar, Ai, Tk, Dk, h, beta, y)))
    stream = _lib.stream_of(dev)

    def ply():
        for a, _ in per_layer:
            _lib.check(lib.rp_step(ctypes.byref(a), stream), lib)

    # the same plies with the cache's beta in rank-1 rows (R, D + N): the
    # rows ping-pong between two buffers (a rank-1 step may not update them
    # in place); h is updated in place as above
    compact = []
    for a, keep_t in per_layer:
        bp = [torch.zeros((R, D + N), **f32), torch.zeros((R, D + N), **f32)]
        pair = []
        for i in range(2):
            ar = _lib.StepArgs.from_buffer_copy(a)
            ar.beta_rank1 = 1
            ar.beta_in, ar.beta_out = bp[i].data_ptr(), bp[1 - i].data_ptr()
            pair.append(ar)
        compact.append((pair, bp, keep_t))
    parity = [0]

    def ply_compact():
        i = parity[0]
        for pair, _, _ in compact:
            _lib.check(lib.rp_step(ctypes.byref(pair[i]), stream), lib)
        parity[0] = 1 - i

    for _ in range(max(args.warmup, 1)):
        ply()
    torch.cuda.synchronize()
    if not keep:  # counter pass: the warm-up dispatches are the sample
        for _ in range(max(args.warmup, 1)):
            ply_compact()
        torch.cuda.synchronize()
        return layers * max(args.warmup, 1)
    t0 = time.perf_counter()
    for _ in range(plies):
        ply()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timer = EventTimer(torch)
    t_launch = timer.time(ply, plies) / layers
    nb = step_bytes(R, D, N, NR, NT)
    # the first ply after a batch-1 cache is fanned out to the R rollouts:
    # every rollout reads the one shared state (no expand copies)
    a0, keep0 = per_layer[0]
    shared_h = torch.randn((1, D, N), generator=gen).to(dev)
    shared_b = torch.randn((1, D, N), generator=gen).to(dev)
    ab = _lib.StepArgs.from_buffer_copy(a0)
    ab.h_in, ab.beta_in, ab.broadcast_state = shared_h.data_ptr(), shared_b.data_ptr(), 1
    t_shared = timer.time(lambda: _lib.check(lib.rp_step(ctypes.byref(ab), stream), lib), 10)
    nb_shared = R * (8 * D * N + 12 * D + 8 * N) + 8 * D * N + (2 * D * NR + D * NT + D) * 4
    for _ in range(max(args.warmup, 1)):
        ply_compact()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(plies):
        ply_compact()
    torch.cuda.synchronize()
    elapsed_c = time.perf_counter() - t0
    t_launch_c = timer.time(ply_compact, plies) / layers
    nb_c = step_bytes_rank1(R, D, N, NR, NT)
    return dict(rollout_steps_s=R * plies / elapsed, plies=plies, elapsed=elapsed,
                t_launch=t_launch, bytes=nb, GBps=nb / t_launch / 1e9,
                t_shared=t_shared, bytes_shared=nb_shared, GBps_shared=nb_shared / t_shared / 1e9,
                rollout_steps_s_rank1=R * plies / elapsed_c, t_launch_rank1=t_launch_c,
                bytes_rank1=nb_c, GBps_rank1=nb_c / t_launch_c / 1e9)


# The whole search-model ply of the step workload: 8 causal layers, d_model
# 512, d_state 16 + 4, mimo_p 2 (the search model's), 4096 rollouts.
PLY_SHAPE = dict(R=4096, layers=8, d_model=512, d_state=20, n_track=4, mimo_p=2)


def bench_ply(torch, args, plies=8, R=None, graphs=False):
    """Whole plies through Mamba.step(input_embed=...) (projections on
    hipBLASLt, norms, the fused step kernel per layer), fp32, no autograd:
    the reference's cache format and rank-1 beta rows."""
    from redpanda_amd import mamba as hm
    sh = dict(PLY_SHAPE) if R is None else dict(PLY_SHAPE, R=R)
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = hm.MambaConfig(d_model=sh["d_model"], n_layer=sh["layers"], d_state=sh["d_state"],
                         n_track_state=sh["n_track"], mimo_p=sh["mimo_p"], vocab_size=64)
    model = hm.Mamba(cfg).to(dev).eval()
    gen = torch.Generator(device=dev).manual_seed(1011)
    emb = torch.randn(plies, sh["R"], sh["d_model"], generator=gen, device=dev)
    out = {}
    with torch.no_grad():
        for name, compact in (("full", False), ("rank1", True)):
            cache = None
            for k in range(2):  # warm-up plies build the cache
                _, cache = model.step(input_embed=emb[k], cache=cache, compact=compact)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for k in range(plies):
                _, cache = model.step(input_embed=emb[k], cache=cache, compact=compact)
            torch.cuda.synchronize()
            dt = (time.perf_counter() - t0) / plies
            out[name] = dict(s_per_ply=dt, rollout_steps_s=sh["R"] / dt)
            del cache
            if graphs:
                # the same plies replayed from HIP graphs (StepGraph)
                from redpanda_amd.step_graph import StepGraph
                sg = StepGraph(model, sh["R"], compact=compact, embed=True)
                for k in range(2):
                    sg(input_embed=emb[k])
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for k in range(plies):
                    sg(input_embed=emb[k])
                torch.cuda.synchronize()
                dt = (time.perf_counter() - t0) / plies
                out[name + "_graph"] = dict(s_per_ply=dt, rollout_steps_s=sh["R"] / dt)
                del sg
    return out


# Rollout counts of the step sweep: MARS advances survivors x simulations
# rollouts per ply (sim_budget 64 by default), and its diagnostics sweep the
# batched step over 1 to 512 (engine/mars_search.py:59,
# engine/mars_diagnostics.py:169-227); 4096 is the headline workload.
STEP_SWEEP_R = (1, 8, 32, 128, 512, 4096)


def bench_step_sweep(torch, args):
    """The step kernel (full and rank-1 caches, 8 layers per ply) and the
    whole ply through Mamba.step at each rollout count of STEP_SWEEP_R."""
    rows = []
    for R in STEP_SWEEP_R:
        st = bench_step(torch, args, plies=16, R=R)
        ply = bench_ply(torch, args, plies=8, R=R, graphs=True)
        rows.append({
            "R": R,
            "step_kernel": {"avg_launch_s": st["t_launch"], "GBps": st["GBps"],
                            "frac": st["GBps"] / HBM_PEAK_GBS,
                            "rollout_steps_s": R / (st["t_launch"] * STEP_SHAPE["layers"])},
            "step_kernel_rank1": {"avg_launch_s": st["t_launch_rank1"], "GBps": st["GBps_rank1"],
                                  "frac": st["GBps_rank1"] / HBM_PEAK_GBS,
                                  "rollout_steps_s":
                                      R / (st["t_launch_rank1"] * STEP_SHAPE["layers"])},
            "whole_ply": {"s_per_ply": ply["full"]["s_per_ply"],
                          "rollout_steps_s": ply["full"]["rollout_steps_s"]},
            "whole_ply_rank1": {"s_per_ply": ply["rank1"]["s_per_ply"],
                                "rollout_steps_s": ply["rank1"]["rollout_steps_s"]},
            "whole_ply_graph": {"s_per_ply": ply["full_graph"]["s_per_ply"],
                                "rollout_steps_s": ply["full_graph"]["rollout_steps_s"]},
            "whole_ply_rank1_graph": {"s_per_ply": ply["rank1_graph"]["s_per_ply"],
                                      "rollout_steps_s": ply["rank1_graph"]["rollout_steps_s"]},
        })
        print(f"[bench] step sweep R={R}: kernel {st['t_launch'] * 1e6:.1f} us/launch "
              f"(rank-1 {st['t_launch_rank1'] * 1e6:.1f}); whole ply "
              f"{ply['full']['s_per_ply'] * 1e3:.3f} ms (rank-1 "
              f"{ply['rank1']['s_per_ply'] * 1e3:.3f}); from graphs "
              f"{ply['full_graph']['s_per_ply'] * 1e3:.3f} ms (rank-1 "
              f"{ply['rank1_graph']['s_per_ply'] * 1e3:.3f})", file=sys.stderr, flush=True)
    return rows


# Training through step() (SearchMamba.dynamics_rollout, the DynamicsTrainer's
# forward, engine/search_mamba.py:252-273, engine/train.py:558): the search
# model of the step workload (8 causal layers, d_model 512, d_state 16 + 4,
# mimo_p 2), the trainer's batch of 64 boards, a 64-token board prefix and
# 8 move plies (max_pv, engine/train.py:491).
DYN_SHAPE = dict(B=64, L_board=64, T=8, d_model=512, layers=8, d_state=20, n_track=4,
                 mimo_p=2, vocab=8192, eval_dim=512)


def bench_dynamics(torch, args, reps=10):
    """Forward + backward of SearchMamba.dynamics_rollout (prime_cache over the
    board, then T differentiable steps with the value, continuation and
    consistency heads), fp32 and under bf16 autocast; also the prime_cache
    part alone, so that the T steps' share is the difference."""
    from redpanda_amd.search_mamba import SearchMamba, SearchMambaConfig
    sh = DYN_SHAPE
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = SearchMambaConfig(d_model=sh["d_model"], n_layer=sh["layers"], d_state=sh["d_state"],
                            n_track_state=sh["n_track"], mimo_p=sh["mimo_p"],
                            vocab_size=sh["vocab"])
    model = SearchMamba(cfg, vocab_size=sh["vocab"], eval_dim=sh["eval_dim"]).to(dev).train()
    gen = torch.Generator(device=dev).manual_seed(1012)
    board = torch.randint(0, sh["vocab"], (sh["B"], sh["L_board"]), generator=gen, device=dev)
    moves = torch.randint(0, sh["vocab"], (sh["B"], sh["T"]), generator=gen, device=dev)

    def full():
        v, c, f = model.dynamics_rollout(board, moves)
        (v.float().sum() + c.float().mean() + f.float().pow(2).mean()).backward()

    def prime():
        fin, _ = model.backbone.prime_cache(board)
        fin.float().pow(2).mean().backward()

    timer = EventTimer(torch)
    out = {}
    for name, amp in (("fp32", None), ("bf16_autocast", torch.bfloat16)):
        ctx = (lambda: torch.autocast("cuda", dtype=amp)) if amp else None
        res = {}
        for part, fn in (("train_step", full), ("prime_only", prime)):
            def run(fn=fn):
                model.zero_grad(set_to_none=True)
                if ctx is None:
                    fn()
                else:
                    with ctx():
                        fn()
            for _ in range(3):
                run()
            torch.cuda.synchronize()
            res[part + "_s"] = timer.time(run, reps)
        res["steps_share_s"] = res["train_step_s"] - res["prime_only_s"]
        res["boards_s"] = sh["B"] / res["train_step_s"]
        out[name] = res
    # the fp32 forward + backward captured with torch.cuda.make_graphed_callables
    # (replayed from HIP graphs: the host's launch work taken out)

    class Rollout(torch.nn.Module):
        def __init__(self, m):
            super().__init__()
            self.m = m

        def forward(self, b, mv):
            return self.m.dynamics_rollout(b, mv)

    graphed = torch.cuda.make_graphed_callables(Rollout(model), (board, moves),
                                                allow_unused_input=True)

    def run_graphed():
        model.zero_grad(set_to_none=True)
        v, c, f = graphed(board, moves)
        (v.float().sum() + c.float().mean() + f.float().pow(2).mean()).backward()

    for _ in range(3):
        run_graphed()
    torch.cuda.synchronize()
    out["fp32_graphed"] = {"train_step_s": timer.time(run_graphed, reps)}
    out["fp32_graphed"]["boards_s"] = sh["B"] / out["fp32_graphed"]["train_step_s"]
    return out


def practical_hbm_peak(torch):
    """GB/s of a 1 GiB device-to-device copy (read + write), best of 5."""
    dev = torch.device("cuda:0")
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    best = None
    for _ in range(5):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(src)
        e1.record()
        e1.synchronize()
        t = e0.elapsed_time(e1) * 1e-3
        best = t if best is None else min(best, t)
    return 2 * src.numel() * 4 / best / 1e9


def mixer_inputs(torch, dev, seed):
    """The mixer gate's operands at the scan shape: y fp32 from the scan,
    u bf16, z bf16 as the second half of a (B, L, 2 d_inner) in_proj output."""
    B, L, D = SCAN_SHAPE["B"], SCAN_SHAPE["L"], SCAN_SHAPE["D"]
    gen = torch.Generator(device=dev).manual_seed(seed)
    y = torch.randn(B, L, D, generator=gen, device=dev)
    u = torch.randn(B, L, D, generator=gen, device=dev).to(torch.bfloat16)
    z = (torch.randn(B, L, 2 * D, generator=gen, device=dev) * 2).to(torch.bfloat16)
    z = z.chunk(2, dim=-1)[1]
    Dp = torch.randn(D, generator=gen, device=dev)
    dout = torch.randn(B, L, D, generator=gen, device=dev)
    return y, u, z, Dp, dout


def mixer_bytes(n):
    """Algorithmic HBM bytes of the gate over n = B*L*d_inner elements
    (bf16 u and z, fp32 y, out, dout, dy): forward reads y, u, z and writes
    out; backward reads y, u, z, dout and writes dy, du, dz."""
    return n * (4 + 2 + 2 + 4), n * (4 + 2 + 2 + 4 + 4 + 2 + 2)


def bench_mixer(torch, args):
    """The fused output gate (y + 2 u D) silu(z) of a bidirectional layer:
    kernel durations through the C ABI, and fwd + bwd through autograd
    against the same ops run by torch (what the reference executes)."""
    import torch.nn.functional as F
    from redpanda_amd import _lib
    from redpanda_amd.mixer import hip_mixer_out, make_mixer_args
    dev = torch.device("cuda:0")
    y, u, z, Dp, dout = mixer_inputs(torch, dev, 1007)
    lib = _lib.load()
    out = torch.empty_like(y)
    a = make_mixer_args(y, u, z, Dp, 2, out)
    dy = torch.empty_like(y)
    du = torch.empty_like(u)
    dz = torch.empty(u.shape, dtype=z.dtype, device=dev)
    dD = torch.empty_like(Dp)
    work = torch.empty(max(lib.rp_mixer_out_work_bytes(ctypes.byref(a)), 256),
                       dtype=torch.uint8, device=dev)
    g = _lib.MixerOutGrad(dout=dout.data_ptr(), dy=dy.data_ptr(), du=du.data_ptr(),
                          dz=dz.data_ptr(), dD=dD.data_ptr(), work=work.data_ptr(),
                          work_bytes=work.numel())
    stream = _lib.stream_of(dev)

    def fwd():
        _lib.check(lib.rp_mixer_out_fwd(ctypes.byref(a), stream), lib)

    def bwd():
        _lib.check(lib.rp_mixer_out_bwd(ctypes.byref(a), ctypes.byref(g), stream), lib)

    leaves = [t.detach().clone().requires_grad_() for t in (y, u, z, Dp)]

    def fused_autograd():
        for t in leaves:
            t.grad = None
        hip_mixer_out(*leaves, 2).backward(dout)

    def torch_autograd():
        for t in leaves:
            t.grad = None
        yv, uv, zv, Dv = leaves
        ((yv + uv * Dv + uv * Dv) * F.silu(zv)).backward(dout)

    for fn in (fwd, bwd, fused_autograd, torch_autograd):
        fn()
    torch.cuda.synchronize()
    timer = EventTimer(torch)
    reps = max(args.steps, 10)
    # the operands (about 300 MB) would otherwise sit partly in the 256 MB
    # Infinity Cache across back-to-back calls; in a layer they arrive cold.
    # The flush reads 512 MB (a write would leave dirty lines whose
    # write-back the timed kernel would pay for)
    scratch = torch.ones(1 << 27, dtype=torch.float32, device=dev)
    flush = lambda: torch.sum(scratch)
    t_f = timer.time_cold(fwd, reps, flush)
    t_b = timer.time_cold(bwd, reps, flush)
    t_f_warm = timer.time(fwd, reps)
    t_b_warm = timer.time(bwd, reps)
    del scratch
    t_fused = timer.time(fused_autograd, reps)
    t_torch = timer.time(torch_autograd, reps)
    fb, bb = mixer_bytes(y.numel())
    return dict(t_fwd=t_f, t_bwd=t_b, fwd_bytes=fb, bwd_bytes=bb, t_fused=t_fused,
                t_torch=t_torch, t_fwd_warm=t_f_warm, t_bwd_warm=t_b_warm)


# One ply of 4096 lockstep rollouts: the Search-Mamba continuation head's
# logits over the 8192-token move vocabulary, the top-8 candidates the
# policy-guided rollout walks (engine/mars_search.py:66, policy_top_k=8), and
# about 40 legal moves per position for the fastchess path.
ROLLOUT_SHAPE = dict(R=4096, V=8192, k=8, legal=40)


def bench_rollout(torch, args, plies=20, sample=256):
    """Host-inclusive time of one ply's transfers: redpanda_amd.rollout's
    pinned boundary against the reference's pattern (a pageable token upload,
    each rollout's continuation row read with .cpu() and its top-k taken in
    numpy, the values read with .cpu().tolist()), the latter timed on
    `sample` rollouts and scaled to R."""
    import numpy as np
    from redpanda_amd import _lib
    from redpanda_amd.rollout import PlyBoundary
    sh = ROLLOUT_SHAPE
    R, V, k, M = sh["R"], sh["V"], sh["k"], sh["legal"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(11)
    cont = torch.randn(R, V, device=dev, generator=g)
    vals = torch.tanh(torch.randn(R, 1, device=dev, generator=g))
    rng = np.random.default_rng(11)
    tokens = rng.integers(0, V, R).tolist()
    legal = rng.integers(0, V, (R, M))
    pb = PlyBoundary(R, top_k=k, device=dev, max_legal=64)
    out = torch.empty((R, 2 * k + 1), dtype=torch.float32, device=dev)
    for _ in range(3):
        pb.push_tokens(tokens)
        pb.pull(vals, cont)
        pb.pull_legal(cont, legal)
    torch.cuda.synchronize()
    # the kernel alone: prebuilt arguments, so the launches outpace the GPU
    lib = _lib.load()
    a = _lib.PlyTopkArgs(R=R, V=V, k=k, dtype_logits=_lib.RP_F32, logits=cont.data_ptr(),
                         logits_sr=V, values=vals.data_ptr(), out=out.data_ptr(), out_sr=2 * k + 1)
    stream = _lib.stream_of(dev)
    t_kernel = EventTimer(torch).time(lambda: lib.rp_ply_topk(ctypes.byref(a), stream), 50)
    t0 = time.perf_counter()
    for _ in range(plies):
        pb.push_tokens(tokens)
        pb.pull(vals, cont)
    t_ours = (time.perf_counter() - t0) / plies
    t0 = time.perf_counter()
    for _ in range(plies):
        pb.pull_legal(cont, legal)
    t_legal = (time.perf_counter() - t0) / plies

    # the reference's per-ply pattern (engine/mars_search.py:262-265, :442-446, :475)
    def ref_fixed():
        tok_t = torch.tensor(tokens, dtype=torch.long, device=dev)
        return tok_t, vals.detach().cpu().tolist()

    def ref_rows(n):
        for i in range(n):
            ln = cont[i].float().cpu().numpy()
            top = np.argpartition(ln, -k)[-k:]
            top = top[np.argsort(ln[top])[::-1]]

    def ref_legal_rows(n):
        for i in range(n):
            idx = torch.from_numpy(legal[i]).to(dev)
            cont[i][idx].float().cpu().numpy()

    ref_fixed(), ref_rows(8), ref_legal_rows(8)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        ref_fixed()
    t_fixed = (time.perf_counter() - t0) / 5
    t0 = time.perf_counter()
    ref_rows(sample)
    t_rows = (time.perf_counter() - t0) / sample
    t0 = time.perf_counter()
    ref_legal_rows(sample)
    t_lrows = (time.perf_counter() - t0) / sample
    return dict(t_kernel=t_kernel, kernel_bytes=R * V * 4 + R * 4 + R * (2 * k + 1) * 4,
                t_ours=t_ours, t_legal=t_legal, t_ref=t_fixed + R * t_rows,
                t_ref_legal=R * t_lrows, sample=sample)


# One Eval-Mamba layer: d_model 768 (d_inner 1536), d_state 32 + 8, mimo_p 4,
# bidirectional, at the scan shape's batch and length, under bf16 autocast.
LAYER_SHAPE = dict(B=256, L=64, d_model=768, d_state=40, n_track=8)


def bench_layer(torch, args):
    """Forward + backward of one bidirectional Mamba3Block: the fused module,
    against the reference's own op sequence for the layer (engine/mamba.py:
    231-267, 284-301, 318-350) with only the scan call swapped for the HIP
    scan, i.e. the one-file drop-in of engine/triton_scan.py."""
    import torch.nn.functional as F
    from redpanda_amd import mamba as hm
    from redpanda_amd.scan import hip_trapezoidal_scan
    sh = LAYER_SHAPE
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = hm.MambaConfig(d_model=sh["d_model"], n_layer=1, d_state=sh["d_state"],
                         n_track_state=sh["n_track"], bidirectional=True)
    blk = hm.Mamba3Block(cfg).to(dev)
    gen = torch.Generator(device=dev).manual_seed(1009)
    x = torch.randn(sh["B"], sh["L"], sh["d_model"], generator=gen, device=dev)
    x.requires_grad_(True)

    def scan_only_dropin(xin):
        # the reference's block with triton_trapezoidal_scan -> HIP scan
        xb, z = blk.in_proj(xin).chunk(2, dim=-1)
        xb = F.silu(xb)
        delta, B, C = blk._ssm_proj(xb)
        Ar, Ai = blk._compute_A()
        track = blk._track_gate()

        def scan(u, d, b, c):
            return hip_trapezoidal_scan(d, u, b.sum(-1), c.sum(-1), Ar, Ai, track,
                                        cfg.n_rot_state, cfg.d_state) + u * blk.D

        y = scan(xb, delta, B, C)
        y = y + scan(xb.flip(1), delta.flip(1), B.flip(1), C.flip(1)).flip(1)
        return blk.out_proj(y * F.silu(z))

    def run(fn):
        def step():
            x.grad = None
            blk.zero_grad(set_to_none=True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                out = fn(x)
            out.float().square().mean().backward()
        return step

    fused, dropin = run(blk), run(scan_only_dropin)
    for fn in (fused, dropin):
        for _ in range(max(args.warmup, 2)):
            fn()
    torch.cuda.synchronize()
    timer = EventTimer(torch)
    reps = max(5, min(args.steps, 10))
    t_fused = min(timer.time(fused, reps) for _ in range(2))
    t_dropin = min(timer.time(dropin, reps) for _ in range(2))
    T = sh["B"] * sh["L"]
    return dict(t_fused=t_fused, t_dropin=t_dropin, tok_fused=T / t_fused, tok_dropin=T / t_dropin)


def long_setup(torch):
    """Device inputs and preallocated buffers of the long-sequence shape
    (generated on the device), and fwd() / bwd() calls through the C ABI."""
    from redpanda_amd import _lib
    from redpanda_amd.scan import make_scan_args
    import torch.nn.functional as F
    sh = LONG_SHAPE
    B, L, D, NR, NT = sh["B"], sh["L"], sh["D"], sh["NR"], sh["NT"]
    N = NR + NT
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(1005)
    u = torch.randn(B, L, D, generator=gen, device=dev)
    dt = F.softplus(torch.randn(B, L, D, generator=gen, device=dev) * 0.5 - 2.0)
    Bc = torch.randn(B, L, N, generator=gen, device=dev)
    Cc = torch.randn(B, L, N, generator=gen, device=dev)
    Bc = Bc / Bc.pow(2).mean(-1, keepdim=True).sqrt()
    Cc = Cc / Cc.pow(2).mean(-1, keepdim=True).sqrt()
    Ar = -torch.exp(torch.rand(D, NR, generator=gen, device=dev) * 3.0)
    Ai = (torch.rand(D, NR, generator=gen, device=dev) * 2 - 1) * math.pi
    Tk = torch.tanh(torch.randn(D, NT, generator=gen, device=dev) * 1.5)
    dy = torch.randn(B, L, D, generator=gen, device=dev)
    lib = _lib.load()
    f32 = dict(dtype=torch.float32, device=dev)
    a = make_scan_args(dt, u, Bc, Cc, Ar, Ai, Tk, False)
    y = torch.empty((B, L, D), **f32)
    ckpt = torch.empty(max(lib.rp_scan_ckpt_bytes(ctypes.byref(a)) // 4, 1), **f32)
    g = [torch.empty((B, L, D), **f32), torch.empty((B, L, D), **f32),
         torch.empty((B, L, N), **f32), torch.empty((B, L, N), **f32),
         torch.empty((D, NR), **f32), torch.empty((D, NR), **f32), torch.empty((D, NT), **f32)]
    work = torch.empty(max(lib.rp_scan_bwd_work_bytes(ctypes.byref(a)), 256), dtype=torch.uint8,
                       device=dev)
    out = _lib.ScanFwdOut(y.data_ptr(), ckpt.data_ptr(), None, None)
    io = _lib.ScanBwdIO(dy=dy.data_ptr(), ckpt=ckpt.data_ptr(), d_delta=g[0].data_ptr(),
                        d_u=g[1].data_ptr(), d_Bc=g[2].data_ptr(), d_Cc=g[3].data_ptr(),
                        d_A_real=g[4].data_ptr(), d_A_imag=g[5].data_ptr(),
                        d_track=g[6].data_ptr(), work=work.data_ptr(), work_bytes=work.numel())
    stream = _lib.stream_of(dev)
    keep = (u, dt, Bc, Cc, Ar, Ai, Tk, dy, y, ckpt, g, work, a, out, io)

    def fwd():
        _lib.check(lib.rp_scan_fwd(ctypes.byref(a), ctypes.byref(out), stream), lib)

    def bwd():
        _lib.check(lib.rp_scan_bwd(ctypes.byref(a), ctypes.byref(io), stream), lib)

    return fwd, bwd, keep


def bench_long(torch, args):
    """Causal fwd + bwd at the long-sequence shape, through the C ABI with
    preallocated buffers (inputs generated on the device)."""
    sh = LONG_SHAPE
    B, L, D, NR, NT = sh["B"], sh["L"], sh["D"], sh["NR"], sh["NT"]
    fwd, bwd, keep = long_setup(torch)
    fwd()
    bwd()
    torch.cuda.synchronize()
    timer = EventTimer(torch)
    reps = max(2, min(args.steps, 5))
    t_f = timer.time(fwd, reps)
    t_b = timer.time(bwd, reps)
    fb, bb = scan_bytes(B, L, D, NR + NT, NR, NT, 4, False)
    del keep
    return dict(tok_s=B * L / (t_f + t_b), t_fwd=t_f, t_bwd=t_b, fwd_bytes=fb, bwd_bytes=bb)


def bench_c1(torch, args):
    """The reference's CPU configuration on the GPU: one causal real-decay
    scan forward (fp32 inputs, no checkpoints), per launch."""
    from redpanda_amd import _lib
    from redpanda_amd.scan import make_scan_args
    sh = C1_SHAPE
    B, L, D, NR = sh["B"], sh["L"], sh["D"], sh["NR"]
    c = c1_inputs(torch, "cuda:0")
    lib = _lib.load()
    a = make_scan_args(c["delta"], c["u"], c["Bc"], c["Cc"], c["Ar"], None, None, False)
    y = torch.empty((B, L, D), dtype=torch.float32, device="cuda:0")
    out = _lib.ScanFwdOut(y.data_ptr(), None, None, None)
    stream = _lib.stream_of(torch.device("cuda:0"))

    def fwd():
        _lib.check(lib.rp_scan_fwd(ctypes.byref(a), ctypes.byref(out), stream), lib)

    for _ in range(3):
        fwd()
    torch.cuda.synchronize()
    t = EventTimer(torch).time(fwd, max(20, args.steps))
    fb, _ = scan_bytes(B, L, D, NR, NR, 0, 4, False)
    return dict(tok_s=B * L / t, t_fwd=t, fwd_bytes=fb)


def c1_inputs(torch, device):
    """C1's inputs: x ~ N(0,1); dt = softplus(N(-2,0.5)); A = -exp(U(log 1,
    log 16)); B and C ~ N(0,1), RMS-normalised per token (fp32)."""
    import torch.nn.functional as F
    sh = C1_SHAPE
    B, L, D, NR = sh["B"], sh["L"], sh["D"], sh["NR"]
    gen = torch.Generator().manual_seed(1001)
    u = torch.randn(B, L, D, generator=gen)
    dt = F.softplus(torch.randn(B, L, D, generator=gen) * 0.5 - 2.0)
    Bc = torch.randn(B, L, NR, generator=gen)
    Cc = torch.randn(B, L, NR, generator=gen)
    Bc = Bc / Bc.pow(2).mean(-1, keepdim=True).sqrt()
    Cc = Cc / Cc.pow(2).mean(-1, keepdim=True).sqrt()
    Ar = -torch.exp(torch.rand(D, NR, generator=gen) * math.log(16.0))
    return {k: v.to(device) for k, v in dict(delta=dt, u=u, Bc=Bc, Cc=Cc, Ar=Ar).items()}


def measured_valu(name="valu.json"):
    """VALU wave-instructions per launch from a committed counter summary
    (profiles/valu.json, written by `python -m redpanda_amd.profiling valu`
    from an SQ_INSTS_VALU pass over `bench.py --profile-pass`;
    profiles/valu_long.json from `--profile-pass-long`), or {}."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as fh:
            k = json.load(fh)["kernels"]
    except (OSError, KeyError, ValueError):
        return {}
    return {name: v.get("SQ_INSTS_VALU") for name, v in k.items()}


def valu_roofline(instr, seconds):
    if not instr:
        return None
    ips = instr / seconds
    return {"bound": "valu", "achieved": ips, "peak": VALU_PEAK_IPS,
            "unit": "wave-instructions/s", "frac": ips / VALU_PEAK_IPS,
            "instructions_per_launch": instr}


def measured_traffic(name="traffic.json"):
    """HBM bytes per launch from a committed counter summary
    (profiles/traffic.json, written by `python -m redpanda_amd.profiling
    traffic` from FETCH_SIZE / WRITE_SIZE passes over `bench.py
    --profile-pass`; profiles/traffic_long.json from `--profile-pass-long`),
    or {} when there is none."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as fh:
            k = json.load(fh)["kernels"]
    except (OSError, KeyError, ValueError):
        return {}
    out = {name: v["bytes"] for name, v in k.items()}
    for total, parts in TRAFFIC_SUMS.items():
        if parts[0] in k:
            # every part must be in the summary: a renamed kernel would
            # otherwise drop its bytes from the total without a trace
            missing = [n for n in parts if n not in k]
            if missing:
                raise KeyError(f"profiles/{name} lacks {missing} for {total}")
            out[total] = sum(k[n]["bytes"] for n in parts)
    return out


def profile_pass(torch):
    """A few dispatches of every kernel at the bench shapes, for counter runs
    (rocprofv3 --pmc collects per dispatch), then one 1 GiB device copy."""
    from redpanda_amd import _lib
    from redpanda_amd.scan import make_scan_args
    sh = SCAN_SHAPE
    B, L, D, NR, NT = sh["B"], sh["L"], sh["D"], sh["NR"], sh["NT"]
    N = NR + NT
    dev = torch.device("cuda:0")
    c = scan_inputs(B, L, D, NR, NT, 1003, dev, torch.bfloat16)
    lib = _lib.load()
    f32 = dict(dtype=torch.float32, device=dev)
    a = make_scan_args(c["delta"], c["u"], c["Bc"], c["Cc"], c["Ar"], c["Ai"], c["Tk"], True)
    y = torch.empty((B, L, D), **f32)
    ckpt = torch.empty(max(lib.rp_scan_ckpt_bytes(ctypes.byref(a)) // 4, 1), **f32)
    g = [torch.empty((B, L, D), **f32), torch.empty((B, L, D), **f32),
         torch.empty((B, L, N), **f32), torch.empty((B, L, N), **f32),
         torch.empty((D, NR), **f32), torch.empty((D, NR), **f32), torch.empty((D, NT), **f32)]
    work = torch.empty(max(lib.rp_scan_bwd_work_bytes(ctypes.byref(a)), 256), dtype=torch.uint8,
                       device=dev)
    out = _lib.ScanFwdOut(y.data_ptr(), ckpt.data_ptr(), None, None)
    io = _lib.ScanBwdIO(dy=c["dy"].data_ptr(), ckpt=ckpt.data_ptr(), d_delta=g[0].data_ptr(),
                        d_u=g[1].data_ptr(), d_Bc=g[2].data_ptr(), d_Cc=g[3].data_ptr(),
                        d_A_real=g[4].data_ptr(), d_A_imag=g[5].data_ptr(),
                        d_track=g[6].data_ptr(), work=work.data_ptr(), work_bytes=work.numel())
    stream = _lib.stream_of(dev)
    for _ in range(3):
        _lib.check(lib.rp_scan_fwd(ctypes.byref(a), ctypes.byref(out), stream), lib)
        _lib.check(lib.rp_scan_bwd(ctypes.byref(a), ctypes.byref(io), stream), lib)
    torch.cuda.synchronize()
    del y, ckpt, g, work, c
    args = argparse.Namespace(warmup=3)
    step_layers = bench_step(torch, args, layers=1, plies=3, keep=False)
    # the mixer gate, three dispatches each way
    from redpanda_amd.mixer import make_mixer_args
    my, mu, mz, mD, mdout = mixer_inputs(torch, dev, 1007)
    mout = torch.empty_like(my)
    ma = make_mixer_args(my, mu, mz, mD, 2, mout)
    mg_t = [torch.empty_like(my), torch.empty_like(mu), torch.empty_like(mu),
            torch.empty_like(mD),
            torch.empty(max(lib.rp_mixer_out_work_bytes(ctypes.byref(ma)), 256),
                        dtype=torch.uint8, device=dev)]
    mg = _lib.MixerOutGrad(dout=mdout.data_ptr(), dy=mg_t[0].data_ptr(), du=mg_t[1].data_ptr(),
                           dz=mg_t[2].data_ptr(), dD=mg_t[3].data_ptr(),
                           work=mg_t[4].data_ptr(), work_bytes=mg_t[4].numel())
    for _ in range(3):
        _lib.check(lib.rp_mixer_out_fwd(ctypes.byref(ma), stream), lib)
        _lib.check(lib.rp_mixer_out_bwd(ctypes.byref(ma), ctypes.byref(mg), stream), lib)
    torch.cuda.synchronize()
    del my, mu, mz, mD, mdout, mout, mg_t
    # calibration: one elementwise dispatch that reads 1 GiB and writes 1 GiB
    # (a device-to-device copy_ is split into several copy dispatches)
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    # the BCNorm prologue at the layer shape (bf16 projections), three each way
    from redpanda_amd.bcnorm import make_bcnorm_args
    T, Nn, P = SCAN_SHAPE["B"] * SCAN_SHAPE["L"], SCAN_SHAPE["NR"] + SCAN_SHAPE["NT"], 4
    xd = torch.randn(T, 48 + 2 * Nn * P, device=dev).to(torch.bfloat16)
    Bx, Cx = xd[:, 48:48 + Nn * P], xd[:, 48 + Nn * P:]
    wB, wC = torch.ones(Nn * P, device=dev), torch.ones(Nn * P, device=dev)
    bo = [torch.empty(T, Nn, device=dev), torch.empty(T, Nn, device=dev)]
    ba = make_bcnorm_args(Bx, Cx, wB, wC, Nn, P, 1e-5, True, bo[0], bo[1])
    bg_t = [torch.randn(T, Nn, device=dev), torch.randn(T, Nn, device=dev),
            torch.empty(T, Nn * P, dtype=torch.bfloat16, device=dev),
            torch.empty(T, Nn * P, dtype=torch.bfloat16, device=dev),
            torch.empty(Nn * P, device=dev), torch.empty(Nn * P, device=dev),
            torch.empty(max(lib.rp_bcnorm_work_bytes(ctypes.byref(ba)), 256), dtype=torch.uint8,
                        device=dev)]
    bgr = _lib.BcNormGrad(*(t.data_ptr() for t in bg_t[:6]), bg_t[6].data_ptr(), bg_t[6].numel())
    for _ in range(3):
        _lib.check(lib.rp_bcnorm_fwd(ctypes.byref(ba), stream), lib)
        _lib.check(lib.rp_bcnorm_bwd(ctypes.byref(ba), ctypes.byref(bgr), stream), lib)
    torch.cuda.synchronize()
    del xd, bo, bg_t
    # the rollout ply's top-k at the rollout shape, three dispatches
    sh = ROLLOUT_SHAPE
    logits = torch.randn(sh["R"], sh["V"], device=dev)
    vals = torch.randn(sh["R"], device=dev)
    pk = torch.empty(sh["R"], 2 * sh["k"] + 1, device=dev)
    pa = _lib.PlyTopkArgs(R=sh["R"], V=sh["V"], k=sh["k"], dtype_logits=_lib.RP_F32,
                          logits=logits.data_ptr(), logits_sr=sh["V"], values=vals.data_ptr(),
                          out=pk.data_ptr(), out_sr=2 * sh["k"] + 1)
    for _ in range(3):
        _lib.check(lib.rp_ply_topk(ctypes.byref(pa), stream), lib)
    torch.cuda.synchronize()
    del logits, vals, pk
    print(f"[bench] profile pass done: scan fwd/bwd x3, step x{step_layers}, "
          f"calibration neg {src.numel() * 4} bytes each way", file=sys.stderr, flush=True)


def profile_pass_long(torch):
    """The long-sequence scan kernels, three dispatches each way, then the
    1 GiB calibration dispatch, for counter runs of their own."""
    fwd, bwd, keep = long_setup(torch)
    for _ in range(3):
        fwd()
        bwd()
    torch.cuda.synchronize()
    del keep
    dev = torch.device("cuda:0")
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print("[bench] long-sequence profile pass done: scan fwd/bwd x3, calibration neg "
          f"{src.numel() * 4} bytes each way", file=sys.stderr, flush=True)


def _host_info():
    import torch
    cpu_model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": cpu_model, "os_cpu_count": os.cpu_count(), "torch": torch.__version__}


def _median_time(run, budget_s, min_runs, max_runs, warm=2):
    for _ in range(warm):
        run()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and
                                    len(times) < max_runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 3 * budget_s:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_c1_baseline(budget_s):
    """C1 in full on the CPU: the reference's fp32 chunk-streaming scan
    (the oracle's restatement of engine/mamba.py:318-423), forward only."""
    import torch
    from oracle import scan_ref
    torch.set_num_threads(os.cpu_count() or 1)
    sh = C1_SHAPE
    c = c1_inputs(torch, "cpu")

    def run():
        with torch.no_grad():
            scan_ref.contracted_scan_ref(c["delta"], c["u"], c["Bc"], c["Cc"], c["Ar"], None,
                                         None, sh["NR"])

    med, n = _median_time(run, budget_s, 5, 50)
    return {"value": sh["B"] * sh["L"] / med, "unit": "tokens/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"the whole configuration: oracle fp32 restatement of the reference CPU "
                       f"scan, causal real decay, forward, B={sh['B']} L={sh['L']} D={sh['D']} "
                       f"N={sh['NR']}; median of {n} runs"), **_host_info()}


def cpu_long_baseline(budget_s):
    """The long-sequence layer on the CPU: the oracle's fp32 restatement of
    the reference's chunk-streaming scan with per-chunk checkpointing,
    causal, forward + autograd backward, at batch 1 and a quarter of the
    channels; channels are independent and the work is linear in them, so
    tokens/s is scaled to the full width."""
    import torch
    import torch.nn.functional as F
    from oracle import scan_ref
    torch.set_num_threads(os.cpu_count() or 1)
    sh = LONG_SHAPE
    Bs, Ds = 1, sh["D"] // 4
    L, NR, NT = sh["L"], sh["NR"], sh["NT"]
    N = NR + NT
    gen = torch.Generator().manual_seed(1005)
    u = torch.randn(Bs, L, Ds, generator=gen)
    dt = F.softplus(torch.randn(Bs, L, Ds, generator=gen) * 0.5 - 2.0)
    Bc = torch.randn(Bs, L, N, generator=gen)
    Cc = torch.randn(Bs, L, N, generator=gen)
    Bc = Bc / Bc.pow(2).mean(-1, keepdim=True).sqrt()
    Cc = Cc / Cc.pow(2).mean(-1, keepdim=True).sqrt()
    Ar = -torch.exp(torch.rand(Ds, NR, generator=gen) * 3.0)
    Ai = (torch.rand(Ds, NR, generator=gen) * 2 - 1) * math.pi
    Tk = torch.tanh(torch.randn(Ds, NT, generator=gen) * 1.5)
    dy = torch.randn(Bs, L, Ds, generator=gen)
    args = (dt, u, Bc, Cc, Ar, Ai, Tk)

    def run():
        lv = [t.clone().requires_grad_(True) for t in args]
        y, _ = scan_ref.contracted_scan_ref(*lv, N, checkpoint=True)
        (y * dy).sum().backward()

    med, n = _median_time(run, budget_s, 3, 20, warm=1)
    scale = Ds / sh["D"]
    return {"value": Bs * L / med * scale, "unit": "tokens/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"oracle fp32 restatement of the reference CPU scan (chunk-streaming "
                       f"Hillis-Steele, per-chunk checkpoint), causal fwd+bwd, B={Bs} L={L} "
                       f"D={Ds} of {sh['D']} N={N}; median of {n} runs, tokens/s scaled by "
                       f"{Ds}/{sh['D']} (the work is linear in the independent channels)"),
            **_host_info()}


def cpu_baseline(budget_s):
    """The reference's CPU PyTorch path: the fp32 chunk-streaming Hillis-Steele
    scan with per-chunk checkpointing (engine/mamba.py:318-423), both
    directions, forward + autograd backward, on a reduced batch of the same
    Eval-Mamba layer shape (bf16-rounded inputs upcast to fp32)."""
    import torch
    from oracle import scan_ref
    torch.set_num_threads(os.cpu_count() or 1)
    sh = SCAN_SHAPE
    Bs = 8
    c = scan_inputs(Bs, sh["L"], sh["D"], sh["NR"], sh["NT"], 1003, "cpu", torch.bfloat16)
    args = [c[k].float() if c[k].dtype != torch.float32 else c[k]
            for k in ("delta", "u", "Bc", "Cc", "Ar", "Ai", "Tk")]
    N = c["N"]

    def run():
        lv = [t.clone().requires_grad_(True) for t in args]
        yf, _ = scan_ref.contracted_scan_ref(*lv, N, checkpoint=True)
        yr, _ = scan_ref.contracted_scan_ref(lv[0].flip(1), lv[1].flip(1), lv[2].flip(1),
                                             lv[3].flip(1), lv[4], lv[5], lv[6], N,
                                             checkpoint=True)
        ((yf + yr.flip(1)) * c["dy"]).sum().backward()

    for _ in range(2):
        run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 3 * budget_s:
            break
    times.sort()
    med = times[len(times) // 2]
    cpu_model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": Bs * sh["L"] / med, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"oracle fp32 restatement of the reference CPU scan (chunk-streaming "
                       f"Hillis-Steele, per-chunk checkpoint), bidirectional fwd+bwd, "
                       f"B={Bs} L={sh['L']} D={sh['D']} N={N}; median of {len(times)} runs"),
            "cpu_model": cpu_model, "os_cpu_count": os.cpu_count(),
            "torch": torch.__version__}


def cpu_layer_baseline(budget_s):
    """The reference's layer on the CPU: the oracle's restatement of
    Mamba3Block (engine/mamba.py:141-380, its PyTorch scan path), fp32
    forward + backward at the layer shape with a reduced batch."""
    import torch
    from oracle import model_ref
    torch.set_num_threads(os.cpu_count() or 1)
    sh = LAYER_SHAPE
    Bs = 4
    torch.manual_seed(0)
    cfg = model_ref.MambaConfig(d_model=sh["d_model"], n_layer=1, d_state=sh["d_state"],
                                n_track_state=sh["n_track"], bidirectional=True)
    blk = model_ref.Mamba3Block(cfg)
    x = torch.randn(Bs, sh["L"], sh["d_model"])

    def run():
        blk.zero_grad(set_to_none=True)
        blk(x).square().mean().backward()

    run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 3 * budget_s:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"value": Bs * sh["L"] / med, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"oracle fp32 restatement of the reference's Mamba3Block on the CPU "
                       f"(its PyTorch scan path), bidirectional fwd+bwd, B={Bs} L={sh['L']} "
                       f"d_model={sh['d_model']} N={sh['d_state']}; median of {len(times)} runs")}


def cpu_step_baseline(budget_s):
    """The reference's per-layer torch step (engine/mamba.py:466-494; the
    oracle's fp32 restatement) at the step workload's layer shape over all
    8 layers, on a bounded sample of rollouts, on this host's cores."""
    import torch
    import torch.nn.functional as F
    from oracle import scan_ref
    torch.set_num_threads(os.cpu_count() or 1)
    sh = STEP_SHAPE
    R, D, NR, NT = sh["R"], sh["D"], sh["NR"], sh["NT"]
    N = NR + NT
    gen = torch.Generator().manual_seed(1004)
    layers = []
    for _ in range(sh["layers"]):  # parameters and one ply's inputs per layer
        layers.append(dict(
            Ar=-torch.exp(torch.rand(D, NR, generator=gen) * 3.0),
            Ai=(torch.rand(D, NR, generator=gen) * 2 - 1) * math.pi,
            Tk=torch.tanh(torch.randn(D, NT, generator=gen) * 1.5),
            Dk=torch.randn(D, generator=gen),
            dt=F.softplus(torch.randn(R, D, generator=gen) * 0.5 - 2.0),
            u=torch.randn(R, D, generator=gen),
            Bc=torch.randn(R, N, generator=gen), Cc=torch.randn(R, N, generator=gen)))
    state = [None] * sh["layers"]

    def ply():
        for i, lp in enumerate(layers):
            _, state[i] = scan_ref.step_core_ref(lp["dt"], lp["u"], lp["Bc"], lp["Cc"], lp["Ar"],
                                                 lp["Ai"], lp["Tk"], lp["Dk"], state[i])

    ply()
    plies, t0 = 0, time.perf_counter()
    while plies < 2 or (time.perf_counter() - t0 < budget_s and plies < 32):
        ply()
        plies += 1
    el = time.perf_counter() - t0
    return {"value": R * plies / el, "unit": "rollout-steps/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"oracle fp32 restatement of the reference torch step (SSM core), "
                       f"{sh['layers']} layers, R={R} rollouts, D={D} N={N}: {plies} of the "
                       f"32 plies after one warm-up ply (a ply costs the same at any depth: "
                       f"the state is O(1))"), **_host_info()}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); "
              "the scan and step shard by batch / rollout with no exchange, so N GPUs "
              "run N independent copies of this workload.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.profile_pass:
        profile_pass(torch)
        return
    if args.profile_pass_long:
        profile_pass_long(torch)
        return
    print(f"[bench] scan fwd+bwd {SCAN_SHAPE} bf16 storage, steps={args.steps} "
          f"warmup={args.warmup}", file=sys.stderr, flush=True)
    sc = bench_scan(torch, args, torch.bfloat16)
    print(f"[bench] scan: {sc['tok_s']:.4g} tokens/s; fwd {sc['t_fwd'] * 1e3:.3f} ms, "
          f"bwd {sc['t_bwd'] * 1e3:.3f} ms", file=sys.stderr, flush=True)
    step = None
    if not args.no_step:
        print(f"[bench] step {STEP_SHAPE}", file=sys.stderr, flush=True)
        step = bench_step(torch, args)
        print(f"[bench] step: {step['rollout_steps_s']:.4g} rollout-steps/s, "
              f"{step['t_launch'] * 1e6:.1f} us/launch, {step['GBps']:.0f} GB/s; rank-1 cache "
              f"{step['rollout_steps_s_rank1']:.4g} rollout-steps/s, "
              f"{step['t_launch_rank1'] * 1e6:.1f} us/launch, {step['GBps_rank1']:.0f} GB/s",
              file=sys.stderr, flush=True)
        step_def = bench_step(torch, args, plies=8, shape=STEP_SHAPE_DEFAULT)
        print(f"[bench] step {STEP_SHAPE_DEFAULT}: {step_def['t_launch'] * 1e6:.1f} us/launch, "
              f"{step_def['GBps']:.0f} GB/s; rank-1 cache {step_def['t_launch_rank1'] * 1e6:.1f} "
              f"us/launch, {step_def['GBps_rank1']:.0f} GB/s", file=sys.stderr, flush=True)
    states = None
    if not args.no_step and not args.no_step_states:
        states = []
        for NR, NT in STEP_STATES:
            sh = dict(R=4096, layers=2, D=1024, NR=NR, NT=NT)
            r = bench_step(torch, args, plies=16, shape=sh)
            states.append({"d_state": NR + NT, "NR": NR, "NT": NT,
                           "avg_launch_s": r["t_launch"], "alg_bytes_per_launch": r["bytes"],
                           "achieved_GBps": r["GBps"], "frac": r["GBps"] / HBM_PEAK_GBS,
                           "rank1_cache": {"avg_launch_s": r["t_launch_rank1"],
                                           "alg_bytes_per_launch": r["bytes_rank1"],
                                           "achieved_GBps": r["GBps_rank1"],
                                           "frac": r["GBps_rank1"] / HBM_PEAK_GBS}})
            print(f"[bench] step d_state {NR + NT:3d} ({NR}+{NT}): {r['t_launch'] * 1e6:7.1f} "
                  f"us/launch, {r['GBps']:.0f} GB/s ({r['GBps'] / HBM_PEAK_GBS:.0%}); rank-1 "
                  f"{r['t_launch_rank1'] * 1e6:7.1f} us, {r['GBps_rank1']:.0f} GB/s "
                  f"({r['GBps_rank1'] / HBM_PEAK_GBS:.0%})", file=sys.stderr, flush=True)
            del r
            torch.cuda.empty_cache()
    lng = None
    if not args.no_long:
        print(f"[bench] long-sequence scan {LONG_SHAPE} fp32", file=sys.stderr, flush=True)
        lng = bench_long(torch, args)
        print(f"[bench] long: {lng['tok_s']:.4g} tokens/s; fwd {lng['t_fwd'] * 1e3:.2f} ms, "
              f"bwd {lng['t_bwd'] * 1e3:.2f} ms", file=sys.stderr, flush=True)
    c1 = bench_c1(torch, args)
    print(f"[bench] C1 (B=8 L=64 D=256 N=16 real, causal fwd): {c1['tok_s']:.4g} tokens/s, "
          f"{c1['t_fwd'] * 1e6:.1f} us/launch", file=sys.stderr, flush=True)
    ply = None
    if not args.no_step:
        ply = bench_ply(torch, args)
        print(f"[bench] whole ply ({PLY_SHAPE['layers']} layers, R={PLY_SHAPE['R']}): "
              f"{ply['full']['s_per_ply'] * 1e3:.3f} ms ({ply['full']['rollout_steps_s']:.4g} "
              f"rollout-steps/s); rank-1 cache {ply['rank1']['s_per_ply'] * 1e3:.3f} ms "
              f"({ply['rank1']['rollout_steps_s']:.4g})", file=sys.stderr, flush=True)
    sweep = dyn = None
    if not args.no_step and not args.no_sweep:
        sweep = bench_step_sweep(torch, args)
        dyn = bench_dynamics(torch, args)
        print(f"[bench] dynamics rollout fwd+bwd ({DYN_SHAPE}): fp32 "
              f"{dyn['fp32']['train_step_s'] * 1e3:.2f} ms (prime part "
              f"{dyn['fp32']['prime_only_s'] * 1e3:.2f} ms); bf16 autocast "
              f"{dyn['bf16_autocast']['train_step_s'] * 1e3:.2f} ms; fp32 from graphs "
              f"{dyn['fp32_graphed']['train_step_s'] * 1e3:.2f} ms",
              file=sys.stderr, flush=True)
    hbm_practical = practical_hbm_peak(torch)
    print(f"[bench] torch 1 GiB copy: {hbm_practical:.0f} GB/s", file=sys.stderr, flush=True)
    lay = mix = None
    if not args.no_layer:
        lay = bench_layer(torch, args)
        print(f"[bench] layer fwd+bwd: fused {lay['t_fused'] * 1e3:.3f} ms "
              f"({lay['tok_fused']:.4g} tokens/s); scan-only drop-in {lay['t_dropin'] * 1e3:.3f} ms "
              f"({lay['tok_dropin']:.4g} tokens/s)", file=sys.stderr, flush=True)
    if not args.no_mixer:
        mix = bench_mixer(torch, args)
        print(f"[bench] mixer gate: fwd {mix['t_fwd'] * 1e6:.1f} us "
              f"({mix['fwd_bytes'] / mix['t_fwd'] / 1e9:.0f} GB/s), bwd {mix['t_bwd'] * 1e6:.1f} us "
              f"({mix['bwd_bytes'] / mix['t_bwd'] / 1e9:.0f} GB/s); fwd+bwd autograd "
              f"{mix['t_fused'] * 1e6:.1f} us fused vs {mix['t_torch'] * 1e6:.1f} us torch ops",
              file=sys.stderr, flush=True)
    roll = None
    if not args.no_rollout:
        roll = bench_rollout(torch, args)
        print(f"[bench] rollout ply boundary (R={ROLLOUT_SHAPE['R']}, V={ROLLOUT_SHAPE['V']}): "
              f"pinned {roll['t_ours'] * 1e3:.3f} ms/ply (top-k kernel "
              f"{roll['t_kernel'] * 1e6:.1f} us, {roll['kernel_bytes'] / roll['t_kernel'] / 1e9:.0f} "
              f"GB/s) vs per-rollout reads {roll['t_ref'] * 1e3:.1f} ms/ply; legal-move logits "
              f"{roll['t_legal'] * 1e3:.3f} vs {roll['t_ref_legal'] * 1e3:.1f} ms/ply",
              file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.cpu_seconds)
        print(f"[bench] cpu: {cpu['value']:.4g} tokens/s on {cpu['cores']} threads",
              file=sys.stderr, flush=True)
        if lay is not None:
            lay["cpu_baseline"] = cpu_layer_baseline(args.cpu_seconds / 3)
            print(f"[bench] cpu layer: {lay['cpu_baseline']['value']:.4g} tokens/s",
                  file=sys.stderr, flush=True)
        if step is not None:
            step["cpu_baseline"] = cpu_step_baseline(args.cpu_seconds / 2)
            print(f"[bench] cpu step: {step['cpu_baseline']['value']:.4g} rollout-steps/s",
                  file=sys.stderr, flush=True)
        c1["cpu_baseline"] = cpu_c1_baseline(args.cpu_seconds / 5)
        print(f"[bench] cpu C1: {c1['cpu_baseline']['value']:.4g} tokens/s", file=sys.stderr,
              flush=True)
        if lng is not None:
            lng["cpu_baseline"] = cpu_long_baseline(args.cpu_seconds / 3)
            print(f"[bench] cpu long: {lng['cpu_baseline']['value']:.4g} tokens/s",
                  file=sys.stderr, flush=True)

    # dominant kernel: the longer of forward (training) and backward
    k_f, k_b = sc["kernels"][0], sc["kernels"][2]
    dom = k_b if k_b["seconds"] >= k_f["seconds"] else k_f
    tr = measured_traffic()
    vc = measured_valu()
    roof = {"bound": "hbm", "kernel": dom["kernel"], "achieved": dom["GBps"],
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": dom["GBps"] / HBM_PEAK_GBS,
            "traffic": tr.get(dom["traffic_key"]), "alg_bytes_per_launch": dom["alg_bytes"],
            "avg_launch_s": dom["seconds"]}
    # the scan kernels are bound by the vector ALU, not by HBM: their issue
    # rate against the VALU peak, from the committed counter pass
    for k in sc["kernels"]:
        key = "scan_bwd_kernel" if k["kernel"].startswith("scan_bwd") else "scan_fwd_kernel"
        k["valu"] = valu_roofline(vc.get(key), k["seconds"]) if k["traffic_key"] else None
    roof["valu"] = dom.get("valu")
    # torch's 1 GiB device-to-device copy (read + write); the step kernel's
    # coalesced non-temporal streaming runs above it
    roof["torch_copy_GBps"] = hbm_practical
    ms = sc["elapsed"] / args.steps * 1e3
    line = {
        "metric": "scan fwd+bwd tokens/s & %HBM peak; batched step() rollout-steps/s",
        "value": sc["tok_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 (bf16-stored inputs)", "data": "synthetic",
        "config": {"workload": "Eval-Mamba bidirectional trapezoidal scan layer, fwd+bwd",
                   "B": SCAN_SHAPE["B"], "L": SCAN_SHAPE["L"], "d_inner": SCAN_SHAPE["D"],
                   "d_state": SCAN_SHAPE["NR"] + SCAN_SHAPE["NT"], "n_rot": SCAN_SHAPE["NR"],
                   "n_track": SCAN_SHAPE["NT"], "input_storage": "bf16",
                   "parallelism": "single GPU"},
        "roofline": roof,
        "kernels": sc["kernels"],
        "fwd_only_tokens_s": sc["T"] / sc["t_inf"],
    }
    if step is not None:
        line["step"] = {
            "metric": "rollout-steps/s", "value": step["rollout_steps_s"],
            "config": {"workload": "Search-Mamba batched step, SSM core over all layers",
                       **STEP_SHAPE, "d_state": STEP_SHAPE["NR"] + STEP_SHAPE["NT"]},
            "roofline": {"bound": "hbm", "kernel": "step_kernel",
                         "achieved": step["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": step["GBps"] / HBM_PEAK_GBS,
                         "traffic": tr.get("step_tile_kernel"),
                         "alg_bytes_per_launch": step["bytes"],
                         "avg_launch_s": step["t_launch"]},
            "cpu_baseline": step.get("cpu_baseline"),
            "whole_ply": None if ply is None else {
                "workload": "Mamba.step(input_embed) over 8 causal layers, d_model 512, "
                            "mimo_p 2, 4096 rollouts, fp32, no autograd (projections, norms "
                            "and the fused step kernel)",
                "rollout_steps_s": ply["full"]["rollout_steps_s"],
                "s_per_ply": ply["full"]["s_per_ply"],
                "rank1_cache": {"rollout_steps_s": ply["rank1"]["rollout_steps_s"],
                                "s_per_ply": ply["rank1"]["s_per_ply"]}},
            "rank1_cache": {
                "workload": "the same plies with each layer's beta cached as rank-1 rows "
                            "[dt*u | B] (D + N floats per rollout; bit-identical results)",
                "value": step["rollout_steps_s_rank1"], "unit": "rollout-steps/s",
                "avg_launch_s": step["t_launch_rank1"],
                "alg_bytes_per_launch": step["bytes_rank1"],
                "achieved_GBps": step["GBps_rank1"],
                "frac": step["GBps_rank1"] / HBM_PEAK_GBS,
                "traffic": tr.get("step_tile_kernel[rank1]")},
            "sweep": None if sweep is None else {
                "workload": "the step kernel over 8 layers (d_inner 1024, d_state 16 + 4) and "
                            "the whole ply through Mamba.step(input_embed) at each rollout count, "
                            "eager and replayed from HIP graphs (StepGraph); kernel times by HIP "
                            "events, whole plies by the host clock",
                "rows": sweep},
            "training_through_step": None if dyn is None else {
                "workload": "SearchMamba.dynamics_rollout forward + backward (prime_cache over "
                            "the board, then differentiable step() plies with the value, "
                            "continuation and consistency heads); no optimizer",
                "config": DYN_SHAPE, **dyn},
            "from_shared_state": {
                "workload": "first ply after a batch-1 cache is fanned out to the rollouts "
                            "(broadcast input state, no copies)",
                "avg_launch_s": step["t_shared"], "alg_bytes_per_launch": step["bytes_shared"],
                "achieved_GBps": step["GBps_shared"]},
            "state_sizes": None if states is None else {
                "workload": "the step kernel across state sizes: 4096 rollouts, d_inner 1024, "
                            "two layers alternating, full and rank-1 caches",
                "shapes": states},
            "search_model_default": {
                "workload": "the step kernel at the reference's default search-model core "
                            "(SearchMambaConfig: 12 layers, d_inner 768, d_state 32 all "
                            "rotational), 4096 rollouts, full and rank-1 caches",
                "config": {**STEP_SHAPE_DEFAULT,
                           "d_state": STEP_SHAPE_DEFAULT["NR"] + STEP_SHAPE_DEFAULT["NT"]},
                "rollout_steps_s": STEP_SHAPE_DEFAULT["R"] / (step_def["t_launch"]
                                                             * STEP_SHAPE_DEFAULT["layers"]),
                "avg_launch_s": step_def["t_launch"], "alg_bytes_per_launch": step_def["bytes"],
                "achieved_GBps": step_def["GBps"], "frac": step_def["GBps"] / HBM_PEAK_GBS,
                "rank1_cache": {"avg_launch_s": step_def["t_launch_rank1"],
                                "alg_bytes_per_launch": step_def["bytes_rank1"],
                                "achieved_GBps": step_def["GBps_rank1"],
                                "frac": step_def["GBps_rank1"] / HBM_PEAK_GBS}},
        }
    if lng is not None:
        trl, vcl = measured_traffic("traffic_long.json"), measured_valu("valu_long.json")

        def lk(kernel, key, secs, nbytes):
            gbs = nbytes / secs / 1e9
            return {"kernel": kernel, "avg_launch_s": secs, "alg_bytes_per_launch": nbytes,
                    "hbm": {"achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": gbs / HBM_PEAK_GBS, "traffic": trl.get(key)},
                    "valu": valu_roofline(vcl.get(key.split("+")[0]), secs)}
        line["long_sequence"] = {
            "metric": "tokens/s", "value": lng["tok_s"],
            "config": {"workload": "causal trapezoidal scan layer, fwd+bwd, fp32 inputs",
                       **LONG_SHAPE, "d_state": LONG_SHAPE["NR"] + LONG_SHAPE["NT"]},
            "fwd_s": lng["t_fwd"], "bwd_s": lng["t_bwd"],
            "alg_bytes_fwd": lng["fwd_bytes"], "alg_bytes_bwd": lng["bwd_bytes"],
            "roofline": [lk("scan_fwd_kernel (causal, checkpoints)", "scan_fwd_kernel",
                            lng["t_fwd"], lng["fwd_bytes"]),
                         lk("scan_bwd_kernel + reductions", "scan_bwd_kernel+reductions",
                            lng["t_bwd"], lng["bwd_bytes"])],
            "cpu_baseline": lng.get("cpu_baseline"),
        }
    line["c1"] = {
        "metric": "tokens/s", "value": c1["tok_s"],
        "config": {"workload": "the reference's CPU configuration: one causal real-decay scan "
                               "layer forward, fp32", **C1_SHAPE, "d_state": C1_SHAPE["NR"]},
        "avg_launch_s": c1["t_fwd"], "alg_bytes_per_launch": c1["fwd_bytes"],
        "cpu_baseline": c1.get("cpu_baseline"),
    }
    if lay is not None:
        line["layer"] = {
            "metric": "tokens/s", "value": lay["tok_fused"],
            "config": {"workload": "one bidirectional Mamba3Block forward + backward under bf16 "
                                   "autocast (projections on hipBLASLt, SSM path fused HIP)",
                       **LAYER_SHAPE, "mimo_p": 4},
            "fwd_bwd_s": lay["t_fused"],
            "scan_only_dropin": {"workload": "the reference's layer ops with only the scan "
                                             "swapped for the HIP scan",
                                 "fwd_bwd_s": lay["t_dropin"], "tokens_s": lay["tok_dropin"]},
            "cpu_baseline": lay.get("cpu_baseline"),
        }
    if mix is not None:
        line["mixer_gate"] = {
            "workload": "(y + 2 u D) silu(z) of the bidirectional layer at the scan shape, "
                        "bf16 u / z (z a chunk of the in_proj output), fp32 y and gradients",
            "fwd": {"kernel": "mixer_out_fwd_vec_kernel", "avg_launch_s": mix["t_fwd"],
                    "alg_bytes_per_launch": mix["fwd_bytes"],
                    "achieved_GBps": mix["fwd_bytes"] / mix["t_fwd"] / 1e9,
                    "frac": mix["fwd_bytes"] / mix["t_fwd"] / 1e9 / HBM_PEAK_GBS,
                    "traffic": tr.get("mixer_out_fwd_vec_kernel")},
            "bwd": {"kernel": "mixer_out_bwd_vec_kernel + reduction", "avg_launch_s": mix["t_bwd"],
                    "alg_bytes_per_launch": mix["bwd_bytes"],
                    "achieved_GBps": mix["bwd_bytes"] / mix["t_bwd"] / 1e9,
                    "frac": mix["bwd_bytes"] / mix["t_bwd"] / 1e9 / HBM_PEAK_GBS,
                    "traffic": tr.get("mixer_out_bwd+reduction")},
            "timing": "each launch after a 512 MB read that displaces the last-level cache",
            "warm_cache_avg_launch_s": {"fwd": mix["t_fwd_warm"], "bwd": mix["t_bwd_warm"]},
            "fwd_bwd_autograd_s": {"fused": mix["t_fused"], "torch_ops": mix["t_torch"]},
        }
    if roll is not None:
        line["rollout_boundary"] = {
            "workload": "one ply's host transfers for 4096 lockstep rollouts: token ids up, "
                        "values and each rollout's top-8 continuation candidates (8192-token "
                        "vocabulary) down; and the fastchess path's logits of 40 legal moves "
                        "per rollout",
            **ROLLOUT_SHAPE,
            "pinned_boundary_s_per_ply": roll["t_ours"],
            "reference_pattern_s_per_ply": roll["t_ref"],
            "legal_logits_s_per_ply": {"pinned": roll["t_legal"], "reference_pattern": roll["t_ref_legal"]},
            "reference_sample": f"{roll['sample']} rollouts' row reads timed and scaled to R",
            "kernel": {"name": "ply_topk_kernel", "avg_launch_s": roll["t_kernel"],
                       "alg_bytes_per_launch": roll["kernel_bytes"],
                       "achieved_GBps": roll["kernel_bytes"] / roll["t_kernel"] / 1e9,
                       "frac": roll["kernel_bytes"] / roll["t_kernel"] / 1e9 / HBM_PEAK_GBS},
            "timing": "host wall clock per ply (perf_counter), the kernel by HIP events",
        }
    line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
