"""Mamba-3 backbone whose SSM core runs on the HIP kernels.

API- and state_dict-compatible with the reference's engine/mamba.py: the same
`MambaConfig` fields, the same module tree and parameter names
(`layers.{i}.mixer.{in_proj,x_proj,dt_proj,out_proj}`, `A_log_mag`,
`A_phase` / `A_log`, `track_theta`, `b_norm`, `c_norm`, `D`,
`layers.{i}.norm`, `embedding`, `norm_f`), the same construction order (so a
seeded init draws the same numbers) and the same forward / step /
prime_cache / forward_with_state entry points.  Reference checkpoints load
unchanged, and callers written against the reference run unchanged.

What differs is where the selective scan and the O(1) step run:
  * `_selective_scan_trapezoidal` (engine/mamba.py:318-380) calls the fused
    HIP scan for every case, including the return_state path the reference
    keeps on PyTorch (:343, :377-379);
  * the bidirectional layer (:254-260) is one fused launch over both
    directions, with no flip copies;
  * `Mamba3Block.step` (:427-498) runs the fused step kernel; under autograd
    (SearchMamba.dynamics_rollout trains through step) it runs the scan
    kernel with L = 1 from the cached state, whose analytic backward carries
    gradients into the previous state.
Projections, norms and the residual stack stay plain torch (GEMMs).  There is
no PyTorch fallback for the SSM core: device tensors on a ROCm GPU are
required, and a missing library raises.  `use_triton_scan` is accepted for
config compatibility; the HIP path does not depend on it.
"""

import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F
import torch.utils.checkpoint

from redpanda_amd.bcnorm import hip_bcnorm_psum
from redpanda_amd.mixer import hip_mixer_out
from redpanda_amd.norm import hip_add_rmsnorm
from redpanda_amd.scan import hip_scan_with_state, hip_trapezoidal_scan
from redpanda_amd.step import compact_beta, full_beta, hip_softplus, hip_step, is_compact

# Chunk length of the reference's streaming scan (engine/mamba.py:101); kept
# as a module constant for callers that read it.  The HIP scan is not chunked.
SCAN_CHUNK = 32


@dataclass
class MambaConfig:
    """Fields and derived values of engine/mamba.py:24-78."""
    d_model: int = 512
    n_layer: int = 16
    vocab_size: int = 8192
    d_state: int = 64
    expand: int = 2
    dt_rank: int = "auto"
    pad_vocab_size_multiple: int = 8
    bias: bool = False
    use_complex: bool = True
    mimo_p: int = 4
    use_bcnorm: bool = True
    n_track_state: int = 0
    bidirectional: bool = False
    grad_checkpoint: bool = False
    scan_checkpoint: bool = True
    use_triton_scan: bool = False

    def __post_init__(self):
        self.d_inner = int(self.expand * self.d_model)
        if self.dt_rank == "auto":
            self.dt_rank = math.ceil(self.d_model / 16)
        assert 0 <= self.n_track_state < self.d_state, "n_track_state must be < d_state"
        self.n_rot_state = self.d_state - self.n_track_state
        rem = self.vocab_size % self.pad_vocab_size_multiple
        if rem:
            self.vocab_size += self.pad_vocab_size_multiple - rem


class RMSNorm(nn.Module):
    """engine/mamba.py:82-89."""

    def __init__(self, d: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight


def _gate_out_dtype():
    """The dtype out_proj will read the gate's output in: autocast's when it
    is on for the device, so the gate writes it directly (the same rounding
    as the cast autocast would insert), else fp32 as the reference's op."""
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return torch.float32


def _need_device(t, what):
    if not t.is_cuda:
        raise RuntimeError(
            f"redpanda_amd.mamba: {what} runs on the HIP kernels and needs ROCm device "
            "tensors; move the model and inputs to the GPU")


class Mamba3Block(nn.Module):
    """One Mamba-3 layer (engine/mamba.py:141-498) with the SSM core on HIP."""

    def __init__(self, config: MambaConfig):
        super().__init__()
        self.config = config
        d_inner, n = config.d_inner, config.d_state
        n_rot, n_track, p = config.n_rot_state, config.n_track_state, config.mimo_p
        self.in_proj = nn.Linear(config.d_model, d_inner * 2, bias=config.bias)
        self.x_proj = nn.Linear(d_inner, config.dt_rank + n * p * 2, bias=True)
        self.dt_proj = nn.Linear(config.dt_rank, d_inner, bias=True)
        with torch.no_grad():
            # dt bias: softplus^-1 of log-uniform timescales in [1e-3, 1e-1]
            lo, hi = math.log(0.001), math.log(0.1)
            dt0 = torch.exp(torch.rand(d_inner) * (hi - lo) + lo)
            self.dt_proj.bias.copy_(dt0 + torch.log(-torch.expm1(-dt0)))
            self.dt_proj.bias._no_reinit = True
        if n_rot > 0:
            base = torch.arange(1, n_rot + 1, dtype=torch.float32).unsqueeze(0).repeat(d_inner, 1)
            if config.use_complex:
                self.A_log_mag = nn.Parameter(torch.log(base))
                self.A_phase = nn.Parameter(torch.zeros(d_inner, n_rot))
            else:
                self.A_log = nn.Parameter(torch.log(base))
        if n_track > 0:
            th = torch.atanh(torch.linspace(-0.95, 0.95, n_track).clamp(-0.999, 0.999))
            self.track_theta = nn.Parameter(th.unsqueeze(0).repeat(d_inner, 1))
        if config.use_bcnorm:
            self.b_norm = RMSNorm(n * p)
            self.c_norm = RMSNorm(n * p)
        self.D = nn.Parameter(torch.ones(d_inner))
        self.out_proj = nn.Linear(d_inner, config.d_model, bias=config.bias)

    # ── gates (engine/mamba.py:211-229) ──

    def _compute_A(self):
        """(A_real, A_imag) of the rotational states, (d_inner, n_rot), or Nones."""
        if self.config.n_rot_state == 0:
            return None, None
        if self.config.use_complex:
            mag = -torch.exp(self.A_log_mag.float())
            phase = self.A_phase.float()
            return mag * torch.cos(phase), mag * torch.sin(phase)
        return -torch.exp(self.A_log.float()), None

    def _track_gate(self):
        """tanh(theta) of the tracking states, (d_inner, n_track)."""
        return torch.tanh(self.track_theta.float())

    def _track_or_none(self):
        return self._track_gate() if self.config.n_track_state > 0 else None

    def _gate_params(self):
        """The parameters the gates are computed from."""
        ps = [getattr(self, n) for n in ("A_log_mag", "A_phase", "A_log", "track_theta")
              if hasattr(self, n)]
        return ps

    def _gates(self, record_grad):
        """(A_real, A_imag, track).  Without an autograd graph to record they
        are computed once and reused until a gate parameter changes (its
        storage or its version counter, which every in-place update such as
        an optimizer step or load_state_dict advances): an inference loop of
        step() calls then skips five small kernels per layer."""
        if record_grad:
            return (*self._compute_A(), self._track_or_none())
        fixed = self.__dict__.get("_gates_fixed")
        if fixed is not None:
            # buffers that a captured graph reads (StepGraph refreshes them
            # from this method's values whenever a gate parameter changes)
            return fixed
        key = tuple((t.data_ptr(), t._version, t.device) for t in self._gate_params())
        hit = self.__dict__.get("_gate_cache")
        if hit is not None and hit[0] == key:
            return hit[1]
        with torch.no_grad():
            val = (*self._compute_A(), self._track_or_none())
        self.__dict__["_gate_cache"] = (key, val)
        return val

    # ── projections (engine/mamba.py:284-301) ──

    def _ssm_proj(self, u):
        cfg = self.config
        lead = u.shape[:-1]
        n, p = cfg.d_state, cfg.mimo_p
        dt_raw, B_raw, C_raw = self.x_proj(u).split([cfg.dt_rank, n * p, n * p], dim=-1)
        if cfg.use_bcnorm:
            B_raw = self.b_norm(B_raw)
            C_raw = self.c_norm(C_raw)
        delta = F.softplus(self.dt_proj(dt_raw))
        return delta, B_raw.view(*lead, n, p), C_raw.view(*lead, n, p)

    def _ssm_proj_contracted(self, u):
        """(x_dt, Bc, Cc): _ssm_proj followed by the sums over p
        (engine/mamba.py:336-337), with BCNorm and the sums in one fused
        kernel; Bc, Cc fp32 (..., d_state).  x_dt is the dt projection
        BEFORE softplus: the scan and step kernels apply softplus on load
        (delta_softplus=True)."""
        cfg = self.config
        n, p = cfg.d_state, cfg.mimo_p
        dt_raw, B_raw, C_raw = self.x_proj(u).split([cfg.dt_rank, n * p, n * p], dim=-1)
        if cfg.use_bcnorm:
            Bc, Cc = hip_bcnorm_psum(B_raw, C_raw, self.b_norm.weight, self.c_norm.weight, p,
                                     self.b_norm.eps)
        else:
            Bc, Cc = hip_bcnorm_psum(B_raw, C_raw, None, None, p, normalize=False)
        return self.dt_proj(dt_raw), Bc, Cc

    def _ssm_proj_raw(self, u):
        """(x_dt, bcnorm): as _ssm_proj_contracted, with BCNorm + the p-sum
        left to the step (hip_step's bcnorm argument: the raw B / C
        projections, BCNorm's weights and eps), which gives the same rows."""
        cfg = self.config
        n, p = cfg.d_state, cfg.mimo_p
        dt_raw, B_raw, C_raw = self.x_proj(u).split([cfg.dt_rank, n * p, n * p], dim=-1)
        if cfg.use_bcnorm:
            bcn = (B_raw, C_raw, self.b_norm.weight, self.c_norm.weight, p, self.b_norm.eps, True)
        else:
            bcn = (B_raw, C_raw, None, None, p, 0.0, False)
        return self.dt_proj(dt_raw), bcn

    # ── scan ──

    def _selective_scan_trapezoidal(self, u, delta, A_real, A_imag, B, C, D,
                                    return_state=False, bidirectional=False):
        """engine/mamba.py:318-380 on the HIP scan: y = scan(u) + u * D, with
        B/C contracted over the MIMO dimension first (:336-337).  With
        `bidirectional` the fused two-direction scan returns
        S(u) + flip(S(flip(u))) and the skip is added once per direction."""
        if return_state:
            y, state = self._scan_core(u, delta, A_real, A_imag, B, C, return_state=True)
            return y + u * D, state
        y = self._scan_core(u, delta, A_real, A_imag, B, C, bidirectional=bidirectional)
        if bidirectional:
            return y + u * D + u * D
        return y + u * D

    def _scan_core(self, u, delta, A_real, A_imag, B, C, return_state=False,
                   bidirectional=False, contracted=False, delta_softplus=False):
        """The scan alone (no D-skip): y, or (y, (h_last, beta_last)).  B, C:
        (..., n, p), or already contracted (..., n) with contracted=True;
        delta_softplus: delta is the dt projection before softplus."""
        _need_device(u, "the selective scan")
        cfg = self.config
        Bc = B if contracted else B.sum(dim=-1)
        Cc = C if contracted else C.sum(dim=-1)
        track = self._track_or_none()
        if return_state:
            return hip_scan_with_state(delta, u, Bc, Cc, A_real, A_imag, track,
                                       delta_softplus=delta_softplus)
        return hip_trapezoidal_scan(delta, u, Bc, Cc, A_real, A_imag, track,
                                    cfg.n_rot_state, cfg.d_state, bidirectional=bidirectional,
                                    delta_softplus=delta_softplus)

    def ssm(self, u, return_state=False):
        delta, B, C = self._ssm_proj(u)
        A_real, A_imag = self._compute_A()
        return self._selective_scan_trapezoidal(u, delta, A_real, A_imag, B, C, self.D,
                                                return_state=return_state)

    def forward(self, x):
        """engine/mamba.py:231-267; the bidirectional branch is one fused launch,
        and the D-skip and silu(z) gate one fused pass after it."""
        x_branch, z = self.in_proj(x).chunk(2, dim=-1)
        x_branch = F.silu(x_branch)
        x_dt, Bc, Cc = self._ssm_proj_contracted(x_branch)
        A_real, A_imag = self._compute_A()
        bi = self.config.bidirectional
        y = self._scan_core(x_branch, x_dt, A_real, A_imag, Bc, Cc, bidirectional=bi,
                            contracted=True, delta_softplus=True)
        return self.out_proj(hip_mixer_out(y, x_branch, z, self.D, 2 if bi else 1,
                                           out_dtype=_gate_out_dtype()))

    def forward_with_state(self, x, compact=False):
        """engine/mamba.py:269-282: output plus the final (h, beta) cache.
        compact=True returns beta as its rank-1 row [dt*u | B] of the last
        token (B, d_inner + d_state), which step() continues from with the
        same results at half the state traffic."""
        x_branch, z = self.in_proj(x).chunk(2, dim=-1)
        x_branch = F.silu(x_branch)
        x_dt, Bc, Cc = self._ssm_proj_contracted(x_branch)
        A_real, A_imag = self._compute_A()
        y, (h, beta) = self._scan_core(x_branch, x_dt, A_real, A_imag, Bc, Cc, return_state=True,
                                       contracted=True, delta_softplus=True)
        if compact:
            beta = self._compact_beta(x_dt[:, -1], x_branch[:, -1], Bc[:, -1])
        return self.out_proj(hip_mixer_out(y, x_branch, z, self.D, 1,
                                           out_dtype=_gate_out_dtype())), (h, beta)

    @staticmethod
    def _compact_beta(x_dt, u, Bc):
        """Rank-1 row [dt*u | B] of one token's beta, dt = softplus(x_dt) in
        fp32 with the kernels' bits (differentiable)."""
        dtu = hip_softplus(x_dt) * u.float()
        return compact_beta(dtu, Bc)

    # ── O(1) step (engine/mamba.py:427-498) ──

    def step(self, x_t, state=None, compact=False, out=None):
        """One token for a batch: x_t (B, d_model), state (h, beta) fp32
        (B, d_inner, d_state) or None.  Returns (out (B, d_model), (h, beta)).
        beta may also be in rank-1 rows (B, d_inner + d_state) (see
        forward_with_state); the new state keeps the form of the one given,
        or with no state the form `compact` asks for.  out: None, or the
        (h, beta) buffers the new state is written to (inference only; see
        hip_step), returned as the new state."""
        _need_device(x_t, "step()")
        cfg = self.config
        x_branch, z = self.in_proj(x_t).chunk(2, dim=-1)
        x_branch = F.silu(x_branch)
        grad = torch.is_grad_enabled() and (
            any(p.requires_grad for p in self.parameters()) or x_t.requires_grad or
            (state is not None and any(s.requires_grad for s in state)))
        if grad:
            x_dt, Bc, Cc = self._ssm_proj_contracted(x_branch)
        else:
            # BCNorm + the p-sum go into the step (one launch fewer per layer)
            x_dt, bcn = self._ssm_proj_raw(x_branch)
        A_real, A_imag, track = self._gates(grad)
        rank1 = is_compact(state[1]) if state is not None else bool(compact)
        if grad and out is not None:
            raise ValueError("step: out buffers are for inference (no autograd graph)")
        if grad:
            # differentiable: a length-1 scan from the cached state (a rank-1
            # beta expanded to its full form first)
            if state is not None and rank1:
                state = (state[0], full_beta(state[1], cfg.d_inner))
            y, (h, beta) = hip_scan_with_state(x_dt.unsqueeze(1), x_branch.unsqueeze(1),
                                               Bc.unsqueeze(1), Cc.unsqueeze(1),
                                               A_real, A_imag, track, state=state,
                                               delta_softplus=True)
            y = y.squeeze(1) + x_branch * self.D
            if rank1:
                beta = self._compact_beta(x_dt, x_branch, Bc)
            y = y * F.silu(z)
        else:
            # the gate y * silu(z) is applied by the step kernel
            y, (h, beta) = hip_step(x_dt, x_branch, None, None, A_real, A_imag, track, self.D,
                                    state, out=None if out is None else (None, *out),
                                    delta_softplus=True, compact=rank1, z=z, bcnorm=bcn)
        return self.out_proj(y), (h, beta)


class Mamba(nn.Module):
    """Embedding + n_layer pre-norm Mamba-3 blocks + final norm (engine/mamba.py:503-620)."""

    def __init__(self, config: MambaConfig):
        super().__init__()
        self.config = config
        self.grad_checkpoint = getattr(config, "grad_checkpoint", False)
        self.embedding = nn.Embedding(config.vocab_size, config.d_model)
        self.layers = nn.ModuleList([
            nn.ModuleDict({"mixer": Mamba3Block(config), "norm": RMSNorm(config.d_model)})
            for _ in range(config.n_layer)])
        self.norm_f = RMSNorm(config.d_model)
        self.apply(self._init_weights)

    def _init_weights(self, module):
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None and not getattr(module.bias, "_no_reinit", False):
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(self, input_ids, input_embeds=None):
        """(B, L) ids or (B, L, d_model) embeddings -> (B, L, d_model)."""
        x = input_embeds if input_embeds is not None else self.embedding(input_ids)
        for layer in self.layers:
            mixer, norm = layer["mixer"], layer["norm"]
            if self.grad_checkpoint and self.training and x.requires_grad:
                # the scan is stateless and deterministic, so recomputation in
                # backward reproduces the forward exactly
                x = x + torch.utils.checkpoint.checkpoint(
                    lambda inp, m=mixer, nm=norm: m(nm(inp)), x, use_reentrant=False)
            else:
                x = x + mixer(norm(x))
        return self.norm_f(x)

    def init_cache(self, batch_size, device):
        """An empty per-layer cache (engine/mamba.py:560-562)."""
        return [None] * len(self.layers)

    def step(self, token_id=None, cache=None, input_embed=None, apply_final_norm=True,
             compact=False, out_cache=None):
        """One token through every layer (engine/mamba.py:564-601).  A layer
        with no cached state starts from zero and, with compact=True, returns
        its beta in rank-1 rows (see Mamba3Block.step).  out_cache: None, or
        per-layer (h, beta) buffers the new cache is written to (inference
        only); it is then the returned cache."""
        assert not self.config.bidirectional, "step() requires a causal model"
        if input_embed is not None:
            x = input_embed
        else:
            if token_id.dim() == 2:
                token_id = token_id.squeeze(1)
            x = self.embedding(token_id)
        if cache is None:
            cache = [None] * len(self.layers)
        new_cache = []
        record = torch.is_grad_enabled() and (
            x.requires_grad or any(p.requires_grad for p in self.parameters()) or
            any(t.requires_grad for st in cache if st is not None for t in st))
        if not record and x.dtype == torch.float32 and x.dim() == 2 and len(self.layers) > 0:
            # inference: each layer's residual add and the next RMSNorm (the
            # next layer's, or norm_f) in one fused pass
            _, xn = hip_add_rmsnorm(x, None, self.layers[0]["norm"].weight,
                                    self.layers[0]["norm"].eps)
            for i, layer in enumerate(self.layers):
                out, st = layer["mixer"].step(xn, cache[i], compact=compact,
                                              out=None if out_cache is None else out_cache[i])
                new_cache.append(st)
                nxt = self.layers[i + 1]["norm"] if i + 1 < len(self.layers) else (
                    self.norm_f if apply_final_norm else None)
                if nxt is None:
                    x = x + out
                else:
                    x, xn = hip_add_rmsnorm(x, out, nxt.weight, nxt.eps)
            return (xn if apply_final_norm else x), new_cache
        for i, layer in enumerate(self.layers):
            out, st = layer["mixer"].step(layer["norm"](x), cache[i], compact=compact,
                                          out=None if out_cache is None else out_cache[i])
            x = x + out
            new_cache.append(st)
        if apply_final_norm:
            x = self.norm_f(x)
        return x, new_cache

    def prime_cache(self, input_ids, compact=False):
        """Full causal forward returning (norm_f(last hidden), per-layer cache)
        (engine/mamba.py:603-620), the scans on HIP with the final state.
        compact=True keeps each layer's beta in rank-1 rows (see
        Mamba3Block.forward_with_state)."""
        assert not self.config.bidirectional, "prime_cache() requires a causal model"
        cur = self.embedding(input_ids)
        cache = []
        for layer in self.layers:
            mixed, st = layer["mixer"].forward_with_state(layer["norm"](cur), compact=compact)
            cur = cur + mixed
            cache.append(st)
        return self.norm_f(cur[:, -1, :]), cache
