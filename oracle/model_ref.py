"""CPU oracle of the Mamba-3 backbone (engine/mamba.py), fp32, pure PyTorch.

TEST INFRASTRUCTURE ONLY (see oracle/scan_ref.py).  It restates the
reference's modules with the same parameter names, shapes and construction
order, so a `state_dict` moves unchanged between this oracle, the reference
and `redpanda_amd.mamba`.  Every SSM computation goes through the fp32
restatement in `oracle.scan_ref`; everything around it (projections, norms,
residual stack) is the reference's plain torch code path restated.

Covers: MambaConfig (:24-78), RMSNorm (:82-89), Mamba3Block (:141-498),
Mamba (:503-620).  Parity status: pinned by the golden fixtures
(tests/golden/model_*.npz) written by importing the reference.
"""

import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import scan_ref


@dataclass
class MambaConfig:
    """Same fields and derived values as engine/mamba.py:24-78."""
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

    def __init__(self, d, eps=1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight


class Mamba3Block(nn.Module):
    """engine/mamba.py:141-498 restated; the scan/step go through scan_ref."""

    def __init__(self, config):
        super().__init__()
        self.config = config
        d_inner, n = config.d_inner, config.d_state
        n_rot, n_track, p = config.n_rot_state, config.n_track_state, config.mimo_p
        self.in_proj = nn.Linear(config.d_model, 2 * d_inner, bias=config.bias)
        self.x_proj = nn.Linear(d_inner, config.dt_rank + 2 * n * p, bias=True)
        self.dt_proj = nn.Linear(config.dt_rank, d_inner, bias=True)
        with torch.no_grad():  # dt bias init (:172-178): same RNG draw order
            lo, hi = math.log(0.001), math.log(0.1)
            dt0 = torch.exp(torch.rand(d_inner) * (hi - lo) + lo)
            self.dt_proj.bias.copy_(dt0 + torch.log(-torch.expm1(-dt0)))
            self.dt_proj.bias._no_reinit = True
        if n_rot > 0:
            base = torch.arange(1, n_rot + 1, dtype=torch.float32).repeat(d_inner, 1)
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

    def _compute_A(self):
        """engine/mamba.py:211-225."""
        if self.config.n_rot_state == 0:
            return None, None
        if self.config.use_complex:
            mag = -torch.exp(self.A_log_mag.float())
            phase = self.A_phase.float()
            return mag * torch.cos(phase), mag * torch.sin(phase)
        return -torch.exp(self.A_log.float()), None

    def _track_gate(self):
        """engine/mamba.py:227-229."""
        return torch.tanh(self.track_theta.float())

    def _ssm_proj(self, u):
        """engine/mamba.py:284-301."""
        cfg = self.config
        lead = u.shape[:-1]
        n, p = cfg.d_state, cfg.mimo_p
        dt_raw, B_raw, C_raw = self.x_proj(u).split([cfg.dt_rank, n * p, n * p], dim=-1)
        if cfg.use_bcnorm:
            B_raw = self.b_norm(B_raw)
            C_raw = self.c_norm(C_raw)
        return (F.softplus(self.dt_proj(dt_raw)),
                B_raw.view(*lead, n, p), C_raw.view(*lead, n, p))

    def _scan(self, u, delta, A_real, A_imag, B, C, return_state=False):
        cfg = self.config
        track = self._track_gate() if cfg.n_track_state > 0 else None
        ckpt = cfg.scan_checkpoint and self.training
        return scan_ref.selective_scan_ref(u, delta, A_real, A_imag, B, C, self.D,
                                           track, cfg.d_state,
                                           return_state=return_state, checkpoint=ckpt)

    def forward(self, x):
        """engine/mamba.py:231-267."""
        x_branch, z = self.in_proj(x).chunk(2, dim=-1)
        x_branch = F.silu(x_branch)
        delta, B, C = self._ssm_proj(x_branch)
        A_real, A_imag = self._compute_A()
        y = self._scan(x_branch, delta, A_real, A_imag, B, C)
        if self.config.bidirectional:
            y = y + self._scan(x_branch.flip(1), delta.flip(1), A_real, A_imag,
                               B.flip(1), C.flip(1)).flip(1)
        return self.out_proj(y * F.silu(z))

    def forward_with_state(self, x):
        """engine/mamba.py:269-282."""
        x_branch, z = self.in_proj(x).chunk(2, dim=-1)
        x_branch = F.silu(x_branch)
        delta, B, C = self._ssm_proj(x_branch)
        A_real, A_imag = self._compute_A()
        y, state = self._scan(x_branch, delta, A_real, A_imag, B, C, return_state=True)
        return self.out_proj(y * F.silu(z)), state

    def step(self, x_t, state=None):
        """engine/mamba.py:427-498."""
        cfg = self.config
        x_branch, z = self.in_proj(x_t).chunk(2, dim=-1)
        x_branch = F.silu(x_branch)
        delta, B_mat, C_mat = self._ssm_proj(x_branch)
        A_real, A_imag = self._compute_A()
        track = self._track_gate() if cfg.n_track_state > 0 else None
        y, new_state = scan_ref.step_core_ref(delta, x_branch, B_mat.sum(-1), C_mat.sum(-1),
                                              A_real, A_imag, track, self.D, state)
        return self.out_proj(y * F.silu(z)), new_state


class Mamba(nn.Module):
    """engine/mamba.py:503-620."""

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.grad_checkpoint = getattr(config, "grad_checkpoint", False)
        self.embedding = nn.Embedding(config.vocab_size, config.d_model)
        self.layers = nn.ModuleList([
            nn.ModuleDict({"mixer": Mamba3Block(config), "norm": RMSNorm(config.d_model)})
            for _ in range(config.n_layer)])
        self.norm_f = RMSNorm(config.d_model)
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(module):
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None and not getattr(module.bias, "_no_reinit", False):
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(self, input_ids, input_embeds=None):
        x = input_embeds if input_embeds is not None else self.embedding(input_ids)
        for layer in self.layers:
            x = x + layer["mixer"](layer["norm"](x))
        return self.norm_f(x)

    def step(self, token_id=None, cache=None, input_embed=None, apply_final_norm=True):
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
        for i, layer in enumerate(self.layers):
            out, st = layer["mixer"].step(layer["norm"](x), cache[i])
            x = x + out
            new_cache.append(st)
        if apply_final_norm:
            x = self.norm_f(x)
        return x, new_cache

    def prime_cache(self, input_ids):
        assert not self.config.bidirectional, "prime_cache() requires a causal model"
        cur = self.embedding(input_ids)
        cache = []
        for layer in self.layers:
            mixed, st = layer["mixer"].forward_with_state(layer["norm"](cur))
            cur = cur + mixed
            cache.append(st)
        return self.norm_f(cur[:, -1, :]), cache
