"""Search Mamba: the causal rollout model MARS advances with O(1) steps.

API- and state_dict-compatible with the reference's engine/search_mamba.py
(SearchMambaConfig :24-36, SearchMamba :39-384) over the HIP backbone in
redpanda_amd.mamba: prime_board (one causal scan returning the cache, on the
HIP scan kernel), _expand_cache, eval_step / backbone.step (the fused step
kernel), dynamics_rollout (trains through step via the scan kernel's analytic
backward), and the line-evaluation helpers.  The heads are plain torch
modules with the reference's names and init.
"""

import json
from dataclasses import asdict
from dataclasses import fields as dc_fields

import torch
import torch.nn as nn

from redpanda_amd.mamba import Mamba, MambaConfig


class SearchMambaConfig(MambaConfig):
    """engine/search_mamba.py:24-36.  Deliberately NOT re-decorated as a
    dataclass, like the reference: the generated __init__ is MambaConfig's,
    so an instance built without arguments carries MambaConfig's defaults
    (d_model 512, 16 layers, d_state 64, mimo_p 4), and the class-level
    values below only show through attribute lookup on the class."""
    d_model: int = 384
    n_layer: int = 12
    d_state: int = 32
    expand: int = 2
    use_complex: bool = True
    mimo_p: int = 2
    use_bcnorm: bool = True


class SearchMamba(nn.Module):
    """Causal value-equivalent dynamics model (engine/search_mamba.py:39-384)."""

    def __init__(self, config: SearchMambaConfig = None, vocab_size: int = 8192,
                 eval_dim: int = 512):
        super().__init__()
        if config is None:
            config = SearchMambaConfig(vocab_size=vocab_size)
        config.bidirectional = False  # the rollout model must be causal
        self.config = config
        self.eval_dim = eval_dim
        self.backbone = Mamba(config)
        d = config.d_model
        self.line_value_head = nn.Sequential(
            nn.Linear(d, d), nn.GELU(), nn.LayerNorm(d),
            nn.Linear(d, d // 2), nn.GELU(), nn.Linear(d // 2, 1))
        self.value_head = nn.Sequential(
            nn.Linear(d, d), nn.GELU(), nn.LayerNorm(d), nn.Linear(d, 1))
        self.continuation_head = nn.Sequential(
            nn.Linear(d, d * 2), nn.GELU(), nn.LayerNorm(d * 2),
            nn.Linear(d * 2, config.vocab_size))
        self.consistency_proj = nn.Sequential(
            nn.Linear(d, d), nn.GELU(), nn.Linear(d, eval_dim))
        self.apply(self._init_weights)

    def _init_weights(self, m):
        if isinstance(m, nn.Linear):
            nn.init.orthogonal_(m.weight, gain=1.0)
            if m.bias is not None:
                nn.init.constant_(m.bias, 0)

    def _device(self):
        return next(self.parameters()).device

    # ── whole-sequence scoring (one causal scan per line) ──

    def forward(self, board_encoding, move_sequences):
        """(B, L_board) + (B, L_moves) token ids -> (B,) line scores."""
        hidden = self.backbone(torch.cat([board_encoding, move_sequences], dim=-1))
        return self.line_value_head(hidden[:, -1, :]).squeeze(-1)

    def evaluate_lines(self, board_encoding, move_sequences):
        if board_encoding.dim() == 1:
            board_encoding = board_encoding.unsqueeze(0)
        k = move_sequences.shape[0]
        return self.forward(board_encoding.expand(k, -1), move_sequences)

    def evaluate_with_continuation(self, board_encoding, move_sequences):
        if board_encoding.dim() == 1:
            board_encoding = board_encoding.unsqueeze(0)
        k = move_sequences.shape[0]
        full = torch.cat([board_encoding.expand(k, -1), move_sequences], dim=-1)
        final = self.backbone(full)[:, -1, :]
        return self.line_value_head(final).squeeze(-1), self.continuation_head(final)

    # ── O(1) cached evaluation ──

    def prime_board(self, board_encoding, compact=False):
        """Encode one board (ids (L,) or (1, L), list or tensor) and return
        (final_hidden, cache) for step() (engine/search_mamba.py:162-175).
        compact=True keeps each layer's beta in rank-1 rows [dt*u | B]
        (half the state bytes per step; same results)."""
        if not torch.is_tensor(board_encoding):
            board_encoding = torch.as_tensor(board_encoding, dtype=torch.long,
                                             device=self._device())
        if board_encoding.dim() == 1:
            board_encoding = board_encoding.unsqueeze(0)
        return self.backbone.prime_cache(board_encoding, compact=compact)

    @staticmethod
    def _expand_cache(cache, k):
        """Broadcast a batch-1 cache to k rows (engine/search_mamba.py:177-187).

        The reference materialises k copies (expand().contiguous()); here the
        rows are stride-0 views of the one state, which the step kernel reads
        in place, and every step returns fresh per-row states.  Callers that
        clone or concatenate the cache get contiguous tensors as before; an
        in-place write into the returned views is not supported (torch
        rejects it)."""
        return [(h.expand(k, *h.shape[1:]), b.expand(k, *b.shape[1:])) for h, b in cache]

    @torch.no_grad()
    def evaluate_lines_fast(self, board_encoding, move_sequences, lengths=None):
        """K lines from one board: prime once, then step every line in lockstep."""
        device = self._device()
        _, cache = self.prime_board(board_encoding.to(device))
        k, L = move_sequences.shape
        move_sequences = move_sequences.to(device)
        cache = self._expand_cache(cache, k)
        hiddens = []
        for t in range(L):
            hidden, cache = self.backbone.step(token_id=move_sequences[:, t], cache=cache)
            hiddens.append(hidden)
        hiddens = torch.stack(hiddens, dim=1)
        if lengths is not None:
            idx = (lengths.to(device).clamp(min=1) - 1).view(k, 1, 1).expand(-1, 1, hiddens.shape[-1])
            final = hiddens.gather(1, idx).squeeze(1)
        else:
            final = hiddens[:, -1, :]
        return self.line_value_head(final).squeeze(-1)

    @torch.no_grad()
    def score_branch(self, board_cache, move_sequence):
        device = self._device()
        cache = self._expand_cache(board_cache, 1)
        hidden = None
        for tok in move_sequence:
            hidden, cache = self.backbone.step(
                token_id=torch.tensor([int(tok)], device=device), cache=cache)
        quality = self.line_value_head(hidden).squeeze(-1)
        return quality.item(), self.continuation_head(hidden).squeeze(0)

    def dynamics_rollout(self, board_encoding, move_tokens):
        """Differentiable: prime on (B, L_board), step through (B, T) moves;
        returns per-step values (B, T), continuation logits (B, T, vocab) and
        consistency features (B, T, eval_dim) (engine/search_mamba.py:252-273)."""
        _, cache = self.backbone.prime_cache(board_encoding)
        vs, cs, fs = [], [], []
        for t in range(move_tokens.shape[1]):
            h, cache = self.backbone.step(token_id=move_tokens[:, t], cache=cache)
            vs.append(torch.tanh(self.value_head(h)).squeeze(-1))
            cs.append(self.continuation_head(h))
            fs.append(self.consistency_proj(h))
        return torch.stack(vs, 1), torch.stack(cs, 1), torch.stack(fs, 1)

    @torch.no_grad()
    def eval_step(self, cache, move_token):
        """One O(1) node evaluation: (value, continuation logits, new cache)."""
        tok = torch.tensor([int(move_token)], device=self._device())
        h, cache = self.backbone.step(token_id=tok, cache=cache)
        value = torch.tanh(self.value_head(h)).squeeze(-1).item()
        return value, self.continuation_head(h).squeeze(0), cache

    # ── checkpoints: state_dict + JSON config, loaded with weights_only=True ──

    @staticmethod
    def _config_path(path):
        cp = path.replace(".pt", "_config.json").replace(".pth", "_config.json")
        return path + ".config.json" if cp == path else cp

    def save_pretrained(self, path):
        torch.save(self.state_dict(), path)
        cfg = asdict(self.config)
        cfg["eval_dim"] = self.eval_dim
        with open(self._config_path(path), "w") as fh:
            json.dump(cfg, fh, indent=2)

    @classmethod
    def from_pretrained(cls, path, device="cpu", config=None):
        eval_dim = 512
        if config is None:
            with open(cls._config_path(path)) as fh:
                cfg = json.load(fh)
            eval_dim = int(cfg.get("eval_dim", 512))
            valid = {f.name for f in dc_fields(SearchMambaConfig)}
            config = SearchMambaConfig(**{k: v for k, v in cfg.items() if k in valid})
        model = cls(config, eval_dim=eval_dim)
        model.load_state_dict(torch.load(path, map_location=device, weights_only=True))
        return model

