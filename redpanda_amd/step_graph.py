"""A fixed-size batched step() captured into HIP graphs and replayed per ply.

At the rollout counts MARS runs (survivors x simulations, a few to a few
hundred rows: engine/mars_search.py:59, :440-449), one Mamba.step ply is
bound by the host: each of the n_layer layers issues seven launches from
Python (four projections, the SiLU, the fused step with BCNorm in its
prologue, the residual add + RMSNorm), about 1.3 ms per ply for 8 layers up
to 512 rows, against 8-43 us of step kernel per layer.  StepGraph records
one ply of Mamba.step for a fixed batch once and replays it: every launch of
the ply is issued by one graph launch.

The state lives in two static cache sets that the two captured graphs use in
turn (graph 0 reads set 0 and writes set 1, graph 1 the reverse), so a ply
moves the state once, as the eager step does.  The gates (A_real, A_imag,
tanh(theta)) depend on the parameters only: the graphs read them from static
buffers, which a call refreshes outside the graph, with the eager step's
own values, when a gate parameter has changed (its storage or version
counter); computing them inside the graph took seven small kernels per
layer in every replay.  The values are those of Mamba.step with the same
inputs and state (the same kernels in the same order); the returned hidden
rows and cache are the graph's buffers, valid until the next call (clone
them to keep them).  Inference only (no autograd graph is recorded).  The
graphs read the model's parameters in place, so an in-place update (an
optimizer step, load_state_dict) reaches the next replay; a model moved or
re-created needs a new StepGraph.
"""

import torch

from redpanda_amd.step import is_compact


class StepGraph:
    """Mamba.step(token_id=..., or input_embed=...) for `rollouts` rows.

    model: a causal redpanda_amd.mamba.Mamba (or SearchMamba's backbone) on
    the GPU; rollouts: the fixed batch; compact: rank-1 beta rows in the
    cache; embed: the ply's input is an (R, d_model) fp32 embedding instead
    of (R,) token ids; apply_final_norm as in Mamba.step.
    """

    def __init__(self, model, rollouts, compact=False, embed=False, apply_final_norm=True,
                 warmup=2):
        if model.config.bidirectional:
            raise ValueError("StepGraph: step() requires a causal model")
        p = next(model.parameters())
        if not p.is_cuda:
            raise RuntimeError("StepGraph: the model must be on a ROCm device")
        cfg = model.config
        dev = p.device
        R, D, N = int(rollouts), cfg.d_inner, cfg.d_state
        self.model, self.R, self.compact, self.embed = model, R, bool(compact), bool(embed)
        self.apply_final_norm = apply_final_norm
        f32 = dict(dtype=torch.float32, device=dev)
        if self.embed:
            self.inp = torch.zeros((R, cfg.d_model), **f32)
        else:
            self.inp = torch.zeros((R,), dtype=torch.long, device=dev)
        bshape = (R, D + N) if self.compact else (R, D, N)
        self.sets = [[(torch.zeros((R, D, N), **f32), torch.zeros(bshape, **f32))
                      for _ in range(cfg.n_layer)] for _ in range(2)]
        self.cur = 0
        self.graphs, self.hidden = [], []
        # static gate buffers per layer, read by the graphs
        self.mixers = [layer["mixer"] for layer in model.layers]
        with torch.no_grad():
            self.gates = [tuple(None if g is None else g.detach().clone() for g in mx._gates(False))
                          for mx in self.mixers]
        self.gate_key = self._gate_key()
        for mx, g in zip(self.mixers, self.gates):
            mx.__dict__["_gates_fixed"] = g
        try:
            self._capture(dev, warmup)
        finally:
            for mx in self.mixers:
                mx.__dict__.pop("_gates_fixed", None)
        self.reset()

    def _gate_key(self):
        return tuple((t.data_ptr(), t._version) for mx in self.mixers for t in mx._gate_params())

    def _refresh_gates(self):
        """The static gate buffers from the eager step's values, when a gate
        parameter has changed since they were filled."""
        key = self._gate_key()
        if key == self.gate_key:
            return
        with torch.no_grad():
            for mx, bufs in zip(self.mixers, self.gates):
                for b, g in zip(bufs, mx._gates(False)):
                    if b is not None:
                        b.copy_(g)
        self.gate_key = key

    def _capture(self, dev, warmup):
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.no_grad(), torch.cuda.stream(side):
            for _ in range(max(int(warmup), 1)):  # first-call work happens outside capture
                for k in range(2):
                    self._ply(k)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        pool = None
        with torch.no_grad():
            for k in range(2):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=pool):
                    h = self._ply(k)
                pool = g.pool()
                self.graphs.append(g)
                self.hidden.append(h)

    def _ply(self, k):
        kw = {"input_embed": self.inp} if self.embed else {"token_id": self.inp}
        h, _ = self.model.step(cache=self.sets[k], out_cache=self.sets[1 - k],
                               apply_final_norm=self.apply_final_norm, compact=self.compact, **kw)
        return h

    @property
    def cache(self):
        """The current state: per-layer (h, beta), the graph's buffers."""
        return self.sets[self.cur]

    def reset(self):
        """A fresh state (zeros: the same values as step() from no cache)."""
        for h, b in self.sets[self.cur]:
            h.zero_()
            b.zero_()

    def load(self, cache):
        """Copy a cache (per-layer (h, beta) of this batch and form, e.g. from
        prime_cache) into the current state."""
        if len(cache) != len(self.sets[0]):
            raise ValueError("StepGraph.load: one (h, beta) per layer expected")
        for (h, b), (hs, bs) in zip(self.sets[self.cur], cache):
            if is_compact(bs) != self.compact or hs.shape != h.shape or bs.shape != b.shape:
                raise ValueError(f"StepGraph.load: state must be h {tuple(h.shape)} and beta "
                                 f"{tuple(b.shape)}")
            h.copy_(hs)
            b.copy_(bs)

    def __call__(self, token_id=None, input_embed=None):
        """One ply: (hidden (R, d_model), cache), both the graph's buffers."""
        x = input_embed if self.embed else token_id
        if x is None:
            raise ValueError("StepGraph: give " + ("input_embed" if self.embed else "token_id"))
        if not self.embed and x.dim() == 2:
            x = x.squeeze(1)
        if x.shape != self.inp.shape:
            raise ValueError(f"StepGraph: input {tuple(x.shape)} must be {tuple(self.inp.shape)}")
        self.inp.copy_(x)
        self._refresh_gates()
        k = self.cur
        self.graphs[k].replay()
        self.cur = 1 - k
        return self.hidden[k], self.sets[self.cur]
