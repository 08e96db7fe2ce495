"""Host boundary of a lockstep rollout ply: pinned buffers and one sync per ply.

The reference's batched MARS rollout (engine/mars_search.py:_rollout_batch,
:_rollout_batch_fast) crosses the host/device boundary once per rollout per
ply:
  * the step's tokens go up as `torch.tensor(tokens, device=...)` from a
    Python list (:442, :553), a pageable copy;
  * every rollout's continuation row comes down on its own in _select_move
    (`cont_logits.float().cpu().numpy()`, :262), to pick from its top-k, or
    in _select_fc_move as a gather of its legal moves' logits (:475);
  * the ply's values come down as `vals.detach().cpu().tolist()` (:446, :556).
With R rollouts that is R + 2 synchronising copies per ply.  `PlyBoundary`
replaces them with one asynchronous upload from a pinned buffer, the
reductions of rp_ply_topk / rp_ply_gather on the device, and one download
into a pinned buffer with one event wait.

What reaches the host is what the reference computes from the full rows:
_select_move's candidate list is the row's top-k logits in descending order
(np.argpartition, then np.argsort(...)[::-1]; ties ordered here by ascending
token id), and _select_fc_move's values are the gathered logits.
`select_policy_move` restates _select_move's policy-guided walk over that
candidate list, so a caller keeps the reference's move choice.
"""

import ctypes

import numpy as np
import torch

from redpanda_amd import _lib


def _code(t):
    try:
        return _lib.DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"redpanda_amd ply: unsupported logits dtype {t.dtype}") from None


def _rows(t, name):
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"ply: {name} must be 2-D with unit inner stride, got {tuple(t.shape)} "
                         f"strides {t.stride()}")
    return t


def ply_topk(logits, k, values=None, out=None):
    """(R, 1 + 2k) fp32 words on the device: per row the value (word 0),
    the k largest logits (words 1..k) and their token ids as int32 bits
    (words k+1..2k).  logits: (R, V) fp32 / bf16 / fp16; values: (R,) or
    None.  `out` may be given (R, >= 2k+1) fp32 contiguous rows."""
    lib = _lib.load()
    _rows(logits, "logits")
    R, V = logits.shape
    if out is None:
        out = torch.empty((R, 2 * k + 1), dtype=torch.float32, device=logits.device)
    a = _lib.PlyTopkArgs(R=R, V=V, k=k, dtype_logits=_code(logits), logits=logits.data_ptr(),
                         logits_sr=logits.stride(0), out=out.data_ptr(), out_sr=out.stride(0))
    if values is not None:
        values = values.reshape(R).to(torch.float32).contiguous()
        a.values = values.data_ptr()
    _lib.check(lib.rp_ply_topk(ctypes.byref(a), _lib.stream_of(logits.device)), lib)
    return out


def ply_gather(logits, tokens, out=None):
    """(R, M) fp32: logits[r, tokens[r, j]], -inf for ids outside [0, V).
    tokens: (R, M) int32 on the device."""
    lib = _lib.load()
    _rows(logits, "logits")
    _rows(tokens, "tokens")
    if tokens.dtype != torch.int32:
        raise TypeError("ply gather: tokens must be int32")
    R, V = logits.shape
    M = tokens.shape[1]
    if tokens.shape[0] != R:
        raise ValueError(f"ply gather: tokens {tuple(tokens.shape)} vs logits {tuple(logits.shape)}")
    if out is None:
        out = torch.empty((R, M), dtype=torch.float32, device=logits.device)
    a = _lib.PlyGatherArgs(R=R, V=V, M=M, dtype_logits=_code(logits), logits=logits.data_ptr(),
                           logits_sr=logits.stride(0), tokens=tokens.data_ptr(),
                           tokens_sr=tokens.stride(0), out=out.data_ptr(), out_sr=out.stride(0))
    _lib.check(lib.rp_ply_gather(ctypes.byref(a), _lib.stream_of(logits.device)), lib)
    return out


class PlyBoundary:
    """Pinned staging for the per-ply transfers of R lockstep rollouts.

    push_tokens(tokens)      -> (R,) int64 device tensor (one async upload)
    pull(values, cont)       -> (values (R,), top ids (R, k), top logits (R, k))
    pull_legal(cont, tokens) -> (R, M) fp32 logits of each rollout's move list
    Each pull is one device-to-host copy and one event wait.  The arrays a
    pull returns are views of the pinned buffers, valid until the next pull.
    """

    def __init__(self, rollouts, top_k=8, device="cuda", max_legal=256):
        if not 1 <= top_k <= 16:
            raise ValueError("PlyBoundary: top_k must be in [1, 16]")
        self.R, self.k, self.device = int(rollouts), int(top_k), torch.device(device)
        self.max_legal = int(max_legal)
        R, k = self.R, self.k
        self._tok_h = torch.empty(R, dtype=torch.int64, pin_memory=True)
        self._tok_d = torch.empty(R, dtype=torch.int64, device=self.device)
        self._pack_d = torch.empty((R, 2 * k + 1), dtype=torch.float32, device=self.device)
        self._pack_h = torch.empty((R, 2 * k + 1), dtype=torch.float32, pin_memory=True)
        self._leg_h = torch.empty((R, self.max_legal), dtype=torch.int32, pin_memory=True)
        self._leg_d = torch.empty((R, self.max_legal), dtype=torch.int32, device=self.device)
        self._lout_d = torch.empty((R, self.max_legal), dtype=torch.float32, device=self.device)
        self._lout_h = torch.empty((R, self.max_legal), dtype=torch.float32, pin_memory=True)
        self._event = torch.cuda.Event()
        self._tok_event = torch.cuda.Event()
        self._tok_event.record()

    def push_tokens(self, tokens):
        """The step's token ids (R ints) on the device, from the pinned
        buffer (replaces torch.tensor(tokens, device=...)).  The pinned
        buffer is rewritten only after the previous upload from it is done."""
        self._tok_event.synchronize()
        self._tok_h.numpy()[:] = np.asarray(tokens, dtype=np.int64)
        self._tok_d.copy_(self._tok_h, non_blocking=True)
        self._tok_event.record()
        return self._tok_d

    def pull(self, values, cont):
        """values: (R,) or (R, 1) device tensor; cont: (R, V) continuation
        logits.  Returns numpy views (values fp32, top ids int32, top logits
        fp32), each rollout's candidates largest logit first."""
        if cont.shape[0] != self.R:
            raise ValueError(f"PlyBoundary.pull: {cont.shape[0]} rows, expected {self.R}")
        ply_topk(cont, self.k, values=values, out=self._pack_d)
        self._pack_h.copy_(self._pack_d, non_blocking=True)
        self._event.record()
        self._event.synchronize()
        h = self._pack_h.numpy()
        k = self.k
        return h[:, 0], h[:, k + 1:].view(np.int32), h[:, 1:k + 1]

    def pull_legal(self, cont, tokens):
        """tokens: (R, M) ints (M <= max_legal), each row a rollout's legal
        move ids padded with -1.  Returns the (R, M) fp32 logits view
        (-inf at the padding)."""
        tokens = np.asarray(tokens)
        R, M = tokens.shape
        if R != self.R or M > self.max_legal:
            raise ValueError(f"PlyBoundary.pull_legal: tokens {tokens.shape}, expected ({self.R}, "
                             f"<= {self.max_legal})")
        # (R, M) views of the flat buffers, contiguous, so each copy is one
        # contiguous transfer
        n = R * M
        leg_h = self._leg_h.view(-1)[:n].view(R, M)
        leg_d = self._leg_d.view(-1)[:n].view(R, M)
        lout_d = self._lout_d.view(-1)[:n].view(R, M)
        lout_h = self._lout_h.view(-1)[:n].view(R, M)
        leg_h.numpy()[:] = tokens
        leg_d.copy_(leg_h, non_blocking=True)
        ply_gather(cont, leg_d, out=lout_d)
        lout_h.copy_(lout_d, non_blocking=True)
        self._event.record()
        self._event.synchronize()
        return lout_h.numpy()


def select_policy_move(top_ids, top_logits, is_legal, rollout_temp, rng=np.random):
    """_select_move's policy-guided walk (engine/mars_search.py:261-276) over
    one rollout's candidate list: the first legal id when rollout_temp <=
    1e-3, else a softmax draw over the legal candidates' logits / temp.
    is_legal(token_id) -> bool decides legality (the reference decodes the id
    and asks the board).  Returns the chosen id, or None when no candidate is
    legal (the reference then enumerates every legal move)."""
    cand = []
    for mid, lg in zip(top_ids, top_logits):
        mid = int(mid)
        if mid < 0 or not is_legal(mid):
            continue
        if rollout_temp <= 1e-3:
            return mid
        cand.append((mid, float(lg)))
    if not cand:
        return None
    lg = np.array([c[1] for c in cand]) / rollout_temp
    lg -= lg.max()
    pr = np.exp(lg)
    pr /= pr.sum()
    return cand[int(rng.choice(len(cand), p=pr))][0]
