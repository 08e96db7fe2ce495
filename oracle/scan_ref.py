"""CPU oracle for the trapezoidal selective scan and the O(1) recurrent step.

TEST INFRASTRUCTURE ONLY. Nothing in the `redpanda_amd` package imports this
module; only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` use it, and only as the checker (or, for the CPU baseline, as the
timed restatement of the reference's CPU path).

Two independent restatements of the same recurrence live here:

1. `selective_scan_ref` / `scan_chunk_ref` / `hillis_steele_scan` /
   `step_core_ref` — an fp32, op-for-op restatement of the reference's
   PyTorch path (engine/mamba.py:104-136, :318-423, :466-494).  Same tensor
   ops in the same association, so on the same torch build it reproduces the
   reference's fp32 bits; the golden fixtures under tests/golden/ (written by
   importing the reference once in the build container) pin that.
2. `scan_sequential` / `scan_adjoint` — a float64 sequential recurrence and its
   hand-derived reverse-time adjoint (engine/triton_scan.py:7-12, :208-237).
   These are pinned by closed forms (g == 1, g == 0, L == 1, geometric series,
   Tk == -1 parity flip), by torch.autograd through the float64 loop, and by
   torch.autograd.gradcheck (finite differences) on tiny shapes.

Notation (one lane = one (b, d) channel, vector over the state index n):
    g_t[n]  = exp(dt_t * Ar[n]) * cos(dt_t * Ai[n])   n <  NR (rotational)
            = Tk[n] = tanh(theta[n])                  n >= NR (tracking)
    beta_t  = dt_t * B_t[n] * u_t
    h_t     = g_t * h_{t-1} + 0.5 * beta_t + 0.5 * g_t * beta_{t-1}
    y_t     = sum_n h_t[n] * C_t[n]      (no D-skip; the caller adds u * D)

Parity status: every function here is pinned (see tests/test_oracle.py).
"""

import torch

# Chunk length of the reference's streaming scan (engine/mamba.py:101).
SCAN_CHUNK = 32


# ─── 1. fp32 op-for-op restatement of the reference PyTorch path ────────────

def hillis_steele_scan(gates, tokens):
    """Inclusive scan of h[t] = gates[t] * h[t-1] + tokens[t] along dim 1.

    Follows engine/mamba.py:104-136: log2(L) doubling rounds, each rebuilding
    the token and gate tensors with torch.cat (same association as the
    reference, so the fp32 rounding matches it exactly).
    """
    acc_g, acc_t = gates, tokens
    span = 1
    length = acc_g.shape[1]
    while span < length:
        head_t = acc_t[:, :span]
        tail_t = acc_g[:, span:] * acc_t[:, :-span] + acc_t[:, span:]
        acc_t = torch.cat([head_t, tail_t], dim=1)
        head_g = acc_g[:, :span]
        tail_g = acc_g[:, span:] * acc_g[:, :-span]
        acc_g = torch.cat([head_g, tail_g], dim=1)
        span *= 2
    return acc_t


def gate_tensor_ref(delta_c, A_real, A_imag, track):
    """Per-step gates (B, c, D, N) exactly as engine/mamba.py:396-405 builds them."""
    parts = []
    if A_real is not None:
        decay = torch.exp(torch.einsum("bld,dn->bldn", delta_c, A_real))
        if A_imag is not None:
            decay = decay * torch.cos(torch.einsum("bld,dn->bldn", delta_c, A_imag))
        parts.append(decay)
    if track is not None:
        b, c, d = delta_c.shape
        parts.append(track.view(1, 1, d, -1).expand(b, c, d, -1))
    return parts[0] if len(parts) == 1 else torch.cat(parts, dim=-1)


def scan_chunk_ref(delta_c, u_c, B_c, C_c, h, beta_prev, A_real, A_imag, track):
    """One chunk of the streaming scan (engine/mamba.py:382-423).

    Returns (y_c (B,c,D), h_last (B,D,N), beta_last (B,D,N)).
    """
    gates = gate_tensor_ref(delta_c, A_real, A_imag, track)
    # beta = (dt * B) * u  — the scan's association (engine/mamba.py:408)
    beta = torch.einsum("bld,bln->bldn", delta_c, B_c) * u_c.unsqueeze(-1)
    if beta_prev is None:
        beta_prev = torch.zeros_like(beta[:, 0])
    beta_shift = torch.cat([beta_prev.unsqueeze(1), beta[:, :-1]], dim=1)
    tokens = 0.5 * beta + 0.5 * gates * beta_shift
    # carry folded into the first token (engine/mamba.py:418-419)
    first = tokens[:, 0] + gates[:, 0] * h.to(gates.dtype)
    tokens = torch.cat([first.unsqueeze(1), tokens[:, 1:]], dim=1)
    hs = hillis_steele_scan(gates, tokens)
    y_c = torch.einsum("bldn,bln->bld", hs, C_c)
    return y_c, hs[:, -1], beta[:, -1]


def selective_scan_ref(u, delta, A_real, A_imag, B, C, D, track, n_state,
                       return_state=False, checkpoint=False):
    """The reference's CPU scan dispatcher (engine/mamba.py:318-380), fp32.

    u, delta: (B, L, D); B, C: (B, L, N, p) MIMO (contracted over p here,
    :336-337); A_real/A_imag: (D, NR) or None; track: (D, NT) tanh gates or
    None; D: (D,) skip.  Returns y (B, L, D) including u * D, and optionally
    the (h_last, beta_last) state that step() continues from (:377-379).
    `checkpoint` recomputes each chunk in backward like scan_checkpoint=True
    (:358-370); the values are identical either way.
    """
    batch, L, d_inner = u.shape
    Bc = B.sum(dim=-1)
    Cc = C.sum(dim=-1)
    h = torch.zeros((batch, d_inner, n_state), dtype=torch.float32, device=u.device)
    beta_last = None
    outs = []
    for s in range(0, L, SCAN_CHUNK):
        e = min(s + SCAN_CHUNK, L)
        args = (delta[:, s:e], u[:, s:e], Bc[:, s:e], Cc[:, s:e], h, beta_last,
                A_real, A_imag, track)
        if checkpoint and torch.is_grad_enabled():
            y_c, h, beta_last = torch.utils.checkpoint.checkpoint(
                scan_chunk_ref, *args, use_reentrant=False)
        else:
            y_c, h, beta_last = scan_chunk_ref(*args)
        outs.append(y_c)
    y = torch.cat(outs, dim=1) + u * D
    if return_state:
        return y, (h, beta_last)
    return y


def contracted_scan_ref(delta, u, Bc, Cc, A_real, A_imag, track, n_state, checkpoint=False):
    """The chunk loop alone on contracted B/C, WITHOUT the D-skip.

    This is exactly what the reference's kernel entry replaces
    (engine/triton_scan.py:318-337 is documented as a drop-in for the chunk
    loop of engine/mamba.py:360-373).  `checkpoint` recomputes each chunk in
    backward as scan_checkpoint=True does in training (:358-370).
    """
    batch, L, d_inner = u.shape
    h = torch.zeros((batch, d_inner, n_state), dtype=torch.float32, device=u.device)
    beta_last = None
    outs = []
    for s in range(0, L, SCAN_CHUNK):
        e = min(s + SCAN_CHUNK, L)
        args = (delta[:, s:e], u[:, s:e], Bc[:, s:e], Cc[:, s:e], h, beta_last,
                A_real, A_imag, track)
        if checkpoint and torch.is_grad_enabled():
            y_c, h, beta_last = torch.utils.checkpoint.checkpoint(
                scan_chunk_ref, *args, use_reentrant=False)
        else:
            y_c, h, beta_last = scan_chunk_ref(*args)
        outs.append(y_c)
    return torch.cat(outs, dim=1), (h, beta_last)


def step_core_ref(delta, u, Bc, Cc, A_real, A_imag, track, D, state):
    """SSM core of Mamba3Block.step (engine/mamba.py:466-494), fp32.

    delta, u: (B, D_inner); Bc, Cc: (B, N) contracted; state (h, beta_prev)
    (B, D_inner, N) or None.  Returns (y (B, D_inner) incl. u*D, (h, beta_t)).
    Note the step's association beta_t = (dt * u) * B (:481), which differs
    from the scan's (dt * B) * u (:408).
    """
    batch, d_inner = delta.shape
    parts = []
    if A_real is not None:
        decay = torch.exp(delta.unsqueeze(-1) * A_real.unsqueeze(0))
        if A_imag is not None:
            decay = decay * torch.cos(delta.unsqueeze(-1) * A_imag.unsqueeze(0))
        parts.append(decay)
    if track is not None:
        parts.append(track.unsqueeze(0).expand(batch, d_inner, -1))
    gates = parts[0] if len(parts) == 1 else torch.cat(parts, dim=-1)
    beta_t = (delta * u).unsqueeze(-1) * Bc.unsqueeze(1)
    if state is None:
        h = torch.zeros(batch, d_inner, Bc.shape[-1], dtype=beta_t.dtype, device=beta_t.device)
        beta_prev = torch.zeros_like(beta_t)
    else:
        h, beta_prev = state
    tokens = 0.5 * beta_t + 0.5 * gates * beta_prev
    h = gates * h + tokens
    y = torch.einsum("bdn,bn->bd", h, Cc)
    y = y + u * D
    return y, (h, beta_t)


# ─── 2. float64 sequential recurrence and its analytic adjoint ──────────────

def _gates64(dt, Ar, Ai, Tk):
    """g (..., N) for per-channel dt (...,) ; Ar/Ai (D, NR) ; Tk (D, NT)."""
    parts = []
    if Ar is not None and Ar.shape[-1] > 0:
        x = dt.unsqueeze(-1) * Ar
        g = torch.exp(x)
        if Ai is not None:
            g = g * torch.cos(dt.unsqueeze(-1) * Ai)
        parts.append(g)
    if Tk is not None and Tk.shape[-1] > 0:
        parts.append(Tk.expand(*dt.shape, Tk.shape[-1]))
    return torch.cat(parts, dim=-1) if len(parts) > 1 else parts[0]


def scan_sequential(delta, u, Bc, Cc, Ar, Ai, Tk, h0=None, beta0=None, reverse=False):
    """float64 sequential trapezoidal scan on contracted inputs.

    delta, u: (B, L, D); Bc, Cc: (B, L, N); Ar, Ai: (D, NR) or None;
    Tk: (D, NT) or None.  `reverse` runs the recurrence from t = L-1 down to 0
    (the reversed direction of the bidirectional layer, expressed in original
    time order).  Returns (y (B,L,D) without skip, h_last, beta_last).
    Differentiable with torch.autograd (used to pin `scan_adjoint`).
    """
    f = lambda t: None if t is None else t.to(torch.float64)
    delta, u, Bc, Cc, Ar, Ai, Tk = map(f, (delta, u, Bc, Cc, Ar, Ai, Tk))
    batch, L, d_inner = u.shape
    n = Bc.shape[-1]
    z64 = dict(dtype=torch.float64, device=u.device)
    h = torch.zeros(batch, d_inner, n, **z64) if h0 is None else f(h0)
    bp = torch.zeros(batch, d_inner, n, **z64) if beta0 is None else f(beta0)
    ys = [None] * L
    order = range(L - 1, -1, -1) if reverse else range(L)
    for t in order:
        g = _gates64(delta[:, t], Ar, Ai, Tk)
        beta = (delta[:, t] * u[:, t]).unsqueeze(-1) * Bc[:, t].unsqueeze(1)
        h = g * h + 0.5 * beta + 0.5 * g * bp
        bp = beta
        ys[t] = (h * Cc[:, t].unsqueeze(1)).sum(-1)
    return torch.stack(ys, dim=1), h, bp


def scan_adjoint(delta, u, Bc, Cc, Ar, Ai, Tk, dy, reverse=False):
    """Hand-derived reverse-time adjoint of `scan_sequential` in float64.

    Follows the recurrence of engine/triton_scan.py:208-237:
        q_t   = dy_t C_t + g_{t+1} q_{t+1}
        dg_t  = q_t (h_{t-1} + beta_{t-1} / 2)
        dbeta = q_t / 2 + g_{t+1} q_{t+1} / 2
    Returns dict of float64 grads: delta, u, Bc, Cc (B,L,·), Ar, Ai (D,NR),
    Tk (D,NT).
    """
    f = lambda t: None if t is None else t.to(torch.float64)
    delta, u, Bc, Cc, Ar, Ai, Tk, dy = map(f, (delta, u, Bc, Cc, Ar, Ai, Tk, dy))
    batch, L, d_inner = u.shape
    n = Bc.shape[-1]
    nr = 0 if Ar is None else Ar.shape[-1]
    order = list(range(L - 1, -1, -1)) if reverse else list(range(L))
    # forward sweep: keep every h_t (float64, small shapes only)
    hs, betas, gs = {}, {}, {}
    z64 = dict(dtype=torch.float64, device=u.device)
    h = torch.zeros(batch, d_inner, n, **z64)
    bp = torch.zeros_like(h)
    prev = None
    for t in order:
        g = _gates64(delta[:, t], Ar, Ai, Tk)
        beta = (delta[:, t] * u[:, t]).unsqueeze(-1) * Bc[:, t].unsqueeze(1)
        h = g * h + 0.5 * beta + 0.5 * g * bp
        hs[t], betas[t], gs[t] = h, beta, g
        bp = beta
    zeros = torch.zeros(batch, d_inner, n, **z64)
    d_delta = torch.zeros_like(delta)
    d_u = torch.zeros_like(u)
    d_B = torch.zeros_like(Bc)
    d_C = torch.zeros_like(Cc)
    d_Ar = torch.zeros(d_inner, nr, **z64)
    d_Ai = torch.zeros(d_inner, nr, **z64)
    d_Tk = torch.zeros(d_inner, n - nr, **z64)
    gq_next = zeros          # g_{t+1} q_{t+1}
    for k in range(L - 1, -1, -1):
        t = order[k]
        tp = order[k - 1] if k > 0 else None
        h_prev = hs[tp] if tp is not None else zeros
        b_prev = betas[tp] if tp is not None else zeros
        q = dy[:, t].unsqueeze(-1) * Cc[:, t].unsqueeze(1) + gq_next
        d_C[:, t] = (dy[:, t].unsqueeze(-1) * hs[t]).sum(1)
        dg = q * (h_prev + 0.5 * b_prev)
        dbeta = 0.5 * q + 0.5 * gq_next
        dt = delta[:, t]
        if nr:
            x = dt.unsqueeze(-1) * Ar
            e = torch.exp(x)
            c = torch.cos(dt.unsqueeze(-1) * Ai) if Ai is not None else torch.ones_like(e)
            s = torch.sin(dt.unsqueeze(-1) * Ai) if Ai is not None else torch.zeros_like(e)
            dgr = dg[..., :nr]
            d_Ar += (dgr * dt.unsqueeze(-1) * e * c).sum(0)
            if Ai is not None:
                d_Ai += (-dgr * dt.unsqueeze(-1) * e * s).sum(0)
            ai = Ai if Ai is not None else torch.zeros_like(Ar)
            d_delta[:, t] += (dgr * (Ar * e * c - ai * e * s)).sum(-1)
        if n - nr:
            d_Tk += dg[..., nr:].sum(0)
        sB = (dbeta * Bc[:, t].unsqueeze(1)).sum(-1)
        d_delta[:, t] += sB * u[:, t]
        d_u[:, t] = sB * dt
        d_B[:, t] = (dbeta * (dt * u[:, t]).unsqueeze(-1)).sum(1)
        gq_next = gs[t] * q
    return {"delta": d_delta, "u": d_u, "Bc": d_B, "Cc": d_C,
            "Ar": d_Ar, "Ai": d_Ai if Ai is not None else None, "Tk": d_Tk}


def rel_err(a, b):
    """Norm-wise relative error max|a - b| / max|b| used by every parity test."""
    a = a.detach().to(torch.float64)
    b = b.detach().to(torch.float64)
    den = b.abs().max().item()
    num = (a - b).abs().max().item() if a.numel() else 0.0
    if den == 0.0:
        return num
    return num / den
