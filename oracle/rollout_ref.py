"""CPU oracle of the rollout ply's host-side reads (engine/mars_search.py).

TEST INFRASTRUCTURE ONLY: imported by tests/ and nothing shipped.  Restates,
in numpy, what the reference computes on the host from each rollout's rows:

  candidates(row, k)       _select_move's candidate list (:262-265):
                           ln = row as fp32; top = np.argpartition(ln, -k)[-k:];
                           top = top[np.argsort(ln[top])[::-1]]
  gather_legal(row, toks)  _select_fc_move's logits of the legal moves
                           (:466-475): row[toks] as fp32 for 0 <= t < vocab
  select_move(...)         the policy-guided walk over the candidates
                           (:266-276), greedy or a softmax draw

Order: numpy's, as the reference's argpartition / argsort apply it: -0 and
+0 are equal and every NaN is above +inf whatever its sign.  The
reference's argsort is not stable, so equal logits come in an unspecified
order there; `candidates` orders them by ascending token id, the order the
device kernel documents, and tests of ties use that rule.  The returned
logits are the canonical values (+0.0 for -0.0, a NaN with its sign bit
cleared), equal in value to the reference's `float(ln[mid])`; NaNs with
different payloads are ordered by payload, which numpy leaves unspecified
(a canonical NaN has one payload).

Parity pins (tests/test_oracle.py): `candidates` against a full stable sort
by (-logit, id), the brute force for tiny rows (with +-0, +-inf and NaNs of
both signs); against the reference's own argpartition/argsort expression on
tie-free rows, NaNs included; and the set property (no logit outside the
list exceeds one inside it).  `gather_legal` against direct indexing.
`select_move`: greedy = the first legal candidate; the draw against what the
mathematics of a softmax at temperature T fixes (equal logits draw
uniformly, a logit many T above the rest is always drawn, draw frequencies
match exp(l/T)/sum over many seeded draws, scaling logits and T by the same
power of two changes no draw), each check failed by a planted mistake.
"""

import numpy as np


def canonical(row):
    """fp32 logits with -0.0 as +0.0 and every NaN's sign bit cleared."""
    bits = np.asarray(row, dtype=np.float32).copy().view(np.uint32)
    nan = (bits & np.uint32(0x7fffffff)) > np.uint32(0x7f800000)
    bits[nan] &= np.uint32(0x7fffffff)
    bits[bits == np.uint32(0x80000000)] = 0
    return bits.view(np.float32)


def candidates(row, k):
    """(ids, logits) of the k largest fp32 logits of `row` in numpy's order
    (NaN largest, -0 == +0), largest first, equal logits by ascending id;
    rows shorter than k give all of them.  Logits come back canonical."""
    ln = canonical(row)
    k = min(k, ln.shape[0])
    bits = ln.view(np.uint32).astype(np.int64)
    # order-preserving integer of each canonical value (NaNs above +inf)
    rank = np.where(bits >= 0x80000000, 0xffffffff - bits, bits + 0x80000000)
    # stable sort on -rank keeps ascending id among equal logits
    order = np.argsort(-rank, kind="stable")[:k]
    return order.astype(np.int64), ln[order]


def candidates_reference_expr(row, k):
    """The reference's own expression (engine/mars_search.py:262-265)."""
    ln = np.asarray(row, dtype=np.float32)
    k = min(k, ln.shape[0])
    top = np.argpartition(ln, -k)[-k:]
    return top[np.argsort(ln[top])[::-1]]


def gather_legal(row, toks):
    """fp32 logits of the ids in `toks` (ids outside [0, len(row)) give
    -inf, which the reference skips)."""
    ln = np.asarray(row, dtype=np.float32)
    toks = np.asarray(toks)
    ok = (toks >= 0) & (toks < ln.shape[0])
    out = np.full(toks.shape, -np.inf, dtype=np.float32)
    out[ok] = ln[toks[ok]]
    return out


def select_move(row, k, is_legal, rollout_temp, rng):
    """_select_move's policy-guided branch (engine/mars_search.py:261-276):
    returns the chosen id, or None when no candidate is legal."""
    ids, lns = candidates(row, k)
    cand = []
    for mid, lg in zip(ids, lns):
        if is_legal(int(mid)):
            if rollout_temp <= 1e-3:
                return int(mid)
            cand.append((int(mid), float(lg)))
    if cand:
        lg = np.array([c[1] for c in cand]) / rollout_temp
        lg -= lg.max()
        pr = np.exp(lg)
        pr /= pr.sum()
        return cand[int(rng.choice(len(cand), p=pr))][0]
    return None
