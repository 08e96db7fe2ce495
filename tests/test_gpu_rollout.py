"""GPU parity of the rollout ply boundary (rp_ply_topk, rp_ply_gather,
redpanda_amd.rollout.PlyBoundary) against the oracle's restatement of the
reference's per-rollout host reads (oracle/rollout_ref.py,
engine/mars_search.py:262-276, :475, :446).

Integer / index outputs are compared exactly; the logits are copies of the
inputs (converted to fp32 exactly), so they are compared bitwise too.
"""

import numpy as np
import pytest
import torch

from oracle import rollout_ref

pytestmark = pytest.mark.gpu
dev = "cuda"


def _rows(R, V, dtype, seed, ties=False, stride_pad=0):
    g = torch.Generator().manual_seed(seed)
    if ties:
        x = torch.randint(-3, 4, (R, V + stride_pad), generator=g).float()
    else:
        x = torch.randn(R, V + stride_pad, generator=g)
    x = x.to(dtype).to(dev)
    return x[:, :V]


def _check_topk(logits, k, values=None):
    from redpanda_amd.rollout import ply_topk
    out = ply_topk(logits, k, values=values)
    torch.cuda.synchronize()
    h = out.cpu().numpy()
    ln = logits.float().cpu().numpy()
    for r in range(ln.shape[0]):
        ids, lns = rollout_ref.candidates(ln[r], k)
        n = len(ids)
        got_ids = h[r, k + 1:].view(np.int32)
        assert np.array_equal(got_ids[:n], ids), (r, got_ids, ids)
        assert np.array_equal(h[r, 1:1 + n].view(np.uint32), lns.view(np.uint32))
        assert np.all(got_ids[n:] == -1) and np.all(np.isneginf(h[r, 1 + n:1 + k]))
        if values is not None:
            assert h[r, 0] == values.cpu().numpy()[r]


# row lengths around the kernel's 1024-element blocks: none full, one full
# (with and without a partial tail), an odd and an even count of full blocks
@pytest.mark.parametrize("R,V,k", [(64, 8192, 8), (37, 1000, 8), (5, 7, 8), (9, 64, 16),
                                   (3, 1, 1), (130, 4097, 5), (2, 20000, 16), (4, 1024, 16),
                                   (7, 1500, 8), (6, 3072, 8), (5, 2048, 3)])
def test_topk_matches_oracle(gpu_lib, R, V, k):
    vals = torch.randn(R, device=dev)
    _check_topk(_rows(R, V, torch.float32, R + V + k), k, values=vals)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_topk_low_precision_and_strided(gpu_lib, dtype):
    _check_topk(_rows(33, 3001, dtype, 3, stride_pad=13), 8)


def test_topk_ties_by_ascending_id(gpu_lib):
    """Integer-valued rows: most logits tie; equal logits come by ascending
    token id (the order the oracle's stable sort defines)."""
    _check_topk(_rows(50, 500, torch.float32, 4, ties=True), 16)


def test_topk_special_values(gpu_lib):
    x = torch.randn(5, 300)
    x[0, 17] = float("inf")
    x[1, 5] = float("-inf")
    x[2, :] = float("-inf")
    x[3, 100] = float("nan")
    x[3, 200] = float("inf")
    x[4, :] = -1.0
    x[4, 7] = -0.0
    x[4, 3] = 0.0
    x[4, 250] = -float("nan")
    from redpanda_amd.rollout import ply_topk
    out = ply_topk(x.to(dev), 4).cpu().numpy()
    ids = out[:, 5:].view(np.int32)
    assert ids[0, 0] == 17 and np.isposinf(out[0, 1])
    assert 5 not in ids[1]
    assert list(ids[2]) == [0, 1, 2, 3] and np.all(np.isneginf(out[2, 1:5]))
    # numpy's order, as the reference's argpartition applies it: a NaN
    # ranks above +inf, whatever its sign; -0 ties with +0 (ascending id)
    assert ids[3, 0] == 100 and np.isnan(out[3, 1]) and ids[3, 1] == 200
    assert list(ids[4]) == [250, 3, 7, 0] and np.isnan(out[4, 1])
    assert out[4, 3].view(np.uint32) == 0  # -0 comes back as +0


def test_topk_tie_heavy_long_rows(gpu_lib):
    """Integer-valued rows of 8192 with +-0 and NaNs of both signs: past the
    first 1024-element block, where the wave-wide bound and the one-compare
    filter decide which elements reach the lists."""
    x = _rows(24, 8192, torch.float32, 9, ties=True).clone()
    g = torch.Generator().manual_seed(10)
    zero = torch.rand(x.shape, generator=g) < 0.05
    x[zero.to(dev)] = -0.0
    x[3, 5000] = float("nan")
    x[4, 6000] = -float("nan")
    x[5, 7000] = float("nan")
    x[5, 100] = -float("nan")
    _check_topk(x, 16)
    _check_topk(x, 3)


def test_gather_matches_oracle(gpu_lib):
    from redpanda_amd.rollout import ply_gather
    R, V, M = 40, 8192, 37
    logits = _rows(R, V, torch.bfloat16, 6)
    g = np.random.default_rng(6)
    toks = g.integers(-2, V + 3, (R, M)).astype(np.int32)
    toks[:, -3:] = -1  # padding
    out = ply_gather(logits, torch.from_numpy(toks).to(dev)).cpu().numpy()
    ln = logits.float().cpu().numpy()
    for r in range(R):
        assert np.array_equal(out[r], rollout_ref.gather_legal(ln[r], toks[r]))


def test_ply_boundary_one_sync_per_ply(gpu_lib):
    """A whole ply through the pinned boundary equals the reference's
    per-rollout reads: tokens up, values + candidate lists down, legal-move
    logits down; the candidate walk picks the reference's move."""
    from redpanda_amd.rollout import PlyBoundary, select_policy_move
    R, V, k = 96, 8192, 8
    pb = PlyBoundary(R, top_k=k, device=dev, max_legal=64)
    toks = np.random.default_rng(7).integers(0, V, R)
    t_d = pb.push_tokens(toks.tolist())
    torch.cuda.synchronize()
    assert np.array_equal(t_d.cpu().numpy(), toks)
    cont = _rows(R, V, torch.float32, 8)
    vals = torch.tanh(torch.randn(R, 1, device=dev))
    v, ids, lns = pb.pull(vals, cont)
    assert np.array_equal(v, vals.squeeze(-1).cpu().numpy())
    ln = cont.cpu().numpy()
    legal = lambda t: t % 3 == 0  # a deterministic stand-in for board.is_legal
    for r in range(R):
        ref_ids, ref_lns = rollout_ref.candidates(ln[r], k)
        assert np.array_equal(ids[r], ref_ids) and np.array_equal(lns[r], ref_lns)
        for temp in (0.0, 0.6):
            a = select_policy_move(ids[r], lns[r], legal, temp, np.random.default_rng(r))
            b = rollout_ref.select_move(ln[r], k, legal, temp, np.random.default_rng(r))
            assert a == b
    # legal-move logits, padded with -1
    leg = np.full((R, 40), -1, dtype=np.int64)
    for r in range(R):
        n = 5 + r % 30
        leg[r, :n] = np.random.default_rng(100 + r).choice(V, n, replace=False)
    got = pb.pull_legal(cont, leg)
    for r in range(R):
        assert np.array_equal(got[r], rollout_ref.gather_legal(ln[r], leg[r]))
    # a second ply through the same buffers
    v2, ids2, _ = pb.pull(vals * 0.5, cont.flip(1).contiguous())
    assert np.array_equal(v2, (vals * 0.5).squeeze(-1).cpu().numpy())
    assert np.array_equal(ids2[0], rollout_ref.candidates(ln[0, ::-1], k)[0])
