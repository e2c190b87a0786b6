"""Pins the routing oracle (oracle/routing.py) on the CPU.

Each check uses an independent method: the reference's own known answers,
brute force over a different algorithm, or a library routine.
"""

import itertools

import numpy as np
import pytest
import torch

from oracle import routing as R


# --- estimate_max_tokens: fused_moe.py:100-113 --------------------------------

def test_estimate_max_tokens_reference_known_answers():
    # tests/test_production.py:37-47
    assert R.estimate_max_tokens(4, 2, 8) == 8
    mt = R.estimate_max_tokens(1024, 2, 8)
    assert 256 <= mt <= 2048


@pytest.mark.parametrize("N,k,E,expect", [
    (256, 2, 4, 256),     # C1: ceil(128) + 128
    (8192, 2, 8, 4096),   # C2
    (64, 2, 8, 32),       # C3
    (16384, 8, 64, 4096),  # C4
    (4096, 8, 256, 256),  # C5
    (3, 2, 8, 6),         # N*k <= 4E -> N*k
    (17, 2, 8, 10),       # N*k = 34 > 32: ceil(34/8) = 5, + max(5, 2)
])
def test_estimate_max_tokens_closed_form(N, k, E, expect):
    assert R.estimate_max_tokens(N, k, E) == expect


# --- top-k rule: fused_topk.py:63-70 ------------------------------------------

def _brute_topk(row, k):
    # iterative argmax with explicit lowest-index tie break, pure Python
    row = [float(v) for v in row]
    picked = []
    for _ in range(k):
        best = None
        for i, v in enumerate(row):
            if i in picked:
                continue
            if best is None or v > row[best]:
                best = i
        picked.append(best)
    return picked


@pytest.mark.parametrize("E,k", [(4, 1), (4, 2), (8, 2), (8, 3), (16, 4), (64, 8), (7, 7)])
def test_topk_matches_bruteforce_on_ties(E, k):
    rng = np.random.default_rng(E * 100 + k)
    scores = rng.integers(-3, 3, size=(200, E)).astype(np.float32)  # tie-heavy
    idx, vals = R.topk_select(scores, k)
    for n in range(scores.shape[0]):
        assert list(idx[n]) == _brute_topk(scores[n], k)
        assert np.array_equal(vals[n], scores[n, idx[n]])


def test_topk_matches_torch_on_tie_free_inputs():
    g = torch.Generator().manual_seed(3)
    s = torch.randn(500, 64, generator=g)
    idx, vals = R.topk_select(s.numpy(), 8)
    tv, ti = torch.topk(s, 8, dim=-1)
    assert np.array_equal(idx, ti.numpy())
    assert np.array_equal(vals, tv.numpy())


def test_softmax_weights_match_float64_softmax():
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(300, 16, generator=g)
    w, idx = R.route(logits.numpy(), 4, "softmax")
    ref = torch.softmax(logits.double().gather(1, torch.from_numpy(idx)), dim=-1)
    np.testing.assert_allclose(w, ref.numpy(), rtol=2e-6, atol=1e-7)
    assert np.all(np.diff(np.take_along_axis(logits.numpy(), idx, 1), axis=1) <= 0)


def test_sigmoid_weights_closed_form():
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(300, 16, generator=g)
    w, idx = R.route(logits.numpy(), 3, "sigmoid")
    s = torch.sigmoid(logits.double())
    sel = s.gather(1, torch.from_numpy(idx))
    np.testing.assert_allclose(w, (sel / (sel.sum(-1, keepdim=True) + 1e-6)).numpy(),
                               rtol=2e-6, atol=1e-7)


# --- permutation: fused_moe.py:344-348, moe_ops.py:84-98 ------------------------

def _brute_rank(flat):
    seen = {}
    out = []
    for e in flat:
        out.append(seen.get(e, 0))
        seen[e] = seen.get(e, 0) + 1
    return np.array(out)


@pytest.mark.parametrize("N,E,k", [(1, 4, 2), (37, 8, 2), (64, 16, 4), (100, 64, 8), (5, 3, 3)])
def test_stable_permutation_bruteforce(N, E, k):
    rng = np.random.default_rng(N + E + k)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(N)])
    sorted_order, counts, starts, rank = R.stable_permutation(idx, E)
    flat = idx.reshape(-1)
    assert np.array_equal(sorted_order, np.argsort(flat, kind="stable"))
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    assert np.array_equal(rank, _brute_rank(list(flat)))
    # sorted position of j is starts[e] + rank[j]: the inverse permutation
    pos = starts[flat] + rank
    assert np.array_equal(sorted_order[pos], np.arange(flat.size))


def test_expand_to_batch_overflow_aliases_row0():
    idx = np.array([[0], [0], [0], [1], [0]])
    e2b, kept = R.expand_to_batch(idx, 2, 2)
    assert list(e2b) == [0, 1, 0, 2, 0]
    assert list(kept) == [True, True, False, True, False]


def test_capacity_keep_and_renormalize():
    idx = np.array([[0, 1], [0, 1], [0, 2], [1, 0]])
    keep = R.capacity_keep(idx, 3, 2)
    # expert 0: j=0,2,4,7 -> first two kept; expert 1: j=1,3,6 -> first two
    assert keep.tolist() == [[True, True], [True, True], [False, True], [False, False]]
    w = np.array([[0.6, 0.4], [0.5, 0.5], [0.7, 0.3], [0.9, 0.1]], dtype=np.float32)
    r = R.capacity_renormalize(w, keep)
    np.testing.assert_allclose(r[2], [0.0, 1.0])
    np.testing.assert_allclose(r[3], [0.0, 0.0])
    np.testing.assert_allclose(r[0], w[0] / w[0].sum())
    assert R.expert_capacity(4, 3, 2, 1.5) == 2
    assert R.expert_capacity(64, 4, 2, 0.01) == 2
