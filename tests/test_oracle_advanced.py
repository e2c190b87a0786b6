"""Pins the oracle's slow-path routing (oracle/fused.py::route_advanced, the
restatement of fused_moe.py:144-251) against independent restatements on
the CPU: a per-row pure-Python brute force for expert-bias selection and the
group-limited top-k, float64 softmax for pre-softmax weights, and the closed
form of the scoring factor.
"""

import math

import numpy as np
import pytest
import torch

from oracle import fused as F_
from oracle import routing as R


def _ranked(vals):
    """Indices ordered by (value desc, index asc)."""
    return [i for _, i in sorted((-float(v), i) for i, v in enumerate(vals))]


def _bf16(v):
    return float(torch.tensor(v, dtype=torch.float32).to(torch.bfloat16))


def _brute_select(sel_row, k, n_group=None, topk_group=None, bf16_scores=False):
    E = len(sel_row)
    if n_group is None:
        return _ranked(sel_row)[:k]
    epg = E // n_group
    per = k // topk_group
    gs = []
    for g in range(n_group):
        members = [sel_row[g * epg + j] for j in range(epg)]
        if 1 < per <= epg:
            top = sorted(members, reverse=True)[:per]
            # a bf16 tensor sums in fp32 and rounds the result to bf16
            gs.append(_bf16(float(np.float32(sum(np.float32(t) for t in top)))) if bf16_scores
                      else sum(top))
        else:
            gs.append(max(members))
    keep = set(_ranked(gs)[:topk_group])
    masked = [v if (e // epg) in keep else -math.inf for e, v in enumerate(sel_row)]
    return _ranked(masked)[:k]


def _logits(N, E, seed, ties=False):
    g = torch.Generator().manual_seed(seed)
    if ties:
        return torch.randint(-3, 4, (N, E), generator=g).to(torch.bfloat16)
    return torch.randn(N, E, generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("gating", ["softmax", "sigmoid"])
@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("pre", [False, True])
@pytest.mark.parametrize("groups", [None, (4, 2), (8, 3), (4, 4)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_selection_matches_brute_force(gating, ties, pre, groups, with_bias):
    N, E, k = 64, 16, 4
    logits = _logits(N, E, seed=E + k + int(ties), ties=ties)
    bias = torch.linspace(-0.3, 0.4, E) if with_bias else None
    ng, tg = groups if groups else (None, None)
    w, idx = F_.route_advanced(logits, gating, k, bias, pre, None, ng, tg)
    lf = logits.double()
    if gating == "softmax":
        base = torch.softmax(lf, -1) if pre else lf
    else:
        base = torch.sigmoid(lf)
    # the oracle selects on fp32 scores (+ fp32 bias); restate in float32 too
    sel = (base.float() + (bias.float() if with_bias else 0.0)).double()
    bf16_scores = gating == "softmax" and not pre and not with_bias
    for n in range(N):
        assert idx[n].tolist() == _brute_select(sel[n].tolist(), k, ng, tg, bf16_scores), n


@pytest.mark.parametrize("gating", ["softmax", "sigmoid"])
def test_weights_use_unbiased_scores(gating):
    N, E, k = 32, 8, 3
    logits = _logits(N, E, seed=3)
    bias = torch.randn(E, generator=torch.Generator().manual_seed(9)) * 0.5
    w, idx = F_.route_advanced(logits, gating, k, bias, False, None, None, None)
    lf = logits.double()
    if gating == "softmax":
        ref = torch.softmax(lf.gather(1, idx), -1)
    else:
        s = torch.sigmoid(lf).gather(1, idx)
        ref = s / (s.sum(-1, keepdim=True) + 1e-6)
    np.testing.assert_allclose(w.numpy(), ref.numpy(), rtol=2e-6, atol=1e-7)


def test_pre_softmax_weights_are_renormalised_probabilities():
    N, E, k = 32, 16, 4
    logits = _logits(N, E, seed=5)
    w, idx = F_.route_advanced(logits, "softmax", k, None, True, None, None, None)
    lf = logits.double().numpy()
    p = np.exp(lf - lf.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ps = np.take_along_axis(p, idx.numpy(), 1)
    np.testing.assert_allclose(w.numpy(), ps / (ps.sum(1, keepdims=True) + 1e-6), rtol=2e-6)
    # selection by probability equals selection by logit (softmax is monotone)
    ridx, _ = R.topk_select(logits.float().numpy(), k)
    assert np.array_equal(idx.numpy(), ridx)


@pytest.mark.parametrize("pre", [False, True])
def test_scoring_factor_scales_by_factor_over_k(pre):
    N, E, k, sf = 32, 8, 2, 2.5
    logits = _logits(N, E, seed=7)
    w0, i0 = F_.route_advanced(logits, "softmax", k, None, pre, None, None, None)
    w1, i1 = F_.route_advanced(logits, "softmax", k, None, pre, sf, None, None)
    assert torch.equal(i0, i1)
    np.testing.assert_allclose(w1.numpy(), w0.numpy() * (sf / k), rtol=1e-6)


def test_group_limited_keeps_only_selected_groups():
    N, E, k, ng, tg = 64, 16, 4, 4, 2
    logits = _logits(N, E, seed=11)
    _, idx = F_.route_advanced(logits, "softmax", k, None, False, None, ng, tg)
    groups = (idx // (E // ng)).numpy()
    for n in range(N):
        assert len(set(groups[n].tolist())) <= tg
