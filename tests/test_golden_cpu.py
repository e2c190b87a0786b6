"""The committed golden fixtures (tests/golden/*.npz) on the CPU.

1. Their input recipes still produce the bytes the fixtures were made from.
2. The oracle still reproduces them (a regression pin for the oracle).
3. They hold what the mathematics fixes, independently of the oracle: top-k by
   brute force over each row, counts by counting, the expert-sorted order by
   its definition (sorted by expert, ascending entry index within an expert),
   the capacity mask by the rank definition, softmax/sigmoid weights summing to
   one.
"""

import numpy as np
import pytest
import torch

import golden as G
from oracle import fused as F_
from oracle import routing as R
from oracle.unfused import unfused_moe


@pytest.fixture(scope="module")
def routing():
    return G.load("routing")


def test_input_recipes_are_unchanged(routing):
    assert str(G.load("c1_fp32")["sha"]) == G.sha256(*G.c1_inputs())
    bf = tuple(t.to(torch.bfloat16) for t in G.c1_inputs()) + (G.c1_grad_out().to(torch.bfloat16),)
    assert str(G.load("c1_bf16")["sha"]) == G.sha256(*bf)
    assert str(routing["tie_sha"]) == G.sha256(G.tie_logits())
    assert str(routing["skew_sha"]) == G.sha256(G.skew_logits())
    assert np.array_equal(routing["tie_logits"], G.bits(G.tie_logits()))


def _brute_topk(row, k):
    # sort key: value descending, then index ascending
    return [i for _, i in sorted(((-float(v), i) for i, v in enumerate(row)))[:k]]


@pytest.mark.parametrize("tag", ["tie", "skew"])
@pytest.mark.parametrize("k", G.KS)
def test_routing_fixture_by_brute_force(routing, tag, k):
    logits = G.from_bits(routing[f"{tag}_logits"]).float().numpy()
    N, E = logits.shape
    rows = range(0, N, 1 if N <= 300 else 7)
    for gating in ("softmax", "sigmoid"):
        idx = routing[f"{tag}_{gating}_k{k}_idx"].astype(np.int64)
        w = routing[f"{tag}_{gating}_k{k}_w"]
        score = logits if gating == "softmax" else 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
        for n in rows:
            assert list(idx[n]) == _brute_topk(score[n], k), (gating, n)
        if gating == "softmax":
            v = np.take_along_axis(logits, idx, 1).astype(np.float64)
            ref = np.exp(v - v.max(1, keepdims=True))
            ref /= ref.sum(1, keepdims=True)
            np.testing.assert_allclose(w, ref, rtol=2e-6, atol=1e-7)
        else:
            s = np.take_along_axis(score, idx, 1)
            np.testing.assert_allclose(w, s / (s.sum(1, keepdims=True) + 1e-6), rtol=2e-6, atol=1e-7)
    # counts, order and capacity keep-mask by their definitions
    idx = routing[f"{tag}_softmax_k{k}_idx"].astype(np.int64)
    flat = idx.reshape(-1)
    counts = routing[f"{tag}_k{k}_counts"]
    assert np.array_equal(counts, [int((flat == e).sum()) for e in range(E)])
    order = routing[f"{tag}_k{k}_order"].astype(np.int64)
    assert sorted(order.tolist()) == list(range(flat.size))
    keys = list(zip(flat[order].tolist(), order.tolist()))
    assert keys == sorted(keys)
    cap = int(routing[f"{tag}_k{k}_capacity"])
    assert cap == max(int(N / E * G.CAPACITY_FACTOR), k)
    seen = np.zeros(E, dtype=np.int64)
    keep = np.zeros(flat.size, dtype=bool)
    for j, e in enumerate(flat):
        keep[j] = seen[e] < cap
        seen[e] += 1
    assert np.array_equal(routing[f"{tag}_k{k}_keep"].reshape(-1), keep)


@pytest.mark.parametrize("tag", ["tie", "skew"])
def test_oracle_reproduces_routing_fixture(routing, tag):
    logits = G.from_bits(routing[f"{tag}_logits"]).float().numpy()
    N, E = logits.shape
    for k in G.KS:
        for gating in ("softmax", "sigmoid"):
            w, idx = R.route(logits, k, gating)
            assert np.array_equal(idx, routing[f"{tag}_{gating}_k{k}_idx"])
            np.testing.assert_allclose(w, routing[f"{tag}_{gating}_k{k}_w"], rtol=1e-6, atol=0)
        order, counts, _, _ = R.stable_permutation(routing[f"{tag}_softmax_k{k}_idx"], E)
        assert np.array_equal(order, routing[f"{tag}_k{k}_order"])
        assert np.array_equal(counts, routing[f"{tag}_k{k}_counts"])
        assert int(routing[f"{tag}_k{k}_max_tokens"]) == R.estimate_max_tokens(N, k, E)


def test_oracle_reproduces_c1_fp32():
    f = G.load("c1_fp32")
    x, gate, wu, wd = G.c1_inputs()
    out, idx, w, _ = unfused_moe(x, gate, wu, wd, G.C1["top_k"])
    assert np.array_equal(idx.numpy(), f["topk_idx"])
    np.testing.assert_allclose(w.numpy(), f["topk_w"], rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(out.numpy(), f["out"], rtol=1e-5, atol=1e-7)


def test_oracle_reproduces_c1_bf16():
    f = G.load("c1_bf16")
    x, gate, wu, wd = (t.to(torch.bfloat16) for t in G.c1_inputs())
    go = G.c1_grad_out().to(torch.bfloat16)
    out, st = F_.forward(x, gate, wu, wd, G.C1["top_k"])
    gr = F_.backward(st, go)
    assert np.array_equal(st["topk_idx"].numpy(), f["topk_idx"])
    assert np.array_equal(G.bits(st["logits"]), f["logits"])
    # bf16 bits can flip on a different CPU summation order: compare values
    for got, key in ((out, "out"), (gr["hidden"], "d_hidden"), (gr["gate"], "d_gate")):
        torch.testing.assert_close(got.float(), G.from_bits(f[key]).float(), rtol=1e-2, atol=1e-3)
    su, sd = torch.from_numpy(f["w_up_sample"]), torch.from_numpy(f["w_down_sample"])
    torch.testing.assert_close(gr["w_up"].reshape(-1)[su].float(),
                               G.from_bits(f["d_w_up_sample"]).float(), rtol=1e-2, atol=1e-3)
    torch.testing.assert_close(gr["w_down"].reshape(-1)[sd].float(),
                               G.from_bits(f["d_w_down_sample"]).float(), rtol=1e-2, atol=1e-3)


def test_c1_fixtures_agree_with_each_other():
    """The bf16 fused path and the fp32 unfused path of the same config stay
    within bf16 error of each other where they route alike."""
    a, b = G.load("c1_fp32"), G.load("c1_bf16")
    same = (a["topk_idx"] == b["topk_idx"]).all(1)
    assert same.mean() > 0.95
    o32 = torch.from_numpy(a["out"])[torch.from_numpy(same)]
    o16 = G.from_bits(b["out"]).float()[torch.from_numpy(same)]
    assert ((o16 - o32).norm() / o32.norm()).item() < 2e-2
