"""Pins the fused oracle (oracle/fused.py) on the CPU against independent
restatements: the unfused per-expert loop (oracle/unfused.py) for the forward,
torch.autograd through that loop for all four gradients, autograd of the GLU
forward for the GLU derivatives, and closed forms for the losses.

Mirrors the reference's own differential tests (tests/test_generality.py,
tests/test_production.py), which compare fused_moe against unfused_moe.
"""

import numpy as np
import pytest
import torch

from oracle import fused as F_
from oracle import routing as R
from oracle.unfused import unfused_moe
from conftest import make_inputs


def _rel(a, b):
    return ((a.double() - b.double()).norm() / (b.double().norm() + 1e-30)).item()


@pytest.mark.parametrize("activation", F_.ACTIVATIONS)
@pytest.mark.parametrize("gating", F_.GATINGS)
@pytest.mark.parametrize("E,k", [(8, 2), (4, 1), (16, 4)])
def test_forward_matches_unfused_fp64(activation, gating, E, k):
    # test_generality.py:27-51 / :127-140 analogue; fp32 intermediates in the
    # GLU and combine (as in the reference's Triton kernels) bound the error.
    x, gate, wu, wd = make_inputs(64, 96, 288, E, torch.float64, seed=E + k)
    out, st = F_.forward(x, gate, wu, wd, k, activation=activation, gating=gating)
    ref, idx, w, _ = unfused_moe(x, gate, wu, wd, k, activation=activation, gating=gating)
    assert torch.equal(st["topk_idx"], idx)
    assert _rel(out, ref) < 1e-5
    torch.testing.assert_close(st["topk_w"], w.float(), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("activation", F_.ACTIVATIONS)
@pytest.mark.parametrize("gating", F_.GATINGS)
def test_backward_matches_autograd_fp64(activation, gating):
    # test_generality.py:58-97 analogue, extended to hidden and gate grads
    # (the reference's test compares only w_up and w_down).
    g = torch.Generator().manual_seed(11)
    N, D, ffn, E, k = 16, 64, 128, 4, 2
    x = torch.randn(N, D, generator=g, dtype=torch.float64)
    gate = torch.randn(E, D, generator=g, dtype=torch.float64) * 0.1
    wu = torch.randn(E, ffn, D, generator=g, dtype=torch.float64) * 0.1
    wd = torch.randn(E, D, ffn // 2, generator=g, dtype=torch.float64) * 0.1
    go = torch.randn(N, D, generator=g, dtype=torch.float64)

    out, st = F_.forward(x, gate, wu, wd, k, activation=activation, gating=gating)
    gr = F_.backward(st, go)

    leaves = [t.clone().requires_grad_(True) for t in (x, gate, wu, wd)]
    ref, _, _, _ = unfused_moe(*leaves, k, activation=activation, gating=gating)
    ref.backward(go)
    # fp32 GLU / combine / weight-grad intermediates (the reference's rounding
    # points) limit the agreement to ~1e-6 relative.
    for name, leaf in zip(("hidden", "gate", "w_up", "w_down"), leaves):
        assert _rel(gr[name], leaf.grad) < 2e-5, name


def test_glu_backward_matches_autograd():
    g = torch.Generator().manual_seed(2)
    up = torch.randn(50, 64, generator=g, dtype=torch.float32) * 2
    ga = torch.randn(50, 32, generator=g, dtype=torch.float32)
    for act in F_.ACTIVATIONS:
        u = up.clone().double().requires_grad_(True)
        H = 32
        gg, uu = u[:, :H], u[:, H:]
        if act == "swiglu":
            r = torch.nn.functional.silu(gg) * uu
        elif act == "geglu":
            r = torch.nn.functional.gelu(gg, approximate="tanh") * uu
        else:
            r = torch.relu(gg) ** 2 * uu
        r.backward(ga.double())
        mine = F_.glu_backward(ga, up, act)
        torch.testing.assert_close(mine.double(), u.grad, rtol=2e-5, atol=2e-6)
        fwd = F_.glu_forward(up, act)
        torch.testing.assert_close(fwd.double(), r.detach(), rtol=2e-6, atol=2e-6)


def test_capacity_matches_unfused():
    # test_production.py:99-110 analogue (the unfused oracle renormalises
    # with +1e-6, the fused path exactly: agreement ~1e-6)
    x, gate, wu, wd = make_inputs(64, 64, 128, 4, torch.float64, seed=7)
    out, st = F_.forward(x, gate, wu, wd, 2, capacity_factor=1.25)
    ref, _, _, _ = unfused_moe(x, gate, wu, wd, 2, capacity_factor=1.25)
    assert _rel(out, ref) < 1e-5
    assert not bool(st["keep"].all())


def test_large_capacity_equals_no_capacity():
    x, gate, wu, wd = make_inputs(32, 64, 128, 4, torch.float64, seed=8)
    a, _ = F_.forward(x, gate, wu, wd, 2)
    b, _ = F_.forward(x, gate, wu, wd, 2, capacity_factor=10.0)
    # renormalising by an fp32 sum that is 1 up to rounding: fp32-ulp level
    assert _rel(a, b) < 1e-6


def test_capacity_backward_matches_autograd_of_unfused_weights():
    # weight grads with capacity dropping vs autograd through the unfused loop
    x, gate, wu, wd = make_inputs(32, 64, 128, 4, torch.float64, seed=9)
    go = torch.randn(32, 64, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    _, st = F_.forward(x, gate, wu, wd, 2, capacity_factor=1.0)
    gr = F_.backward(st, go)
    leaves = [t.clone().requires_grad_(True) for t in (wu, wd)]
    ref, _, _, _ = unfused_moe(x, gate, *leaves, 2, capacity_factor=1.0)
    ref.backward(go)
    assert _rel(gr["w_up"], leaves[0].grad) < 1e-5
    assert _rel(gr["w_down"], leaves[1].grad) < 1e-5


def test_overflow_aliases_row0_forward():
    # moe_ops.py:87-91 + :138-140: an overflowed entry reads padded row 0
    x, gate, wu, wd = make_inputs(64, 64, 128, 4, torch.float64, seed=42)
    gate = gate.clone()
    gate[0] += 100.0
    with pytest.raises(RuntimeError, match="MoE routing overflow"):
        F_.forward(x, gate, wu, wd, 1, max_tokens_per_expert=16)
    out, st = F_.forward(x, gate, wu, wd, 1, max_tokens_per_expert=16, allow_dropped_tokens=True)
    # brute force: kept tokens get their own expert output, dropped ones get
    # weight * (expert-0 output of the first token routed to expert 0)
    full, _, w, _ = unfused_moe(x, gate, wu, wd, 1)
    keep = st["keep"].view(-1)
    first0 = int(torch.nonzero(st["topk_idx"].view(-1) == 0)[0])
    own = full / w.to(full.dtype)  # top_k = 1: full = w * expert_out
    expect = torch.where(keep.unsqueeze(1), full, w.to(full.dtype) * own[first0])
    assert _rel(out, expect) < 1e-6


def test_losses_closed_forms():
    g = torch.Generator().manual_seed(6)
    logits = torch.randn(128, 8, generator=g, dtype=torch.float64)
    w, idx = F_.apply_routing(logits, "softmax", 2)
    ls = F_.losses(logits, w, idx, 8, aux_loss_coeff=0.01, z_loss_coeff=0.001,
                   return_metrics=True)
    counts = np.bincount(idx.numpy().reshape(-1), minlength=8)
    P = np.zeros(8)
    for n in range(128):
        for s in range(2):
            P[idx[n, s]] += w[n, s]
    aux = 0.01 * 8 * np.sum(counts / 128.0 * P / 128.0)
    assert abs(ls["aux_loss"].item() - aux) < 1e-7
    lse = np.log(np.exp(logits.numpy()).sum(-1))
    assert abs(ls["z_loss"].item() - 0.001 * np.mean(lse ** 2)) < 1e-8
    assert ls["tokens_per_expert"].sum().item() == 256
    assert ls["expert_load_imbalance"].item() >= 1.0


def test_loss_grads_match_autograd():
    g = torch.Generator().manual_seed(12)
    logits = torch.randn(64, 8, generator=g)
    for gating in F_.GATINGS:
        l = logits.clone().requires_grad_(True)
        w, idx = F_.apply_routing(l.detach(), gating, 2)
        z = 0.01 * torch.logsumexp(l.float(), -1).square().mean()
        tot = z
        if gating == "sigmoid":
            f = torch.bincount(idx.view(-1), minlength=8).float() / 64
            tot = tot + 0.02 * 8 * (f * torch.sigmoid(l).mean(0)).sum()
        tot.backward()
        mine = F_.loss_grads(logits, idx, 8, gating, 0.02, 0.01)
        torch.testing.assert_close(mine, l.grad, rtol=1e-5, atol=1e-8)


def test_bf16_rounding_points_stay_within_tolerance_of_fp64():
    # the bf16 oracle (reference rounding points) vs the fp64 oracle on the
    # same bf16-representable inputs: the bf16 tolerance used by GPU tests
    x, gate, wu, wd = make_inputs(128, 128, 256, 8, torch.bfloat16, seed=1)
    logits = F_.gemm(x, gate.t())
    out16, _ = F_.forward(x, gate, wu, wd, 2, logits=logits)
    out64, _ = F_.forward(x.double(), gate.double(), wu.double(), wd.double(), 2,
                          logits=logits.double())
    torch.testing.assert_close(out16.double(), out64, rtol=2e-2, atol=2e-2)
