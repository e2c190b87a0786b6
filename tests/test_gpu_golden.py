"""GPU parity against the committed golden fixtures (tests/golden/*.npz),
through the C ABI and through the Python API.

* routing.npz: top-k indices bit-exact and weights within fp32 rounding for
  tie-heavy and Zipf-skewed logits, k in (1, 2, 4, 8), both gatings; counts,
  expert offsets and every entry's compact row (the stable expert-sorted
  order, with and without capacity) bit-exact.
* c1_bf16.npz: the BASELINE configs[0] inputs in bf16 through ``fused_moe``
  forward + backward: output and all four gradients within the bf16 tolerance
  (rtol 2e-2, atol 2e-3), routing bit-exact, aux / z losses within 1e-4.
* c1_fp32.npz: the same config's fp32 unfused forward, against ``fused_moe``
  under bf16 autocast (bf16 tolerance; routing equal on at least 95% of the
  tokens, since fp32 and bf16 logits may order near-ties differently).
"""

import numpy as np
import pytest
import torch

import golden as G
from gpu_helpers import check_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def routing():
    return G.load("routing")


def _route_from_logits(logits, k, gating, mt, capacity):
    """route_fwd (from logits) -> route_scan -> permute, through the C ABI.
    x carries each token's index so the compact rows can be checked."""
    from flashfusedmoe_amd import _lib as L
    N, E = logits.shape
    dev = logits.device
    st = L.stream_ptr(dev)
    D = 8
    n = torch.arange(N, device=dev)
    x = torch.stack([n // 256, n % 256] + [torch.zeros_like(n)] * (D - 2), 1).to(torch.bfloat16)
    ws = torch.empty(L.route_workspace_bytes(N, E, k), dtype=torch.uint8, device=dev)
    idx = torch.empty(N, k, dtype=torch.int64, device=dev)
    w = torch.empty(N, k, dtype=torch.float32, device=dev)
    lse = torch.empty(N, dtype=torch.float32, device=dev)
    L.call("ffmoe_route_fwd", None, None, L.ptr(logits), None, N, D, E, k, L.GATING[gating], 0,
           None, L.ptr(idx), L.ptr(w), L.ptr(lse), L.ptr(ws), st)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    tiles = torch.empty(E + 1, dtype=torch.int32, device=dev)
    stats = torch.empty(L.NUM_STATS, dtype=torch.float32, device=dev)
    istats = torch.empty(L.NUM_ISTATS, dtype=torch.int32, device=dev)
    L.call("ffmoe_route_scan", N, E, k, mt, L.gemm_tile_rows(N * k, E), 0.0, 0.0,
           L.GATING[gating], L.ptr(ws), L.ptr(counts), L.ptr(offsets), L.ptr(tiles),
           L.ptr(stats), L.ptr(istats), None, None, st)
    xs = torch.empty(max(N * k, 1), D, dtype=torch.bfloat16, device=dev)
    row_of = torch.empty(N * k, dtype=torch.int32, device=dev)
    tw = w.clone()
    L.call("ffmoe_permute", L.ptr(x), L.ptr(idx), L.ptr(tw), L.ptr(offsets), L.ptr(counts), N, D, E,
           k, mt, int(capacity), L.ptr(ws), L.ptr(xs), L.ptr(row_of), st)
    torch.cuda.synchronize()
    return dict(idx=idx.cpu(), w=w.cpu(), counts=counts.cpu(), offsets=offsets.cpu(),
                row_of=row_of.cpu(), xs=xs.cpu(), istats=istats.cpu())


@pytest.mark.parametrize("tag", ["tie", "skew"])
@pytest.mark.parametrize("k", G.KS)
@pytest.mark.parametrize("gating", ["softmax", "sigmoid"])
def test_topk_matches_golden(routing, tag, k, gating):
    from flashfusedmoe_amd.kernels import fused_topk_routing
    logits = G.from_bits(routing[f"{tag}_logits"]).cuda()
    w, idx = fused_topk_routing(logits, gating, k)
    assert np.array_equal(idx.cpu().numpy(), routing[f"{tag}_{gating}_k{k}_idx"])
    np.testing.assert_allclose(w.cpu().numpy(), routing[f"{tag}_{gating}_k{k}_w"], rtol=2e-6,
                               atol=1e-7)


def _golden_rows(routing, tag, k, mt, capacity):
    idx = routing[f"{tag}_softmax_k{k}_idx"].astype(np.int64)
    flat = idx.reshape(-1)
    E = routing[f"{tag}_k{k}_counts"].size
    counts = routing[f"{tag}_k{k}_counts"].astype(np.int64)
    order = routing[f"{tag}_k{k}_order"].astype(np.int64)
    starts = np.concatenate([[0], np.cumsum(counts)])
    rank = np.empty_like(flat)
    rank[order] = np.arange(flat.size) - starts[flat[order]]
    kept_rows = np.minimum(counts, mt)
    off = np.concatenate([[0], np.cumsum(kept_rows)])
    rows = np.where(rank < mt, off[flat] + rank, -1 if capacity else -2)
    return rows, counts, off


@pytest.mark.parametrize("tag", ["tie", "skew"])
@pytest.mark.parametrize("k", G.KS)
@pytest.mark.parametrize("capacity", [False, True])
def test_permutation_matches_golden(routing, tag, k, capacity):
    N = routing[f"{tag}_logits"].shape[0]
    mt = int(routing[f"{tag}_k{k}_capacity" if capacity else f"{tag}_k{k}_max_tokens"])
    got = _route_from_logits(G.from_bits(routing[f"{tag}_logits"]).cuda(), k, "softmax", mt,
                             capacity)
    rows, counts, off = _golden_rows(routing, tag, k, mt, capacity)
    if capacity:
        assert np.array_equal(rows >= 0, routing[f"{tag}_k{k}_keep"].reshape(-1))
    elif counts[0] == 0:
        rows = np.where(rows == -2, -1, rows)
    assert np.array_equal(got["idx"].numpy(), routing[f"{tag}_softmax_k{k}_idx"])
    assert np.array_equal(got["counts"].numpy(), counts)
    assert np.array_equal(got["offsets"].numpy(), off)
    assert np.array_equal(got["row_of"].numpy(), rows)
    assert int(got["istats"][0]) == counts.max()
    own = rows >= 0
    tok = np.nonzero(own)[0] // k
    xs = got["xs"].float()[rows[own]]
    assert np.array_equal((xs[:, 0] * 256 + xs[:, 1]).long().numpy(), tok)


def _c1_bf16_run(f):
    from flashfusedmoe_amd import fused_moe
    x, gate, wu, wd = (t.to(torch.bfloat16).cuda().requires_grad_(True) for t in G.c1_inputs())
    go = G.c1_grad_out().to(torch.bfloat16).cuda()
    out, losses = fused_moe(x, gate, wu, wd, top_k=G.C1["top_k"], aux_loss_coeff=0.01,
                            z_loss_coeff=1e-3, return_metrics=True)
    out.backward(go)
    return out.detach().cpu(), losses, [t.grad.cpu() for t in (x, gate, wu, wd)]


def test_c1_bf16_forward_backward_matches_golden():
    f = G.load("c1_bf16")
    out, losses, (gx, gg, gwu, gwd) = _c1_bf16_run(f)
    E = G.C1["E"]
    counts = np.bincount(f["topk_idx"].reshape(-1).astype(np.int64), minlength=E)
    assert np.array_equal(losses["tokens_per_expert"].cpu().numpy(), counts)
    check_close(out, G.from_bits(f["out"]), "output")
    check_close(gx, G.from_bits(f["d_hidden"]), "grad hidden")
    check_close(gg, G.from_bits(f["d_gate"]), "grad gate")
    su, sd = torch.from_numpy(f["w_up_sample"]), torch.from_numpy(f["w_down_sample"])
    check_close(gwu.reshape(-1)[su], G.from_bits(f["d_w_up_sample"]), "grad w_up (sample)")
    check_close(gwd.reshape(-1)[sd], G.from_bits(f["d_w_down_sample"]), "grad w_down (sample)")
    assert abs(losses["aux_loss"].item() - float(f["aux_loss"])) <= 1e-4 * abs(float(f["aux_loss"]))
    assert abs(losses["z_loss"].item() - float(f["z_loss"])) <= 1e-4 * abs(float(f["z_loss"])) + 1e-9


def test_c1_topk_indices_match_golden():
    from flashfusedmoe_amd import ops
    f = G.load("c1_bf16")
    x, gate, _, _ = (t.to(torch.bfloat16).cuda() for t in G.c1_inputs())
    res = ops.route(x, gate, None, G.C1["top_k"], 0, 1, 0.0, 0.0, False)
    assert np.array_equal(res[1].cpu().numpy(), f["topk_idx"])
    np.testing.assert_allclose(res[2].cpu().numpy(), f["topk_w"], rtol=2e-6, atol=1e-7)


def test_c1_fp32_under_autocast_matches_golden():
    from flashfusedmoe_amd import fused_moe
    f = G.load("c1_fp32")
    x, gate, wu, wd = (t.cuda() for t in G.c1_inputs())
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out, losses = fused_moe(x, gate, wu, wd, top_k=G.C1["top_k"], return_metrics=True)
    from flashfusedmoe_amd import ops
    idx = ops.route(x.bfloat16(), gate.bfloat16(), None, G.C1["top_k"], 0, 1, 0.0, 0.0, False)[1]
    same = (idx.cpu().numpy() == f["topk_idx"]).all(1)
    assert same.mean() >= 0.95
    m = torch.from_numpy(same)
    check_close(out.float().cpu()[m], torch.from_numpy(f["out"])[m], "output (fp32 golden)")
