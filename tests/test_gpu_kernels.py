"""GPU tests of the reference's kernel-level boundary (flashfusedmoe_amd.kernels,
mirroring src/flashfusemoe/kernels/moe_ops.py:109-332 and
activations.py:145-231) on the reference's padded [E*max_tokens, D] layout,
of the grouped GEMMs' workspace check, and of tracing fused_moe under
torch.compile.

Expected values come from the CPU oracle (oracle/routing.py, oracle/fused.py)
on the same seeded inputs; index results must be bit-exact, bf16 results
within the tolerance of gpu_helpers.check_close.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import check_close, seeded
from oracle import fused as F_
from oracle import routing as R

pytestmark = pytest.mark.gpu


def _routing(N, E, k, seed, skew=False):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(N, E, generator=g)
    if skew:  # most tokens prefer expert 0: overflows a small max_tokens
        logits[:, 0] += 3.0
    w, idx = F_.apply_routing(logits.to(torch.bfloat16), "softmax", k)
    return w, idx


@pytest.mark.parametrize("N,D,E,k,mt,skew", [(300, 128, 8, 2, None, False), (257, 264, 16, 4, 40, True),
                                             (64, 64, 4, 1, 5, True)])
def test_fused_routing_scatter_matches_oracle(N, D, E, k, mt, skew):
    from flashfusedmoe_amd.kernels import fused_routing_scatter
    _, idx = _routing(N, E, k, seed=N + D, skew=skew)
    mt = mt if mt is not None else R.estimate_max_tokens(N, k, E)
    x = torch.randn(N, D, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    sorted_order, counts, starts, _ = R.stable_permutation(idx.numpy(), E)
    hb, e2b = fused_routing_scatter(torch.from_numpy(sorted_order).cuda(), idx.reshape(-1).cuda(),
                                    torch.from_numpy(starts).cuda(), x.cuda(), E, mt, k)
    exp_e2b, kept = R.expand_to_batch(idx.numpy(), E, mt)
    assert np.array_equal(e2b.cpu().numpy(), exp_e2b)
    exp_hb = torch.zeros(E * mt, D, dtype=torch.bfloat16)
    flat_x = x.repeat_interleave(k, dim=0)
    exp_hb[torch.from_numpy(exp_e2b[kept])] = flat_x[torch.from_numpy(kept)]
    assert torch.equal(hb.cpu(), exp_hb)
    if skew:
        assert not kept.all()  # the overflow path ran


def test_fused_routing_scatter_num_sorted():
    """num_sorted < N*k processes only the first sorted positions
    (moe_ops.py:141-146, the capacity-dropping caller)."""
    from flashfusedmoe_amd.kernels import fused_routing_scatter
    N, D, E, k = 200, 64, 8, 2
    _, idx = _routing(N, E, k, seed=5)
    mt = R.estimate_max_tokens(N, k, E)
    x = torch.randn(N, D, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    sorted_order, counts, starts, rank = R.stable_permutation(idx.numpy(), E)
    ns = 150
    hb, e2b = fused_routing_scatter(torch.from_numpy(sorted_order).cuda(), idx.reshape(-1).cuda(),
                                    torch.from_numpy(starts).cuda(), x.cuda(), E, mt, k, num_sorted=ns)
    flat = idx.reshape(-1).numpy()
    exp = np.zeros(N * k, dtype=np.int64)
    done = sorted_order[:ns]
    exp[done] = flat[done] * mt + rank[done]
    assert np.array_equal(e2b.cpu().numpy(), exp)
    exp_hb = torch.zeros(E * mt, D, dtype=torch.bfloat16)
    exp_hb[torch.from_numpy(exp[done])] = x[torch.from_numpy(done // k)]
    assert torch.equal(hb.cpu(), exp_hb)


@pytest.mark.parametrize("N,D,E,k,weighted", [(300, 128, 8, 2, True), (123, 520, 16, 4, True),
                                              (77, 64, 4, 3, False)])
def test_fused_gather_reduce_matches_oracle(N, D, E, k, weighted):
    from flashfusedmoe_amd.kernels import fused_gather_reduce
    w, idx = _routing(N, E, k, seed=N + k)
    mt = R.estimate_max_tokens(N, k, E)
    e2b, _ = R.expand_to_batch(idx.numpy(), E, mt)
    batched = torch.randn(E * mt, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    wb = w.to(torch.bfloat16) if weighted else None  # the forward passes bf16(topk_w) (fused_moe.py:412)
    out = fused_gather_reduce(batched.cuda(), torch.from_numpy(e2b).cuda(),
                              None if wb is None else wb.cuda(), N, k)
    exp = F_.gather_reduce(batched, torch.from_numpy(e2b), wb, N, k)
    check_close(out, exp, "gather_reduce")
    # fp32 slot-order accumulation of bf16 products: the same bits as the oracle
    assert torch.equal(out.cpu(), exp)


@pytest.mark.parametrize("N,D,E,k", [(300, 128, 8, 2), (99, 264, 16, 4)])
def test_fused_weighted_scatter_matches_oracle(N, D, E, k):
    from flashfusedmoe_amd.kernels import fused_weighted_scatter
    w, idx = _routing(N, E, k, seed=7 * N)
    mt = R.estimate_max_tokens(N, k, E)
    e2b, kept = R.expand_to_batch(idx.numpy(), E, mt)
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    flat_w = w.to(torch.bfloat16).reshape(-1)
    out = fused_weighted_scatter(go.cuda(), torch.from_numpy(e2b).cuda(), flat_w.cuda(), E, mt, k)
    exp = F_.weighted_scatter(go, torch.from_numpy(e2b), flat_w, E * mt, k, torch.from_numpy(kept))
    assert torch.equal(out.cpu(), exp)
    rows = E * mt + 3
    out2 = fused_weighted_scatter(go.cuda(), torch.from_numpy(e2b).cuda(), flat_w.cuda(), E, mt, k,
                                  output_rows=rows)
    assert out2.shape == (rows, D)
    assert torch.equal(out2[: E * mt].cpu(), exp)
    assert not out2[E * mt:].any()


@pytest.mark.parametrize("activation", ["swiglu", "geglu", "relu_squared"])
def test_activation_forward_backward_match_oracle(activation):
    from flashfusedmoe_amd.kernels import activation_backward, activation_forward
    g = torch.Generator().manual_seed(11)
    M, H = 517, 264
    up = (torch.randn(3, M, 2 * H, generator=g) * 2.0).to(torch.bfloat16)
    ga = torch.randn(3, M, H, generator=g).to(torch.bfloat16)
    act = activation_forward(up.cuda(), activation)
    assert act.shape == (3, M, H)
    check_close(act, F_.glu_forward(up, activation), f"{activation} forward", max_bad_frac=0.0)
    gup = activation_backward(ga.cuda(), up.cuda(), activation)
    assert gup.shape == up.shape
    check_close(gup, F_.glu_backward(ga, up, activation), f"{activation} backward", max_bad_frac=0.0)


def test_fused_topk_routing_matches_oracle():
    from flashfusedmoe_amd.kernels import fused_topk_routing
    N, E, k = 1000, 32, 4
    logits = torch.randn(N, E, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    for gating in ("softmax", "sigmoid"):
        w, idx = fused_topk_routing(logits.cuda(), gating, k)
        rw, ridx = R.route(logits.float().numpy(), k, gating)
        assert np.array_equal(idx.cpu().numpy(), ridx)
        np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)


def test_gemm_workspace_error_word_is_reported_and_cleared():
    """A set error word (what a timed-out stream-K wait leaves) makes
    ffmoe_gemm_check raise and clears the workspace.  The word is set from
    the host: no kernel waits on anything in this test."""
    from flashfusedmoe_amd import _lib as L
    dev = torch.device("cuda")
    st = L.stream_ptr(dev)
    ws = L.gemm_workspace(dev, st)
    L.call("ffmoe_gemm_check", ws.data_ptr(), st)  # clean workspace: no error
    G = torch.cuda.get_device_properties(dev).multi_processor_count
    flags = ws[:8192].view(torch.int32)
    flags[2 * G] = 1       # the error word
    flags[G + 3] = 5       # a stale publication a late partner could leave
    with pytest.raises(L.FFMoEError, match="stream-K"):
        L.check_gemm_workspaces()
    assert not ws[:8192].any()
    L.check_gemm_workspaces()  # cleared: sound again


def test_fused_moe_traces_under_torch_compile():
    """fused_moe forward + backward through torch.compile (AOTAutograd over
    the custom ops' fake implementations; the reference marks its autograd
    Function allow_in_graph, fused_moe.py:293) gives the eager results."""
    from flashfusedmoe_amd import fused_moe
    N, D, ffn, E, k = 512, 128, 256, 8, 2
    x, gate, wu, wd = (t.cuda() for t in seeded(N, D, ffn, E, seed=21))
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16).cuda()

    def f(x, gate, wu, wd):
        out, losses = fused_moe(x, gate, wu, wd, top_k=k, aux_loss_coeff=0.01, z_loss_coeff=1e-3,
                                allow_dropped_tokens=True)
        return out, losses["z_loss"]

    def run(fn):
        leaves = [t.clone().requires_grad_(True) for t in (x, gate, wu, wd)]
        out, z = fn(*leaves)
        torch.autograd.backward([out, z], [go, torch.ones((), device="cuda")])
        torch.cuda.synchronize()
        return out.detach(), z.detach(), [t.grad for t in leaves]

    torch._dynamo.reset()
    eo, ez, eg = run(f)
    co, cz, cg = run(torch.compile(f, backend="aot_eager"))
    assert torch.equal(eo, co)
    assert torch.equal(ez, cz)
    for a, b in zip(eg, cg):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_kernel_boundary_fp32_fp64(dtype):
    """The kernel-level wrappers on fp32 / fp64 tensors, as the reference's
    Triton kernels take them (fp32 math, the input dtype stored): index
    results bit-exact, copies exact, sums and GLU within fp32 rounding of
    the oracle's."""
    from flashfusedmoe_amd.kernels import (activation_backward, activation_forward, fused_gather_reduce,
                                           fused_routing_scatter, fused_topk_routing,
                                           fused_weighted_scatter)
    N, D, E, k = 257, 64, 8, 2
    g = torch.Generator().manual_seed(31)
    logits = torch.randn(N, E, generator=g).to(dtype)
    w, idx = fused_topk_routing(logits.cuda(), "softmax", k)
    rw, ridx = R.route(logits.float().numpy(), k, "softmax")
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)
    mt = R.estimate_max_tokens(N, k, E)
    x = torch.randn(N, D, generator=g).to(dtype)
    sorted_order, counts, starts, _ = R.stable_permutation(ridx, E)
    hb, e2b = fused_routing_scatter(torch.from_numpy(sorted_order).cuda(), idx.reshape(-1),
                                    torch.from_numpy(starts).cuda(), x.cuda(), E, mt, k)
    exp_e2b, kept = R.expand_to_batch(ridx, E, mt)
    assert np.array_equal(e2b.cpu().numpy(), exp_e2b)
    exp_hb = torch.zeros(E * mt, D, dtype=dtype)
    exp_hb[torch.from_numpy(exp_e2b[kept])] = x.repeat_interleave(k, dim=0)[torch.from_numpy(kept)]
    assert torch.equal(hb.cpu(), exp_hb)
    batched = torch.randn(E * mt, D, generator=g).to(dtype)
    wt = torch.from_numpy(rw).to(dtype)
    out = fused_gather_reduce(batched.cuda(), e2b, wt.cuda(), N, k)
    exp = F_.gather_reduce(batched, torch.from_numpy(exp_e2b), wt, N, k)
    torch.testing.assert_close(out.cpu(), exp, rtol=1e-6, atol=1e-6)
    go = torch.randn(N, D, generator=g).to(dtype)
    ws = fused_weighted_scatter(go.cuda(), e2b, wt.cuda(), E, mt, k)
    exp_ws = F_.weighted_scatter(go, torch.from_numpy(exp_e2b), wt.reshape(-1), E * mt, k,
                                 torch.from_numpy(kept))
    torch.testing.assert_close(ws.cpu(), exp_ws, rtol=1e-6, atol=1e-7)
    up = (torch.randn(3, 40, 2 * 48, generator=g) * 2).to(dtype)
    ga = torch.randn(3, 40, 48, generator=g).to(dtype)
    for act in ("swiglu", "geglu", "relu_squared"):
        a = activation_forward(up.cuda(), act)
        assert a.dtype == dtype
        torch.testing.assert_close(a.cpu(), F_.glu_forward(up, act).to(dtype), rtol=1e-5, atol=1e-6)
        gu = activation_backward(ga.cuda(), up.cuda(), act)
        torch.testing.assert_close(gu.cpu(), F_.glu_backward(ga, up, act).to(dtype), rtol=1e-5, atol=1e-6)
