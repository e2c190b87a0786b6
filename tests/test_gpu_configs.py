"""GPU parity at the full sizes of BASELINE.json's other configurations:

* C3: Mixtral-shaped decode batch, forward only (N 64, D 4096, ffn 28672,
  E 8, k 2), about 2.8 GB of expert weights;
* C4: fine-grained, load-imbalanced layer, forward + backward (N 16384,
  D 2048, ffn 2816, E 64, k 8) with a per-expert Zipf bias (s = 1.1) that
  skews the expert counts;
* C5: DeepSeek-V3-style layer, forward + backward (N 4096, D 7168, E 256,
  ffn 4096, k 8), about 23 GB of expert weights, and its shared expert.

The CPU oracle does not finish these sizes in seconds, so the expected values
come from a plain fp32 PyTorch restatement on the GPU of the same algorithm
with the oracle's rounding points (tests/gpu_helpers.moe_reference; its GLU
math is the oracle's own, device-agnostic glu_forward / glu_backward).
Routing is checked bit-exact against the CPU oracle's top-k on the GPU's own
logits (a [N, E] problem the oracle finishes quickly); everything else within
the bf16 tolerance of gpu_helpers.check_close.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import check_close, moe_reference
from oracle import fused as F_
from oracle import routing as R

pytestmark = pytest.mark.gpu


def _randn(shape, std, gen):
    return (torch.randn(shape, device="cuda", generator=gen) * std).to(torch.bfloat16)


def _check_routing(logits, idx, w, k, bias=None):
    if bias is None:
        rw, ridx = R.route(logits.float().cpu().numpy(), k)
        np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)
        assert np.array_equal(idx.cpu().numpy(), ridx)
    else:
        rw, ridx = F_.route_advanced(logits.cpu(), "softmax", k, bias.cpu(), False, None, None, None)
        assert np.array_equal(idx.cpu().numpy(), ridx.numpy())
        np.testing.assert_allclose(w.cpu().numpy(), rw.numpy(), rtol=2e-6, atol=1e-7)


def _run(x, gate, wu, wd, k, go=None, bias=None, **kw):
    from flashfusedmoe_amd import fused_moe, ops
    leaves = [t.requires_grad_(go is not None) for t in (x, gate, wu, wd)]
    out, _ = fused_moe(*leaves, top_k=k, expert_bias=bias, **kw)
    if go is not None:
        out.backward(go)
    torch.cuda.synchronize()
    r = ops.route(x.detach(), gate.detach(), bias, k, 0, x.shape[0] * k, 0.0, 0.0, False)
    return out.detach(), [t.grad for t in leaves], r[0], r[1], r[2]


def test_c3_decode_forward():
    g = torch.Generator(device="cuda").manual_seed(3)
    N, D, ffn, E, k = 64, 4096, 28672, 8, 2
    H = ffn // 2
    x = _randn((N, D), 1.0, g)
    gate = _randn((E, D), 0.02, g)
    wu = _randn((E, ffn, D), 0.02, g)
    wd = _randn((E, D, H), 0.02, g)
    out, _, logits, idx, w = _run(x, gate, wu, wd, k)
    _check_routing(logits, idx, w, k)
    ref = moe_reference(x, gate, wu, wd, idx, w)
    check_close(out, ref["out"], "C3 output")


def test_c4_skewed_forward_backward():
    g = torch.Generator(device="cuda").manual_seed(4)
    N, D, ffn, E, k = 16384, 2048, 2816, 64, 8
    x = _randn((N, D), 1.0, g)
    gate = _randn((E, D), 0.02, g)
    wu = _randn((E, ffn, D), D ** -0.5, g)
    wd = _randn((E, D, ffn // 2), (ffn // 2) ** -0.5, g)
    go = _randn((N, D), 1.0, g)
    ranks = torch.randperm(E, generator=torch.Generator().manual_seed(4)).float() + 1.0
    pz = ranks ** -1.1
    bias = (2.0 * torch.log(pz / pz.sum())).cuda()
    out, grads, logits, idx, w = _run(x, gate, wu, wd, k, go=go, bias=bias,
                                      max_tokens_per_expert=N * k)
    _check_routing(logits, idx, w, k, bias)
    counts = torch.bincount(idx.reshape(-1), minlength=E)
    assert counts.max().item() > 4 * counts.float().mean().item()  # the skew is real
    ref = moe_reference(x, gate, wu, wd, idx, w, go)
    check_close(out, ref["out"], "C4 output")
    check_close(grads[0], ref["dx"], "C4 grad hidden")
    check_close(grads[1], ref["dgate"], "C4 grad gate",
                atol=2e-3 * max(1.0, ref["dgate"].abs().max().item()))
    for e in range(E):  # per expert, so the comparison stays on the GPU's scale
        check_close(grads[2][e], ref["dwu"][e], f"C4 grad w_up[{e}]",
                    atol=2e-3 * max(1.0, ref["dwu"][e].abs().max().item()))
        check_close(grads[3][e], ref["dwd"][e], f"C4 grad w_down[{e}]",
                    atol=2e-3 * max(1.0, ref["dwd"][e].abs().max().item()))


def test_c5_deepseek_forward_backward():
    g = torch.Generator(device="cuda").manual_seed(5)
    N, D, ffn, E, k = 4096, 7168, 4096, 256, 8
    x = _randn((N, D), 1.0, g)
    gate = _randn((E, D), 0.006, g)
    wu = _randn((E, ffn, D), 0.006, g)
    wd = _randn((E, D, ffn // 2), 0.006, g)
    go = _randn((N, D), 1.0, g)
    out, grads, logits, idx, w = _run(x, gate, wu, wd, k, go=go, max_tokens_per_expert=N * k)
    _check_routing(logits, idx, w, k)
    sample = torch.randperm(E, generator=torch.Generator().manual_seed(5))[:16].tolist()
    ref = moe_reference(x, gate, wu, wd, idx, w, go, wgrad_experts=sample)
    check_close(out, ref["out"], "C5 output")
    check_close(grads[0], ref["dx"], "C5 grad hidden")
    check_close(grads[1], ref["dgate"], "C5 grad gate",
                atol=2e-3 * max(1.0, ref["dgate"].abs().max().item()))
    for e in sample:
        check_close(grads[2][e], ref["dwu"][e], f"C5 grad w_up[{e}]",
                    atol=2e-3 * max(1.0, ref["dwu"][e].abs().max().item()))
        check_close(grads[3][e], ref["dwd"][e], f"C5 grad w_down[{e}]",
                    atol=2e-3 * max(1.0, ref["dwd"][e].abs().max().item()))


def test_c5_shared_expert():
    from flashfusedmoe_amd import ops
    g = torch.Generator(device="cuda").manual_seed(6)
    N, D, H = 4096, 7168, 2048
    x = _randn((N, D), 1.0, g)
    w_gu = _randn((2 * H, D), 0.006, g)
    wd = _randn((D, H), 0.006, g)
    go = _randn((N, D), 1.0, g)
    out, up, act = ops.dense_glu_forward(x, w_gu, wd, 0)
    dx, dwgu, dwd = ops.dense_glu_backward(go, x, w_gu, wd, up, act, 0)
    up_ref = F_.gemm(x, w_gu.t())
    check_close(up, up_ref, "C5 shared up")
    act_ref = F_.glu_forward(up, "swiglu")
    check_close(act, act_ref, "C5 shared act")
    check_close(out, F_.gemm(act, wd.t()), "C5 shared out")
    gup = F_.glu_backward(F_.gemm(go, wd), up, "swiglu")
    check_close(dx, F_.gemm(gup, w_gu), "C5 shared grad x")
    check_close(dwd, F_.gemm(go.t(), act), "C5 shared grad w_down")
    ref = F_.gemm(gup.t(), x)
    check_close(dwgu, ref, "C5 shared grad w_gate|w_up",
                atol=2e-3 * max(1.0, ref.abs().max().item()))
