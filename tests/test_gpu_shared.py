"""GPU parity of the shared expert (reference nn.py:22-44, added to the routed
output at nn.py:156-159), which this build runs through the grouped-GEMM
kernels as one dense row group with the GLU fused into the epilogues.

* ops.dense_glu_forward / dense_glu_backward against plain fp32 PyTorch
  (torch.erf for the shared expert's exact GELU), from the kernels' own bf16
  intermediates, for the three activations.
* MoELayer(num_shared_experts=1) forward + backward: the routed part against
  the CPU oracle (routing bit-exact on the GPU's logits), the shared part
  against torch autograd through the reference's three-linear formula on the
  CPU (_GLUFFN.forward), every parameter gradient within the bf16 tolerance.
"""

import ctypes

import pytest
import torch
import torch.nn.functional as F

from gpu_helpers import check_close
from oracle import fused as F_

pytestmark = pytest.mark.gpu

ACTS = ["swiglu", "geglu", "relu_squared"]


def _act_ref(name, g, u):
    if name == "swiglu":
        return F.silu(g) * u
    if name == "geglu":  # exact erf GELU, as F.gelu in the reference's shared expert
        return 0.5 * g * (1.0 + torch.erf(g * 0.7071067811865476)) * u
    return F.relu(g).square() * u


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("N,D,H", [(1000, 256, 192), (4096, 1024, 2048), (7, 64, 32)])
def test_dense_glu_against_fp32(act, N, D, H):
    from flashfusedmoe_amd import ops
    from flashfusedmoe_amd.nn import _SHARED_ACT
    g = torch.Generator().manual_seed(N + D + H)
    x = torch.randn(N, D, generator=g).to(torch.bfloat16).cuda()
    w_gu = (torch.randn(2 * H, D, generator=g) * D ** -0.5).to(torch.bfloat16).cuda()
    wd = (torch.randn(D, H, generator=g) * H ** -0.5).to(torch.bfloat16).cuda()
    go = torch.randn(N, D, generator=g).to(torch.bfloat16).cuda()
    a = _SHARED_ACT[act]
    out, up, actv = ops.dense_glu_forward(x, w_gu, wd, a)
    dx, dwgu, dwd = ops.dense_glu_backward(go, x, w_gu, wd, up, actv, a)
    torch.cuda.synchronize()
    f = lambda t: t.float()  # noqa: E731
    check_close(up, f(x) @ f(w_gu).t(), "up")
    gg, uu = f(up[:, :H]).requires_grad_(True), f(up[:, H:]).requires_grad_(True)
    ref_act = _act_ref(act, gg, uu)
    check_close(actv, ref_act, "act")
    check_close(out, f(actv) @ f(wd).t(), "out")
    gact = (f(go) @ f(wd)).to(torch.bfloat16).float()
    dg, du = torch.autograd.grad(ref_act, (gg, uu), gact)
    gup = torch.cat([dg, du], 1)
    dwgu_ref = gup.t() @ f(x)
    dx_ref = gup @ f(w_gu)
    check_close(dx, dx_ref, "grad x", atol=2e-3 * max(1.0, dx_ref.abs().max().item()))
    check_close(dwd, f(go).t() @ f(actv), "grad w_down")
    check_close(dwgu, dwgu_ref, "grad w_gate|w_up",
                atol=2e-3 * max(1.0, dwgu_ref.abs().max().item()))


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("D,ffn,fold", [(128, 256, True), (136, 208, False)])
def test_moelayer_shared_expert_forward_backward(act, D, ffn, fold):
    """fold: D and ffn/2 multiples of 64, the shared expert runs as a dense
    row group of the routed GEMM launches; otherwise as its own dense GEMMs
    (ffmoe_glu_fwd / ffmoe_glu_bwd between them)."""
    from flashfusedmoe_amd import MoELayer
    from flashfusedmoe_amd import _lib as L
    from flashfusedmoe_amd import ops
    torch.manual_seed(3)
    E, k, N = 8, 2, 512
    layer = MoELayer(D, ffn, E, top_k=k, activation=act, num_shared_experts=1)
    layer = layer.to(torch.bfloat16)
    ref_shared = layer.shared_expert  # CPU copy of the parameters (reference formula)
    params_cpu = {n: p.detach().clone() for n, p in layer.named_parameters()}
    layer = layer.cuda()
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, N // 2, D, generator=g).to(torch.bfloat16)
    go = torch.randn(2, N // 2, D, generator=g).to(torch.bfloat16)
    xg = x.cuda().requires_grad_(True)
    called = []
    L.call_hook = lambda name, phase: called.append(name) if phase == 0 else None
    try:
        out, _ = layer(xg)
        out.backward(go.cuda())
        torch.cuda.synchronize()
    finally:
        L.call_hook = None
    assert ("ffmoe_glu_fwd" in called) == (not fold)
    assert ("ffmoe_glu_bwd" in called) == (not fold)

    # routed part: the oracle on the GPU's own gate logits
    xf = x.reshape(N, D)
    gate, wu, wd = params_cpu["gate.weight"], params_cpu["w_up"], params_cpu["w_down"]
    logits = ops.route(xf.cuda(), gate.cuda(), None, 1, 0, 1, 0.0, 0.0, False)[0].cpu()
    r_out, st = F_.forward(xf, gate, wu, wd, k, activation=act, allow_dropped_tokens=True,
                           logits=logits)
    gr = F_.backward(st, go.reshape(N, D))
    # shared part: torch autograd through the reference formula on the CPU
    sh = ref_shared.__class__(D, ffn, act).to(torch.bfloat16)
    with torch.no_grad():
        for name in ("w_gate", "w_up", "w_down"):
            getattr(sh, name).weight.copy_(params_cpu[f"shared_expert.{name}.weight"])
    xs = xf.clone().requires_grad_(True)
    s_out = sh(xs)
    s_out.backward(go.reshape(N, D))

    exp_out = r_out.float() + s_out.detach().float()
    check_close(out.detach().cpu().reshape(N, D), exp_out, "output")
    exp_dx = gr["hidden"].float() + xs.grad.float()
    check_close(xg.grad.cpu().reshape(N, D), exp_dx, "grad hidden")
    grads = {n: p.grad.cpu() for n, p in layer.named_parameters()}
    check_close(grads["gate.weight"], gr["gate"], "grad gate",
                atol=2e-3 * max(1.0, gr["gate"].abs().max().item()))
    check_close(grads["w_up"], gr["w_up"], "grad w_up")
    check_close(grads["w_down"], gr["w_down"], "grad w_down")
    for name in ("w_gate", "w_up", "w_down"):
        ref = getattr(sh, name).weight.grad
        check_close(grads[f"shared_expert.{name}.weight"], ref, f"grad shared {name}",
                    atol=2e-3 * max(1.0, ref.abs().max().item()))


@pytest.mark.parametrize("rows,split", [(5000, True), (4095, False), (300, False)])
def test_wgrad_dense_group_split_k(rows, split):
    """ffmoe_gemm_wgrad_shared with the persistent GEMMs' workspace: a dense
    group of >= 4096 rows has its K cut into two halves (here 2560 + 2440
    rows), each tile finished by the half that arrives second.  Checked
    against fp64 (routed experts and the dense group), bit-identical over
    two calls (the two fp32 halves are added in either order: the same
    bits), and without the workspace (one K range) to within bf16
    rounding of the output.  The routed experts' outputs are unaffected."""
    from flashfusedmoe_amd import _lib as L
    g = torch.Generator().manual_seed(rows)
    E, M, Nc = 4, 512, 768
    counts = torch.tensor([700, 0, 1300, 333])
    offs = torch.zeros(E + 1, dtype=torch.int32)
    offs[1:] = torch.cumsum(counts, 0)
    T = int(offs[-1])
    a = torch.randn(T, M, generator=g).to(torch.bfloat16)
    b = torch.randn(T, Nc, generator=g).to(torch.bfloat16)
    xa = torch.randn(rows, M, generator=g).to(torch.bfloat16)
    xb = torch.randn(rows, Nc, generator=g).to(torch.bfloat16)
    dev = torch.device("cuda")
    a_d, b_d, xa_d, xb_d, offs_d = (t.to(dev) for t in (a, b, xa, xb, offs))
    st = L.stream_ptr(dev)
    ws = L.gemm_workspace(dev, st)

    def run(workspace):
        c = torch.empty(E, M, Nc, dtype=torch.bfloat16, device=dev)
        xc = torch.empty(M, Nc, dtype=torch.bfloat16, device=dev)
        grp = L.dense_group(xa_d, xb_d, xc, rows, 0)
        L.call("ffmoe_gemm_wgrad_shared", L.ptr(a_d), L.ptr(b_d), L.ptr(offs_d), E, M, Nc, L.ptr(c),
               ctypes.byref(grp), workspace, st)
        return c, xc

    c1, x1 = run(L.ptr(ws))
    c2, x2 = run(L.ptr(ws))
    c0, x0 = run(None)
    L.check_gemm_workspaces()  # no cut tile's wait timed out; flags left clear
    torch.cuda.synchronize()
    assert torch.equal(x1, x2) and torch.equal(c1, c2)
    assert torch.equal(c1, c0)  # routed experts: same kernel path either way
    f = torch.float64
    exp_x = xa.to(f).t() @ xb.to(f)
    check_close(x1, exp_x, "dense group (split)" if split else "dense group")
    for e in range(E):
        lo, hi = int(offs[e]), int(offs[e + 1])
        exp = a[lo:hi].to(f).t() @ b[lo:hi].to(f)
        if hi > lo:
            check_close(c1[e], exp, f"expert {e}")
    d = (x1.double() - x0.double()).abs()
    if split:  # different fp32 summation grouping: at most bf16 rounding apart
        assert (d <= 2.0 ** -7 * x0.double().abs() + 1e-2).all()
    else:
        assert torch.equal(x1, x0)
    assert not ws[:8192].any()  # the cut-tile counters and publications were cleared
