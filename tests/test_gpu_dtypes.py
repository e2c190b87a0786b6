"""GPU parity of the fp32 / fp64 compute path (the reference computes in the
input dtype when autocast is off, fused_moe.py:93-97, :318-327).

* The fp32 / fp64 GEMM entry points against torch fp64 products on the
  CPU, on ragged expert groups (empty experts, row counts off the 64-row
  tile, K off the 16-deep slice).
* fused_moe in fp64 against the reference's unfused test oracle
  (oracle/unfused.py, tests/conftest.py:58-137) with the reference's own
  tolerances (tests/test_generality.py:27-96: forward rel L2 < 1e-5;
  output atol 1e-6 / rtol 1e-5, weight gradients atol 1e-5 / rtol 1e-4
  against torch autograd).
* fused_moe in fp32 against the fused oracle (oracle/fused.py, the
  reference's rounding points: fp32 GEMMs, fp32 GLU / sums) on the GPU's
  own fp32 logits, routing bit-exact, losses, capacity and recompute.
* C1 (fp32) against tests/golden/c1_fp32.npz: routing
  bit-exact, output rel L2 <= 1e-6.
* MoELayer with its default fp32 parameters (no autocast) and a shared
  expert, forward and backward.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import seeded
from oracle import fused as F_
from oracle import unfused as U

pytestmark = pytest.mark.gpu

F64 = torch.float64
F32 = torch.float32


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / (b.norm() + 1e-30)).item()


def _close(actual, expected, name, rtol, atol):
    a, e = actual.detach().double().cpu(), expected.detach().double().cpu()
    assert a.shape == e.shape, name
    err = (a - e).abs()
    bound = atol + rtol * e.abs()
    worst = (err - bound).max().item()
    assert worst <= 0, f"{name}: max excess {worst:.3e} (max err {err.max().item():.3e})"


# ---------------------------------------------------------------------------
# GEMM entry points
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [F32, F64])
def test_t_gemm_entry_points_against_fp64(dtype):
    from flashfusedmoe_amd import _lib as L
    dt = 1 if dtype == F32 else 2
    g = torch.Generator().manual_seed(5)
    dev = torch.device("cuda")
    st = L.stream_ptr(dev)
    P = L.ptr
    tol = dict(rtol=1e-5, atol=1e-5) if dtype == F32 else dict(rtol=1e-12, atol=1e-12)
    # dense, all four transposition combinations, ragged sizes
    M, N, K = 77, 130, 45
    for ta in (0, 1):
        for tb in (0, 1):
            a = torch.randn(*((K, M) if ta else (M, K)), generator=g, dtype=F64)
            b = torch.randn(*((N, K) if tb else (K, N)), generator=g, dtype=F64)
            c = torch.empty(M, N, dtype=dtype, device=dev)
            ad, bd = a.to(dtype).cuda(), b.to(dtype).cuda()
            L.call("ffmoe_t_gemm_dense", dt, ta, tb, P(ad), P(bd), P(c), M, N, K, a.shape[1], b.shape[1], N,
                   0, st)
            ref = (a.to(dtype).double().t() if ta else a.to(dtype).double()) @ \
                  (b.to(dtype).double().t() if tb else b.to(dtype).double())
            _close(c, ref, f"dense ta={ta} tb={tb}", **tol)
    # grouped rows (NT and NN) and grouped K over ragged experts
    E, Kd, Nd = 5, 72, 100
    counts = torch.tensor([70, 0, 1, 129, 64])
    offs = torch.zeros(E + 1, dtype=torch.int32)
    offs[1:] = torch.cumsum(counts, 0)
    tiles = torch.zeros(E + 1, dtype=torch.int32)
    tiles[1:] = torch.cumsum((counts + 63) // 64, 0)
    T = int(offs[-1])
    a = torch.randn(T, Kd, generator=g, dtype=F64).to(dtype)
    w_nt = torch.randn(E, Nd, Kd, generator=g, dtype=F64).to(dtype)
    w_nn = torch.randn(E, Kd, Nd, generator=g, dtype=F64).to(dtype)
    ad, od, td = a.cuda(), offs.cuda(), tiles.cuda()
    for b_kn, w in ((0, w_nt), (1, w_nn)):
        c = torch.empty(T, Nd, dtype=dtype, device=dev)
        L.call("ffmoe_t_gemm_rows", dt, P(ad), P(w.cuda()), P(od), P(td), E, T, Kd, Nd, b_kn, P(c), st)
        for e in range(E):
            lo, hi = int(offs[e]), int(offs[e + 1])
            we = w[e].double().t() if b_kn == 0 else w[e].double()
            if hi > lo:
                _close(c[lo:hi], a[lo:hi].double() @ we, f"rows b_kn={b_kn} e={e}", **tol)
    b = torch.randn(T, Nd, generator=g, dtype=F64).to(dtype)
    c = torch.empty(E, Kd, Nd, dtype=dtype, device=dev)
    L.call("ffmoe_t_gemm_wgrad", dt, P(ad), P(b.cuda()), P(od), E, Kd, Nd, P(c), st)
    for e in range(E):
        lo, hi = int(offs[e]), int(offs[e + 1])
        _close(c[e], a[lo:hi].double().t() @ b[lo:hi].double(), f"wgrad e={e}", **tol)
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# fp64: the reference's generality tests
# ---------------------------------------------------------------------------

def _gen_inputs(N, D, ffn, E, dtype, seed=42, gate_scale=0.01):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, D, generator=g, dtype=F64)
    gate = torch.randn(E, D, generator=g, dtype=F64) * gate_scale
    wu = torch.randn(E, ffn, D, generator=g, dtype=F64) * (2.0 / D) ** 0.5
    wd = torch.randn(E, D, ffn // 2, generator=g, dtype=F64) * (2.0 / (ffn // 2)) ** 0.5
    return [t.to(dtype) for t in (x, gate, wu, wd)]


@pytest.mark.parametrize("D", [64, 256, 1024])
@pytest.mark.parametrize("activation", ["swiglu", "geglu", "relu_squared"])
@pytest.mark.parametrize("gating", ["softmax", "sigmoid"])
def test_fp64_forward_matches_unfused(D, activation, gating):
    """tests/test_generality.py:27-51: N 64, E 8, k 2, ffn 3D, rel L2 < 1e-5."""
    from flashfusedmoe_amd import fused_moe
    x, gate, wu, wd = _gen_inputs(64, D, 3 * D, 8, F64)
    out, _ = fused_moe(x.cuda(), gate.cuda(), wu.cuda(), wd.cuda(), 2, activation=activation,
                       gating=gating)
    assert out.dtype == F64
    ref, _, _, _ = U.unfused_moe(x, gate, wu, wd, 2, activation=activation, gating=gating)
    assert _rel(out, ref) < 1e-5


@pytest.mark.parametrize("activation", ["swiglu", "geglu", "relu_squared"])
@pytest.mark.parametrize("gating", ["softmax", "sigmoid"])
def test_fp64_gradients_match_autograd(activation, gating):
    """tests/test_generality.py:58-96 (N 16, D 64, ffn 128, E 4, k 2, all
    weights x0.1): output and weight gradients against torch autograd
    through the unfused oracle with the reference's tolerances; the hidden
    and gate gradients too, at the weight-gradient tolerance."""
    from flashfusedmoe_amd import fused_moe
    g = torch.Generator().manual_seed(42)
    N, D, ffn, E, k = 16, 64, 128, 4, 2
    data = [torch.randn(N, D, generator=g, dtype=F64), torch.randn(E, D, generator=g, dtype=F64) * 0.1,
            torch.randn(E, ffn, D, generator=g, dtype=F64) * 0.1,
            torch.randn(E, D, ffn // 2, generator=g, dtype=F64) * 0.1]
    go = torch.randn(N, D, generator=g, dtype=F64)
    leaves = [t.cuda().requires_grad_(True) for t in data]
    out, _ = fused_moe(*leaves, k, activation=activation, gating=gating)
    out.backward(go.cuda())
    ref_leaves = [t.clone().requires_grad_(True) for t in data]
    ref, _, _, _ = U.unfused_moe(*ref_leaves, k, activation=activation, gating=gating)
    ref.backward(go)
    _close(out, ref, "output", rtol=1e-5, atol=1e-6)
    for name, a, b in zip(("hidden", "gate", "w_up", "w_down"), leaves, ref_leaves):
        _close(a.grad, b.grad, f"grad {name}", rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("E,k", [(4, 1), (8, 2), (16, 4), (64, 8)])
def test_fp64_expert_configs(E, k):
    """tests/test_generality.py:121-136: N 128, D 512, ffn 1024."""
    from flashfusedmoe_amd import fused_moe
    x, gate, wu, wd = _gen_inputs(128, 512, 1024, E, F64)
    out, _ = fused_moe(x.cuda(), gate.cuda(), wu.cuda(), wd.cuda(), k)
    ref, _, _, _ = U.unfused_moe(x, gate, wu, wd, k)
    assert _rel(out, ref) < 1e-5


# ---------------------------------------------------------------------------
# fp32 against the fused oracle
# ---------------------------------------------------------------------------

def _fp32_case(N, D, ffn, E, k, gating, activation, capacity_factor=None, recompute=False, seed=3):
    from flashfusedmoe_amd import fused_moe, ops
    x, gate, wu, wd = (t.float() for t in seeded(N, D, ffn, E, seed=seed))
    go = torch.randn(N, D, generator=torch.Generator().manual_seed(seed + 1))
    leaves = [t.cuda().requires_grad_(True) for t in (x, gate, wu, wd)]
    out, losses = fused_moe(*leaves, top_k=k, gating=gating, activation=activation,
                            capacity_factor=capacity_factor, aux_loss_coeff=0.01, z_loss_coeff=1e-3,
                            allow_dropped_tokens=True, recompute_activations=recompute,
                            return_metrics=True)
    one = torch.ones((), device="cuda")
    outs, grads_in = [out, losses["z_loss"]], [go.cuda(), one]
    if losses["aux_loss"].requires_grad:  # sigmoid gating only (softmax aux has no gradient)
        outs.append(losses["aux_loss"])
        grads_in.append(one)
    torch.autograd.backward(outs, grads_in)
    torch.cuda.synchronize()
    logits = ops.route(x.cuda(), gate.cuda(), None, k, 0 if gating == "softmax" else 1, 1, 0.0, 0.0,
                       False)[0].cpu()
    return (x, gate, wu, wd, go), out.detach().cpu(), losses, [t.grad.cpu() for t in leaves], logits


@pytest.mark.parametrize("gating", ["softmax", "sigmoid"])
@pytest.mark.parametrize("activation", ["swiglu", "geglu", "relu_squared"])
def test_fp32_forward_backward_matches_oracle(gating, activation):
    N, D, ffn, E, k = 512, 128, 256, 8, 2
    (x, gate, wu, wd, go), out, losses, grads, logits = _fp32_case(N, D, ffn, E, k, gating, activation)
    assert logits.dtype == F32
    # the gate product in fp32 against fp64, then routing bit-exact on it
    exact = x.double() @ gate.double().t()
    assert (logits.double() - exact).abs().max().item() <= 1e-5 * max(1.0, exact.abs().max().item())
    r_out, st = F_.forward(x, gate, wu, wd, k, activation=activation, gating=gating,
                           allow_dropped_tokens=True, logits=logits)
    gr = F_.backward(st, go)
    _close(out, r_out, "output", rtol=1e-4, atol=1e-5)
    lg = F_.loss_grads(logits, st["topk_idx"], E, gating, 0.01, 1e-3).double()
    ref = {"hidden": gr["hidden"].double() + lg @ gate.double(),
           "gate": gr["gate"].double() + lg.t() @ x.double(),
           "w_up": gr["w_up"], "w_down": gr["w_down"]}
    for name, g in zip(("hidden", "gate", "w_up", "w_down"), grads):
        scale = ref[name].abs().max().item()
        _close(g, ref[name], f"grad {name}", rtol=1e-4, atol=1e-5 * max(1.0, scale))
    lo = F_.losses(logits, st["topk_w"], st["topk_idx"], E, gating=gating, aux_loss_coeff=0.01,
                   z_loss_coeff=1e-3)
    for key in ("aux_loss", "z_loss"):
        assert abs(losses[key].item() - lo[key].item()) <= 1e-5 * abs(lo[key].item()) + 1e-9, key
    counts = np.bincount(st["topk_idx"].reshape(-1).numpy(), minlength=E)
    assert np.array_equal(losses["tokens_per_expert"].cpu().numpy(), counts)


def test_fp32_capacity_and_recompute():
    """Capacity dropping (keep + renormalise) in fp32 against the oracle, and
    recompute_activations bitwise equal to the saved-activation run."""
    N, D, ffn, E, k = 300, 64, 128, 4, 2
    (x, gate, wu, wd, go), out, _, grads, logits = _fp32_case(N, D, ffn, E, k, "softmax", "swiglu",
                                                              capacity_factor=1.0, seed=9)
    r_out, st = F_.forward(x, gate, wu, wd, k, capacity_factor=1.0, logits=logits)
    assert not st["keep"].all()  # the drop ran
    _close(out, r_out, "output (capacity)", rtol=1e-4, atol=1e-5)
    gr = F_.backward(st, go)
    _close(grads[2], gr["w_up"], "grad w_up (capacity)", rtol=1e-4, atol=1e-5)
    _, out2, _, grads2, _ = _fp32_case(N, D, ffn, E, k, "softmax", "swiglu", capacity_factor=1.0, seed=9,
                                       recompute=True)
    assert torch.equal(out, out2)
    for a, b in zip(grads, grads2):
        assert torch.equal(a, b)


def test_c1_fp32_matches_golden():
    """BASELINE configs[0] in fp32 without autocast: routing indices equal to
    the golden fixture's, weights to 2e-6, output rel L2 <= 1e-6."""
    import golden as G
    from flashfusedmoe_amd import fused_moe
    f = G.load("c1_fp32")
    x, gate, wu, wd = (t.cuda() for t in G.c1_inputs())
    out, losses = fused_moe(x, gate, wu, wd, top_k=G.C1["top_k"], return_metrics=True)
    assert out.dtype == F32
    from flashfusedmoe_amd import ops
    res = ops.route(x, gate, None, G.C1["top_k"], 0, 1, 0.0, 0.0, False)
    assert np.array_equal(res[1].cpu().numpy(), f["topk_idx"])
    np.testing.assert_allclose(res[2].cpu().numpy(), f["topk_w"], rtol=2e-6, atol=1e-7)
    assert _rel(out, torch.from_numpy(f["out"])) <= 1e-6
    counts = np.bincount(f["topk_idx"].reshape(-1).astype(np.int64), minlength=G.C1["E"])
    assert np.array_equal(losses["tokens_per_expert"].cpu().numpy(), counts)


def test_moelayer_fp32_default_parameters_with_shared_expert():
    """MoELayer as constructed (fp32 parameters), no autocast: the routed
    part against the fused oracle on the GPU's logits, the shared expert
    against torch autograd through the reference formula (nn.py:22-44), in
    fp64 on the CPU."""
    from flashfusedmoe_amd import MoELayer, ops
    torch.manual_seed(3)
    D, ffn, E, k, N = 128, 256, 8, 2, 256
    layer = MoELayer(D, ffn, E, top_k=k, activation="geglu", num_shared_experts=1)
    params = {n: p.detach().clone() for n, p in layer.named_parameters()}
    layer = layer.cuda()
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, N // 2, D, generator=g)
    go = torch.randn(2, N // 2, D, generator=g)
    xg = x.cuda().requires_grad_(True)
    out, _ = layer(xg)
    assert out.dtype == F32
    out.backward(go.cuda())
    torch.cuda.synchronize()
    xf = x.reshape(N, D)
    gate, wu, wd = params["gate.weight"], params["w_up"], params["w_down"]
    logits = ops.route(xf.cuda(), gate.cuda(), None, k, 0, 1, 0.0, 0.0, False)[0].cpu()
    r_out, st = F_.forward(xf, gate, wu, wd, k, activation="geglu", allow_dropped_tokens=True, logits=logits)
    gr = F_.backward(st, go.reshape(N, D))
    sw = [params[f"shared_expert.{n}.weight"].double().requires_grad_(True) for n in ("w_gate", "w_up", "w_down")]
    xs = xf.double().requires_grad_(True)
    s_out = U.shared_expert(xs, *sw, activation="geglu")
    s_out.backward(go.reshape(N, D).double())
    _close(out.reshape(N, D), r_out.double() + s_out.detach(), "output", rtol=1e-4, atol=1e-5)
    _close(xg.grad.reshape(N, D), gr["hidden"].double() + xs.grad, "grad hidden", rtol=1e-4, atol=1e-5)
    grads = {n: p.grad.cpu() for n, p in layer.named_parameters()}
    _close(grads["w_up"], gr["w_up"], "grad w_up", rtol=1e-4, atol=1e-5)
    _close(grads["w_down"], gr["w_down"], "grad w_down", rtol=1e-4, atol=1e-5)
    _close(grads["gate.weight"], gr["gate"], "grad gate", rtol=1e-4, atol=1e-5)
    for name, w in zip(("w_gate", "w_up", "w_down"), sw):
        _close(grads[f"shared_expert.{name}.weight"], w.grad, f"grad shared {name}", rtol=1e-4, atol=1e-5)


def test_fp16_compute_raises():
    from flashfusedmoe_amd import fused_moe
    x, gate, wu, wd = (t.half().cuda() for t in seeded(64, 64, 128, 4, seed=1))
    with pytest.raises(TypeError, match="bfloat16, float32 or float64"):
        fused_moe(x, gate, wu, wd, top_k=2)
