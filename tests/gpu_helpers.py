"""Helpers shared by the GPU parity tests."""

import ctypes
import os

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE_LIB = os.path.join(ROOT, "tests", "hip", "libtrprobe.so")

# bf16 tolerance of the HIP path against the CPU oracle with the reference's
# rounding points: rtol 2e-2 / atol 2e-3 (fp32 accumulation).  Elementwise,
# at most 0.1% of the elements may exceed atol + rtol*|expected| (a bf16
# rounding flip upstream of a cancellation), and the relative L2 error must
# stay below rtol.
RTOL = 2e-2
ATOL = 2e-3


def check_close(actual, expected, name, rtol=RTOL, atol=ATOL, max_bad_frac=1e-3):
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    err = (a - e).abs()
    rel_l2 = (err.norm() / (e.norm() + 1e-30)).item()
    bad = (err > atol + rtol * e.abs()).double().mean().item()
    scale = e.abs().max().item()
    assert rel_l2 < rtol, f"{name}: relative L2 error {rel_l2:.3e} >= {rtol}"
    assert bad <= max_bad_frac, f"{name}: {bad:.2e} of elements outside atol+rtol*|e|"
    assert err.max().item() <= 10 * (atol + rtol * scale), \
        f"{name}: max abs error {err.max().item():.3e} (scale {scale:.3e})"
    return rel_l2


def check_as_accurate(actual, oracle_bf16, exact, name, slack=1.25):
    """The HIP result is at least about as close to an fp64 restatement as
    the bf16 oracle is: relative L2 error against ``exact`` within ``slack``
    times the oracle's own."""
    a, o, t = (v.detach().double().cpu() for v in (actual, oracle_bf16, exact))
    ea = ((a - t).norm() / t.norm()).item()
    eo = ((o - t).norm() / t.norm()).item()
    assert ea <= slack * eo + 1e-7, f"{name}: error vs fp64 {ea:.3e} > {slack} x oracle's {eo:.3e}"
    return ea, eo


def seeded(N, D, ffn, E, seed=0, gate_scale=None, w_scale=None, dtype=torch.bfloat16):
    """Inputs generated on the CPU in fp32 then cast: CPU oracle and GPU see
    identical bits.  Default weights ~ N(0, 1/fan_in)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, D, generator=g)
    gs = gate_scale if gate_scale is not None else D ** -0.5
    gate = torch.randn(E, D, generator=g) * gs
    wu = torch.randn(E, ffn, D, generator=g) * (w_scale if w_scale is not None else D ** -0.5)
    wd = torch.randn(E, D, ffn // 2, generator=g) * (w_scale if w_scale is not None else (ffn // 2) ** -0.5)
    return tuple(t.to(dtype) for t in (x, gate, wu, wd))


def cuda(*ts):
    return tuple(t.cuda() for t in ts)


def probe_lds_transpose():
    lib = ctypes.CDLL(PROBE_LIB)
    lib.ffmoe_probe_lds_tr.argtypes = [ctypes.c_void_p]
    lib.ffmoe_probe_lds_tr.restype = ctypes.c_int
    out = torch.zeros(64 * 4, dtype=torch.int16, device="cuda")
    assert lib.ffmoe_probe_lds_tr(out.data_ptr()) == 0
    return out.cpu().numpy().astype(np.uint16).reshape(64, 4)


def expected_rows(idx, E, mt, capacity_mode):
    """Compact row of every entry from the oracle's stable permutation."""
    from oracle import routing as R
    idx = np.asarray(idx)
    _, counts, _, rank = R.stable_permutation(idx, E)
    rows = np.minimum(counts, mt)
    off = np.zeros(E + 1, dtype=np.int64)
    off[1:] = np.cumsum(rows)
    flat = idx.reshape(-1)
    own = rank < mt
    out = np.where(own, off[flat] + rank, -1)
    if not capacity_mode and counts[0] > 0:
        out = np.where(own, out, -2)
    return out, counts, off


def moe_reference(x, gate, wu, wd, idx, w, go=None, activation="swiglu", wgrad_experts=None):
    """fp32 PyTorch restatement on the GPU of the fused MoE forward and
    backward for a given routing (idx [N,k] int64, w [N,k] fp32), with the
    oracle's rounding points (oracle/fused.py forward/backward): up, act and
    down rounded to bf16; the combine in fp32 slot order with bf16 weights;
    the weighted grad rows go*bf16(w) rounded to bf16; the top-k softmax
    backward in fp32 over the selected slots; grad_logits rounded to bf16
    before both gate products.  No token is dropped; no aux / z terms.
    Returns dict(out, dx, dgate, dwu, dwd), the weight gradients as
    {expert: tensor} for wgrad_experts (default: all)."""
    from oracle import fused as F_
    bf = torch.bfloat16
    N, D = x.shape
    E = wu.shape[0]
    H = wd.shape[2]
    k = idx.shape[1]
    T = N * k
    dev = x.device
    flat = idx.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=E).tolist()
    starts = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    pos = torch.empty_like(order)
    pos[order] = torch.arange(T, device=dev)
    xs = x[order // k]
    up = torch.empty(T, 2 * H, dtype=bf, device=dev)
    act = torch.empty(T, H, dtype=bf, device=dev)
    down = torch.empty(T, D, dtype=bf, device=dev)
    for e in range(E):
        r0, r1 = int(starts[e]), int(starts[e + 1])
        if r1 > r0:
            up[r0:r1] = F_.gemm(xs[r0:r1], wu[e].t())
            act[r0:r1] = F_.glu_forward(up[r0:r1], activation)
            down[r0:r1] = F_.gemm(act[r0:r1], wd[e].t())
    wb = w.to(bf).float()
    dn = down[pos].view(N, k, D).float()
    acc = torch.zeros(N, D, device=dev)
    for s in range(k):
        acc = acc + dn[:, s] * wb[:, s:s + 1]
    res = {"out": acc.to(bf)}
    if go is None:
        return res
    gof = go.float()
    g_w = (dn * gof[:, None, :]).sum(-1)
    del dn, acc
    wgo = (gof[:, None, :] * wb[:, :, None]).to(bf).view(T, D)[order]
    gup = torch.empty(T, 2 * H, dtype=bf, device=dev)
    ghb = torch.empty(T, D, dtype=bf, device=dev)
    experts = set(range(E) if wgrad_experts is None else wgrad_experts)
    dwu, dwd = {}, {}
    for e in range(E):
        r0, r1 = int(starts[e]), int(starts[e + 1])
        if r1 > r0:
            gact = F_.gemm(wgo[r0:r1], wd[e])
            gup[r0:r1] = F_.glu_backward(gact, up[r0:r1], activation)
            ghb[r0:r1] = F_.gemm(gup[r0:r1], wu[e])
        if e in experts:
            if r1 > r0:
                dwd[e] = F_.gemm(wgo[r0:r1].t(), act[r0:r1])
                dwu[e] = F_.gemm(gup[r0:r1].t(), xs[r0:r1])
            else:
                dwd[e] = torch.zeros(D, H, dtype=bf, device=dev)
                dwu[e] = torch.zeros(2 * H, D, dtype=bf, device=dev)
    rows = ghb[pos].view(N, k, D).float()
    gh = torch.zeros(N, D, device=dev)
    for s in range(k):
        gh = gh + rows[:, s]
    gh = gh.to(bf)
    gtl = w * (g_w - (g_w * w).sum(-1, keepdim=True))
    gl = torch.zeros(N, E, device=dev).scatter_add_(1, idx, gtl).to(bf)
    res["dx"] = (gh.float() + F_.gemm(gl, gate).float()).to(bf)
    res["dgate"] = F_.gemm(gl.t().contiguous(), x)
    res["dwu"], res["dwd"] = dwu, dwd
    return res


def exact_expert_wgrads(x, wu, wd, idx, w, go, experts):
    """fp64 restatement (no intermediate rounding) of the SwiGLU experts'
    weight gradients for a given routing, for the experts listed: rows of
    expert e in ascending j = n*k + slot order, up = x w_up[e]^T,
    act = silu(g) * u, wgo = go[n] * bf16(w[n, slot]) (the combine weights
    are bf16 on both sides, fused_moe.py:412), gact = wgo w_down[e],
    dW_down = wgo^T act, dW_up = gup^T x with gup the SwiGLU backward.
    Returns ({e: dW_up}, {e: dW_down}) in fp64 on x's device."""
    f = torch.float64
    N, k = idx.shape
    H = wd.shape[2]
    flat = idx.reshape(-1)
    dwu, dwd = {}, {}
    for e in experts:
        j = torch.nonzero(flat == e).flatten()
        n = j // k
        xs = x[n].to(f)
        up = xs @ wu[e].to(f).t()
        g, u = up[:, :H], up[:, H:]
        sg = torch.sigmoid(g)
        act = g * sg * u
        wgo = go[n].to(f) * w.reshape(-1)[j].to(torch.bfloat16).to(f)[:, None]
        gact = wgo @ wd[e].to(f)
        gg = gact * u * (sg * (1.0 + g * (1.0 - sg)))
        gu = gact * g * sg
        gup = torch.cat([gg, gu], dim=1)
        dwd[e] = wgo.t() @ act
        dwu[e] = gup.t() @ xs
    return dwu, dwd
