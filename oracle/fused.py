"""torch-CPU restatement of the reference's fused (non-EP) MoE op -- test oracle.

Follows ``_FusedMoEAutograd`` (fused_moe.py:293-595) and the losses/metrics
block of ``fused_moe()`` (fused_moe.py:1159-1217) on the reference's padded
``[E*mt, D]`` batched layout, with the reference's rounding points:

* GEMMs take storage-dtype operands, accumulate in fp32 (fp64 for fp64
  storage) and round once to the storage dtype (cuBLAS bmm semantics);
* GLU forward/backward, gather-reduce, weighted scatter and the routing
  weight gradient compute in fp32 whatever the storage dtype, because the
  reference's Triton kernels cast every load ``.to(tl.float32)``
  (activations.py:237-238, :287-294; moe_ops.py:195-198, :283-286) and the
  weight gradient calls ``.float()`` (fused_moe.py:535);
* routing weights are fp32; the combine uses them rounded to the storage
  dtype (fused_moe.py:412); the routing backward uses the fp32 ones (:574).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may use this.
"""

import math

import numpy as np
import torch

from oracle import routing as R

ACTIVATIONS = ("swiglu", "geglu", "relu_squared")
GATINGS = ("softmax", "sigmoid")
_SQRT_2_OVER_PI = 0.7978845608028654


def acc_dtype(dtype):
    return torch.float64 if dtype == torch.float64 else torch.float32


def gemm(a, b):
    """a @ b with fp32 (fp64) accumulation, result rounded to a.dtype."""
    ad = acc_dtype(a.dtype)
    return torch.matmul(a.to(ad), b.to(ad)).to(a.dtype)


def _tanh_via_sigmoid(z):
    # activations.py:21-24: tanh(z) = 2*sigmoid(2z) - 1
    return 2.0 * torch.sigmoid(2.0 * z) - 1.0


def glu_forward(up, activation):
    """activations.py:27-74: act(gate)*up on the two halves, fp32 math."""
    H = up.shape[-1] // 2
    g = up[..., :H].float()
    u = up[..., H:].float()
    if activation == "swiglu":
        r = g * torch.sigmoid(g) * u
    elif activation == "geglu":
        inner = _SQRT_2_OVER_PI * (g + 0.044715 * g * g * g)
        r = 0.5 * g * (1.0 + _tanh_via_sigmoid(inner)) * u
    elif activation == "relu_squared":
        rg = torch.clamp(g, min=0.0)
        r = rg * rg * u
    else:
        raise ValueError(activation)
    return r.to(up.dtype)


def glu_backward(grad_act, up, activation):
    """activations.py:77-142: grad_gate -> [:H], grad_up -> [H:], fp32 math."""
    H = up.shape[-1] // 2
    ga = grad_act.float()
    g = up[..., :H].float()
    u = up[..., H:].float()
    if activation == "swiglu":
        sig = torch.sigmoid(g)
        gu = ga * (g * sig)
        gg = ga * u * (sig * (1.0 + g * (1.0 - sig)))
    elif activation == "geglu":
        inner = _SQRT_2_OVER_PI * (g + 0.044715 * g * g * g)
        th = _tanh_via_sigmoid(inner)
        gelu = 0.5 * g * (1.0 + th)
        gu = ga * gelu
        dinner = _SQRT_2_OVER_PI * (1.0 + 3.0 * 0.044715 * g * g)
        dgelu = 0.5 * (1.0 + th) + 0.5 * g * (1.0 - th * th) * dinner
        gg = ga * u * dgelu
    elif activation == "relu_squared":
        rg = torch.clamp(g, min=0.0)
        gu = ga * rg * rg
        gg = ga * u * 2.0 * rg
    else:
        raise ValueError(activation)
    return torch.cat([gg, gu], dim=-1).to(up.dtype)


def gather_reduce(batched, e2b, weights, N, k):
    """moe_ops.py:156-241: out[n] = sum_s w[n*k+s] * B[e2b[n*k+s]], fp32
    accumulation in slot order, rounded to the storage dtype."""
    rows = batched[e2b].float().view(N, k, -1)
    acc = torch.zeros(N, batched.shape[1], dtype=torch.float32)
    for s in range(k):
        v = rows[:, s, :]
        if weights is not None:
            v = v * weights.view(N, k)[:, s : s + 1].float()
        acc = acc + v
    return acc.to(batched.dtype)


def weighted_scatter(go, e2b, flat_w, rows, k, owner):
    """moe_ops.py:248-332: out[e2b[j]] = go[j//k] * w[j] (fp32 math), into a
    zeroed [rows, D] buffer.  ``owner[j]`` is False for overflow entries,
    whose e2b aliases padded row 0; the row's rightful entry wins here, where
    the reference's write order to that row is a race."""
    N, D = go.shape
    out = torch.zeros(rows, D, dtype=go.dtype)
    vals = (go.float().repeat_interleave(k, dim=0) * flat_w.float().view(-1, 1)).to(go.dtype)
    out[e2b[owner]] = vals[owner]
    return out


def apply_routing(logits, gating, top_k, expert_bias=None, pre_softmax=False,
                  scoring_factor=None, n_group=None, topk_group=None):
    """fused_moe.py:116-200 (fast path :139-142 -> fused_topk.py).

    Only the fast path is restated here; the advanced options (expert bias,
    pre-softmax, scoring factor, group-limited) are in ``route_advanced``.
    """
    advanced = (n_group is not None or expert_bias is not None or pre_softmax
                or scoring_factor is not None)
    if advanced:
        return route_advanced(logits, gating, top_k, expert_bias, pre_softmax,
                              scoring_factor, n_group, topk_group)
    w, idx = R.route(logits.float().numpy(), top_k, gating)
    return torch.from_numpy(w), torch.from_numpy(idx)


def _topk_stable(scores, k):
    """top-k of a float tensor, ties to the lowest index (see DESIGN notes:
    the reference's torch.topk tie order is implementation-defined)."""
    idx, _ = R.topk_select(scores.detach().float().numpy(), k)
    idx = torch.from_numpy(idx)
    return scores.gather(1, idx), idx


def route_advanced(logits, gating, top_k, expert_bias, pre_softmax, scoring_factor,
                   n_group, topk_group):
    """fused_moe.py:144-200 and _group_limited_topk :203-251.

    Selection runs on biased scores, weights use unbiased ones.  Arithmetic
    follows the reference's dtype promotion: ``logits + expert_bias`` is done
    in the promoted dtype of the two tensors.
    """
    def group_limited(sel, wsrc):
        N, E = sel.shape
        epg = E // n_group
        grouped = sel.view(N, n_group, epg)
        per = top_k // topk_group
        if 1 < per <= epg:
            gs = _topk_stable(grouped.reshape(N * n_group, epg), per)[0].sum(-1).view(N, n_group)
        else:
            gs = grouped.max(dim=-1).values
        _, gidx = _topk_stable(gs, topk_group)
        gmask = torch.zeros(N, n_group, dtype=torch.bool)
        gmask.scatter_(1, gidx, True)
        emask = gmask.unsqueeze(-1).expand(-1, -1, epg).reshape(N, E)
        masked = sel.clone()
        masked[~emask] = float("-inf")
        _, idx = _topk_stable(masked, top_k)
        return wsrc.gather(1, idx), idx

    if gating == "softmax":
        if pre_softmax:
            probs = torch.softmax(logits.float(), dim=-1)
            sel = probs + expert_bias.float().unsqueeze(0) if expert_bias is not None else probs
            if n_group is not None and topk_group is not None:
                w, idx = group_limited(sel, probs)
            else:
                _, idx = _topk_stable(sel, top_k)
                w = probs.gather(1, idx)
            w = w / (w.sum(-1, keepdim=True) + R.WEIGHT_EPS)
        else:
            sel = logits + expert_bias.unsqueeze(0) if expert_bias is not None else logits
            if n_group is not None and topk_group is not None:
                w, idx = group_limited(sel, logits)
                w = torch.softmax(w.float(), dim=-1)
            else:
                _, idx = _topk_stable(sel, top_k)
                w = torch.softmax(logits.gather(1, idx).float(), dim=-1)
    elif gating == "sigmoid":
        sc = torch.sigmoid(logits.float())
        sel = sc + expert_bias.float().unsqueeze(0) if expert_bias is not None else sc
        if n_group is not None and topk_group is not None:
            w, idx = group_limited(sel, sc)
        else:
            _, idx = _topk_stable(sel, top_k)
            w = sc.gather(1, idx)
        w = w / (w.sum(-1, keepdim=True) + R.WEIGHT_EPS)
    else:
        raise ValueError(gating)
    if scoring_factor is not None:
        w = w * (scoring_factor / top_k)
    return w.float(), idx


def forward(x, gate, w_up, w_down, top_k, activation="swiglu", gating="softmax",
            capacity_factor=None, max_tokens_per_expert=None, allow_dropped_tokens=False,
            logits=None, **routing_cfg):
    """_FusedMoEAutograd.forward (fused_moe.py:308-478) on CPU.

    All tensors are in one storage dtype (the reference's compute dtype).
    ``logits`` may be given to pin routing to externally computed logits.
    Returns (output [N,D], state dict for ``backward``).
    """
    N, D = x.shape
    E = gate.shape[0]
    dtype = x.dtype
    if logits is None:
        logits = gemm(x, gate.t())                                  # :334
    w, idx = apply_routing(logits, gating, top_k, **routing_cfg)  # :336-341
    flat = idx.reshape(-1)
    sorted_order, counts, starts, rank = R.stable_permutation(idx.numpy(), E)  # :344-348

    if capacity_factor is not None:                                # :351-390
        cap = R.expert_capacity(N, E, top_k, capacity_factor)
        keep = torch.from_numpy(rank < cap)
        w = torch.from_numpy(R.capacity_renormalize(w.numpy(), keep.view(N, top_k).numpy()))
        mt = cap
        keep_f = keep.to(dtype)
    else:
        keep_f = None
        mt = max_tokens_per_expert if max_tokens_per_expert is not None else \
            R.estimate_max_tokens(N, top_k, E)
        if not allow_dropped_tokens and counts.max() > mt:         # :400-410
            raise RuntimeError(f"MoE routing overflow: expert received {counts.max()} tokens "
                               f"but buffer is {mt}.")
        keep = torch.from_numpy(rank < mt)

    flat_w = w.to(dtype).reshape(-1)                               # :412
    rank_t = torch.from_numpy(rank)
    e2b = torch.where(keep, flat * mt + rank_t, torch.zeros_like(flat))  # moe_ops.py:84-98,:138-140
    if capacity_factor is not None:
        e2b = torch.where(keep, e2b, torch.full_like(e2b, E * mt))  # :428-430 sentinel
    rows = E * mt + (1 if capacity_factor is not None else 0)

    hb = torch.zeros(rows, D, dtype=dtype)                         # moe_ops.py:137
    hb[e2b[keep]] = x.repeat_interleave(top_k, dim=0)[keep]
    hbv = hb[: E * mt].view(E, mt, D)
    up = gemm(hbv, w_up.transpose(1, 2))                           # :435
    act = glu_forward(up, activation)                              # :438
    down = gemm(act, w_down.transpose(1, 2))                       # :441
    down_flat = down.reshape(E * mt, D)
    if capacity_factor is not None:
        down_flat = torch.cat([down_flat, torch.zeros(1, D, dtype=dtype)])  # :447-450
    out = gather_reduce(down_flat, e2b, flat_w, N, top_k)           # :451-453

    st = dict(x=x, gate=gate, w_up=w_up, w_down=w_down, logits=logits, topk_w=w,
              topk_idx=idx, flat_w=flat_w, e2b=e2b, keep=keep, keep_f=keep_f, mt=mt,
              hb=hb, up=up, act=act, down=down, counts=torch.from_numpy(counts),
              sorted_order=torch.from_numpy(sorted_order), rank=rank_t,
              top_k=top_k, activation=activation, gating=gating,
              has_capacity=capacity_factor is not None)
    return out, st


def backward(st, grad_out):
    """_FusedMoEAutograd.backward (fused_moe.py:482-595) on CPU.

    Returns dict(hidden, gate, w_up, w_down, grad_topk_w, grad_logits).
    """
    x, gate, w_up, w_down = st["x"], st["gate"], st["w_up"], st["w_down"]
    k, mt = st["top_k"], st["mt"]
    E = gate.shape[0]
    N, D = grad_out.shape
    dtype = x.dtype
    go = grad_out.to(dtype)
    e2b, keep, flat_w = st["e2b"], st["keep"], st["flat_w"]
    pad = st["has_capacity"]

    down_flat = st["down"].reshape(E * mt, D)
    if pad:
        down_flat = torch.cat([down_flat, torch.zeros(1, D, dtype=dtype)])
    gathered = down_flat[e2b]                                       # :533
    g_w = (gathered.float() * go.float().repeat_interleave(k, dim=0)).sum(-1).view(N, k)  # :534-535

    # capacity-dropped entries point at the zero sentinel row: letting them
    # write there is harmless, since the reference slices it off (:544)
    owner = keep | pad
    wgo = weighted_scatter(go, e2b, flat_w, E * mt + (1 if pad else 0), k, owner)  # :539-544
    wgo = wgo[: E * mt].view(E, mt, D)
    gact = gemm(wgo, w_down)                                        # :547
    gup = glu_backward(gact, st["up"], st["activation"])           # :550
    ghb = gemm(gup, w_up)                                           # :553
    ghb_flat = ghb.reshape(E * mt, D)
    if pad:
        ghb_flat = torch.cat([ghb_flat, torch.zeros(1, D, dtype=dtype)])
    gh = gather_reduce(ghb_flat, e2b, st["keep_f"], N, k)           # :556-561
    gwd = gemm(wgo.transpose(1, 2), st["act"])                      # :564
    gwu = gemm(gup.transpose(1, 2), st["hb"][: E * mt].view(E, mt, D))  # :565

    w = st["topk_w"]
    if pad:                                                         # :569-571
        g_w = g_w * (w.sum(-1, keepdim=True) > 0).float()
    if st["gating"] == "softmax":                                   # :573-576
        sg = (g_w * w).sum(-1, keepdim=True)
        gtl = w * (g_w - sg)
    else:                                                           # :577-584
        sc = torch.sigmoid(st["logits"].float())
        ts = sc.gather(1, st["topk_idx"])
        gdw = (g_w * w).sum(-1, keepdim=True)
        gts = (g_w - gdw) / (ts.sum(-1, keepdim=True) + R.WEIGHT_EPS)
        gtl = gts * ts * (1.0 - ts)
    gl32 = torch.zeros(N, E, dtype=torch.float32)
    gl32.scatter_add_(1, st["topk_idx"], gtl.float())               # :587-588
    gl = gl32.to(dtype)
    gh = (gh.to(acc_dtype(dtype)) + gemm(gl, gate).to(acc_dtype(dtype))).to(dtype)  # :590
    ggate = gemm(gl.t(), x)                                         # :591
    return dict(hidden=gh, gate=ggate, w_up=gwu, w_down=gwd, grad_topk_w=g_w,
                grad_logits=gl32, wgo=wgo, gup=gup, ghb=ghb, gact=gact)


def losses(logits, topk_w, topk_idx, E, gating="softmax", aux_loss_coeff=0.0,
           z_loss_coeff=0.0, return_metrics=False, capacity_factor=None, top_k=None):
    """fused_moe.py:1159-1217 (values only; gradients are in ``loss_grads``)."""
    out = {}
    N = logits.shape[0]
    flat = topk_idx.reshape(-1)
    tpe = torch.bincount(flat, minlength=E).float()
    if aux_loss_coeff > 0.0:
        f = tpe / N
        if gating == "softmax":
            P = torch.zeros(E, dtype=torch.float32)
            P.scatter_add_(0, flat, topk_w.reshape(-1).float())
            P = P / N
        else:
            P = torch.sigmoid(logits.float()).mean(dim=0)
        out["aux_loss"] = aux_loss_coeff * E * (f * P).sum()
    if z_loss_coeff > 0.0:
        out["z_loss"] = z_loss_coeff * torch.logsumexp(logits.float(), dim=-1).square().mean()
    if return_metrics:
        out["tokens_per_expert"] = tpe.int()
        out["max_expert_load"] = tpe.max().int()
        out["min_expert_load"] = tpe.min().int()
        out["expert_load_imbalance"] = tpe.max().float() / (tpe.float().mean() + R.WEIGHT_EPS)
        if capacity_factor is not None:
            cap = R.expert_capacity(N, E, top_k, capacity_factor)
            _, _, _, rank = R.stable_permutation(topk_idx.numpy(), E)
            dropped = int((rank >= cap).sum())
            out["dropped_token_count"] = torch.tensor(dropped)
            out["dropped_token_fraction"] = torch.tensor(dropped, dtype=torch.float32) / (N * top_k)
    return out


def loss_grads(logits, topk_idx, E, gating, aux_loss_coeff, z_loss_coeff, g_aux=1.0, g_z=1.0):
    """d(aux, z)/d logits in fp32, as autograd produces them on the GPU fast
    path: softmax aux has no gradient (the fused top-k outputs are not
    differentiable), sigmoid aux flows through P = mean(sigmoid(logits)),
    z-loss flows through logsumexp (fused_moe.py:1178-1194)."""
    N = logits.shape[0]
    l32 = logits.float()
    g = torch.zeros(N, E, dtype=torch.float32)
    if z_loss_coeff > 0.0:
        lse = torch.logsumexp(l32, dim=-1, keepdim=True)
        g = g + g_z * z_loss_coeff * (2.0 * lse / N) * torch.softmax(l32, dim=-1)
    if aux_loss_coeff > 0.0 and gating == "sigmoid":
        f = torch.bincount(topk_idx.reshape(-1), minlength=E).float() / N
        s = torch.sigmoid(l32)
        g = g + g_aux * aux_loss_coeff * E * f.unsqueeze(0) * s * (1.0 - s) / N
    return g
