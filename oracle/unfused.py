"""torch-CPU restatement of the reference's unfused MoE test oracle.

Restates ``unfused_moe`` (tests/conftest.py:58-137): gate GEMM, torch.topk,
fp32 softmax/sigmoid weights, optional capacity drop with a ``+1e-6``
renormalisation, then a per-slot, per-expert masked loop accumulating
``w * down`` into the output in the input dtype.  Differentiable end to end
with torch.autograd, which is how the fused oracle's hand-written backward is
checked.  This is also the CPU baseline that bench.py times ("port").

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may use this.
"""

import torch
import torch.nn.functional as F

WEIGHT_EPS = 1e-6


def unfused_moe(hidden_states, gate_weight, w_up, w_down, top_k, activation="swiglu",
                gating="softmax", capacity_factor=None, aux_loss_coeff=0.0,
                z_loss_coeff=0.0):
    """Returns (output, topk_indices, topk_weights, losses) like conftest.py:58."""
    N, D = hidden_states.shape
    E = gate_weight.shape[0]
    H = w_up.shape[1] // 2
    losses = {}

    logits = hidden_states @ gate_weight.T                          # :69
    if gating == "softmax":                                         # :71-76
        vals, idx = torch.topk(logits, top_k, dim=-1)
        w = F.softmax(vals, dim=-1, dtype=torch.float32)
    elif gating == "sigmoid":                                       # :77-81
        sc = torch.sigmoid(logits.float())
        _, idx = torch.topk(sc, top_k, dim=-1)
        w = sc.gather(1, idx)
        w = w / (w.sum(dim=-1, keepdim=True) + WEIGHT_EPS)
    else:
        raise ValueError(gating)

    flat = idx.reshape(-1)
    tpe = torch.bincount(flat, minlength=E).float()
    if aux_loss_coeff > 0.0:                                        # :86-95
        f = tpe / N
        if gating == "softmax":
            P = torch.zeros(E, dtype=torch.float32).scatter_add(0, flat, w.reshape(-1).float()) / N
        else:
            P = torch.sigmoid(logits.float()).mean(dim=0)
        losses["aux_loss"] = aux_loss_coeff * E * (f * P).sum()
    if z_loss_coeff > 0.0:                                          # :97-98
        losses["z_loss"] = z_loss_coeff * torch.logsumexp(logits.float(), dim=-1).square().mean()

    if capacity_factor is not None:                                 # :100-113
        cap = max(int((N / E) * capacity_factor), top_k)
        order = torch.argsort(flat, stable=True)
        starts = torch.zeros(E + 1, dtype=torch.long)
        starts[1:] = torch.cumsum(tpe.long(), dim=0)
        rank = torch.zeros_like(flat)
        rank[order] = torch.arange(flat.numel()) - starts[flat[order]]
        keep = (rank < cap).view(N, top_k).float()
        w = w * keep
        w = w / (w.sum(dim=-1, keepdim=True) + WEIGHT_EPS)

    out = torch.zeros(N, D, dtype=hidden_states.dtype)               # :115
    for s in range(top_k):                                          # :116-135
        ids = idx[:, s]
        ws = w[:, s]
        for e in range(E):
            m = ids == e
            if not bool(m.any()):
                continue
            t = hidden_states[m]
            g = t @ w_up[e, :H, :].T
            u = t @ w_up[e, H:, :].T
            if activation == "swiglu":
                a = F.silu(g) * u
            elif activation == "geglu":
                a = F.gelu(g, approximate="tanh") * u
            elif activation == "relu_squared":
                a = F.relu(g).square() * u
            else:
                raise ValueError(activation)
            d = a @ w_down[e].T
            out = out.index_put((m.nonzero(as_tuple=True)[0],),
                                ws[m].unsqueeze(-1).to(d.dtype) * d, accumulate=True)
    return out, idx, w, losses


def shared_expert(x, w_gate, w_up, w_down, activation="swiglu"):
    """The reference's shared expert ``_GLUFFN.forward`` (nn.py:33-44):
    three bias-free linears; GeGLU here is the exact (erf) GELU."""
    g = x @ w_gate.T
    u = x @ w_up.T
    if activation == "swiglu":
        a = F.silu(g) * u
    elif activation == "geglu":
        a = F.gelu(g) * u
    elif activation == "relu_squared":
        a = F.relu(g).square() * u
    else:
        raise ValueError(activation)
    return a @ w_down.T
