"""The reference's kernel-level Python boundary, over libffmoe.so.

Same names, arguments and results as the reference's wrappers in
src/flashfusemoe/kernels/ (fused_topk.py:139-179, moe_ops.py:109-332,
activations.py:145-231), for callers that use the kernels directly.  They
work on the reference's padded [E*max_tokens, D] layout; ``fused_moe`` itself
uses the compact layout and does not go through these.  Tensors may be
bfloat16, float32 or float64, as the reference's Triton kernels accept any
of them (they compute in fp32 and store the input dtype).
"""

import torch

from . import _lib as L
from .ops import T_DTYPES

_BF16 = torch.bfloat16


def _gpu(name, t):
    if t.device.type != "cuda" or (t.dtype != _BF16 and t.dtype not in T_DTYPES):
        raise TypeError(f"{name} must be a bfloat16, float32 or float64 tensor on a ROCm GPU "
                        f"(got {t.dtype} on {t.device})")
    return t.contiguous()


def fused_topk_routing(logits, gating, top_k):
    """Top-k routing of bf16 logits [N, E] -> (weights fp32 [N,k], indices
    int64 [N,k]); lowest index wins ties, slots in descending order
    (fused_topk.py:139-179)."""
    logits = _gpu("logits", logits)
    N, E = logits.shape
    if gating not in L.GATING:
        raise ValueError(f"Unknown gating: {gating}")
    dev = logits.device
    ws = torch.empty(L.route_workspace_bytes(N, E, top_k), dtype=torch.uint8, device=dev)
    idx = torch.empty(N, top_k, dtype=torch.int64, device=dev)
    w = torch.empty(N, top_k, dtype=torch.float32, device=dev)
    if logits.dtype == _BF16:
        L.call("ffmoe_route_fwd", None, None, L.ptr(logits), None, N, 8, E, top_k, L.GATING[gating], 0,
               None, L.ptr(idx), L.ptr(w), None, L.ptr(ws), L.stream_ptr(dev))
    else:  # the reference's kernel loads logits .to(tl.float32) (fused_topk.py:52)
        lf = logits.float().contiguous()
        L.call("ffmoe_route_logits_f32", L.ptr(lf), None, 0, 0.0, 0, 0, N, E, top_k, L.GATING[gating], 0,
               L.ptr(idx), L.ptr(w), None, L.ptr(ws), L.stream_ptr(dev))
    return w, idx


def fused_routing_scatter(sorted_order, flat_expert_ids, expert_starts, hidden_states, E,
                          max_tokens, top_k, num_sorted=None):
    """Padded scatter (moe_ops.py:109-149): for sorted position p,
    j = sorted_order[p], e = flat_expert_ids[j], rank = p - expert_starts[e];
    if rank < max_tokens: expand_to_batch[j] = e*max_tokens + rank and
    out[e*max_tokens + rank] = hidden_states[j // top_k].  Returns
    (out [E*max_tokens, D] zero-initialised, expand_to_batch int64 [N*k])."""
    x = _gpu("hidden_states", hidden_states)
    N, D = x.shape
    dev = x.device
    ns = N * top_k if num_sorted is None else int(num_sorted)
    so = sorted_order.to(device=dev, dtype=torch.int64).contiguous()
    fl = flat_expert_ids.to(device=dev, dtype=torch.int64).contiguous()
    st = expert_starts.to(device=dev, dtype=torch.int64).contiguous()
    if so.numel() < ns or fl.numel() != N * top_k or st.numel() < E + 1:
        raise ValueError("fused_routing_scatter: sorted_order, flat_expert_ids or expert_starts "
                         "is shorter than the problem")
    out = torch.zeros(E * max_tokens, D, dtype=x.dtype, device=dev)
    e2b = torch.zeros(N * top_k, dtype=torch.int64, device=dev)
    if x.dtype == _BF16:
        L.call("ffmoe_routing_scatter_padded", L.ptr(so), L.ptr(fl), L.ptr(st), L.ptr(x), N, D, E,
               max_tokens, top_k, ns, L.ptr(out), L.ptr(e2b), L.stream_ptr(dev))
    else:
        L.call("ffmoe_t_routing_scatter_padded", T_DTYPES[x.dtype], L.ptr(so), L.ptr(fl), L.ptr(st), L.ptr(x),
               N, D, E, max_tokens, top_k, ns, L.ptr(out), L.ptr(e2b), L.stream_ptr(dev))
    return out, e2b


def fused_gather_reduce(batched, expand_to_batch, weights, N, top_k):
    """out[n] = sum_s w[n*k+s] * batched[expand_to_batch[n*k+s]] (fp32 in slot
    order, moe_ops.py:206-241); weights None -> unweighted."""
    b = _gpu("batched", batched)
    D = b.shape[1]
    dev = b.device
    rows = expand_to_batch.to(torch.int32).contiguous()
    w = None if weights is None else weights.reshape(-1).float().contiguous()
    out = torch.empty(N, D, dtype=b.dtype, device=dev)
    if b.dtype == _BF16:
        L.call("ffmoe_combine", L.ptr(b), L.ptr(rows), L.ptr(w), None, N, D, top_k, L.ptr(out),
               L.stream_ptr(dev))
    else:
        L.call("ffmoe_t_combine", T_DTYPES[b.dtype], L.ptr(b), L.ptr(rows), L.ptr(w), None, N, D, top_k,
               L.ptr(out), L.stream_ptr(dev))
    return out


def fused_weighted_scatter(grad_output, expand_to_batch, topk_weights, E, max_tokens, top_k,
                           output_rows=None):
    """out[expand_to_batch[j]] = grad_output[j // k] * w[j] into a zeroed
    [output_rows or E*max_tokens, D] buffer (moe_ops.py:291-332)."""
    go = _gpu("grad_output", grad_output)
    N, D = go.shape
    dev = go.device
    rows = output_rows if output_rows is not None else E * max_tokens
    out = torch.zeros(rows, D, dtype=go.dtype, device=dev)
    w = topk_weights.reshape(-1).float().contiguous()
    dst = expand_to_batch.to(torch.int64).contiguous()
    if go.dtype == _BF16:
        L.call("ffmoe_scatter_rows", L.ptr(go), L.ptr(dst), L.ptr(w), N * top_k, top_k, D, rows,
               L.ptr(out), L.stream_ptr(dev))
    else:
        L.call("ffmoe_t_scatter_rows", T_DTYPES[go.dtype], L.ptr(go), L.ptr(dst), L.ptr(w), N * top_k, top_k, D,
               rows, L.ptr(out), L.stream_ptr(dev))
    return out


def activation_forward(up, activation):
    """GLU forward on [..., 2H] -> [..., H] (activations.py:145-186)."""
    u = _gpu("up", up)
    H = u.shape[-1] // 2
    M = u.numel() // (2 * H)
    out = torch.empty(*u.shape[:-1], H, dtype=u.dtype, device=u.device)
    if u.dtype == _BF16:
        L.call("ffmoe_glu_fwd", L.ptr(u), M, H, L.ACTIVATION[activation], L.ptr(out),
               L.stream_ptr(u.device))
    else:  # fp32 math, the input dtype stored (activations.py:58-74)
        L.call("ffmoe_t_glu_fwd", T_DTYPES[u.dtype], L.ptr(u), M, H, L.ACTIVATION[activation], 0, L.ptr(out),
               L.stream_ptr(u.device))
    return out


def activation_backward(grad_act, up, activation):
    """GLU backward: (grad [..., H], up [..., 2H]) -> grad_up [..., 2H]
    (activations.py:189-231)."""
    u = _gpu("up", up)
    g = _gpu("grad_act", grad_act)
    if g.dtype != u.dtype:
        raise TypeError(f"grad_act ({g.dtype}) and up ({u.dtype}) must have one dtype")
    H = u.shape[-1] // 2
    M = u.numel() // (2 * H)
    out = torch.empty_like(u)
    if u.dtype == _BF16:
        L.call("ffmoe_glu_bwd", L.ptr(g), L.ptr(u), M, H, L.ACTIVATION[activation], L.ptr(out),
               L.stream_ptr(u.device))
    else:
        L.call("ffmoe_t_glu_bwd", T_DTYPES[u.dtype], L.ptr(g), L.ptr(u), M, H, L.ACTIVATION[activation], 0,
               L.ptr(out), L.stream_ptr(u.device))
    return out
