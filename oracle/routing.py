"""numpy restatement of the reference's routing index work (test oracle only).

Every function cites the reference file:line it restates.  Integer results
are exact; the float weights follow the reference's fp32 formulas.
"""

import numpy as np

WEIGHT_EPS = 1e-6  # fused_moe.py:29


def estimate_max_tokens(N, top_k, E):
    """Per-expert buffer rows when max_tokens_per_expert is None.

    fused_moe.py:100-113: m = ceil(N*k/E), then m += max(m, k); when
    N*k <= 4E the absolute bound N*k is used instead.
    """
    m = -(-N * top_k // E)
    m = m + max(m, top_k)
    if N * top_k <= 4 * E:
        m = N * top_k
    return m


def topk_select(scores, k):
    """Iterative-argmax top-k over fp32 scores, lowest index wins a tie.

    fused_topk.py:63-70: k rounds of ``tl.argmax`` (tie_break_left=True), the
    chosen lane masked out after each round.  That equals ordering the row by
    (value descending, index ascending) and keeping the first k, which is how
    it is computed here.  Returns (indices int64 [N,k], values fp32 [N,k]),
    slots in descending order.
    """
    s = np.asarray(scores, dtype=np.float32)
    N, E = s.shape
    # lexsort: the last key is primary.  Primary -value, secondary index.
    cols = np.broadcast_to(np.arange(E), s.shape)
    order = np.lexsort((cols, -s.astype(np.float64)), axis=1)
    idx = np.ascontiguousarray(order[:, :k]).astype(np.int64)
    vals = np.take_along_axis(s, idx, axis=1)
    return idx, vals


def softmax_selected(vals):
    """fused_topk.py:72-78: exp(v - max) / sum, in fp32 over the k picks."""
    v = np.asarray(vals, dtype=np.float32)
    m = v.max(axis=1, keepdims=True)
    e = np.exp(v - m, dtype=np.float32)
    return (e / e.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)


def sigmoid32(x):
    x = np.asarray(x, dtype=np.float32)
    return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x, dtype=np.float32))).astype(np.float32)


def route(logits, k, gating="softmax"):
    """Fast-path routing (fused_topk.py:139-179, kernels :30-136).

    softmax: select on fp32(logits), weights = softmax over the k picks.
    sigmoid: select on fp32 sigmoid(logits), weights = s / (sum s + 1e-6).
    Returns (weights fp32 [N,k], indices int64 [N,k]).
    """
    l32 = np.asarray(logits, dtype=np.float32)
    if gating == "softmax":
        idx, vals = topk_select(l32, k)
        return softmax_selected(vals), idx
    if gating == "sigmoid":
        sc = sigmoid32(l32)
        idx, vals = topk_select(sc, k)
        w = vals / (vals.sum(axis=1, keepdims=True, dtype=np.float32) + np.float32(WEIGHT_EPS))
        return w.astype(np.float32), idx
    raise ValueError(gating)


def stable_permutation(idx, E):
    """fused_moe.py:344-348: flat = idx.view(-1) (j = n*k + slot);
    sorted_order = argsort(flat, stable); counts = bincount; starts = [0, cumsum].
    Also returns rank[j] = position of j inside its expert's run.
    """
    flat = np.asarray(idx, dtype=np.int64).reshape(-1)
    sorted_order = np.argsort(flat, kind="stable").astype(np.int64)
    counts = np.bincount(flat, minlength=E).astype(np.int64)
    starts = np.zeros(E + 1, dtype=np.int64)
    starts[1:] = np.cumsum(counts)
    rank = np.empty_like(flat)
    rank[sorted_order] = np.arange(flat.size) - starts[flat[sorted_order]]
    return sorted_order, counts, starts, rank


def expand_to_batch(idx, E, max_tokens):
    """moe_ops.py:84-98, :138-140: e2b[j] = e*mt + rank when rank < mt,
    else e2b stays 0 (the overflow row aliases padded row 0)."""
    flat = np.asarray(idx, dtype=np.int64).reshape(-1)
    _, _, _, rank = stable_permutation(idx, E)
    kept = rank < max_tokens
    e2b = np.where(kept, flat * max_tokens + rank, 0).astype(np.int64)
    return e2b, kept


def expert_capacity(N, E, top_k, capacity_factor):
    """fused_moe.py:352-353: max(int(N/E*cf), k)."""
    return max(int((N / E) * capacity_factor), top_k)


def capacity_keep(idx, E, capacity):
    """fused_moe.py:355-367: keep (n, slot) iff its rank within its expert
    (in j = n*k + slot order) is below the capacity."""
    _, _, _, rank = stable_permutation(idx, E)
    return (rank < capacity).reshape(np.asarray(idx).shape)


def capacity_renormalize(weights, keep):
    """fused_moe.py:371-375: w*keep / (sum + (1 - has_any)), fp32."""
    w = np.asarray(weights, dtype=np.float32) * keep.astype(np.float32)
    s = w.sum(axis=1, keepdims=True, dtype=np.float32)
    has_any = (s > 0).astype(np.float32)
    return (w / (s + (np.float32(1.0) - has_any))).astype(np.float32)
