"""fused_moe(): gate -> top-k route -> GLU experts -> weighted combine, on MI355X.

Drop-in for the reference's non-expert-parallel ``fused_moe``
(src/flashfusemoe/fused_moe.py:1073-1246): same signature and defaults, same
validation messages, same losses dict, same overflow error.  Every step runs
as a hand-written HIP kernel behind libffmoe.so (see ops.py).  The compute
dtype is the reference's: the autocast dtype if autocast is on, else the
input dtype.  bfloat16 runs on the MFMA pipeline; float32 and float64 run
on this library's fp32 / fp64 kernels with the reference's fp32 internals
(routing on logits.float(), GLU and gather sums in fp32); float16 is not
supported and raises.

Layout differences that are invisible through this API: expert rows are
stored compactly (no [E, max_tokens] padding rows are allocated or computed),
and the routing statistics of the losses block come from the same routing
kernel as the forward instead of a second gate GEMM.
"""

import torch

from . import _lib as L
from . import ops

_WEIGHT_EPS = 1e-6  # the reference's weight-normalisation guard


def _estimate_max_tokens(N, top_k, E):
    """Static rows-per-expert bound when max_tokens_per_expert is None
    (fused_moe.py:100-113): ceil(N*k/E) plus a 100% margin (at least k); the
    absolute bound N*k when N*k <= 4E."""
    max_tokens = (N * top_k + E - 1) // E
    max_tokens = max_tokens + max(max_tokens, top_k)
    if N * top_k <= 4 * E:
        max_tokens = N * top_k
    return max_tokens


def _validate_inputs(hidden_states, gate_weight, w_up, w_down, top_k, activation, gating):
    """Shape/device/enum checks with the reference's messages
    (fused_moe.py:254-276, non-EP branch)."""
    assert hidden_states.dim() == 2, f"hidden_states must be 2D [N, D], got {hidden_states.shape}"
    N, D = hidden_states.shape
    E = gate_weight.shape[0]
    E_w = w_up.shape[0]
    ffn_dim = w_up.shape[1]
    assert gate_weight.shape == (E, D), f"gate_weight must be [{E}, {D}], got {gate_weight.shape}"
    assert w_up.shape == (E_w, ffn_dim, D), \
        f"w_up must be [{E_w}, {ffn_dim}, {D}], got {w_up.shape}"
    assert w_down.shape == (E_w, D, ffn_dim // 2), \
        f"w_down must be [{E_w}, {D}, {ffn_dim // 2}], got {w_down.shape}"
    assert E_w == E, f"w_up must have {E} experts, got {E_w}"
    assert ffn_dim % 2 == 0, f"ffn_dim must be even, got {ffn_dim}"
    assert 1 <= top_k <= E, f"top_k must be in [1, {E}], got {top_k}"
    dev = hidden_states.device
    assert all(t.device == dev for t in [gate_weight, w_up, w_down]), \
        "All tensors must be on same device"
    assert activation in ("swiglu", "geglu", "relu_squared"), f"Unknown activation: {activation}"
    assert gating in ("softmax", "sigmoid"), f"Unknown gating: {gating}"


def _check_kernel_limits(N, D, E, H, top_k):
    if E > L.MAX_EXPERTS:
        raise NotImplementedError(f"ffmoe kernels support up to {L.MAX_EXPERTS} experts, got {E}")
    if top_k > L.MAX_TOPK:
        raise NotImplementedError(f"ffmoe kernels support top_k up to {L.MAX_TOPK}, got {top_k}")
    if D % 8 != 0 or H % 8 != 0:
        raise NotImplementedError(
            f"ffmoe kernels need d_model and ffn_dim/2 to be multiples of 8 (got D={D}, H={H})")


def _compute_dtype(fallback):
    """Autocast dtype if autocast is on, else the input dtype
    (fused_moe.py:93-97)."""
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return fallback


SUPPORTED_DTYPES = (torch.bfloat16, torch.float32, torch.float64)


def _check_compute_dtype(dtype):
    if dtype not in SUPPORTED_DTYPES:
        raise TypeError(
            f"ffmoe computes in bfloat16, float32 or float64; got compute dtype {dtype} (pass "
            "tensors of one of those or run under torch.autocast('cuda', dtype=torch.bfloat16))")


def _overflow_message(actual_max, max_tokens):
    # fused_moe.py:403-410 (same text, so callers matching on it keep working)
    return (
        f"MoE routing overflow: expert received {actual_max} tokens but buffer "
        f"is {max_tokens}. {actual_max - max_tokens} tokens would be silently "
        f"dropped. Fix options:\n"
        f"  1. Set max_tokens_per_expert={actual_max} (or higher) via calibration\n"
        f"  2. Set capacity_factor to enable intentional token dropping\n"
        f"  3. Set allow_dropped_tokens=True to suppress this error"
    )


class _FusedMoEFunction(torch.autograd.Function):
    """Forward: route -> permute -> up GEMM + GLU -> down GEMM -> combine.
    Backward: routing backward (weight grads, weighted scatter, top-k
    softmax/sigmoid backward, z-loss / sigmoid-aux gradients) -> dgrad GEMM +
    GLU backward -> dgrad GEMM -> dX reduce -> wgrad GEMMs.

    Outputs: (output [N,D], aux_loss fp32 scalar, z_loss fp32 scalar,
    routing tensors for the losses dict).  Mirrors _FusedMoEAutograd
    (fused_moe.py:293-595) together with the autograd of the losses block
    (fused_moe.py:1159-1194).
    """

    @staticmethod
    def forward(ctx, x, gate, w_up, w_down, expert_bias, s_gate, s_up, s_down, cfg, rcfg, s_act):
        (top_k, activation, gating, capacity_factor, recompute, mt_user, allow_dropped,
         aux_coeff, z_coeff) = cfg
        pre_softmax, scoring, n_group, topk_group, jitter, advanced = rcfg
        N, D = x.shape
        E = gate.shape[0]
        dtype = _compute_dtype(x.dtype)
        _check_compute_dtype(dtype)
        xc = x.to(dtype).contiguous()
        gc = gate.to(dtype).contiguous()
        wu = w_up.to(dtype).contiguous()
        wd = w_down.to(dtype).contiguous()

        capacity_mode = capacity_factor is not None
        if capacity_mode:
            mt = max(int((N / E) * capacity_factor), top_k)       # fused_moe.py:352-353
        elif mt_user is not None:
            mt = int(mt_user)
        else:
            mt = _estimate_max_tokens(N, top_k, E)
        gate_id = L.GATING[gating]
        act_id = L.ACTIVATION[activation]
        need_ssum = gating == "sigmoid" and aux_coeff > 0.0
        # a bf16 bias is added to the bf16 logits in bf16 (fused_moe.py:176)
        bias_round = (dtype == torch.bfloat16 and expert_bias is not None and expert_bias.dtype == torch.bfloat16
                      and gating == "softmax" and not pre_softmax)
        ropts = (bool(bias_round), bool(pre_softmax), float(scoring or 0.0), int(n_group or 0),
                 int(topk_group or 0))

        # routing of the losses block (and of dispatch, without jitter)
        (logits, topk_idx, topk_w, lse, counts, offsets, tile_offsets, stats, istats, ws, aux,
         z) = ops.route(xc, gc, expert_bias, top_k, gate_id, mt, float(aux_coeff),
                        float(z_coeff), need_ssum, *ropts)
        aux_idx = aux_counts = None
        istats_d = istats
        if jitter > 0.0:
            # dispatch routes bf16(x * noise) (fused_moe.py:329-332); the losses
            # block, the metrics and the sigmoid / z / aux gradients keep the
            # un-jittered logits (fused_moe.py:1165, :577-579)
            noise = torch.empty_like(xc).uniform_(1.0 - jitter, 1.0 + jitter)
            aux_idx, aux_counts = topk_idx, counts
            (_, topk_idx, topk_w, _, counts, offsets, tile_offsets, _, istats_d, ws, _,
             _) = ops.route(xc, gc, expert_bias, top_k, gate_id, mt, 0.0, 0.0, False, *ropts,
                            noise)

        if not capacity_mode and not allow_dropped:
            actual_max = int(istats_d[L.ISTAT_MAX].item())          # fused_moe.py:400-410
            # the stream is idle here anyway: surface a failed stream-K wait
            # of an earlier call's GEMMs before anything else runs
            L.check_gemm_workspaces()
            if actual_max > mt:
                raise RuntimeError(_overflow_message(actual_max, mt))

        # MoELayer's shared expert (s_gate/s_up/s_down, nn.py:22-44) runs as a
        # dense row group of the routed GEMM launches; its output is added by
        # the combine (nn.py:156-159)
        has_sh = s_gate is not None
        w_gu = w_sd = None
        if has_sh:
            w_gu = torch.cat([s_gate.to(dtype), s_up.to(dtype)], 0).contiguous()
            w_sd = s_down.to(dtype).contiguous()
        (out, tw, row_of, xs, up, act, down, up_sh, act_sh) = ops.experts_forward(
            xc, wu, wd, topk_idx, topk_w, counts, offsets, tile_offsets, ws, top_k, act_id, mt,
            capacity_mode, not recompute, shared_w_gu=w_gu, shared_w_down=w_sd,
            shared_act=int(s_act or 0))
        if not capacity_mode:
            tw = topk_w

        ctx.cfg = (top_k, act_id, gate_id, capacity_mode, float(aux_coeff), float(z_coeff))
        ctx.rcfg = (bool(advanced and gating == "softmax"), bool(pre_softmax),
                    float(scoring or 0.0))
        ctx.in_dtypes = (x.dtype, gate.dtype, w_up.dtype, w_down.dtype)
        ctx.has_sh = has_sh
        ctx.s_act = int(s_act or 0)
        ctx.sh_dtypes = (s_gate.dtype, s_up.dtype, s_down.dtype) if has_sh else None
        ctx.save_for_backward(xc, gc, wu, wd, logits, topk_idx, tw, lse, counts, offsets,
                              tile_offsets, row_of, xs, up, act, down, aux_idx, aux_counts,
                              w_gu, w_sd, up_sh, act_sh)
        ctx.set_materialize_grads(False)  # unused outputs get no zero-filled gradients
        # the softmax aux loss has a gradient only on the reference's slow
        # routing path, whose weights are differentiable torch ops
        # (fused_topk_routing outputs are not): fused_moe.py:136-142, :1165-1189
        ctx.aux_has_grad = gating == "sigmoid" or bool(advanced)
        # metrics come from the losses block's (un-jittered) routing
        m_counts = aux_counts if aux_counts is not None else counts
        non_diff = [m_counts, stats, istats]
        if not ctx.aux_has_grad:
            non_diff.append(aux)
        ctx.mark_non_differentiable(*non_diff)
        return out, aux, z, m_counts, stats, istats

    @staticmethod
    def backward(ctx, grad_out, g_aux, g_z, _gc, _gs, _gis):
        (xc, gc, wu, wd, logits, topk_idx, tw, lse, counts, offsets, tile_offsets, row_of, xs,
         up, act, down, aux_idx, aux_counts, w_gu, w_sd, up_sh, act_sh) = ctx.saved_tensors
        top_k, act_id, gate_id, capacity_mode, aux_coeff, z_coeff = ctx.cfg
        aux_through, pre_softmax, scoring = ctx.rcfg
        if grad_out is None:
            grad_out = torch.zeros_like(xc)
        go = grad_out.to(xc.dtype).contiguous()
        ga = g_aux if (ctx.aux_has_grad and aux_coeff > 0.0) else None
        gz = g_z if z_coeff > 0.0 else None
        # the sigmoid aux gradient's expert fractions come from the losses
        # block's routing (the un-jittered one under input jitter)
        dx, dgate, dwu, dwd, dw_gu, dw_sd = ops.experts_backward(
            go, xc, gc, wu, wd, logits, topk_idx, tw, lse,
            counts if aux_counts is None else aux_counts, offsets, tile_offsets, row_of, xs, up,
            act, down, ga, gz, top_k, act_id, gate_id, capacity_mode, aux_coeff, z_coeff,
            aux_through, aux_idx, aux_counts, pre_softmax, scoring,
            shared_w_gu=w_gu if ctx.has_sh else None, shared_w_down=w_sd if ctx.has_sh else None,
            up_sh=up_sh if ctx.has_sh else None, act_sh=act_sh if ctx.has_sh else None,
            shared_act=ctx.s_act)
        xd, gd, ud, dd = ctx.in_dtypes
        gs = (None, None, None)
        if ctx.has_sh:
            H = w_sd.shape[1]
            sg, su, sd = ctx.sh_dtypes
            gs = (dw_gu[:H].to(sg), dw_gu[H:].to(su), dw_sd.to(sd))
        return (dx.to(xd), dgate.to(gd), dwu.to(ud), dwd.to(dd), None, *gs, None, None, None)


def set_ep_group(group, backend="nccl"):
    """Expert parallelism is outside this build: only ``None`` is accepted
    (the reference's set_ep_group, fused_moe.py:1025-1040)."""
    if group is not None:
        raise NotImplementedError("expert parallelism is not part of this single-GPU build")


def fused_moe(
    hidden_states,
    gate_weight,
    w_up,
    w_down,
    top_k=2,
    activation="swiglu",
    gating="softmax",
    capacity_factor=None,
    aux_loss_coeff=0.0,
    z_loss_coeff=0.0,
    recompute_activations=False,
    ep_group=None,
    max_tokens_per_expert=None,
    allow_dropped_tokens=False,
    return_metrics=False,
    shared_expert_weights=None,
    latent_weights=None,
    n_group=None,
    topk_group=None,
    scoring_factor=None,
    pre_softmax=False,
    input_jitter=0.0,
    expert_bias=None,
    _shared=None,
):
    """Fused MoE layer forward (differentiable).

    Args and returns follow the reference (fused_moe.py:1073-1140):
      hidden_states [N, D]; gate_weight [E, D]; w_up [E, ffn_dim, D] (rows
      [0, ffn_dim/2) gate half, the rest up half); w_down [E, D, ffn_dim/2].
      Returns (output [N, D], losses) where losses may hold "aux_loss",
      "z_loss" and, with return_metrics, "tokens_per_expert",
      "max_expert_load", "min_expert_load", "expert_load_imbalance" and (with
      capacity_factor) "dropped_token_count", "dropped_token_fraction".

    shared_expert_weights / latent_weights only matter to the reference's
    expert-parallel path and are ignored here, as the reference's
    single-GPU path ignores them.  ``_shared`` (internal, used by MoELayer)
    is (w_gate [H,D], w_up [H,D], w_down [D,H], activation id): the shared
    expert then runs inside the same GEMM launches and the returned output
    is bf16(routed + shared).
    """
    if ep_group is not None:
        raise NotImplementedError("expert parallelism is not part of this single-GPU build")
    _validate_inputs(hidden_states, gate_weight, w_up, w_down, top_k, activation, gating)

    N, D = hidden_states.shape
    E = gate_weight.shape[0]
    H = w_up.shape[1] // 2
    _check_kernel_limits(N, D, E, H, top_k)
    # the reference's slow routing path (fused_moe.py:136-138)
    advanced = (n_group is not None or expert_bias is not None or pre_softmax
                or scoring_factor is not None)
    groups = n_group is not None and topk_group is not None          # fused_moe.py:158, :175
    if groups:
        assert E % n_group == 0, f"E ({E}) must be divisible by n_group ({n_group})"  # fused_moe.py:221
        if not 1 <= topk_group <= min(n_group, L.MAX_TOPK):
            raise NotImplementedError(f"ffmoe kernels need 1 <= topk_group <= min(n_group, "
                                      f"{L.MAX_TOPK}), got {topk_group}")
        if topk_group * (E // n_group) < top_k:
            raise NotImplementedError("the selected groups must hold at least top_k experts")
    jitter = float(input_jitter) if (input_jitter > 0.0 and hidden_states.requires_grad) else 0.0

    cfg = (top_k, activation, gating, capacity_factor, bool(recompute_activations),
           max_tokens_per_expert, bool(allow_dropped_tokens), float(aux_loss_coeff),
           float(z_loss_coeff))
    rcfg = (bool(pre_softmax), scoring_factor, n_group if groups else None,
            topk_group if groups else None, jitter, bool(advanced))
    s_gate = s_up = s_down = s_act = None
    if _shared is not None:
        s_gate, s_up, s_down, s_act = _shared
    out, aux, z, counts, stats, istats = _FusedMoEFunction.apply(
        hidden_states, gate_weight, w_up, w_down, expert_bias, s_gate, s_up, s_down, cfg, rcfg, s_act)

    losses = {}
    if aux_loss_coeff > 0.0:
        losses["aux_loss"] = aux
    if z_loss_coeff > 0.0:
        losses["z_loss"] = z
    if return_metrics:                                                  # fused_moe.py:1196-1217
        losses["tokens_per_expert"] = counts
        losses["max_expert_load"] = istats[L.ISTAT_MAX]
        losses["min_expert_load"] = istats[L.ISTAT_MIN]
        losses["expert_load_imbalance"] = stats[L.STAT_IMBALANCE]
        if capacity_factor is not None:
            losses["dropped_token_count"] = istats[L.ISTAT_DROPPED].long()
            losses["dropped_token_fraction"] = stats[L.STAT_DROP_FRAC]
    return out, losses
