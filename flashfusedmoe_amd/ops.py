"""torch custom ops over libffmoe.so: routing, expert forward, expert backward.

Each op enqueues HIP kernels on the current stream through the C ABI of
include/ffmoe.h and allocates its outputs with the torch caching allocator.
Fake (meta) implementations make the ops traceable by torch.compile.

The compute dtype is bfloat16 (the MFMA pipeline) or float32 / float64 (the
reference's computation in the input dtype, on this library's fp32 / fp64
kernels, ffmoe_t_* in include/ffmoe.h).  Tensors must be on a ROCm GPU;
there is no CPU path.
"""

import ctypes
import os
from typing import List, Optional

import torch
from torch import Tensor

from . import _lib as L

_BF16 = torch.bfloat16
# FFMOE_CHECK_GEMM=1: check the grouped GEMMs' stream-K workspace after every
# expert forward / backward (synchronises the stream; a debugging aid)
_CHECK_GEMM = os.environ.get("FFMOE_CHECK_GEMM", "0") not in ("", "0")


def _require(cond, msg):
    if not cond:
        raise ValueError(msg)


# compute dtypes of the fp32 / fp64 path -> FFMOE_DTYPE_* codes
T_DTYPES = {torch.float32: 1, torch.float64: 2}
# row tile of the fp32 / fp64 grouped GEMM (ffmoe_t_gemm_rows)
T_TILE_ROWS = 64


def _check_t_gpu(name, t, dtype):
    if t.device.type != "cuda":
        raise RuntimeError(f"ffmoe: {name} must be on a ROCm GPU (got {t.device}); "
                           "the fused MoE kernels have no CPU path")
    if t.dtype != dtype:
        raise TypeError(f"ffmoe: {name} must be {dtype} like the hidden states (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"ffmoe: {name} must be contiguous")


def _check_bf16_gpu(name, t):
    if t.device.type != "cuda":
        raise RuntimeError(f"ffmoe: {name} must be on a ROCm GPU (got {t.device}); "
                           "the fused MoE kernels have no CPU path")
    if t.dtype != _BF16:
        raise TypeError(f"ffmoe: {name} must be bfloat16 (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"ffmoe: {name} must be contiguous")


# ---------------------------------------------------------------------------
# routing: gate GEMM + top-k + histogram scan + losses/metrics
# ---------------------------------------------------------------------------

# Largest gate matrix (E x D elements) whose GEMM runs inside the route
# kernel, which streams the whole gate through every 16-token block.  Above
# it the logits come from this library's MFMA gate GEMM (ffmoe_gate_logits)
# and the route kernel routes them (the fused kernel took 134 us at N 16384 /
# E 64 / D 2048 and 1099 us at N 4096 / E 256 / D 7168; at E 8 / D 1024 and
# E 8 / D 4096 it is the faster by ~20 us).
FUSED_GATE_MAX_ELEMS = 32768


def _pad_cols(t, mult):
    """t [R, C] with its columns zero-padded to a multiple of `mult`."""
    C = t.shape[1]
    Cp = -(-C // mult) * mult
    if Cp == C:
        return t
    out = t.new_zeros(t.shape[0], Cp)
    out[:, :C] = t
    return out


def _pad_rows(t, mult):
    """t [R, C] with zero rows appended up to a multiple of `mult` rows."""
    R = t.shape[0]
    Rp = -(-R // mult) * mult
    if Rp == R:
        return t
    out = t.new_zeros(Rp, t.shape[1])
    out[:R] = t
    return out


def gate_logits(x, gate):
    """bf16 logits [N, E] = x gate^T on the MFMA gate GEMM; experts are
    zero-padded to a multiple of 8 (padded logits are sliced off)."""
    N, D = x.shape
    E = gate.shape[0]
    g = _pad_rows(gate, 8)
    Ep = g.shape[0]
    out = torch.empty(N, Ep, dtype=_BF16, device=x.device)
    ws = torch.empty(max(1, int(L.load().ffmoe_gate_logits_workspace_bytes(N, D, Ep))), dtype=torch.uint8,
                     device=x.device)
    L.call("ffmoe_gate_logits", L.ptr(x), L.ptr(g), N, D, Ep, L.ptr(out), L.ptr(ws), L.stream_ptr(x.device))
    return out if Ep == E else out[:, :E].contiguous()


def gate_dx(gl, gate):
    """bf16 [N, D] = gl gate on the MFMA pipeline; experts zero-padded to a
    multiple of 64 (zero columns of gl meet zero rows of the gate)."""
    N, E = gl.shape
    D = gate.shape[1]
    glp = _pad_cols(gl, 64)
    gp = _pad_rows(gate, 64)
    out = torch.empty(N, D, dtype=_BF16, device=gl.device)
    L.call("ffmoe_gate_dx", L.ptr(glp), L.ptr(gp), N, D, glp.shape[1], L.ptr(out), L.stream_ptr(gl.device))
    return out


def gate_grad(gl, x):
    """bf16 dgate [E, D] = gl^T x: the fused dot2 kernel up to 32 experts,
    the MFMA pipeline above (experts zero-padded to a multiple of 8)."""
    N, E = gl.shape
    D = x.shape[1]
    glp = gl if E <= L.MAX_FUSED_GATE_E else _pad_cols(gl, 8)
    Ep = glp.shape[1]
    dgate = torch.empty(Ep, D, dtype=_BF16, device=x.device)
    part = torch.empty(max(1, int(L.load().ffmoe_gate_grad_workspace_bytes(N, D, Ep))), dtype=torch.uint8,
                       device=x.device)
    L.call("ffmoe_gate_grad", L.ptr(glp), L.ptr(x), N, D, Ep, L.ptr(part), L.ptr(dgate),
           L.stream_ptr(x.device))
    return dgate if Ep == E else dgate[:E].contiguous()


@torch.library.custom_op("ffmoe::route", mutates_args=())
def route(x: Tensor, gate: Tensor, expert_bias: Optional[Tensor], top_k: int, gating: int,
          mt: int, aux_coeff: float, z_coeff: float, need_ssum: bool, bias_round: bool = False,
          pre_softmax: bool = False, scoring: float = 0.0, n_group: int = 0, topk_group: int = 0,
          noise: Optional[Tensor] = None) -> List[Tensor]:
    """Returns [logits bf16 [N,E], topk_idx int64 [N,k], topk_w fp32 [N,k],
    lse fp32 [N], counts int32 [E], offsets int32 [E+1], tile_offsets int32
    [E+1], stats fp32 [4], istats int32 [4], workspace uint8, aux_loss fp32 [],
    z_loss fp32 []] (the two losses repeat stats[AUX] and stats[Z] as
    separate tensors).  bias_round / pre_softmax / scoring / n_group /
    topk_group / noise are ffmoe_route_fwd_ex's routing options.  With fp32
    / fp64 hidden states the logits are fp32 (x gate^T in the dtype, then
    rounded as the reference's logits.float()) and bias_round is unused."""
    if x.dtype in T_DTYPES:
        return _route_t(x, gate, expert_bias, top_k, gating, mt, aux_coeff, z_coeff, need_ssum,
                        pre_softmax, scoring, n_group, topk_group, noise)
    _check_bf16_gpu("hidden_states", x)
    _check_bf16_gpu("gate_weight", gate)
    N, D = x.shape
    E = gate.shape[0]
    k = top_k
    dev = x.device
    ws = torch.empty(L.route_workspace_bytes(N, E, k), dtype=torch.uint8, device=dev)
    logits = torch.empty(N, E, dtype=_BF16, device=dev)
    topk_idx = torch.empty(N, k, dtype=torch.int64, device=dev)
    topk_w = torch.empty(N, k, dtype=torch.float32, device=dev)
    lse = torch.empty(N, dtype=torch.float32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    tile_offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    stats = torch.empty(L.NUM_STATS, dtype=torch.float32, device=dev)
    istats = torch.empty(L.NUM_ISTATS, dtype=torch.int32, device=dev)
    aux = torch.empty((), dtype=torch.float32, device=dev)
    z = torch.empty((), dtype=torch.float32, device=dev)
    bias = None
    if expert_bias is not None:
        bias = expert_bias.to(device=dev, dtype=torch.float32).contiguous()
    st = L.stream_ptr(dev)
    if noise is not None:
        _check_bf16_gpu("input jitter noise", noise)
    logits_in = None
    if E * D > FUSED_GATE_MAX_ELEMS and D % 64 == 0:
        # the route kernel streams the whole gate matrix through every
        # 16-token block; a large gate goes through the MFMA gate GEMM and
        # the kernel routes its bf16 logits
        xin = x if noise is None else x * noise  # bf16(x * noise), as the kernel's jitter
        logits = gate_logits(xin, gate)
        logits_in, noise = logits, None
    L.call("ffmoe_route_fwd_ex", L.ptr(x), L.ptr(gate), L.ptr(logits_in), L.ptr(bias),
           int(bias_round), int(pre_softmax), float(scoring), int(n_group), int(topk_group),
           L.ptr(noise), N, D, E, k, gating, int(need_ssum),
           None if logits_in is not None else L.ptr(logits), L.ptr(topk_idx), L.ptr(topk_w),
           L.ptr(lse), L.ptr(ws), st)
    L.call("ffmoe_route_scan", N, E, k, mt, L.gemm_tile_rows(N * k, E), aux_coeff, z_coeff, gating,
           L.ptr(ws), L.ptr(counts), L.ptr(offsets), L.ptr(tile_offsets), L.ptr(stats),
           L.ptr(istats), L.ptr(aux), L.ptr(z), st)
    return [logits, topk_idx, topk_w, lse, counts, offsets, tile_offsets, stats, istats, ws, aux, z]


def _route_t(x, gate, expert_bias, top_k, gating, mt, aux_coeff, z_coeff, need_ssum, pre_softmax,
             scoring, n_group, topk_group, noise):
    """route() for fp32 / fp64 hidden states: the gate product in the dtype
    (fp32 output), the route kernel on the fp32 logits, the scan with the
    fp32 / fp64 GEMM's 64-row tiles."""
    _check_t_gpu("hidden_states", x, x.dtype)
    _check_t_gpu("gate_weight", gate, x.dtype)
    dt = T_DTYPES[x.dtype]
    N, D = x.shape
    E = gate.shape[0]
    k = top_k
    dev = x.device
    f32 = torch.float32
    ws = torch.empty(L.route_workspace_bytes(N, E, k), dtype=torch.uint8, device=dev)
    logits = torch.empty(N, E, dtype=f32, device=dev)
    topk_idx = torch.empty(N, k, dtype=torch.int64, device=dev)
    topk_w = torch.empty(N, k, dtype=f32, device=dev)
    lse = torch.empty(N, dtype=f32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    tile_offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    stats = torch.empty(L.NUM_STATS, dtype=f32, device=dev)
    istats = torch.empty(L.NUM_ISTATS, dtype=torch.int32, device=dev)
    aux = torch.empty((), dtype=f32, device=dev)
    z = torch.empty((), dtype=f32, device=dev)
    bias = None if expert_bias is None else expert_bias.to(device=dev, dtype=f32).contiguous()
    st = L.stream_ptr(dev)
    xin = x
    if noise is not None:  # (x * noise) gate^T in the dtype (fused_moe.py:329-332)
        _check_t_gpu("input jitter noise", noise, x.dtype)
        xin = x * noise
    L.call("ffmoe_t_gemm_dense", dt, 0, 1, L.ptr(xin), L.ptr(gate), L.ptr(logits), N, E, D, D, D, E, 1, st)
    L.call("ffmoe_route_logits_f32", L.ptr(logits), L.ptr(bias), int(pre_softmax), float(scoring),
           int(n_group), int(topk_group), N, E, k, gating, int(need_ssum), L.ptr(topk_idx), L.ptr(topk_w),
           L.ptr(lse), L.ptr(ws), st)
    L.call("ffmoe_route_scan", N, E, k, mt, T_TILE_ROWS, aux_coeff, z_coeff, gating, L.ptr(ws),
           L.ptr(counts), L.ptr(offsets), L.ptr(tile_offsets), L.ptr(stats), L.ptr(istats), L.ptr(aux),
           L.ptr(z), st)
    return [logits, topk_idx, topk_w, lse, counts, offsets, tile_offsets, stats, istats, ws, aux, z]


@route.register_fake
def _route_fake(x, gate, expert_bias, top_k, gating, mt, aux_coeff, z_coeff, need_ssum,
                bias_round=False, pre_softmax=False, scoring=0.0, n_group=0, topk_group=0,
                noise=None):
    N, D = x.shape
    E = gate.shape[0]
    f = lambda *s, dtype: x.new_empty(s, dtype=dtype)  # noqa: E731
    return [f(N, E, dtype=_BF16 if x.dtype == _BF16 else torch.float32), f(N, top_k, dtype=torch.int64), f(N, top_k, dtype=torch.float32),
            f(N, dtype=torch.float32), f(E, dtype=torch.int32), f(E + 1, dtype=torch.int32),
            f(E + 1, dtype=torch.int32), f(L.NUM_STATS, dtype=torch.float32),
            f(L.NUM_ISTATS, dtype=torch.int32), f(0, dtype=torch.uint8), f(dtype=torch.float32),
            f(dtype=torch.float32)]


# ---------------------------------------------------------------------------
# experts forward: permute + up GEMM/GLU + down GEMM + combine
# ---------------------------------------------------------------------------

def _byref(g):
    return None if g is None else ctypes.byref(g)


def _up_down(xs, w_up, w_down, offsets, tile_offsets, activation, save_up, st, shared=None):
    """Routed up GEMM + GLU and down GEMM.  shared = (x, w_gu, w_sd, act) adds
    the shared expert as a dense row group of the same launches and returns
    its (up, act, down) as well."""
    T, D = xs.shape
    E, H2, _ = w_up.shape
    H = H2 // 2
    dev = xs.device
    up = torch.empty(T, H2, dtype=_BF16, device=dev) if save_up else None
    act = torch.empty(T, H, dtype=_BF16, device=dev)
    down = torch.empty(T, D, dtype=_BF16, device=dev)
    tr = L.gemm_tile_rows(T, E)
    ws = L.ptr(L.gemm_workspace(dev, st))
    g_up = g_down = None
    sh = None
    if shared is not None:
        x, w_gu, w_sd, sact = shared
        N = x.shape[0]
        sh = (torch.empty(N, H2, dtype=_BF16, device=dev), torch.empty(N, H, dtype=_BF16, device=dev),
              torch.empty(N, D, dtype=_BF16, device=dev))
        g_up = L.dense_group(x, w_gu, sh[1], N, sact, c2=sh[0])
        g_down = L.dense_group(sh[1], w_sd, sh[2], N, 0)
    # one persistent launch where it applies (a row tile's down tiles start
    # as soon as its up tiles are done), else the two GEMMs
    L.call("ffmoe_gemm_up_down_shared", L.ptr(xs), L.ptr(w_up), L.ptr(w_down), L.ptr(offsets),
           L.ptr(tile_offsets), tr, E, T, D, H, activation, L.ptr(up), L.ptr(act), L.ptr(down),
           _byref(g_up), _byref(g_down), ws, st)
    return up, act, down, sh


@torch.library.custom_op("ffmoe::experts_forward", mutates_args=())
def experts_forward(x: Tensor, w_up: Tensor, w_down: Tensor, topk_idx: Tensor, topk_w: Tensor,
                    counts: Tensor, offsets: Tensor, tile_offsets: Tensor, ws: Tensor, top_k: int,
                    activation: int, mt: int, capacity_mode: bool,
                    save_activations: bool, shared_w_gu: Optional[Tensor] = None,
                    shared_w_down: Optional[Tensor] = None, shared_act: int = 0) -> List[Tensor]:
    """Returns [out bf16 [N,D], topk_w fp32 [N,k] renormalised under capacity
    dropping (empty without capacity: the weights are topk_w unchanged),
    row_of int32 [N*k], x_sorted bf16 [N*k,D], up, act, down, up_sh, act_sh]
    where up/act/down are empty when save_activations is False.  With
    shared_w_gu [2H,D] (gate rows, then up rows) and shared_w_down [D,H] the
    shared expert runs as a dense row group of the same GEMM launches and
    `out` is bf16(routed + shared) (nn.py:156-159); up_sh / act_sh are its
    pre-activation and activation (empty without it).  fp32 / fp64 x: the
    fp32 / fp64 kernels (no shared-expert group there)."""
    if x.dtype in T_DTYPES:
        _require(shared_w_gu is None, "the shared-expert group runs on the bf16 path only")
        return _experts_forward_t(x, w_up, w_down, topk_idx, topk_w, counts, offsets, tile_offsets, ws,
                                  top_k, activation, mt, capacity_mode, save_activations)
    _check_bf16_gpu("w_up", w_up)
    _check_bf16_gpu("w_down", w_down)
    N, D = x.shape
    E = w_up.shape[0]
    k = top_k
    T = N * k
    dev = x.device
    st = L.stream_ptr(dev)
    tw = topk_w.clone() if capacity_mode else topk_w
    xs = torch.empty(T, D, dtype=_BF16, device=dev)
    row_of = torch.empty(T, dtype=torch.int32, device=dev)
    L.call("ffmoe_permute", L.ptr(x), L.ptr(topk_idx), L.ptr(tw), L.ptr(offsets), L.ptr(counts),
           N, D, E, k, mt, int(capacity_mode), L.ptr(ws), L.ptr(xs), L.ptr(row_of), st)
    shared = None
    if shared_w_gu is not None:
        _check_bf16_gpu("shared expert w_gate|w_up", shared_w_gu)
        _check_bf16_gpu("shared expert w_down", shared_w_down)
        shared = (x, shared_w_gu, shared_w_down, shared_act)
    up, act, down, sh = _up_down(xs, w_up, w_down, offsets, tile_offsets, activation,
                                 save_activations, st, shared)
    out = torch.empty(N, D, dtype=_BF16, device=dev)
    # the shared expert's output is the combine's addend: bf16(bf16(sum) + shared)
    L.call("ffmoe_combine", L.ptr(down), L.ptr(row_of), L.ptr(tw), None if sh is None else L.ptr(sh[2]),
           N, D, k, L.ptr(out), st)
    if _CHECK_GEMM:
        L.check_gemm_workspaces()
    tw_out = tw if capacity_mode else topk_w.new_empty(0)
    empty = x.new_empty(0)
    sh_out = [empty.clone(), empty.clone()] if sh is None else [sh[0], sh[1]]
    if not save_activations:
        return [out, tw_out, row_of, xs, empty, empty.clone(), empty.clone(), *sh_out]
    return [out, tw_out, row_of, xs, up, act, down, *sh_out]


def _up_down_t(xs, w_up, w_down, offsets, tile_offsets, activation, st):
    """fp32 / fp64 routed up product, GLU (fp32 math), down product."""
    dt = T_DTYPES[xs.dtype]
    T, D = xs.shape
    E, H2, _ = w_up.shape
    H = H2 // 2
    e = lambda *s: xs.new_empty(s)  # noqa: E731
    up, act, down = e(T, H2), e(T, H), e(T, D)
    P = L.ptr
    L.call("ffmoe_t_gemm_rows", dt, P(xs), P(w_up), P(offsets), P(tile_offsets), E, T, D, H2, 0, P(up), st)
    L.call("ffmoe_t_glu_fwd", dt, P(up), T, H, activation, 0, P(act), st)
    L.call("ffmoe_t_gemm_rows", dt, P(act), P(w_down), P(offsets), P(tile_offsets), E, T, H, D, 0, P(down), st)
    return up, act, down


def _experts_forward_t(x, w_up, w_down, topk_idx, topk_w, counts, offsets, tile_offsets, ws, top_k,
                       activation, mt, capacity_mode, save_activations):
    """experts_forward() in fp32 / fp64: the same permutation and combine
    order as the bf16 path; products in the dtype, GLU and combine sums in
    fp32 stored in the dtype (activations.py:58-74, moe_ops.py:190-203)."""
    dtype = x.dtype
    for name, t in (("hidden_states", x), ("w_up", w_up), ("w_down", w_down)):
        _check_t_gpu(name, t, dtype)
    dt = T_DTYPES[dtype]
    N, D = x.shape
    E = w_up.shape[0]
    k = top_k
    T = N * k
    dev = x.device
    st = L.stream_ptr(dev)
    P = L.ptr
    tw = topk_w.clone() if capacity_mode else topk_w
    xs = torch.empty(T, D, dtype=dtype, device=dev)
    row_of = torch.empty(T, dtype=torch.int32, device=dev)
    L.call("ffmoe_t_permute", dt, P(x), P(topk_idx), P(tw), P(offsets), P(counts), N, D, E, k, mt,
           int(capacity_mode), P(ws), P(xs), P(row_of), st)
    up, act, down = _up_down_t(xs, w_up, w_down, offsets, tile_offsets, activation, st)
    out = torch.empty(N, D, dtype=dtype, device=dev)
    L.call("ffmoe_t_combine", dt, P(down), P(row_of), P(tw), None, N, D, k, P(out), st)
    tw_out = tw if capacity_mode else topk_w.new_empty(0)
    empty = x.new_empty(0)
    if not save_activations:
        up, act, down = empty, empty.clone(), empty.clone()
    return [out, tw_out, row_of, xs, up, act, down, empty.clone(), empty.clone()]


@experts_forward.register_fake
def _experts_forward_fake(x, w_up, w_down, topk_idx, topk_w, counts, offsets, tile_offsets, ws,
                          top_k, activation, mt, capacity_mode, save_activations, shared_w_gu=None,
                          shared_w_down=None, shared_act=0):
    N, D = x.shape
    H2 = w_up.shape[1]
    T = N * top_k
    e = x.new_empty
    if save_activations:
        acts = [e(T, H2), e(T, H2 // 2), e(T, D)]
    else:
        acts = [e(0), e(0), e(0)]
    sh = [e(N, H2), e(N, H2 // 2)] if shared_w_gu is not None else [e(0), e(0)]
    tw = topk_w.new_empty(topk_w.shape) if capacity_mode else topk_w.new_empty(0)
    return [e(N, D), tw, e(T, dtype=torch.int32), e(T, D), *acts, *sh]


# ---------------------------------------------------------------------------
# experts backward
# ---------------------------------------------------------------------------

@torch.library.custom_op("ffmoe::experts_backward", mutates_args=())
def experts_backward(go: Tensor, x: Tensor, gate: Tensor, w_up: Tensor, w_down: Tensor,
                     logits: Tensor, topk_idx: Tensor, topk_w: Tensor, lse: Tensor, counts: Tensor,
                     offsets: Tensor, tile_offsets: Tensor, row_of: Tensor, xs: Tensor, up: Tensor,
                     act: Tensor, down: Tensor, g_aux: Optional[Tensor], g_z: Optional[Tensor],
                     top_k: int, activation: int, gating: int, capacity_mode: bool,
                     aux_coeff: float, z_coeff: float, aux_through_weights: bool = False,
                     aux_idx: Optional[Tensor] = None, aux_counts: Optional[Tensor] = None,
                     pre_softmax: bool = False, scoring: float = 0.0,
                     shared_w_gu: Optional[Tensor] = None, shared_w_down: Optional[Tensor] = None,
                     up_sh: Optional[Tensor] = None, act_sh: Optional[Tensor] = None,
                     shared_act: int = 0) -> List[Tensor]:
    """Returns [grad_hidden [N,D], grad_gate [E,D], grad_w_up [E,2H,D],
    grad_w_down [E,D,H], grad_shared_w_gu [2H,D], grad_shared_w_down [D,H]],
    all bf16 (the last two empty without the shared expert).  Empty
    up/act/down trigger recompute.  logits / lse are the un-jittered ones;
    aux_* describe the aux loss's own routing (ffmoe_route_bwd_ex).  With the
    shared expert (its weights and saved up_sh / act_sh) its four GEMMs run as
    a dense row group of the routed launches, and grad_hidden includes its
    input gradient.  fp32 / fp64 x: the fp32 / fp64 kernels (logits fp32)."""
    if x.dtype in T_DTYPES:
        _require(shared_w_gu is None, "the shared-expert group runs on the bf16 path only")
        return _experts_backward_t(go, x, gate, w_up, w_down, logits, topk_idx, topk_w, lse, counts,
                                   offsets, tile_offsets, row_of, xs, up, act, down, g_aux, g_z, top_k,
                                   activation, gating, capacity_mode, aux_coeff, z_coeff,
                                   aux_through_weights, aux_idx, aux_counts, pre_softmax, scoring)
    _check_bf16_gpu("grad_output", go)
    N, D = x.shape
    E, H2, _ = w_up.shape
    H = H2 // 2
    k = top_k
    T = N * k
    dev = x.device
    st = L.stream_ptr(dev)
    if up.numel() == 0:  # recompute_activations: same kernels, same bits
        up, act, down, _ = _up_down(xs, w_up, w_down, offsets, tile_offsets, activation, True, st)
    has_sh = shared_w_gu is not None
    g_wd = g_dg = g_wu = g_dx = None
    if has_sh:
        dw_gu_sh = torch.empty(H2, D, dtype=_BF16, device=dev)
        dw_sd_sh = torch.empty(D, H, dtype=_BF16, device=dev)
        gup_sh = torch.empty(N, H2, dtype=_BF16, device=dev)
        dx_sh = torch.empty(N, D, dtype=_BF16, device=dev)
        # the shared expert's grads (nn.py:22-44 under autograd): its output
        # gradient is go itself
        g_wd = L.dense_group(go, act_sh, dw_sd_sh, N, 0)           # go^T act
        g_dg = L.dense_group(go, shared_w_down, gup_sh, N, shared_act, up=up_sh)  # GLU'(go w_down)
        g_wu = L.dense_group(gup_sh, x, dw_gu_sh, N, 0)            # gup^T x
        g_dx = L.dense_group(gup_sh, shared_w_gu, dx_sh, N, 0)     # gup w_gu
    wgo = torch.empty(T, D, dtype=_BF16, device=dev)
    gl = torch.empty(N, E, dtype=_BF16, device=dev)
    ga = None if g_aux is None else g_aux.to(device=dev, dtype=torch.float32).contiguous()
    gz = None if g_z is None else g_z.to(device=dev, dtype=torch.float32).contiguous()
    L.call("ffmoe_route_bwd_ex", L.ptr(go), L.ptr(down), L.ptr(row_of), L.ptr(topk_idx),
           L.ptr(topk_w), L.ptr(logits), L.ptr(lse), L.ptr(counts), L.ptr(ga), L.ptr(gz),
           aux_coeff, z_coeff, N, D, E, k, gating, int(capacity_mode), int(aux_through_weights),
           L.ptr(aux_idx), L.ptr(aux_counts), int(pre_softmax), float(scoring), L.ptr(wgo),
           L.ptr(gl), None, st)
    # the down-projection weight gradient first, while the `wgo` rows the
    # routing backward just wrote are cache-resident (measured 0.5% faster per
    # C2 step than after the dX GEMMs)
    dwd = torch.empty(E, D, H, dtype=_BF16, device=dev)
    ws = L.ptr(L.gemm_workspace(dev, st))
    L.call("ffmoe_gemm_wgrad_shared", L.ptr(wgo), L.ptr(act), L.ptr(offsets), E, D, H, L.ptr(dwd),
           _byref(g_wd), ws, st)
    gup = torch.empty(T, H2, dtype=_BF16, device=dev)
    tr = L.gemm_tile_rows(T, E)
    L.call("ffmoe_gemm_dgrad_glu_shared", L.ptr(wgo), L.ptr(w_down), L.ptr(up), L.ptr(offsets),
           L.ptr(tile_offsets), tr, E, T, D, H, activation, L.ptr(gup), _byref(g_dg), ws, st)
    # the up-projection weight gradient and dX's GEMM both read `gup`, right
    # after the GEMM that wrote it (128 MiB at C2): one persistent launch
    # where it applies, else the wgrad then the dgrad
    dwu = torch.empty(E, H2, D, dtype=_BF16, device=dev)
    ghb = torch.empty(T, D, dtype=_BF16, device=dev)
    L.call("ffmoe_gemm_dgrad_wgrad_shared", L.ptr(gup), L.ptr(w_up), L.ptr(xs), L.ptr(offsets),
           L.ptr(tile_offsets), tr, E, T, H, D, L.ptr(ghb), L.ptr(dwu), _byref(g_dx), _byref(g_wu), ws, st)
    dx = torch.empty(N, D, dtype=_BF16, device=dev)
    fused_gate = E <= L.MAX_FUSED_GATE_E
    if fused_gate:  # the gl @ gate term is computed inside the dX reduce
        L.call("ffmoe_dx_reduce", L.ptr(ghb), L.ptr(row_of), L.ptr(gl), L.ptr(gate), N, D, E, k,
               L.ptr(dx), st)
    else:  # many experts: gl @ gate on the MFMA pipeline, added by the combine
        addend = gate_dx(gl, gate)
        L.call("ffmoe_combine", L.ptr(ghb), L.ptr(row_of), None, L.ptr(addend), N, D, k, L.ptr(dx),
               st)
    dgate = gate_grad(gl, x)
    if _CHECK_GEMM:
        L.check_gemm_workspaces()
    if not has_sh:
        e0 = x.new_empty(0)
        return [dx, dgate, dwu, dwd, e0, e0.clone()]
    # x's gradient from both branches, bf16 + bf16 as autograd accumulates it
    return [dx + dx_sh, dgate, dwu, dwd, dw_gu_sh, dw_sd_sh]


def _experts_backward_t(go, x, gate, w_up, w_down, logits, topk_idx, topk_w, lse, counts, offsets,
                        tile_offsets, row_of, xs, up, act, down, g_aux, g_z, top_k, activation, gating,
                        capacity_mode, aux_coeff, z_coeff, aux_through_weights, aux_idx, aux_counts,
                        pre_softmax, scoring):
    """experts_backward() in fp32 / fp64 (fused_moe.py:511-591): routing
    backward and weighted scatter, dgrad products with the GLU backward
    between them, the unweighted dX gather plus gl gate, the four weight
    gradients, all products in the dtype."""
    dtype = x.dtype
    _check_t_gpu("grad_output", go, dtype)
    dt = T_DTYPES[dtype]
    N, D = x.shape
    E, H2, _ = w_up.shape
    H = H2 // 2
    k = top_k
    T = N * k
    dev = x.device
    st = L.stream_ptr(dev)
    P = L.ptr
    if up.numel() == 0:  # recompute_activations: same kernels, same bits
        up, act, down = _up_down_t(xs, w_up, w_down, offsets, tile_offsets, activation, st)
    e = lambda *s: x.new_empty(s)  # noqa: E731
    wgo, gl = e(T, D), e(N, E)
    ga = None if g_aux is None else g_aux.to(device=dev, dtype=torch.float32).contiguous()
    gz = None if g_z is None else g_z.to(device=dev, dtype=torch.float32).contiguous()
    L.call("ffmoe_t_route_bwd", dt, P(go), P(down), P(row_of), P(topk_idx), P(topk_w), P(logits), P(lse),
           P(counts), P(ga), P(gz), aux_coeff, z_coeff, N, D, E, k, gating, int(capacity_mode),
           int(aux_through_weights), P(aux_idx), P(aux_counts), int(pre_softmax), float(scoring), P(wgo),
           P(gl), None, st)
    gact, gup, ghb = e(T, H), e(T, H2), e(T, D)
    L.call("ffmoe_t_gemm_rows", dt, P(wgo), P(w_down), P(offsets), P(tile_offsets), E, T, D, H, 1, P(gact), st)
    L.call("ffmoe_t_glu_bwd", dt, P(gact), P(up), T, H, activation, 0, P(gup), st)
    L.call("ffmoe_t_gemm_rows", dt, P(gup), P(w_up), P(offsets), P(tile_offsets), E, T, H2, D, 1, P(ghb), st)
    dwd, dwu = e(E, D, H), e(E, H2, D)
    L.call("ffmoe_t_gemm_wgrad", dt, P(wgo), P(act), P(offsets), E, D, H, P(dwd), st)
    L.call("ffmoe_t_gemm_wgrad", dt, P(gup), P(xs), P(offsets), E, H2, D, P(dwu), st)
    # grad_hidden = gather(ghb) + gl gate (fused_moe.py:556-561, :590)
    glg, dx = e(N, D), e(N, D)
    L.call("ffmoe_t_gemm_dense", dt, 0, 0, P(gl), P(gate), P(glg), N, D, E, E, D, D, 0, st)
    L.call("ffmoe_t_combine", dt, P(ghb), P(row_of), None, P(glg), N, D, k, P(dx), st)
    dgate = e(E, D)
    L.call("ffmoe_t_gemm_dense", dt, 1, 0, P(gl), P(x), P(dgate), E, D, N, E, D, D, 0, st)
    e0 = x.new_empty(0)
    return [dx, dgate, dwu, dwd, e0, e0.clone()]


@experts_backward.register_fake
def _experts_backward_fake(go, x, gate, w_up, w_down, logits, topk_idx, topk_w, lse, counts, offsets,
                           tile_offsets, row_of, xs, up, act, down, g_aux, g_z, top_k, activation,
                           gating, capacity_mode, aux_coeff, z_coeff, aux_through_weights=False,
                           aux_idx=None, aux_counts=None, pre_softmax=False, scoring=0.0,
                           shared_w_gu=None, shared_w_down=None, up_sh=None, act_sh=None,
                           shared_act=0):
    sh = ([shared_w_gu.new_empty(shared_w_gu.shape), shared_w_down.new_empty(shared_w_down.shape)]
          if shared_w_gu is not None else [x.new_empty(0), x.new_empty(0)])
    return [x.new_empty(x.shape), gate.new_empty(gate.shape), w_up.new_empty(w_up.shape),
            w_down.new_empty(w_down.shape), *sh]


# ---------------------------------------------------------------------------
# shared expert: a dense GLU FFN.  Its products are plain dense GEMMs (no
# routing, one row group), which go to hipBLASLt; the gate and up
# projections are one GEMM against the stacked [w_gate; w_up], and the GLU
# forward / backward each run as one fused kernel of this library.
# ---------------------------------------------------------------------------

@torch.library.custom_op("ffmoe::dense_glu_forward", mutates_args=())
def dense_glu_forward(x: Tensor, w_gu: Tensor, w_down: Tensor, activation: int) -> List[Tensor]:
    """x [N,D], w_gu [2H,D] (gate rows, then up rows), w_down [D,H] ->
    [out [N,D], up [N,2H] (pre-activation), act [N,H]], all bf16."""
    N, D = x.shape
    H = w_down.shape[1]
    _require(w_gu.shape == (2 * H, D) and w_down.shape == (D, H), "shared expert weight shapes")
    st = L.stream_ptr(x.device)
    if x.dtype in T_DTYPES:  # products and the GLU in the dtype, as the torch ops (nn.py:31-40)
        for name, t in (("x", x), ("w_gate|w_up", w_gu), ("w_down", w_down)):
            _check_t_gpu(name, t, x.dtype)
        dt, P = T_DTYPES[x.dtype], L.ptr
        up, act, out = x.new_empty(N, 2 * H), x.new_empty(N, H), x.new_empty(N, D)
        L.call("ffmoe_t_gemm_dense", dt, 0, 1, P(x), P(w_gu), P(up), N, 2 * H, D, D, D, 2 * H, 0, st)
        L.call("ffmoe_t_glu_fwd", dt, P(up), N, H, activation, 1, P(act), st)
        L.call("ffmoe_t_gemm_dense", dt, 0, 1, P(act), P(w_down), P(out), N, D, H, H, H, D, 0, st)
        return [out, up, act]
    for name, t in (("x", x), ("w_gate|w_up", w_gu), ("w_down", w_down)):
        _check_bf16_gpu(name, t)
    up = x @ w_gu.t()
    act = torch.empty(N, H, dtype=_BF16, device=x.device)
    L.call("ffmoe_glu_fwd", L.ptr(up), N, H, activation, L.ptr(act), st)
    out = act @ w_down.t()
    return [out, up, act]


@dense_glu_forward.register_fake
def _dense_glu_forward_fake(x, w_gu, w_down, activation):
    N, D = x.shape
    H = w_down.shape[1]
    return [x.new_empty(N, D), x.new_empty(N, 2 * H), x.new_empty(N, H)]


@torch.library.custom_op("ffmoe::dense_glu_backward", mutates_args=())
def dense_glu_backward(go: Tensor, x: Tensor, w_gu: Tensor, w_down: Tensor, up: Tensor,
                       act: Tensor, activation: int) -> List[Tensor]:
    """Returns [grad_x [N,D], grad_w_gu [2H,D], grad_w_down [D,H]] in x's dtype."""
    N, D = x.shape
    H = w_down.shape[1]
    st = L.stream_ptr(x.device)
    if x.dtype in T_DTYPES:
        _check_t_gpu("grad_output", go, x.dtype)
        dt, P = T_DTYPES[x.dtype], L.ptr
        gact, gup = x.new_empty(N, H), x.new_empty(N, 2 * H)
        dx, dwgu, dwd = x.new_empty(N, D), x.new_empty(2 * H, D), x.new_empty(D, H)
        L.call("ffmoe_t_gemm_dense", dt, 0, 0, P(go), P(w_down), P(gact), N, H, D, D, H, H, 0, st)
        L.call("ffmoe_t_glu_bwd", dt, P(gact), P(up), N, H, activation, 1, P(gup), st)
        L.call("ffmoe_t_gemm_dense", dt, 0, 0, P(gup), P(w_gu), P(dx), N, D, 2 * H, 2 * H, D, D, 0, st)
        L.call("ffmoe_t_gemm_dense", dt, 1, 0, P(go), P(act), P(dwd), D, H, N, D, H, H, 0, st)
        L.call("ffmoe_t_gemm_dense", dt, 1, 0, P(gup), P(x), P(dwgu), 2 * H, D, N, 2 * H, D, D, 0, st)
        return [dx, dwgu, dwd]
    _check_bf16_gpu("grad_output", go)
    gact = go @ w_down
    gup = torch.empty(N, 2 * H, dtype=_BF16, device=x.device)
    L.call("ffmoe_glu_bwd", L.ptr(gact), L.ptr(up), N, H, activation, L.ptr(gup), st)
    dx = gup @ w_gu
    dwd = go.t() @ act
    dwgu = gup.t() @ x
    return [dx, dwgu, dwd]


@dense_glu_backward.register_fake
def _dense_glu_backward_fake(go, x, w_gu, w_down, up, act, activation):
    return [x.new_empty(x.shape), w_gu.new_empty(w_gu.shape), w_down.new_empty(w_down.shape)]
