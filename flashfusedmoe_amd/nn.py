"""MoELayer: drop-in nn.Module over fused_moe() (reference src/flashfusemoe/nn.py).

Same constructor arguments, parameter names, initialisation order (so a given
torch seed yields the same parameters) and forward contract
``forward(x[*, D]) -> (out[*, D], losses)``.  The shared expert, when
present, keeps the reference's three bias-free linears as parameters
(nn.py:22-44) and is added to the routed output (nn.py:156-159); its gate
and up projections run as one dense GEMM against the stacked weights, and
its GLU forward / backward as single fused kernels of this library.
"""

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .fused_moe import _check_compute_dtype, _compute_dtype, fused_moe

# the shared expert's activations (nn.py:33-40); its GeGLU is the exact erf
# GELU of F.gelu, unlike the routed experts' tanh form
_SHARED_ACT = {"swiglu": 0, "geglu": 3, "relu_squared": 2}


class _SharedGLU(torch.autograd.Function):
    """down(act(x w_gate^T) * (x w_up^T)) w_down^T with its backward: five
    dense GEMMs (one for the stacked gate and up projections) and two fused
    GLU kernels, instead of nine GEMMs and the elementwise chain of three
    nn.Linear modules."""

    @staticmethod
    def forward(ctx, x, w_gate, w_up, w_down, act_id):
        dtype = _compute_dtype(x.dtype)
        _check_compute_dtype(dtype)
        xc = x.to(dtype).contiguous()
        w_gu = torch.cat([w_gate.to(dtype), w_up.to(dtype)], 0).contiguous()
        wd = w_down.to(dtype).contiguous()
        out, up, act = ops.dense_glu_forward(xc, w_gu, wd, act_id)
        ctx.save_for_backward(xc, w_gu, wd, up, act)
        ctx.act_id = act_id
        ctx.dtypes = (x.dtype, w_gate.dtype, w_up.dtype, w_down.dtype)
        return out

    @staticmethod
    def backward(ctx, go):
        xc, w_gu, wd, up, act = ctx.saved_tensors
        dx, dwgu, dwd = ops.dense_glu_backward(go.to(xc.dtype).contiguous(), xc, w_gu, wd,
                                               up, act, ctx.act_id)
        H = wd.shape[1]
        xd, gd, ud, dd = ctx.dtypes
        return dx.to(xd), dwgu[:H].to(gd), dwgu[H:].to(ud), dwd.to(dd), None


class _GLUFFN(nn.Module):
    """Shared-expert GLU FFN (nn.py:22-44): three bias-free linears; GeGLU
    here is the exact (erf) GELU, as in the reference's shared expert."""

    def __init__(self, d_model, ffn_dim, activation="swiglu"):
        super().__init__()
        intermediate = ffn_dim // 2
        self.w_gate = nn.Linear(d_model, intermediate, bias=False)
        self.w_up = nn.Linear(d_model, intermediate, bias=False)
        self.w_down = nn.Linear(intermediate, d_model, bias=False)
        self.activation = activation

    def forward(self, x):
        g = self.w_gate(x)
        u = self.w_up(x)
        if self.activation == "swiglu":
            a = F.silu(g) * u
        elif self.activation == "geglu":
            a = F.gelu(g) * u
        elif self.activation == "relu_squared":
            a = F.relu(g).square() * u
        else:
            raise ValueError(f"Unknown activation: {self.activation}")
        return self.w_down(a)


class MoELayer(nn.Module):
    """Fused Mixture-of-Experts layer (nn.py:47-176).

    Returns (output, losses); losses is empty unless aux/z losses are on.
    Computes in the autocast dtype, else the input dtype: bfloat16 on the
    MFMA kernels (the shared expert folded into the routed GEMM launches
    when d_model and ffn_dim/2 are multiples of 64), float32 / float64 on the
    fp32 / fp64 kernels (the default fp32 parameters without autocast);
    float16 raises TypeError.
    """

    def __init__(
        self,
        d_model: int,
        ffn_dim: int,
        num_experts: int,
        top_k: int = 2,
        activation: str = "swiglu",
        gating: str = "softmax",
        num_shared_experts: int = 0,
        latent_dim=None,
        capacity_factor=None,
        max_tokens_per_expert=None,
        allow_dropped_tokens: bool = True,
        aux_loss_coeff: float = 0.0,
        z_loss_coeff: float = 0.0,
        recompute_activations: bool = False,
    ):
        super().__init__()
        self.d_model = d_model
        self.ffn_dim = ffn_dim
        self.num_experts = num_experts
        self.top_k = top_k
        self.activation = activation
        self.gating = gating
        self.half_ffn = ffn_dim // 2
        self.max_tokens_per_expert = max_tokens_per_expert
        self.allow_dropped_tokens = allow_dropped_tokens
        self.aux_loss_coeff = aux_loss_coeff
        self.z_loss_coeff = z_loss_coeff
        self.capacity_factor = capacity_factor
        self.recompute_activations = recompute_activations
        self._ep_group = None
        self._ep_size = 1

        # initialisation order and distributions follow nn.py:93-117
        self.gate = nn.Linear(d_model, num_experts, bias=False)
        nn.init.kaiming_uniform_(self.gate.weight, a=math.sqrt(5))
        self.gate.weight.data *= 0.01
        self.w_up = nn.Parameter(torch.empty(num_experts, ffn_dim, d_model))
        self.w_down = nn.Parameter(torch.empty(num_experts, d_model, self.half_ffn))
        self._init_expert_weights()
        self.shared_expert = _GLUFFN(d_model, ffn_dim, activation) if num_shared_experts > 0 else None
        # latent projections exist for the reference's expert-parallel
        # all-to-all compression; they are created (same RNG use) but unused
        self.latent_dim = latent_dim
        if latent_dim is not None:
            self.proj_down = nn.Linear(d_model, latent_dim, bias=False)
            self.proj_up = nn.Linear(latent_dim, d_model, bias=False)

    def _init_expert_weights(self):
        for e in range(self.w_up.shape[0]):
            nn.init.kaiming_uniform_(self.w_up.data[e], a=math.sqrt(5))
            nn.init.kaiming_uniform_(self.w_down.data[e], a=math.sqrt(5))

    def forward(self, x):
        """x: [*, D] -> ([*, D], dict)"""
        leading = x.shape[:-1]
        D = x.shape[-1]
        x_flat = x.reshape(-1, D)
        se = self.shared_expert
        if se is not None and se.activation not in _SHARED_ACT:
            raise ValueError(f"Unknown activation: {se.activation}")
        # the shared expert runs inside the routed GEMM launches (a dense row
        # group) when its dimensions suit the direct-to-LDS pipeline; else
        # as its own dense GEMMs after the routed op
        fold = (se is not None and _compute_dtype(x.dtype) == torch.bfloat16 and D % 64 == 0
                and self.half_ffn % 64 == 0)
        shared = None
        if fold:
            shared = (se.w_gate.weight, se.w_up.weight, se.w_down.weight, _SHARED_ACT[se.activation])
        routed, losses = fused_moe(
            x_flat, self.gate.weight, self.w_up, self.w_down, self.top_k,
            activation=self.activation,
            gating=self.gating,
            capacity_factor=self.capacity_factor,
            aux_loss_coeff=self.aux_loss_coeff,
            z_loss_coeff=self.z_loss_coeff,
            recompute_activations=self.recompute_activations,
            max_tokens_per_expert=self.max_tokens_per_expert,
            allow_dropped_tokens=self.allow_dropped_tokens,
            _shared=shared,
        )
        if se is not None and not fold:
            routed = routed + _SharedGLU.apply(x_flat, se.w_gate.weight, se.w_up.weight,
                                               se.w_down.weight, _SHARED_ACT[se.activation])
        return routed.reshape(*leading, D), losses

    def shard_experts(self, ep_group, ep_backend="nccl"):
        raise NotImplementedError("expert parallelism is not part of this single-GPU build")

    @property
    def expert_params(self):
        """Routed-expert parameters (nn.py:173-176)."""
        return [self.w_up, self.w_down]
