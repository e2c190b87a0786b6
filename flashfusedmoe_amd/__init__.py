"""flashfusedmoe_amd: a fused Mixture-of-Experts layer for AMD Instinct MI355X.

Drop-in for the non-expert-parallel API of AdaMLLab/FlashFusedMoE
(``fused_moe``, ``MoELayer``), computed by hand-written HIP kernels for gfx950
in libffmoe.so (C ABI: include/ffmoe.h).
"""

from .fused_moe import fused_moe, set_ep_group, _estimate_max_tokens
from .nn import MoELayer

__version__ = "0.1.0"

__all__ = ["fused_moe", "set_ep_group", "MoELayer"]
