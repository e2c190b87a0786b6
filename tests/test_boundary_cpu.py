"""CPU-side checks of the drop-in boundary: the C-ABI library loads and exports
every entry point include/ffmoe.h declares (no compute is launched), the
Python API validates like the reference, and MoELayer initialises its
parameters exactly as the reference does under the same seed.
"""

import math
import os
import re

import pytest
import torch

from flashfusedmoe_amd import _lib as L
from flashfusedmoe_amd import MoELayer, fused_moe, _estimate_max_tokens

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ffmoe.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ffmoe_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    declared = _declared_functions()
    assert declared, "no entry points parsed from include/ffmoe.h"
    assert sorted(L.SIGNATURES) == declared


def test_library_exports_every_declared_symbol():
    lib = L.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.ffmoe_version() >= 1
    # pure host queries (no GPU work)
    assert L.gemm_tile_rows(16384, 8) == 256
    assert L.gemm_tile_rows(32768, 256) == 128
    assert L.route_workspace_bytes(8192, 8, 2) >= 8192 * 2 * 4


def test_constants_match_header():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (FFMOE_\w+) \(?(-?\d+)\)?", text))
    assert int(consts["FFMOE_ROW_DROPPED"]) == L.ROW_DROPPED
    assert int(consts["FFMOE_ROW_ALIAS0"]) == L.ROW_ALIAS0
    assert int(consts["FFMOE_MAX_EXPERTS"]) == L.MAX_EXPERTS
    assert int(consts["FFMOE_MAX_TOPK"]) == L.MAX_TOPK
    assert int(consts["FFMOE_GATING_SIGMOID"]) == L.GATING["sigmoid"]
    assert int(consts["FFMOE_ACT_RELU2"]) == L.ACTIVATION["relu_squared"]
    assert int(consts["FFMOE_STAT_Z"]) == L.STAT_Z
    assert int(consts["FFMOE_ISTAT_DROPPED"]) == L.ISTAT_DROPPED


def test_entry_points_reject_bad_arguments_without_launching():
    lib = L.load()
    # E = 0 and k > E are rejected before any launch; the message is kept
    assert lib.ffmoe_route_fwd(None, None, None, None, 16, 64, 0, 1, 0, 0, None, None, None,
                               None, None, None) != 0
    assert b"E out of range" in lib.ffmoe_last_error()
    assert lib.ffmoe_gemm_wgrad(None, None, None, 4, 12, 16, None, None) != 0
    assert b"multiples of 8" in lib.ffmoe_last_error()
    with pytest.raises(L.FFMoEError, match="ffmoe_combine"):
        L.call("ffmoe_combine", None, None, None, None, 4, 12, 2, None, None)


# --- reference validation messages (tests/test_generality.py:179-218) ---------

def _inputs(N=8, D=16, ffn=32, E=4):
    return (torch.randn(N, D), torch.randn(E, D), torch.randn(E, ffn, D), torch.randn(E, D, ffn // 2))


@pytest.mark.parametrize("mutate,match", [
    (lambda a: (a[0].unsqueeze(0), *a[1:]), "hidden_states must be 2D"),
    (lambda a: (a[0], a[1][:, :8], *a[2:]), "gate_weight must be"),
    (lambda a: (a[0], a[1], a[2][:, :, :8], a[3]), "w_up must be"),
    (lambda a: (a[0], a[1], a[2], a[3][:, :, :4]), "w_down must be"),
])
def test_shape_validation_messages(mutate, match):
    args = mutate(_inputs())
    with pytest.raises(AssertionError, match=match):
        fused_moe(*args, top_k=2)


def test_topk_activation_gating_validation():
    a = _inputs()
    with pytest.raises(AssertionError, match="top_k must be in"):
        fused_moe(*a, top_k=5)
    with pytest.raises(AssertionError, match="top_k must be in"):
        fused_moe(*a, top_k=0)
    with pytest.raises(AssertionError, match="Unknown activation"):
        fused_moe(*a, top_k=2, activation="gelu")
    with pytest.raises(AssertionError, match="Unknown gating"):
        fused_moe(*a, top_k=2, gating="relu")


def test_cpu_tensors_have_no_fallback():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fused_moe(*(t.bfloat16() for t in _inputs()), top_k=2)


def test_fp16_compute_dtype_is_rejected():
    with pytest.raises(TypeError, match="bfloat16, float32 or float64"):
        fused_moe(*(t.half() for t in _inputs()), top_k=2)


def test_fp32_cpu_tensors_are_rejected_not_computed():
    # fp32 is a supported compute dtype, but there is no CPU path
    with pytest.raises(RuntimeError, match="no CPU path"):
        fused_moe(*_inputs(), top_k=2)


def test_estimate_max_tokens_known_answers():
    # tests/test_production.py:37-47
    assert _estimate_max_tokens(4, 2, 8) == 8
    assert 256 <= _estimate_max_tokens(1024, 2, 8) <= 2048
    assert _estimate_max_tokens(8192, 2, 8) == 4096


def test_moelayer_initialisation_matches_reference_order():
    # nn.py:93-117: gate Linear -> kaiming_uniform(a=sqrt5) -> *0.01; then per
    # expert w_up[e], w_down[e] kaiming; then the shared expert's three Linears
    torch.manual_seed(123)
    layer = MoELayer(64, 256, 4, top_k=2, num_shared_experts=1)
    torch.manual_seed(123)
    g = torch.nn.Linear(64, 4, bias=False)
    torch.nn.init.kaiming_uniform_(g.weight, a=math.sqrt(5))
    g.weight.data *= 0.01
    wu = torch.empty(4, 256, 64)
    wd = torch.empty(4, 64, 128)
    for e in range(4):
        torch.nn.init.kaiming_uniform_(wu[e], a=math.sqrt(5))
        torch.nn.init.kaiming_uniform_(wd[e], a=math.sqrt(5))
    sg = torch.nn.Linear(64, 128, bias=False)
    su = torch.nn.Linear(64, 128, bias=False)
    sd = torch.nn.Linear(128, 64, bias=False)
    assert torch.equal(layer.gate.weight, g.weight)
    assert torch.equal(layer.w_up, wu)
    assert torch.equal(layer.w_down, wd)
    assert torch.equal(layer.shared_expert.w_gate.weight, sg.weight)
    assert torch.equal(layer.shared_expert.w_up.weight, su.weight)
    assert torch.equal(layer.shared_expert.w_down.weight, sd.weight)
    assert layer.expert_params[0] is layer.w_up


def test_ep_is_rejected():
    with pytest.raises(NotImplementedError):
        fused_moe(*_inputs(), top_k=2, ep_group=object())
