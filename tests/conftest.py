"""Shared pytest setup.

``gpu`` marks tests that need a ROCm GPU (run with ``-m gpu`` on an MI355X);
everything else runs on the CPU.  The repository root is put on sys.path so
the tests can import both ``flashfusedmoe_amd`` and the test-only ``oracle``.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def make_inputs(N, D, ffn_dim, E, dtype, seed=0, gate_scale=0.01, device="cpu"):
    """Seeded inputs generated on the CPU in fp32, then cast and moved, so a
    CPU oracle and the GPU see identical bits."""
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, D, generator=g)
    gate = torch.randn(E, D, generator=g) * gate_scale
    w_up = torch.randn(E, ffn_dim, D, generator=g) * (2.0 / D) ** 0.5
    w_down = torch.randn(E, D, ffn_dim // 2, generator=g) * (2.0 / (ffn_dim // 2)) ** 0.5
    return tuple(t.to(dtype).to(device) for t in (x, gate, w_up, w_down))
