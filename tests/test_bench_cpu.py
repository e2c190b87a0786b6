"""Host-side checks of the benchmark entry points (no GPU needed)."""

import json
import os
import subprocess
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_bench_configs_match_the_baseline_shapes():
    from bench_configs import CONFIGS
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        configs = json.load(f)["configs"]
    # configs[2..4] are C3, C4, C5 in the baseline's own order
    for name, text in zip(("c3", "c4", "c5"), configs[2:5]):
        c = CONFIGS[name]
        compact = text.replace(" ", "")
        for key, label in (("N", "N="), ("D", "D="), ("ffn", "ffn_dim="), ("E", "E="), ("k", "top_k=")):
            assert f"{label}{c[key]}" in compact, (name, key)
    assert CONFIGS["c3"]["bwd"] is False
    assert CONFIGS["c4"]["bwd"] and CONFIGS["c5"]["bwd"]
    assert CONFIGS["c4"]["zipf"] and not CONFIGS["c5"]["zipf"]


def test_zipf_bias_is_twice_the_log_of_normalised_zipf_weights():
    from bench_configs import zipf_bias
    E = 64
    b = zipf_bias(E)
    p = torch.exp(b.double() / 2)
    assert abs(p.sum().item() - 1.0) < 1e-6
    # the weights are r^-1.1 over the ranks 1..E, in some order
    expected = torch.arange(1, E + 1, dtype=torch.float64) ** -1.1
    expected /= expected.sum()
    assert torch.allclose(p.sort().values, expected.sort().values, rtol=1e-5)
    assert not torch.equal(p, p.sort(descending=True).values)  # permuted, not rank order
