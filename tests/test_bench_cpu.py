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


def _pmc_csv(path, seq):
    """A counter_collection.csv of rocprofv3's layout for dispatches seq =
    [(kernel name, value)], one counter row per dispatch (the split of
    FETCH_SIZE over two rows of one dispatch is summed)."""
    import csv
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Correlation_Id", "Dispatch_Id", "Agent_Id", "Kernel_Name", "Counter_Name",
                    "Counter_Value"])
        for i, (name, v) in enumerate(seq, start=1):
            w.writerow([i, i, 1, name, "FETCH_SIZE", v / 2])
            w.writerow([i, i, 1, name, "FETCH_SIZE", v / 2])


def test_traffic_summary_splits_dispatches_by_flush(tmp_path):
    """traffic_mode's tail: calibration copy, then per kernel two
    (flush fill, kernel dispatches...) groups.  Earlier fills (setup) must
    not shift the split, a kernel of two dispatches is summed, and the
    scaled bytes use the calibration's factor."""
    import bench
    fill = "void at::native::vectorized_elementwise_kernel<16, at::native::FillFunctor<unsigned char>>"
    cal = "void at::native::vectorized_elementwise_kernel<4, at::native::AUnaryFunctor<float, float, float, at::native::binary_internal::MulFunctor<float>>>"
    seq = [(fill, 5.0), ("ffmoe::route_fwd_kernel", 7.0), ("uniform", 1.0), (cal, 131072.0)]
    for j, name in enumerate(bench.TRAFFIC_ORDER):
        for rep in range(2):
            seq.append((fill, 1.0))
            if name == "gate_grad":  # two kernels per launch
                seq += [("partial", 10.0 + rep), ("final", 1.0)]
            else:
                seq.append((name, 100.0 * (j + 1) + 2 * rep))
    f = tmp_path / "f.csv"
    _pmc_csv(f, seq)
    rows = bench.read_pmc_csv(str(f))
    per, cal_v, cal_name = bench.traffic_per_kernel(rows)
    assert cal_v == 131072.0 and "MulFunctor" in cal_name
    for j, name in enumerate(bench.TRAFFIC_ORDER):
        exp = 10.5 + 1.0 if name == "gate_grad" else 100.0 * (j + 1) + 1
        assert per[name] == exp, name
    # a missing calibration copy is refused, not misread
    bad = tmp_path / "bad.csv"
    _pmc_csv(bad, [s for s in seq if s[0] != cal])
    import pytest
    with pytest.raises(ValueError, match="calibration"):
        bench.traffic_per_kernel(bench.read_pmc_csv(str(bad)))
    # the written summary reads back through measured_traffic: FETCH scale x2
    out = tmp_path / "t.md"
    orig = bench.TRAFFIC_FILE
    bench.traffic_summary(str(f), str(f), str(out), ["cmd"])
    bench.TRAFFIC_FILE = str(out)
    try:
        t = bench.measured_traffic()
    finally:
        bench.TRAFFIC_FILE = orig
    assert t[bench.TRAFFIC_ORDER[0]] == int(round((101.0 * 2 + 101.0 * 2) * 1024))


def test_algorithmic_bytes_of_the_gemms_at_c2():
    import bench
    a = bench.algorithmic_bytes(bench.CFG, 16384)
    MiB = 1 << 20
    assert a["gemm_up_glu"] == 288 * MiB     # xs 32 + w_up 64 + up 128 + act 64
    assert a["gemm_down"] == 128 * MiB       # act 64 + w_down 32 + down 32
    assert a["gemm_up_down"] == a["gemm_up_glu"] + a["gemm_down"]
    assert a["gemm_dgrad_glu"] == 320 * MiB  # wgo 32 + w_down 32 + up 128 + gup 128
    assert a["gemm_dgrad"] == 224 * MiB
    assert a["gemm_wgrad_down"] == 128 * MiB
