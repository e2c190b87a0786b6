"""Step timing of fused_moe at the reference benchmark's other configurations.

    python bench_configs.py [--config c3|c4|c5|all] [--steps K] [--warmup W]

bench.py measures the headline configuration (C2); this runs the others on
one GPU, with synthetic inputs of the stated shapes and distributions, and
prints one JSON line per configuration:

* c3: Mixtral-shaped decode batch, forward only: N 64, D 4096, ffn 28672,
  E 8, k 2, weights ~ N(0, 0.02);
* c4: fine-grained, load-imbalanced layer, forward + backward: N 16384,
  D 2048, ffn 2816, E 64, k 8, gate ~ N(0, 0.02) plus a per-expert bias
  2·log(p) with p the normalised Zipf weights (s = 1.1) of a seeded
  permutation of the ranks, so the expert counts are skewed;
* c5: DeepSeek-V3-style layer, forward + backward: N 4096, D 7168, E 256,
  ffn 4096, k 8, weights ~ N(0, 0.006) (about 23 GB of expert weights).

A step is one fused_moe call (and its backward) with the inputs resident in
HBM; the parameter gradients are reset before each step, so no gradient
accumulation is timed.  `expert_tflops` counts the six expert GEMMs' useful
flops (routed rows only) per step.
"""

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

CONFIGS = {
    "c3": dict(N=64, D=4096, ffn=28672, E=8, k=2, std=0.02, bwd=False, zipf=False),
    "c4": dict(N=16384, D=2048, ffn=2816, E=64, k=8, std=0.02, bwd=True, zipf=True),
    "c5": dict(N=4096, D=7168, ffn=4096, E=256, k=8, std=0.006, bwd=True, zipf=False),
}


def zipf_bias(E, s=1.1, seed=4):
    """Per-expert logit bias 2·log(p_e), p the Zipf(s) weights of a seeded rank permutation."""
    ranks = torch.randperm(E, generator=torch.Generator().manual_seed(seed)).float() + 1.0
    pz = ranks ** -s
    return 2.0 * torch.log(pz / pz.sum())


def run(name, cfg, steps, warmup, instr_steps=3):
    import bench
    from flashfusedmoe_amd import fused_moe
    N, D, ffn, E, k, std = (cfg[key] for key in ("N", "D", "ffn", "E", "k", "std"))
    H = ffn // 2
    g = torch.Generator(device="cuda").manual_seed(1)

    def randn(shape, sd):
        return (torch.randn(shape, device="cuda", generator=g) * sd).to(torch.bfloat16)

    x, gate, wu, wd = randn((N, D), 1.0), randn((E, D), std), randn((E, ffn, D), std), randn((E, D, H), std)
    go = randn((N, D), 1.0) if cfg["bwd"] else None
    bias = zipf_bias(E).cuda() if cfg["zipf"] else None
    leaves = [t.requires_grad_(cfg["bwd"]) for t in (x, gate, wu, wd)]

    def step():
        if cfg["bwd"]:
            for t in leaves:
                t.grad = None
            out, _ = fused_moe(*leaves, top_k=k, expert_bias=bias, max_tokens_per_expert=N * k)
            out.backward(go)
        else:
            with torch.no_grad():
                fused_moe(*leaves, top_k=k, expert_bias=bias, max_tokens_per_expert=N * k)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / steps
    T = N * k
    flop = (2.0 * T * D * 2 * H + 2.0 * T * H * D) * (3 if cfg["bwd"] else 1)
    # in-step durations of every kernel (HIP events around each launch of a
    # few more steps), rated against the MFMA or HBM peak; nothing is
    # dropped here (max_tokens_per_expert = N*k), so every entry is a row
    in_step = bench.instrumented_steps(step, instr_steps)
    work = bench.algorithmic_work(cfg, T)
    if "gate_logits" in in_step:  # the route kernel reads the logits, not x and the gate
        work["route_fwd"] = (N * E * 2 + T * 12, "byte")
    kernels = bench.kernel_rates(in_step, work)
    # few rows per expert (C3's decode, C5's 128) make the expert GEMMs stream
    # their weights (or, for the wgrads, write them): rate each GEMM's operand
    # + output bytes against HBM as well
    for n, b in bench.algorithmic_bytes(cfg, T).items():
        if n.startswith("gemm_") and n in kernels:
            r = b / (kernels[n]["in_step_ms"] * 1e-3) / 1e9
            kernels[n]["weight_stream"] = {"bytes": int(b), "rate": round(r, 1), "unit": "GB/s",
                                           "frac": round(r / bench.PEAK_HBM_GBS, 4)}
    hbm = {n: dict(role=role, bound="hbm", achieved=kernels[n]["rate"], peak=bench.PEAK_HBM_GBS,
                   unit="GB/s", frac=kernels[n]["frac"], timing="in-step")
           for n, role in bench.HBM_ROLES.items() if n in kernels and "rate" in kernels[n]}
    print(json.dumps({
        "config": name, "pass": "fwd+bwd" if cfg["bwd"] else "fwd", "ms_per_step": round(ms, 4),
        "tokens_per_s": round(N / (ms * 1e-3), 1), "expert_tflops": round(flop / (ms * 1e-3) / 1e12, 2),
        "steps": steps, "warmup": warmup, "dtype": "bf16", "data": "synthetic",
        "shape": {key: cfg[key] for key in ("N", "D", "ffn", "E", "k")}, "wall_s_timed": round(wall, 3),
        "hbm_rooflines": hbm, "kernels": kernels,
    }), flush=True)
    del x, gate, wu, wd, go, leaves
    torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", choices=[*CONFIGS, "all"], default="all")
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("bench_configs needs a GPU (the fused MoE path has no CPU fallback)")
    names = list(CONFIGS) if args.config == "all" else [args.config]
    for name in names:
        run(name, CONFIGS[name], args.steps, args.warmup)


if __name__ == "__main__":
    main()
