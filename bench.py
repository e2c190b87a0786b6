"""Benchmark of the fused MoE layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Workload (configuration C2, the reference README's Quick Start layer):
fused_moe forward + backward, N = 8192 tokens (B=4, T=2048), D = 1024,
ffn_dim = 4096 (H = 2048), E = 8, top_k = 2, swiglu, softmax gating,
aux_loss_coeff = 0.01, z_loss_coeff = 1e-3, bf16.  Synthetic inputs from a
seeded CPU generator: x ~ N(0,1), weights ~ N(0, 1/fan_in), upstream grad
~ N(0,1).  A step is one forward + backward of the routed op with inputs
resident in HBM.  The shared expert of MoELayer is timed separately.

Prints ONE JSON line.  Besides the contract fields it carries:
  roofline      the dominant kernel's achieved rate vs MI355X peak, from HIP
                events around repeated launches of that kernel alone;
  kernels       the same measurement for every hot kernel;
  cpu_baseline  the reference's unfused PyTorch path (restated in
                oracle/unfused.py) timed on this host on a bounded sample.
"""

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E

CFG = dict(N=8192, D=1024, ffn=4096, E=8, k=2, activation="swiglu", gating="softmax",
           aux=0.01, z=1e-3)


def make_inputs(N, D, ffn, E, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, D, generator=g)
    gate = torch.randn(E, D, generator=g) * D ** -0.5
    wu = torch.randn(E, ffn, D, generator=g) * D ** -0.5
    wd = torch.randn(E, D, ffn // 2, generator=g) * (ffn // 2) ** -0.5
    go = torch.randn(N, D, generator=g)
    return x, gate, wu, wd, go


def time_events(fn, reps):
    """Average ms of fn() over reps launches, HIP events on torch's current
    stream (every ffmoe kernel is launched on that stream)."""
    fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "gemm_hbm_traffic_c2.md")


def measured_traffic():
    """HBM bytes per launch of each grouped GEMM at C2, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (calibrated against a copy of
    known size); {} when the summary is absent."""
    out = {}
    try:
        for line in open(TRAFFIC_FILE):
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes":
                out[parts[1]] = int(parts[2])
    except OSError:
        pass
    return out


def kernel_rates(c, x, gate, wu, wd, go, reps=20):
    """Times each hot kernel alone (launched through the C ABI) and returns
    {name: {ms, rate, unit, frac, work}} with algorithmic work per launch."""
    from flashfusedmoe_amd import _lib as L
    from flashfusedmoe_amd import ops
    N, D, E, k = c["N"], c["D"], c["E"], c["k"]
    H = c["ffn"] // 2
    T = N * k
    mt = (N * k + E - 1) // E
    mt += max(mt, k)
    (logits, idx, tw, lse, counts, off, til, stats, istats, ws, _aux, _z) = ops.route(
        x, gate, None, k, 0, mt, c["aux"], c["z"], False)
    out, tw2, row_of, xs, up, act, down = ops.experts_forward(
        x, wu, wd, idx, tw, counts, off, til, ws, k, 0, mt, False, True)
    rows = int(off[-1].item())
    st = L.stream_ptr()
    P = L.ptr
    dev = x.device
    wgo = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    gl = torch.empty(N, E, dtype=torch.bfloat16, device=dev)
    gup = torch.empty(T, 2 * H, dtype=torch.bfloat16, device=dev)
    ghb = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    dwd = torch.empty(E, D, H, dtype=torch.bfloat16, device=dev)
    dwu = torch.empty(E, 2 * H, D, dtype=torch.bfloat16, device=dev)
    dx = torch.empty(N, D, dtype=torch.bfloat16, device=dev)
    gpart = torch.empty(int(L.load().ffmoe_gate_grad_workspace_bytes(N, D, E)), dtype=torch.uint8,
                        device=dev)
    dgate = torch.empty(E, D, dtype=torch.bfloat16, device=dev)
    xs2 = torch.empty_like(xs)
    row2 = torch.empty_like(row_of)
    tw3 = tw.clone()
    gz = torch.ones((), device=dev)
    up_f = 2.0 * rows * D * 2 * H
    dn_f = 2.0 * rows * H * D
    b = 2  # bytes per bf16
    tr = L.gemm_tile_rows(T, E)
    gws = P(L.gemm_workspace(xs.device, st))
    launches = {
        "gemm_up_glu": (lambda: L.call("ffmoe_gemm_up_glu", P(xs), P(wu), P(off), P(til), tr, E, T, D,
                                       H, 0, P(up), P(act), gws, st), up_f, "flop"),
        "gemm_down": (lambda: L.call("ffmoe_gemm_down", P(act), P(wd), P(off), P(til), tr, E, T, H, D,
                                     P(down), gws, st), dn_f, "flop"),
        "gemm_dgrad_glu": (lambda: L.call("ffmoe_gemm_dgrad_glu", P(wgo), P(wd), P(up), P(off), P(til),
                                          tr, E, T, D, H, 0, P(gup), gws, st), dn_f, "flop"),
        "gemm_dgrad": (lambda: L.call("ffmoe_gemm_dgrad", P(gup), P(wu), P(off), P(til), tr, E, T, H,
                                      D, P(ghb), gws, st), up_f, "flop"),
        "gemm_wgrad_down": (lambda: L.call("ffmoe_gemm_wgrad", P(wgo), P(act), P(off), E, D, H, P(dwd),
                                           st), dn_f, "flop"),
        "gemm_wgrad_up": (lambda: L.call("ffmoe_gemm_wgrad", P(gup), P(xs), P(off), E, 2 * H, D, P(dwu),
                                         st), up_f, "flop"),
        # bandwidth kernels: algorithmic bytes (read token rows once, write k rows)
        "route_fwd": (lambda: L.call("ffmoe_route_fwd", P(x), P(gate), None, None, N, D, E, k, 0, 0,
                                     P(logits), P(idx), P(tw3), P(lse), P(ws), st),
                      N * D * b + E * D * b + N * k * 12 + N * E * b, "byte"),
        "permute": (lambda: L.call("ffmoe_permute", P(x), P(idx), P(tw3), P(off), P(counts), N, D, E, k,
                                   mt, 0, P(ws), P(xs2), P(row2), st),
                    N * D * b + rows * D * b + N * k * 12, "byte"),
        "combine": (lambda: L.call("ffmoe_combine", P(down), P(row_of), P(tw), None, N, D, k, P(out),
                                   st), rows * D * b + N * D * b + N * k * 8, "byte"),
        "route_bwd": (lambda: L.call("ffmoe_route_bwd", P(go), P(down), P(row_of), P(idx), P(tw),
                                     P(logits), P(lse), P(counts), None, P(gz), c["aux"], c["z"], N, D,
                                     E, k, 0, 0, P(wgo), P(gl), None, st),
                      N * D * b + 2 * rows * D * b + N * E * 2 * b + N * k * 16, "byte"),
        "dx_reduce": (lambda: L.call("ffmoe_dx_reduce", P(ghb), P(row_of), P(gl), P(gate), N, D, E, k,
                                     P(dx), st),
                      rows * D * b + N * D * b + N * E * b + E * D * b + N * k * 4, "byte"),
        "gate_grad": (lambda: L.call("ffmoe_gate_grad", P(gl), P(x), N, D, E, P(gpart), P(dgate), st),
                      N * D * b + N * E * b + E * D * b, "byte"),
    }
    res = {}
    for name, (fn, work, kind) in launches.items():
        ms = time_events(fn, reps)
        if kind == "flop":
            rate = work / (ms * 1e-3) / 1e12
            res[name] = dict(ms=ms, rate=rate, unit="TFLOP/s", frac=rate / PEAK_BF16_TFLOPS,
                             work=work, bound="mfma")
        else:
            rate = work / (ms * 1e-3) / 1e9
            res[name] = dict(ms=ms, rate=rate, unit="GB/s", frac=rate / PEAK_HBM_GBS, work=work,
                             bound="hbm")
    return res


def cpu_baseline(c, sample_tokens):
    """The reference's unfused CPU path (oracle/unfused.py restates
    tests/conftest.py:58-137) forward + backward in fp32 on a bounded sample
    of the workload: sample_tokens tokens, the full expert weights."""
    from oracle.unfused import unfused_moe
    threads = torch.get_num_threads()
    x, gate, wu, wd, go = make_inputs(sample_tokens, c["D"], c["ffn"], c["E"], seed=1)
    leaves = [t.clone().requires_grad_(True) for t in (x, gate, wu, wd)]

    def step():
        for t in leaves:
            t.grad = None
        out, _, _, losses = unfused_moe(*leaves, c["k"], activation=c["activation"],
                                        aux_loss_coeff=c["aux"], z_loss_coeff=c["z"])
        torch.autograd.backward([out, losses["aux_loss"], losses["z_loss"]],
                                [go, torch.ones(()), torch.ones(())])

    step()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[1]
    return dict(value=sample_tokens / med, unit="tokens/s", cores=threads, kind="port",
                sample=f"{sample_tokens} tokens of the C2 layer (D1024 ffn4096 E8 k2 swiglu, aux+z), "
                       f"fp32 fwd+bwd, median of 3 after 1 warm-up ({med:.2f} s/run)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-tokens", type=int, default=8192)
    ap.add_argument("--no-kernels", action="store_true", help="skip per-kernel timing")
    ap.add_argument("--no-layer", action="store_true", help="skip the MoELayer (shared expert) timing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    from flashfusedmoe_amd import MoELayer, fused_moe
    from flashfusedmoe_amd import _lib
    _lib.load()
    c = CFG
    dev = torch.device("cuda:0")
    x, gate, wu, wd, go = (t.to(torch.bfloat16).to(dev) for t in make_inputs(c["N"], c["D"], c["ffn"], c["E"]))
    params = [t.requires_grad_(True) for t in (x, gate, wu, wd)]
    one = torch.ones((), device=dev)

    def step():
        for p in params:
            p.grad = None
        out, losses = fused_moe(*params, top_k=c["k"], activation=c["activation"], gating=c["gating"],
                                aux_loss_coeff=c["aux"], z_loss_coeff=c["z"], allow_dropped_tokens=True)
        torch.autograd.backward([out, losses["z_loss"]], [go, one])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / args.steps
    tokens_per_s = c["N"] / (ms * 1e-3)
    H = c["ffn"] // 2
    T = c["N"] * c["k"]
    expert_flop = 3 * (2.0 * T * c["D"] * 2 * H + 2.0 * T * H * c["D"])
    step_mfma_frac = expert_flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS

    # MoELayer with the shared expert (config C2 as the reference's README quotes it)
    torch.manual_seed(0)
    layer = MoELayer(c["D"], c["ffn"], c["E"], top_k=c["k"], num_shared_experts=1,
                     aux_loss_coeff=c["aux"], z_loss_coeff=c["z"]).to(dev, torch.bfloat16)
    xl = x.detach().clone().requires_grad_(True)

    def layer_step():
        layer.zero_grad(set_to_none=True)
        xl.grad = None
        out, losses = layer(xl)
        torch.autograd.backward([out, losses["z_loss"]], [go, one])

    layer_ms = None if args.no_layer else time_events(layer_step, max(5, args.steps // 2))

    kernels = {} if args.no_kernels else kernel_rates(
        c, *(p.detach() for p in params), go)
    gemms = {n: v for n, v in kernels.items() if v["bound"] == "mfma"}
    dom_name = max(gemms, key=lambda n: gemms[n]["ms"]) if gemms else None
    roofline = None
    if dom_name:
        d = kernels[dom_name]
        roofline = dict(kernel=dom_name, bound="mfma", achieved=round(d["rate"], 2),
                        peak=PEAK_BF16_TFLOPS, unit="TFLOP/s", frac=round(d["frac"], 4),
                        traffic=measured_traffic().get(dom_name))

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(c, args.cpu_tokens)

    line = {
        "metric": "fused_moe fwd+bwd tokens/s (D1024 E8 k2 bf16); % bf16 MFMA peak; HBM GB/s",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs, N(0,1/fan_in) weights)",
        "config": {"workload": "C2: fused_moe fwd+bwd N8192 D1024 ffn4096 E8 k2 swiglu softmax "
                               "aux0.01 z1e-3 allow_dropped_tokens=True",
                   "global_batch": c["N"], "parallelism": "none (1 GPU)"},
        "expert_gemm_mfma_frac_of_step": round(step_mfma_frac, 4),
        "moelayer_shared_expert": None if layer_ms is None else {
            "ms_per_step": round(layer_ms, 4), "tokens_per_s": round(c["N"] / (layer_ms * 1e-3), 1)},
        "roofline": roofline,
        "kernels": {n: {"ms": round(v["ms"], 5), "rate": round(v["rate"], 2), "unit": v["unit"],
                        "frac": round(v["frac"], 4)} for n, v in kernels.items()},
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
