"""Benchmark of the fused MoE layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--traffic]

Workload (configuration C2, the reference README's Quick Start layer):
fused_moe forward + backward, N = 8192 tokens (B=4, T=2048), D = 1024,
ffn_dim = 4096 (H = 2048), E = 8, top_k = 2, swiglu, softmax gating,
aux_loss_coeff = 0.01, z_loss_coeff = 1e-3, bf16.  Synthetic inputs from a
seeded CPU generator: x ~ N(0,1), weights ~ N(0, 1/fan_in), upstream grad
~ N(0,1).  A step is one forward + backward of the routed op with inputs
resident in HBM.  The shared expert of MoELayer is timed separately.

Prints ONE JSON line.  Besides the contract fields it carries:
  roofline       the dominant kernel (the grouped GEMM with the longest
                 in-step time): algorithmic flops / its average in-step
                 launch duration (HIP events on the launch stream around
                 every launch of a run of instrumented steps), vs the bf16
                 MFMA peak;
  hbm_rooflines  the same for the bandwidth kernels (scatter = permute,
                 combine, weighted scatter = route_bwd, gather = dX reduce,
                 route), in-step and cold (launched alone after a 1 GiB
                 write that evicts the L2 and the MALL), vs the HBM peak;
  kernels        in-step duration and rate of every hot kernel;
  cpu_baseline   the reference's unfused PyTorch path (restated in
                 oracle/unfused.py) timed on this host on a bounded sample.

``--traffic`` runs each hot kernel twice, after a 256 MiB calibration copy
and with a 1 GiB flush before every launch, and prints nothing else: the
driver of the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes.
``--traffic-summary FETCH_CSV WRITE_CSV`` (no GPU) turns the two passes'
counter CSVs into profiles/hbm_traffic_c2.md, which bench.py reads back for
the `traffic` fields.
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

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_c2.md")

# entry point -> kernel name(s) in the order a step calls it
STEP_KERNELS = {
    "ffmoe_route_fwd_ex": ["route_fwd"],
    "ffmoe_route_scan": ["route_scan"],
    "ffmoe_permute": ["permute"],
    # up + GLU and down: one persistent launch (C2), or the two GEMMs where
    # the fused schedule does not apply (timed together then)
    "ffmoe_gemm_up_down": ["gemm_up_down"],
    "ffmoe_combine": ["combine", "dx_combine"],  # E > 32: the backward's dX gather is a combine
    "ffmoe_gate_logits": ["gate_logits"],
    "ffmoe_gate_dx": ["gate_dx"],
    "ffmoe_route_bwd_ex": ["route_bwd"],
    "ffmoe_gemm_wgrad": ["gemm_wgrad_down"],
    "ffmoe_gemm_dgrad_glu": ["gemm_dgrad_glu"],
    # dX's GEMM and the up-side weight gradient: one persistent launch, or
    # the two GEMMs where the fused schedule does not apply (timed together)
    "ffmoe_gemm_dgrad_wgrad": ["gemm_dgrad_wgrad"],
    "ffmoe_dx_reduce": ["dx_reduce"],
    "ffmoe_gate_grad": ["gate_grad"],
}
# what each bandwidth kernel is in the reference's vocabulary
HBM_ROLES = {"permute": "scatter", "combine": "combine", "route_bwd": "weighted scatter",
             "dx_reduce": "gather", "dx_combine": "gather", "route_fwd": "route"}


def kernel_rates(in_step, work):
    """{kernel: {in_step_ms, rate, unit, frac}} from in-step durations and
    algorithmic work (flop: vs the bf16 MFMA peak; byte: vs HBM)."""
    kernels = {}
    for name, ms_in in sorted(in_step.items()):
        w, kind = work.get(name, (None, "byte"))
        ent = {"in_step_ms": round(ms_in, 5)}
        if w is not None:
            if kind == "flop":
                rate = w / (ms_in * 1e-3) / 1e12
                ent.update(rate=round(rate, 2), unit="TFLOP/s", frac=round(rate / PEAK_BF16_TFLOPS, 4))
            else:
                rate = w / (ms_in * 1e-3) / 1e9
                ent.update(rate=round(rate, 1), unit="GB/s", frac=round(rate / PEAK_HBM_GBS, 4))
        kernels[name] = ent
    return kernels


def make_inputs(N, D, ffn, E, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, D, generator=g)
    gate = torch.randn(E, D, generator=g) * D ** -0.5
    wu = torch.randn(E, ffn, D, generator=g) * D ** -0.5
    wd = torch.randn(E, D, ffn // 2, generator=g) * (ffn // 2) ** -0.5
    go = torch.randn(N, D, generator=g)
    return x, gate, wu, wd, go


def algorithmic_work(c, rows):
    """Algorithmic flops (GEMMs) or bytes (bandwidth kernels) of one launch
    at configuration c with `rows` routed rows (N*k at C2: nothing dropped).
    Padding is never counted."""
    N, D, E, k = c["N"], c["D"], c["E"], c["k"]
    H = c["ffn"] // 2
    T = N * k
    b = 2  # bytes per bf16
    up_f = 2.0 * rows * D * 2 * H
    dn_f = 2.0 * rows * H * D
    return {
        "gemm_up_glu": (up_f, "flop"), "gemm_down": (dn_f, "flop"), "gemm_up_down": (up_f + dn_f, "flop"),
        "gemm_dgrad_glu": (dn_f, "flop"), "gemm_dgrad": (up_f, "flop"),
        "gemm_wgrad_down": (dn_f, "flop"), "gemm_wgrad_up": (up_f, "flop"),
        "gemm_dgrad_wgrad": (2 * up_f, "flop"),
        # x, gate read once; idx (8) + w (4) per entry and the bf16 logits written
        "route_fwd": (N * D * b + E * D * b + T * 12 + N * E * b, "byte"),
        "route_scan": (None, "byte"),
        # scatter: token rows read once, routed rows written, idx / row_of
        "permute": (N * D * b + rows * D * b + T * 12, "byte"),
        # combine: routed rows read, token rows written, row_of + weight per entry
        "combine": (rows * D * b + N * D * b + T * 12, "byte"),
        # weighted scatter + routing-weight grad: go read, down rows read for
        # the dots, wgo rows written, logits read and grad_logits written
        "route_bwd": (N * D * b + 2 * rows * D * b + 2 * N * E * b + T * 16, "byte"),
        # dX gather: ghb rows read, dx written, gl and gate for the gate term
        "dx_reduce": (rows * D * b + N * D * b + N * E * b + E * D * b + T * 4, "byte"),
        "gate_grad": (N * D * b + N * E * b + E * D * b, "byte"),
        # E > 32: dX as a combine of ghb rows plus the gl.gate addend
        "dx_combine": (rows * D * b + 2 * N * D * b + T * 4, "byte"),
        "gate_logits": (2.0 * N * D * E, "flop"),
        "gate_dx": (2.0 * N * E * D, "flop"),
    }


def measured_traffic():
    """HBM bytes per launch of each hot kernel at C2, from the committed
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


class StepRecorder:
    """Records a HIP event pair around every libffmoe launch (on torch's
    current stream, where every ffmoe kernel is enqueued) and averages the
    durations per kernel name."""

    def __init__(self):
        self.pairs = []   # (kernel name, start event, end event)
        self.seen = {}
        self.open = None

    def new_step(self):
        self.seen = {}

    def __call__(self, name, phase):
        # the *_shared GEMM entry points are the same launches (no dense group here)
        name = name.removesuffix("_shared")
        names = STEP_KERNELS.get(name)
        if names is None:
            return
        if phase == 0:
            i = self.seen.get(name, 0)
            self.seen[name] = i + 1
            label = names[min(i, len(names) - 1)]
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self.open = (label, ev)
        else:
            label, ev0 = self.open
            ev1 = torch.cuda.Event(enable_timing=True)
            ev1.record()
            self.pairs.append((label, ev0, ev1))
            self.open = None

    def averages_ms(self):
        torch.cuda.synchronize()
        acc = {}
        for label, e0, e1 in self.pairs:
            acc.setdefault(label, []).append(e0.elapsed_time(e1))
        return {k: sum(v) / len(v) for k, v in acc.items()}


def instrumented_steps(step, n):
    """Runs n steps with every launch bracketed by HIP events; returns the
    average in-step duration (ms) of each kernel."""
    from flashfusedmoe_amd import _lib as L
    rec = StepRecorder()
    L.call_hook = rec
    try:
        for _ in range(n):
            rec.new_step()
            step()
    finally:
        L.call_hook = None
    return rec.averages_ms()


def kernel_launches(c, x, gate, wu, wd, go):
    """Standalone launches of every hot kernel of the C2 step through the C
    ABI, on inputs from one real forward: {name: fn}, plus the routed row
    count."""
    from flashfusedmoe_amd import _lib as L
    from flashfusedmoe_amd import ops
    N, D, E, k = c["N"], c["D"], c["E"], c["k"]
    H = c["ffn"] // 2
    T = N * k
    mt = (N * k + E - 1) // E
    mt += max(mt, k)
    (logits, idx, tw, lse, counts, off, til, stats, istats, ws, _aux, _z) = ops.route(
        x, gate, None, k, 0, mt, c["aux"], c["z"], False)
    out, tw2, row_of, xs, up, act, down, _, _ = ops.experts_forward(
        x, wu, wd, idx, tw, counts, off, til, ws, k, 0, mt, False, True)
    rows = int(off[-1].item())
    st = L.stream_ptr()
    P = L.ptr
    dev = x.device
    bf = torch.bfloat16
    wgo = torch.empty(T, D, dtype=bf, device=dev)
    gl = torch.empty(N, E, dtype=bf, device=dev)
    gup = torch.empty(T, 2 * H, dtype=bf, device=dev)
    ghb = torch.empty(T, D, dtype=bf, device=dev)
    dwd = torch.empty(E, D, H, dtype=bf, device=dev)
    dwu = torch.empty(E, 2 * H, D, dtype=bf, device=dev)
    dx = torch.empty(N, D, dtype=bf, device=dev)
    gpart = torch.empty(int(L.load().ffmoe_gate_grad_workspace_bytes(N, D, E)), dtype=torch.uint8,
                        device=dev)
    dgate = torch.empty(E, D, dtype=bf, device=dev)
    xs2 = torch.empty_like(xs)
    row2 = torch.empty_like(row_of)
    tw3 = tw.clone()
    gz = torch.ones((), device=dev)
    tr = L.gemm_tile_rows(T, E)
    gws = P(L.gemm_workspace(xs.device, st))
    # realistic operands for the backward GEMMs: one routing backward first
    L.call("ffmoe_route_bwd", P(go), P(down), P(row_of), P(idx), P(tw), P(logits), P(lse), P(counts),
           None, P(gz), c["aux"], c["z"], N, D, E, k, 0, 0, P(wgo), P(gl), None, st)
    L.call("ffmoe_gemm_dgrad_glu", P(wgo), P(wd), P(up), P(off), P(til), tr, E, T, D, H, 0, P(gup),
           gws, st)
    L.call("ffmoe_gemm_dgrad", P(gup), P(wu), P(off), P(til), tr, E, T, H, D, P(ghb), gws, st)
    fns = {
        "gemm_up_down": lambda: L.call("ffmoe_gemm_up_down_shared", P(xs), P(wu), P(wd), P(off), P(til), tr,
                                       E, T, D, H, 0, P(up), P(act), P(down), None, None, gws, st),
        "gemm_dgrad_glu": lambda: L.call("ffmoe_gemm_dgrad_glu", P(wgo), P(wd), P(up), P(off), P(til),
                                         tr, E, T, D, H, 0, P(gup), gws, st),
        "gemm_dgrad_wgrad": lambda: L.call("ffmoe_gemm_dgrad_wgrad_shared", P(gup), P(wu), P(xs), P(off),
                                           P(til), tr, E, T, H, D, P(ghb), P(dwu), None, None, gws, st),
        "gemm_wgrad_down": lambda: L.call("ffmoe_gemm_wgrad", P(wgo), P(act), P(off), E, D, H, P(dwd),
                                          st),
        "route_fwd": lambda: L.call("ffmoe_route_fwd", P(x), P(gate), None, None, N, D, E, k, 0, 0,
                                    P(logits), P(idx), P(tw3), P(lse), P(ws), st),
        "permute": lambda: L.call("ffmoe_permute", P(x), P(idx), P(tw3), P(off), P(counts), N, D, E, k,
                                  mt, 0, P(ws), P(xs2), P(row2), st),
        "combine": lambda: L.call("ffmoe_combine", P(down), P(row_of), P(tw), None, N, D, k, P(out),
                                  st),
        "route_bwd": lambda: L.call("ffmoe_route_bwd", P(go), P(down), P(row_of), P(idx), P(tw),
                                    P(logits), P(lse), P(counts), None, P(gz), c["aux"], c["z"], N, D,
                                    E, k, 0, 0, P(wgo), P(gl), None, st),
        "dx_reduce": lambda: L.call("ffmoe_dx_reduce", P(ghb), P(row_of), P(gl), P(gate), N, D, E, k,
                                    P(dx), st),
        "gate_grad": lambda: L.call("ffmoe_gate_grad", P(gl), P(x), N, D, E, P(gpart), P(dgate), st),
    }
    keep = (logits, idx, tw, lse, counts, off, til, ws, out, row_of, xs, up, act, down, wgo, gl, gup,
            ghb, dwd, dwu, dx, gpart, dgate, xs2, row2, tw3, gz)
    return fns, rows, keep


def cold_launch_ms(fn, flush, reps):
    """Average duration (ms) of fn() launched alone after a write of `flush`
    (1 GiB: evicts the 4 MiB L2s and the 256 MiB MALL), HIP events on the
    launch stream around the kernel only."""
    fn()
    torch.cuda.synchronize()
    pairs = []
    for _ in range(reps):
        flush.zero_()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        pairs.append((e0, e1))
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in pairs) / reps


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(c, sample_tokens, runs=7):
    """The reference's unfused CPU path (oracle/unfused.py restates
    tests/conftest.py:58-137) forward + backward in fp32 on a bounded sample
    of the workload: sample_tokens tokens, the full expert weights; median
    of `runs` after one warm-up.  Threads: every core this process may use
    (os.cpu_count(), capped by OMP_NUM_THREADS where the host sets the
    process's CPU share)."""
    from oracle.unfused import unfused_moe
    ncpu = os.cpu_count() or 1
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(ncpu, cap) if cap > 0 else ncpu
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
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
        for _ in range(runs):
            t0 = time.perf_counter()
            step()
            times.append(time.perf_counter() - t0)
        used = torch.get_num_threads()
    finally:
        torch.set_num_threads(prev)
    times.sort()
    med = times[len(times) // 2]
    return dict(value=sample_tokens / med, unit="tokens/s", cores=used, cpu_count=ncpu,
                torch_threads=used, cpu_model=cpu_model(), kind="port",
                sample=f"{sample_tokens} tokens of the C2 layer (D1024 ffn4096 E8 k2 swiglu, aux+z), "
                       f"fp32 fwd+bwd, median of {runs} after 1 warm-up ({med:.2f} s/run, "
                       f"{sum(times):.1f} s timed)")


# the order traffic_mode launches the hot kernels in (each twice, after a flush)
TRAFFIC_ORDER = ["gemm_up_down", "gemm_dgrad_glu", "gemm_dgrad_wgrad", "gemm_wgrad_down",
                 "route_fwd", "permute", "combine", "route_bwd", "dx_reduce",
                 "gate_grad"]
CAL_KIB = 256 * 1024  # the calibration copy reads and writes 256 MiB


def traffic_mode(c, x, gate, wu, wd, go):
    """Each hot kernel twice, after a 256 MiB calibration copy, with a 1 GiB
    flush before every launch (the rocprofv3 --pmc driver)."""
    fns, _, keep = kernel_launches(c, x, gate, wu, wd, go)
    assert sorted(fns) == sorted(TRAFFIC_ORDER)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=x.device)
    src = torch.empty(CAL_KIB * 256, dtype=torch.float32, device=x.device).uniform_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.mul(src, 1.0, out=dst)  # calibration: a plain elementwise copy kernel
    torch.cuda.synchronize()
    del src, dst
    for name in TRAFFIC_ORDER:
        for _ in range(2):
            flush.zero_()
            fns[name]()
        torch.cuda.synchronize()
        print(f"traffic: {name} launched twice", flush=True)
    del keep
    print("traffic done", flush=True)


def read_pmc_csv(path):
    """[(dispatch id, kernel name, value)] in dispatch order from a rocprofv3
    --pmc counter_collection.csv holding one counter."""
    import csv
    acc = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            d = int(r["Dispatch_Id"])
            name, v = acc.get(d, (r["Kernel_Name"], 0.0))
            acc[d] = (name, v + float(r["Counter_Value"]))
    return [(d, *acc[d]) for d in sorted(acc)]


def traffic_per_kernel(rows):
    """Splits traffic_mode's dispatches (the tail of the run): the last
    2*len(TRAFFIC_ORDER) flush fills each open one launch of the next kernel
    in TRAFFIC_ORDER; the dispatch before the first of them is the
    calibration copy.  Returns ({kernel: mean counter over its 2 launches},
    calibration counter, calibration kernel name)."""
    fills = [i for i, r in enumerate(rows) if "FillFunctor" in r[1]]
    n = 2 * len(TRAFFIC_ORDER)
    if len(fills) < n:
        raise ValueError(f"expected at least {n} flush fills, found {len(fills)}")
    loop = fills[-n:]
    cal = rows[loop[0] - 1]
    if "FillFunctor" in cal[1] or "Mul" not in cal[1]:
        raise ValueError(f"the dispatch before the first flush is not the calibration copy: {cal[1]}")
    bounds = loop + [len(rows)]
    per = {}
    for j, name in enumerate(TRAFFIC_ORDER):
        vals = []
        for l in (2 * j, 2 * j + 1):
            seg = rows[bounds[l] + 1:bounds[l + 1]]
            if not seg:
                raise ValueError(f"no dispatch after flush {l} ({name})")
            vals.append(sum(r[2] for r in seg))
        per[name] = sum(vals) / 2
    return per, cal[2], cal[1]


def algorithmic_bytes(c, rows):
    """Operand + output bytes of one launch of each grouped GEMM (every
    operand read once, every output written once) and the bandwidth
    kernels' algorithmic bytes."""
    N, D, E = c["N"], c["D"], c["E"]
    H = c["ffn"] // 2
    b = 2
    out = {
        "gemm_up_glu": rows * D * b + E * 2 * H * D * b + rows * 2 * H * b + rows * H * b,
        "gemm_down": rows * H * b + E * D * H * b + rows * D * b,
        # the two above: act written once and read back once
        "gemm_up_down": (rows * D * b + E * 2 * H * D * b + rows * 2 * H * b + rows * H * b
                         + rows * H * b + E * D * H * b + rows * D * b),
        "gemm_dgrad_glu": rows * D * b + E * D * H * b + 2 * rows * 2 * H * b,
        "gemm_dgrad": rows * 2 * H * b + E * 2 * H * D * b + rows * D * b,
        "gemm_wgrad_down": rows * D * b + rows * H * b + E * D * H * b,
        "gemm_wgrad_up": rows * 2 * H * b + rows * D * b + E * 2 * H * D * b,
    }
    # the two above: gup read by both
    out["gemm_dgrad_wgrad"] = out["gemm_dgrad"] + out["gemm_wgrad_up"]
    for name, (w, kind) in algorithmic_work(c, rows).items():
        if kind == "byte" and w is not None:
            out[name] = int(w)
    return out


def traffic_summary(fetch_csv, write_csv, out_path, commands):
    """Writes the FETCH_SIZE / WRITE_SIZE summary (markdown, with the
    machine-readable traffic_bytes lines measured_traffic reads)."""
    fetch, cal_f, cal_name = traffic_per_kernel(read_pmc_csv(fetch_csv))
    write, cal_w, _ = traffic_per_kernel(read_pmc_csv(write_csv))
    sf, sw = CAL_KIB / cal_f, CAL_KIB / cal_w
    c = CFG
    alg = algorithmic_bytes(c, c["N"] * c["k"])
    lines = [
        "# HBM traffic per launch of the hot kernels (C2: N8192 D1024 ffn4096 E8 k2, all rows routed)",
        "",
        "Commands (from the repository root on one MI355X; two passes, one counter each; then the",
        "summary is written from the two counter_collection.csv files):",
        "",
        "```",
        *commands,
        "```",
        "",
        f"Calibration: `{cal_name[:90]}` copies 256 MiB (reads 262144 KiB, writes 262144 KiB).",
        f"FETCH_SIZE reads {cal_f:.0f} KiB for it (scale x{sf:.3f}), WRITE_SIZE {cal_w:.0f} KiB "
        f"(scale x{sw:.3f}).",
        "Every kernel runs twice, each launch after a 1 GiB write that evicts the L2s and the MALL;",
        "the table averages the two launches.  FETCH_SIZE counts the L2's requests to the memory",
        "fabric, so a MALL hit inside one launch still counts as traffic.",
        "",
        "| Kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes (scaled) | algorithmic bytes | ratio |",
        "|---|---:|---:|---:|---:|---:|",
    ]
    mach = []
    for name in TRAFFIC_ORDER:
        tb = int(round((fetch[name] * sf + write[name] * sw) * 1024))
        a = alg.get(name)
        ratio = f"{tb / a:.2f}" if a else "-"
        lines.append(f"| {name} | {fetch[name]:.0f} | {write[name]:.0f} | {tb} | {a if a else '-'} | {ratio} |")
        mach.append(f"traffic_bytes {name} {tb}")
    low = [(n, (fetch[n] * sf + write[n] * sw) * 1024 / alg[n]) for n in TRAFFIC_ORDER if alg.get(n)]
    low = [(n, r) for n, r in low if r < 0.9]
    if low:
        lines += ["", "Below the algorithmic bytes (the counters miss part of what these kernels must move,",
                  "so their figure is a lower bound): " + ", ".join(f"{n} ({r:.2f})" for n, r in low) + "."]
    lines += ["", "Machine-readable (read by bench.py for `traffic`):", "", "```", *mach, "```", ""]
    with open(out_path, "w") as f:
        f.write("\n".join(lines))


def gemm_step_order(symbols, fwd_only):
    """The GEMM roles of one step's grouped-GEMM dispatches (kernel symbols
    in launch order): the forward's up + down as one fused launch or two,
    the backward's up-side wgrad and dgrad as one fused launch or two."""
    fused_fwd = bool(symbols) and "updown" in symbols[0]
    order = ["gemm_up_down"] if fused_fwd else ["gemm_up_glu", "gemm_down"]
    if fwd_only:
        return order
    order += ["gemm_wgrad_down", "gemm_dgrad_glu"]
    if len(symbols) > len(order) and "gemm_dw" in symbols[len(order)]:
        return order + ["gemm_dgrad_wgrad"]
    return order + ["gemm_wgrad_up", "gemm_dgrad"]


def stats_summary(prof_dir, bench_log, out_path, title, command):
    """Writes a markdown summary of a rocprofv3 --kernel-trace --stats run of
    bench.py: the kernel table, which kernel symbol runs each GEMM of the
    step (read from the trace: the step's first GEMM dispatches in launch
    order), and the dominant GEMM's rocprof average next to bench.py's
    in-step HIP-event average."""
    import csv
    import glob
    stats_csv = glob.glob(os.path.join(prof_dir, "*kernel_stats.csv"))[0]
    trace_csv = glob.glob(os.path.join(prof_dir, "*kernel_trace.csv"))[0]
    with open(stats_csv, newline="") as f:
        stats = list(csv.DictReader(f))
    with open(trace_csv, newline="") as f:
        trace = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    line = None
    for ln in open(bench_log):
        if ln.startswith("{"):
            line = json.loads(ln)
    # the grouped GEMMs only (not the dense gate GEMMs or their split-K reduce)
    gemm = [r["Kernel_Name"] for r in trace
            if "ffmoe::gemm_" in r["Kernel_Name"] and "dense" not in r["Kernel_Name"]]
    order = gemm_step_order(gemm, (line or {}).get("pass") == "fwd")
    role_sym = dict(zip(order, gemm[:len(order)]))
    total = sum(float(r["TotalDurationNs"]) for r in stats)
    prefix = "rocprofv3 kernel statistics: "
    while title.startswith(prefix):  # a title taken from an earlier summary's header
        title = title[len(prefix):]
    out = [f"# {prefix}{title}", "",
           "Command (from the repository root on one MI355X):", "", "```", command, "```", "",
           f"Total kernel time: {total / 1e6:.3f} ms over the whole run.", "",
           "| Kernel | Calls | Avg (us) | Min (us) | Max (us) | % of kernel time |",
           "|---|---:|---:|---:|---:|---:|"]
    for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"]))[:28]:
        out.append(f"| `{r['Name'][:110]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                   f"{float(r['Percentage']):.2f} |")
    out += ["", "Kernel symbol of each grouped GEMM of the step (the first step's GEMM dispatches):", ""]
    for role in order:
        sym = role_sym.get(role, "?")
        durs = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in trace
                if r["Kernel_Name"] == sym]
        shared = [k for k, v in role_sym.items() if v == sym and k != role]
        note = f" (same symbol as {', '.join(shared)})" if shared else ""
        avg = sum(durs) / len(durs) if durs else float("nan")
        out.append(f"* {role}: `{sym[:100]}`, {len(durs)} launches, avg {avg:.2f} us{note}")
    if line is not None and line.get("roofline"):
        rf = line["roofline"]
        dom = rf["kernel"]
        sym = role_sym.get(dom)
        st = next((r for r in stats if r["Name"] == sym), None)
        out += ["", f"Dominant kernel (`roofline` of the bench line printed by this run): `{dom}`.",
                f"bench.py's in-step HIP events: {rf['avg_launch_ms'] * 1e3:.2f} us per launch "
                f"({rf['achieved']} TFLOP/s, {rf['frac'] * 100:.1f}% of the bf16 MFMA peak)."]
        if st is not None:
            out.append(f"rocprofv3's average over the {st['Calls']} launches of its symbol in this run: "
                       f"{float(st['AverageNs']) / 1e3:.2f} us.")
        out.append(f"Step time of this run: {line['ms_per_step']} ms ({line['value']} tokens/s).")
    elif line is not None:
        out += ["", f"Step time of this run: {line['ms_per_step']} ms ({line.get('tokens_per_s')} tokens/s, "
                    f"{line.get('expert_tflops')} TFLOP/s of expert GEMMs)."]
        if line.get("kernels"):
            out += ["", "In-step durations from the same run (HIP events around each launch):", "",
                    "| Kernel | in-step ms | rate |", "|---|---:|---:|"]
            for n, k in line["kernels"].items():
                rate = f"{k['rate']} {k['unit']} ({k['frac'] * 100:.1f}%)" if "rate" in k else "-"
                if "weight_stream" in k:
                    w = k["weight_stream"]
                    rate += f"; operand + output bytes at {w['rate']} GB/s ({w['frac'] * 100:.1f}% of HBM)"
                out.append(f"| {n} | {k['in_step_ms']} | {rate} |")
    out.append("")
    with open(out_path, "w") as f:
        f.write("\n".join(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-tokens", type=int, default=8192)
    ap.add_argument("--no-kernels", action="store_true", help="skip per-kernel timing")
    ap.add_argument("--no-layer", action="store_true", help="skip the MoELayer (shared expert) timing")
    ap.add_argument("--instr-steps", type=int, default=10, help="instrumented steps for in-step kernel times")
    ap.add_argument("--traffic", action="store_true", help="rocprofv3 --pmc driver mode")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write the traffic summary from the two --pmc passes' counter CSVs (no GPU)")
    ap.add_argument("--stats-summary", nargs=5, metavar=("PROF_DIR", "BENCH_LOG", "OUT_MD", "TITLE", "COMMAND"),
                    help="write a kernel-statistics summary of a rocprofv3 run of bench.py (no GPU)")
    args = ap.parse_args()
    if args.stats_summary:
        stats_summary(*args.stats_summary)
        return
    if args.traffic_summary:
        fcsv, wcsv = args.traffic_summary
        cmds = [f"cd /tmp && export TMPDIR=/tmp && timeout -s KILL 90 rocprofv3 --pmc {ctr} "
                f"--output-format csv -d $REPO/gpurun_out/pmc_{tag} -o p -- python3 $REPO/bench.py --traffic"
                for ctr, tag in (("FETCH_SIZE", "fetch"), ("WRITE_SIZE", "write"))]
        cmds.append("python3 bench.py --traffic-summary gpurun_out/pmc_fetch/p_counter_collection.csv "
                    "gpurun_out/pmc_write/p_counter_collection.csv")
        traffic_summary(fcsv, wcsv, TRAFFIC_FILE, cmds)
        return
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
    if args.traffic:
        traffic_mode(c, x, gate, wu, wd, go)
        return
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

    kernels, roofline, hbm = {}, None, {}
    if not args.no_kernels:
        in_step = instrumented_steps(step, args.instr_steps)
        missing = [n for v in STEP_KERNELS.values() for n in v
                   if n.startswith("gemm_") and n not in in_step]
        if missing:  # an entry point the step calls is not in STEP_KERNELS
            raise RuntimeError(f"bench: no in-step timing for {missing}")
        xd, gd, ud, dd = (p.detach() for p in params)
        fns, rows, keep = kernel_launches(c, xd, gd, ud, dd, go)
        work = algorithmic_work(c, rows)
        flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        traffic = measured_traffic()
        kernels = kernel_rates(in_step, work)
        gemms = [n for n in kernels if n.startswith("gemm_")]
        if gemms:
            dom = max(gemms, key=lambda n: kernels[n]["in_step_ms"])
            d = kernels[dom]
            roofline = dict(kernel=dom, bound="mfma", achieved=d["rate"], peak=PEAK_BF16_TFLOPS,
                            unit="TFLOP/s", frac=d["frac"], traffic=traffic.get(dom),
                            algorithmic_flop=work[dom][0], avg_launch_ms=d["in_step_ms"],
                            timing="in-step: HIP events around every launch of "
                                   f"{args.instr_steps} instrumented fwd+bwd steps")
        for name, role in HBM_ROLES.items():
            if name not in kernels or name not in fns:
                continue
            w = work[name][0]
            cold = cold_launch_ms(fns[name], flush, 20)
            kernels[name]["cold_ms"] = round(cold, 5)
            a_in = w / (kernels[name]["in_step_ms"] * 1e-3) / 1e9
            a_cold = w / (cold * 1e-3) / 1e9
            hbm[name] = dict(role=role, bound="hbm", achieved=round(a_in, 1), peak=PEAK_HBM_GBS,
                             unit="GB/s", frac=round(a_in / PEAK_HBM_GBS, 4),
                             cold_achieved=round(a_cold, 1), cold_frac=round(a_cold / PEAK_HBM_GBS, 4),
                             traffic=traffic.get(name), algorithmic_bytes=int(w))
        del keep, flush

    # MoELayer with the shared expert (config C2 as the reference's README quotes it)
    layer_ms = None
    if not args.no_layer:
        torch.manual_seed(0)
        layer = MoELayer(c["D"], c["ffn"], c["E"], top_k=c["k"], num_shared_experts=1,
                         aux_loss_coeff=c["aux"], z_loss_coeff=c["z"]).to(dev, torch.bfloat16)
        xl = x.detach().clone().requires_grad_(True)

        def layer_step():
            layer.zero_grad(set_to_none=True)
            xl.grad = None
            out, losses = layer(xl)
            torch.autograd.backward([out, losses["z_loss"]], [go, one])

        for _ in range(3):
            layer_step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = max(5, args.steps // 2)
        e0.record()
        for _ in range(reps):
            layer_step()
        e1.record()
        torch.cuda.synchronize()
        layer_ms = e0.elapsed_time(e1) / reps

    cpu = None if args.no_cpu else cpu_baseline(c, args.cpu_tokens)

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
        "hbm_rooflines": hbm,
        "kernels": kernels,
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
