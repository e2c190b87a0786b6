"""Runs each grouped GEMM of the C2 layer (N 8192, D 1024, ffn 4096, E 8,
k 2) twice through the C ABI, after a 256 MiB device-to-device copy that
calibrates the HBM counters.  A profiling driver for

    rocprofv3 --pmc FETCH_SIZE ... -- python3 flashfusedmoe_amd/gemm_probe.py
    rocprofv3 --pmc WRITE_SIZE ... -- python3 flashfusedmoe_amd/gemm_probe.py

``GEMMS`` (comma-separated: up, down, dgrad_glu, dgrad, wgrad) selects a
subset.  Synthetic seeded inputs; nothing is checked here (the parity tests
do that).
"""

import os
import sys

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from flashfusedmoe_amd import _lib as L  # noqa: E402
from flashfusedmoe_amd import ops  # noqa: E402


def main():
    N, D, H, E, k = 8192, 1024, 2048, 8, 2
    T = N * k
    g = torch.Generator().manual_seed(0)
    dev = "cuda"
    x = torch.randn(N, D, generator=g).bfloat16().to(dev)
    gate = (torch.randn(E, D, generator=g) * D ** -0.5).bfloat16().to(dev)
    wu = (torch.randn(E, 2 * H, D, generator=g) * D ** -0.5).bfloat16().to(dev)
    wd = (torch.randn(E, D, H, generator=g) * H ** -0.5).bfloat16().to(dev)
    mt = 4096
    r = ops.route(x, gate, None, k, 0, mt, 0.0, 0.0, False)
    idx, tw, counts, off, til, ws = r[1], r[2], r[4], r[5], r[6], r[9]
    _, _, _, xs, up, act, _ = ops.experts_forward(x, wu, wd, idx, tw, counts, off, til, ws, k, 0,
                                                  mt, False, True)
    P = L.ptr
    st = L.stream_ptr()
    tr = L.gemm_tile_rows(T, E)
    gws = P(L.gemm_workspace(x.device, st))
    gup = torch.randn(T, 2 * H, device=dev).bfloat16()
    wgo = torch.randn(T, D, device=dev).bfloat16()
    o_up, o_act, o_gup = torch.empty_like(up), torch.empty_like(act), torch.empty_like(up)
    o_d = torch.empty(T, D, device=dev, dtype=torch.bfloat16)
    dwu = torch.empty(E, 2 * H, D, device=dev, dtype=torch.bfloat16)
    calls = {
        "up": lambda: L.call("ffmoe_gemm_up_glu", P(xs), P(wu), P(off), P(til), tr, E, T, D, H, 0,
                             P(o_up), P(o_act), gws, st),
        "down": lambda: L.call("ffmoe_gemm_down", P(act), P(wd), P(off), P(til), tr, E, T, H, D,
                               P(o_d), gws, st),
        "dgrad_glu": lambda: L.call("ffmoe_gemm_dgrad_glu", P(wgo), P(wd), P(up), P(off), P(til), tr,
                                    E, T, D, H, 0, P(o_gup), gws, st),
        "dgrad": lambda: L.call("ffmoe_gemm_dgrad", P(gup), P(wu), P(off), P(til), tr, E, T, H, D,
                                P(o_d), gws, st),
        "wgrad": lambda: L.call("ffmoe_gemm_wgrad", P(gup), P(xs), P(off), E, 2 * H, D, P(dwu), st),
    }
    which = os.environ.get("GEMMS", ",".join(calls)).split(",")
    # calibration: 256 MiB read + 256 MiB written by the runtime's copy kernel
    src = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device=dev).uniform_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    for name in which:
        for _ in range(2):
            calls[name]()
        torch.cuda.synchronize()
    print("gemm_probe done", flush=True)


if __name__ == "__main__":
    main()
