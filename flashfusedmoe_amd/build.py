"""Builds libffmoe.so (the HIP kernels behind include/ffmoe.h) in-tree.

    python -m flashfusedmoe_amd.build        # or: from flashfusedmoe_amd.build import build

hipcc cross-compiles for gfx950 without a GPU, so this runs on any machine
with ROCm.  Every call recompiles every source.
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libffmoe.so")
# (source, object, extra flags): route.hip is compiled once per expert-count
# tier of its routing kernel (FFMOE_ROUTE_PART), so the units build in parallel
UNITS = (
    ("status.hip", "status.o", ()),
    ("route.hip", "route.o", ("-DFFMOE_ROUTE_PART=0",)),
    *((("route.hip", f"route_et{et}.o", (f"-DFFMOE_ROUTE_PART={et}",)) for et in (1, 2, 4, 8, 16))),
    ("combine.hip", "combine.o", ()),
    ("gemm.hip", "gemm.o", ()),
)
ARCH = os.environ.get("FFMOE_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 VALU ops are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
    "-Wall", "-Wno-unused-function",
]


# Kernels whose hand-counted vmcnt waits assume that no scratch (register
# spill) access ever joins the vector-memory queue: the build fails if the
# compiler gives any of them scratch.
NO_SCRATCH_KERNELS = ("gemm_pp_kernel",)


def _scratch_kernels(remarks):
    """Names of kernels with a nonzero ScratchSize in hipcc's
    -Rpass-analysis=kernel-resource-usage remarks."""
    bad, name = [], None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:", 1)[1].split()[0]
        elif "ScratchSize [bytes/lane]:" in line and name is not None:
            size = int(line.split("ScratchSize [bytes/lane]:", 1)[1].split()[0])
            if size > 0 and any(k in name for k in NO_SCRATCH_KERNELS):
                bad.append(f"{name} ({size} B/lane)")
    return bad


def _compile(unit, objdir):
    src, obj, extra = unit
    obj = os.path.join(objdir, obj)
    cmd = [HIPCC, *FLAGS, *extra, "-Rpass-analysis=kernel-resource-usage", "-c",
           os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    bad = _scratch_kernels(r.stderr)
    if bad:
        raise RuntimeError(f"{src}: kernels that must not spill use scratch: {', '.join(bad)}")
    return obj


def build(verbose=True):
    """Compiles every source and links libffmoe.so next to this file."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    jobs = max(1, min(len(UNITS), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda u: _compile(u, objdir), UNITS))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
