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
    ("generic.hip", "generic.o", ()),
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


# The grouped GEMMs count their outstanding vector-memory operations by hand
# (s_waitcnt vmcnt(N) with N > 0 after the direct-to-LDS operand loads).  A
# register spill placed between such a load and such a wait would join the
# counted sequence and let the wait pass early, so every build checks the
# device assembly of gemm.hip for that pattern and fails if it finds one.
CHECKED_ASM = ("gemm.hip",)


def unsafe_scratch_ops(asm_text):
    """(kernel, wait, line) for every scratch access that lies, in
    straight-line code, between a direct-to-LDS buffer load and a later
    s_waitcnt vmcnt(N > 0) with no vmcnt(0) wait, label or branch between
    them."""
    import re
    out = []
    kernel, seen_dma, scratch = None, False, []
    for i, line in enumerate(asm_text.splitlines()):
        t = line.strip()
        m = re.match(r"^(_Z\S+):", line)
        if m:
            kernel, seen_dma, scratch = m.group(1), False, []
        elif t.startswith(".L") or t.startswith("s_branch") or t.startswith("s_cbranch"):
            seen_dma, scratch = False, []
        elif "offen lds" in t:
            seen_dma, scratch = True, []
        elif "scratch_" in t and seen_dma:
            scratch.append(i)
        elif t.startswith("s_waitcnt") and "vmcnt(" in t:
            n = int(re.search(r"vmcnt\((\d+)\)", t).group(1))
            if n > 0:
                out.extend((kernel, t, j) for j in scratch)
            else:
                seen_dma, scratch = False, []
    return out


def unwaited_claim_reads(asm_text):
    """(kernel, line, instruction) for every path from an assembly-issued
    returning atomic (`global_atomic_add vN, ..., off sc0`: the fused
    up+down launch's claims, whose return register the compiler does not
    know is pending) to an instruction that reads or writes vN, or to the
    end of the kernel, with no s_waitcnt vmcnt(0) on the way.  Such a read
    would see the register before the atomic's value arrives (a spill or a
    copy of it, typically)."""
    import re

    def vregs(t):
        out = set()
        for m in re.finditer(r"\bv\[(\d+):(\d+)\]", t):
            out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
        for m in re.finditer(r"\bv(\d+)\b", t):
            out.add(int(m.group(1)))
        return out

    bad = []
    for km in re.finditer(r"^(_Z\S+):", asm_text, re.M):
        end = asm_text.find(".Lfunc_end", km.start())
        lines = [ln.split(";")[0].strip() for ln in asm_text[km.start():end].splitlines()]
        labels = {ln[:-1]: i for i, ln in enumerate(lines) if re.match(r"^\.LBB\d+_\d+:$", ln)}
        for i, ln in enumerate(lines):
            m = re.match(r"global_atomic_add v(\d+), .*\boff sc0$", ln)
            if not m:
                continue
            reg, seen, stack = int(m.group(1)), set(), [i + 1]
            while stack:
                p = stack.pop()
                while p < len(lines) and p not in seen:
                    seen.add(p)
                    t = lines[p]
                    if not t or t.endswith(":"):
                        p += 1
                        continue
                    if t.startswith("s_waitcnt") and "vmcnt(0)" in t:
                        break
                    if t.startswith("s_endpgm") or (reg in vregs(t) and not t.startswith("s_")):
                        bad.append((km.group(1), p, t))
                        break
                    b = re.match(r"s_cbranch_\w+\s+(\.LBB\d+_\d+)", t)
                    if b:
                        stack.append(labels[b.group(1)])
                    b = re.match(r"s_branch\s+(\.LBB\d+_\d+)", t)
                    if b:
                        p = labels[b.group(1)]
                        continue
                    p += 1
    return bad


def _compile(unit, objdir):
    src, obj, extra = unit
    obj = os.path.join(objdir, obj)
    cmd = [HIPCC, *FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def _check_asm(src, objdir):
    out = os.path.join(objdir, src.replace(".hip", ".s"))
    cmd = [HIPCC, *FLAGS, "--cuda-device-only", "-S", "-c", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src}:\n{r.stderr}")
    with open(out) as f:
        text = f.read()
    os.remove(out)
    bad = unsafe_scratch_ops(text)
    if bad:
        names = sorted({k for k, _, _ in bad})
        raise RuntimeError(f"{src}: register spills inside hand-counted vmcnt sequences in {names}")
    bad = unwaited_claim_reads(text)
    if bad:
        names = sorted({k for k, _, _ in bad})
        raise RuntimeError(f"{src}: an assembly claim's return register is used before its vmcnt(0) in {names}")


def build(verbose=True):
    """Compiles every source and links libffmoe.so next to this file."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    jobs = max(1, min(len(UNITS) + len(CHECKED_ASM), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        checks = [ex.submit(_check_asm, src, objdir) for src in CHECKED_ASM]
        objs = list(ex.map(lambda u: _compile(u, objdir), UNITS))
        for c in checks:
            c.result()
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
