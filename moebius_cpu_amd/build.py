"""Builds the HIP library in-tree: every csrc/*.hip and csrc/*.cpp compiled for
gfx950 with hipcc, linked into moebius_cpu_amd/libmoebius_hip.so.

    python -m moebius_cpu_amd.build        # or __graft_entry__.build()
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmoebius_hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -ffp-contract=off: every fused multiply-add is written out (fmaf), so the
# device arithmetic matches the CPU engine's where the kernels restate it.
# The packed-fp32 feature is switched off for all device code.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
]


def _compile(src: str, incremental: bool = False) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    if incremental and os.path.exists(obj):
        deps = [src, *glob.glob(os.path.join(CSRC, "*.hpp")), *glob.glob(os.path.join(HERE, "..", "include", "*.h"))]
        if os.path.getmtime(obj) >= max(os.path.getmtime(d) for d in deps if os.path.exists(d)):
            return obj
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    warn = "\n".join(l for l in r.stderr.splitlines() if "warning" in l and "packed-fp32-ops" not in l
                     and "target-feature" not in l)
    if warn:
        print(f"[build] {os.path.basename(src)}:\n{warn}", file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = True, incremental: bool = False) -> str:
    """Compiles every source and links the library; returns its path.
    incremental: reuse objects newer than their source and every header."""
    if not os.path.exists(HIPCC) and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found")
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, incremental), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[build] {LIB} ({len(objs)} objects)")
    return LIB


if __name__ == "__main__":
    build(incremental="-i" in sys.argv[1:])
