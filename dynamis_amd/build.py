"""Compile libdynamis_graph.so (gfx950) in-tree with hipcc.

    python -m dynamis_amd.build            # or dynamis_amd.build.build()

Flags: -ffp-contract=off keeps the canonical fp64 predicate's operation order exactly
as written (explicit fma only); packed fp32 ops are disabled for the target.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libdynamis_graph.so")
SOURCES = ["dg_graph.hip", "dg_count.hip", "dg_sfc.hip", "dg_halo.hip", "dg_batch.hip"]
# Per-source flags.  The count kernel's sweep is bound by VALU issue: LLVM's iterative ILP
# scheduler orders it better (C3 count 0.464 -> 0.440 ms), while the default scheduler
# suits the store-bound write kernels of dg_graph.hip (0.660 vs 0.671 ms under ILP).
# The halo plan's edge pass (random gathers, latency-bound) gains from the ILP scheduler too
# (C3, 8 ranks: 0.176 -> 0.170 ms per plan).
SOURCE_FLAGS = {"dg_count.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
                "dg_halo.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]}
ARCH = os.environ.get("DG_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"),
    "-Wall",
    "-Wextra",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + out)
    return out


def build(verbose: bool = False) -> str:
    objs = []
    bdir = os.path.join(HERE, "_build")
    os.makedirs(bdir, exist_ok=True)
    for src in SOURCES:
        obj = os.path.join(bdir, src.replace(".hip", ".o"))
        out = _run([HIPCC, *FLAGS, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj])
        if verbose and out.strip():
            print(out)
        objs.append(obj)
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
