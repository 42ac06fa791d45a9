"""Build of libomq_tree_ops.so with hipcc for gfx950 (in-tree, next to this file).

Flags: -ffp-contract=off and -fhip-fp32-correctly-rounded-divide-sqrt keep every fp32
expression IEEE round-to-nearest in source order (the selection argmax depends on the exact
bits); packed-fp32 instructions are disabled.  -falign-loops=64 starts every loop on a 64-byte
instruction-cache line: the selection chain's step loop (one wave, about 65 instructions per
pick) otherwise gains or loses a few percent with unrelated code changes ahead of it.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_HERE)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-falign-loops=64",
    "-Wall",
]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(_HERE, "csrc", "*.hip")))


def build_library(out: str | None = None, verbose: bool = False) -> str:
    out = out or os.path.join(_HERE, "libomq_tree_ops.so")
    tmp = out + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, "-I", os.path.join(_ROOT, "include"), "-o", tmp, *sources()]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    errs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs, file=sys.stderr)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_library(verbose=True))
