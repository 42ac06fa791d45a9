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


def build_torch_ops(out: str | None = None, verbose: bool = False) -> str:
    """libomq_torch_ops.so: the torch operators (csrc/torch_ops.cpp), host C++ over the C ABI,
    linked against libomq_tree_ops.so beside it (build that first)."""
    import torch
    from torch.utils import cpp_extension

    out = out or os.path.join(_HERE, "libomq_torch_ops.so")
    tmp = out + ".tmp"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
           "-D__HIP_PLATFORM_AMD__", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *(f"-I{p}" for p in cpp_extension.include_paths()), "-I/opt/rocm/include",
           "-I", os.path.join(_ROOT, "include"),
           "-o", tmp, os.path.join(_HERE, "csrc", "torch_ops.cpp"),
           f"-L{_HERE}", "-lomq_tree_ops", "-Wl,-rpath,$ORIGIN",
           *(f"-L{p}" for p in cpp_extension.library_paths()),
           *(f"-Wl,-rpath,{p}" for p in cpp_extension.library_paths()),
           "-lc10", "-lc10_hip", "-ltorch_cpu"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"c++ failed ({r.returncode}):\n{r.stdout}{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_library(verbose=True))
    print(build_torch_ops(verbose=True))
