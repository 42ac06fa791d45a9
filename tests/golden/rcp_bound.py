"""Build of the reciprocal-bound checker (tests/golden/rcp_bound.hip) next to its source."""
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(_HERE, "rcp_bound.hip")
BIN = os.path.join(_HERE, "rcp_bound")


def build(hipcc: str = "/opt/rocm/bin/hipcc") -> str:
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-o", BIN + ".tmp", SRC]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{r.stdout}{r.stderr}")
    os.replace(BIN + ".tmp", BIN)
    return BIN
