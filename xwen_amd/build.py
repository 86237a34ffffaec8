"""Build libxsamp.so for gfx950 with hipcc (no PyTorch, no cmake)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc", "xs_sampler.hip")
HOST_SRC = os.path.join(HERE, "csrc", "xs_host.cpp")  # host-only C ABI (also built alone for ASan)
OUT = os.path.join(HERE, "libxsamp.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # every float operation rounds as written: no contraction into FMA
    "-ffp-contract=off",
    # IEEE f32 denormals (probabilities and exp values reach the subnormal range)
    "-fno-gpu-flush-denormals-to-zero",
    # no packed-FP32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build(verbose: bool = False) -> str:
    tmp = OUT + ".tmp"
    cmd = [HIPCC, *FLAGS, SRC, HOST_SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{r.stderr[-4000:]}")
    if verbose and r.stderr:
        print(r.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
