"""Build libxsamp.so for gfx950 with hipcc (no PyTorch, no cmake).

The device code and the host code are compiled in separate passes, so the
device-only target feature (-packed-fp32-ops) reaches only the gfx950 pass:
  1. the device pass of xs_sampler.hip -> an offload bundle (.hipfb);
  2. the host pass of xs_sampler.hip, embedding that bundle;
  3. the host-only C ABI (xs_host.cpp);
  4. one shared library linked against the HIP runtime.
"""
from __future__ import annotations

import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc", "xs_sampler.hip")
HOST_SRC = os.path.join(HERE, "csrc", "xs_host.cpp")  # host-only C ABI (also built alone for ASan)
OUT = os.path.join(HERE, "libxsamp.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

ARCH = "--offload-arch=gfx950"
COMMON = [
    "-O3", "-std=c++17", "-fPIC",
    # every float operation rounds as written: no contraction into FMA
    "-ffp-contract=off",
]
DEVICE = [
    # IEEE f32 denormals (probabilities and exp values reach the subnormal range)
    "-fno-gpu-flush-denormals-to-zero",
    # no packed-FP32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> str:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}): {' '.join(cmd)}\n{r.stderr[-4000:]}")
    return r.stderr


def build(verbose: bool = False) -> str:
    with tempfile.TemporaryDirectory(prefix="xsamp_build_") as tmpd:
        fb = os.path.join(tmpd, "xs_sampler.hipfb")
        ho = os.path.join(tmpd, "xs_sampler.o")
        co = os.path.join(tmpd, "xs_host.o")
        tmp = OUT + ".tmp"
        log = _run([HIPCC, "-x", "hip", ARCH, "--offload-device-only", *COMMON, *DEVICE,
                    "-c", SRC, "-o", fb])
        log += _run([HIPCC, "-x", "hip", ARCH, "--offload-host-only", *COMMON,
                     "-Xclang", "-fcuda-include-gpubinary", "-Xclang", fb, "-c", SRC, "-o", ho])
        log += _run([HIPCC, "-x", "hip", ARCH, "--offload-host-only", *COMMON, "-c", HOST_SRC, "-o", co])
        log += _run([HIPCC, "--hip-link", "-shared", "-fPIC", ho, co, "-o", tmp])
    if verbose and log:
        print(log)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
