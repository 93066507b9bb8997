"""Builds libcubicsplat_hip.so (gfx950) in-tree with hipcc.

Flags that are part of the numerical contract:
  -ffp-contract=off     no implicit FMA contraction; the kernels write the
                        fused multiply-adds they want explicitly (the CPU
                        oracle restates the same expressions).
  -fno-fast-math        IEEE division and square root.
  -munsafe-fp-atomics   hardware fp32 global atomics instead of CAS loops.
  -packed-fp32-ops off  no v_pk_*_f32 generation.

Code-generation flag:
  -amdgpu-atomic-optimizer-strategy=None
                        every global atomic in these kernels is issued by one
                        lane after an explicit wave reduction; the compiler's
                        atomic optimizer would wrap each in a redundant
                        scan loop.
"""
from __future__ import annotations

import os
import subprocess
import sys
import warnings

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libcubicsplat_hip.so")
SOURCES = ["binning.hip", "raster.hip", "metric.hip", "optim.hip", "rings.hip", "gaussian.hip"]
ARCH = os.environ.get("CS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-mcode-object-version=5",
    "-ffp-contract=off", "-fno-fast-math", "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc"), "hipcc"):
        if os.path.isabs(cand) and os.path.exists(cand):
            return cand
    return "hipcc"


def build(verbose: bool = False) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(HERE, "..", "include"), "-o", tmp, *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.check_call(cmd)
    os.replace(tmp, LIB)
    from . import fastcall
    try:
        fastcall.build(LIB, verbose=verbose)
    except (OSError, subprocess.CalledProcessError) as e:
        # The compiled binding is an optional speed-up: without it the host
        # path calls the same library through ctypes.
        warnings.warn(f"the compiled binding _cs_fast was not built ({e}); using ctypes")
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
