"""Compile the cq35 HIP library in-tree for gfx950.

The library is one translation unit (csrc/runtime.hip + the kernel headers)
built with hipcc. Flags that carry semantics:
  -ffp-contract=off                        every multiply and add rounds
                                           separately, as the reference's
                                           numerics require (numeric.hex:10)
  -fhip-fp32-correctly-rounded-divide-sqrt IEEE division
  -fno-gpu-flush-denormals-to-zero         keep F32 subnormals
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                           no packed-FP32 instructions
"""
from __future__ import annotations

import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
SOURCE = os.path.join(ROOT, "csrc", "runtime.hip")
LIBRARY = os.path.join(PKG_DIR, "libcq35.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-value", "-Wno-unused-result",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


TRACE_LIBRARY = os.path.join(PKG_DIR, "libcq35_trace.so")


def build(verbose: bool = False, trace: bool = False) -> str:
    """Always recompile (the driver's build check relies on this). With
    trace=True, build the phase-trace variant (-DCQ35_PHASE_TRACE) into
    libcq35_trace.so instead."""
    out = TRACE_LIBRARY if trace else LIBRARY
    tmp = out + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *(["-DCQ35_PHASE_TRACE"] if trace else []), "-o", tmp, SOURCE]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + proc.stderr[-8000:])
    if verbose and proc.stderr.strip():
        print(proc.stderr[-4000:])
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
