"""Build libintentir_hip.so in-tree with hipcc for gfx950.

    python -m intent_ir_amd.build          # compile, print the command
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libintentir_hip.so"
SOURCES = ["capi.hip", "rows.hip", "elementwise.hip", "gather.hip", "gemm.hip", "gemm_fast.hip", "gemm_pack.hip",
           "gemm_m16.hip", "gemm_f32.hip", "layernorm_f32.hip", "ewprog.hip", "ewjit.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Keep the compiler from forming packed-FP32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The first kernel arguments arrive in SGPRs at wave launch (gfx950 kernarg preloading; code
    # objects keep a loading prologue for firmware without it): the row kernels issue their first
    # loads without waiting on an argument load.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-function",
]
# hiprtc specialises element-wise programs at run time (ewjit.hip).
LINK_FLAGS = ["-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP backend cannot be built")


def build_library(verbose: bool = False) -> Path:
    """Compile every kernel source into one shared library (always recompiles)."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", str(tmp), *[str(CSRC / s) for s in SOURCES], *LINK_FLAGS]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build_library(verbose=True)
    print(f"built {LIB}")
    sys.exit(0)
