#!/usr/bin/env python3
"""Build the reference CPU execution path into oracle/_ref/.  TEST INFRASTRUCTURE ONLY.

The reference's CPU path for an IntentIR function is: the C++ codegen tool
(backends/spmd_rvv/cpp_codegen/intentir_codegen.cpp, CLI at :2085-2424) turns the
IR JSON plus shape bindings into a standalone C program, which is compiled
against the C runtime (backends/spmd_rvv/runtime/intentir_{ops,driver,runtime}.c).
This recipe compiles those sources where they lie under the reference tree
(nothing is copied into the repository) with the reference's own remote flags
minus the RISC-V target (scripts/rvv_remote_run.py:715,730): -O3 -fopenmp.  The C
compiler is the image's LLVM clang with its OpenMP runtime: gcc 11 rejects the
runtime's `collapse(2)` over imperfectly nested loops (intentir_ops.c:3303-3306).

Outputs (git-ignored, shipped to the GPU box with the tree):
  oracle/_ref/intentir_codegen      the reference codegen tool
  oracle/_ref/<cfg>_sample          verify-mode program at the CPU-baseline sample size
  oracle/_ref/<cfg>_tiny            verify-mode program at a tiny size (parity tests)
  oracle/_ref/manifest.json         bindings each program was generated for

Verify-mode programs read <input>.bin (float32, bool as bytes) from the working
directory, run the computation, run INTENTIR_BENCH_ITERS timed iterations
(intentir_driver.c:59-83) and compare against <output>_ref.bin.

    python oracle/build_ref.py [--reference /root/reference]
"""

from __future__ import annotations

import argparse
import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
OUT = HERE / "_ref"

# Sample bindings: a bounded slice of each workload (rows scaled down, row length kept) so a
# timed run is seconds of CPU work; bench.py reports bytes (or flops) per second.
SAMPLE_BINDINGS = {
    "any": {"M": 2048, "N": 4096},
    "softmax": {"M": 4096, "N": 1024},
    "layernorm": {"M": 2048, "N": 4096},
    "gelu": {"M": 1024, "N": 8192},
    "matmul": {"M": 32, "N": 8192, "K": 8192},
}
C_COMPILER = os.environ.get("IHIP_REF_CC", "/opt/rocm/llvm/bin/clang")
OMP_LIB_DIR = "/opt/rocm/llvm/lib"

TINY_BINDINGS = {
    "any": {"M": 5, "N": 33},
    "softmax": {"M": 4, "N": 17},
    "layernorm": {"M": 3, "N": 24},
    "gelu": {"M": 3, "N": 16},
    "matmul": {"M": 3, "N": 5, "K": 7},
}


def _run(cmd, **kw):
    res = subprocess.run(cmd, capture_output=True, text=True, **kw)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(map(str, cmd))}\n{res.stderr[-2000:]}")
    return res.stdout


def build(reference: Path, verbose: bool = False) -> Path:
    sys.path.insert(0, str(REPO))
    from intent_ir_amd.configs import WORKLOADS
    from intent_ir_amd.ir import as_intent
    from intent_ir_amd.macros import expand_macros

    spmd = reference / "backends" / "spmd_rvv"
    tool_src = spmd / "cpp_codegen" / "intentir_codegen.cpp"
    runtime = [spmd / "runtime" / f for f in ("intentir_ops.c", "intentir_driver.c", "intentir_runtime.c")]
    for f in [tool_src, *runtime]:
        if not f.exists():
            raise FileNotFoundError(f)
    OUT.mkdir(parents=True, exist_ok=True)
    cc, omp_dir = C_COMPILER, OMP_LIB_DIR
    tool = OUT / "intentir_codegen"
    if not tool.exists() or tool.stat().st_mtime < tool_src.stat().st_mtime:
        _run(["g++", "-std=c++17", "-O2", "-I", str(spmd / "cpp_codegen" / "third_party"), str(tool_src), "-o", str(tool)])
    gen = OUT / "gen"
    gen.mkdir(exist_ok=True)
    manifest = {}
    for key, w in WORKLOADS.items():
        ir = expand_macros(as_intent(w.ir())).to_json_dict()
        (gen / f"{key}.json").write_text(json.dumps(ir, indent=1))
        for size, binds in (("sample", SAMPLE_BINDINGS[key]), ("tiny", TINY_BINDINGS[key])):
            shapes = gen / f"{key}_{size}_shapes.json"
            shapes.write_text(json.dumps(binds))
            csrc = _run([str(tool), "--intent", str(gen / f"{key}.json"), "--shapes", str(shapes), "--mode", "verify",
                         "--atol", "1e-3", "--rtol", "1e-3"])
            cfile = gen / f"{key}_{size}.c"
            cfile.write_text(csrc)
            exe = OUT / f"{key}_{size}"
            _run([cc, "-O3", "-std=gnu11", "-fopenmp", "-I", str(spmd / "runtime"), str(cfile), *map(str, runtime),
                  "-lm", f"-L{omp_dir}", f"-Wl,-rpath,{omp_dir}", "-o", str(exe)])
            manifest[f"{key}_{size}"] = binds
            if verbose:
                print(f"built {exe.relative_to(REPO)} for {binds}", flush=True)
    (OUT / "manifest.json").write_text(json.dumps(manifest, indent=1))
    return OUT


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default=os.environ.get("IHIP_REFERENCE_ROOT", "/root/reference"))
    args = ap.parse_args()
    ref = Path(args.reference)
    if not ref.exists():
        print(f"reference tree {ref} not present; oracle/_ref not rebuilt", flush=True)
        return 0
    if shutil.which("g++") is None or not Path(C_COMPILER).exists():
        print("g++ or the LLVM clang is missing; oracle/_ref not built", flush=True)
        return 0
    build(ref, verbose=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
