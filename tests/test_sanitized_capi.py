"""Host AddressSanitizer + UndefinedBehaviorSanitizer build of the C-ABI (CPU only).

Every library source is compiled with the sanitizers on the host code only (hipcc's
-Xarch_host; device code is compiled as usual and never launched) and linked with
tests/sanitize/capi_checks.cpp, which drives the argument validation of every entry point,
the element-wise program checker (hand-written malformed programs and 20000 random ones)
and the native-code planner and source generator.  A sanitizer report fails the run."""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from intent_ir_amd.build import CSRC, SOURCES

ROOT = Path(__file__).resolve().parents[1]
DRIVER = ROOT / "tests" / "sanitize" / "capi_checks.cpp"
OUT = ROOT / "intent_ir_amd" / "_build" / "sanitize"
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-Xarch_host",
       "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]
FLAGS = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops"]


def _hipcc():
    return shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if Path("/opt/rocm/bin/hipcc").exists() else None)


def _build(hipcc: str) -> Path:
    OUT.mkdir(parents=True, exist_ok=True)
    exe = OUT / "capi_checks"
    srcs = [CSRC / s for s in SOURCES] + [DRIVER]
    deps = srcs + [ROOT / "include" / "intentir_hip.h", CSRC / "common.hpp"]
    if exe.exists() and exe.stat().st_mtime > max(p.stat().st_mtime for p in deps):
        return exe

    def compile_one(src: Path):
        obj = OUT / (src.stem + ".o")
        cmd = [hipcc, "-x", "hip", *FLAGS, *SAN, "-c", str(src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"{' '.join(cmd)}\n{r.stderr[-3000:]}")
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, srcs))
    cmd = [hipcc, *SAN, "-o", str(exe), *map(str, objs), "-L/opt/rocm/lib", "-lhiprtc", "-lamdhip64",
           "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-3000:]}")
    return exe


def test_c_abi_argument_checks_under_asan_and_ubsan():
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    exe = _build(hipcc)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0 and "ALL OK" in r.stdout, f"rc={r.returncode}\n{r.stdout[-2000:]}\n{r.stderr[-4000:]}"
