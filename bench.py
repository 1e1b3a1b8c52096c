#!/usr/bin/env python3
"""Benchmark of the IntentIR MI355X backend on the five workloads of BASELINE.json.

One step = one launch of the lowered gfx950 kernel over one batch of the
workload (inputs already resident in HBM).  The headline line is the row-softmax
workload; the four other workloads are measured the
same way and reported under "kernels", each with its own roofline block and CPU
baseline.

Timing: W eager warmup launches, then K launches captured in one HIP graph on
torch's current stream.  The graph is replayed once untimed (upload), then
REPEATS = 5 times, each replay between two HIP events on that stream with a
device synchronisation on both sides; ms_per_step is the median replay time / K,
with the fastest and slowest replay reported beside it.  For workloads whose
per-launch footprint fits in the 256 MB Infinity Cache, launches rotate over
enough buffer sets (> 512 MiB in total) that reads must come from HBM.

CPU baseline: the reference's own CPU path (spmd_rvv C codegen + runtime, built
from the reference sources into oracle/_ref) on a bounded slice of each
workload, on all of this host's cores (nproc), by the reference driver's timing
method; the oracle restatement when that build is absent.

    python bench.py [--steps K] [--warmup W] [--config softmax|any|layernorm|gelu|matmul] [--only] [--no-cpu]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "HBM GB/s (% peak) per IntentIR kernel; matmul TFLOP/s; 1 MI355X"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
ROTATE_MIN_BYTES = 640 << 20   # > 2.5x the 256 MB Infinity Cache
REPEATS = 5                    # timed replays of the K-launch graph; the median is reported

WORKLOAD_NAMES = {
    "any": "any_kernel_dim reduce_any dim=1, f32 [8192,4096] -> bool[8192]",
    "softmax": "softmax_inner row softmax, f32 [16384,1024]",
    "layernorm": "layer_norm_persistent fwd, f16 [8192,4096], f32 stats",
    "gelu": "bias + GELU-tanh * 0.5 + x, bf16 [32768,8192]",
    "matmul": "relu(A@B + bias), bf16 8192^3, f32 acc",
}
DTYPES = {"any": "f32", "softmax": "f32", "layernorm": "f16", "gelu": "bf16", "matmul": "bf16"}


class Launcher:
    """Pre-bound C-ABI calls for R buffer sets (ctypes arguments built once)."""

    def __init__(self, lowered, sets, torch):
        from intent_ir_amd.runtime import load_library, launch_lowered

        self.lib = load_library()
        self.fn = getattr(self.lib, lowered.kernel_id)
        self.sets = sets
        self.torch = torch
        for bufs in sets:  # validates shapes/dtypes on the host before anything runs
            launch_lowered(lowered, bufs)
        torch.cuda.synchronize()
        self.args = []
        self.workspaces = []
        for bufs in sets:
            a = []
            for kind, v in lowered.call_args:
                if kind == "tensor":
                    a.append(ctypes.c_void_p(bufs[v].data_ptr()))
                elif kind == "i64":
                    a.append(ctypes.c_int64(int(v)))
                elif kind == "i32":
                    a.append(ctypes.c_int(int(v)))
                elif kind == "f32":
                    a.append(ctypes.c_float(float(v)))
                elif kind == "null":
                    a.append(ctypes.c_void_p(None))
                elif kind == "workspace":  # one workspace per buffer set, held for the run
                    t = torch.empty(max(1, int(v)), dtype=torch.uint8, device="cuda")
                    self.workspaces.append(t)
                    a += [ctypes.c_void_p(t.data_ptr()), ctypes.c_int64(int(v))]
                else:
                    raise RuntimeError(f"bench launcher does not bind call argument kind {kind}")
            self.args.append(a)

    def launch(self, i):
        s = ctypes.c_void_p(self.torch.cuda.current_stream().cuda_stream)
        st = self.fn(*self.args[i % len(self.args)], s)
        if st != 0:
            raise RuntimeError(f"launch failed: {self.lib.ihip_last_error().decode()}")


def measure(key, steps, warmup, torch, log, timing="eager"):
    from intent_ir_amd import lower_intent_to_hip_kernel
    from intent_ir_amd.configs import WORKLOADS, algorithmic_bytes, gen_device
    from intent_ir_amd.runtime import tensor_shapes, torch_dtype

    w = WORKLOADS[key]
    b = dict(w.bindings)
    lowered = lower_intent_to_hip_kernel(w.ir(), shape_bindings=b)
    shapes = tensor_shapes(lowered.io_spec, lowered.bindings)
    per_launch = algorithmic_bytes(key, b)
    nsets = 1 if key in ("matmul", "gelu") else max(2, math.ceil(ROTATE_MIN_BYTES / per_launch))
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    sets = []
    for _ in range(nsets):
        bufs = gen_device(key, b, torch, g)
        for n in lowered.output_names:
            spec = lowered.io_spec["tensors"][n]
            bufs[n] = torch.empty(shapes[n], dtype=torch_dtype(spec["dtype"]), device="cuda")
        sets.append(bufs)
    L = Launcher(lowered, sets, torch)
    log(f"[bench] {key}: kernel={lowered.kernel_id} sets={nsets} warmup={warmup} steps={steps}")
    for i in range(warmup):
        L.launch(i)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    if timing == "graph":
        graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            graph.capture_begin()
            for i in range(steps):
                L.launch(i)
            graph.capture_end()
        torch.cuda.current_stream().wait_stream(stream)
        graph.replay()  # untimed: first replay uploads the graph
        torch.cuda.synchronize()
        for _ in range(REPEATS):  # events on the stream the replay launches on (torch's current stream)
            t0.record()
            graph.replay()
            t1.record()
            torch.cuda.synchronize()
            times.append(t0.elapsed_time(t1) / steps)
        del graph
    else:
        for _ in range(REPEATS):
            torch.cuda.synchronize()
            t0.record()
            for i in range(steps):
                L.launch(i)
            t1.record()
            torch.cuda.synchronize()
            times.append(t0.elapsed_time(t1) / steps)
    ms = statistics.median(times)
    # cheap property check on the last written set (no oracle in the timed path)
    last = sets[(steps - 1) % nsets]
    if key == "softmax":
        rs = last["output_ptr"].double().sum(dim=1)
        assert torch.allclose(rs, torch.ones_like(rs), atol=1e-5), "softmax rows do not sum to 1"
    res = {"kernel": lowered.kernel_id, "ms_per_launch": ms, "ms_min": min(times), "ms_max": max(times),
           "repeats": REPEATS, "steps": steps, "warmup": warmup, "buffer_sets": nsets, "timing": timing,
           "algo_bytes": per_launch}
    if key == "matmul":
        flops = w.algorithmic_flops(b)
        tf = flops / (ms * 1e-3) / 1e12
        res.update(value=tf, unit="TFLOP/s", frac=tf / BF16_PEAK_TFLOPS, algo_flops=flops)
    else:
        gbs = per_launch / (ms * 1e-3) / 1e9
        res.update(value=gbs, unit="GB/s", frac=gbs / HBM_PEAK_GBS)
    res["roofline"] = roofline(key, res)
    del L, sets
    torch.cuda.empty_cache()
    return res


def roofline(key, res):
    """Roofline block of one workload's kernel: algorithmic work per launch / median launch time
    against MI355X's published peak; traffic = HBM bytes per launch from rocprofv3 counters
    (profiles/hbm_traffic.json, calibrated against a copy of known size), null if unmeasured."""
    tfile = ROOT / "profiles" / "hbm_traffic.json"
    traffic = json.loads(tfile.read_text()).get(res["kernel"]) if tfile.exists() else None
    if key == "matmul":
        return {"bound": "mfma", "achieved": res["value"], "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": res["frac"], "traffic": traffic}
    return {"bound": "hbm", "achieved": res["value"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": res["frac"],
            "traffic": traffic}


def host_threads():
    """This host's core count as `nproc` reports it (affinity mask and OMP_NUM_THREADS honoured)."""
    try:
        return max(1, int(subprocess.run(["nproc"], capture_output=True, text=True, timeout=10).stdout.strip()))
    except (OSError, ValueError, subprocess.SubprocessError):
        return max(1, len(os.sched_getaffinity(0)))


def host_cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def measure_in_child(key, steps, warmup, timing, log):
    """measure() in a fresh process (a child; its log lines are passed through)."""
    cmd = [sys.executable, str(ROOT / "bench.py"), "--config", key, "--only", "--no-cpu", "--steps", str(steps),
           "--warmup", str(warmup), "--timing", timing, "--kernel-json"]
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    for line in p.stderr.splitlines():
        if line.startswith("[bench]"):
            log(line)
    if p.returncode != 0:
        raise RuntimeError(f"bench child for {key} failed ({p.returncode}):\n{p.stderr[-2000:]}")
    return json.loads(p.stdout.strip().splitlines()[-1])


def cpu_baseline(key, log, target_s=5.0):
    """Reference CPU path on a bounded sample of the workload, timed on this host's cores.

    Preferred: the reference's own C path (oracle/_ref/<cfg>_sample, built from the reference
    sources by oracle/build_ref.py), run on the sample's real inputs with OpenMP on all nproc
    host threads (OMP_NUM_THREADS = INTENTIR_OMP_THREADS = nproc, OMP_PROC_BIND=close), timed by the
    reference driver (intentir_driver.c:59-83: 1 warmup, then iterations sized to ~target_s; the
    matmul 1 iteration and no warmup, its naive fp64 triple loop being slow); the program also
    checks its result against the oracle.  Fallback when that build is absent: the numpy oracle on
    the same sample, single-threaded."""
    from intent_ir_amd.configs import WORKLOADS, algorithmic_bytes
    from intent_ir_amd.dtypes import to_compute_f32
    from intent_ir_amd.ir import as_intent
    from intent_ir_amd.macros import expand_macros
    from oracle import ref_runner
    from oracle.interpreter import execute_intent

    w = WORKLOADS[key]
    if ref_runner.available(key, "sample"):
        b = ref_runner.bindings(key, "sample")
    else:
        b = dict(w.bindings)
        b["M"] = max(1, b["M"] // 16)
    fn = expand_macros(as_intent(w.ir()))
    raw = w.gen(b)
    f32 = {n: to_compute_f32(v, fn.tensors[n].dtype) for n, v in raw.items()}
    work = w.algorithmic_flops(b) if key == "matmul" else algorithmic_bytes(key, b)
    unit = "TFLOP/s" if key == "matmul" else "GB/s"
    scale = 1e12 if key == "matmul" else 1e9
    sample = f"{b} slice of the {w.bindings} workload"
    threads, cpu = host_threads(), host_cpu_model()
    if ref_runner.available(key, "sample"):
        ref = execute_intent(w.ir(), f32, b)
        if key == "matmul":
            iters, warm = 1, 0
        else:
            probe = ref_runner.run(key, "sample", fn, f32, ref, iters=1, threads=threads)
            iters = max(1, min(1000, int(target_s * 1e9 / probe.ns_per_iter))) if probe.ns_per_iter else 0
            warm = 1
        r = ref_runner.run(key, "sample", fn, f32, ref, iters=iters, warmup=warm, threads=threads) if iters else None
        if r is not None and r.ns_per_iter:
            log(f"[bench] {key} cpu reference path: {r.ns_per_iter / 1e6:.2f} ms/iter x {iters}, "
                f"{r.threads} threads, result {'PASS' if r.passed else 'FAIL'}")
            return {"value": work / (r.ns_per_iter * 1e-9) / scale, "unit": unit, "cores": r.threads,
                    "kind": "reference",
                    "sample": f"reference spmd_rvv C path (codegen + runtime built from the reference sources, "
                              f"-O3 -fopenmp), {sample}, {iters} timed iteration(s) after {warm} warmup, "
                              f"OMP_NUM_THREADS={r.threads} (nproc) on {cpu}, "
                              f"result vs oracle {'PASS' if r.passed else 'FAIL'}"}
        log(f"[bench] {key}: reference CPU path did not report timing")
    t0 = time.perf_counter()
    iters = 0
    while time.perf_counter() - t0 < target_s:
        execute_intent(w.ir(), f32, b)
        iters += 1
    dt = (time.perf_counter() - t0) / iters
    return {"value": work / dt / scale, "unit": unit, "cores": 1, "kind": "port",
            "sample": f"numpy oracle (restated interpreter), {sample}, {iters} iterations on {cpu}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="softmax", choices=sorted(WORKLOAD_NAMES))
    ap.add_argument("--only", action="store_true", help="measure the headline workload only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--timing", default="graph", choices=["eager", "graph"],
                    help="eager: K stream-ordered launches between two events; graph: one replay of K captured launches")
    ap.add_argument("--kernel-json", action="store_true",
                    help="(internal) measure --config only and print its result as one JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (every path here runs on one "
              "MI355X: the row workloads would shard by rows with no exchange, the GEMM by C tiles)", file=sys.stderr)
        sys.exit(2)
    import torch

    log = lambda m: print(m, file=sys.stderr, flush=True)  # noqa: E731
    if not torch.cuda.is_available():
        log("bench.py needs a ROCm device")
        sys.exit(1)
    key = args.config
    head = measure(key, args.steps, args.warmup, torch, log, args.timing)
    if args.kernel_json:
        print(json.dumps(head), flush=True)
        return
    log(f"[bench] {key}: {head['value']:.1f} {head['unit']} ({100 * head['frac']:.1f}% of peak), "
        f"{head['ms_per_launch'] * 1e3:.2f} us/launch (median of {REPEATS}; "
        f"{head['ms_min'] * 1e3:.2f}-{head['ms_max'] * 1e3:.2f})")
    kernels = {key: head}
    if not args.only:
        for other in WORKLOAD_NAMES:
            if other == key:
                continue
            # Each workload runs in a process of its own: buffers allocated after an earlier
            # workload's were freed measured up to ~7% slower for the same kernel (physical
            # placement the kernel does not control), which would make each number depend on the
            # order of the list.  Every workload gets the headline's warmup and step count.
            r = measure_in_child(other, args.steps, args.warmup, args.timing, log)
            log(f"[bench] {other}: {r['value']:.1f} {r['unit']} ({100 * r['frac']:.1f}% of peak), "
                f"{r['ms_per_launch'] * 1e3:.2f} us/launch (median of {REPEATS}; "
                f"{r['ms_min'] * 1e3:.2f}-{r['ms_max'] * 1e3:.2f})")
            kernels[other] = r
    for k, r in kernels.items():
        r["cpu_baseline"] = None if args.no_cpu else cpu_baseline(k, log, 10.0 if k == key else 5.0)
    line = {
        "metric": METRIC, "value": head["value"], "unit": head["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_launch"], "ms_per_step_min": head["ms_min"],
        "ms_per_step_max": head["ms_max"], "repeats": REPEATS, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": DTYPES[key], "data": "synthetic (seeded, workload distributions)",
        "config": {"workload": WORKLOAD_NAMES[key], "kernel": head["kernel"], "buffer_sets": head["buffer_sets"]},
        "roofline": head["roofline"], "cpu_baseline": head["cpu_baseline"],
        "kernels": {k: {kk: v[kk] for kk in ("kernel", "value", "unit", "frac", "ms_per_launch", "ms_min", "ms_max",
                                              "roofline", "cpu_baseline") if kk in v}
                    for k, v in kernels.items()},
    }
    for k, v in line["kernels"].items():
        v["dtype"] = DTYPES[k]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
