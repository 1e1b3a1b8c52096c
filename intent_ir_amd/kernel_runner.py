"""Launch one workload's kernel a fixed number of times (for profilers).

    python -m intent_ir_amd.kernel_runner --config softmax --launches 20 [--copy-mib 512]
    python -m intent_ir_amd.kernel_runner --config matmul --bindings M=4096,N=50257,K=4096 --transpose-b
    python -m intent_ir_amd.kernel_runner --ew-chain all --launches 20
    python -m intent_ir_amd.kernel_runner --row-reduce sum --bindings M=64,N=1048576 --launches 20
    python -m intent_ir_amd.kernel_runner --gather --bindings M=8192,N=8192,L=16777216 --launches 20
    python -m intent_ir_amd.kernel_runner --f32 matmul --launches 10        # 8192^3 on the fp32 matrix cores
    python -m intent_ir_amd.kernel_runner --f32 layernorm --launches 20     # [8192, 4096] f32
    python -m intent_ir_amd.kernel_runner --sweep softmax --launches 100    # fixed cost vs a copy
    python -m intent_ir_amd.kernel_runner --sweep softmax-rows --launches 20  # rows per workgroup
    python -m intent_ir_amd.kernel_runner --sweep gemm-tile --launches 10   # the GEMM tile rule
    python -m intent_ir_amd.kernel_runner --sweep gemm-split --launches 10  # the split-K rule

``--ew-chain`` runs generic element-wise programs (ihip_elementwise_program, native code)
on 8192 x 8192 operands and prints each chain's rate: per launch, every input's bytes
read once and every output's written once, timed like bench.py (median of 5 graph replays
of ``--launches`` launches after a compile-and-warm-up launch, buffer sets rotated over
>= 640 MiB).  ``--row-reduce``
times reduce_sum / reduce_max over the last axis of an f32 [M, N] tensor the same way
(rotating buffer sets over > 640 MiB), default [64, 1048576]: few long rows, which the
library splits over several workgroups per row with partial results in a workspace.
``--gather`` times gather2d (ihip_gather2d_f32) over L uniformly random index pairs into an
f32 [M, N] tensor (default 8192 x 8192, L = 2^24), 16 algorithmic bytes per element.

Inputs are generated on the GPU; launches rotate over enough buffer sets that
reads come from HBM rather than the Infinity Cache (as in bench.py).  With
``--copy-mib`` the run ends with plain device-to-device copies of that size
(torch ``copy_``), whose FETCH_SIZE/WRITE_SIZE readings calibrate the HBM byte
counters against a known transfer.  ``--bindings`` replaces the workload's shape
bindings; ``--transpose-b`` (matmul) gives B as [N, K] with matmul{transpose_b};
``--no-workspace`` passes an empty workspace, so a GEMM whose operands would be packed runs
the guarded kernel instead, and a softmax over rows longer than 65536 floats the
workgroup-per-row kernel instead of the split one.
"""

from __future__ import annotations

import argparse
import dataclasses
import math
import sys

ROTATE_MIN_BYTES = 640 << 20


def _t(dtype, *shape):
    return {"dtype": dtype, "shape": list(shape)}


def _op(name, inputs, output, **attrs):
    d = {"op": name, "inputs": list(inputs), "output": output}
    if attrs:
        d["attrs"] = attrs
    return d


def _gelu_ir(dt):
    from .configs import bias_gelu_axpy_ir  # noqa: PLC0415

    return bias_gelu_axpy_ir(dt)


# Element-wise chains timed by --ew-chain: (IR, bindings, extra bindings).  8192 x 8192 unless
# stated; 16-bit inputs where the chain says so.
EW_CHAINS = {
    "leaky_where_f32": lambda: ({"name": "leaky", "tensors": {
        "x": _t("f32", "M", "N"), "z": _t("f32"), "p": _t("i1", "M", "N"), "s": _t("f32", "M", "N"),
        "y": _t("f32", "M", "N")},
        "ops": [_op("const", [], "z", value=0.0, dtype="f32"), _op("gt", ["x", "z"], "p"),
                _op("mul", ["x"], "s", mul_factor=0.1), _op("where", ["p", "x", "s"], "y")], "outputs": ["y"]},
        {"M": 8192, "N": 8192}),
    "bias_relu_f32": lambda: ({"name": "bias_relu", "tensors": {
        "x": _t("f32", "M", "N"), "b": _t("f32", "N"), "t": _t("f32", "M", "N"), "y": _t("f32", "M", "N")},
        "ops": [_op("add", ["x", "b"], "t"), _op("relu", ["t"], "y")], "outputs": ["y"]}, {"M": 8192, "N": 8192}),
    "gelu_f32": lambda: (_gelu_ir("f32"), {"M": 8192, "N": 8192}),
    "scale_f16_bf16": lambda: ({"name": "scale", "tensors": {
        "x": _t("f16", "M", "N"), "w": _t("bf16", "N"), "t": _t("f32", "M", "N"), "y": _t("bf16", "M", "N")},
        "ops": [_op("mul", ["x", "w"], "t"), _op("add", ["t"], "y", addend=0.25)], "outputs": ["y"]},
        {"M": 8192, "N": 8192}),
    "transpose_bias_f32": lambda: ({"name": "tb", "tensors": {
        "x": _t("f32", "N", "M"), "b": _t("f32", "N"), "xt": _t("f32", "M", "N"), "y": _t("f32", "M", "N")},
        "ops": [_op("transpose", ["x"], "xt", perm=[1, 0]), _op("add", ["xt", "b"], "y")], "outputs": ["y"]},
        {"M": 8192, "N": 8192}),
    "sigmoid_bf16": lambda: ({"name": "sigmoid", "tensors": {
        "x": _t("bf16", "M", "N"), "u": _t("f32", "M", "N"), "e": _t("f32", "M", "N"), "one": _t("f32"),
        "d": _t("f32", "M", "N"), "y": _t("bf16", "M", "N")},
        "ops": [_op("mul", ["x"], "u", mul_factor=-1.0), _op("exp", ["u"], "e"),
                _op("const", [], "one", value=1.0, dtype="f32"), _op("add", ["e", "one"], "d"),
                _op("div", ["one", "d"], "y")], "outputs": ["y"]}, {"M": 8192, "N": 8192}),
    # the GELU workload (bf16 [32768, 8192]) through the generic program instead of its kernel
    "gelu_bf16_workload": lambda: (_gelu_ir("bf16"), {"M": 32768, "N": 8192, "HIP_ELEMENTWISE_PROGRAM": 1}),
}


def _ew_inputs(k, torch, g):
    from .runtime import tensor_shapes, torch_dtype  # noqa: PLC0415

    shapes = tensor_shapes(k.io_spec, k.bindings)
    bufs, nbytes = {}, 0
    for n, spec in k.io_spec["tensors"].items():
        dt = torch_dtype(spec["dtype"])
        if n in k.output_names:
            bufs[n] = torch.empty(shapes[n], dtype=dt, device="cuda")
        elif dt == torch.bool:
            bufs[n] = torch.rand(shapes[n], generator=g, device="cuda") < 0.5
        else:
            bufs[n] = torch.randn(shapes[n], generator=g, device="cuda").to(dt)
        nbytes += bufs[n].numel() * bufs[n].element_size()
    return bufs, nbytes


def run_ew_chains(names, launches, torch) -> int:
    from . import lower_intent_to_hip_kernel  # noqa: PLC0415
    from .runtime import launch_lowered  # noqa: PLC0415

    g = torch.Generator(device="cuda")
    g.manual_seed(4321)
    for name in names:
        ir, b = EW_CHAINS[name]()
        k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
        assert k.kernel_id == "ihip_elementwise_program", k.kernel_id
        bufs, nbytes = _ew_inputs(k, torch, g)
        sets = [bufs] + [_ew_inputs(k, torch, g)[0] for _ in range(max(2, math.ceil(ROTATE_MIN_BYTES / nbytes)) - 1)]
        launch_lowered(k, bufs)  # compiles the native code, warms up

        def launch(i, k=k, sets=sets):
            launch_lowered(k, sets[i % len(sets)])

        ms = _graph_time(launch, len(sets), launches, torch)
        prog = k.call_args[0][1]
        print(f"[runner] ew {name}: {len(prog.code)} instructions, {nbytes / 2**20:.0f} MiB/launch, "
              f"{len(sets)} buffer sets, {ms * 1e3:.1f} us/launch, {nbytes / (ms * 1e-3) / 1e12:.2f} TB/s "
              f"({100 * nbytes / (ms * 1e-3) / 8e12:.1f}% of 8 TB/s)", flush=True)
        del bufs, sets
        torch.cuda.empty_cache()
    return 0


def run_row_reduce(kind, bindings, launches, torch) -> int:
    import statistics  # noqa: PLC0415

    from . import lower_intent_to_hip_kernel  # noqa: PLC0415
    from .runtime import launch_lowered  # noqa: PLC0415

    op = {"sum": "reduce_sum", "max": "reduce_max"}[kind]
    ir = {"name": f"row_{op}", "tensors": {"x": _t("f32", "M", "N"), "out": _t("f32", "M")},
          "ops": [_op(op, ["x"], "out", dims=[1])], "outputs": ["out"]}
    b = {"M": 64, "N": 1 << 20, **bindings}
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    per = 4 * b["M"] * b["N"] + 4 * b["M"]
    nsets = max(2, math.ceil(ROTATE_MIN_BYTES / per))
    g = torch.Generator(device="cuda")
    g.manual_seed(99)
    sets = [{"x": torch.randn((b["M"], b["N"]), generator=g, device="cuda"),
             "out": torch.empty(b["M"], device="cuda")} for _ in range(nsets)]
    for i in range(nsets):
        launch_lowered(k, sets[i])
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(5):
        t0.record()
        for i in range(launches):
            launch_lowered(k, sets[i % nsets])
        t1.record()
        torch.cuda.synchronize()
        times.append(t0.elapsed_time(t1) / launches)
    ms = statistics.median(times)
    print(f"[runner] row {op} {b}: {k.kernel_id}, {ms * 1e3:.1f} us/launch, {per / (ms * 1e-3) / 1e12:.2f} TB/s",
          flush=True)
    return 0


def run_f32(family, bindings, launches, torch) -> int:
    """The reference's own f32 IR of a family (matmul_bias_relu2d, pipeline/tilelang/core.py:886-910,
    on ihip_gemm_f32_bias_relu; layer_norm_persistent, :1322-1384, on ihip_layernorm_rows_f32),
    timed like bench.py (median of 5 graph replays of ``launches`` launches), the LayerNorm's
    buffer sets rotated over >= 640 MiB.  Prints TFLOP/s against the 157.3 TFLOP/s
    dense fp32 matrix peak (2*M*N*K flops) or TB/s against 8 TB/s (x and y 4 bytes per element,
    w and b 4 bytes per column, mean and rstd 4 bytes per row)."""
    from . import lower_intent_to_hip_kernel  # noqa: PLC0415
    from .configs import layer_norm_persistent_ir, matmul_bias_relu2d_ir  # noqa: PLC0415
    from .runtime import launch_lowered  # noqa: PLC0415

    g = torch.Generator(device="cuda")
    g.manual_seed(17)
    if family == "matmul":
        b = {"M": 8192, "N": 8192, "K": 8192, **bindings}
        M, N, K = b["M"], b["N"], b["K"]
        ir = matmul_bias_relu2d_ir("f32")
        work, unit, peak = 2 * M * N * K, "TFLOP/s", 157.3e12
        nsets = 1
        mk = lambda: {"A": torch.randn((M, K), generator=g, device="cuda") / math.sqrt(K),  # noqa: E731
                      "B": torch.randn((K, N), generator=g, device="cuda"),
                      "bias": torch.randn((N,), generator=g, device="cuda") * 0.1,
                      "C": torch.empty((M, N), device="cuda")}
    else:
        b = {"M": 8192, "N": 4096, **bindings}
        M, N = b["M"], b["N"]
        ir = layer_norm_persistent_ir("f32")
        work, unit, peak = 8 * M * N + 8 * N + 8 * M, "TB/s", 8e12
        nsets = max(2, math.ceil(ROTATE_MIN_BYTES / work))
        mk = lambda: {"in_ptr": torch.randn((M, N), generator=g, device="cuda"),  # noqa: E731
                      "weight_ptr": 1 + 0.1 * torch.randn((N,), generator=g, device="cuda"),
                      "bias_ptr": 0.1 * torch.randn((N,), generator=g, device="cuda"),
                      "out_ptr": torch.empty((M, N), device="cuda"), "out_mean_ptr": torch.empty(M, device="cuda"),
                      "out_rstd_ptr": torch.empty(M, device="cuda")}
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    sets = [mk() for _ in range(nsets)]

    def launch(i):
        launch_lowered(k, sets[i % nsets])

    ms = _graph_time(launch, nsets, launches, torch)
    rate = work / (ms * 1e-3)
    print(f"[runner] f32 {family} {b}: {k.kernel_id}, {ms * 1e3:.1f} us/launch, {rate / 1e12:.2f} {unit} "
          f"({100 * rate / peak:.1f}% of peak)", flush=True)
    return 0


def _graph_time(launch, nsets, steps, torch) -> float:
    """Median over 5 replays of a graph of `steps` launches (launch(i) uses buffer set i % nsets),
    in ms per launch: the bench's timing, without launch gaps from the host."""
    import statistics  # noqa: PLC0415

    for i in range(max(nsets, 10)):
        launch(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph.capture_begin()
        for i in range(steps):
            launch(i)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(stream)
    graph.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(5):
        t0.record()
        graph.replay()
        t1.record()
        torch.cuda.synchronize()
        times.append(t0.elapsed_time(t1) / steps)
    return statistics.median(times)


def run_sweep(family, launches, torch) -> int:
    """Fixed cost and asymptotic rate of the softmax kernel against a plain copy of the same
    bytes.  For M = 2048 .. 65536 rows of 1024 f32 (read + write 8 KiB per row), both are timed
    like bench.py (graph replays of `launches` launches, buffer sets rotated over >= 640 MiB,
    median of 5) and each fitted as t = t0 + bytes / R by least squares: t0 is the per-launch
    cost that does not scale with the data (ramp-up of the first loads, drain of the last
    workgroups), R the streaming rate.  The copy is the identity element-wise program
    (ihip_elementwise_program, native code: one 16-byte load and store per lane)."""
    from . import lower_intent_to_hip_kernel  # noqa: PLC0415
    from .configs import softmax_inner_ir  # noqa: PLC0415
    from .runtime import ew_program_args, load_library  # noqa: PLC0415

    if family != "softmax":
        raise SystemExit(f"--sweep {family}: only softmax")
    import ctypes  # noqa: PLC0415

    lib = load_library()
    copy_ir = {"name": "copy2d", "tensors": {"x": _t("f32", "M", "N"), "y": _t("f32", "M", "N")},
               "ops": [_op("identity", ["x"], "y")], "outputs": ["y"]}
    rows = (2048, 4096, 8192, 16384, 32768, 65536)
    fits = {}
    for name, ir, xn, yn in (("softmax", softmax_inner_ir(), "input_ptr", "output_ptr"), ("copy", copy_ir, "x", "y")):
        pts = []
        for M in rows:
            b = {"M": M, "N": 1024}
            k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
            byt = 2 * 4 * M * 1024
            nsets = max(2, math.ceil(ROTATE_MIN_BYTES / byt))
            g = torch.Generator(device="cuda")
            g.manual_seed(M)
            sets = [(torch.randn((M, 1024), generator=g, device="cuda") * 2, torch.empty((M, 1024), device="cuda"))
                    for _ in range(nsets)]
            fn = getattr(lib, k.kernel_id)
            if k.kernel_id == "ihip_elementwise_program":
                prog = k.call_args[0][1]
                argv = []
                for x, y in sets:
                    a = ew_program_args(prog, {xn: x.data_ptr(), yn: y.data_ptr()}, {xn: "f32", yn: "f32"})
                    argv.append(a)
            else:
                argv = [[ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()), ctypes.c_int64(M),
                         ctypes.c_int64(1024)] for x, y in sets]

            def launch(i, fn=fn, argv=argv):
                a = argv[i % len(argv)]
                st = fn(*a[:8] if len(a) == 9 else a, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                if st != 0:
                    raise RuntimeError(lib.ihip_last_error().decode())

            ms = _graph_time(launch, nsets, launches, torch)
            pts.append((byt, ms * 1e-3))
            print(f"[runner] sweep {name} M={M}: {ms * 1e3:.2f} us, {byt / (ms * 1e-3) / 1e12:.2f} TB/s "
                  f"({100 * byt / (ms * 1e-3) / 8e12:.1f}% of 8 TB/s)", flush=True)
            del sets
            torch.cuda.empty_cache()
        n = len(pts)
        sx = sum(x for x, _ in pts)
        sy = sum(y for _, y in pts)
        sxx = sum(x * x for x, _ in pts)
        sxy = sum(x * y for x, y in pts)
        slope = (n * sxy - sx * sy) / (n * sxx - sx * sx)
        t0 = (sy - slope * sx) / n
        fits[name] = (t0, 1.0 / slope)
        print(f"[runner] sweep {name}: fixed {t0 * 1e6:.2f} us per launch, streaming rate {1e-12 / slope:.2f} TB/s "
              f"({100 / slope / 8e12:.1f}% of 8 TB/s)", flush=True)
    (t0s, rs), (t0c, rc) = fits["softmax"], fits["copy"]
    byt = 2 * 4 * 16384 * 1024
    print(f"[runner] at [16384, 1024]: softmax {1e6 * (t0s + byt / rs):.2f} us, copy {1e6 * (t0c + byt / rc):.2f} us; "
          f"without the fixed cost softmax would run at {100 * rs / 8e12:.1f}% of 8 TB/s", flush=True)
    return 0


# Row lengths behind the softmax's default rows per workgroup (rows.hip launch_softmax_reg).
SOFTMAX_ROWS_SHAPES = [(65536, 200), (65536, 256), (49152, 300), (43690, 384), (32768, 512), (21845, 768), (16777, 1000), (16384, 1024), (8192, 2048), (4096, 4096)]


def run_softmax_rows_sweep(launches, torch) -> int:
    """The measurement behind the softmax's default rows per workgroup: for rows held by one
    wave (N <= 4096), ihip_softmax_rows_f32_ex with rows_per_wg = 0 (the default: for N <= 1024
    four waves of two rows each, else four waves of one row) against the knob's 1, 2 and 4,
    timed like bench.py (graph replays of ``launches`` launches, buffer sets rotated over
    >= 640 MiB, median of 5)."""
    import ctypes  # noqa: PLC0415

    from .runtime import load_library  # noqa: PLC0415

    lib = load_library()
    P = ctypes.c_void_p
    for M, N in SOFTMAX_ROWS_SHAPES:
        byt = 2 * 4 * M * N
        nsets = max(2, math.ceil(ROTATE_MIN_BYTES / byt))
        g = torch.Generator(device="cuda")
        g.manual_seed(M + N)
        sets = [(torch.randn((M, N), generator=g, device="cuda") * 2, torch.empty((M, N), device="cuda"))
                for _ in range(nsets)]
        us = {}
        for rows in (0, 1, 2, 4):
            def launch(i, rows=rows):
                x, y = sets[i % nsets]
                st = lib.ihip_softmax_rows_f32_ex(P(x.data_ptr()), P(y.data_ptr()), M, N, rows,
                                                   P(torch.cuda.current_stream().cuda_stream))
                if st != 0:
                    raise RuntimeError(lib.ihip_last_error().decode())
            us[rows] = 1e3 * _graph_time(launch, nsets, launches, torch)
        best = min(us, key=us.get)
        row = ", ".join(f"{'default' if r == 0 else r} {t:.2f}" for r, t in us.items())
        print(f"[runner] softmax-rows [{M}, {N}]: {row} us; default {100 * byt / (us[0] * 1e-6) / 8e12:.1f}% of "
              f"8 TB/s, fastest {'default' if best == 0 else best}", flush=True)
        del sets
        torch.cuda.empty_cache()
    return 0


# Shapes behind the GEMM's shipped rules (M, N, K, B given as [N, K]).
GEMM_TILE_SHAPES = [
    (1000, 4096, 4096, False), (512, 8192, 8192, False), (2048, 2048, 8192, False), (1024, 1024, 8192, False),
    (256, 4096, 4096, False), (4096, 2048, 8192, False), (2048, 3072, 4096, False), (1536, 2048, 4096, True),
    (2304, 2816, 4096, True), (3072, 3072, 4096, False), (4096, 4096, 4096, True), (200, 32000, 4096, True),
    (32, 128256, 4096, True), (128, 128256, 4096, True), (16, 50257, 4096, True),
]
GEMM_SPLIT_SHAPES = [
    (1024, 1024, 8192, False), (512, 512, 16384, False), (768, 768, 16384, True), (256, 4096, 8192, False),
    (2048, 1024, 8192, False), (1000, 1000, 3000, False), (1536, 1280, 4096, False), (1024, 1024, 2048, False),
    (2048, 2048, 4096, False),
]
GEMM_SPLITS = (1, 2, 3, 4, 6, 8, 12, 16)


def _gemm_operands(M, N, K, tb, torch, g):
    a = (torch.randn((M, K), generator=g, device="cuda") / math.sqrt(K)).bfloat16()
    b = torch.randn((N, K) if tb else (K, N), generator=g, device="cuda").bfloat16()
    bias = torch.randn((N,), generator=g, device="cuda") * 0.1
    c = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
    return a, b, bias, c


def run_gemm_sweep(family, launches, torch) -> int:
    """The measurements behind two GEMM rules the library and the lowering ship, timed like
    bench.py (graph replays of ``launches`` launches, median of 5):

    gemm-tile: gemm_fast_tile_extent's choice between 256x256 and 128x128 C tiles, on grids of
    16-1024 tiles of 256x256 and on skinny vocabulary-width products; each shape runs with
    both tile knobs (ihip_gemm_bf16_bias_relu_ex, no workspace, so no split) and prints the
    rule's pick and the faster one.

    gemm-split: split_plan's segment count, on small grids; each shape runs unsplit and split
    into S = 2 .. 16 K segments (ihip_gemm_bf16_bias_relu_splitk) and prints the time of
    every S, the rule's S and the best S."""
    import ctypes  # noqa: PLC0415

    from .lowering import _gemm_tile_extent, gemm_split_plan  # noqa: PLC0415
    from .runtime import load_library  # noqa: PLC0415

    lib = load_library()
    P = ctypes.c_void_p
    g = torch.Generator(device="cuda")
    g.manual_seed(2024)

    def stream():
        return P(torch.cuda.current_stream().cuda_stream)

    def check(st):
        if st != 0:
            raise RuntimeError(lib.ihip_last_error().decode())

    if family == "gemm-tile":
        agree = 0
        for M, N, K, tb in GEMM_TILE_SHAPES:
            a, b, bias, c = _gemm_operands(M, N, K, tb, torch, g)
            us = {}
            for tile in (256, 128):
                def launch(i, tile=tile):
                    check(lib.ihip_gemm_bf16_bias_relu_ex(P(a.data_ptr()), P(b.data_ptr()), P(bias.data_ptr()),
                                                          P(c.data_ptr()), M, N, K, 0, int(tb), 1, tile, stream()))
                us[tile] = 1e3 * _graph_time(launch, 1, launches, torch)
            rule = _gemm_tile_extent(M, N)
            best = min(us, key=us.get)
            agree += rule == best
            t256 = -(-M // 256) * -(-N // 256)
            print(f"[runner] gemm-tile {M}x{N}x{K} B as {'[N, K]' if tb else '[K, N]'} ({t256} tiles of 256): "
                  f"256 {us[256]:.1f} us ({2 * M * N * K / us[256] / 1e6:.0f} TFLOP/s), 128 {us[128]:.1f} us "
                  f"({2 * M * N * K / us[128] / 1e6:.0f} TFLOP/s); rule {rule}, faster {best}", flush=True)
            del a, b, bias, c
        print(f"[runner] gemm-tile: the rule picks the faster tile on {agree} of {len(GEMM_TILE_SHAPES)} shapes",
              flush=True)
        return 0
    if family == "gemm-split":
        for M, N, K, tb in GEMM_SPLIT_SHAPES:
            a, b, bias, c = _gemm_operands(M, N, K, tb, torch, g)
            need = max(lib.ihip_gemm_splitk_workspace_size(M, N, K, S) for S in (*GEMM_SPLITS, 0))
            ws = torch.empty(max(1, need), dtype=torch.uint8, device="cuda")
            us = {}
            rule = gemm_split_plan(M, N, K)[0]
            for S in sorted(set(GEMM_SPLITS) | {rule}):
                if gemm_split_plan(M, N, K, S)[0] != S:
                    continue  # more segments than 64-k steps

                def launch(i, S=S):
                    check(lib.ihip_gemm_bf16_bias_relu_splitk(P(a.data_ptr()), P(b.data_ptr()), P(bias.data_ptr()),
                                                              P(c.data_ptr()), M, N, K, 0, int(tb), 1, 0, S,
                                                              P(ws.data_ptr()), need, stream()))
                us[S] = 1e3 * _graph_time(launch, 1, launches, torch)
            best = min(us, key=us.get)
            row = ", ".join(f"S={S} {t:.1f}" for S, t in us.items())
            print(f"[runner] gemm-split {M}x{N}x{K} B as {'[N, K]' if tb else '[K, N]'}: {row} us; rule S={rule} "
                  f"({us.get(rule, float('nan')):.1f} us), best S={best} ({us[best]:.1f} us)", flush=True)
            del a, b, bias, c, ws
        return 0
    raise SystemExit(f"--sweep {family}: unknown")


def run_gather(bindings, launches, torch) -> int:
    """gather(inp [M, N] f32, row [L] i32, col [L] i32) -> out [L] (ihip_gather2d_f32) with
    uniformly random in-range indices; algorithmic bytes 16 per element (two indices, one inp
    value, one output), index and output sets rotated over >= 640 MiB."""
    import statistics  # noqa: PLC0415

    from . import lower_intent_to_hip_kernel  # noqa: PLC0415
    from .runtime import launch_lowered  # noqa: PLC0415

    ir = {"name": "gather2d", "tensors": {"A": _t("f32", "M", "N"), "row": _t("i32", "L"), "col": _t("i32", "L"),
                                          "Out": _t("f32", "L")},
          "ops": [_op("gather", ["A", "row", "col"], "Out", other_value=0.0)], "outputs": ["Out"]}
    b = {"M": 8192, "N": 8192, "L": 1 << 24, **bindings}
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    per = 16 * b["L"]
    nsets = max(2, math.ceil(ROTATE_MIN_BYTES / (12 * b["L"])))
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    A = torch.randn((b["M"], b["N"]), generator=g, device="cuda")
    sets = [{"A": A, "row": torch.randint(0, b["M"], (b["L"],), generator=g, device="cuda", dtype=torch.int32),
             "col": torch.randint(0, b["N"], (b["L"],), generator=g, device="cuda", dtype=torch.int32),
             "Out": torch.empty(b["L"], device="cuda")} for _ in range(nsets)]
    for i in range(nsets):
        launch_lowered(k, sets[i])
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(5):
        t0.record()
        for i in range(launches):
            launch_lowered(k, sets[i % nsets])
        t1.record()
        torch.cuda.synchronize()
        times.append(t0.elapsed_time(t1) / launches)
    ms = statistics.median(times)
    print(f"[runner] gather {b}: {k.kernel_id}, {ms * 1e3:.1f} us/launch, {per / (ms * 1e-3) / 1e12:.2f} TB/s "
          f"algorithmic, {b['L'] / (ms * 1e-3) / 1e9:.2f} G elements/s", flush=True)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", choices=["any", "softmax", "layernorm", "gelu", "matmul"])
    ap.add_argument("--ew-chain", choices=sorted(EW_CHAINS) + ["all"],
                    help="time a generic element-wise program chain (or all of them)")
    ap.add_argument("--row-reduce", choices=["sum", "max"], help="time a row reduction (f32 [M, N], --bindings)")
    ap.add_argument("--gather", action="store_true", help="time gather2d (inp f32 [M, N], L random index pairs)")
    ap.add_argument("--sweep", choices=["softmax", "softmax-rows", "gemm-tile", "gemm-split"],
                    help="softmax: fixed cost and streaming rate against a copy of the same bytes; gemm-tile, "
                         "gemm-split: the measurements behind the GEMM's tile and split-K rules")
    ap.add_argument("--f32", choices=["matmul", "layernorm"],
                    help="time the reference's f32 IR of a family (default 8192^3 / [8192, 4096], --bindings)")
    ap.add_argument("--launches", type=int, default=20)
    ap.add_argument("--copy-mib", type=int, default=0)
    ap.add_argument("--bindings", default="", help="comma-separated SYMBOL=VALUE overrides, e.g. M=1000,N=4096")
    ap.add_argument("--transpose-b", action="store_true", help="matmul: B given as [N, K] (matmul{transpose_b})")
    ap.add_argument("--no-workspace", action="store_true",
                    help="pass an empty workspace (a GEMM that would be packed runs the guarded kernel, a long-row "
                         "softmax the workgroup-per-row kernel)")
    args = ap.parse_args(argv)
    if sum(x is not None for x in (args.config, args.ew_chain, args.row_reduce, args.f32, args.sweep)) + args.gather != 1:
        ap.error("give exactly one of --config, --ew-chain, --row-reduce, --f32, --sweep and --gather")
    if args.transpose_b and args.config != "matmul":
        ap.error("--transpose-b applies to --config matmul only")

    import torch

    if args.sweep:
        if args.sweep.startswith("gemm"):
            return run_gemm_sweep(args.sweep, args.launches, torch)
        if args.sweep == "softmax-rows":
            return run_softmax_rows_sweep(args.launches, torch)
        return run_sweep(args.sweep, args.launches, torch)
    if args.ew_chain:
        return run_ew_chains(sorted(EW_CHAINS) if args.ew_chain == "all" else [args.ew_chain], args.launches, torch)
    if args.row_reduce or args.gather or args.f32:
        rb = {n: int(v) for n, _, v in (item.partition("=") for item in filter(None, args.bindings.split(",")))}
        if args.f32:
            return run_f32(args.f32, rb, args.launches, torch)
        if args.gather:
            return run_gather(rb, args.launches, torch)
        return run_row_reduce(args.row_reduce, rb, args.launches, torch)

    from . import lower_intent_to_hip_kernel
    from .configs import WORKLOADS, algorithmic_bytes, gen_device
    from .runtime import launch_lowered, tensor_shapes, torch_dtype

    w = WORKLOADS[args.config]
    b = dict(w.bindings)
    for item in filter(None, args.bindings.split(",")):
        name, _, value = item.partition("=")
        if name not in b:
            ap.error(f"--bindings: {name!r} is not a symbol of {args.config} ({sorted(b)})")
        b[name] = int(value)
    ir = w.ir()
    if args.transpose_b:
        ir["tensors"]["B"]["shape"] = ["N", "K"]
        ir["ops"][0]["attrs"] = {"transpose_b": True}
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    if args.no_workspace and k.kernel_id == "ihip_softmax_rows_f32_ws":
        # the workspace entry rejects a split plan without room for it: the entry without one
        k = dataclasses.replace(k, kernel_id="ihip_softmax_rows_f32",
                                call_args=tuple(a for a in k.call_args if a[0] != "workspace"))
    elif args.no_workspace:
        k = dataclasses.replace(k, call_args=tuple(("workspace", 0) if kind == "workspace" else (kind, v)
                                                   for kind, v in k.call_args))
    shapes = tensor_shapes(k.io_spec, k.bindings)
    per = algorithmic_bytes(args.config, b)
    nsets = 1 if args.config in ("matmul", "gelu") else max(2, math.ceil(ROTATE_MIN_BYTES / per))
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    sets = []
    for _ in range(nsets):
        bufs = gen_device(args.config, b, torch, g)
        if args.transpose_b:  # same values, read as [N, K]
            bufs["B"] = bufs["B"].reshape(b["N"], b["K"])
        for n in k.output_names:
            bufs[n] = torch.empty(shapes[n], dtype=torch_dtype(k.io_spec["tensors"][n]["dtype"]), device="cuda")
        sets.append(bufs)
    torch.cuda.synchronize()
    for i in range(args.launches):
        launch_lowered(k, sets[i % nsets])
    torch.cuda.synchronize()
    print(f"[runner] {args.config}: {args.launches} launches of {k.kernel_id}, {nsets} buffer sets, "
          f"{per} algorithmic bytes per launch", flush=True)
    if args.copy_mib:
        n = (args.copy_mib << 20) // 4
        src = torch.randn(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[runner] calibration: 3 copies of {args.copy_mib} MiB", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
