"""Parity of the gfx950 kernels with the CPU oracle (restated verify/interpreter.py).

Every case lowers the IntentIR document through ``lower_intent_to_hip_kernel``,
runs it through the C-ABI (``run_hip_kernel``) and judges the outputs against
``oracle.interpreter.execute_intent`` on the same seeded inputs with the
reference pass/fail rule (``oracle.compare.compare_outputs`` =
verify/diff_runner.py:357-418).  Tolerances are the workload contract:

  reduce_any ........ bit-exact (bool)
  softmax f32 ....... rtol 1e-5, atol 1e-7
  LayerNorm f16 ..... y: rtol 1e-2, atol 1e-3 (the f16/bf16 floor of verify/tolerances.py:111-113);
                      mean/rstd: rtol 1e-5, atol 1e-7
  GELU chain bf16 ... rtol 1e-2, atol 1e-3 (same floor); plus a strict rtol 1e-2, atol 1e-6 check
  GEMM bf16 ......... rtol 2e-2, atol 2e-2 (verify/tolerances.py:44); plus a strict atol 1e-4 check

Small shapes use the reference's edge sizes (verify/gen_cases.py:27).  At the full
workload sizes every output is checked in full against the oracle (the GEMM and the
GELU chain in blocks of rows), and the GEMM and GELU also against a float32 torch
evaluation of the same formula; size-independent properties (softmax row sums,
LayerNorm shift invariance) on top.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from intent_ir_amd import lower_intent_to_hip_kernel, run_lowered
from intent_ir_amd.configs import WORKLOADS, bias_gelu_axpy_ir, matmul_bias_relu2d_ir
from intent_ir_amd.lowering import gemm_pack_bytes, gemm_split_plan, gemm_workspace_bytes
from intent_ir_amd.dtypes import bf16_bits_to_f32, f32_to_bf16_bits, to_compute_f32
from intent_ir_amd.ir import as_intent
from oracle.compare import compare_outputs
from oracle.interpreter import execute_intent

pytestmark = pytest.mark.gpu

EDGE = [1, 2, 3, 7, 8, 15, 16, 17, 31, 32, 33]  # verify/gen_cases.py:27

TOL = {
    "softmax": {"atol": 1e-7, "rtol": 1e-5},
    "ln_y": {"atol": 1e-3, "rtol": 1e-2},
    "ln_stats": {"atol": 1e-7, "rtol": 1e-5},
    "gelu": {"atol": 1e-3, "rtol": 1e-2},
    "gelu_strict": {"atol": 1e-6, "rtol": 1e-2},
    "matmul": {"atol": 2e-2, "rtol": 2e-2},
    "matmul_strict": {"atol": 1e-4, "rtol": 2e-2},
}


def oracle_outputs(ir: dict, inputs: dict, bindings: dict) -> dict:
    fn = as_intent(ir)
    f32 = {n: to_compute_f32(v, fn.tensors[n].dtype) for n, v in inputs.items()}
    return execute_intent(ir, f32, bindings)


def run_case(ir: dict, inputs: dict, bindings: dict) -> dict:
    k = lower_intent_to_hip_kernel(ir, shape_bindings=bindings)
    print(f"[case] {k.kernel_id} bindings={bindings}", flush=True)
    return run_lowered(k, inputs)


def check(pred, ref, names, tol, what=""):
    d = compare_outputs(pred, ref, names, tol)
    assert d.ok, f"{what}: {d.summary} at {d.first_bad_index} (max_abs={d.max_abs_err:.3g} max_rel={d.max_rel_err:.3g})"
    return d


# ------------------------------------------------------------------ reduce_any
@pytest.mark.parametrize("M", [1, 3, 17, 33])
@pytest.mark.parametrize("N", EDGE + [64, 255, 256, 1023, 4096, 4099, 4100, 65537])
def test_reduce_any_edge_shapes(hip, M, N):
    w = WORKLOADS["any"]
    b = {"M": M, "N": N}
    rng = np.random.default_rng(M * 1000 + N)
    x = np.zeros((M, N), np.float32)
    x[rng.random((M, N)) < 0.05] = 1.5
    inp = {"inp": x}
    out = run_case(w.ir(), inp, b)
    ref = oracle_outputs(w.ir(), inp, b)
    assert out["out"].dtype == np.bool_
    np.testing.assert_array_equal(out["out"], ref["out"])


def test_reduce_any_special_values(hip):
    """-0.0 counts as zero, NaN/inf/denormals as non-zero (np.any semantics)."""
    w = WORKLOADS["any"]
    M, N = 8, 4096
    x = np.zeros((M, N), np.float32)
    x[1, 4095] = -0.0
    x[2, 0] = np.nan
    x[3, 17] = np.inf
    x[4, 2048] = np.float32(1e-45)  # smallest denormal
    x[5, 100] = -np.float32(1e-45)
    x[6, :] = -0.0
    x[7, 5] = -3.0
    out = run_case(w.ir(), {"inp": x}, {"M": M, "N": N})
    np.testing.assert_array_equal(out["out"], np.any(x != 0, axis=1))
    assert out["out"].tolist() == [False, False, True, True, True, True, False, True]


@pytest.mark.parametrize("M,N", [(1, 16), (3, 4096), (17, 4112), (33, 17), (5, 4100), (2, 65536), (300, 1024),
                                 (4, 15), (7, 1), (64, 16385), (9, 20001)])
def test_reduce_any_bool_input(hip, M, N):
    """reduce_any over an i1 tensor (interpreter.py:489-494): 16-byte words over each row's
    aligned body, a head and tail of < 16 bytes when rows do not start 16-byte aligned (N % 16
    != 0); rows with a single true at either end."""
    ir = {"name": "anyb", "tensors": {"x": {"dtype": "i1", "shape": ["M", "N"]}, "out": {"dtype": "i1", "shape": ["M"]}},
          "ops": [{"op": "reduce_any", "inputs": ["x"], "output": "out", "attrs": {"dims": [1]}}], "outputs": ["out"]}
    rng = np.random.default_rng(M * 31 + N)
    x = rng.random((M, N)) < 2.0 / N
    x[0, :] = False
    if M > 1:
        x[1, :] = False
        x[1, N - 1] = True
    if M > 2:
        x[2, :] = False
        x[2, 0] = True
    out = run_case(ir, {"x": x}, {"M": M, "N": N})
    np.testing.assert_array_equal(out["out"], oracle_outputs(ir, {"x": x}, {"M": M, "N": N})["out"])
    np.testing.assert_array_equal(out["out"], x.any(axis=1))


@pytest.mark.parametrize("N", [1, 15, 16, 17, 31, 64, 129, 1000, 1023, 1025, 16401])
@pytest.mark.parametrize("off", [0, 1, 7, 15])
def test_reduce_any_bool_at_every_alignment(hip, N, off):
    """Through the C-ABI with x placed off bytes past a 256-byte aligned base: each row's head,
    body and tail move with the offset; a single true byte at every position class (head, body,
    tail) of some row, and rows of all zeros, give exactly numpy's any."""
    import ctypes

    import torch

    M = 48
    x = np.zeros((M, N), dtype=np.uint8)
    for r in range(1, M, 2):
        x[r, (r * 7919) % N] = 1 + (r % 5)  # any non-zero byte counts as true
    x[2, 0] = 1
    x[4, N - 1] = 1
    buf = torch.zeros(M * N + off, dtype=torch.uint8, device="cuda")
    buf[off:] = torch.from_numpy(x.reshape(-1)).cuda()
    out = torch.full((M,), 9, dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    print(f"[case] reduce_any_rows_u8 N={N} offset={off}", flush=True)
    assert hip.ihip_reduce_any_rows_u8(ctypes.c_void_p(buf.data_ptr() + off), ctypes.c_void_p(out.data_ptr()), M, N,
                                       ctypes.c_void_p(s)) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), (x != 0).any(axis=1).astype(np.uint8))


@pytest.mark.parametrize("N", [1, 3, 4, 5, 63, 64, 65, 255, 256, 1023, 1025])
@pytest.mark.parametrize("off", [0, 1, 3])
@pytest.mark.parametrize("c", [0.0, 1.0])
def test_reduce_any_f32_short_rows(hip, N, off, c):
    """Rows of at most 64 16-byte vectors run several per wave (4-32 lanes per row); through the
    C-ABI with x placed off floats past an aligned base, rows equal to c everywhere but one
    position (head, body or tail of the row), rows of -0.0 (equal to 0), NaN, against numpy."""
    import ctypes

    import torch

    M = 77
    x = np.full((M, N), c, dtype=np.float32)
    if c == 0.0:
        x[1::4] = -0.0
    for r in range(2, M, 3):
        x[r, (r * 131) % N] = 2.5 if r % 2 else np.nan
    x[5, 0] = -7.0
    x[8, N - 1] = 1e-45
    buf = torch.zeros(M * N + off, dtype=torch.float32, device="cuda")
    buf[off:] = torch.from_numpy(x.reshape(-1)).cuda()
    out = torch.full((M,), 9, dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    print(f"[case] reduce_any_rows_f32 N={N} offset={off} c={c}", flush=True)
    assert hip.ihip_reduce_any_rows_f32(ctypes.c_void_p(buf.data_ptr() + 4 * off), ctypes.c_void_p(out.data_ptr()), M,
                                        N, ctypes.c_float(c), ctypes.c_void_p(s)) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), (x != np.float32(c)).any(axis=1).astype(np.uint8))


def test_reduce_any_ne_form_with_nonzero_constant(hip):
    """`const, ne, reduce_any` form (tests/backends/cuda/test_cuda_backend_smoke.py:249-267) with c != 0."""
    ir = {
        "name": "any_ne", "tensors": {"A": {"dtype": "f32", "shape": ["M", "N"]}, "z": {"dtype": "f32", "shape": []},
                                      "T": {"dtype": "i1", "shape": ["M", "N"]}, "Out": {"dtype": "i1", "shape": ["M"]}},
        "ops": [{"op": "const", "inputs": [], "output": "z", "attrs": {"value": 1.0}},
                {"op": "ne", "inputs": ["A", "z"], "output": "T"},
                {"op": "reduce_any", "inputs": ["T"], "output": "Out", "attrs": {"dims": [1]}}],
        "outputs": ["Out"],
    }
    rng = np.random.default_rng(0)
    A = rng.integers(0, 2, size=(33, 257)).astype(np.float32)
    A[::3] = 1.0
    out = run_case(ir, {"A": A}, {"M": 33, "N": 257})
    np.testing.assert_array_equal(out["Out"], oracle_outputs(ir, {"A": A}, {"M": 33, "N": 257})["Out"])


def test_reduce_any_full_config(hip):
    w = WORKLOADS["any"]
    inp = w.gen(w.bindings)
    out = run_case(w.ir(), inp, w.bindings)
    ref = oracle_outputs(w.ir(), inp, w.bindings)
    np.testing.assert_array_equal(out["out"], ref["out"])
    assert 0.2 < out["out"].mean() < 0.5  # ~33% of rows hold a Bernoulli(1e-4) hit


# ------------------------------------------------------------------ row reduce_sum / reduce_max
def _row_reduce_ir(op: str) -> dict:
    return {"name": f"row_{op}", "tensors": {"x": {"dtype": "f32", "shape": ["M", "N"]},
                                             "out": {"dtype": "f32", "shape": ["M"]}},
            "ops": [{"op": op, "inputs": ["x"], "output": "out", "attrs": {"dims": [1]}}], "outputs": ["out"]}


ROW_REDUCE_SHAPES = ([(m, n) for m in (1, 3, 17) for n in EDGE + [64, 255, 256, 1023, 1025, 4096, 4100, 65536]]
                     + [(2048, 256), (2048, 4100), (4096, 1024), (1000, 2048), (2048, 4099), (64, 65537),
                        (65536, 32), (20001, 61), (100, 257), (3000, 512), (77, 515)])


@pytest.mark.parametrize("op", ["reduce_sum", "reduce_max"])
@pytest.mark.parametrize("M,N", ROW_REDUCE_SHAPES)
def test_row_reduce_edge_shapes(hip, op, M, N):
    """reduce_sum / reduce_max over the last axis (interpreter.py:478-500): sums within rtol 1e-5
    (a different f32 summation order than numpy's pairwise one), maxima bit-exact.  Covers the
    wave-per-row and 16-waves-per-row forms, with rows that start at every alignment (N % 4 != 0:
    a head and tail of < 4 elements around the 16-byte body)."""
    ir = _row_reduce_ir(op)
    b = {"M": M, "N": N}
    x = np.random.default_rng(M * 7 + N).standard_normal((M, N)).astype(np.float32)
    out = run_case(ir, {"x": x}, b)["out"]
    ref = oracle_outputs(ir, {"x": x}, b)["out"]
    if op == "reduce_max":
        np.testing.assert_array_equal(out, ref)
    else:
        check({"out": out}, {"out": ref}, ["out"], {"atol": 1e-4, "rtol": 1e-5}, f"{op} {b}")


@pytest.mark.parametrize("N", [7, 8, 4096, 4099, 4100])
def test_row_reduce_special_values(hip, N):
    """NaN propagates through both; inf and -inf as in numpy (inf + -inf = NaN); a row of -0.0
    sums to +0.0 (numpy's add.reduce starts from +0.0) and has max -0.0; an empty row sums to
    +0.0."""
    M = 6
    x = np.ones((M, N), np.float32)
    x[0, N // 2] = np.nan
    x[1, N - 1] = np.inf
    x[2, 0] = -np.inf
    x[3, 1], x[3, N - 2] = np.inf, -np.inf
    x[4, :] = -0.0
    x[5, :] = -3.0
    for op in ("reduce_sum", "reduce_max"):
        out = run_case(_row_reduce_ir(op), {"x": x}, {"M": M, "N": N})["out"]
        ref = x.sum(axis=1) if op == "reduce_sum" else x.max(axis=1)
        np.testing.assert_array_equal(out, ref.astype(np.float32))
        assert np.signbit(out[4]) == np.signbit(ref[4]), f"{op} of a -0.0 row: sign of zero as numpy"
    empty = run_case(_row_reduce_ir("reduce_sum"), {"x": np.zeros((3, 0), np.float32)}, {"M": 3, "N": 0})["out"]
    assert empty.tolist() == [0.0, 0.0, 0.0] and not np.signbit(empty).any()


def test_row_reduce_full_size(hip):
    """[8192, 4096] f32, the reduce_any workload's shape: sums against the oracle."""
    ir = _row_reduce_ir("reduce_sum")
    b = {"M": 8192, "N": 4096}
    x = np.random.default_rng(5).standard_normal((8192, 4096)).astype(np.float32)
    check(run_case(ir, {"x": x}, b), oracle_outputs(ir, {"x": x}, b), ["out"], {"atol": 1e-4, "rtol": 1e-5}, "sum full")


# ------------------------------------------------------------------ softmax
@pytest.mark.parametrize("M", [1, 7, 33])
@pytest.mark.parametrize("N", EDGE + [4, 12, 64, 100, 128, 132, 256, 1000, 1001, 1024, 1025, 4096, 4097, 4100, 5000, 8191,
                                      8192, 8196, 16384, 32000, 32768, 50257, 65535, 65536, 65537, 65540])
def test_softmax_edge_shapes(hip, M, N):
    """N % 4 == 0: one wave per row up to N = 4096, 2-16 waves per row up to 65536 (4100, 8196:
    the first size past a form's capacity).  N % 4 != 0: the row in registers through 4-byte
    loads up to 65535 (1025, 4097: past a form's capacity).  The three-pass kernel beyond."""
    w = WORKLOADS["softmax"]
    b = {"M": M, "N": N}
    inp = w.gen(b, seed=M + N)
    check(run_case(w.ir(), inp, b), oracle_outputs(w.ir(), inp, b), ["output_ptr"], TOL["softmax"], f"softmax {b}")


@pytest.mark.parametrize("M,N", [(65536, 64), (100003, 32), (4099, 128), (777, 4), (65537, 31), (3001, 127), (999, 1),
                                 (20000, 99)])
def test_softmax_many_short_rows(hip, M, N):
    """Rows of at most 128 floats run several per wave (N / 4 rounded up to a power of two lanes
    each for N % 4 == 0, up to 4 elements per lane otherwise): many rows, row counts that leave
    a partial wave, against the oracle."""
    w = WORKLOADS["softmax"]
    b = {"M": M, "N": N}
    inp = w.gen(b, seed=M + N)
    check(run_case(w.ir(), inp, b), oracle_outputs(w.ir(), inp, b), ["output_ptr"], TOL["softmax"], f"softmax {b}")


def test_softmax_expanded_chain_form(hip):
    """reduce_max, sub, exp, reduce_sum, div (tests/test_diff_runner.py:73-101) lowers to the same kernel."""
    ir = {
        "name": "softmax_like",
        "tensors": {n: {"dtype": "f32", "shape": s} for n, s in
                    {"X": ["M", "N"], "mx": ["M"], "Xc": ["M", "N"], "E": ["M", "N"], "sm": ["M"], "out": ["M", "N"]}.items()},
        "ops": [{"op": "reduce_max", "inputs": ["X"], "output": "mx", "attrs": {"axis": [1], "keepdims": False}},
                {"op": "sub", "inputs": ["X", "mx"], "output": "Xc"},
                {"op": "exp", "inputs": ["Xc"], "output": "E"},
                {"op": "reduce_sum", "inputs": ["E"], "output": "sm", "attrs": {"axis": [1], "keepdims": False}},
                {"op": "div", "inputs": ["E", "sm"], "output": "out"}],
        "outputs": ["out"],
    }
    b = {"M": 64, "N": 1024}
    X = WORKLOADS["softmax"].gen(b)["input_ptr"]
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    assert k.kernel_id == "ihip_softmax_rows_f32"
    check(run_lowered(k, {"X": X}), oracle_outputs(ir, {"X": X}, b), ["out"], TOL["softmax"], "softmax chain")


def test_softmax_full_config(hip):
    w = WORKLOADS["softmax"]
    inp = w.gen(w.bindings)
    out = run_case(w.ir(), inp, w.bindings)
    check(out, oracle_outputs(w.ir(), inp, w.bindings), ["output_ptr"], TOL["softmax"], "softmax full")
    np.testing.assert_allclose(out["output_ptr"].astype(np.float64).sum(axis=1), 1.0, rtol=0, atol=1e-5)


# ------------------------------------------------------------------ LayerNorm
LN_OUTS = ["out_ptr", "out_mean_ptr", "out_rstd_ptr"]


def _check_ln(out, ref, what):
    check(out, ref, ["out_ptr"], TOL["ln_y"], what + " y")
    check(out, ref, ["out_mean_ptr", "out_rstd_ptr"], TOL["ln_stats"], what + " stats")


@pytest.mark.parametrize("M", [1, 3, 17, 777])
@pytest.mark.parametrize("N", EDGE + [64, 100, 120, 129, 255, 256, 257, 264, 1000, 1024, 4096, 4104, 8192, 8200, 16384,
                                      20000, 65536, 65544, 65545, 100000, 100003, 262144])
def test_layernorm_edge_shapes(hip, M, N):
    """One wave per row up to N = 4096; 2-16 waves per row up to 65536 (rows per workgroup
    16 / waves, so M = 17 leaves waves past the last row); beyond, a 1024-thread workgroup per
    row with 16-byte accesses (N % 8 == 0) or 2-byte ones (65545, 100003)."""
    w = WORKLOADS["layernorm"]
    b = {"M": M, "N": N}
    inp = w.gen(b, seed=M * 7 + N)
    _check_ln(run_case(w.ir(), inp, b), oracle_outputs(w.ir(), inp, b), f"LN {b}")


@pytest.mark.parametrize("M", [3, 64])
@pytest.mark.parametrize("N", [4097, 4099, 4103, 5000 + 3, 8191, 12345, 32767, 50257, 65535])
def test_layernorm_rows_not_16_byte_aligned(hip, M, N):
    """N % 8 != 0: each row splits into a head of < 8 halves, a 16-byte aligned body held in
    registers and a tail of < 8 halves (1-16 waves per row), at every row alignment."""
    w = WORKLOADS["layernorm"]
    b = {"M": M, "N": N}
    inp = w.gen(b, seed=M + N)
    _check_ln(run_case(w.ir(), inp, b), oracle_outputs(w.ir(), inp, b), f"LN {b}")


@pytest.mark.parametrize("N", [33, 200, 1000, 4099, 8200, 70000])
@pytest.mark.parametrize("ox,oy,ow", [(1, 1, 0), (3, 3, 0), (7, 7, 0), (1, 2, 0), (0, 5, 0), (3, 3, 1), (0, 0, 3)])
def test_layernorm_at_every_alignment(hip, N, ox, oy, ow):
    """Through the C-ABI with x and y offset by ox, oy halves from a 16-byte boundary: equal
    offsets take the head/body/tail form (up to 65543 halves), unequal ones (and N = 70000 at
    any offset) the workgroup-per-row kernel with 2-byte accesses; w and b offset by ow halves
    are read element by element instead of as realigned 16-byte vectors.  All against the
    oracle."""
    import ctypes

    import torch

    w = WORKLOADS["layernorm"]
    M = 5
    inp = w.gen({"M": M, "N": N}, seed=N + ox)
    xs = torch.zeros(M * N + 16, dtype=torch.float16, device="cuda")
    ys = torch.zeros(M * N + 16, dtype=torch.float16, device="cuda")
    xs[ox:ox + M * N] = torch.from_numpy(inp["in_ptr"].reshape(-1)).cuda()
    wt = torch.zeros(N + 8, dtype=torch.float16, device="cuda")
    bt = torch.zeros(N + 8, dtype=torch.float16, device="cuda")
    wt[ow:ow + N] = torch.from_numpy(inp["weight_ptr"]).cuda()
    bt[ow:ow + N] = torch.from_numpy(inp["bias_ptr"]).cuda()
    mean = torch.empty(M, device="cuda")
    rstd = torch.empty(M, device="cuda")
    st = hip.ihip_layernorm_rows_f16(ctypes.c_void_p(xs.data_ptr() + 2 * ox), ctypes.c_void_p(wt.data_ptr() + 2 * ow),
                                     ctypes.c_void_p(bt.data_ptr() + 2 * ow), ctypes.c_void_p(ys.data_ptr() + 2 * oy),
                                     ctypes.c_void_p(mean.data_ptr()), ctypes.c_void_p(rstd.data_ptr()), M, N,
                                     ctypes.c_float(1e-5), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, hip.ihip_last_error()
    torch.cuda.synchronize()
    out = {"out_ptr": ys[oy:oy + M * N].cpu().numpy().reshape(M, N).astype(np.float32),
           "out_mean_ptr": mean.cpu().numpy(), "out_rstd_ptr": rstd.cpu().numpy()}
    _check_ln(out, oracle_outputs(w.ir(), inp, {"M": M, "N": N}), f"LN N={N} offsets {ox},{oy}")
    assert (ys[:oy] == 0).all() and (ys[oy + M * N:] == 0).all(), "writes outside y"


@pytest.mark.parametrize("N", [512, 1024, 2048, 4096])
def test_layernorm_exact_and_tail_paths_agree(hip, N):
    """Rows per workgroup: M % 16 == 0 with full-width rows takes the unmasked kernel, M = 31 the
    masked one (its last workgroup has a wave past the last row).  Shared rows must be identical."""
    w = WORKLOADS["layernorm"]
    inp = w.gen({"M": 32, "N": N}, seed=N)
    full = run_case(w.ir(), inp, {"M": 32, "N": N})
    part_in = dict(inp, in_ptr=np.ascontiguousarray(inp["in_ptr"][:31]))
    part = run_case(w.ir(), part_in, {"M": 31, "N": N})
    for name in ("out_ptr", "out_mean_ptr", "out_rstd_ptr"):
        np.testing.assert_array_equal(part[name], full[name][:31], err_msg=name)
    _check_ln(full, oracle_outputs(w.ir(), inp, {"M": 32, "N": N}), f"LN exact N={N}")
    _check_ln(part, oracle_outputs(w.ir(), part_in, {"M": 31, "N": N}), f"LN tail N={N}")


def test_layernorm_full_config(hip):
    w = WORKLOADS["layernorm"]
    inp = w.gen(w.bindings)
    _check_ln(run_case(w.ir(), inp, w.bindings), oracle_outputs(w.ir(), inp, w.bindings), "LN full")


def test_layernorm_shift_invariance(hip):
    """verify/metamorphic.py:409-482: y and rstd unchanged, mean shifted, for x + c (c exact in f16)."""
    w = WORKLOADS["layernorm"]
    b = {"M": 64, "N": 4096}
    inp = w.gen(b)
    base = run_case(w.ir(), inp, b)
    shifted = dict(inp, in_ptr=(inp["in_ptr"].astype(np.float32) + 4.0).astype(np.float16))
    exact = shifted["in_ptr"].astype(np.float32) - 4.0 == inp["in_ptr"].astype(np.float32)
    rows = exact.all(axis=1)
    out = run_case(w.ir(), shifted, b)
    np.testing.assert_allclose(out["out_rstd_ptr"][rows], base["out_rstd_ptr"][rows], rtol=1e-4)
    np.testing.assert_allclose(out["out_mean_ptr"][rows], base["out_mean_ptr"][rows] + 4.0, rtol=0, atol=1e-5)
    np.testing.assert_allclose(out["out_ptr"][rows].astype(np.float32), base["out_ptr"][rows].astype(np.float32),
                               rtol=1e-2, atol=4e-3)


def test_layernorm_reference_naming_variant(hip):
    """The reference CUDA lowering needs outputs named Y/Mean/Rstd (intentir_to_cuda.py:2163); any names lower here."""
    ir = WORKLOADS["layernorm"].ir()
    ren = {"out_ptr": "Y", "out_mean_ptr": "Mean", "out_rstd_ptr": "Rstd"}
    ir["tensors"] = {ren.get(k, k): v for k, v in ir["tensors"].items()}
    for op in ir["ops"]:
        op["output"] = ren.get(op["output"], op["output"])
    ir["outputs"] = ["Mean", "Y", "Rstd"]
    b = {"M": 33, "N": 1024}
    inp = WORKLOADS["layernorm"].gen(b)
    out = run_case(ir, inp, b)
    ref = oracle_outputs(ir, inp, b)
    check(out, ref, ["Y"], TOL["ln_y"], "LN renamed")
    check(out, ref, ["Mean", "Rstd"], TOL["ln_stats"], "LN renamed stats")


# ------------------------------------------------------------------ GELU chain
@pytest.mark.parametrize("M", [1, 3, 17])
@pytest.mark.parametrize("N", EDGE + [64, 1000, 8192])
def test_gelu_edge_shapes(hip, M, N):
    w = WORKLOADS["gelu"]
    b = {"M": M, "N": N}
    inp = w.gen(b, seed=M * 13 + N)
    out = run_case(w.ir(), inp, b)
    ref = oracle_outputs(w.ir(), inp, b)
    check(out, ref, ["y"], TOL["gelu"], f"gelu {b}")
    check(out, ref, ["y"], TOL["gelu_strict"], f"gelu strict {b}")


def test_gelu_matches_tanh_form(hip):
    """y = 0.5*(0.5*z*(1+tanh(sqrt(2/pi)(z+0.044715 z^3)))) + x computed with math.tanh in float64."""
    w = WORKLOADS["gelu"]
    b = {"M": 16, "N": 512}
    x = np.linspace(-8, 8, 16 * 512, dtype=np.float32).reshape(16, 512)
    bias = np.linspace(-0.1, 0.1, 512, dtype=np.float32)
    inp = {"x": f32_to_bf16_bits(x), "bias": f32_to_bf16_bits(bias)}
    out = run_case(w.ir(), inp, b)["y"].astype(np.float64)
    xf, bf = bf16_bits_to_f32(inp["x"]).astype(np.float64), bf16_bits_to_f32(inp["bias"]).astype(np.float64)
    z = xf + bf
    gelu = np.vectorize(lambda v: 0.5 * v * (1.0 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3))))(z)
    np.testing.assert_allclose(out, 0.5 * gelu + xf, rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("M,N", [(100001, 64), (4097, 8), (777, 120), (20000, 264), (3, 2048), (5, 2056)])
def test_gelu_short_and_ragged_rows(hip, M, N):
    """Rows of fewer than 256 16-byte vectors share a workgroup (N / 8 rounded up to a power of
    two lanes per row, 256 / lanes rows per workgroup), with row counts that leave partial
    groups; checked in full against the oracle."""
    w = WORKLOADS["gelu"]
    b = {"M": M, "N": N}
    inp = w.gen(b, seed=M + N)
    out = run_case(w.ir(), inp, b)
    ref = oracle_outputs(w.ir(), inp, b)
    check(out, ref, ["y"], TOL["gelu"], f"gelu {b}")
    check(out, ref, ["y"], TOL["gelu_strict"], f"gelu strict {b}")


@pytest.mark.parametrize("M,N", [(72, 2048), (256, 64), (64, 8)])
def test_gelu_exact_tiling_matches_the_guarded_path(hip, M, N):
    """When the grid tiles the tensor exactly the kernel drops its row guards and addresses rows
    from a uniform base; one more row sends the same rows through the guarded loop.  Both
    against the oracle, and bit for bit against each other on the shared rows."""
    w = WORKLOADS["gelu"]
    big = {"M": M + 1, "N": N}
    inp = w.gen(big, seed=M * 7 + N)
    sub = {"x": inp["x"][:M], "bias": inp["bias"]}
    b = {"M": M, "N": N}
    out_exact = run_case(w.ir(), sub, b)["y"]
    out_guarded = run_case(w.ir(), inp, big)["y"]
    assert np.array_equal(out_exact, out_guarded[:M])
    ref = oracle_outputs(w.ir(), sub, b)
    check({"y": out_exact}, ref, ["y"], TOL["gelu_strict"], f"gelu exact {b}")


def test_gelu_full_config(hip):
    import torch

    w = WORKLOADS["gelu"]
    inp = w.gen(w.bindings)
    out = run_case(w.ir(), inp, w.bindings)["y"]
    # every row against the oracle, in blocks of 1024 rows (the chain is row-independent; blocks
    # keep numpy's temporaries at 32 MiB, where the whole tensor's take minutes)
    blk = 1024
    for r0 in range(0, w.bindings["M"], blk):
        rows = slice(r0, min(r0 + blk, w.bindings["M"]))
        sub = {"x": inp["x"][rows], "bias": inp["bias"]}
        sb = {"M": rows.stop - rows.start, "N": w.bindings["N"]}
        ref = oracle_outputs(w.ir(), sub, sb)
        check({"y": out[rows]}, ref, ["y"], TOL["gelu"], f"gelu full rows {r0}+")
        check({"y": out[rows]}, ref, ["y"], TOL["gelu_strict"], f"gelu full rows {r0}+ strict")
    # whole tensor against a float32 torch evaluation of the same formula
    xt = torch.from_numpy(bf16_bits_to_f32(inp["x"])).cuda()
    bt = torch.from_numpy(bf16_bits_to_f32(inp["bias"])).cuda()
    z = xt + bt
    g = z / (1.0 + torch.exp(-2.0 * math.sqrt(2.0 / math.pi) * (z + 0.044715 * z * z * z)))
    yref = (0.5 * g + xt).cpu().numpy()
    np.testing.assert_allclose(out, yref, rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("N", [31, 127, 1029, 4099, 8195, 50257, 65533])
@pytest.mark.parametrize("ox,oy", [(0, 0), (1, 1), (2, 2), (3, 3), (1, 2), (0, 3)])
def test_softmax_odd_rows_at_every_alignment(hip, N, ox, oy):
    """N % 4 != 0 through the C-ABI with x and y placed ox, oy floats past 256-byte aligned
    allocations: equal offsets take the head / aligned body / tail kernel (every row starts at
    another alignment), unequal ones the 4-byte-load kernel.  Judged against the oracle."""
    import ctypes

    import torch

    w = WORKLOADS["softmax"]
    out = w.ir()["outputs"][0]
    M = 7
    b = {"M": M, "N": N}
    inp = w.gen(b, seed=N + 10 * ox + oy)
    xt = torch.empty(M * N + ox, dtype=torch.float32, device="cuda")
    xt[ox:] = torch.from_numpy(inp["input_ptr"].reshape(-1)).cuda()
    yt = torch.full((M * N + oy + 4,), 7.0, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    print(f"[case] softmax odd rows N={N} ox={ox} oy={oy}", flush=True)
    st = hip.ihip_softmax_rows_f32(ctypes.c_void_p(xt.data_ptr() + 4 * ox), ctypes.c_void_p(yt.data_ptr() + 4 * oy),
                                   M, N, ctypes.c_void_p(s))
    assert st == 0, hip.ihip_last_error().decode()
    torch.cuda.synchronize()
    yh = yt.cpu().numpy()
    assert (yh[:oy] == 7.0).all() and (yh[oy + M * N:] == 7.0).all(), "write outside y"
    ref = oracle_outputs(w.ir(), inp, b)
    check({out: yh[oy:oy + M * N].reshape(M, N)}, ref, [out], TOL["softmax"], f"softmax N={N} {ox},{oy}")


@pytest.mark.parametrize("kind,N", [("softmax", 31), ("softmax", 97), ("layernorm", 33), ("layernorm", 200)])
@pytest.mark.parametrize("ox,oy", [(0, 0), (1, 2), (3, 3), (2, 7)])
def test_short_rows_staged_in_lds_at_offsets(hip, kind, N, ox, oy):
    """Short rows of other lengths are staged through LDS a workgroup's rows at a time (16-byte
    accesses from each block's own offset modulo 16 bytes; y rewritten in place when x and y share
    it, after a barrier otherwise): 3001 rows (many workgroups, a partial last one) with x and y
    placed ox, oy elements past aligned allocations, against the oracle, with nothing written
    outside y."""
    import ctypes

    import torch

    w = WORKLOADS[kind]
    M = 3001
    b = {"M": M, "N": N}
    inp = w.gen(b, seed=N + 10 * ox + oy)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"[case] staged short rows {kind} N={N} ox={ox} oy={oy}", flush=True)
    if kind == "softmax":
        ox, oy = ox % 4, oy % 4  # floats: offsets within one 16-byte vector
        xt = torch.empty(M * N + ox, dtype=torch.float32, device="cuda")
        xt[ox:] = torch.from_numpy(inp["input_ptr"].reshape(-1)).cuda()
        yt = torch.full((M * N + oy + 4,), 7.0, dtype=torch.float32, device="cuda")
        st = hip.ihip_softmax_rows_f32(ctypes.c_void_p(xt.data_ptr() + 4 * ox), ctypes.c_void_p(yt.data_ptr() + 4 * oy),
                                       M, N, s)
        assert st == 0, hip.ihip_last_error().decode()
        torch.cuda.synchronize()
        yh = yt.cpu().numpy()
        assert (yh[:oy] == 7.0).all() and (yh[oy + M * N:] == 7.0).all(), "write outside y"
        out = w.ir()["outputs"][0]
        check({out: yh[oy:oy + M * N].reshape(M, N)}, oracle_outputs(w.ir(), inp, b), [out], TOL["softmax"],
              f"softmax N={N} {ox},{oy}")
        return
    xs = torch.zeros(M * N + 16, dtype=torch.float16, device="cuda")
    ys = torch.zeros(M * N + 16, dtype=torch.float16, device="cuda")
    xs[ox:ox + M * N] = torch.from_numpy(inp["in_ptr"].reshape(-1)).cuda()
    wt = torch.from_numpy(inp["weight_ptr"]).cuda()
    bt = torch.from_numpy(inp["bias_ptr"]).cuda()
    mean = torch.empty(M, device="cuda")
    rstd = torch.empty(M, device="cuda")
    st = hip.ihip_layernorm_rows_f16(ctypes.c_void_p(xs.data_ptr() + 2 * ox), ctypes.c_void_p(wt.data_ptr()),
                                     ctypes.c_void_p(bt.data_ptr()), ctypes.c_void_p(ys.data_ptr() + 2 * oy),
                                     ctypes.c_void_p(mean.data_ptr()), ctypes.c_void_p(rstd.data_ptr()), M, N,
                                     ctypes.c_float(1e-5), s)
    assert st == 0, hip.ihip_last_error()
    torch.cuda.synchronize()
    out = {"out_ptr": ys[oy:oy + M * N].cpu().numpy().reshape(M, N).astype(np.float32),
           "out_mean_ptr": mean.cpu().numpy(), "out_rstd_ptr": rstd.cpu().numpy()}
    _check_ln(out, oracle_outputs(w.ir(), inp, b), f"LN N={N} offsets {ox},{oy}")
    assert (ys[:oy] == 0).all() and (ys[oy + M * N:] == 0).all(), "writes outside y"


# ------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (17, 33, 31), (32, 48, 16), (256, 256, 64), (255, 257, 65),
                                   (512, 256, 128), (300, 600, 1000)])
def test_gemm_edge_shapes(hip, M, N, K):
    w = WORKLOADS["matmul"]
    b = {"M": M, "N": N, "K": K}
    inp = w.gen(b, seed=M + N + K, sigma=1.0)  # unit-scale operands: the product dominates the bias
    out = run_case(w.ir(), inp, b)
    ref = oracle_outputs(w.ir(), inp, b)
    check(out, ref, ["C"], TOL["matmul"], f"gemm {b}")
    check(out, ref, ["C"], TOL["matmul_strict"], f"gemm strict {b}")


def _gemm_abi(hip, A, B, bias, M, N, K, ta=False, tb=False, offset=0):
    """C (bf16 bits) through ihip_gemm_bf16_bias_relu_t on device copies of A and B placed `offset`
    elements past a 256-byte aligned allocation (offset 1: 2-byte aligned, so the guarded
    kernel runs instead of the tiled fast path)."""
    import ctypes

    import torch

    def dev(bits):
        t = torch.empty(bits.size + offset, dtype=torch.int16, device="cuda")
        t[offset:] = torch.from_numpy(bits.reshape(-1).view(np.int16)).cuda()
        return t

    a, b = dev(A), dev(B)
    bt = torch.from_numpy(bias).cuda()
    c = torch.empty(M * N, dtype=torch.int16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    st = hip.ihip_gemm_bf16_bias_relu_t(ctypes.c_void_p(a.data_ptr() + 2 * offset), ctypes.c_void_p(b.data_ptr() + 2 * offset),
                                        ctypes.c_void_p(bt.data_ptr()), ctypes.c_void_p(c.data_ptr()), M, N, K,
                                        int(ta), int(tb), 1, ctypes.c_void_p(s))
    assert st == 0, hip.ihip_last_error().decode()
    torch.cuda.synchronize()
    return c.cpu().numpy().view(np.uint16).reshape(M, N)


def _gemm_ws(hip, A, B, bias, M, N, K, ta=False, tb=False, offset=0, c_offset=0, ws_bytes=None):
    """C (bf16 bits) through ihip_gemm_bf16_bias_relu_ws with a workspace of ws_bytes (default:
    ihip_gemm_workspace_size, or room for both operands when a base is misaligned); A, B and C
    placed offset / c_offset elements past 256-byte aligned allocations."""
    import ctypes

    import torch

    def dev(bits, off):
        t = torch.zeros(bits.size + off, dtype=torch.int16, device="cuda")
        t[off:] = torch.from_numpy(bits.reshape(-1).view(np.int16)).cuda()
        return t

    a, b = dev(A, offset), dev(B, offset)
    bt = torch.from_numpy(bias).cuda()
    c = torch.empty(M * N + c_offset, dtype=torch.int16, device="cuda")
    if ws_bytes is None:
        k8 = -(-K // 8) * 8
        ws_bytes = hip.ihip_gemm_workspace_size(M, N, K, int(ta), int(tb))
        if offset or c_offset:  # room for copies of both operands, none for split-K partials
            ws_bytes = -(-(M * k8 * 2) // 256) * 256 + -(-(N * k8 * 2) // 256) * 256
    ws = torch.empty(max(1, ws_bytes), dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    st = hip.ihip_gemm_bf16_bias_relu_ws(ctypes.c_void_p(a.data_ptr() + 2 * offset),
                                         ctypes.c_void_p(b.data_ptr() + 2 * offset), ctypes.c_void_p(bt.data_ptr()),
                                         ctypes.c_void_p(c.data_ptr() + 2 * c_offset), M, N, K, int(ta), int(tb), 1, 0,
                                         ctypes.c_void_p(ws.data_ptr() if ws_bytes else None), ws_bytes,
                                         ctypes.c_void_p(s))
    assert st == 0, hip.ihip_last_error().decode()
    torch.cuda.synchronize()
    return c[c_offset:].cpu().numpy().view(np.uint16).reshape(M, N)


def _assert_near_unsplit(split, unsplit):
    """A split-K result against the unsplit kernel's: the two differ only in the order of f32
    additions, so after rounding to bf16 an element moves by at most a unit or two in its last
    place (plus a hair of the output's scale where cancellation leaves a small value)."""
    a, b = bf16_bits_to_f32(split).astype(np.float64), bf16_bits_to_f32(unsplit).astype(np.float64)
    scale = max(1e-30, float(np.abs(b).max()))
    bad = np.abs(a - b) > 2.0 ** -7 * np.abs(b) + 1e-5 * scale
    assert not bad.any(), f"split and unsplit differ beyond rounding in {int(bad.sum())} elements"


def _gemm_splitk(hip, A, B, bias, M, N, K, ta, tb, splits, tile=0, c_offset=0):
    """C (bf16 bits) through ihip_gemm_bf16_bias_relu_splitk with a workspace of exactly
    ihip_gemm_splitk_workspace_size bytes; C placed c_offset elements past an aligned base."""
    import ctypes

    import torch

    a = torch.from_numpy(A.reshape(-1).view(np.int16)).cuda()
    b = torch.from_numpy(B.reshape(-1).view(np.int16)).cuda()
    bt = torch.from_numpy(bias).cuda()
    c = torch.full((M * N + c_offset,), 0x7FC0, dtype=torch.int16, device="cuda")  # NaN: unwritten shows
    wb = hip.ihip_gemm_splitk_workspace_size(M, N, K, splits)
    ws = torch.full((max(1, wb),), 0xFF, dtype=torch.uint8, device="cuda")  # NaN partials if one is not written
    s = torch.cuda.current_stream().cuda_stream
    st = hip.ihip_gemm_bf16_bias_relu_splitk(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                                             ctypes.c_void_p(bt.data_ptr()), ctypes.c_void_p(c.data_ptr() + 2 * c_offset),
                                             M, N, K, int(ta), int(tb), 1, tile, splits,
                                             ctypes.c_void_p(ws.data_ptr() if wb else None), wb, ctypes.c_void_p(s))
    assert st == 0, hip.ihip_last_error().decode()
    torch.cuda.synchronize()
    return c[c_offset:].cpu().numpy().view(np.uint16).reshape(M, N)


@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("M,N,K", [(16, 65792, 512), (128, 66048, 256), (100, 65800, 200)])
def test_gemm_skinny_products_take_128_tiles(hip, M, N, K, tb):
    """M <= 128 with more than 256 tiles of 256x256 (N > 65536, a vocabulary projection in a
    decode step) runs 128x128 tiles by default: the same bits as either tile size on request
    (same MFMA over the same k order), and the oracle's values."""
    w = WORKLOADS["matmul"]
    b = {"M": M, "N": N, "K": K}
    inp = w.gen(b, seed=M + N + K, sigma=1.0)
    B = np.ascontiguousarray(inp["B"].T) if tb else inp["B"]
    print(f"[case] gemm skinny M={M} N={N} K={K} tb={tb}", flush=True)
    auto = _gemm_splitk(hip, inp["A"], B, inp["bias"], M, N, K, False, tb, 1)
    for tile in (128, 256):
        assert np.array_equal(auto, _gemm_splitk(hip, inp["A"], B, inp["bias"], M, N, K, False, tb, 1, tile=tile))
    ref = oracle_outputs(w.ir(), inp, b)
    check({"C": bf16_bits_to_f32(auto)}, ref, ["C"], TOL["matmul_strict"], f"skinny {b}")


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K,splits", [
    (1024, 1024, 8192, 0),   # the split rule: 64 tiles of 128x128, 4 segments of 2048
    (1000, 1000, 1000, 3),   # segments 384, 384, 232: the last one ends inside a 32-k step; edge tiles
    (8, 8, 4096, 64),        # one 64-k step per segment on a one-tile grid
    (256, 136, 520, 5),      # segments of 128, the last of 8 k (a single ragged K step)
    (304, 264, 96, 2),       # segments 64 and 32
    (128, 4104, 2048, 0),    # the rule: 33 tiles, 4 segments
    (1400, 8, 65536, 0),     # the rule: 11 tiles, 23 segments of 2880 (the last 2176)
    (4096, 4096, 1024, 2),   # 256x256 tiles, split on request
])
def test_gemm_split_k(hip, M, N, K, splits, ta, tb):
    """Split-K: K cut into segments of whole 64-k steps, each (tile, segment) workgroup's f32
    sums written to the workspace, then added in segment order with bias and ReLU.  Judged
    against the oracle, against the unsplit tiled kernel (equal up to f32 summation order),
    run to run (bit for bit), across the 128 and 256 tile knobs (bit for bit: the same
    segments in the same MFMA order; under the rule a forced 256x256 tile runs unsplit) and
    with a 2-byte aligned C (bit for bit)."""
    w = WORKLOADS["matmul"]
    b = {"M": M, "N": N, "K": K}
    inp = w.gen(b, seed=M + 5 * N + 7 * K + splits, sigma=1.0)
    A = np.ascontiguousarray(inp["A"].T) if ta else inp["A"]
    B = np.ascontiguousarray(inp["B"].T) if tb else inp["B"]
    S = gemm_split_plan(M, N, K, splits)[0]
    print(f"[case] gemm split-K M={M} N={N} K={K} splits={splits} (S={S}) ta={ta} tb={tb}", flush=True)
    assert S > 1
    split = _gemm_splitk(hip, A, B, inp["bias"], M, N, K, ta, tb, splits)
    ref = oracle_outputs(w.ir(), inp, b)
    check({"C": bf16_bits_to_f32(split)}, ref, ["C"], TOL["matmul"], f"split {b}")
    check({"C": bf16_bits_to_f32(split)}, ref, ["C"], TOL["matmul_strict"], f"split strict {b}")
    unsplit = _gemm_splitk(hip, A, B, inp["bias"], M, N, K, ta, tb, 1)
    assert np.array_equal(unsplit, _gemm_abi(hip, A, B, inp["bias"], M, N, K, ta, tb)), "splits=1 is the tiled kernel"
    _assert_near_unsplit(split, unsplit)
    assert np.array_equal(split, _gemm_splitk(hip, A, B, inp["bias"], M, N, K, ta, tb, splits)), "run to run"
    for tile in (128, 256):
        other = _gemm_splitk(hip, A, B, inp["bias"], M, N, K, ta, tb, splits, tile=tile)
        if splits == 0 and tile == 256 and gemm_split_plan(M, N, K, 0, tile=256)[0] == 1:
            # the rule splits grids of 128x128 tiles only: 256x256 tiles on request run unsplit
            other_ref = _gemm_splitk(hip, A, B, inp["bias"], M, N, K, ta, tb, 1, tile=256)
            assert np.array_equal(other, other_ref), "tile 256 under the rule is the unsplit kernel"
            continue
        assert np.array_equal(split, other), f"tile {tile}: {int((split != other).sum())} elements differ"
    assert np.array_equal(split, _gemm_splitk(hip, A, B, inp["bias"], M, N, K, ta, tb, splits, c_offset=1))
    if splits == 0:  # the workspace entry applies the same rule
        assert np.array_equal(split, _gemm_ws(hip, A, B, inp["bias"], M, N, K, ta, tb))


@pytest.mark.parametrize("M,N,K", [(1000, 1001, 4096), (64, 3, 8192), (200, 4097, 4096)])
def test_gemm_split_k_odd_n_with_b_as_nk(hip, M, N, K):
    """With B given as [N, K] any N runs in place; the partial rows are padded to a multiple of
    4 floats and the reduce writes C with 2-byte stores where a row is not 8-byte aligned."""
    w = WORKLOADS["matmul"]
    b = {"M": M, "N": N, "K": K}
    inp = w.gen(b, seed=M + N + K, sigma=1.0)
    B = np.ascontiguousarray(inp["B"].T)
    print(f"[case] gemm split-K odd N M={M} N={N} K={K}", flush=True)
    assert gemm_split_plan(M, N, K)[0] > 1
    split = _gemm_splitk(hip, inp["A"], B, inp["bias"], M, N, K, False, True, 0)
    check({"C": bf16_bits_to_f32(split)}, oracle_outputs(w.ir(), inp, b), ["C"], TOL["matmul"], f"split {b}")
    _assert_near_unsplit(split, _gemm_abi(hip, inp["A"], B, inp["bias"], M, N, K, False, True))
    assert np.array_equal(split, _gemm_ws(hip, inp["A"], B, inp["bias"], M, N, K, False, True))


def test_gemm_split_k_rejects_what_it_cannot_read_in_place(hip):
    """The explicit split entry takes operands the tiled kernel reads in place only, K > 0, and
    a workspace of at least ihip_gemm_splitk_workspace_size bytes: anything else is an
    argument error, with nothing launched."""
    import ctypes

    import torch

    a = torch.zeros(64 * 1024, dtype=torch.int16, device="cuda")
    c = torch.zeros(64 * 64, dtype=torch.int16, device="cuda")
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    P = ctypes.c_void_p
    s = P(torch.cuda.current_stream().cuda_stream)
    call = lambda M, N, K, tb, splits, wsp, wb: hip.ihip_gemm_bf16_bias_relu_splitk(  # noqa: E731
        P(a.data_ptr()), P(a.data_ptr()), None, P(c.data_ptr()), M, N, K, 0, tb, 0, 0, splits, wsp, wb, s)
    assert call(64, 64, 1020, 0, 2, P(ws.data_ptr()), 1 << 20) != 0  # K % 8 != 0
    assert call(64, 60, 1024, 0, 2, P(ws.data_ptr()), 1 << 20) != 0  # B as [K, N], N % 8 != 0
    assert call(64, 64, 1024, 0, 2, P(ws.data_ptr()), 100) != 0      # workspace too small
    assert call(64, 64, 1024, 0, 2, P(ws.data_ptr() + 16), 1 << 19) != 0  # workspace not 256-byte aligned
    assert call(64, 64, 0, 0, 2, P(ws.data_ptr()), 1 << 20) != 0     # K = 0
    assert call(64, 64, 1024, 0, -1, P(ws.data_ptr()), 1 << 20) != 0
    assert call(64, 64, 1024, 0, 2, P(ws.data_ptr()), 1 << 20) == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(7, 9, 3), (300, 263, 64), (257, 250, 60), (1000, 1001, 100), (513, 264, 1000),
                                   (4100, 4099, 72), (4096, 4095, 4095), (31, 4104, 33), (1001, 57, 4104)])
def test_gemm_packed_path(hip, M, N, K, ta, tb):
    """Rows that cannot start 16-byte aligned (K % 8 != 0, N % 8 != 0 with B as [K, N], M % 8 != 0
    with A as [K, M]) are packed into the workspace as K-contiguous rows of K rounded up to 8
    and run on the tiled kernel: bit for bit the guarded kernel (the same zeros in the same k
    slots, the same MFMA order), and the oracle's result within the GEMM tolerance.  2-byte
    aligned bases of A, B or C take the same path when the workspace holds their copies."""
    w = WORKLOADS["matmul"]
    b = {"M": M, "N": N, "K": K}
    inp = w.gen(b, seed=M + 7 * N + 3 * K, sigma=1.0)
    A = np.ascontiguousarray(inp["A"].T) if ta else inp["A"]
    B = np.ascontiguousarray(inp["B"].T) if tb else inp["B"]
    print(f"[case] gemm packed M={M} N={N} K={K} ta={ta} tb={tb}", flush=True)
    # a workspace for the copies only: the packed path unsplit
    packed = _gemm_ws(hip, A, B, inp["bias"], M, N, K, ta, tb, ws_bytes=gemm_pack_bytes(M, N, K, ta, tb))
    guarded = _gemm_ws(hip, A, B, inp["bias"], M, N, K, ta, tb, ws_bytes=0)
    assert np.array_equal(packed, guarded), f"packed and guarded differ in {int((packed != guarded).sum())} elements"
    ref = oracle_outputs(w.ir(), inp, b) if M * N * K <= 1 << 31 else None
    if ref is not None:
        check({"C": bf16_bits_to_f32(packed)}, ref, ["C"], TOL["matmul"], f"packed {b}")
    if gemm_split_plan(M, N, -(-K // 8) * 8)[0] > 1:  # the full workspace: packed, then split along K
        split = _gemm_ws(hip, A, B, inp["bias"], M, N, K, ta, tb)
        if ref is not None:
            check({"C": bf16_bits_to_f32(split)}, ref, ["C"], TOL["matmul"], f"packed split {b}")
        _assert_near_unsplit(split, packed)
    if M * N <= 1 << 22:
        for off, c_off in ((1, 0), (0, 1), (1, 3)):  # misaligned operand or C bases
            print(f"[case]   offsets {off} {c_off}", flush=True)
            mis = _gemm_ws(hip, A, B, inp["bias"], M, N, K, ta, tb, offset=off, c_offset=c_off)
            if gemm_split_plan(M, N, -(-K // 8) * 8)[0] > 1:  # split where the workspace holds the partials
                _assert_near_unsplit(mis, guarded)
            else:
                assert np.array_equal(mis, guarded), f"offsets {off}/{c_off}: {int((mis != guarded).sum())} elements differ"


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(300, 264, 64), (8, 8, 32), (257, 8, 32), (513, 520, 96), (1000, 1000, 256),
                                   (2000, 136, 4096), (300, 264, 1000), (257, 136, 40), (64, 64, 8), (512, 512, 264),
                                   (4100, 4104, 72), (4100, 4104, 64), (3968, 4104, 1000),
                                   (4096, 4352, 32), (4096, 4352, 96), (4352, 4096, 160),
                                   (300, 263, 64), (1000, 1001, 256), (257, 50257, 64), (4100, 4099, 64)])
def test_gemm_edge_tiles_fast_path(hip, M, N, K, ta, tb):
    """Shapes that are not multiples of the tile or of the 32-deep K step, with 16-byte aligned
    rows (K % 8 == 0; M % 8 != 0 sends a transposed A to the guarded kernel), run
    the tiled fast kernel with range-checked copies, k-chunks past K loaded as zeros and
    masked edge stores: 128x128 tiles up to 128 tiles of 256x256, 256x256 tiles above (4100 x
    4104 and the like).  4096 x 4352 with K = 32, 96, 160 (1, 3 and 5 K slices) runs full 256x256
    tiles with a single K slice (range-checked, a paired A would reach past K) and with a last A
    pair that holds one slice.  N % 8 != 0 (the last four shapes) runs the tiled kernel with 2-byte C
    stores when B is given as [N, K], the guarded kernel otherwise.  Judged against the oracle,
    and bit for bit against the guarded kernel (same MFMA over the same k order) run on 2-byte
    aligned copies."""
    w = WORKLOADS["matmul"]
    b = {"M": M, "N": N, "K": K}
    inp = w.gen(b, seed=M + 3 * N + 5 * K, sigma=1.0)
    A = np.ascontiguousarray(inp["A"].T) if ta else inp["A"]
    B = np.ascontiguousarray(inp["B"].T) if tb else inp["B"]
    print(f"[case] gemm edge tiles M={M} N={N} K={K} ta={ta} tb={tb}", flush=True)
    fast = _gemm_abi(hip, A, B, inp["bias"], M, N, K, ta, tb)
    ref = oracle_outputs(w.ir(), inp, b)
    check({"C": bf16_bits_to_f32(fast)}, ref, ["C"], TOL["matmul"], f"fast {b}")
    check({"C": bf16_bits_to_f32(fast)}, ref, ["C"], TOL["matmul_strict"], f"fast strict {b}")
    guarded = _gemm_abi(hip, A, B, inp["bias"], M, N, K, ta, tb, offset=1)
    assert np.array_equal(fast, guarded), f"fast and guarded kernels differ in {int((fast != guarded).sum())} elements"


def test_gemm_ones_known_answer(hip):
    """tests/test_diff_runner.py:35-43: ones @ ones + 1 -> K + 1 everywhere."""
    M, N, K = 256, 256, 192
    ir = matmul_bias_relu2d_ir()
    inp = {"A": f32_to_bf16_bits(np.ones((M, K), np.float32)), "B": f32_to_bf16_bits(np.ones((K, N), np.float32)),
           "bias": np.ones(N, np.float32)}
    out = run_case(ir, inp, {"M": M, "N": N, "K": K})
    assert np.all(out["C"] == K + 1.0)


def test_gemm_plain_and_epilogue_forms(hip):
    """Lone matmul (no bias/relu) and matmul{epilogue} lower to the same kernel."""
    M = N = K = 256
    rng = np.random.default_rng(11)
    A = f32_to_bf16_bits(rng.standard_normal((M, K), dtype=np.float32))
    B = f32_to_bf16_bits(rng.standard_normal((K, N), dtype=np.float32))
    bias = rng.standard_normal(N).astype(np.float32)
    plain = {"name": "mm", "tensors": {"A": {"dtype": "bf16", "shape": ["M", "K"]}, "B": {"dtype": "bf16", "shape": ["K", "N"]},
                                        "C": {"dtype": "bf16", "shape": ["M", "N"]}},
             "ops": [{"op": "matmul", "inputs": ["A", "B"], "output": "C"}], "outputs": ["C"]}
    b = {"M": M, "N": N, "K": K}
    out = run_case(plain, {"A": A, "B": B}, b)
    check(out, oracle_outputs(plain, {"A": A, "B": B}, b), ["C"], TOL["matmul_strict"], "plain gemm")
    epi = {"name": "mm_epi", "tensors": dict(plain["tensors"], bias={"dtype": "f32", "shape": ["N"]}),
           "ops": [{"op": "matmul", "inputs": ["A", "B"], "output": "C",
                    "attrs": {"epilogue": {"op": "relu", "inputs": [{"op": "add", "inputs": ["$x", "bias"]}]}}}],
           "outputs": ["C"]}
    inp = {"A": A, "B": B, "bias": bias}
    out = run_case(epi, inp, b)
    check(out, oracle_outputs(epi, inp, b), ["C"], TOL["matmul_strict"], "epilogue gemm")


def _transposed_ir(ta: bool, tb: bool) -> dict:
    ir = matmul_bias_relu2d_ir()
    ir["tensors"]["A"]["shape"] = ["K", "M"] if ta else ["M", "K"]
    ir["tensors"]["B"]["shape"] = ["N", "K"] if tb else ["K", "N"]
    ir["ops"][0]["attrs"] = {"transpose_a": ta, "transpose_b": tb}
    return ir


@pytest.mark.parametrize("ta,tb", [(False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(512, 256, 96), (256, 512, 8192), (17, 33, 31), (300, 260, 100)])
def test_gemm_transposed_operands(hip, ta, tb, M, N, K):
    """matmul{transpose_a, transpose_b} (interpreter.py:507-520): parity with the oracle, and the
    same bits as the plain layout on explicitly transposed copies (same MFMA order)."""
    w = WORKLOADS["matmul"]
    b = {"M": M, "N": N, "K": K}
    inp = w.gen(b, seed=M + 2 * N + 3 * K, sigma=1.0)
    tin = {"A": np.ascontiguousarray(inp["A"].T) if ta else inp["A"],
           "B": np.ascontiguousarray(inp["B"].T) if tb else inp["B"], "bias": inp["bias"]}
    ir = _transposed_ir(ta, tb)
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    # rows that cannot start 16-byte aligned (K % 8 != 0) go through the packed path
    assert k.kernel_id == ("ihip_gemm_bf16_bias_relu_ws" if gemm_workspace_bytes(M, N, K, ta, tb)
                           else "ihip_gemm_bf16_bias_relu_t")
    out = run_case(ir, tin, b)
    check(out, oracle_outputs(ir, tin, b), ["C"], TOL["matmul_strict"], f"gemm ta={ta} tb={tb} {b}")
    plain = run_case(w.ir(), inp, b)
    np.testing.assert_array_equal(out["C"], plain["C"])


def test_gemm_full_config(hip):
    import torch

    w = WORKLOADS["matmul"]
    inp = w.gen(w.bindings)
    out = run_case(w.ir(), inp, w.bindings)["C"]
    # every row against the oracle (np.matmul in f32), in blocks of rows to bound its temporaries
    # (a row of C depends on the same row of A only)
    blk = 2048
    for r0 in range(0, w.bindings["M"], blk):
        rows = slice(r0, min(r0 + blk, w.bindings["M"]))
        sb = dict(w.bindings, M=rows.stop - rows.start)
        ref = oracle_outputs(w.ir(), dict(inp, A=inp["A"][rows]), sb)
        check({"C": out[rows]}, ref, ["C"], TOL["matmul"], f"gemm full rows {r0}+")
        check({"C": out[rows]}, ref, ["C"], TOL["matmul_strict"], f"gemm full rows {r0}+ strict")
    at = torch.from_numpy(bf16_bits_to_f32(inp["A"])).cuda()
    bt = torch.from_numpy(bf16_bits_to_f32(inp["B"])).cuda()
    cref = torch.relu(at @ bt + torch.from_numpy(inp["bias"]).cuda()).cpu().numpy()
    np.testing.assert_allclose(out, cref, rtol=2e-2, atol=1e-4)
