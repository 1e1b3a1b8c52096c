"""Parity of the generic element-wise program kernel (ihip_elementwise_program) with the oracle.

Every chain of ``tests/ew_cases.py`` is lowered, run through the C-ABI and judged
against ``oracle.interpreter.execute_intent`` with the reference rule; then
larger shapes exercise the vector load/store paths, more rows than one grid
dimension holds, and misaligned operands (scalar paths).
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest

from intent_ir_amd import launch_lowered, load_library, lower_intent_to_hip_kernel, run_lowered
from intent_ir_amd.runtime import to_device, to_host, torch_dtype
from tests.ew_cases import CASES, T, op
from tests.test_ewprogram import check_output, oracle_outputs

pytestmark = pytest.mark.gpu

MODES = {"native": 2, "interp": 1}  # IHIP_EW_MODE_NATIVE / IHIP_EW_MODE_INTERP


@pytest.fixture(params=sorted(MODES))
def ew_mode(request, hip):
    """Run the test with specialised native code, then with the interpreter kernel."""
    prev = hip.ihip_elementwise_mode(MODES[request.param])
    yield request.param
    hip.ihip_elementwise_mode(prev)


def _run(ir, bindings, inputs):
    k = lower_intent_to_hip_kernel(ir, shape_bindings=bindings)
    assert k.kernel_id == "ihip_elementwise_program"
    print(f"[case] {ir['name']} bindings={bindings} mode={load_library().ihip_elementwise_mode(-1)}", flush=True)
    return k, run_lowered(k, inputs)


@pytest.mark.parametrize("name,ir,bindings,gen", CASES, ids=[c[0] for c in CASES])
def test_chain_matches_oracle(ew_mode, name, ir, bindings, gen):
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    inputs = gen(rng, bindings)
    k, got = _run(ir, bindings, inputs)
    ref = oracle_outputs(ir, inputs, bindings)
    dtypes = {n: t["dtype"] for n, t in k.io_spec["tensors"].items()}
    for o in k.output_names:
        check_output(got, ref, o, dtypes[o], f"{name}/{o}")


BIG = [
    ("add_bias_relu", {"M": 1024, "N": 4096}),
    ("half_inputs_bf16_out", {"M": 512, "N": 4096}),
    ("compare_logic_bool", {"M": 256, "N": 1024}),
    ("int_and_bool_inputs", {"N": 1 << 20}),
    ("transpose_add", {"M": 1000, "N": 1024}),
    ("rank4_broadcast", {"A": 4, "B": 8, "C": 64, "D": 256}),
    ("gelu_f32_chain", {"M": 256, "N": 8192}),
    ("two_outputs_shared", {"M": 70000, "N": 4}),  # more rows than grid.y: the row loop strides
    ("transpose_half_bf16_out", {"M": 1000, "N": 1024}),  # LDS-staged transpose, 16-byte staging reads
    ("transpose_half_bf16_out", {"M": 999, "N": 1001}),  # staging falls back to element reads
    ("transpose_batched_3d", {"A": 4, "M": 256, "N": 520}),
]


@pytest.mark.parametrize("name,bindings", BIG, ids=[b[0] for b in BIG])
def test_chain_large_shapes(ew_mode, name, bindings):
    _, ir, _, gen = next(c for c in CASES if c[0] == name)
    rng = np.random.default_rng(7)
    inputs = gen(rng, bindings)
    k, got = _run(ir, bindings, inputs)
    ref = oracle_outputs(ir, inputs, bindings)
    dtypes = {n: t["dtype"] for n, t in k.io_spec["tensors"].items()}
    for o in k.output_names:
        check_output(got, ref, o, dtypes[o], f"{name}/{o}")


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16", "i1", "i32"])
def test_misaligned_operands_take_the_scalar_path(ew_mode, dtype):
    """Operands that start one element past an aligned address are read and written element by element."""
    import torch

    n = 4099
    ir = {"name": "copy_mis", "tensors": {"x": T(dtype, "N"), "y": T(dtype, "N")},
          "ops": [op("identity", ["x"], "y")], "outputs": ["y"]}
    k = lower_intent_to_hip_kernel(ir, shape_bindings={"N": n})
    rng = np.random.default_rng(3)
    vals = (rng.standard_normal(n + 1) * 100).astype(np.float32)
    if dtype == "i1":
        vals = vals > 0
    elif dtype == "i32":
        vals = vals.astype(np.int32)
    xb = to_device(vals, dtype)
    yb = torch.zeros(n + 1, dtype=torch_dtype(dtype), device="cuda")
    x, y = xb[1:], yb[1:]
    assert x.data_ptr() % 16 != 0 and y.data_ptr() % 16 != 0
    launch_lowered(k, {"x": x, "y": y})
    torch.cuda.synchronize()
    got = to_host(y, dtype)
    want = to_host(x, dtype)
    np.testing.assert_array_equal(got, want)
    assert to_host(yb[:1], dtype)[0] == 0  # nothing written before the view


def test_row_offsets_not_multiple_of_four(ew_mode):
    """[M,N] with N % 4 != 0: rows start at unaligned offsets, so loads and stores go element-wise."""
    _, ir, _, gen = next(c for c in CASES if c[0] == "add_bias_relu")
    for n in (1, 2, 3, 5, 6, 7, 9):
        b = {"M": 65, "N": n}
        inputs = gen(np.random.default_rng(n), b)
        k, got = _run(ir, b, inputs)
        ref = oracle_outputs(ir, inputs, b)
        check_output(got, ref, "y", "f32", f"N={n}")
