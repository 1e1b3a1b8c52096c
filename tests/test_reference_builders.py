"""Every deterministic builder IR of the reference's kernel families lowers to its HIP entry
point (CPU only: lowering, argument plans and the oracle on tiny inputs; no launches).

The IRs are restated in tests/reference_builder_irs.py from pipeline/tilelang/core.py,
pipeline/cuda/core.py:409-546 and tests/backends/cuda/test_cuda_backend_smoke.py."""

from __future__ import annotations

import numpy as np
import pytest

from intent_ir_amd import lower_intent_to_hip_kernel
from intent_ir_amd.ir import as_intent, resolve_shape
from intent_ir_amd.runtime import SIGNATURES
from oracle.interpreter import execute_intent
from tests.reference_builder_irs import BUILDERS, builder_ir

NAMES = sorted(BUILDERS)


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("b", [{"M": 1, "N": 1, "K": 1}, {"M": 3, "N": 17, "K": 5}, {"M": 64, "N": 4096, "K": 64},
                               {"M": 7, "N": 70001, "K": 9}])
def test_builder_lowers_to_its_kernel(name, b):
    _, ir, kid, _ = BUILDERS[name]
    k = lower_intent_to_hip_kernel(builder_ir(name), shape_bindings=b)
    assert k.kernel_id in (kid, kid + "_ws")  # _ws: the split form of few long rows
    # the argument plan matches the C signature (the element-wise program expands to 8 arguments)
    n_args = sum(8 if kind == "ew_program" else 2 if kind == "workspace" else 1 for kind, _ in k.call_args)
    assert n_args + 1 == len(SIGNATURES[k.kernel_id][1]), k.call_args
    assert set(k.output_names) == set(ir["outputs"])
    for kind, v in k.call_args:
        if kind == "tensor":
            assert v in k.io_spec["tensors"]


def _inputs(ir: dict, b: dict, seed: int) -> dict:
    fn = as_intent(ir)
    produced = {o.output for o in fn.ops}
    rng = np.random.default_rng(seed)
    out = {}
    for n, t in fn.tensors.items():
        if n in produced:
            continue
        shp = resolve_shape(t, b)
        if t.dtype in ("bool", "i1"):
            out[n] = rng.random(shp) < 0.5
        else:
            out[n] = rng.standard_normal(shp).astype(np.float32)
    return out


@pytest.mark.parametrize("name", NAMES)
def test_oracle_runs_every_builder(name):
    """The fixtures are IR the oracle executes (shapes and names consistent), so the GPU parity
    test of each builder has a reference."""
    b = {"M": 3, "N": 5, "K": 4}
    ir = builder_ir(name)
    ref = execute_intent(ir, _inputs(ir, b, 0), b)
    for o in ir["outputs"]:
        assert o in ref and np.asarray(ref[o]).size == int(np.prod(resolve_shape(as_intent(ir).tensors[o], b)))


def test_softmax_statistics_are_matched_structurally():
    """Any subset of the statistics may be returned; an unrelated extra output is not softmax."""
    ir = builder_ir("cuda.softmax_inner")
    ir["outputs"] = ["output_ptr", "row_sum_ptr"]
    k = lower_intent_to_hip_kernel(ir, shape_bindings={"M": 4, "N": 8})
    assert k.kernel_id == "ihip_softmax_rows_f32_stats"
    assert k.call_args[2] == ("null", None) and k.call_args[3] == ("tensor", "row_sum_ptr")
    ir = builder_ir("cuda.softmax_inner")
    ir["tensors"]["other"] = {"dtype": "f32", "shape": ["M"]}
    ir["ops"].append({"op": "reduce_sum", "inputs": ["input_ptr"], "output": "other", "attrs": {"dims": [1]}})
    ir["outputs"].append("other")
    with pytest.raises(Exception):
        lower_intent_to_hip_kernel(ir, shape_bindings={"M": 4, "N": 8})


def test_scaled_row_sum_lowers_with_its_factor():
    """reduce_sum{scale} alone: the _ex entry with the factor the interpreter computes
    (numbers, bindings and arithmetic of bindings)."""
    for scale, want in ((0.25, 0.25), ("N", 8.0), ("1.0/N", 0.125), ("2**-3", 0.125), ("(N-4)*0.5", 2.0)):
        ir = {"name": "mean", "tensors": {"x": {"dtype": "f32", "shape": ["M", "N"]}, "m": {"dtype": "f32", "shape": ["M"]}},
              "ops": [{"op": "reduce_sum", "inputs": ["x"], "output": "m", "attrs": {"dims": [1], "scale": scale}}],
              "outputs": ["m"]}
        k = lower_intent_to_hip_kernel(ir, shape_bindings={"M": 4, "N": 8})
        assert k.kernel_id == "ihip_reduce_rows_f32_ex" and k.call_args[5] == ("f32", want)
    ir["ops"][0]["attrs"]["scale"] = "__import__('os')"
    with pytest.raises(Exception, match="unresolved reduce scale"):
        lower_intent_to_hip_kernel(ir, shape_bindings={"M": 4, "N": 8})


def test_large_elementwise_programs_compile_for_the_native_form():
    """Chains past the interpreter kernel's limits (8 inputs, 8 live values, 64 instructions)
    compile for the native form instead of being refused."""
    from intent_ir_amd.ewprogram import fits_interpreter

    t = {f"a{i}": {"dtype": "f32", "shape": ["M", "N"]} for i in range(12)}
    t["y"] = {"dtype": "f32", "shape": ["M", "N"]}
    ops, acc = [], "a0"
    for i in range(1, 12):
        ops.append({"op": "add", "inputs": [acc, f"a{i}"], "output": f"s{i}" if i < 11 else "y"})
        acc = f"s{i}"
    k = lower_intent_to_hip_kernel({"name": "sum12", "tensors": t, "ops": ops, "outputs": ["y"]},
                                   shape_bindings={"M": 4, "N": 8})
    prog = k.call_args[0][1]
    assert len(prog.inputs) == 12 and not fits_interpreter(prog)
