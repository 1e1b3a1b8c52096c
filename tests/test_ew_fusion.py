"""Logistic fusion in the native element-wise code (CPU only: source inspection and hiprtc).

x / (exp(u) + 1), the shape of GELU-tanh and sigmoid, is emitted as one fused step when the
exp and the add feed only the division; ihip_elementwise_source returns the HIP source a
launch would compile (the role of the reference lowering's cuda_src), so these tests see
whether the fusion fired and that the result still compiles."""

from __future__ import annotations

import copy
import re

import numpy as np
import pytest

from intent_ir_amd import lower_intent_to_hip_kernel
from intent_ir_amd.runtime import elementwise_source, ew_program_args, load_library
from tests.ew_cases import CASES, T, op

FUSED = "ew_logistic_div_fast(r["  # a fused step (the prelude defines the function)


def _source(ir, bindings):
    k = lower_intent_to_hip_kernel(ir, shape_bindings=bindings)
    assert k.kernel_id == "ihip_elementwise_program"
    prog = k.call_args[0][1]
    dt = {n: t["dtype"] for n, t in k.io_spec["tensors"].items()}
    names = [n for n, _ in prog.inputs] + list(prog.outputs)
    ptrs = {n: 0x100000 * (i + 1) for i, n in enumerate(names)}
    src = elementwise_source(prog, ptrs, dt)
    st = load_library().ihip_elementwise_prepare_operands(*ew_program_args(prog, ptrs, dt)[:8])
    assert st == 0, load_library().ihip_last_error().decode()  # the fused source compiles
    return src


def _case(name):
    c = next(c for c in CASES if c[0] == name)
    return copy.deepcopy(c[1]), dict(c[2])


@pytest.mark.parametrize("name", ["gelu_f32_chain", "logistic_special"])
def test_logistic_shapes_are_fused(name):
    ir, b = _case(name)
    src = _source(ir, b)
    assert src.count(FUSED) == 1
    assert "ew_exp(x)" not in src.split("ihip_ew_jit")[-1]  # the exp is not emitted on its own


def _bits(v: float) -> str:
    return f"__builtin_bit_cast(float, {int(np.float32(v).view(np.uint32))}u)"


def test_constant_multiplies_fold_into_the_exponent():
    """u = x * k feeds the fused step as t = x * (k log2 e); GELU-tanh's
    u = (z + 0.044715 z^3) * k as t = z * fma(z * z, 0.044715 k log2 e, k log2 e), each
    constant rounded once from the double product of the program's f32 constants."""
    log2e = 1.4426950408889634
    ir, b = _case("logistic_special")
    src = _source(ir, b)
    assert re.search(r"ew_logistic_div_fast\(r\[\d+\]\[j\], s\d+_\d+\[j\] \* " + re.escape(_bits(float(np.float32(-1.7)) * log2e)), src)
    ir, b = _case("gelu_f32_chain")
    src = _source(ir, b)
    k = -2.0 * np.sqrt(2.0 / np.pi)  # the macro's exp(-2 sqrt(2/pi) w) form
    fold = re.search(r"s(\d+)_(\d+)\[j\] \* __builtin_fmaf\(s\1_\2\[j\] \* s\1_\2\[j\], "
                     r"__builtin_bit_cast\(float, (\d+)u\), __builtin_bit_cast\(float, (\d+)u\)\)", src)
    assert fold, src
    got = [np.uint32(int(g)).view(np.float32) for g in fold.groups()[2:]]
    np.testing.assert_allclose(got, [0.044715 * k * log2e, k * log2e], rtol=2e-7)


def test_exp_with_another_use_is_not_fused():
    ir, b = _case("logistic_special")
    ir["outputs"] = ["y", "e"]
    src = _source(ir, b)
    assert FUSED not in src and "ew_exp(x)" in src


def test_other_constants_and_orders_are_not_fused():
    ir, b = _case("logistic_special")
    ir["ops"][2]["attrs"]["value"] = 2.0  # x / (exp(u) + 2)
    assert FUSED not in _source(ir, b)
    ir, b = _case("logistic_special")
    ir["ops"][4]["inputs"] = ["d", "x"]  # (exp(u) + 1) / x
    assert FUSED not in _source(ir, b)


def test_add_with_the_constant_first_is_fused():
    ir, b = _case("logistic_special")
    ir["ops"][3]["inputs"] = ["one", "e"]
    assert _source(ir, b).count(FUSED) == 1


def test_sigmoid_of_a_bf16_tensor():
    """sigmoid(x) = 1 / (1 + exp(-x)) on bf16 in and out: the numerator is a constant register."""
    ir = {"name": "sigmoid_bf16",
          "tensors": {"x": T("bf16", "M", "N"), "u": T("f32", "M", "N"), "e": T("f32", "M", "N"), "one": T("f32"),
                      "d": T("f32", "M", "N"), "y": T("bf16", "M", "N")},
          "ops": [op("mul", ["x"], "u", mul_factor=-1.0), op("exp", ["u"], "e"),
                  op("const", [], "one", value=1.0, dtype="f32"), op("add", ["e", "one"], "d"),
                  op("div", ["one", "d"], "y")], "outputs": ["y"]}
    assert _source(ir, {"M": 64, "N": 256}).count(FUSED) == 1
