"""Element-wise chains for the generic program path (``ihip_elementwise_program``).

Each case is (IR, bindings, input generator).  They cover the op families of
the reference interpreter's element-wise tables (verify/interpreter.py:16-48),
its broadcast rules (name-based 1-D alignment :752-841, broadcast_in_dim
:594-608, [M,1] columns, scalars, scalar attrs :216-232), transpose, iota,
cast, where, multiple outputs, ranks 0..4, and the shapes the kernel must mask:
inner sizes that are not a multiple of 4, a single column, empty tensors.
Sizes follow the reference's edge list (verify/gen_cases.py:27) where they
matter.
"""

from __future__ import annotations

from typing import Callable, Dict, List, Tuple

import numpy as np


def T(dtype, *shape):
    return {"dtype": dtype, "shape": list(shape)}


def op(name, inputs, output, **attrs):
    d = {"op": name, "inputs": list(inputs), "output": output}
    if attrs:
        d["attrs"] = attrs
    return d


def _f(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


Case = Tuple[str, dict, Dict[str, int], Callable[[np.random.Generator, Dict[str, int]], Dict[str, np.ndarray]]]
CASES: List[Case] = []


def case(name, ir, bindings, gen):
    ir = dict(ir, name=name)
    CASES.append((name, ir, bindings, gen))


# bias add + ReLU, bias aligned on N by its symbol; N % 4 != 0 exercises the masked tail
case("add_bias_relu", {
    "tensors": {"x": T("f32", "M", "N"), "b": T("f32", "N"), "t": T("f32", "M", "N"), "y": T("f32", "M", "N")},
    "ops": [op("add", ["x", "b"], "t"), op("relu", ["t"], "y")], "outputs": ["y"]},
    {"M": 37, "N": 50}, lambda r, b: {"x": _f(r, b["M"], b["N"]), "b": _f(r, b["N"])})

# leaky ReLU through where / gt / scalar attr
case("leaky_relu_where", {
    "tensors": {"x": T("f32", "M", "N"), "z": T("f32"), "p": T("i1", "M", "N"), "s": T("f32", "M", "N"),
                "y": T("f32", "M", "N")},
    "ops": [op("const", [], "z", value=0.0, dtype="f32"), op("gt", ["x", "z"], "p"),
            op("mul", ["x"], "s", mul_factor=0.1), op("where", ["p", "x", "s"], "y")], "outputs": ["y"]},
    {"M": 16, "N": 64}, lambda r, b: {"x": _f(r, b["M"], b["N"])})

# 1-D operand named by the leading symbol: [M] aligns to axis 0, not the trailing axis
case("row_vector_by_symbol", {
    "tensors": {"x": T("f32", "M", "N"), "m": T("f32", "M"), "d": T("f32", "M", "N"), "y": T("f32", "M", "N")},
    "ops": [op("sub", ["x", "m"], "d"), op("exp", ["d"], "y")], "outputs": ["y"]},
    {"M": 33, "N": 17}, lambda r, b: {"x": _f(r, b["M"], b["N"]), "m": _f(r, b["M"])})

# [M,1] column and broadcast_in_dim of a vector
case("column_and_broadcast_in_dim", {
    "tensors": {"x": T("f32", "M", "N"), "c": T("f32", "M", 1), "v": T("f32", "N"), "vb": T("f32", "M", "N"),
                "t": T("f32", "M", "N"), "y": T("f32", "M", "N")},
    "ops": [op("broadcast_in_dim", ["v"], "vb", out_shape=["M", "N"], broadcast_dims=[1]),
            op("mul", ["x", "c"], "t"), op("add", ["t", "vb"], "y")], "outputs": ["y"]},
    {"M": 31, "N": 33}, lambda r, b: {"x": _f(r, b["M"], b["N"]), "c": _f(r, b["M"], 1), "v": _f(r, b["N"])})

# comparisons and logic to a bool output
case("compare_logic_bool", {
    "tensors": {"x": T("f32", "M", "N"), "y": T("f32", "M", "N"), "z": T("f32"), "a": T("i1", "M", "N"),
                "n": T("i1", "M", "N"), "o": T("i1", "M", "N"), "q": T("i1", "M", "N"), "q2": T("i1", "M", "N"),
                "out": T("i1", "M", "N")},
    "ops": [op("const", [], "z", value=0.0, dtype="f32"), op("lt", ["x", "y"], "a"), op("ne", ["x", "z"], "n"),
            op("and", ["a", "n"], "o"), op("ge", ["y", "z"], "q"), op("not", ["q"], "q2"),
            op("or", ["o", "q2"], "out")], "outputs": ["out"]},
    {"M": 8, "N": 15}, lambda r, b: {"x": np.where(r.random((b["M"], b["N"])) < 0.2, 0.0,
                                                   _f(r, b["M"], b["N"])).astype(np.float32),
                                     "y": _f(r, b["M"], b["N"])})

# rsqrt, div, floor, abs, min, max, sub with scalar attrs
case("math_mix", {
    "tensors": {"x": T("f32", "M", "N"), "a": T("f32", "M", "N"), "s": T("f32", "M", "N"), "r": T("f32", "M", "N"),
                "q": T("f32", "M", "N"), "f": T("f32", "M", "N"), "m": T("f32", "M", "N"), "y": T("f32", "M", "N")},
    "ops": [op("abs", ["x"], "a"), op("add", ["a"], "s", addend=1.0), op("rsqrt", ["s"], "r"),
            op("div", ["x", "r"], "q"), op("floor", ["q"], "f"), op("min", ["f"], "m", other=2.0),
            op("max", ["m", "x"], "y")], "outputs": ["y"]},
    {"M": 7, "N": 64}, lambda r, b: {"x": _f(r, b["M"], b["N"], scale=4.0)})

# div by a bound symbol (LayerNorm's div{divisor:"N"} form)
case("div_by_symbol", {
    "tensors": {"x": T("f32", "M", "N"), "y": T("f32", "M", "N")},
    "ops": [op("div", ["x"], "y", divisor="N")], "outputs": ["y"]},
    {"M": 3, "N": 1023}, lambda r, b: {"x": _f(r, b["M"], b["N"])})

# f16 and bf16 operands, bf16 output (RNE on store)
case("half_inputs_bf16_out", {
    "tensors": {"x": T("f16", "M", "N"), "w": T("bf16", "N"), "t": T("f32", "M", "N"), "y": T("bf16", "M", "N")},
    "ops": [op("mul", ["x", "w"], "t"), op("add", ["t"], "y", addend=0.25)], "outputs": ["y"]},
    {"M": 16, "N": 256}, lambda r, b: {"x": _f(r, b["M"], b["N"]).astype(np.float16), "w": _f(r, b["N"])})

# f16 output
case("f16_out", {
    "tensors": {"x": T("f32", "M", "N"), "y": T("f16", "M", "N")},
    "ops": [op("mul", ["x"], "y", mul_factor=3.0)], "outputs": ["y"]},
    {"M": 5, "N": 8}, lambda r, b: {"x": _f(r, b["M"], b["N"])})

# transpose: strided reads of x, bias named by its symbol on the transposed axis
case("transpose_add", {
    "tensors": {"x": T("f32", "M", "N"), "xt": T("f32", "N", "M"), "b": T("f32", "M"), "y": T("f32", "N", "M")},
    "ops": [op("transpose", ["x"], "xt", perm=[1, 0]), op("add", ["xt", "b"], "y")], "outputs": ["y"]},
    {"M": 17, "N": 32}, lambda r, b: {"x": _f(r, b["M"], b["N"]), "b": _f(r, b["M"])})

# transposes staged through LDS tiles: 16-bit operands (8-wide lanes, 16-byte staging reads),
# a batched 3-D transpose (batch axis outside the tile), tails on both tile axes
case("transpose_half_bf16_out", {
    "tensors": {"x": T("f16", "M", "N"), "xt": T("f16", "N", "M"), "w": T("bf16", "M"), "t": T("f32", "N", "M"),
                "y": T("bf16", "N", "M")},
    "ops": [op("transpose", ["x"], "xt", perm=[1, 0]), op("mul", ["xt", "w"], "t"), op("add", ["t"], "y", addend=0.25)],
    "outputs": ["y"]},
    {"M": 24, "N": 40}, lambda r, b: {"x": _f(r, b["M"], b["N"]).astype(np.float16), "w": _f(r, b["M"])})

case("transpose_batched_3d", {
    "tensors": {"x": T("f32", "A", "M", "N"), "xt": T("f32", "A", "N", "M"), "y": T("f32", "A", "N", "M")},
    "ops": [op("transpose", ["x"], "xt", perm=[0, 2, 1]), op("relu", ["xt"], "y")], "outputs": ["y"]},
    {"A": 3, "M": 70, "N": 66}, lambda r, b: {"x": _f(r, b["A"], b["M"], b["N"])})

# iota along the inner axis
case("iota_inner", {
    "tensors": {"x": T("f32", "M", "N"), "i": T("i32", "M", "N"), "y": T("f32", "M", "N")},
    "ops": [op("iota", [], "i", shape=["M", "N"], axis=1, dtype="i32"), op("add", ["x", "i"], "y")],
    "outputs": ["y"]},
    {"M": 4, "N": 9}, lambda r, b: {"x": _f(r, b["M"], b["N"])})

# iota along the outer axis of a 3-D space
case("iota_outer_3d", {
    "tensors": {"i": T("i32", "A", "B", "C"), "y": T("f32", "A", "B", "C")},
    "ops": [op("iota", [], "i", shape=["A", "B", "C"], axis=0, dtype="i32"), op("mul", ["i"], "y", mul_factor=2.0)],
    "outputs": ["y"]},
    {"A": 3, "B": 5, "C": 8}, lambda r, b: {})

# 3-D with a vector named by the middle symbol and one by the last
case("rank3_named_vectors", {
    "tensors": {"x": T("f32", "A", "B", "C"), "s": T("f32", "B"), "t": T("f32", "C"), "u": T("f32", "A", "B", "C"),
                "y": T("f32", "A", "B", "C")},
    "ops": [op("mul", ["x", "s"], "u"), op("add", ["u", "t"], "y")], "outputs": ["y"]},
    {"A": 3, "B": 7, "C": 16}, lambda r, b: {"x": _f(r, b["A"], b["B"], b["C"]), "s": _f(r, b["B"]),
                                             "t": _f(r, b["C"])})

# 4-D with broadcast_in_dim of a [B, D] operand
case("rank4_broadcast", {
    "tensors": {"x": T("f32", "A", "B", "C", "D"), "g": T("f32", "B", "D"), "gb": T("f32", "A", "B", "C", "D"),
                "y": T("f32", "A", "B", "C", "D")},
    "ops": [op("broadcast_in_dim", ["g"], "gb", out_shape=["A", "B", "C", "D"], broadcast_dims=[1, 3]),
            op("sub", ["x", "gb"], "y")], "outputs": ["y"]},
    {"A": 2, "B": 3, "C": 5, "D": 12}, lambda r, b: {"x": _f(r, b["A"], b["B"], b["C"], b["D"]),
                                                     "g": _f(r, b["B"], b["D"])})

# two outputs sharing a subexpression
case("two_outputs_shared", {
    "tensors": {"x": T("f32", "M", "N"), "b": T("f32", "N"), "y1": T("f32", "M", "N"), "y2": T("f32", "M", "N")},
    "ops": [op("add", ["x", "b"], "y1"), op("mul", ["y1", "x"], "y2")], "outputs": ["y1", "y2"]},
    {"M": 9, "N": 40}, lambda r, b: {"x": _f(r, b["M"], b["N"]), "b": _f(r, b["N"])})

# casts: f16 rounding inside the chain, bool and i32 results
case("casts", {
    "tensors": {"x": T("f32", "M", "N"), "h": T("f16", "M", "N"), "hf": T("f32", "M", "N"), "y": T("f32", "M", "N"),
                "bi": T("i1", "M", "N"), "ii": T("i32", "M", "N")},
    "ops": [op("cast", ["x"], "h", to="f16"), op("cast", ["h"], "hf", to="f32"), op("mul", ["hf"], "y", mul_factor=2.0),
            op("cast", ["x"], "bi", to="bool"), op("cast", ["x"], "ii", to="i32")], "outputs": ["y", "bi", "ii"]},
    {"M": 6, "N": 20}, lambda r, b: {"x": np.where(r.random((b["M"], b["N"])) < 0.2, 0.0,
                                                   _f(r, b["M"], b["N"], scale=50.0)).astype(np.float32)})

# integer and bool inputs
case("int_and_bool_inputs", {
    "tensors": {"i": T("i32", "N"), "m": T("i1", "N"), "x": T("f32", "N"), "s": T("f32", "N"), "y": T("f32", "N")},
    "ops": [op("mul", ["x", "i"], "s"), op("where", ["m", "s", "x"], "y")], "outputs": ["y"]},
    {"N": 1000}, lambda r, b: {"i": r.integers(-50, 50, b["N"]).astype(np.int32), "m": r.random(b["N"]) < 0.5,
                               "x": _f(r, b["N"])})

# the GELU-tanh macro chain in f32 (the bf16 workload has its own kernel): a long chain
case("gelu_f32_chain", {
    "tensors": {"x": T("f32", "M", "N"), "b": T("f32", "N"), "z": T("f32", "M", "N"), "g": T("f32", "M", "N"),
                "y": T("f32", "M", "N")},
    "ops": [op("add", ["x", "b"], "z"), op("gelu_tanh", ["z"], "g"), op("add", ["g", "x"], "y")], "outputs": ["y"]},
    {"M": 8, "N": 128}, lambda r, b: {"x": _f(r, b["M"], b["N"]), "b": _f(r, b["N"], scale=0.1)})

# the logistic shape x / (exp(u) + 1), which native code evaluates in one fused step: values
# past exp's range (u > 80 and u = +-inf from x = -+inf), NaN, -0.0 and large |x| take the
# unfused fallback, the rest the fused form
def _logistic_special(r, b):
    x = (r.standard_normal(b["N"]) * 30.0).astype(np.float32)
    special = np.array([np.inf, -np.inf, np.nan, -0.0, 0.0, -60.0, 60.0, -47.0, -48.0, 3.0e38, -3.0e38, 1e-30],
                       np.float32)
    n = min(len(special), b["N"])
    x[:n] = special[:n]
    return {"x": x}


case("logistic_special", {
    "tensors": {"x": T("f32", "N"), "u": T("f32", "N"), "e": T("f32", "N"), "one": T("f32"),
                "d": T("f32", "N"), "y": T("f32", "N")},
    "ops": [op("mul", ["x"], "u", mul_factor=-1.7), op("exp", ["u"], "e"), op("const", [], "one", value=1.0, dtype="f32"),
            op("add", ["e", "one"], "d"), op("div", ["x", "d"], "y")], "outputs": ["y"]},
    {"N": 1000}, _logistic_special)

# copy of a bool tensor
case("identity_bool", {
    "tensors": {"x": T("i1", "M", "N"), "y": T("i1", "M", "N")},
    "ops": [op("identity", ["x"], "y")], "outputs": ["y"]},
    {"M": 3, "N": 31}, lambda r, b: {"x": r.random((b["M"], b["N"])) < 0.5})

# rank 0
case("scalar", {
    "tensors": {"x": T("f32"), "y": T("f32")},
    "ops": [op("mul", ["x"], "y", mul_factor=-2.5)], "outputs": ["y"]},
    {}, lambda r, b: {"x": np.array(1.75, np.float32)})

# single column: every row is one masked vector
case("single_column", {
    "tensors": {"x": T("f32", "M", "N"), "y": T("f32", "M", "N")},
    "ops": [op("exp", ["x"], "y")], "outputs": ["y"]},
    {"M": 1000, "N": 1}, lambda r, b: {"x": _f(r, b["M"], b["N"])})

# special values through max/min/relu/compare (NaN propagation, -0.0, inf)
case("special_values", {
    "tensors": {"x": T("f32", "N"), "z": T("f32"), "r": T("f32", "N"), "mx": T("f32", "N"), "ne": T("i1", "N")},
    "ops": [op("const", [], "z", value=0.0, dtype="f32"), op("relu", ["x"], "r"), op("max", ["x", "r"], "mx"),
            op("ne", ["x", "z"], "ne")], "outputs": ["mx", "ne"]},
    {"N": 8}, lambda r, b: {"x": np.array([np.nan, -0.0, 0.0, np.inf, -np.inf, -1.0, 1e-45, 3.0], np.float32)})

# division and rsqrt where the reciprocal form fails (zero, inf, NaN, denormal and huge
# divisors, overflowing quotients), mixed into vectors of ordinary values
def _div_special(r, b):
    n = b["N"]
    x, y = _f(r, n), _f(r, n)
    sx = [1.0, 3e38, -2.0, np.inf, np.nan, 1e-30, 0.0, -1.0, 5.0, 1e-45, 2.0, -np.inf]
    sy = [0.0, 1e-3, -0.0, 2.0, 1.0, 1e10, 0.0, np.inf, 1e-40, 3e-39, 1e38, np.nan]
    for i, (a, c) in enumerate(zip(sx, sy)):
        if 5 * i + 1 < n:
            x[5 * i + 1], y[5 * i + 1] = a, c
    return {"x": x, "y": y}


case("div_rsqrt_special", {
    "tensors": {"x": T("f32", "N"), "y": T("f32", "N"), "q": T("f32", "N"), "s": T("f32", "N")},
    "ops": [op("div", ["x", "y"], "q"), op("rsqrt", ["y"], "s")], "outputs": ["q", "s"]},
    {"N": 67}, _div_special)

# empty iteration space
case("empty", {
    "tensors": {"x": T("f32", "M", "N"), "y": T("f32", "M", "N")},
    "ops": [op("sub", ["x"], "y", subtract=1.0)], "outputs": ["y"]},
    {"M": 0, "N": 16}, lambda r, b: {"x": np.zeros((0, b["N"]), np.float32)})

TOL = {"f32": (1e-6, 2e-6), "f16": (1e-3, 1e-3), "bf16": (1e-3, 1e-2)}  # (atol, rtol) per output dtype

__all__ = ["CASES", "TOL"]
