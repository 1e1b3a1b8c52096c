#!/usr/bin/env python3
"""Write golden vectors by running the REFERENCE interpreter (verify/interpreter.py).

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py /root/reference [case ...]

For each case it stores the IntentIR document (after this backend's macro
expansion, which only emits ops the reference interpreter knows), the inputs
and the reference outputs in ``tests/golden/<case>.npz``, plus the numpy
version that produced them.  The cases cover what no closed form pins:
end-to-end ``execute_intent`` on the five workload IRs at tiny bindings, and the
interpreter's helpers for 1-D/2-D alignment by symbol name, reduce-dims
fallback, string-valued consts, 1-input scalar-attr ops and reduce scale, and
every element-wise table entry, where, cast and iota on special values.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))


def _cases():
    from intent_ir_amd.configs import WORKLOADS
    from intent_ir_amd.dtypes import to_compute_f32
    from intent_ir_amd.ir import as_intent
    from intent_ir_amd.macros import expand_macros

    tiny = {"any": {"M": 5, "N": 33}, "softmax": {"M": 4, "N": 17}, "layernorm": {"M": 3, "N": 24},
            "gelu": {"M": 3, "N": 16}, "matmul": {"M": 3, "N": 5, "K": 7}}
    for key, b in tiny.items():
        w = WORKLOADS[key]
        fn = expand_macros(as_intent(w.ir()))
        inp = w.gen(b, seed=100 + len(key))
        if key == "any":
            inp["inp"][1, :] = 0.0
            inp["inp"][2, 7] = -0.0
            inp["inp"][3, 3] = 2.5
        f32 = {n: to_compute_f32(v, fn.tensors[n].dtype) for n, v in inp.items()}
        yield f"workload_{key}", fn.to_json_dict(), f32, b

    def t(dt, shape):
        return {"dtype": dt, "shape": shape, "layout": "row_major"}

    # 1-D vs 2-D alignment by declared symbol (interpreter.py:752-841): [M] joins axis 0, [N] joins axis 1.
    yield "align_by_symbol", {
        "name": "align", "tensors": {"X": t("f32", ["M", "N"]), "r": t("f32", ["M"]), "c": t("f32", ["N"]),
                                     "a": t("f32", ["M", "N"]), "y": t("f32", ["M", "N"])},
        "ops": [{"op": "sub", "inputs": ["X", "r"], "output": "a"}, {"op": "mul", "inputs": ["a", "c"], "output": "y"}],
        "outputs": ["y"]}, {"X": np.arange(12, dtype=np.float32).reshape(3, 4), "r": np.array([1, 2, 3], np.float32),
                            "c": np.array([1, -1, 2, 0.5], np.float32)}, {"M": 3, "N": 4}
    # Square case, distinct symbols: still resolved by name (R and C both bind 3).
    yield "align_square_by_name", {
        "name": "align_sq", "tensors": {"X": t("f32", ["R", "C"]), "v": t("f32", ["R"]), "y": t("f32", ["R", "C"])},
        "ops": [{"op": "add", "inputs": ["X", "v"], "output": "y"}], "outputs": ["y"]}, \
        {"X": np.arange(9, dtype=np.float32).reshape(3, 3), "v": np.array([10, 20, 30], np.float32)}, {"R": 3, "C": 3}
    # Reduce dims given as strings / unusable -> fallback to all non-leading axes (interpreter.py:676-694).
    yield "reduce_dims_fallback", {
        "name": "rdf", "tensors": {"X": t("f32", ["A", "B", "C"]), "s": t("f32", ["A"]), "m": t("f32", ["A", "C"])},
        # The validator reads "dims"; the interpreter reads "axes" first, so "axes" carries the odd forms.
        "ops": [{"op": "reduce_sum", "inputs": ["X"], "output": "s", "attrs": {"axes": ["rows"], "dims": [1]}},
                {"op": "reduce_max", "inputs": ["X"], "output": "m", "attrs": {"axes": ["1"], "dims": [2]}}],
        "outputs": ["s", "m"]}, {"X": np.linspace(-3, 3, 24, dtype=np.float32).reshape(2, 3, 4)}, {"A": 2, "B": 3, "C": 4}
    # String-valued consts: binding symbol, numeric string, "eps", expression (interpreter.py:521-544);
    # 1-input scalar-attr ops (:215-226) and reduce scale (:646-673).
    yield "const_and_scalar_attrs", {
        "name": "consts", "tensors": {"X": t("f32", ["M", "N"]), "cn": t("f32", []), "cs": t("f32", []),
                                      "ce": t("f32", []), "cx": t("f32", []), "y1": t("f32", ["M", "N"]),
                                      "y2": t("f32", ["M", "N"]), "y3": t("f32", ["M", "N"]), "y4": t("f32", ["M", "N"]),
                                      "y5": t("f32", ["M", "N"]), "y6": t("f32", ["M", "N"]), "s": t("f32", ["M"])},
        "ops": [{"op": "const", "inputs": [], "output": "cn", "attrs": {"value": "N", "dtype": "f32"}},
                {"op": "const", "inputs": [], "output": "cs", "attrs": {"value": "0.25", "dtype": "f32"}},
                {"op": "const", "inputs": [], "output": "ce", "attrs": {"value": "eps", "dtype": "f32"}},
                {"op": "const", "inputs": [], "output": "cx", "attrs": {"value": "M*N+1", "dtype": "f32"}},
                {"op": "div", "inputs": ["X"], "output": "y1", "attrs": {"divisor": "N"}},
                {"op": "add", "inputs": ["y1"], "output": "y2", "attrs": {"addend": 1.5}},
                {"op": "sub", "inputs": ["y2"], "output": "y3", "attrs": {"subtract": "cs"}},
                {"op": "mul", "inputs": ["y3"], "output": "y4", "attrs": {"mul_factor": "2"}},
                {"op": "max", "inputs": ["y4"], "output": "y5", "attrs": {"other": 0.0}},
                {"op": "add", "inputs": ["y5", "cx"], "output": "y6"},
                {"op": "reduce_sum", "inputs": ["y6"], "output": "s", "attrs": {"dims": [1], "scale": "1/N"}}],
        "outputs": ["cn", "ce", "y6", "s"]}, {"X": np.linspace(-2, 2, 15, dtype=np.float32).reshape(3, 5)}, \
        {"M": 3, "N": 5}
    # Every element-wise table entry (interpreter.py:14-47), where, cast, iota, transpose and
    # reshape (:253-302) on special values: NaN, +-inf, +-0, denormals, ties, overflow.
    X = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.5, -1.5, 2.0, -2.5, 0.5, 3.75, -7.25, 100.0, -100.0, 1e-3,
                  -1e-3, 2.0, 3.0, -3.0, 0.0, 5.5, -0.5, 88.0, -88.0, 1e-40, -1e-40, 7.0, 0.25, -0.25, 65504.0, 1e30,
                  -1e30], np.float32).reshape(4, 8)
    Y = np.array([1.0, np.inf, 2.0, -0.0, 0.0, 1.5, 1.5, np.nan, -2.5, 0.25, -3.75, 7.25, 100.0, 50.0, -1e-3, 1e-3,
                  2.0, -3.0, -3.0, 1.0, -5.5, 0.5, 1.0, -1.0, 1e-40, 0.0, -7.0, 4.0, 0.25, 2.0, -1e30, 1e30],
                 np.float32).reshape(4, 8)
    Z = np.array([-2.5, -1.5, -0.5, 0.5, 1.5, 2.5, -0.0, 0.0, 1.0 / 3, -2.0 / 3, 2049.0, 2051.0, 65519.0, -65521.0,
                  6e-8, -6e-8, 1e-5, 7.9999, -7.9999, 123.456, 1e4, -1e4, 0.099975586, 1.0009766, 2.999, -2.999,
                  0.25, -0.75, 1023.5, -1023.5, 3e-5, 5.96e-8], np.float32).reshape(4, 8)
    full = ["M", "N"]
    tens = {"X": t("f32", full), "Y": t("f32", full), "Z": t("f32", full), "tr": t("f32", ["N", "M"]),
            "rs": t("f32", ["N", "M"]), "io": t("i32", full), "k_i32": t("i32", full), "k_f16": t("f16", full),
            "k_bool": t("bool", full), "w": t("f32", full)}
    ops = []
    for o in ("add", "sub", "mul", "div", "max", "min"):
        tens[f"b_{o}"] = t("f32", full)
        ops.append({"op": o, "inputs": ["X", "Y"], "output": f"b_{o}"})
    for o in ("relu", "exp", "rsqrt", "abs", "floor", "identity"):
        tens[f"u_{o}"] = t("f32", full)
        ops.append({"op": o, "inputs": ["X"], "output": f"u_{o}"})
    for o in ("ne", "lt", "le", "gt", "ge"):
        tens[f"c_{o}"] = t("bool", full)
        ops.append({"op": o, "inputs": ["X", "Y"], "output": f"c_{o}"})
    for name, o, ins in (("l_and", "and", ["c_lt", "c_ne"]), ("l_or", "or", ["c_le", "c_ge"]), ("l_not", "not", ["c_ne"])):
        tens[name] = t("bool", full)
        ops.append({"op": o, "inputs": ins, "output": name})
    ops += [{"op": "where", "inputs": ["c_lt", "X", "Y"], "output": "w"},
            {"op": "cast", "inputs": ["Z"], "output": "k_i32", "attrs": {"to": "i32"}},
            {"op": "cast", "inputs": ["Z"], "output": "k_f16", "attrs": {"to": "f16"}},
            {"op": "cast", "inputs": ["X"], "output": "k_bool", "attrs": {"to": "bool"}},
            {"op": "iota", "inputs": [], "output": "io", "attrs": {"shape": full, "axis": 1, "dtype": "i32"}},
            {"op": "transpose", "inputs": ["X"], "output": "tr", "attrs": {"perm": [1, 0]}},
            {"op": "reshape", "inputs": ["Z"], "output": "rs", "attrs": {"shape": ["N", "M"]}}]
    outs = [o["output"] for o in ops]
    yield "elementwise_tables", {"name": "ew_tables", "tensors": tens, "ops": ops, "outputs": outs}, \
        {"X": X, "Y": Y, "Z": Z}, {"M": 4, "N": 8}


def main(ref_root: str, only: set | None = None) -> None:
    sys.path.insert(0, ref_root)
    from intent_ir.ir import IntentFunction  # reference
    from verify.interpreter import execute_intent  # reference

    for name, ir, inputs, bindings in _cases():
        if only and name not in only:
            continue
        fn = IntentFunction.from_json_dict(ir)
        out = execute_intent(fn, {k: np.asarray(v) for k, v in inputs.items()}, dict(bindings))
        blob = {f"in__{k}": np.asarray(v) for k, v in inputs.items()}
        blob.update({f"out__{k}": np.asarray(v) for k, v in out.items()})
        blob["meta"] = np.frombuffer(json.dumps({"ir": ir, "bindings": bindings, "numpy": np.__version__}).encode(),
                                     dtype=np.uint8)
        np.savez_compressed(HERE / f"{name}.npz", **blob)
        print(f"wrote {name}: " + ", ".join(f"{k}{np.shape(v)}:{np.asarray(v).dtype}" for k, v in out.items()))


if __name__ == "__main__":
    # usage: make_golden.py [reference_root] [case ...]   (no case names: every case)
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", set(sys.argv[2:]) or None)
