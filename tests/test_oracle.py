"""Pins the CPU oracle (oracle/interpreter.py, oracle/compare.py) — CPU only.

Each check is chosen so a plausible restatement mistake (dropped term, wrong
sign, wrong axis, transposed operand, wrong promotion) fails it:
  * golden vectors written by the reference interpreter (tests/golden/*.npz);
  * the reference's own known-answer tests (tests/test_diff_runner.py:35-101,
    tests/test_tolerances.py:7-39);
  * closed forms in float64 and invariants (softmax shift/permutation,
    LayerNorm shift, GELU logistic == tanh form, brute-force reduce_any);
  * planted mistakes in a copy of the oracle that the golden vectors must catch.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from intent_ir_amd.configs import WORKLOADS, matmul_bias_relu2d_ir, softmax_inner_ir
from intent_ir_amd.dtypes import bf16_bits_to_f32, f32_to_bf16_bits, round_to_bf16, to_compute_f32
from intent_ir_amd.ir import as_intent
from oracle import interpreter as oi
from oracle.compare import LEGACY_DEFAULT, compare_outputs, infer_tolerances
from oracle.interpreter import execute_intent

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = sorted(p.stem for p in GOLDEN.glob("*.npz"))


def load_golden(name):
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    ins = {k[4:]: z[k] for k in z.files if k.startswith("in__")}
    outs = {k[5:]: z[k] for k in z.files if k.startswith("out__")}
    return meta, ins, outs


def test_golden_fixtures_present():
    assert {"workload_any", "workload_softmax", "workload_layernorm", "workload_gelu", "workload_matmul"} <= set(CASES)


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_reference_interpreter_native(name):
    """Same numpy as the fixture writer -> identical values and dtypes (matmul: BLAS order aside)."""
    meta, ins, outs = load_golden(name)
    got = execute_intent(meta["ir"], ins, meta["bindings"], numpy_semantics="native")
    for k, ref in outs.items():
        assert np.asarray(got[k]).dtype == ref.dtype, f"{name}.{k} dtype"
        if name == "workload_matmul":
            np.testing.assert_allclose(got[k], ref, rtol=1e-6, atol=1e-7)
        else:
            np.testing.assert_array_equal(np.asarray(got[k]), ref, err_msg=f"{name}.{k}")


@pytest.mark.parametrize("name", CASES)
def test_oracle_numpy126_semantics_stay_float32(name):
    """Pinned numpy 1.26 keeps f32 / 0-d int in float32; values agree with the float64 fixture to f32 precision."""
    meta, ins, outs = load_golden(name)
    got = execute_intent(meta["ir"], ins, meta["bindings"], numpy_semantics="1.26")
    for k, ref in outs.items():
        g = np.asarray(got[k])
        if ref.dtype == np.float64 and g.dtype != np.float64:
            assert g.dtype == np.float32
        if ref.dtype == np.bool_:
            np.testing.assert_array_equal(g, ref)
        else:
            np.testing.assert_allclose(g.astype(np.float64), ref.astype(np.float64), rtol=2e-6, atol=1e-6)


def test_layernorm_float64_promotion_under_numpy2_is_the_only_difference():
    meta, ins, outs = load_golden("workload_layernorm")
    assert outs["out_ptr"].dtype == np.float64  # NEP 50: f32 / np.array(N) -> f64 in numpy 2
    got = execute_intent(meta["ir"], ins, meta["bindings"])
    assert got["out_ptr"].dtype == np.float32


# ------------------------------------------------------------- planted mistakes
def _golden_catches() -> bool:
    """True when some golden vector disagrees with (or breaks) the current oracle."""
    for name in CASES:
        meta, ins, outs = load_golden(name)
        try:
            got = execute_intent(meta["ir"], ins, meta["bindings"], numpy_semantics="native")
            for k, ref in outs.items():
                g = np.asarray(got[k], dtype=np.float64)
                if g.shape != ref.shape or not np.allclose(g, ref.astype(np.float64), rtol=1e-5, atol=1e-6,
                                                           equal_nan=True) or not np.array_equal(np.signbit(g),
                                                                                                 np.signbit(ref)):
                    return True
        except Exception:
            return True
    return False


def test_unplanted_oracle_passes_all_goldens():
    assert not _golden_catches()


@pytest.mark.parametrize("op,wrong", [("sub", np.add), ("div", np.multiply), ("max", np.minimum),
                                      ("add", np.subtract), ("mul", np.add)])
def test_planted_arithmetic_mistake_is_caught(monkeypatch, op, wrong):
    monkeypatch.setitem(oi.NUM_BIN_OPS, op, wrong)
    assert _golden_catches(), f"a wrong '{op}' went unnoticed by every golden vector"


@pytest.mark.parametrize("table,op,wrong", [
    ("NUM_BIN_OPS", "max", np.fmax), ("NUM_BIN_OPS", "min", np.fmin), ("NUM_BIN_OPS", "div", np.floor_divide),
    ("NUM_UNARY_OPS", "floor", np.ceil), ("NUM_UNARY_OPS", "floor", np.trunc),
    ("NUM_UNARY_OPS", "relu", lambda x: np.fmax(x, 0)), ("NUM_UNARY_OPS", "relu", lambda x: np.maximum(0, x)),
    ("NUM_UNARY_OPS", "rsqrt", lambda x: np.sqrt(1.0 / x)), ("NUM_UNARY_OPS", "exp", np.exp2),
    ("CMP_BIN_OPS", "lt", np.less_equal), ("CMP_BIN_OPS", "ge", np.greater), ("CMP_BIN_OPS", "ne", np.equal),
    ("BOOL_BIN_OPS", "and", np.logical_xor), ("BOOL_BIN_OPS", "or", np.logical_xor)])
def test_planted_elementwise_table_mistake_is_caught(monkeypatch, table, op, wrong):
    """The elementwise_tables fixture (reference interpreter on NaN, +-inf, +-0, denormals)
    catches plausible table mistakes: NaN-dropping fmax/fmin, ceil or trunc for floor, a
    relu that returns +0 for -0 or drops NaN, reordered rsqrt, comparisons off by equality."""
    import warnings

    monkeypatch.setitem(getattr(oi, table), op, wrong)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        assert _golden_catches(), f"a wrong '{op}' went unnoticed by every golden vector"


def test_planted_wrong_cast_is_caught(monkeypatch):
    """cast to i32 truncates toward zero (astype); rounding instead must be caught."""
    import warnings

    orig = oi._Exec.op

    def op(self, o, env):
        if o.op == "cast" and o.attrs.get("to") == "i32":
            return np.rint(np.asarray(env[o.inputs[0]])).astype(np.int32)
        return orig(self, o, env)

    monkeypatch.setattr(oi._Exec, "op", op)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        assert _golden_catches()


def test_planted_wrong_reduce_axis_is_caught(monkeypatch):
    monkeypatch.setattr(oi._Exec, "resolve_dims", staticmethod(lambda raw, x: (0,) if x.ndim > 1 else (0,)))
    assert _golden_catches()


def test_planted_wrong_broadcast_alignment_is_caught(monkeypatch):
    monkeypatch.setattr(oi._Exec, "_match_axis", lambda self, v, t, r: None)  # numpy trailing alignment only
    assert _golden_catches()


def test_planted_transposed_matmul_is_caught(monkeypatch):
    orig = oi._Exec.op

    def op(self, o, env):
        if o.op == "matmul":
            a, b = np.asarray(env[o.inputs[0]]), np.asarray(env[o.inputs[1]])
            return (b.T @ a.T).T if a.shape[0] == b.shape[1] else np.matmul(a, b) * 1.0001
        return orig(self, o, env)

    monkeypatch.setattr(oi._Exec, "op", op)
    assert _golden_catches()


# ------------------------------------------------------------- reference known answers
def test_known_answer_gemm_ones():
    """tests/test_diff_runner.py:35-43."""
    M, K, N = 2, 3, 4
    out = execute_intent(matmul_bias_relu2d_ir(), {"A": np.ones((M, K), np.float32), "B": np.ones((K, N), np.float32),
                                                   "bias": np.ones(N, np.float32)})
    assert out["C"].shape == (M, N) and np.all(out["C"] == K + 1.0)


def test_known_answer_softmax_chain():
    """tests/test_diff_runner.py:73-101: reduce result [M] broadcasts row-wise by symbol."""
    ir = {"name": "sm", "tensors": {n: {"dtype": "f32", "shape": s} for n, s in
                                    {"X": ["M", "N"], "mx": ["M"], "Xc": ["M", "N"], "E": ["M", "N"], "sm": ["M"],
                                     "out": ["M", "N"]}.items()},
          "ops": [{"op": "reduce_max", "inputs": ["X"], "output": "mx", "attrs": {"axis": [1], "keepdims": False}},
                  {"op": "sub", "inputs": ["X", "mx"], "output": "Xc"}, {"op": "exp", "inputs": ["Xc"], "output": "E"},
                  {"op": "reduce_sum", "inputs": ["E"], "output": "sm", "attrs": {"axis": [1], "keepdims": False}},
                  {"op": "div", "inputs": ["E", "sm"], "output": "out"}], "outputs": ["out"]}
    X = np.arange(6, dtype=np.float32).reshape(2, 3)
    out = execute_intent(ir, {"X": X})["out"]
    E = np.exp(X - X.max(axis=1, keepdims=True))
    np.testing.assert_allclose(out, E / E.sum(axis=1, keepdims=True), atol=1e-6, rtol=1e-6)


def test_tolerance_ordering_matches_reference():
    """tests/test_tolerances.py:7-39."""
    sm = as_intent({"name": "s", "tensors": {"x": {"dtype": "f32", "shape": ["M", "N"]}, "y": {"dtype": "f32", "shape": ["M", "N"]}},
                    "ops": [{"op": "softmax", "inputs": ["x"], "output": "y", "attrs": {"axis": 1}}], "outputs": ["y"]})
    t = infer_tolerances(sm)
    assert t.atol < 1e-3 and t.rtol < 1e-3
    mm = as_intent({"name": "m", "tensors": {"A": {"dtype": "f16", "shape": ["M", "K"]}, "B": {"dtype": "f16", "shape": ["K", "N"]},
                                             "C": {"dtype": "f32", "shape": ["M", "N"]}},
                    "ops": [{"op": "matmul", "inputs": ["A", "B"], "output": "C"}], "outputs": ["C"]})
    t = infer_tolerances(mm)
    assert t.atol > 1e-3 and t.rtol > 1e-3
    any_ir = as_intent(WORKLOADS["any"].ir())
    assert infer_tolerances(any_ir).to_dict() == {"atol": 1e-4, "rtol": 1e-4}  # start value wins over reduce_any's 0
    ln = as_intent(WORKLOADS["layernorm"].ir())
    assert infer_tolerances(ln) == LEGACY_DEFAULT  # f16 tensors floor at the legacy 1e-3 (tolerances.py:111-113)
    mm = as_intent(WORKLOADS["matmul"].ir())
    assert infer_tolerances(mm).to_dict() == {"atol": 2e-2, "rtol": 2e-2}


def test_compare_rules():
    r = {"y": np.array([1.0, 2.0, np.nan], np.float32), "b": np.array([True, False])}
    assert compare_outputs({"y": np.array([1.0, 2.0, np.nan], np.float32)}, r, ["y"], {"atol": 0, "rtol": 0}).summary \
        == "non-finite values mismatch in y"  # NaN never equals NaN in the reference rule
    assert not compare_outputs({"b": np.array([True, True])}, r, ["b"], {"atol": 1, "rtol": 1}).ok
    ok = compare_outputs({"y": np.array([[1.0005]], np.float32)}, {"y": np.array([1.0], np.float32)}, ["y"],
                         {"atol": 1e-3, "rtol": 0})
    assert ok.ok  # unit-dim squeeze (diff_runner.py:368-376)
    bad = compare_outputs({"y": np.array([1.0, 3.0], np.float32)}, {"y": np.array([1.0, 2.0], np.float32)}, ["y"],
                          {"atol": 1e-3, "rtol": 1e-3})
    assert not bad.ok and bad.first_bad_index == (1,)


# ------------------------------------------------------------- closed forms / invariants
def _run(key, b, inp):
    fn = as_intent(WORKLOADS[key].ir())
    return execute_intent(WORKLOADS[key].ir(), {n: to_compute_f32(v, fn.tensors[n].dtype) for n, v in inp.items()}, b)


def test_reduce_any_brute_force():
    b = {"M": 6, "N": 9}
    x = np.zeros((6, 9), np.float32)
    x[0, 3], x[1, 8], x[2, 0], x[3, 4], x[4, 1] = 1.0, -0.0, np.nan, np.float32(1e-45), np.inf
    got = _run("any", b, {"inp": x})["out"]
    brute = [any(float(v) != 0.0 or math.isnan(float(v)) for v in row) for row in x]
    assert got.tolist() == brute == [True, False, True, True, True, False]


def test_softmax_closed_form_and_invariants():
    b = {"M": 5, "N": 33}
    x = WORKLOADS["softmax"].gen(b)["input_ptr"]
    y = _run("softmax", b, {"input_ptr": x})["output_ptr"]
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    np.testing.assert_allclose(y, e / e.sum(axis=1, keepdims=True), rtol=1e-5, atol=1e-12)
    np.testing.assert_allclose(y.sum(axis=1), 1.0, atol=1e-6)
    y_shift = _run("softmax", b, {"input_ptr": x + np.float32(3.0)})["output_ptr"]  # verify/metamorphic.py:350-406
    np.testing.assert_allclose(y_shift, y, rtol=1e-4, atol=1e-9)
    y_rev = _run("softmax", b, {"input_ptr": x[:, ::-1].copy()})["output_ptr"]
    np.testing.assert_allclose(y_rev, y[:, ::-1], rtol=1e-6, atol=1e-12)


def test_layernorm_closed_form_and_shift():
    b = {"M": 4, "N": 64}
    inp = WORKLOADS["layernorm"].gen(b)
    out = _run("layernorm", b, inp)
    x = inp["in_ptr"].astype(np.float64)
    w, bb = inp["weight_ptr"].astype(np.float64), inp["bias_ptr"].astype(np.float64)
    mu = x.mean(axis=1)
    var = ((x - mu[:, None]) ** 2).mean(axis=1)
    rstd = 1 / np.sqrt(var + 1e-5)
    np.testing.assert_allclose(out["out_mean_ptr"], mu, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(out["out_rstd_ptr"], rstd, rtol=1e-5)
    np.testing.assert_allclose(out["out_ptr"], (x - mu[:, None]) * rstd[:, None] * w + bb, rtol=1e-5, atol=1e-6)
    sh = dict(inp, in_ptr=(inp["in_ptr"].astype(np.float32) + 2.0).astype(np.float16))
    out2 = _run("layernorm", b, sh)  # verify/metamorphic.py:409-482
    exact = np.all(sh["in_ptr"].astype(np.float32) - 2.0 == inp["in_ptr"].astype(np.float32), axis=1)
    np.testing.assert_allclose(out2["out_rstd_ptr"][exact], out["out_rstd_ptr"][exact], rtol=1e-4)
    np.testing.assert_allclose(out2["out_mean_ptr"][exact], out["out_mean_ptr"][exact] + 2.0, atol=1e-5)


def test_gelu_chain_equals_tanh_form():
    b = {"M": 2, "N": 64}
    x = np.linspace(-6, 6, 128, dtype=np.float32).reshape(2, 64)
    bias = np.linspace(-0.05, 0.05, 64, dtype=np.float32)
    inp = {"x": f32_to_bf16_bits(x), "bias": f32_to_bf16_bits(bias)}
    y = _run("gelu", b, inp)["y"].astype(np.float64)
    xf, bf = bf16_bits_to_f32(inp["x"]).astype(np.float64), bf16_bits_to_f32(inp["bias"]).astype(np.float64)
    z = xf + bf
    tanh_form = np.vectorize(lambda v: 0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3))))(z)
    np.testing.assert_allclose(y, 0.5 * tanh_form + xf, rtol=1e-5, atol=1e-6)


def test_matmul_bias_relu_brute_force():
    b = {"M": 3, "N": 4, "K": 5}
    inp = WORKLOADS["matmul"].gen(b, sigma=1.0)
    C = _run("matmul", b, inp)["C"]
    A, B = bf16_bits_to_f32(inp["A"]).astype(np.float64), bf16_bits_to_f32(inp["B"]).astype(np.float64)
    brute = np.array([[max(0.0, sum(A[i, k] * B[k, j] for k in range(5)) + inp["bias"][j]) for j in range(4)]
                      for i in range(3)])
    np.testing.assert_allclose(C, brute, rtol=1e-5, atol=1e-6)


def test_bf16_rounding_is_rne():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -2.5, 3.0e38, np.inf, np.nan], np.float32)
    r = round_to_bf16(vals)
    assert r[0] == 1.0 and r[1] == 1.0  # tie to even
    assert r[2] == np.float32(1.0 + 4 * 2 ** -8)  # tie to even (up)
    assert r[3] == 1.0 and r[4] == -2.5 and np.isinf(r[6]) and np.isnan(r[7])
    assert np.isinf(round_to_bf16(np.array([3.4e38], np.float32)))[0]  # overflow rounds to inf


def test_softmax_ir_validates_like_reference():
    from intent_ir_amd.ir import IntentIRValidationError
    bad = softmax_inner_ir()
    bad["ops"][0]["attrs"] = {"axis": "last"}
    with pytest.raises(IntentIRValidationError):
        as_intent(bad)
