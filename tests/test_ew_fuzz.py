"""Randomised element-wise chains through the program compiler and kernels.

Each seed builds an IR over x, y [M, N], a bias b [N] (aligned by its symbol), a
column c [M, 1] and a scalar attribute, with 4-14 ops drawn from the
interpreter's element-wise tables (verify/interpreter.py:16-48) and one or two
outputs.  Ops are kept well conditioned so that f32 rounding differences stay
small: exp only of non-positive values, division only by 1 + |t|, no
comparison of computed values against each other.

* CPU: the numpy model of the program kernel (tests/test_ewprogram.py) is
  judged against the oracle; it performs the same f32 operations, so this
  checks the compiler (hash-consed DAG, Sethi-Ullman order, register
  assignment by last use, broadcast strides), not rounding.
* GPU: the native and interpreted kernels, at sizes with tails, are judged
  against the oracle within f32 tolerances (bf16 outputs: one RNE rounding).

Variants: f32, bf16 or f16 x, y and outputs (16-bit operands run 8 elements per lane),
with or without an input read through transpose (the LDS-tiled form).
"""

from __future__ import annotations

import numpy as np
import pytest

from intent_ir_amd import HipLoweringError, lower_intent_to_hip_kernel
from intent_ir_amd.dtypes import bf16_bits_to_f32, f32_to_bf16_bits
from tests.test_ewprogram import oracle_outputs, run_model

UNARY = ["relu", "abs", "negate", "expneg", "sq", "floor"]
BINARY = ["add", "sub", "mul", "max", "min", "div1"]


SHAPE = {"full": ["M", "N"], "row": ["N"], "col": ["M", 1]}


def _join(a: str, b: str) -> str:
    """Shape class of a binary op's result: [N] with [M, 1] broadcasts to [M, N]."""
    return a if a == b else "full"


def random_chain(seed: int, dt: str = "f32", transpose: bool = False) -> dict:
    """dt: dtype of x, y and the outputs (b, c stay f32).  transpose: a further input z [N, M]
    enters the chain as transpose(z), which the kernels stage through LDS tiles."""
    rng = np.random.default_rng(seed)
    tensors = {"x": {"dtype": dt, "shape": SHAPE["full"]}, "y": {"dtype": dt, "shape": SHAPE["full"]},
               "b": {"dtype": "f32", "shape": SHAPE["row"]}, "c": {"dtype": "f32", "shape": SHAPE["col"]}}
    kind = {"x": "full", "y": "full", "b": "row", "c": "col"}
    ops, vals = [], ["x", "y", "b", "c"]
    if transpose:
        tensors["z"] = {"dtype": "f32", "shape": ["N", "M"]}
        tensors["zt"] = {"dtype": "f32", "shape": SHAPE["full"]}
        kind["zt"] = "full"
        ops.append({"op": "transpose", "inputs": ["z"], "output": "zt", "attrs": {"perm": [1, 0]}})
        vals.append("zt")
    n_ops = int(rng.integers(4, 15))
    k = 0

    def fresh(shape_kind):
        nonlocal k
        k += 1
        name = f"t{k}"
        tensors[name] = {"dtype": "f32", "shape": SHAPE[shape_kind]}
        kind[name] = shape_kind
        return name

    def pick():
        # favour recent values so chains get deep, but reuse old ones for shared subexpressions
        i = len(vals) - 1 - int(min(len(vals) - 1, rng.geometric(0.35) - 1))
        return vals[i]

    for _ in range(n_ops):
        if rng.random() < 0.4:
            u, a = UNARY[int(rng.integers(len(UNARY)))], pick()
            ka = kind[a]
            if u == "expneg":  # exp(-|a|) in (0, 1]
                t1, t2, out = fresh(ka), fresh(ka), fresh(ka)
                ops += [{"op": "abs", "inputs": [a], "output": t1},
                        {"op": "mul", "inputs": [t1], "output": t2, "attrs": {"mul_factor": -1.0}},
                        {"op": "exp", "inputs": [t2], "output": out}]
            elif u == "sq":
                out = fresh(ka)
                ops.append({"op": "mul", "inputs": [a, a], "output": out})
            elif u == "negate":
                out = fresh(ka)
                ops.append({"op": "mul", "inputs": [a], "output": out, "attrs": {"mul_factor": -1.0}})
            else:
                out = fresh(ka)
                ops.append({"op": u, "inputs": [a], "output": out})
        else:
            bop, a, b = BINARY[int(rng.integers(len(BINARY)))], pick(), pick()
            kab = _join(kind[a], kind[b])
            if bop == "div1":  # a / (1 + |b|)
                t1, t2, out = fresh(kind[b]), fresh(kind[b]), fresh(kab)
                ops += [{"op": "abs", "inputs": [b], "output": t1},
                        {"op": "add", "inputs": [t1], "output": t2, "attrs": {"addend": 1.0}},
                        {"op": "div", "inputs": [a, t2], "output": out}]
            elif rng.random() < 0.2:  # scalar-attribute form
                out = fresh(kind[a])
                attr = {"add": ("addend", 0.5), "sub": ("subtract", 0.25), "mul": ("mul_factor", -1.5),
                        "max": ("other", 0.1), "min": ("other", -0.1)}[bop]
                ops.append({"op": bop, "inputs": [a], "output": out, "attrs": {attr[0]: attr[1]}})
            else:
                out = fresh(kab)
                ops.append({"op": bop, "inputs": [a, b], "output": out})
        vals.append(out)
    if kind[vals[-1]] != "full":  # outputs span the whole [M, N] space
        out = fresh("full")
        ops.append({"op": "add", "inputs": [vals[-1], "x"], "output": out})
        vals.append(out)
    outs = [vals[-1]]
    if len(vals) > 6 and rng.random() < 0.4 and vals[-3] not in ("x", "y", "b", "c", "zt") and kind[vals[-3]] == "full":
        outs.append(vals[-3])
    for o in outs:
        tensors[o]["dtype"] = dt
    return {"name": f"fuzz{seed}", "tensors": tensors, "ops": ops, "outputs": outs}


def inputs_for(seed: int, M: int, N: int, dt: str = "f32", transpose: bool = False) -> dict:
    rng = np.random.default_rng(seed + 1)
    full = lambda: rng.standard_normal((M, N)).astype(np.float32)  # noqa: E731
    cast = {"f32": lambda a: a, "bf16": f32_to_bf16_bits, "f16": lambda a: a.astype(np.float16)}[dt]
    x, y = cast(full()), cast(full())
    d = {"x": x, "y": y, "b": rng.standard_normal(N).astype(np.float32),
         "c": rng.standard_normal((M, 1)).astype(np.float32)}
    if transpose:
        d["z"] = rng.standard_normal((N, M)).astype(np.float32)
    return d


def lower_or_skip(ir: dict, b: dict):
    try:
        k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    except HipLoweringError as e:
        assert "live" in str(e) or "register" in str(e), str(e)  # only the 8-register limit may refuse a chain
        pytest.skip(f"needs more than 8 live values: {e}")
    assert k.kernel_id == "ihip_elementwise_program"
    return k


VARIANTS = [("f32", False), ("f32", True), ("bf16", False), ("bf16", True), ("f16", False), ("f16", True)]
# (atol, rtol); 16-bit outputs: one RNE rounding (bf16 2^-9, f16 2^-11 relative)
TOLS = {"f32": (1e-6, 2e-6), "bf16": (1e-3, 1e-2), "f16": (1e-3, 1e-3)}


def _check(got, ref, ir, dt, what):
    atol, rtol = TOLS[dt]
    for o in ir["outputs"]:
        g = np.asarray(got[o])
        g = bf16_bits_to_f32(g) if g.dtype == np.uint16 else g.astype(np.float32)
        np.testing.assert_allclose(g.reshape(ref[o].shape), ref[o], rtol=rtol, atol=atol, err_msg=f"{what} {o}")


@pytest.mark.parametrize("dt,transpose", VARIANTS, ids=[f"{d}{'-T' if t else ''}" for d, t in VARIANTS])
@pytest.mark.parametrize("seed", range(120))
def test_random_chain_compiles_to_the_oracle(seed, dt, transpose):
    ir = random_chain(seed, dt, transpose)
    b = {"M": 5, "N": 12}
    k = lower_or_skip(ir, b)
    storage = inputs_for(seed, 5, 12, dt, transpose)
    got = run_model(k.call_args[0][1], storage, {n: t["dtype"] for n, t in ir["tensors"].items()})
    _check(got, oracle_outputs(ir, storage, b), ir, dt, f"seed {seed}")


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1], ids=["native", "interp"])
@pytest.mark.parametrize("dt,transpose", VARIANTS, ids=[f"{d}{'-T' if t else ''}" for d, t in VARIANTS])
@pytest.mark.parametrize("seed", range(0, 120, 4))
def test_random_chain_on_gpu(hip, seed, dt, transpose, mode):
    from intent_ir_amd import run_lowered

    ir = random_chain(seed, dt, transpose)
    M, N = 67, 1029 if dt == "f32" else 1032  # tails in both axes (16-bit: 8-wide vectors)
    b = {"M": M, "N": N}
    k = lower_or_skip(ir, b)
    storage = inputs_for(seed, M, N, dt, transpose)
    prev = hip.ihip_elementwise_mode(mode)
    try:
        print(f"[case] fuzz seed={seed} dt={dt} transpose={transpose} mode={mode} M={M} N={N}", flush=True)
        got = run_lowered(k, storage)
    finally:
        hip.ihip_elementwise_mode(prev)
    _check(got, oracle_outputs(ir, storage, b), ir, dt, f"seed {seed}")
