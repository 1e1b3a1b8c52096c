"""The element-wise program kernels against the reference interpreter's own outputs.

tests/golden/elementwise_tables.npz holds what verify/interpreter.py computed for every
element-wise table entry (:14-47), where, cast, iota and transpose (:253-302) on NaN, +-inf,
+-0, denormals, ties and overflow.  Each output is lowered on its own (with the ops it depends
on) and run through both kernel modes.  NaN must meet NaN and the sign of zero must match;
values are bit-exact except div, exp and rsqrt, which meet the f32 element-wise tolerance.
One exception to the sign of zero: max/min of +0 and -0.  numpy returns one of the two
equal operands depending on its loop (numpy 2.2 the second; the reference pins 1.26), the
kernels follow IEEE maximum/minimum (-0 < +0), and the reference's compare rule
(verify/diff_runner.py:407-417) treats the two zeros as equal.
The fixture's reshape [M, N] -> [N, M] moves data between axes, which the lowering rejects.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from intent_ir_amd import HipLoweringError, lower_intent_to_hip_kernel

FIXTURE = Path(__file__).resolve().parent / "golden" / "elementwise_tables.npz"
ROUNDED = {"b_div": (1e-6, 2e-6), "u_exp": (1e-6, 2e-6), "u_rsqrt": (1e-6, 2e-6)}  # (atol, rtol)


def _load():
    z = np.load(FIXTURE, allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    ins = {k[4:]: z[k] for k in z.files if k.startswith("in__")}
    outs = {k[5:]: z[k] for k in z.files if k.startswith("out__")}
    return meta, ins, outs


def sub_ir(ir: dict, out: str) -> dict:
    """The ops `out` depends on, as an IR of their own with `out` as its only output."""
    prod = {o["output"]: o for o in ir["ops"]}
    need, seen = [out], set()
    while need:
        n = need.pop()
        if n in prod and n not in seen:
            seen.add(n)
            need += prod[n]["inputs"]
    ops = [o for o in ir["ops"] if o["output"] in seen]
    names = {n for o in ops for n in o["inputs"] + [o["output"]]}
    return {"name": f"golden_{out}", "tensors": {n: ir["tensors"][n] for n in names}, "ops": ops, "outputs": [out]}


META, INS, OUTS = _load()
NAMES = [o for o in META["ir"]["outputs"] if o != "rs"]


def test_reshape_across_axes_is_rejected():
    with pytest.raises(HipLoweringError, match="reshape"):
        lower_intent_to_hip_kernel(sub_ir(META["ir"], "rs"), shape_bindings=META["bindings"])


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1], ids=["native", "interp"])
@pytest.mark.parametrize("out", NAMES)
def test_program_matches_reference_interpreter(hip, out, mode):
    from intent_ir_amd import run_lowered

    ir = sub_ir(META["ir"], out)
    k = lower_intent_to_hip_kernel(ir, shape_bindings=META["bindings"])
    assert k.kernel_id == "ihip_elementwise_program"
    inputs = {n: v for n, v in INS.items() if n in ir["tensors"]}
    prev = hip.ihip_elementwise_mode(mode)
    try:
        print(f"[case] golden element-wise {out} mode={mode}", flush=True)
        got = np.asarray(run_lowered(k, inputs)[out])
    finally:
        hip.ihip_elementwise_mode(prev)
    ref = OUTS[out]
    got = got.reshape(ref.shape)
    if ref.dtype == np.bool_:
        np.testing.assert_array_equal(got.astype(bool), ref, err_msg=out)
        return
    if ref.dtype.kind in "iu":
        np.testing.assert_array_equal(got.astype(ref.dtype), ref, err_msg=out)
        return
    g = got.astype(np.float64)
    r = ref.astype(np.float64)
    np.testing.assert_array_equal(np.isnan(g), np.isnan(r), err_msg=f"{out}: NaN positions")
    np.testing.assert_array_equal(np.isinf(g) * np.sign(g), np.isinf(r) * np.sign(r), err_msg=f"{out}: inf positions")
    zero = g == 0
    if out in ("b_max", "b_min"):  # ties of +0 and -0: numpy's pick is loop-dependent
        x, y = INS["X"].astype(np.float64), INS["Y"].astype(np.float64)
        zero &= ~((x == 0) & (y == 0))
    np.testing.assert_array_equal(np.signbit(g[zero]), np.signbit(r[zero]), err_msg=f"{out}: sign of zero")
    if out in ROUNDED:
        atol, rtol = ROUNDED[out]
        np.testing.assert_allclose(g, r, rtol=rtol, atol=atol, equal_nan=True, err_msg=out)
    else:
        np.testing.assert_array_equal(g, r, err_msg=out)  # bit-exact up to the sign of zero checked above
