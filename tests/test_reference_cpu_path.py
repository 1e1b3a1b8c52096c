"""The oracle agrees with the reference's own CPU execution path (CPU only).

oracle/build_ref.py compiles the reference codegen tool and C runtime from the
reference tree into oracle/_ref/; each `<cfg>_tiny` program is the C program the
reference generates for that workload IR.  Feeding it the oracle's outputs as
`<out>_ref.bin` must make it print "PASS lowered" (its own compare rule:
backends/spmd_rvv/runtime/intentir_runtime.c:32-61, atol = rtol = 1e-3; bool exact).
Skipped where oracle/_ref was not built (no reference tree at build time).
"""

from __future__ import annotations

import numpy as np
import pytest

from intent_ir_amd.configs import WORKLOADS
from intent_ir_amd.dtypes import to_compute_f32
from intent_ir_amd.ir import as_intent
from intent_ir_amd.macros import expand_macros
from oracle import ref_runner
from oracle.interpreter import execute_intent


@pytest.mark.parametrize("key", sorted(WORKLOADS))
def test_reference_c_path_accepts_oracle_outputs(key):
    if not ref_runner.available(key, "tiny"):
        pytest.skip("oracle/_ref not built (python oracle/build_ref.py)")
    w = WORKLOADS[key]
    b = ref_runner.bindings(key, "tiny")
    fn = expand_macros(as_intent(w.ir()))
    raw = w.gen(b, seed=7)
    f32 = {n: to_compute_f32(v, fn.tensors[n].dtype) for n, v in raw.items()}
    ref = execute_intent(w.ir(), f32, b)
    r = ref_runner.run(key, "tiny", fn, f32, ref)
    assert r.passed, r.stdout


def test_reference_c_path_rejects_a_wrong_answer():
    """A planted error in the oracle's output is caught by the reference program."""
    if not ref_runner.available("softmax", "tiny"):
        pytest.skip("oracle/_ref not built")
    w = WORKLOADS["softmax"]
    b = ref_runner.bindings("softmax", "tiny")
    fn = as_intent(w.ir())
    f32 = w.gen(b, seed=3)
    ref = execute_intent(w.ir(), f32, b)
    bad = {"output_ptr": ref["output_ptr"] * np.float32(1.01)}
    assert not ref_runner.run("softmax", "tiny", fn, f32, bad).passed
