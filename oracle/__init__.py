"""CPU oracle for the IntentIR HIP backend.  TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm the HIP kernels must
match: the numpy interpreter ``verify/interpreter.py`` (``oracle.interpreter``),
the pass/fail rule of ``verify/diff_runner.py`` and the tolerance heuristic of
``verify/tolerances.py`` (``oracle.compare``), and the reference CPU execution
path of ``backends/spmd_rvv`` (``oracle/cpu_ref``, plain C, used only as the
timed CPU baseline).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import or run anything here, and only as the checker.  The product
package ``intent_ir_amd`` never imports it.

Pinning (what checks each function, beyond restating its formula):
  * golden vectors written by running the reference interpreter
    (``tests/golden/make_golden.py`` -> ``tests/golden/*.npz``);
  * the reference's own known-answer tests (ones-GEMM -> K+1,
    tests/test_diff_runner.py:35-43; softmax chain vs numpy, :73-101; tolerance
    ordering, tests/test_tolerances.py:7-39);
  * closed forms and invariants in ``tests/test_oracle.py`` (softmax shift
    invariance and row sums, LayerNorm shift invariance, GELU logistic form vs
    ``math.tanh`` in float64, brute-force reduce_any, bool/NaN/-0.0 cases).
"""
