"""The run_diff restatement (oracle/diff_runner.py) on the CPU: case generation and verdicts.

A planted-mistake runner must be caught, a correct runner (the oracle itself) must pass,
and a runner failure or a wrong input view must become a failed case."""

from __future__ import annotations

import numpy as np

from intent_ir_amd.configs import WORKLOADS
from oracle.diff_runner import EDGE_VALUES, TestCase, generate_cases, run_diff
from oracle.interpreter import execute_intent


def test_generate_cases_follows_the_reference_rule():
    ir = WORKLOADS["softmax"].ir()  # schedule tile hints + explicit ones
    cases = generate_cases(ir, limit=10 ** 6, tile_hints=[64])
    sizes = sorted({c.shapes["M"] for c in cases})
    assert {1, 2, 3, 63, 64, 65, 129} <= set(sizes)
    assert len(cases) == len(sizes) ** 2  # Cartesian product over M, N
    assert generate_cases(ir, limit=5)[0].shapes == {"M": 1, "N": 1}
    masked = generate_cases(ir, limit=3, tile_hints=[4], needs_mask=True)
    assert all(any(v % 4 for v in c.shapes.values()) for c in masked)
    assert EDGE_VALUES[:3] == [1, 2, 3]


def _oracle_runner(ir, plant=None):
    def run(case):
        w = WORKLOADS["softmax"]
        inp = w.gen(dict(case.shapes), seed=3)
        out = execute_intent(ir, inp, dict(case.shapes))
        if plant:
            out = plant(out)
        return {**inp, **out}
    return run


def test_run_diff_verdicts():
    ir = WORKLOADS["softmax"].ir()
    cases = generate_cases(ir, limit=6, tile_hints=[4])
    diffs, bad = run_diff(ir, _oracle_runner(ir), cases)
    assert len(diffs) == 6 and not bad
    diffs, bad = run_diff(ir, _oracle_runner(ir, lambda o: {"output_ptr": o["output_ptr"] * 1.001}), cases)
    assert len(bad) == 6  # a 0.1% error fails every case under the inferred softmax tolerance

    def boom(case):
        raise RuntimeError("no device")
    diffs, bad = run_diff(ir, boom, cases[:2])
    assert [d.ok for d in diffs] == [False, False] and "ref runner error" in diffs[0].summary

    def wrong_view(case):
        out = _oracle_runner(ir)(case)
        out["input_ptr"] = out["input_ptr"].reshape(-1)
        return out
    diffs, bad = run_diff(ir, wrong_view, [TestCase(shapes={"M": 4, "N": 8})])
    assert not diffs[0].ok and "input shape mismatch" in diffs[0].summary
    _, bad = run_diff(ir, boom, cases, stop_on_first_fail=True)
    assert len(bad) == 1
