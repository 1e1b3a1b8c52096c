"""Differential runner: the oracle interpreter against a kernel runner, per test case.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): tests import this to judge the
HIP backend the way the reference judges its backends.

Restates, for the paths this build runs:
  * ``TestCase`` / ``EDGE_VALUES`` / ``generate_cases`` (verify/gen_cases.py:17-27,178-274,
    277-293): per symbolic axis the sizes {1,2,3} and, for every schedule tile hint t,
    {t-1, t, t+1, 2t+1}; the deterministic Cartesian product truncated to ``limit``;
    ``needs_mask`` moves a non-divisible size first;
  * ``run_diff`` (verify/diff_runner.py:37-275): run the reference runner on a case, take
    the true external inputs from what it returns, check them against the declared
    shapes (strict original view), evaluate the oracle on them and compare with the
    reference rule (oracle.compare.compare_outputs = diff_runner.py:357-418); a runner or
    interpreter exception becomes a failed case, not an error.
The reference's alias repairs for LLM-named tensors and derived symbols
(diff_runner.py:96-190) have no counterpart: the IR here is written, not lifted.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from itertools import product
from typing import Any, Callable, Dict, Iterable, List, Optional, Sequence, Tuple

import numpy as np

from intent_ir_amd.ir import as_intent, resolve_shape
from intent_ir_amd.macros import expand_macros

from .compare import DiffResult, compare_outputs, infer_tolerances
from .interpreter import execute_intent

EDGE_VALUES = [1, 2, 3, 7, 8, 15, 16, 17, 31, 32, 33]  # verify/gen_cases.py:27


@dataclass
class TestCase:
    shapes: Dict[str, int]
    dtypes: Dict[str, str] = field(default_factory=dict)
    seed: int = 0
    inputs: Optional[Dict[str, np.ndarray]] = None
    __test__ = False  # not a pytest class


@dataclass
class Counterexample:
    case: TestCase
    diff: DiffResult
    hints: List[str]


def _axes(fn) -> List[str]:
    """gen_cases.py:277-283: every symbolic dim of every tensor."""
    out = set()
    for t in fn.tensors.values():
        for d in t.shape:
            if d.kind == "sym":
                out.add(d.value)
    return sorted(out)


def _tile_hints(fn) -> List[int]:
    """gen_cases.py:286-293: tile_m, tile_n, tile_k, vec_width of the schedule, else [16]."""
    tiles = []
    sch = getattr(fn, "schedule", None)
    if sch is not None:
        for k in ("tile_m", "tile_n", "tile_k", "vec_width"):
            v = getattr(sch, k, None)
            if isinstance(v, int):
                tiles.append(v)
    return tiles or [16]


def generate_cases(intent, *, limit: int = 10, seed: int = 0, tile_hints: Sequence[int] = (),
                   extra_sizes: Sequence[int] = (), needs_mask: bool = False,
                   axes: Optional[Sequence[str]] = None) -> List[TestCase]:
    fn = as_intent(intent)
    axes_list = list(axes) if axes is not None else _axes(fn)
    tiles = [int(t) for t in tile_hints] + _tile_hints(fn)
    if not axes_list:
        return [TestCase(shapes={}, seed=seed)]
    per_axis = []
    for _ in axes_list:
        vals = set(EDGE_VALUES[:3])
        for t in tiles:
            if t > 0:
                vals.update([max(1, t - 1), t, t + 1, 2 * t + 1])
        vals.update(int(x) for x in extra_sizes if int(x) > 0)
        ordered = sorted(vals)
        if needs_mask:
            ordered = sorted(ordered, key=lambda v: (all(v % t == 0 for t in tiles if t > 1), v))
        per_axis.append(ordered)
    cases: List[TestCase] = []
    for combo in product(*per_axis):
        shapes = dict(zip(axes_list, combo))
        if needs_mask and all(all(shapes[a] % t == 0 for t in tiles if t > 1) for a in axes_list):
            continue
        cases.append(TestCase(shapes=shapes, seed=seed))
        if len(cases) >= limit:
            break
    return cases


def run_diff(intent, run_ref_fn: Callable[[TestCase], Dict[str, np.ndarray]], cases: Iterable[TestCase],
             tolerances: Optional[Dict[str, float]] = None,
             stop_on_first_fail: bool = False) -> Tuple[List[DiffResult], List[Counterexample]]:
    fn = expand_macros(as_intent(intent))
    tol = None if tolerances is None else dict(tolerances)
    produced = {op.output for op in fn.ops}
    used = {i for op in fn.ops for i in op.inputs}
    external = {n for n in used if n in fn.tensors and n not in produced}
    diffs: List[DiffResult] = []
    bad: List[Counterexample] = []

    def fail(case, summary, hint):
        d = DiffResult(False, 0.0, 0.0, None, summary)
        diffs.append(d)
        bad.append(Counterexample(case, d, [hint]))

    for case in cases:
        try:
            ref = run_ref_fn(case)
        except Exception as e:  # noqa: BLE001 - a runner failure is a failed case (diff_runner.py:69-94)
            fail(case, f"ref runner error: {type(e).__name__}: {e}", "runner failed on this case")
            if stop_on_first_fail:
                break
            continue
        if tol is None:
            tol = infer_tolerances(fn, ref_out=ref).to_dict()
        bindings = dict(case.shapes)
        inputs = {k: v for k, v in ref.items() if k in external}
        mismatch = None
        for name, arr in inputs.items():
            try:
                want = resolve_shape(fn.tensors[name], bindings)
            except KeyError:
                mismatch = f"unbound symbols in input shape for {name}"
                break
            if tuple(np.shape(arr)) != tuple(want):
                mismatch = f"input shape mismatch for {name}: ref {np.shape(arr)} vs intent {tuple(want)}"
                break
        if mismatch:
            fail(case, mismatch, "keep the original input view")
            if stop_on_first_fail:
                break
            continue
        try:
            with np.errstate(all="ignore"):
                pred = execute_intent(fn.to_json_dict(), inputs, bindings)
            d = compare_outputs(pred, ref, fn.outputs, tol)
        except Exception as e:  # noqa: BLE001 (diff_runner.py:249-262)
            d = DiffResult(False, 0.0, 0.0, None, f"interpreter error: {type(e).__name__}: {e}")
        diffs.append(d)
        if not d.ok:
            bad.append(Counterexample(case, d, ["check ops, broadcasts and reduce axes"]))
            if stop_on_first_fail:
                break
    return diffs, bad


__all__ = ["EDGE_VALUES", "TestCase", "Counterexample", "generate_cases", "run_diff"]
