"""Pass/fail rule and tolerance heuristic of the reference verifier.  TEST INFRASTRUCTURE ONLY.

* ``compare_outputs``  restates ``_compare_outputs`` (verify/diff_runner.py:357-418)
  with its unit-dim squeeze/unsqueeze alignment (:420-484).
* ``infer_tolerances`` restates verify/tolerances.py:68-129 with the per-op table
  of :34-47.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Mapping, Optional, Sequence, Tuple

import numpy as np


@dataclass
class DiffResult:
    ok: bool
    max_abs_err: float
    max_rel_err: float
    first_bad_index: Optional[Tuple[int, ...]]
    summary: str


@dataclass(frozen=True)
class Tolerances:
    atol: float
    rtol: float

    def to_dict(self) -> Dict[str, float]:
        return {"atol": float(self.atol), "rtol": float(self.rtol)}


# verify/tolerances.py:34-47
OP_TOL_F32 = {
    "softmax": Tolerances(1e-4, 1e-4), "exp": Tolerances(3e-4, 3e-4), "rsqrt": Tolerances(3e-4, 3e-4),
    "matmul": Tolerances(2e-2, 2e-2), "reduce_sum": Tolerances(1e-3, 1e-3), "reduce_max": Tolerances(1e-3, 1e-3),
    "reduce_any": Tolerances(0.0, 0.0),
}
LEGACY_DEFAULT = Tolerances(1e-3, 1e-3)  # verify/tolerances.py:50


def _dtype_kind(dt) -> str:
    d = np.dtype(dt)
    if d == np.float16:
        return "f16"
    if d == np.float32:
        return "f32"
    if d == np.float64:
        return "f64"
    if d == np.bool_:
        return "bool"
    if np.issubdtype(d, np.integer):
        return "int"
    return str(d)


def infer_tolerances(fn, ref_out: Optional[Mapping[str, np.ndarray]] = None) -> Tolerances:
    """verify/tolerances.py:68-129: max over the op table, f16/bf16 floor, matmul-aware cap."""
    n_mm = sum(1 for o in fn.ops if o.op == "matmul")
    tol = Tolerances(1e-4, 1e-4)
    for o in fn.ops:
        t = OP_TOL_F32.get(o.op)
        if t is not None:
            tol = Tolerances(max(tol.atol, t.atol), max(tol.rtol, t.rtol))
    if n_mm > 1:
        base = 2e-2 * (1.0 + 0.5 * (n_mm - 1))
        tol = Tolerances(max(tol.atol, base), max(tol.rtol, base))
    kinds = set()
    if ref_out is not None:
        for name in set(fn.outputs) | set(fn.tensors):
            if name in ref_out:
                kinds.add(_dtype_kind(np.asarray(ref_out[name]).dtype))
    else:
        kinds = {t.dtype for t in fn.tensors.values()}
    if "f16" in kinds or "bf16" in kinds:
        tol = Tolerances(max(tol.atol, LEGACY_DEFAULT.atol), max(tol.rtol, LEGACY_DEFAULT.rtol))
    if tol.atol == 0.0 and tol.rtol == 0.0:
        return LEGACY_DEFAULT
    cap = LEGACY_DEFAULT
    if n_mm > 0:
        c = 2e-2 * (1.0 + 0.5 * max(0, n_mm - 1))
        cap = Tolerances(max(cap.atol, c), max(cap.rtol, c))
    return Tolerances(min(max(tol.atol, 0.0), cap.atol), min(max(tol.rtol, 0.0), cap.rtol))


def _squeeze_to(arr: np.ndarray, shape: Tuple[int, ...]) -> Optional[np.ndarray]:
    """diff_runner.py:420-456: drop only size-1 dims of ``arr`` to reach ``shape``."""
    p = tuple(arr.shape)
    if p == shape:
        return arr
    if len(p) < len(shape):
        return None
    drop, i, j = [], 0, 0
    while i < len(p) and j < len(shape):
        if p[i] == shape[j]:
            i, j = i + 1, j + 1
        elif p[i] == 1:
            drop.append(i)
            i += 1
        else:
            return None
    while i < len(p):
        if p[i] != 1:
            return None
        drop.append(i)
        i += 1
    if j != len(shape) or not drop:
        return None
    s = np.squeeze(arr, axis=tuple(drop))
    return s if tuple(s.shape) == shape else None


def _unsqueeze_to(arr: np.ndarray, shape: Tuple[int, ...]) -> Optional[np.ndarray]:
    """diff_runner.py:459-484: insert only size-1 dims of ``arr`` to reach ``shape``."""
    p = tuple(arr.shape)
    if p == shape:
        return arr
    if len(p) > len(shape):
        return None
    new, i = [], 0
    for d in shape:
        if i < len(p) and p[i] == d:
            new.append(d)
            i += 1
        elif d == 1:
            new.append(1)
        else:
            return None
    if i != len(p):
        return None
    return np.reshape(arr, tuple(new))


def compare_outputs(pred: Mapping[str, np.ndarray], ref: Mapping[str, np.ndarray], outputs: Sequence[str],
                    tol: Mapping[str, float]) -> DiffResult:
    """verify/diff_runner.py:357-418.

    bool outputs must match exactly; non-finite patterns and values must match;
    otherwise every finite element must satisfy |p - r| <= atol + rtol*|r|."""
    max_abs = max_rel = 0.0
    for name in outputs:
        if name not in ref:
            return DiffResult(False, max_abs, max_rel, None, f"reference missing output {name}")
        if name not in pred:
            return DiffResult(False, max_abs, max_rel, None, f"missing output {name}")
        r = np.asarray(ref[name])
        p = np.asarray(pred[name])
        if p.shape != r.shape:
            p2 = _squeeze_to(p, tuple(r.shape))
            if p2 is None:
                p2 = _unsqueeze_to(p, tuple(r.shape))
            if p2 is None:
                return DiffResult(False, max_abs, max_rel, None, f"shape mismatch for {name}: {p.shape} vs {r.shape}")
            p = p2
        if r.dtype == bool or p.dtype == bool:
            neq = p.astype(bool) != r.astype(bool)
            if neq.any():
                bi = tuple(int(v) for v in np.unravel_index(int(np.argmax(neq)), neq.shape))
                return DiffResult(False, float("inf"), float("inf"), bi, f"mismatch in {name} (bool)")
            continue
        pn, rn = ~np.isfinite(p), ~np.isfinite(r)
        if pn.any() or rn.any():
            if not np.array_equal(pn, rn):
                return DiffResult(False, float("inf"), float("inf"), None, f"non-finite pattern mismatch in {name}")
            if not np.array_equal(p[pn], r[rn]):
                return DiffResult(False, float("inf"), float("inf"), None, f"non-finite values mismatch in {name}")
        fin = ~(pn | rn)
        pf, rf = p.astype(np.float64), r.astype(np.float64)
        abs_err = np.zeros(r.shape, dtype=np.float64)
        abs_err[fin] = np.abs(pf[fin] - rf[fin])
        rel_err = np.zeros(r.shape, dtype=np.float64)
        rel_err[fin] = abs_err[fin] / (np.abs(rf[fin]) + 1e-8)
        max_abs = max(max_abs, float(abs_err.max()) if abs_err.size else 0.0)
        max_rel = max(max_rel, float(rel_err.max()) if rel_err.size else 0.0)
        thresh = float(tol.get("atol", 1e-3)) + float(tol.get("rtol", 1e-3)) * np.abs(rf)
        viol = (abs_err > thresh) & fin
        if viol.any():
            margin = np.where(viol, abs_err - thresh, -np.inf)
            bi = tuple(int(v) for v in np.unravel_index(int(np.argmax(margin)), margin.shape))
            return DiffResult(False, max_abs, max_rel, bi, f"mismatch in {name}")
    return DiffResult(True, max_abs, max_rel, None, "ok")


__all__ = ["DiffResult", "Tolerances", "OP_TOL_F32", "LEGACY_DEFAULT", "infer_tolerances", "compare_outputs"]
