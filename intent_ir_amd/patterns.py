"""Structural view of an IntentIR function for pattern matching.

The CUDA lowering of the reference picks its kernel from the op-name sequence
and, for LayerNorm, from the output names (backends/cuda/codegen/
intentir_to_cuda.py:2157-2168).  This module instead rebuilds, for every output,
the expression it computes in terms of external inputs and constants, with
shape-only ops folded into explicit broadcasts.  Kernel families are then
recognised by unifying those expressions with templates, so the choice depends
on what the IR computes, not on how its ops are named, ordered or whether a
reduction keeps its dims.

Expression trees are nested tuples:
  ("in", name)                      external input
  ("const", value)                  scalar constant (float)
  (op, child, ...)                  element-wise op (add, mul, exp, ...)
  ("rsum"|"rmax"|"rany", child, axes)
  ("bcast", child, kept_axes, rank) value placed on ``kept_axes`` of a rank-``rank`` result
  ("softmax", child, axis)
  ("matmul", a, b, transpose_a, transpose_b)

Broadcast semantics follow the reference interpreter: a 1-D operand next to an
n-D one is placed on the axis whose declared symbol it names
(verify/interpreter.py:752-841), falling back to numpy's trailing-axis rule;
kept unit dims (keepdims reductions, [M,1] tensors) broadcast along themselves.
"""

from __future__ import annotations

import ast
import math
import operator
from dataclasses import dataclass
from typing import Any, Dict, List, Mapping, Optional, Sequence, Tuple

from .ir import IntentFunction, Op, SCALAR_ATTR_OF, reduce_dims_attr

COMMUTATIVE = frozenset({"add", "mul", "max", "min", "ne", "and", "or"})
BINARY = frozenset({"add", "sub", "mul", "div", "max", "min", "ne", "lt", "le", "gt", "ge", "and", "or"})
UNARY = frozenset({"exp", "relu", "rsqrt", "abs", "floor", "not"})


class PatternError(ValueError):
    """The IR cannot be put in the structural form (unsupported op or shape use)."""


@dataclass(frozen=True)
class Val:
    tree: Any
    rank: int
    unit: Tuple[int, ...] = ()  # axes of size 1 that broadcast (kept reduction dims)

    def full(self) -> Any:
        """Tree of this value with its unit axes expanded to a full-rank operand."""
        if not self.unit:
            return self.tree
        kept = tuple(a for a in range(self.rank) if a not in self.unit)
        return ("bcast", self.tree, kept, self.rank)


def _num(v: Any, bindings: Mapping[str, Any]) -> Optional[float]:
    if isinstance(v, bool):
        return float(v)
    if isinstance(v, (int, float)):
        return float(v)
    if isinstance(v, str):
        if v in bindings:
            return float(bindings[v])
        try:
            return float(v)
        except ValueError:
            return 1e-5 if v == "eps" else None
    return None


_SCALE_BINOPS = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul, ast.Div: operator.truediv,
                 ast.Pow: operator.pow, ast.FloorDiv: operator.floordiv, ast.Mod: operator.mod}


def reduce_scale_factor(scale: Any, bindings: Mapping[str, Any]) -> float:
    """The factor of reduce_sum{scale} as the interpreter resolves it (verify/interpreter.py:646-673):
    a number; a binding name; or an arithmetic expression over numbers and bindings (such as
    "1.0/N"), with num_elements = group_size * HW when both are bound.  The interpreter hands
    the expression to Python's eval; here it is parsed and only numbers, bound names, + - * /
    // % ** and parentheses are accepted, so an unresolvable scale raises PatternError."""
    if isinstance(scale, bool) or not isinstance(scale, (int, float, str)):
        raise PatternError(f"unsupported reduce scale {scale!r}")
    if not isinstance(scale, str):
        return float(scale)
    names = dict(bindings)
    if "num_elements" not in names and isinstance(names.get("group_size"), int) and isinstance(names.get("HW"), int):
        names["num_elements"] = names["group_size"] * names["HW"]
    if scale in names:
        return float(names[scale])

    def ev(node: ast.AST) -> Any:
        if isinstance(node, ast.Expression):
            return ev(node.body)
        if isinstance(node, ast.Constant) and isinstance(node.value, (int, float)) and not isinstance(node.value, bool):
            return node.value
        if isinstance(node, ast.Name) and isinstance(names.get(node.id), (int, float)):
            return names[node.id]
        if isinstance(node, ast.BinOp) and type(node.op) in _SCALE_BINOPS:
            lhs, rhs = ev(node.left), ev(node.right)
            if isinstance(node.op, ast.Pow) and abs(rhs) > 64:
                raise PatternError(f"reduce scale {scale!r}: exponent {rhs} out of range")
            return _SCALE_BINOPS[type(node.op)](lhs, rhs)
        if isinstance(node, ast.UnaryOp) and isinstance(node.op, (ast.USub, ast.UAdd)):
            v = ev(node.operand)
            return -v if isinstance(node.op, ast.USub) else v
        raise PatternError(f"unresolved reduce scale {scale!r}")

    try:
        return float(ev(ast.parse(scale.strip(), mode="eval")))
    except (SyntaxError, ZeroDivisionError, OverflowError, ValueError) as e:
        raise PatternError(f"unresolved reduce scale {scale!r}: {e}") from e


class ExprBuilder:
    """Turns each op output into a ``Val`` (expression tree + rank + unit axes)."""

    def __init__(self, fn: IntentFunction, bindings: Mapping[str, Any]):
        self.fn = fn
        self.b = dict(bindings)
        self.env: Dict[str, Val] = {}
        for op in fn.ops:
            self.env[op.output] = self._op(op)

    # -- declared-shape helpers (interpreter.py:771-821 axis matching) -------
    def _tokens(self, name: str) -> Optional[List[Any]]:
        t = self.fn.tensors.get(name)
        return None if t is None else [d.value for d in t.shape]

    def _resolved(self, tok: Any) -> Optional[int]:
        if isinstance(tok, int):
            return tok
        if isinstance(tok, str) and tok in self.b:
            return int(self.b[tok])
        return None

    def _match_axis(self, vec: str, ten: str, rank: int) -> Optional[int]:
        v, t = self._tokens(vec), self._tokens(ten)
        if not v or len(v) != 1 or not t or len(t) != rank:
            return None
        if isinstance(v[0], str):
            hits = [i for i, x in enumerate(t) if x == v[0]]
            if len(hits) == 1:
                return hits[0]
        vn = self._resolved(v[0])
        if vn is None:
            return None
        hits = [i for i, x in enumerate(t) if self._resolved(x) == vn]
        return hits[0] if len(hits) == 1 else None

    def get(self, name: str) -> Val:
        if name in self.env:
            return self.env[name]
        t = self.fn.tensors.get(name)
        if t is None:
            raise PatternError(f"undeclared input {name}")
        unit = tuple(i for i, d in enumerate(t.shape) if d.kind == "const" and d.value == 1 and t.rank > 1)
        return Val(("in", name), t.rank, unit)

    # -- broadcasting of two operands ---------------------------------------
    def _pair(self, an: Optional[str], a: Val, bn: Optional[str], b: Val) -> Tuple[Any, Any, Val]:
        if a.rank == 0 or b.rank == 0:
            big = b if a.rank == 0 else a
            return a.tree, b.tree, Val(None, big.rank, big.unit)
        if a.rank == b.rank:
            if a.unit == b.unit:
                return a.tree, b.tree, Val(None, a.rank, a.unit)
            return a.full(), b.full(), Val(None, a.rank, ())
        lo, hi, lo_n, hi_n, swap = (a, b, an, bn, False) if a.rank < b.rank else (b, a, bn, an, True)
        if lo.rank != 1 or lo.unit:
            raise PatternError("only 1-D operands broadcast against higher rank")
        ax = self._match_axis(lo_n, hi_n, hi.rank) if (lo_n and hi_n) else None
        if ax is None:
            ax = hi.rank - 1  # numpy trailing alignment
        wrapped = ("bcast", lo.tree, (ax,), hi.rank)
        hi_t = hi.full()
        return (hi_t, wrapped, Val(None, hi.rank, ())) if swap else (wrapped, hi_t, Val(None, hi.rank, ()))

    def _norm_axes(self, raw: Any, rank: int) -> Tuple[int, ...]:
        if raw is None:
            return tuple(range(rank))
        dims = [raw] if isinstance(raw, int) else list(raw)
        out = []
        for d in dims:
            if isinstance(d, str) and d.isdigit():
                d = int(d)
            if not isinstance(d, int):
                continue
            out.append(d + rank if d < 0 else d)
        if not out:  # the interpreter's fallback: all non-leading axes (interpreter.py:691-693)
            out = list(range(1, rank))
        if any(not (0 <= d < rank) for d in out):
            raise PatternError(f"reduce axes {dims} out of range for rank {rank}")
        return tuple(sorted(set(out)))

    def _shape_of_attr(self, s: Sequence[Any]) -> Tuple[Optional[int], ...]:
        return tuple(self._resolved(x) if not (isinstance(x, str) and x.isdigit()) else int(x) for x in s)

    # -- ops ------------------------------------------------------------------
    def _op(self, op: Op) -> Val:  # noqa: C901
        name, ins, at = op.op, op.inputs, op.attrs or {}
        if name == "const":
            v = _num(at.get("value"), self.b)
            if v is None:
                raise PatternError(f"const {op.output} has no numeric value")
            return Val(("const", v), 0)
        if name in ("identity", "layout_cast"):
            return self.get(ins[0])
        if name == "reshape":
            src = self.get(ins[0])
            tgt = self._shape_of_attr(at.get("shape") or [])
            src_decl = self._tokens(ins[0])
            src_shape = tuple(self._resolved(x) for x in src_decl) if src_decl else None
            if src_shape is None or None in src_shape or None in tgt:
                raise PatternError("reshape with unresolved shape")
            nz = lambda s: [d for d in s if d != 1]  # noqa: E731
            if nz(src_shape) != nz(tgt):
                raise PatternError("reshape that moves data between axes")
            kept_src = [i for i, d in enumerate(src_shape) if d != 1]
            if src.unit and any(i in src.unit for i in kept_src):
                raise PatternError("reshape of a broadcast value")
            return Val(src.tree, len(tgt), tuple(i for i, d in enumerate(tgt) if d == 1 and len(tgt) > 1))
        if name == "broadcast_in_dim":
            src = self.get(ins[0])
            out_rank = len(at.get("out_shape") or [])
            bd = tuple(int(x) for x in at.get("broadcast_dims") or [])
            if len(bd) != src.rank:
                raise PatternError("broadcast_in_dim dims do not cover the input rank")
            if src.rank == 0:
                return Val(src.tree, 0)
            src_decl = self._tokens(ins[0]) or []
            src_shape = [self._resolved(x) for x in src_decl]
            out_shape = self._shape_of_attr(at.get("out_shape") or [])
            # A source dim is kept unless a size-1 dim is stretched to a larger output dim.
            kept = tuple(d for d, s in zip(bd, src_shape) if not (s == 1 and out_shape[d] != 1)) if src_shape else bd
            inner = src.tree
            if src.unit:  # a [M,1] value: its unit axes are broadcast now
                kept = tuple(bd[i] for i in range(src.rank) if i not in src.unit)
            if kept == tuple(range(out_rank)):
                return Val(inner, out_rank)
            return Val(("bcast", inner, kept, out_rank), out_rank)
        if name in BINARY:
            args = list(ins)
            if len(args) == 1 and SCALAR_ATTR_OF.get(name) in at:
                v = _num(at[SCALAR_ATTR_OF[name]], self.b)
                if v is None:
                    if at[SCALAR_ATTR_OF[name]] in self.env:
                        args.append(at[SCALAR_ATTR_OF[name]])
                    else:
                        raise PatternError(f"{name} scalar attr unresolved")
                else:
                    a = self.get(args[0])
                    return Val((name, a.tree, ("const", v)), a.rank, a.unit)
            a, b = self.get(args[0]), self.get(args[1])
            ta, tb, shape = self._pair(args[0], a, args[1], b)
            if name == "max" and tb == ("const", 0.0):
                return Val(("relu", ta), shape.rank, shape.unit)
            return Val((name, ta, tb), shape.rank, shape.unit)
        if name in UNARY:
            a = self.get(ins[0])
            return Val((name, a.tree), a.rank, a.unit)
        if name == "cast":  # interpreter.py:270-273
            a = self.get(ins[0])
            return Val(("cast", a.tree, str(at.get("to"))), a.rank, a.unit)
        if name == "where":  # interpreter.py:292-302
            return self._where(ins)
        if name == "transpose":  # interpreter.py:258-263
            a = self.get(ins[0])
            perm = tuple(int(p) for p in at.get("perm") or [])
            if sorted(perm) != list(range(a.rank)):
                raise PatternError(f"transpose perm {perm} does not fit rank {a.rank}")
            return Val(("transpose", a.full(), perm), a.rank)
        if name == "iota":  # interpreter.py:274-283
            shp = at.get("shape") or []
            axis = int(at.get("axis", 0))
            if not 0 <= axis < len(shp):
                raise PatternError(f"iota axis {axis} out of range")
            return Val(("iota", axis, len(shp)), len(shp))
        if name in ("reduce_sum", "reduce_max", "reduce_any"):
            a = self.get(ins[0])
            axes = self._norm_axes(reduce_dims_attr(at), a.rank)
            kind = {"reduce_sum": "rsum", "reduce_max": "rmax", "reduce_any": "rany"}[name]
            if name == "reduce_sum" and at.get("reduction_type") == "any":
                kind = "rany"
            tree = (kind, a.full(), axes)
            if name == "reduce_sum" and kind == "rsum" and at.get("scale") is not None:
                # the sum times the scale factor (interpreter.py:487, :646-673)
                tree = ("mul", tree, ("const", reduce_scale_factor(at["scale"], self.b)))
            if at.get("keepdims"):
                return Val(tree, a.rank, axes)
            return Val(tree, a.rank - len(axes))
        if name == "softmax":
            a = self.get(ins[0])
            ax = int(at.get("axis", -1))
            return Val(("softmax", a.full(), ax + a.rank if ax < 0 else ax), a.rank)
        if name == "matmul":
            a, b = self.get(ins[0]), self.get(ins[1])
            mm = Val(("matmul", a.full(), b.full(), bool(at.get("transpose_a")), bool(at.get("transpose_b"))), 2)
            ep = at.get("epilogue")
            return self._epilogue(ep, mm) if ep else mm
        raise PatternError(f"op {name} has no structural form")

    def _where(self, ins: Sequence[str]) -> Val:
        """np.where after the interpreter's pairwise name-based alignment: 1-D operands go
        on the axis of a full-rank operand whose declared symbol they name, else the
        trailing axis; scalars broadcast."""
        if len(ins) != 3:
            raise PatternError("where takes (cond, x, y)")
        vals = [self.get(n) for n in ins]
        rank = max(v.rank for v in vals)
        big = next(n for n, v in zip(ins, vals) if v.rank == rank)
        trees = []
        for n, v in zip(ins, vals):
            if v.rank == rank or v.rank == 0:
                trees.append(v.full())
            elif v.rank == 1 and not v.unit:
                ax = self._match_axis(n, big, rank)
                trees.append(("bcast", v.tree, (rank - 1 if ax is None else ax,), rank))
            else:
                raise PatternError("where operands of mixed rank > 1")
        return Val(("where", *trees), rank)

    def _epilogue(self, node: Any, x: Val) -> Val:
        """matmul epilogue trees (interpreter.py:567-591): plain numpy broadcasting."""
        if isinstance(node, str):
            if node == "$x":
                return x
            v = self.get(node)
            if v.rank == 1:
                return Val(("bcast", v.tree, (1,), 2), 2)
            return v
        op, args = node.get("op"), [self._epilogue(i, x) for i in node.get("inputs", [])]
        if op in BINARY and len(args) == 2:
            if op == "max" and args[1].tree == ("const", 0.0):
                return Val(("relu", args[0].tree), 2)
            return Val((op, args[0].tree, args[1].tree), 2)
        if op in UNARY and len(args) == 1:
            return Val((op, args[0].tree), args[0].rank)
        raise PatternError(f"epilogue op {op} has no structural form")


# ---------------------------------------------------------------- unification
def unify(tree: Any, tmpl: Any, env: Dict[str, Any]) -> Optional[Dict[str, Any]]:
    """Match ``tree`` against ``tmpl``; placeholders bind consistently.

    Placeholders: ("?", k) any subtree; ("?in", k) an external input;
    ("?c", k) a constant.  Commutative ops are tried in both operand orders."""
    if isinstance(tmpl, tuple) and tmpl and tmpl[0] in ("?", "?in", "?c"):
        kind, key = tmpl
        if kind == "?in" and not (isinstance(tree, tuple) and tree[0] == "in"):
            return None
        if kind == "?c" and not (isinstance(tree, tuple) and tree[0] == "const"):
            return None
        if key in env:
            return env if env[key] == tree else None
        out = dict(env)
        out[key] = tree
        return out
    if isinstance(tmpl, tuple):
        if not isinstance(tree, tuple) or len(tree) != len(tmpl) or tree[0] != tmpl[0]:
            return None
        orders = [tree[1:]]
        if tree[0] in COMMUTATIVE and len(tree) == 3:
            orders.append((tree[2], tree[1]))
        for kids in orders:
            e: Optional[Dict[str, Any]] = env
            for t_kid, p_kid in zip(kids, tmpl[1:]):
                e = unify(t_kid, p_kid, e)
                if e is None:
                    break
            if e is not None:
                return e
        return None
    return env if tree == tmpl else None


def close(a: float, b: float, rel: float = 1e-6) -> bool:
    return math.isclose(float(a), float(b), rel_tol=rel, abs_tol=0.0)


__all__ = ["ExprBuilder", "Val", "PatternError", "unify", "close", "COMMUTATIVE", "reduce_scale_factor"]
