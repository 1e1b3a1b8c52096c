"""Compile element-wise expression trees into the register program run by
``ihip_elementwise_program`` (include/intentir_hip.h, IHIP_EW_*).

The reference lowers a fused element-wise chain by emitting one CUDA kernel
per chain (backends/cuda/codegen/intentir_to_cuda.py:229-534).  This backend
runs every such chain on one precompiled gfx950 kernel and passes the chain
as a short program: a DAG of the outputs' expression trees (common
subexpressions shared), scheduled in Sethi-Ullman order and given registers
by last use.  A chain within the interpreter kernel's limits (``MAX_*``: 64
instructions, 8 live values, 8 inputs, 4 outputs) runs in every execution
mode; a larger one is compiled for the native form's limits (``NATIVE_MAX_*``)
and runs only as hiprtc-compiled code.

Index maps: broadcasts, transposes and kept unit dims of the expression trees
(``patterns.py``) are pushed down to the leaves, so every input is read
through per-axis element strides over the iteration space (stride 0 =
broadcast).  Nothing is materialised.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, List, Mapping, Optional, Sequence, Tuple

MAX_CODE, MAX_REGS, MAX_INPUTS, MAX_OUTPUTS, MAX_RANK = 64, 8, 8, 4, 4
# The native (hiprtc) form's limits, include/intentir_hip.h IHIP_EW_NATIVE_MAX_*: a program
# over the interpreter limits above runs only as native code.
NATIVE_MAX_CODE, NATIVE_MAX_REGS, NATIVE_MAX_INPUTS, NATIVE_MAX_OUTPUTS = 1024, 255, 32, 8

# Opcodes of include/intentir_hip.h.
OP = {
    "load": 1, "imm": 2, "iota": 3, "store": 4, "mov": 5,
    "add": 10, "sub": 11, "mul": 12, "div": 13, "max": 14, "min": 15,
    "ne": 20, "lt": 21, "le": 22, "gt": 23, "ge": 24, "eq": 25,
    "and": 30, "or": 31, "not": 32,
    "relu": 40, "exp": 41, "rsqrt": 42, "abs": 43, "floor": 44, "neg": 45,
    "where": 50,
    "cast_f16": 60, "cast_bf16": 61, "cast_bool": 62, "cast_i32": 63,
}
BINARY = ("add", "sub", "mul", "div", "max", "min", "ne", "lt", "le", "gt", "ge", "and", "or")
UNARY = ("not", "relu", "exp", "rsqrt", "abs", "floor")

# Element types of include/intentir_hip.h (IHIP_DT_*).
DTYPE_CODE = {"f32": 0, "f16": 1, "bf16": 2, "bool": 3, "i1": 3, "i32": 4}

# `cast{to}` as the reference interpreter evaluates it (x.astype(_np_dtype(to)),
# verify/interpreter.py:270-273 and :81-106): bf16 maps to numpy float16 there,
# so a cast to bf16 rounds to f16.
CAST_OP = {"f16": "cast_f16", "bf16": "cast_f16", "f32": None, "f64": None, "bool": "cast_bool", "i1": "cast_bool",
           "i32": "cast_i32", "i64": "cast_i32"}


class EwCompileError(ValueError):
    """The trees are not an element-wise chain the program kernel runs."""


class EwLimitError(EwCompileError):
    """The chain is element-wise but exceeds the limits it was compiled for."""


@dataclass(frozen=True)
class EwProgram:
    code: Tuple[Tuple[int, int, int, int, int, float], ...]  # (op, dst, a, b, c, imm)
    inputs: Tuple[Tuple[str, Tuple[int, int, int, int]], ...]  # (tensor, element strides over the rank-4 space)
    outputs: Tuple[str, ...]
    shape: Tuple[int, ...]  # iteration shape, rank 0..4

    def listing(self) -> List[str]:
        names = {v: k for k, v in OP.items()}
        out = []
        for op, d, a, b, c, imm in self.code:
            n = names[op]
            if n == "load":
                out.append(f"r{d} = load {self.inputs[a][0]} strides={self.inputs[a][1]}")
            elif n == "imm":
                out.append(f"r{d} = {imm!r}")
            elif n == "iota":
                out.append(f"r{d} = iota axis {a}")
            elif n == "store":
                out.append(f"{self.outputs[b]} = r{a}")
            elif n == "where":
                out.append(f"r{d} = where r{a} r{b} r{c}")
            elif n in BINARY:
                out.append(f"r{d} = {n} r{a} r{b}")
            else:
                out.append(f"r{d} = {n} r{a}")
        return out


def _contiguous_strides(shape: Sequence[int]) -> List[int]:
    st, acc = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        st[i] = acc
        acc *= int(shape[i])
    return st


class _Dag:
    """Hash-consed nodes: (kind, payload, child ids)."""

    def __init__(self) -> None:
        self.nodes: List[Tuple[str, Any, Tuple[int, ...]]] = []
        self.index: Dict[Tuple[str, Any, Tuple[int, ...]], int] = {}

    def add(self, kind: str, payload: Any = None, kids: Tuple[int, ...] = ()) -> int:
        key = (kind, payload, kids)
        if key not in self.index:
            self.index[key] = len(self.nodes)
            self.nodes.append(key)
        return self.index[key]


class _Builder:
    def __init__(self, shape: Tuple[int, ...], decl: Mapping[str, Tuple[int, ...]],
                 units: Mapping[str, Tuple[int, ...]], max_inputs: int = MAX_INPUTS):
        self.max_inputs = max_inputs
        self.shape = shape
        self.rank = len(shape)
        self.decl = decl
        self.units = units
        self.dag = _Dag()
        self.inputs: List[Tuple[str, Tuple[int, int, int, int]]] = []

    def _pad(self, axis: int) -> int:
        return MAX_RANK - self.rank + axis

    def _leaf(self, name: str, amap: Tuple[int, ...]) -> int:
        if name not in self.decl:
            raise EwCompileError(f"input {name} has no resolved shape")
        shp = self.decl[name]
        unit = self.units.get(name, ())
        if len(shp) == 0:  # a rank-0 tensor: one element, broadcast over every axis (stride 0)
            amap = ()
        if len(shp) != len(amap):
            # a value with kept unit dims ([M,1]) is placed by its other axes only
            if len(shp) - len(unit) != len(amap):
                raise EwCompileError(f"input {name} of rank {len(shp)} used at rank {len(amap)}")
            it = iter(amap)
            amap = tuple(-1 if j in unit else next(it) for j in range(len(shp)))
        st4 = [0, 0, 0, 0]
        for j, (d, cs) in enumerate(zip(shp, _contiguous_strides(shp))):
            ax = amap[j]
            if d == 1 or ax < 0:
                continue  # size-1 axis: broadcast
            if d != self.shape[ax]:
                raise EwCompileError(f"input {name} axis {j} has size {d}, iteration axis {ax} has {self.shape[ax]}")
            st4[self._pad(ax)] += cs
        key = (name, tuple(st4))
        if key not in self.inputs:
            if len(self.inputs) == self.max_inputs:
                raise EwLimitError(f"more than {self.max_inputs} distinct input views")
            self.inputs.append(key)
        return self.dag.add("load", self.inputs.index(key))

    def node(self, tree: Any, amap: Tuple[int, ...]) -> int:  # noqa: C901
        if not isinstance(tree, tuple) or not tree:
            raise EwCompileError(f"not an expression: {tree!r}")
        k = tree[0]
        if k == "in":
            return self._leaf(tree[1], amap)
        if k == "const":
            return self.dag.add("imm", float(tree[1]))
        if k == "bcast":
            _, child, kept, rank = tree
            if len(amap) != rank:
                raise EwCompileError("broadcast rank mismatch")
            return self.node(child, tuple(amap[a] for a in kept))
        if k == "transpose":
            _, child, perm = tree
            inner = [0] * len(perm)
            for i, p in enumerate(perm):
                inner[p] = amap[i]
            return self.node(child, tuple(inner))
        if k == "iota":
            _, axis, rank = tree
            if len(amap) != rank:
                raise EwCompileError("iota rank mismatch")
            return self.dag.add("iota", self._pad(amap[axis]))
        if k == "cast":
            _, child, to = tree
            if to not in CAST_OP:
                raise EwCompileError(f"cast to {to} is not lowered")
            c = self.node(child, amap)
            return c if CAST_OP[to] is None else self.dag.add(CAST_OP[to], None, (c,))
        if k == "where":
            return self.dag.add("where", None, tuple(self.node(t, amap) for t in tree[1:]))
        if k in BINARY:
            return self.dag.add(k, None, (self.node(tree[1], amap), self.node(tree[2], amap)))
        if k in UNARY:
            return self.dag.add(k, None, (self.node(tree[1], amap),))
        raise EwCompileError(f"{k} is not element-wise")


def fits_interpreter(prog: EwProgram) -> bool:
    """True when the program runs on the interpreter kernel too (every mode); else it needs
    the native form (capi.hip fits_interpreter)."""
    regs = [d for op, d, *_ in prog.code if op != OP["store"]]
    return (len(prog.code) <= MAX_CODE and len(prog.inputs) <= MAX_INPUTS and len(prog.outputs) <= MAX_OUTPUTS
            and (max(regs) if regs else 0) < MAX_REGS)


def _schedule(dag: _Dag, roots: Sequence[int]) -> List[int]:
    """Post-order over the DAG, children needing more registers first (Sethi-Ullman)."""
    need: Dict[int, int] = {}

    def regs(n: int) -> int:
        if n not in need:
            kids = dag.nodes[n][2]
            if not kids:
                need[n] = 1
            else:
                ks = sorted((regs(c) for c in kids), reverse=True)
                need[n] = max(max(r + i for i, r in enumerate(ks)), len(kids))
        return need[n]

    order: List[int] = []
    seen = set()

    def visit(n: int) -> None:
        if n in seen:
            return
        for c in sorted(dag.nodes[n][2], key=regs, reverse=True):
            visit(c)
        seen.add(n)
        order.append(n)

    for r in roots:
        visit(r)
    return order


def compile_elementwise(out_trees: Sequence[Tuple[str, Any]], shape: Tuple[int, ...],
                        decl: Mapping[str, Tuple[int, ...]],
                        units: Optional[Mapping[str, Tuple[int, ...]]] = None, native: bool = False) -> EwProgram:
    """``out_trees``: (output name, expression tree at the iteration rank), in output order;
    ``shape``: the iteration shape; ``decl``: resolved shape of every input tensor;
    ``units``: per input, the declared size-1 axes the expression trees broadcast along
    (``patterns.Val.unit``).  ``native``: compile for the native form's limits instead of
    the interpreter kernel's (the program then runs only as native code)."""
    max_code, max_regs, max_inputs, max_outputs = ((NATIVE_MAX_CODE, NATIVE_MAX_REGS, NATIVE_MAX_INPUTS,
                                                    NATIVE_MAX_OUTPUTS) if native
                                                   else (MAX_CODE, MAX_REGS, MAX_INPUTS, MAX_OUTPUTS))
    if len(shape) > MAX_RANK:
        raise EwCompileError(f"rank {len(shape)} exceeds {MAX_RANK}")
    if not out_trees:
        raise EwCompileError("need at least one output")
    if len(out_trees) > max_outputs:
        raise EwLimitError(f"{len(out_trees)} outputs exceed {max_outputs}")
    b = _Builder(tuple(int(d) for d in shape), decl, units or {}, max_inputs)
    ident = tuple(range(len(shape)))
    roots = [b.node(t, ident) for _, t in out_trees]
    order = _schedule(b.dag, roots)
    uses: Dict[int, int] = {}
    for n in order:
        for c in b.dag.nodes[n][2]:
            uses[c] = uses.get(c, 0) + 1
    stores: Dict[int, List[int]] = {}
    for k, r in enumerate(roots):
        stores.setdefault(r, []).append(k)
        uses[r] = uses.get(r, 0) + 1
    reg_of: Dict[int, int] = {}
    free = list(range(max_regs - 1, -1, -1))
    code: List[Tuple[int, int, int, int, int, float]] = []
    for n in order:
        kind, payload, kids = b.dag.nodes[n]
        src = [reg_of[c] for c in kids]
        for c in kids:  # operands that die here give their register to the result
            uses[c] -= 1
            if uses[c] == 0:
                free.append(reg_of[c])
        if not free:
            raise EwLimitError(f"chain needs more than {max_regs} live values")
        d = free.pop()
        reg_of[n] = d
        a, bb, c = (src + [0, 0, 0])[:3]
        if kind == "load":
            code.append((OP["load"], d, int(payload), 0, 0, 0.0))
        elif kind == "imm":
            code.append((OP["imm"], d, 0, 0, 0, float(payload)))
        elif kind == "iota":
            code.append((OP["iota"], d, int(payload), 0, 0, 0.0))
        else:
            code.append((OP[kind], d, a, bb, c, 0.0))
        for k in stores.get(n, []):
            code.append((OP["store"], 0, d, k, 0, 0.0))
            uses[n] -= 1
            if uses[n] == 0:
                free.append(d)
    if len(code) > max_code:
        raise EwLimitError(f"program of {len(code)} instructions exceeds {max_code}")
    return EwProgram(tuple(code), tuple(b.inputs), tuple(n for n, _ in out_trees), tuple(int(d) for d in shape))


__all__ = ["EwProgram", "EwCompileError", "EwLimitError", "compile_elementwise", "OP", "DTYPE_CODE",
           "MAX_CODE", "MAX_REGS", "MAX_INPUTS", "MAX_OUTPUTS", "MAX_RANK", "NATIVE_MAX_CODE", "NATIVE_MAX_REGS",
           "NATIVE_MAX_INPUTS", "NATIVE_MAX_OUTPUTS", "fits_interpreter"]
