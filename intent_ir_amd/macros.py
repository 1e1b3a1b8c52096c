"""Macro expansion: semantic macro ops -> primitive IntentIR ops.

Same contract as the reference pass ``expand_macros``
(``intent_ir/macros/macro_expand.py:25-44``): an IR without macro ops is
returned unchanged; otherwise every macro op is replaced, in place, by
primitive ops, new intermediate tensors are declared, and the result is
re-validated.  The registry mirrors ``macro_lowering/registry.py:12-24``.

``gelu_tanh`` is this backend's macro (the reference has no GELU op in its
interpreter, ``verify/interpreter.py:16-78``).  It expands into ops the
reference interpreter executes, so the expanded IR runs unchanged on it:

    g = z / (1 + exp(-2*sqrt(2/pi) * (z + 0.044715*z^3)))

which equals the tanh-form 0.5*z*(1 + tanh(sqrt(2/pi)*(z + 0.044715*z^3)))
because (1 + tanh a)/2 = 1/(1 + exp(-2a)).  All constants are typed f32 so the
interpreter stays in float32 under numpy's NEP-50 promotion rules.
"""

from __future__ import annotations

import math
from dataclasses import replace
from typing import Callable, Dict, List

from .ir import IntentFunction, IntentIRValidationError, Op, TensorType, as_intent

GELU_CUBIC = 0.044715
# -2*sqrt(2/pi): the exponent scale of the logistic form of tanh-GELU.
GELU_NEG_2_SQRT_2_OVER_PI = -2.0 * math.sqrt(2.0 / math.pi)


class ExpansionBuilder:
    """Appends primitive ops and declares their tensors with fresh names."""

    def __init__(self, fn: IntentFunction):
        self.tensors: Dict[str, TensorType] = dict(fn.tensors)
        self.ops: List[Op] = []
        self._names = set(self.tensors) | {o.output for o in fn.ops}

    def fresh(self, base: str) -> str:
        name, i = base, 0
        while name in self._names:
            i += 1
            name = f"{base}_{i}"
        self._names.add(name)
        return name

    def emit(self, op: str, inputs: List[str], out: str, like: TensorType | None, attrs=None, dtype=None) -> str:
        self.ops.append(Op(op, list(inputs), out, dict(attrs or {})))
        if out not in self.tensors:
            if like is None:
                raise IntentIRValidationError(f"macro expansion cannot type {out}")
            self.tensors[out] = TensorType(dtype or like.dtype, list(like.shape), like.layout)
        return out

    def const(self, value: float, base: str, like: TensorType) -> str:
        name = self.fresh(base)
        self.ops.append(Op("const", [], name, {"value": float(value), "dtype": "f32"}))
        self.tensors[name] = TensorType("f32", [], like.layout)
        return name


def _expand_gelu_tanh(b: ExpansionBuilder, op: Op) -> None:
    if len(op.inputs) != 1:
        raise IntentIRValidationError("gelu_tanh requires 1 input")
    z = op.inputs[0]
    zt = b.tensors.get(z)
    if zt is None:
        raise IntentIRValidationError(f"gelu_tanh input {z} has no declared type")
    f32 = TensorType("f32", list(zt.shape), zt.layout)
    stem = op.output
    z2 = b.emit("mul", [z, z], b.fresh(f"{stem}_z2"), f32)
    z3 = b.emit("mul", [z2, z], b.fresh(f"{stem}_z3"), f32)
    c0 = b.const(GELU_CUBIC, f"{stem}_c_cubic", zt)
    t1 = b.emit("mul", [z3, c0], b.fresh(f"{stem}_cz3"), f32)
    u = b.emit("add", [z, t1], b.fresh(f"{stem}_u"), f32)
    c1 = b.const(GELU_NEG_2_SQRT_2_OVER_PI, f"{stem}_c_scale", zt)
    t2 = b.emit("mul", [u, c1], b.fresh(f"{stem}_t"), f32)
    e = b.emit("exp", [t2], b.fresh(f"{stem}_e"), f32)
    one = b.const(1.0, f"{stem}_c_one", zt)
    d = b.emit("add", [e, one], b.fresh(f"{stem}_d"), f32)
    b.emit("div", [z, d], op.output, f32)


MacroLowerFn = Callable[[ExpansionBuilder, Op], None]

_REGISTRY: Dict[str, MacroLowerFn] = {
    "gelu_tanh": _expand_gelu_tanh,
}


def supports_macro(op_name: str) -> bool:
    return op_name in _REGISTRY


def expand_macros(intent) -> IntentFunction:
    fn = as_intent(intent)
    if not any(supports_macro(o.op) for o in fn.ops):
        return fn
    b = ExpansionBuilder(fn)
    for op in fn.ops:
        if supports_macro(op.op):
            _REGISTRY[op.op](b, op)
        else:
            b.ops.append(op)
    out = replace(fn, tensors=b.tensors, ops=b.ops)
    out.validate()
    return out


__all__ = ["expand_macros", "supports_macro", "GELU_CUBIC", "GELU_NEG_2_SQRT_2_OVER_PI"]
