"""IntentIR document model: the input format of the HIP backend.

The backend consumes the IntentIR v1.1 JSON schema unchanged, so it can take the
dict a reference caller would pass to ``IntentFunction.from_json_dict`` or a
reference ``IntentFunction`` object itself (duck-typed through its
``to_json_dict()``).  Field names, dtype names and the op-attribute rules follow
``intent_ir/ir/ir_types.py`` of the reference:

* dtype set ........................ ir_types.py:52-64
* Dim / TensorLayout / TensorType / Op / ScheduleSketch / IntentFunction
                                     ir_types.py:171-307
* JSON dims: int -> const, str -> sym  ir_types.py:312-317
* layout strings ("scalar"/"dense" -> row_major)  ir_types.py:320-334
* outputs default to the last op's output  ir_types.py:233-235
* op-attribute validation ......... ir_types.py:536-764

Only the validation that decides how the backend reads an op is restated here
(arity, reduce dims, softmax axis, const value, cast target, broadcast attrs);
LLM-repair diagnostics of the reference are out of scope for an execution
backend.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Mapping, Optional, Union

from .opset import SUPPORTED_OPS

DTYPES = frozenset({"f16", "bf16", "f32", "f64", "i8", "i16", "u8", "i1", "i32", "i64", "bool"})
LAYOUT_KINDS = frozenset({"row_major", "col_major", "blocked", "custom"})


class IntentIRValidationError(Exception):
    """The IntentIR document is malformed (same role as the reference's error type)."""


@dataclass(frozen=True)
class Dim:
    kind: str  # "sym" | "const"
    value: Union[str, int]


@dataclass(frozen=True)
class TensorLayout:
    kind: str = "row_major"
    params: Dict[str, Any] = field(default_factory=dict)


@dataclass(frozen=True)
class TensorType:
    dtype: str
    shape: List[Dim]
    layout: TensorLayout = TensorLayout()

    @property
    def rank(self) -> int:
        return len(self.shape)

    def dims(self) -> List[Union[str, int]]:
        return [d.value for d in self.shape]


@dataclass
class Op:
    op: str
    inputs: List[str]
    output: str
    attrs: Dict[str, Any] = field(default_factory=dict)


@dataclass
class ScheduleSketch:
    tile_m: Union[str, int, None] = None
    tile_n: Union[str, int, None] = None
    tile_k: Union[str, int, None] = None
    vec_width: Union[str, int, None] = None
    pipeline_depth: Union[str, int, None] = None
    axis_bindings: Dict[str, str] = field(default_factory=dict)
    vec_axis: Optional[str] = None
    parallel_axes: List[str] = field(default_factory=list)
    memory_hint: Dict[str, Any] = field(default_factory=dict)

    _FIELDS = ("tile_m", "tile_n", "tile_k", "vec_width", "pipeline_depth")

    @classmethod
    def from_json(cls, d: Mapping[str, Any]) -> "ScheduleSketch":
        if not isinstance(d, Mapping):
            raise IntentIRValidationError("schedule must be an object")
        s = cls(**{k: d.get(k) for k in cls._FIELDS})
        s.axis_bindings = dict(d.get("axis_bindings") or {})
        s.vec_axis = d.get("vec_axis") if isinstance(d.get("vec_axis"), str) else None
        s.parallel_axes = [str(x) for x in (d.get("parallel_axes") or [])]
        s.memory_hint = dict(d.get("memory_hint") or {})
        for k in cls._FIELDS:
            v = getattr(s, k)
            if v is not None and not isinstance(v, (int, str)):
                raise IntentIRValidationError(f"schedule.{k} must be int/str/None")
        return s

    def to_json(self) -> Dict[str, Any]:
        out = {k: getattr(self, k) for k in self._FIELDS}
        out.update(axis_bindings=dict(self.axis_bindings), vec_axis=self.vec_axis,
                   parallel_axes=list(self.parallel_axes), memory_hint=dict(self.memory_hint))
        return out


def _dim(x: Any) -> Dim:
    if isinstance(x, bool):
        raise IntentIRValidationError(f"invalid dimension: {x!r}")
    if isinstance(x, int):
        return Dim("const", int(x))
    if isinstance(x, str):
        return Dim("sym", x)
    raise IntentIRValidationError(f"invalid dimension type: {type(x).__name__}")


def _layout(x: Any) -> TensorLayout:
    if isinstance(x, str):
        if x in ("scalar", "dense"):
            return TensorLayout("row_major")
        if x not in ("row_major", "col_major"):
            raise IntentIRValidationError(f"unsupported layout: {x}")
        return TensorLayout(x)
    if isinstance(x, Mapping):
        kind = x.get("kind")
        params = x.get("params", {}) or {}
        if kind not in LAYOUT_KINDS or not isinstance(params, Mapping):
            raise IntentIRValidationError(f"unsupported layout: {x!r}")
        return TensorLayout(kind, dict(params))
    raise IntentIRValidationError("layout must be string or object")


def _tensor(name: str, d: Any) -> TensorType:
    if not isinstance(d, Mapping):
        raise IntentIRValidationError(f"tensor {name} must be an object")
    dt = d.get("dtype")
    if dt not in DTYPES:
        raise IntentIRValidationError(f"tensors.{name}.dtype unsupported: {dt}")
    shape = d.get("shape")
    if not isinstance(shape, list):
        raise IntentIRValidationError(f"tensors.{name}.shape must be a list")
    return TensorType(dt, [_dim(s) for s in shape], _layout(d.get("layout", "row_major")))


def _op(d: Any) -> Op:
    if not isinstance(d, Mapping):
        raise IntentIRValidationError("each op must be an object")
    name, inputs, output, attrs = d.get("op"), d.get("inputs") or [], d.get("output"), d.get("attrs") or {}
    if not isinstance(name, str):
        raise IntentIRValidationError("op.op must be a string")
    if not isinstance(inputs, list) or not all(isinstance(i, str) for i in inputs):
        raise IntentIRValidationError(f"op.inputs must be a list of names for op {name}")
    if not isinstance(output, str):
        raise IntentIRValidationError(f"op.output must be a string for op {name}")
    if not isinstance(attrs, Mapping):
        raise IntentIRValidationError(f"op.attrs must be an object for op {name}")
    return Op(name, list(inputs), output, dict(attrs))


# Ops whose arity is fixed (reference ir_types.py:620-700).
_UNARY = {"exp", "relu", "rsqrt", "abs", "floor", "not", "identity", "cast", "reduce_sum", "reduce_max",
          "reduce_any", "softmax", "broadcast_in_dim", "transpose", "reshape", "layout_cast"}
_BINARY_STRICT = {"ne", "lt", "le", "gt", "ge", "and", "or", "matmul"}
# 1-input + scalar-attr shorthands accepted for arithmetic (ir_types.py:626-643).
SCALAR_ATTR_OF = {"div": "divisor", "add": "addend", "sub": "subtract", "mul": "mul_factor",
                  "max": "other", "min": "other"}


def reduce_dims_attr(attrs: Mapping[str, Any]) -> Any:
    """The reduce-axes attribute, in the lookup order of verify/interpreter.py:480,491,497."""
    return attrs.get("axes", attrs.get("dims", attrs.get("axis")))


def _check_attrs(idx: int, op: Op) -> None:
    a, n = op.attrs, len(op.inputs)
    where = f"op[{idx}] {op.op}"
    if op.op in _UNARY and n != 1:
        raise IntentIRValidationError(f"{where} requires 1 input")
    if op.op in _BINARY_STRICT and n != 2:
        raise IntentIRValidationError(f"{where} requires 2 inputs")
    if op.op in SCALAR_ATTR_OF and not (n == 2 or (n == 1 and SCALAR_ATTR_OF[op.op] in a)):
        raise IntentIRValidationError(f"{where} requires 2 inputs (or 1+scalar attr)")
    if op.op == "where" and n != 3:
        raise IntentIRValidationError(f"{where} requires 3 inputs (cond, x, y)")
    if op.op == "const":
        if n:
            raise IntentIRValidationError(f"{where} requires 0 inputs")
        if "value" not in a:
            raise IntentIRValidationError(f"{where} requires attrs.value")
        if a.get("dtype") is not None and a["dtype"] not in DTYPES:
            raise IntentIRValidationError(f"{where} attrs.dtype unsupported: {a['dtype']}")
    elif op.op == "cast":
        if a.get("to") not in DTYPES:
            raise IntentIRValidationError(f"{where} requires attrs.to in the dtype set")
    elif op.op in ("reduce_sum", "reduce_max", "reduce_any"):
        dims = a.get("dims", a.get("reduce_dims", a.get("axis")))
        if isinstance(dims, int) and not isinstance(dims, bool):
            dims = [dims]
        if not isinstance(dims, list) or not dims or not all(isinstance(x, int) for x in dims):
            raise IntentIRValidationError(f"{where}.dims must be list[int]")
    elif op.op == "softmax":
        if not isinstance(a.get("axis"), int):
            raise IntentIRValidationError(f"{where} requires an int axis")
    elif op.op == "broadcast_in_dim":
        if not isinstance(a.get("out_shape"), list) or not a["out_shape"]:
            raise IntentIRValidationError(f"{where}.out_shape must be non-empty list")
        for d in a["out_shape"]:
            _dim(d)
        bd = a.get("broadcast_dims")
        if not isinstance(bd, list) or not all(isinstance(x, int) for x in bd):
            raise IntentIRValidationError(f"{where}.broadcast_dims must be list[int]")
    elif op.op == "reshape":
        if not isinstance(a.get("shape"), list) or not a["shape"]:
            raise IntentIRValidationError(f"{where}.shape must be non-empty list")
        for d in a["shape"]:
            _dim(d)
    elif op.op == "transpose":
        p = a.get("perm")
        if not isinstance(p, list) or not p or not all(isinstance(x, int) for x in p):
            raise IntentIRValidationError(f"{where}.perm must be list of int")
    elif op.op == "identity" and a:
        raise IntentIRValidationError(f"{where} must not have attrs")


@dataclass
class IntentFunction:
    name: str
    tensors: Dict[str, TensorType]
    ops: List[Op]
    outputs: List[str]
    parallel_axes: List[str] = field(default_factory=list)
    schedule: Optional[ScheduleSketch] = None
    meta: Dict[str, Any] = field(default_factory=dict)
    axis_roles: Dict[str, str] = field(default_factory=dict)
    contract: Optional[Dict[str, Any]] = None

    @classmethod
    def from_json_dict(cls, data: Mapping[str, Any]) -> "IntentFunction":
        if not isinstance(data, Mapping):
            raise IntentIRValidationError("IntentIR document must be an object")
        tj = data.get("tensors") or {}
        if not isinstance(tj, Mapping):
            raise IntentIRValidationError("tensors must be an object")
        oj = data.get("ops") or []
        if not isinstance(oj, list):
            raise IntentIRValidationError("ops must be a list")
        ops = [_op(o) for o in oj]
        outputs = data.get("outputs")
        if outputs is None:
            outputs = [ops[-1].output] if ops else []
        if not isinstance(outputs, list):
            raise IntentIRValidationError("outputs must be a list if provided")
        sched = ScheduleSketch.from_json(data["schedule"]) if data.get("schedule") is not None else None
        par = list(data.get("parallel_axes") or [])
        if sched is not None and sched.parallel_axes:
            par = list(sched.parallel_axes)
        meta = dict(data.get("meta") or {}) if isinstance(data.get("meta"), Mapping) else {}
        contract = data.get("contract")
        if contract is None and isinstance(meta.get("contract"), Mapping):
            contract = meta.pop("contract")
        fn = cls(
            name=str(data.get("name") or data.get("kernel_type") or "intent_fn"),
            tensors={str(k): _tensor(str(k), v) for k, v in tj.items()},
            ops=ops,
            outputs=[str(o) for o in outputs],
            parallel_axes=[str(x) for x in par],
            schedule=sched,
            meta=meta,
            axis_roles=dict(data.get("axis_roles") or {}),
            contract=dict(contract) if isinstance(contract, Mapping) else None,
        )
        fn.validate()
        return fn

    def to_json_dict(self) -> Dict[str, Any]:
        def lay(l: TensorLayout) -> Any:
            return l.kind if (l.kind in ("row_major", "col_major") and not l.params) else {"kind": l.kind, "params": dict(l.params)}

        out: Dict[str, Any] = {
            "name": self.name,
            "tensors": {k: {"dtype": t.dtype, "shape": t.dims(), "layout": lay(t.layout)} for k, t in self.tensors.items()},
            "ops": [dict(op=o.op, inputs=list(o.inputs), output=o.output, **({"attrs": dict(o.attrs)} if o.attrs else {}))
                    for o in self.ops],
            "outputs": list(self.outputs),
            "parallel_axes": list(self.parallel_axes),
        }
        if self.contract is not None:
            out["contract"] = dict(self.contract)
        if self.schedule is not None:
            out["schedule"] = self.schedule.to_json()
        if self.axis_roles:
            out["axis_roles"] = dict(self.axis_roles)
        if self.meta:
            out["meta"] = dict(self.meta)
        return out

    def validate(self) -> None:
        if not self.ops:
            raise IntentIRValidationError("ops must not be empty")
        known = set(self.tensors)
        produced: set = set()
        for i, op in enumerate(self.ops):
            if op.op not in SUPPORTED_OPS:
                raise IntentIRValidationError(f"op[{i}].op unsupported: {op.op}")
            for inp in op.inputs:
                if inp not in known:
                    raise IntentIRValidationError(f"op[{i}] '{op.op}' references undefined tensor '{inp}'")
            _check_attrs(i, op)
            if op.output in produced:
                raise IntentIRValidationError(f"op[{i}].output duplicates previous op output: {op.output}")
            produced.add(op.output)
            known.add(op.output)
        if not self.outputs:
            raise IntentIRValidationError("outputs must not be empty")
        for o in self.outputs:
            if o not in self.tensors:
                raise IntentIRValidationError(f"output not found in tensors: {o}")

    def producer(self, name: str) -> Optional[Op]:
        for op in self.ops:
            if op.output == name:
                return op
        return None

    def external_inputs(self) -> List[str]:
        """Declared tensors that no op produces and some op reads, in first-use order."""
        produced = {o.output for o in self.ops}
        seen: List[str] = []
        for op in self.ops:
            for i in op.inputs:
                if i not in produced and i in self.tensors and i not in seen:
                    seen.append(i)
        return seen


IntentLike = Union[IntentFunction, Mapping[str, Any], Any]


def as_intent(obj: IntentLike) -> IntentFunction:
    """Coerce a dict, this module's IntentFunction, or a reference IntentFunction."""
    if isinstance(obj, IntentFunction):
        return obj
    if isinstance(obj, Mapping):
        return IntentFunction.from_json_dict(obj)
    to_json = getattr(obj, "to_json_dict", None)
    if callable(to_json):
        return IntentFunction.from_json_dict(to_json())
    raise TypeError(f"expected an IntentIR dict or IntentFunction, got {type(obj).__name__}")


def resolve_dim(d: Union[str, int, Dim], bindings: Mapping[str, Any]) -> int:
    v = d.value if isinstance(d, Dim) else d
    if isinstance(v, int):
        return int(v)
    s = str(v)
    if s.isdigit():
        return int(s)
    if s not in bindings:
        raise KeyError(f"unbound symbolic dim: {s}")
    return int(bindings[s])


def resolve_shape(t: TensorType, bindings: Mapping[str, Any]) -> tuple:
    return tuple(resolve_dim(d, bindings) for d in t.shape)


__all__ = [
    "DTYPES", "IntentIRValidationError", "Dim", "TensorLayout", "TensorType", "Op", "ScheduleSketch",
    "IntentFunction", "IntentLike", "as_intent", "resolve_dim", "resolve_shape", "reduce_dims_attr",
    "SCALAR_ATTR_OF",
]
