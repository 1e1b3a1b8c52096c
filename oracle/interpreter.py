"""numpy restatement of the reference IntentIR interpreter.  TEST INFRASTRUCTURE ONLY.

Restates ``verify/interpreter.py`` of the reference for every op the HIP path
can be handed (the out-of-scope semantic ops dropout/correlation/resize/warp/
rope are not restated).  Each function cites the reference lines it follows.

numpy semantics.  The reference pins numpy 1.26.4 (requirements/core.txt:1),
whose value-based casting keeps ``f32_array / np.array(4096)`` in float32; this
container and the GPU box run numpy 2.x, where NEP 50 promotes that to
float64.  ``execute_intent(..., numpy_semantics="1.26")`` (the default) emulates
the pinned behaviour for 0-d operands; ``"native"`` runs the same op sequence on
whatever numpy is installed, which is what the golden vectors written by the
reference interpreter in this container record (tests/golden/make_golden.py).
"""

from __future__ import annotations

from typing import Any, Dict, Mapping, Optional, Tuple

import numpy as np

# verify/interpreter.py:16-49
NUM_BIN_OPS = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide,
               "max": np.maximum, "min": np.minimum}
NUM_UNARY_OPS = {"relu": lambda x: np.maximum(x, 0), "exp": np.exp, "rsqrt": lambda x: 1.0 / np.sqrt(x),
                 "abs": np.abs, "floor": np.floor, "identity": lambda x: x}
CMP_BIN_OPS = {"ne": np.not_equal, "lt": np.less, "le": np.less_equal, "gt": np.greater, "ge": np.greater_equal}
BOOL_BIN_OPS = {"and": np.logical_and, "or": np.logical_or}
# Scalar-attr shorthands of 1-input arithmetic ops (verify/interpreter.py:215-226).
_SCALAR_ATTR = {"div": "divisor", "add": "addend", "sub": "subtract", "mul": "mul_factor", "max": "other",
                "min": "other"}


def np_dtype(dt: Optional[str]):
    """verify/interpreter.py:81-106 (bf16 maps to float16 there, :87-89)."""
    if dt is None:
        return None
    table = {"f16": np.float16, "bf16": np.float16, "f32": np.float32, "f64": np.float64, "i32": np.int32,
             "i64": np.int64, "i8": np.int8, "i16": np.int16, "u8": np.uint8, "bool": np.bool_, "i1": np.bool_}
    if dt not in table:
        raise ValueError(f"unsupported dtype for interpreter: {dt}")
    return table[dt]


def _weak_scalar(a: np.ndarray, b: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """numpy-1.26 value-based casting for a 0-d operand against an n-d array.

    A 0-d operand whose kind is not higher than the array's (bool < int < float)
    takes the array's dtype, as numpy 1.26 did; otherwise both are left as is."""
    order = {"b": 0, "u": 1, "i": 1, "f": 2}

    def fix(s, arr):
        if s.ndim == 0 and arr.ndim > 0 and s.dtype.kind in order and arr.dtype.kind in order:
            if order[s.dtype.kind] <= order[arr.dtype.kind] and arr.dtype.kind != "b":
                return s.astype(arr.dtype)
        return s

    a, b = np.asarray(a), np.asarray(b)
    if a.ndim == 0 and b.ndim > 0:
        a = fix(a, b)
    elif b.ndim == 0 and a.ndim > 0:
        b = fix(b, a)
    return a, b


class _Exec:
    def __init__(self, fn, bindings: Mapping[str, int], numpy_semantics: str):
        self.fn = fn
        self.bindings = dict(bindings)
        if numpy_semantics not in ("1.26", "native"):
            raise ValueError("numpy_semantics must be '1.26' or 'native'")
        self.np126 = numpy_semantics == "1.26"

    # ---- helpers ---------------------------------------------------------
    def decl_tokens(self, name):
        """Declared dims of a tensor as symbol names / ints (interpreter.py:771-792)."""
        if not name or name not in self.fn.tensors:
            return None
        return [d.value if d.kind in ("sym", "const") else None for d in self.fn.tensors[name].shape]

    def _resolved(self, tok):
        if isinstance(tok, int):
            return tok
        if isinstance(tok, str) and tok in self.bindings:
            return int(self.bindings[tok])
        return None

    def _match_axis(self, vec_name, ten_name, rank):
        """interpreter.py:803-821: exact unique symbol hit, else unique resolved-size hit."""
        v, t = self.decl_tokens(vec_name), self.decl_tokens(ten_name)
        if not v or len(v) != 1 or not t or len(t) != rank:
            return None
        v0 = v[0]
        if isinstance(v0, str):
            hits = [i for i, tt in enumerate(t) if tt == v0]
            if len(hits) == 1:
                return hits[0]
        vn = self._resolved(v0)
        if vn is None:
            return None
        hits = [i for i, tt in enumerate(t) if self._resolved(tt) == vn]
        return hits[0] if len(hits) == 1 else None

    def align(self, an, a, bn, b):
        """interpreter.py:752-841: place a 1-D operand on the axis its declared symbol names."""
        def put(vec, axis, ref):
            if vec.ndim != 1 or not (0 <= axis < ref.ndim) or vec.shape[0] != ref.shape[axis]:
                return vec
            shp = [1] * ref.ndim
            shp[axis] = vec.shape[0]
            return vec.reshape(shp)

        if a.ndim == 1 and b.ndim >= 2:
            ax = self._match_axis(an, bn, b.ndim)
            if ax is not None:
                a = put(a, ax, b)
        if b.ndim == 1 and a.ndim >= 2:
            ax = self._match_axis(bn, an, a.ndim)
            if ax is not None:
                b = put(b, ax, a)
        return a, b

    def shape_attr(self, s):
        """interpreter.py:611-622."""
        if s is None:
            return ()
        out = []
        for d in s:
            if isinstance(d, (int, np.integer)) or str(d).isdigit():
                out.append(int(d))
            elif isinstance(d, str) and d in self.bindings:
                out.append(int(self.bindings[d]))
            else:
                raise ValueError(f"unbound symbolic dim in shape: {d}")
        return tuple(out)

    def resolve_value(self, v, env):
        """interpreter.py:633-643."""
        if isinstance(v, str):
            if v in env:
                return env[v]
            if v in self.bindings:
                return np.array(self.bindings[v])
            try:
                return np.array(float(v))
            except ValueError as e:
                raise ValueError(f"unresolved scalar value: {v}") from e
        return np.array(v)

    @staticmethod
    def resolve_dims(raw, x):
        """interpreter.py:676-694 (string digits accepted; nothing usable -> all non-leading axes)."""
        if raw is None:
            return tuple(range(x.ndim))
        dims = [int(raw)] if isinstance(raw, (int, np.integer)) else list(raw)
        out = [int(d) for d in dims if isinstance(d, (int, np.integer)) or (isinstance(d, str) and d.isdigit())]
        return tuple(out) if out else tuple(range(1, x.ndim))

    def reduce_scale(self, out, scale):
        """interpreter.py:646-673."""
        if scale is None:
            return out
        if isinstance(scale, (int, float, np.number)):
            f = float(scale)
        elif isinstance(scale, str):
            loc = dict(self.bindings)
            if "num_elements" not in loc and isinstance(loc.get("group_size"), int) and isinstance(loc.get("HW"), int):
                loc["num_elements"] = loc["group_size"] * loc["HW"]
            f = float(loc[scale]) if scale in loc else float(eval(scale, {}, loc))  # noqa: S307 - bindings only
        else:
            raise ValueError(f"unsupported reduce scale type: {type(scale)}")
        return out * f

    def binary(self, fn, a, b):
        if self.np126:
            a, b = _weak_scalar(a, b)
        return fn(a, b)

    # ---- ops ---------------------------------------------------------------
    def op(self, op, env):  # noqa: C901 - one branch per op, as in the reference
        name, ins, at = op.op, list(op.inputs), dict(op.attrs or {})
        get = lambda n: env[n]  # noqa: E731
        if name in NUM_BIN_OPS:                                           # :212-232
            args = [get(n) for n in ins]
            if len(args) == 1 and _SCALAR_ATTR.get(name) in at:
                args.append(self.resolve_value(at[_SCALAR_ATTR[name]], env))
            if len(args) != 2:
                raise ValueError(f"{name} requires 2 inputs (or 1+attrs)")
            a, b = self.align(ins[0] if ins else None, np.asarray(args[0]),
                              ins[1] if len(ins) > 1 else None, np.asarray(args[1]))
            return self.binary(NUM_BIN_OPS[name], a, b)
        if name in NUM_UNARY_OPS:                                         # :233-235
            return NUM_UNARY_OPS[name](get(ins[0]))
        if name in CMP_BIN_OPS:                                           # :236-242
            a, b = self.align(ins[0], np.asarray(get(ins[0])), ins[1], np.asarray(get(ins[1])))
            return self.binary(CMP_BIN_OPS[name], a, b)
        if name in BOOL_BIN_OPS:                                          # :243-249
            a, b = self.align(ins[0], np.asarray(get(ins[0])).astype(bool), ins[1],
                              np.asarray(get(ins[1])).astype(bool))
            return BOOL_BIN_OPS[name](a, b)
        if name == "not":                                                 # :250-252
            return np.logical_not(np.asarray(get(ins[0])).astype(bool))
        if name == "broadcast_in_dim":                                    # :253-257, :594-608
            x = np.asarray(get(ins[0]))
            out_shape = self.shape_attr(at.get("out_shape"))
            bd = at.get("broadcast_dims", [])
            if not isinstance(bd, list):
                raise ValueError("broadcast_in_dim requires attrs.broadcast_dims as list[int]")
            tmp = [1] * len(out_shape)
            for i, od in enumerate(bd):
                if i < x.ndim:
                    tmp[od] = x.shape[i]
            return np.broadcast_to(np.reshape(x, tmp), out_shape)
        if name == "transpose":                                           # :258-263
            return np.transpose(get(ins[0]), axes=at["perm"])
        if name == "reshape":                                             # :264-267
            return np.reshape(get(ins[0]), self.shape_attr(at.get("shape")))
        if name == "layout_cast":                                         # :268-269
            return get(ins[0])
        if name == "cast":                                                # :270-273
            return np.asarray(get(ins[0])).astype(np_dtype(at.get("to")))
        if name == "iota":                                                # :274-283
            shp = self.shape_attr(at.get("shape"))
            axis = int(at.get("axis", 0))
            ar = np.arange(shp[axis], dtype=np_dtype(at.get("dtype", "i32")))
            view = [1] * len(shp)
            view[axis] = shp[axis]
            return np.broadcast_to(ar.reshape(view), shp)
        if name == "gather":                                              # :284-291
            data = get(ins[0])
            idx = [np.asarray(i, dtype=np.int64) for i in np.broadcast_arrays(*[get(n) for n in ins[1:]])]
            return data[tuple(idx)]
        if name == "where":                                               # :292-302
            c, x, y = np.asarray(get(ins[0])).astype(bool), np.asarray(get(ins[1])), np.asarray(get(ins[2]))
            c, x = self.align(ins[0], c, ins[1], x)
            c, y = self.align(ins[0], c, ins[2], y)
            x, y = self.align(ins[1], x, ins[2], y)
            if self.np126:
                x, y = _weak_scalar(x, y)
            return np.where(c, x, y)
        if name in ("reduce_sum", "reduce_any", "reduce_max"):            # :478-500
            x = np.asarray(get(ins[0]))
            dims = self.resolve_dims(at.get("axes", at.get("dims", at.get("axis"))), x)
            keep = bool(at.get("keepdims", False))
            if name == "reduce_max":
                return np.max(x, axis=dims, keepdims=keep)
            if name == "reduce_any" or at.get("reduction_type") == "any":
                out = np.any(x, axis=dims, keepdims=keep)
            else:
                out = np.sum(x, axis=dims, keepdims=keep)
            return self.reduce_scale(out, at.get("scale")) if name == "reduce_sum" else out
        if name == "softmax":                                             # :501-506
            x = np.asarray(get(ins[0]))
            axis = at.get("axis", -1)
            e = np.exp(x - np.max(x, axis=axis, keepdims=True))
            return e / np.sum(e, axis=axis, keepdims=True)
        if name == "matmul":                                              # :507-520
            a, b = np.asarray(get(ins[0])), np.asarray(get(ins[1]))
            if at.get("transpose_a"):
                a = np.swapaxes(a, -1, -2)
            if at.get("transpose_b"):
                b = np.swapaxes(b, -1, -2)
            acc = np.matmul(a, b)
            if at.get("epilogue"):
                acc = self.epilogue(at["epilogue"], {**env, "$x": acc})
            return acc
        if name == "const":                                               # :521-544
            val = at.get("value")
            if isinstance(val, str):
                if val.startswith("placeholder:"):
                    raise ValueError(f"placeholder const is not a valid semantic value: {val}")
                if val in env:
                    val = env[val]
                elif val in self.bindings:
                    val = self.bindings[val]
                else:
                    try:
                        val = float(val)
                    except ValueError:
                        if val == "eps":
                            val = 1e-5
                        else:
                            val = eval(val, {}, dict(self.bindings))  # noqa: S307 - bindings only
            return np.array(val, dtype=np_dtype(at.get("dtype")) if at.get("dtype") is not None else None)
        raise ValueError(f"Unsupported op: {name}")

    def epilogue(self, node, env):
        """interpreter.py:567-591 (epilogue operands are not re-aligned there: :745-749)."""
        if isinstance(node, str):
            return env[node]
        op = node.get("op")
        args = [self.epilogue(i, env) if isinstance(i, dict) else env[i] for i in node.get("inputs", [])]
        if op in NUM_BIN_OPS:
            return self.binary(NUM_BIN_OPS[op], np.asarray(args[0]), np.asarray(args[1]))
        if op in NUM_UNARY_OPS:
            return NUM_UNARY_OPS[op](args[0])
        if op in CMP_BIN_OPS:
            return CMP_BIN_OPS[op](args[0], args[1])
        if op in BOOL_BIN_OPS:
            return BOOL_BIN_OPS[op](np.asarray(args[0]).astype(bool), np.asarray(args[1]).astype(bool))
        if op == "not":
            return np.logical_not(np.asarray(args[0]).astype(bool))
        raise ValueError(f"Unsupported epilogue op: {op}")


def infer_shape_bindings(fn, inputs: Mapping[str, np.ndarray]) -> Dict[str, int]:
    """verify/interpreter.py:844-863."""
    out: Dict[str, int] = {}
    for name, t in fn.tensors.items():
        if name not in inputs:
            continue
        shp = np.shape(inputs[name])
        for i, d in enumerate(t.shape):
            if d.kind != "sym":
                continue
            v = int(shp[i])
            if d.value in out and out[d.value] != v:
                raise ValueError(f"Inconsistent binding for {d.value}: {out[d.value]} vs {v}")
            out[d.value] = v
    return out


def execute_intent(intent, inputs: Mapping[str, np.ndarray], shape_bindings: Optional[Mapping[str, int]] = None,
                   *, numpy_semantics: str = "1.26", keep_env: bool = False):
    """verify/interpreter.py:109-115: run every op in order, return the declared outputs.

    ``intent`` may be an IntentIR dict or any object ``intent_ir_amd.ir.as_intent``
    accepts; macro ops (``gelu_tanh``) are expanded first, as the reference's
    diff runner does before interpreting (verify/diff_runner.py:48)."""
    from intent_ir_amd.ir import as_intent
    from intent_ir_amd.macros import expand_macros

    fn = expand_macros(as_intent(intent))
    env: Dict[str, Any] = dict(inputs)
    ex = _Exec(fn, shape_bindings or infer_shape_bindings(fn, inputs), numpy_semantics)
    for op in fn.ops:
        env[op.output] = ex.op(op, env)
    outs = {n: env[n] for n in fn.outputs}
    return (outs, env) if keep_env else outs


__all__ = ["execute_intent", "infer_shape_bindings", "np_dtype", "NUM_BIN_OPS", "NUM_UNARY_OPS", "CMP_BIN_OPS"]
