"""Generic element-wise programs on the CPU: compiler, program semantics and C-ABI checks.

The programs that ``lower_intent_to_hip_kernel`` builds for element-wise chains
are run here through a host model of ``ihip_elementwise_program`` (the kernel's
load/store conversions and f32 registers, written with numpy) and judged
against the oracle with the same rule and tolerances as the GPU parity tests.
This pins the compiler (index maps, register allocation, CSE, casts) without
a device; the GPU tests then pin the kernel against the same oracle.
"""

from __future__ import annotations

import ctypes
import zlib

import numpy as np
import pytest

from intent_ir_amd import HipLoweringError, lower_intent_to_hip_kernel
from intent_ir_amd.dtypes import bf16_bits_to_f32, round_to_bf16, to_compute_f32, to_storage
from intent_ir_amd.ewprogram import MAX_REGS, OP, EwCompileError, compile_elementwise
from intent_ir_amd.ir import as_intent
from intent_ir_amd.runtime import EW_MODE_INTERP, load_library
from oracle.compare import compare_outputs
from oracle.interpreter import execute_intent
from tests.ew_cases import CASES, TOL

_NAMES = {v: k for k, v in OP.items()}


def run_model(prog, storage: dict, dtypes: dict) -> dict:
    """numpy model of ew_program_kernel: loads widen to f32, registers are f32, stores convert."""
    shape4 = (1,) * (4 - len(prog.shape)) + tuple(prog.shape)
    idx = np.indices(shape4, dtype=np.int64)
    f32 = np.float32
    regs, out = {}, {}

    def load(k):
        name, st = prog.inputs[k]
        a = np.asarray(storage[name])
        if dtypes[name] == "bf16":
            a = bf16_bits_to_f32(a)
        flat = a.reshape(-1).astype(f32)
        if flat.size == 0:
            return np.zeros(shape4, f32)
        return flat[sum(idx[i] * st[i] for i in range(4))]

    def store(name, v):
        dt = dtypes[name]
        v = v.reshape(prog.shape)
        if dt == "f16":
            return v.astype(np.float16).astype(f32)
        if dt == "bf16":
            return round_to_bf16(v)
        if dt in ("bool", "i1"):
            return v != 0
        if dt == "i32":
            return np.trunc(v).astype(np.int32)
        return v

    with np.errstate(all="ignore"):
        for op, d, a, b, c, imm in prog.code:
            n = _NAMES[op]
            x, y = regs.get(a), regs.get(b)
            if n == "load":
                regs[d] = load(a)
            elif n == "imm":
                regs[d] = np.full(shape4, imm, f32)
            elif n == "iota":
                regs[d] = idx[a].astype(f32)
            elif n == "store":
                out[prog.outputs[b]] = store(prog.outputs[b], regs[a])
            else:
                r = {"mov": lambda: x, "add": lambda: x + y, "sub": lambda: x - y, "mul": lambda: x * y,
                     "div": lambda: x / y, "max": lambda: np.maximum(x, y), "min": lambda: np.minimum(x, y),
                     "ne": lambda: x != y, "lt": lambda: x < y, "le": lambda: x <= y, "gt": lambda: x > y,
                     "ge": lambda: x >= y, "eq": lambda: x == y, "and": lambda: (x != 0) & (y != 0),
                     "or": lambda: (x != 0) | (y != 0), "not": lambda: x == 0,
                     "relu": lambda: np.maximum(x, f32(0)), "exp": lambda: np.exp(x),
                     "rsqrt": lambda: f32(1) / np.sqrt(x), "abs": lambda: np.abs(x), "floor": lambda: np.floor(x),
                     "neg": lambda: -x, "where": lambda: np.where(x != 0, y, regs[c]),
                     "cast_f16": lambda: x.astype(np.float16), "cast_bf16": lambda: round_to_bf16(x),
                     "cast_bool": lambda: x != 0, "cast_i32": lambda: np.trunc(x)}[n]()
                regs[d] = np.asarray(r).astype(f32)
    return out


def oracle_outputs(ir, storage, bindings):
    fn = as_intent(ir)
    return execute_intent(ir, {n: to_compute_f32(v, fn.tensors[n].dtype) for n, v in storage.items()}, bindings)


def tol_for(dtype):
    atol, rtol = TOL.get(dtype, (0.0, 0.0))
    return {"atol": atol, "rtol": rtol}


def check_output(got, ref, name, dtype, what=""):
    """The reference rule (verify/diff_runner.py:357-418), except where the reference output
    holds NaN: that rule compares non-finite values with np.array_equal (:390-391), which is
    never true for NaN, so there NaN must meet NaN and the finite rest the tolerance."""
    r = np.asarray(ref[name])
    if r.dtype.kind == "f" and np.isnan(r).any():
        p = np.asarray(got[name]).reshape(r.shape).astype(np.float64)
        atol, rtol = TOL.get(dtype, (0.0, 0.0))
        np.testing.assert_allclose(p, r.astype(np.float64), rtol=rtol, atol=atol, equal_nan=True, err_msg=what)
        return
    d = compare_outputs(got, ref, [name], tol_for(dtype))
    assert d.ok, f"{what}: {d.summary} (max_abs={d.max_abs_err:.3g})"


@pytest.mark.parametrize("name,ir,bindings,gen", CASES, ids=[c[0] for c in CASES])
def test_program_model_matches_oracle(name, ir, bindings, gen):
    k = lower_intent_to_hip_kernel(ir, shape_bindings=bindings)
    assert k.kernel_id == "ihip_elementwise_program"
    prog = k.call_args[0][1]
    fn = as_intent(ir)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    storage = {n: to_storage(v, fn.tensors[n].dtype) for n, v in gen(rng, bindings).items()}
    dtypes = {n: t["dtype"] for n, t in k.io_spec["tensors"].items()}
    got = run_model(prog, storage, dtypes)
    ref = oracle_outputs(ir, storage, bindings)
    for o in k.output_names:
        check_output(got, ref, o, dtypes[o], f"{name}/{o}\n" + "\n".join(prog.listing()))


def test_listing_and_cse():
    name, ir, b, _ = next(c for c in CASES if c[0] == "two_outputs_shared")
    prog = lower_intent_to_hip_kernel(ir, shape_bindings=b).call_args[0][1]
    ops = [_NAMES[c[0]] for c in prog.code]
    assert ops.count("load") == 2 and ops.count("add") == 1 and ops.count("store") == 2  # x loaded once, x+b shared
    assert prog.listing()[-1].startswith("y2 = ")


def test_register_pressure_limit():
    names = {n: (16,) for n in "abcd"}
    # a left-deep chain keeps one value live whatever its length
    deep = ("in", "a")
    for i in range(20):
        deep = ("add", deep, ("const", float(i)))
    assert len(compile_elementwise([("y", deep)], (16,), names).code) == 42
    # repeated subtrees are computed once
    wide = ("add", ("add", ("in", "a"), ("in", "b")), ("add", ("in", "c"), ("in", "d")))
    for _ in range(3):
        wide = ("add", wide, ("mul", wide, ("const", 2.0)))
    assert sum(1 for c in compile_elementwise([("y", wide)], (16,), names).code if c[0] == OP["load"]) == 4

    # a complete tree of distinct subtrees needs one more register per level
    def full(depth, tag):
        if depth == 0:
            return ("mul", ("in", "a"), ("const", float(tag)))
        return ("sub", full(depth - 1, 2 * tag), full(depth - 1, 2 * tag + 1))

    compile_elementwise([("y", full(4, 1))], (16,), names)  # needs 6 registers, 49 instructions
    with pytest.raises(EwCompileError, match="live values"):
        compile_elementwise([("y", full(MAX_REGS, 1))], (16,), names)


def test_lowering_errors():
    base = {"name": "e", "tensors": {"x": {"dtype": "i64", "shape": ["N"]}, "y": {"dtype": "i64", "shape": ["N"]}},
            "ops": [{"op": "add", "inputs": ["x", "x"], "output": "y"}], "outputs": ["y"]}
    with pytest.raises(HipLoweringError, match="does not take i64"):
        lower_intent_to_hip_kernel(base, shape_bindings={"N": 4})
    r5 = {"name": "r5", "tensors": {"x": {"dtype": "f32", "shape": ["A", "B", "C", "D", "E"]},
                                    "y": {"dtype": "f32", "shape": ["A", "B", "C", "D", "E"]}},
          "ops": [{"op": "exp", "inputs": ["x"], "output": "y"}], "outputs": ["y"]}
    with pytest.raises(HipLoweringError, match="rank 5"):
        lower_intent_to_hip_kernel(r5, shape_bindings=dict(A=1, B=2, C=3, D=4, E=5))
    c8 = {"name": "c8", "tensors": {"x": {"dtype": "f32", "shape": ["N"]}, "y": {"dtype": "f32", "shape": ["N"]},
                                    "z": {"dtype": "f32", "shape": ["N"]}},
          "ops": [{"op": "cast", "inputs": ["x"], "output": "y", "attrs": {"to": "i8"}},
                  {"op": "add", "inputs": ["y", "x"], "output": "z"}], "outputs": ["z"]}
    with pytest.raises(HipLoweringError, match="cast to i8"):
        lower_intent_to_hip_kernel(c8, shape_bindings={"N": 4})
    mixed = {"name": "m", "tensors": {"x": {"dtype": "f32", "shape": ["M", "N"]}, "y": {"dtype": "f32", "shape": ["M", "N"]},
                                      "s": {"dtype": "f32", "shape": ["M"]}},
             "ops": [{"op": "exp", "inputs": ["x"], "output": "y"},
                     {"op": "reduce_sum", "inputs": ["x"], "output": "s", "attrs": {"dims": [1]}}],
             "outputs": ["y", "s"]}
    with pytest.raises(HipLoweringError):
        lower_intent_to_hip_kernel(mixed, shape_bindings={"M": 2, "N": 4})


# ---------------------------------------------------------------- C-ABI checks (no device needed)
def _prog_call(lib, code, n_in=1, n_out=1, in_dt=0, out_dt=0, rank=2, shape=(4, 8)):
    from intent_ir_amd.runtime import EwInstr, EwOperand

    c = (EwInstr * max(1, len(code)))()
    for i, (op, d, a, b, cc) in enumerate(code):
        c[i].op, c[i].dst, c[i].a, c[i].b, c[i].c = op, d, a, b, cc
    ins = (EwOperand * max(1, n_in))()
    for i in range(n_in):
        ins[i].ptr, ins[i].dtype = 0x1000, in_dt
    outs = (EwOperand * max(1, n_out))()
    for i in range(n_out):
        outs[i].ptr, outs[i].dtype = 0x2000, out_dt
    sh = (ctypes.c_int64 * 5)(*(list(shape) + [1] * (5 - len(shape))))
    st = lib.ihip_elementwise_program(c, len(code), ins, n_in, outs, n_out, sh, rank, None)
    return st, lib.ihip_last_error().decode()


@pytest.mark.parametrize("code,kw,msg", [
    ([(99, 0, 0, 0, 0)], {}, "unknown opcode"),
    ([(OP["load"], 0, 0, 0, 0), (OP["add"], 1, 0, 3, 0), (OP["store"], 0, 1, 0, 0)], {}, "unwritten register 3"),
    ([(OP["load"], 0, 1, 0, 0), (OP["store"], 0, 0, 0, 0)], {}, "loads input 1"),
    ([(OP["load"], 0, 0, 0, 0), (OP["store"], 0, 0, 0, 0), (OP["store"], 0, 0, 0, 0)], {}, "stored 2 times"),
    ([(OP["load"], 0, 0, 0, 0)], {}, "stored 0 times"),
    ([(OP["load"], 255, 0, 0, 0), (OP["store"], 0, 255, 0, 0)], {}, "writes register 255"),
    ([(OP["iota"], 0, 4, 0, 0), (OP["store"], 0, 0, 0, 0)], {}, "iota axis 4"),
    ([(OP["load"], 0, 0, 0, 0), (OP["store"], 0, 0, 0, 0)], {"in_dt": 7}, "unknown dtype 7"),
    ([(OP["load"], 0, 0, 0, 0), (OP["store"], 0, 0, 0, 0)], {"rank": 5, "shape": (1, 2, 3, 4, 5)}, "rank 5"),
    ([(OP["load"], 0, 0, 0, 0), (OP["store"], 0, 0, 0, 0)], {"shape": (-1, 8)}, "invalid shape"),
    ([], {}, "need 1..1024 instructions"),
])
def test_c_abi_rejects_bad_programs(code, kw, msg):
    from intent_ir_amd.runtime import load_library

    st, err = _prog_call(load_library(), code, **kw)
    assert st == -1 and msg in err, err


def test_programs_beyond_the_interpreter_limits_need_native_code():
    """Register 9 (or more than 64 instructions, 8 inputs, 4 outputs) is past the interpreter
    kernel's register file: in INTERP mode the call is refused before any launch, with the
    reason; in AUTO / NATIVE mode such a program runs as native code (GPU tests)."""
    lib = load_library()
    prev = lib.ihip_elementwise_mode(EW_MODE_INTERP)
    try:
        st, msg = _prog_call(lib, [(OP["load"], 9, 0, 0, 0), (OP["store"], 0, 9, 0, 0)])
        assert st == -1 and "exceed the interpreter kernel's limits" in msg
        code = [(OP["load"], 0, 0, 0, 0)] + [(OP["add"], 0, 0, 0, 0)] * 70 + [(OP["store"], 0, 0, 0, 0)]
        st, msg = _prog_call(lib, code)
        assert st == -1 and "72 instructions" in msg
    finally:
        lib.ihip_elementwise_mode(prev)



@pytest.mark.parametrize("name,ir,bindings,gen", CASES, ids=[c[0] for c in CASES])
def test_native_code_compiles(name, ir, bindings, gen):
    """ihip_elementwise_prepare turns every program into gfx950 code with hiprtc (no device needed)."""
    from intent_ir_amd.ewprogram import DTYPE_CODE
    from intent_ir_amd.runtime import EwInstr, load_library

    lib = load_library()
    k = lower_intent_to_hip_kernel(ir, shape_bindings=bindings)
    prog = k.call_args[0][1]
    dt = {n: t["dtype"] for n, t in k.io_spec["tensors"].items()}
    code = (EwInstr * len(prog.code))()
    for i, (o, d, a, b, c, imm) in enumerate(prog.code):
        code[i].op, code[i].dst, code[i].a, code[i].b, code[i].c, code[i].imm = o, d, a, b, c, imm
    ind = (ctypes.c_int32 * 8)(*[DTYPE_CODE[dt[n]] for n, _ in prog.inputs])
    outd = (ctypes.c_int32 * 4)(*[DTYPE_CODE[dt[n]] for n in prog.outputs])
    st = lib.ihip_elementwise_prepare(code, len(prog.code), ind, len(prog.inputs), outd, len(prog.outputs))
    assert st == 0, lib.ihip_last_error().decode()


@pytest.mark.parametrize("misalign", [0, 4], ids=["aligned", "misaligned"])
@pytest.mark.parametrize("name,ir,bindings,gen", CASES, ids=[c[0] for c in CASES])
def test_native_code_compiles_for_launch_operands(name, ir, bindings, gen, misalign):
    """ihip_elementwise_prepare_operands compiles the form a launch with these operands runs: the
    access form of each operand follows its strides and alignment (4 bytes off 16 selects narrower
    or element-wise accesses), transposed operands select the LDS-tiled form.  No device needed:
    the pointers are only inspected for alignment."""
    from intent_ir_amd.runtime import ew_program_args, load_library

    lib = load_library()
    k = lower_intent_to_hip_kernel(ir, shape_bindings=bindings)
    prog = k.call_args[0][1]
    dt = {n: t["dtype"] for n, t in k.io_spec["tensors"].items()}
    names = [n for n, _ in prog.inputs] + list(prog.outputs)
    ptrs = {n: 0x100000 * (i + 1) + misalign for i, n in enumerate(names)}
    args = ew_program_args(prog, ptrs, dt)
    st = lib.ihip_elementwise_prepare_operands(*args[:8])
    assert st == 0, lib.ihip_last_error().decode()


def test_prepare_rejects_bad_programs():
    from intent_ir_amd.runtime import EwInstr, load_library

    lib = load_library()
    code = (EwInstr * 1)()
    code[0].op = OP["store"]
    outd = (ctypes.c_int32 * 1)(0)
    assert lib.ihip_elementwise_prepare(code, 1, None, 0, outd, 1) == -1
    assert b"unwritten register" in lib.ihip_last_error()
    assert lib.ihip_elementwise_mode(-1) == 0  # AUTO by default
    assert lib.ihip_elementwise_mode(7) == -1


def test_c_abi_accepts_empty_iteration_space_without_a_device():
    """A valid program over zero elements returns before any HIP call."""
    from intent_ir_amd.runtime import load_library

    st, err = _prog_call(load_library(), [(OP["load"], 0, 0, 0, 0), (OP["exp"], 1, 0, 0, 0),
                                          (OP["store"], 0, 1, 0, 0)], shape=(0, 8))
    assert st == 0, err


@pytest.mark.parametrize("name,bindings,launch", [
    ("transpose_add", {"M": 8192, "N": 8192}, ((128, 128, 1), 16640)),          # LDS-tiled: 64 x 64 tiles
    ("transpose_batched_3d", {"A": 4, "M": 256, "N": 520}, ((4, 36, 1), 16640)),
    ("half_inputs_bf16_out", {"M": 8192, "N": 8192}, ((4, 2048, 1), 0)),       # 16-bit operands: 8 per lane
    ("add_bias_relu", {"M": 8192, "N": 8192}, ((8, 2048, 1), 0)),              # f32: 4 per lane, 4 rows a trip
])
def test_launch_descriptor_follows_the_native_plan(name, bindings, launch):
    """The lowering's launch plan is the one ihip_elementwise_program uses for dense aligned operands."""
    ir = next(c[1] for c in CASES if c[0] == name)
    k = lower_intent_to_hip_kernel(ir, shape_bindings=bindings)
    assert (k.launch.grid, k.launch.lds_bytes) == launch
