"""IntentIR -> (gfx950 kernel entry point, argument plan, launch plan).

Python side of the HIP backend, with the interface of the reference CUDA
lowering ``lower_intent_to_cuda_kernel(intent, *, shape_bindings,
schedule_override=None)`` (backends/cuda/codegen/intentir_to_cuda.py:2047-2201):
the same arguments, bindings normalisation (:2059-2072), schedule-override
handling (:2074-2097) and an error type raised for unsupported IR (:23-24,
:2201).  Instead of CUDA source to compile, the result names a precompiled
C-ABI entry point of ``libintentir_hip.so`` (``kernel_id``) and the argument
list to call it with (``call_args``).

Schedule knobs (the reference's ``CUDA_RESPECT_SCHEDULE`` and knobs-in-bindings
convention, intentir_to_cuda.py:1012,1175-1200,2074-2097): a schedule is authoritative
when ``schedule_override`` is given or the bindings set ``HIP_RESPECT_SCHEDULE=1``, and
is otherwise a hint the backend ignores.  The precompiled kernels offer a few
variants: ``HIP_GEMM_TILE`` / schedule ``tile_m``, ``tile_n`` (128 or 256) for the GEMM
and ``HIP_ROWS_PER_WG`` / schedule ``tile_m`` (1, 2 or 4 rows per workgroup) for the
one-wave-per-row softmax.  A knob or authoritative schedule field that the selected
kernel cannot honour raises ``HipLoweringError`` instead of being ignored, and so does
an unknown ``HIP_*`` binding.

Kernel families are recognised structurally (``patterns.py``), in this order:
GEMM (+bias, +ReLU, incl. ``matmul{epilogue}``), reduce_any (incl.
``const, ne, reduce_any``), softmax (op or expanded chain), LayerNorm
(chain with any output names), bias + GELU-tanh + axpy, row reduce_sum/max,
and last any other element-wise chain (a register program, ``ewprogram.py``).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Mapping, Optional, Tuple

from .ir import IntentFunction, ScheduleSketch, as_intent, resolve_shape
from .macros import GELU_CUBIC, GELU_NEG_2_SQRT_2_OVER_PI, expand_macros
from .opset import HIP_SUPPORTED_OPS
from .ewprogram import BINARY as EW_BINARY, DTYPE_CODE as EW_DTYPE_CODE, UNARY as EW_UNARY
from .ewprogram import EwCompileError, EwLimitError, compile_elementwise
from .patterns import ExprBuilder, PatternError, close, unify


class HipLoweringError(RuntimeError):
    """The IR is outside what the HIP backend lowers (role of CudaLoweringError)."""


MI355X_CUS = 256  # compute units of one MI355X (the persistent GEMM runs one workgroup per CU)


@dataclass(frozen=True)
class HipLaunch:
    """Launch plan the C-ABI entry uses for 16-byte-aligned buffers (torch allocations are)."""
    grid: Tuple[int, int, int]
    block: Tuple[int, int, int]
    lds_bytes: int = 0


@dataclass(frozen=True)
class HipLoweredKernel:
    kernel_name: str
    kernel_id: str                      # C-ABI symbol in libintentir_hip.so
    io_spec: Dict[str, Any]             # {"arg_names", "tensors": {name: {dtype, shape}}, "scalars": {}}
    launch: HipLaunch
    output_names: List[str]
    bindings: Dict[str, Any]
    # Arguments of the C call in order: ("tensor", name) | ("i64", v) | ("i32", v) | ("f32", v)
    # | ("null", None) | ("workspace", nbytes): a device workspace the caller provides, passed as
    # pointer + byte count | ("ew_program", EwProgram): the program, operand table and shape of
    # ihip_elementwise_program.  io_spec["hip_call"] holds the same plan as JSON.
    call_args: Tuple[Tuple[str, Any], ...] = field(default_factory=tuple)


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def _normalize_bindings(shape_bindings: Mapping[str, Any]) -> Dict[str, Any]:
    """intentir_to_cuda.py:2059-2072: bools -> int, integral floats -> int, junk dropped."""
    out: Dict[str, Any] = {}
    for k, v in dict(shape_bindings).items():
        if isinstance(v, bool):
            out[str(k)] = int(v)
            continue
        if isinstance(v, int):
            out[str(k)] = int(v)
            continue
        try:
            fv = float(v)
        except (TypeError, ValueError):
            continue
        out[str(k)] = int(fv) if fv.is_integer() else fv
    return out


# Knobs carried in the bindings and the values each accepts (None: any 0/1 flag).
KNOBS: Dict[str, Optional[Tuple[int, ...]]] = {
    "HIP_RESPECT_SCHEDULE": None,
    "HIP_GEMM_TILE": (64, 128, 256),
    "HIP_ROWS_PER_WG": (1, 2, 4),
    # 1: an element-wise chain that has a specialised kernel (bias + GELU + axpy) runs as a
    # generic element-wise program instead (the role of INTENTIR_CUDA_CODEGEN's choice of
    # code generator in the reference, intentir_to_cuda.py:2099-2104)
    "HIP_ELEMENTWISE_PROGRAM": None,
}
_SCHED_FIELDS = ("tile_m", "tile_n", "tile_k", "vec_width", "pipeline_depth")

# The reference CUDA backend's own binding knobs (backends/cuda/codegen/intentir_to_cuda.py:577,
# 600-844,1012-1041,1175-1202,1357-1392; cpp_codegen/intentir_cuda_codegen.cpp:598,1764,4866)
# and the value at which each requests nothing.  CUDA_RESPECT_SCHEDULE means what
# HIP_RESPECT_SCHEDULE means; ALLOW_TF32 only permits reduced precision, which the exact f32
# GEMM never uses; every other knob tunes a CUDA launch shape or code path that has no HIP
# counterpart, so a value other than its no-request value raises HipLoweringError.
REFERENCE_KNOBS: Dict[str, Any] = {
    "CUDA_SPECIALIZE_DIMS": 0, "CUDA_AUTO_SPECIALIZE_DIMS": 0, "CUDA_MAX_SMEM_OPTIN": 0, "CUDA_DROPOUT_VEC4": 1,
    "SOFTMAX_THREADS": 0, "SOFTMAX_MAX_EPT": 16, "SOFTMAX_USE_EXP2": 0,
    "DROPOUT_THREADS": 0, "DROPOUT_EPT": 0,
    "ROPE_HEADS_PER_BLOCK": 1, "ROPE_VEC": 4, "ROPE_THREADS": 0,
    "WMMA_WARPS_M": 0, "WMMA_WARPS_N": 0, "WMMA_FRAG_M": 1, "WMMA_FRAG_N": 1, "WMMA_STAGE_K": 0,
    "WMMA_CP_A_POLICY": "", "WMMA_CP_B_POLICY": "", "WMMA_USE_CP_ASYNC": -1, "WMMA_PIPE_STAGES": 0,
    "WMMA_AS_PAD": 8, "WMMA_BS_PAD": 8, "WMMA_DISABLE_FASTPATH": 0, "WMMA_TINY_SEARCH": 1,
}
_HIP_ALTERNATIVE = {"SOFTMAX_THREADS": "; the HIP softmax runs a wave per row of up to 4096 floats "
                                       "(HIP_ROWS_PER_WG chooses rows per workgroup)",
                    "WMMA_": "; HIP_GEMM_TILE chooses the GEMM's C tile"}


def _reference_knobs(raw: Mapping[str, Any], bindings: Dict[str, Any]) -> None:
    """Honour or reject the reference's own knobs in ``raw`` (the caller's bindings), updating
    the normalised ``bindings`` in place."""
    if "CUDA_RESPECT_SCHEDULE" in raw:
        v = bindings.pop("CUDA_RESPECT_SCHEDULE", raw["CUDA_RESPECT_SCHEDULE"])
        if v not in (0, 1):
            raise HipLoweringError(f"CUDA_RESPECT_SCHEDULE={v!r} is not one of (0, 1)")
        if bindings.get("HIP_RESPECT_SCHEDULE", v) != v:
            raise HipLoweringError("CUDA_RESPECT_SCHEDULE and HIP_RESPECT_SCHEDULE disagree")
        bindings["HIP_RESPECT_SCHEDULE"] = v
    if "ALLOW_TF32" in raw:
        v = bindings.pop("ALLOW_TF32", raw["ALLOW_TF32"])
        if v not in (0, 1):
            raise HipLoweringError(f"ALLOW_TF32={v!r} is not one of (0, 1)")
    for k, idle in REFERENCE_KNOBS.items():
        if k not in raw:
            continue
        v = bindings.pop(k, raw[k])  # the normalised value where there is one ("16" -> 16)
        if v is None or v == idle or (isinstance(idle, str) and str(v).strip().lower() == idle):
            continue
        hint = _HIP_ALTERNATIVE.get(k) or next((h for p, h in _HIP_ALTERNATIVE.items() if k.startswith(p)), "")
        raise HipLoweringError(f"{k}={v!r} tunes the reference CUDA backend and has no HIP counterpart{hint}")


class _Knobs:
    """Launch-variant requests: binding knobs, and the schedule when it is authoritative.

    Matchers take what their kernel can honour (``gemm_tile``, ``rows_per_wg``);
    ``check_used`` then rejects whatever is left, so nothing is silently ignored."""

    def __init__(self, fn: IntentFunction, b: Mapping[str, Any]):
        for k in b:
            if k.startswith("HIP_") and k not in KNOBS:
                raise HipLoweringError(f"unknown HIP knob {k} (known: {sorted(KNOBS)})")
        self.values: Dict[str, int] = {}
        for k, allowed in KNOBS.items():
            if k not in b:
                continue
            v = b[k]
            if not isinstance(v, int) or (allowed is not None and v not in allowed) or (allowed is None and v not in (0, 1)):
                raise HipLoweringError(f"{k}={v!r} is not one of {allowed or (0, 1)}")
            self.values[k] = v
        self.respect = bool(self.values.get("HIP_RESPECT_SCHEDULE", 0))
        self.sched: Dict[str, int] = {}
        if self.respect and fn.schedule is not None:
            for f in _SCHED_FIELDS:
                v = getattr(fn.schedule, f)
                if v is None:
                    continue
                if isinstance(v, str):
                    if v not in b or not isinstance(b[v], int):
                        raise HipLoweringError(f"schedule.{f}={v!r} names no integer binding")
                    v = b[v]
                self.sched[f] = int(v)
        self.used: set = {"HIP_RESPECT_SCHEDULE"}

    def _fields(self, allowed: Mapping[str, Tuple[Optional[int], ...]], what: str) -> None:
        for f, v in self.sched.items():
            if f in allowed and v not in allowed[f]:
                raise HipLoweringError(f"schedule.{f}={v} is not available for {what} "
                                       f"(choices: {[a for a in allowed[f] if a is not None]})")
        self.used |= set(allowed)

    def gemm_tile(self, f32: bool = False) -> int:
        """C tile extent the GEMM must use: 0 = the kernel's own choice, else 128 or 256 (bf16)
        or 64 or 128 (f32)."""
        self.used.add("HIP_GEMM_TILE")
        knob = self.values.get("HIP_GEMM_TILE")
        tiles = (64, 128) if f32 else (128, 256)
        if knob is not None and knob not in tiles:
            raise HipLoweringError(f"HIP_GEMM_TILE={knob} is not available for the {'f32' if f32 else 'bf16'} GEMM "
                                   f"(choices: {list(tiles)})")
        allowed: Dict[str, Tuple[Optional[int], ...]] = (
            {"tile_k": (32,), "pipeline_depth": (2,), "vec_width": (4,)} if f32
            else {"tile_k": (32,), "pipeline_depth": (4,), "vec_width": (8,)})
        if knob is None:
            allowed.update(tile_m=tiles, tile_n=tiles)
        else:  # the binding knob overrides the schedule's tile (as SOFTMAX_THREADS does in the reference)
            self.used |= {"tile_m", "tile_n"}
        self._fields(allowed, "the f32 GEMM (k steps of 32, double-buffered, 16-byte copies)" if f32
                     else "the GEMM (K slices of 32, 16-byte copies)")
        if knob is not None:
            return knob
        tm, tn = self.sched.get("tile_m"), self.sched.get("tile_n")
        if tm is not None and tn is not None and tm != tn:
            raise HipLoweringError(f"GEMM tiles are square: schedule tile_m={tm}, tile_n={tn}")
        return tm or tn or 0

    def rows_per_wg(self) -> int:
        """Rows per workgroup the one-wave-per-row softmax must use: 0 = its own choice."""
        self.used.add("HIP_ROWS_PER_WG")
        knob = self.values.get("HIP_ROWS_PER_WG")
        allowed: Dict[str, Tuple[Optional[int], ...]] = {"vec_width": (4,)}
        if knob is None:
            allowed["tile_m"] = (1, 2, 4)
        else:
            self.used.add("tile_m")
        self._fields(allowed, "softmax (rows per workgroup; 16-byte vectors)")
        return knob if knob is not None else self.sched.get("tile_m", 0)

    def check_used(self, kernel_id: str) -> None:
        for k in self.values:
            if k not in self.used:
                raise HipLoweringError(f"{k} does not apply to {kernel_id}")
        left = sorted(f for f in self.sched if f not in self.used)
        if left:
            raise HipLoweringError(f"authoritative schedule fields {left} are not available for {kernel_id}: "
                                   "it has a single launch schedule")


class _Ctx:
    def __init__(self, fn: IntentFunction, bindings: Dict[str, Any]):
        self.fn = fn
        self.b = bindings
        self.knobs = _Knobs(fn, bindings)
        self.eb = ExprBuilder(fn, bindings)
        self.outs = {o: self.eb.get(o) for o in fn.outputs}

    def dtype(self, name: str) -> str:
        return self.fn.tensors[name].dtype

    def shape(self, name: str) -> Tuple[int, ...]:
        try:
            return resolve_shape(self.fn.tensors[name], self.b)
        except KeyError as e:
            raise HipLoweringError(f"missing binding for {name}: {e}") from e

    def rows(self, name: str) -> Tuple[int, int]:
        shp = self.shape(name)
        if not shp:
            raise HipLoweringError(f"{name} is a scalar; row kernels need rank >= 1")
        m = 1
        for d in shp[:-1]:
            m *= d
        return m, shp[-1]

    def io(self, names: List[str]) -> Dict[str, Any]:
        tensors = {n: {"dtype": self.dtype(n), "shape": self.fn.tensors[n].dims()} for n in names}
        return {"arg_names": list(names), "tensors": tensors, "scalars": {}}


# ---------------------------------------------------------------- matchers
def _row_launch(m: int, rows_per_block: int = 4) -> HipLaunch:
    return HipLaunch((max(1, _cdiv(m, rows_per_block)), 1, 1), (64 * rows_per_block, 1, 1), 0)


def _match_gemm(c: _Ctx) -> Optional[HipLoweredKernel]:
    if len(c.outs) != 1:
        return None
    (oname, ov), = c.outs.items()
    mm = ("matmul", ("?in", "A"), ("?in", "B"), ("?", "ta"), ("?", "tb"))
    bias = ("bcast", ("?in", "bias"), (1,), 2)
    env = None
    relu = has_bias = False
    for t, r, hb in ((mm, False, False), (("relu", mm), True, False), (("add", mm, bias), False, True),
                     (("relu", ("add", mm, bias)), True, True)):
        env = unify(ov.tree, t, {})
        if env is not None:
            relu, has_bias = r, hb
            break
    if env is None:
        return None
    ta, tb = bool(env["ta"]), bool(env["tb"])
    a, b = env["A"][1], env["B"][1]
    dts = {c.dtype(n) for n in (a, b, oname)}
    if dts not in ({"bf16"}, {"f32"}):
        raise HipLoweringError(f"HIP GEMM takes A, B and C all bf16 or all f32; got A {c.dtype(a)}, "
                               f"B {c.dtype(b)}, C {c.dtype(oname)}")
    sa, sb, so = c.shape(a), c.shape(b), c.shape(oname)
    if len(sa) != 2 or len(sb) != 2:
        raise HipLoweringError(f"HIP GEMM takes rank-2 operands: A{sa} B{sb}")
    (M, K), (K2, N) = (sa[::-1] if ta else sa), (sb[::-1] if tb else sb)  # interpreter.py:510-515
    if K != K2 or so != (M, N):
        raise HipLoweringError(f"matmul shapes do not agree: A{sa} B{sb} C{so} (transpose_a={ta}, transpose_b={tb})")
    names = [a, b] + ([env["bias"][1]] if has_bias else []) + [oname]
    if has_bias:
        bn = env["bias"][1]
        if c.dtype(bn) != "f32" or c.shape(bn) != (N,):
            raise HipLoweringError(f"GEMM bias must be f32 [{N}]")
    if dts == {"f32"}:
        return _gemm_f32(c, a, b, env["bias"][1] if has_bias else None, oname, M, N, K, ta, tb, relu, names)
    tile = c.knobs.gemm_tile()
    args = [("tensor", a), ("tensor", b), ("tensor", env["bias"][1]) if has_bias else ("null", None),
            ("tensor", oname), ("i64", M), ("i64", N), ("i64", K)]
    args += [("i32", int(ta)), ("i32", int(tb))] if (ta or tb or tile) else []
    args += [("i32", int(relu))] + ([("i32", tile)] if tile else [])
    # tiled fast path (any M and N; rows 16-byte aligned), packed copies then the tiled path
    # (rows that cannot start 16-byte aligned), or the guarded kernel, as gemm_fast_fits and
    # launch_gemm_packed decide for 16-byte aligned tensors; the tiled path split along K into
    # S segments when the grid has too few tiles (gemm_pack.hip split_plan)
    full = _gemm_fast_fits(M, N, K, ta, tb)
    pack_ws = 0 if full else gemm_pack_bytes(M, N, K, ta, tb)
    K8 = _cdiv(K, 8) * 8
    ta2 = ta and not _gemm_packs_a(M, K, ta)
    tb2 = tb or _gemm_packs_b(N, K, tb)
    km_copy = (ta and not ta2) or (not tb and tb2)  # a transposing copy: (K8 / 64)-tile grid rows
    packed = (pack_ws > 0 and _gemm_fast_fits(M, N, K8, ta2, tb2, packed=True)
              and not (km_copy and _cdiv(K8, 64) > 65535))
    S = gemm_split_plan(M, N, K8, tile=tile)[0] if (full or packed) else 1
    ws = pack_ws + _gemm_split_bytes(M, N, S) if (full or packed) else 0
    # 256x256 tiles, or 128x128 tiles when at most 128 tiles of 256x256 (half the CUs) would
    # be busy (gemm_fast_tile_extent)
    t = tile or _gemm_tile_extent(M, N)
    grid = (max(1, _cdiv(M, t) * _cdiv(N, t)) * S, 1, 1)  # a split: tiles x segments workgroups
    if full and S == 1 and t == 256 and _gemm_m16_fits(M, N, K, ta):
        # 256x256 tiles, K in 64-k slices: gemm_m16.hip (three A and two B slices of 32 KiB), a
        # persistent grid of one workgroup per CU (MI355X: 256) taking the tiles in turn
        launch = HipLaunch((min(grid[0], MI355X_CUS), 1, 1), (256, 1, 1), 163840)
    elif full or packed:
        launch = HipLaunch(grid, (256, 1, 1), _gemm_fast_lds(t, ta2 if packed else ta))
    else:  # guarded kernel: the same tile choice, a double-buffered {A, Bt} tile pair of 64-k slices
        launch = HipLaunch(grid, (256, 1, 1), 147456 if t == 256 else 73728)
    if ws > 0:
        args = [("tensor", a), ("tensor", b), ("tensor", env["bias"][1]) if has_bias else ("null", None),
                ("tensor", oname), ("i64", M), ("i64", N), ("i64", K), ("i32", int(ta)), ("i32", int(tb)),
                ("i32", int(relu)), ("i32", tile), ("workspace", ws)]
        return HipLoweredKernel(c.fn.name, "ihip_gemm_bf16_bias_relu_ws", c.io(names), launch, [oname], dict(c.b),
                                tuple(args))
    kid = ("ihip_gemm_bf16_bias_relu_ex" if tile else "ihip_gemm_bf16_bias_relu_t" if (ta or tb)
           else "ihip_gemm_bf16_bias_relu")
    return HipLoweredKernel(c.fn.name, kid, c.io(names), launch, [oname], dict(c.b), tuple(args))


def gemm_f32_tile_extent(M: int, N: int) -> int:
    """gemm_f32.hip gemm_f32_tile_extent: 128x128 tiles, 64x64 when fewer than 256 tiles of
    128x128 (the CU count) would run."""
    return 64 if _cdiv(M, 128) * _cdiv(N, 128) < 256 else 128


def _gemm_f32(c: "_Ctx", a: str, b: str, bias: Optional[str], oname: str, M: int, N: int, K: int, ta: bool,
              tb: bool, relu: bool, names: List[str]) -> HipLoweredKernel:
    """The reference's own matmul IR (f32 A, B, C: intentir_to_cuda.py:537-985, with the bias +
    ReLU epilogue of pipeline/tilelang/core.py:886-910) on the fp32 matrix cores."""
    tile = c.knobs.gemm_tile(f32=True)
    t = tile or gemm_f32_tile_extent(M, N)
    lds = {128: 71680, 64: 36864}[t]  # the [row][k] / [k][row] double buffers of gemm_f32.hip
    launch = HipLaunch((max(1, _cdiv(M, t) * _cdiv(N, t)), 1, 1), (256, 1, 1), lds)
    args = (("tensor", a), ("tensor", b), ("tensor", bias) if bias else ("null", None), ("tensor", oname),
            ("i64", M), ("i64", N), ("i64", K), ("i32", int(ta)), ("i32", int(tb)), ("i32", int(relu)),
            ("i32", tile))
    return HipLoweredKernel(c.fn.name, "ihip_gemm_f32_bias_relu", c.io(names), launch, [oname], dict(c.b), args)


def _gemm_fast_fits(M: int, N: int, K: int, ta: bool, tb: bool, packed: bool = False) -> bool:
    """gemm_fast.hip gemm_fast_fits for 16-byte aligned tensors.  packed: the operands are the
    workspace copies (A as [M, K], B as [N, K] where packed), of the same sizes."""
    lim = 1 << 32
    ragged_k_ok = K % 32 == 0 or (M * K * 2 < (1 << 31) and K * N * 2 < (1 << 31))
    return (M > 0 and N > 0 and K > 0 and (N % 8 == 0 or tb) and K % 8 == 0 and (not ta or M % 8 == 0)
            and K * 512 < lim and N * 128 < lim and M * 128 < lim and ragged_k_ok)


def _gemm_m16_fits(M: int, N: int, K: int, ta: bool) -> bool:
    """gemm_m16.hip gemm_m16_fits for 16-byte aligned tensors (C aligned too)."""
    return (not ta and M > 0 and N > 0 and K >= 64 and N % 8 == 0 and K % 64 == 0
            and K * 512 < (1 << 32) and N * 128 < (1 << 32) and _cdiv(M, 256) * _cdiv(N, 256) <= (1 << 30))


def _gemm_fast_lds(tile: int, ta: bool) -> int:
    """LDS bytes of the tiled kernel (gemm_fast.hip fast_lds_bytes): the operand rings (A as
    [M, K]: three paired-slice regions of tile x 128 bytes; A as [K, M]: four stages of
    tile x 64 bytes; B: four stages of tile x 64 bytes), at least the bf16 C tile (pitch
    2 * tile + 16) and the bias."""
    ring = (3 * tile * 128 if not ta else 4 * tile * 64) + 4 * tile * 64
    return max(ring, tile * (2 * tile + 16) + 4 * tile)


def _gemm_packs_a(M: int, K: int, ta: bool) -> bool:
    return K % 8 != 0 or (ta and M % 8 != 0)


def _gemm_packs_b(N: int, K: int, tb: bool) -> bool:
    return K % 8 != 0 or (not tb and N % 8 != 0)


def _al256(n: int) -> int:
    return _cdiv(n, 256) * 256


def _gemm_tile_extent(M: int, N: int) -> int:
    """gemm_fast.hip gemm_fast_tile_extent: 128x128 tiles when at most 128 tiles of 256x256
    (half the CUs) would be busy, unless M is 129-256 and the 128x128 grid needs more than
    one round, or for M <= 128 with more than 256 such tiles; else 256x256."""
    tiles256 = _cdiv(M, 256) * _cdiv(N, 256)
    tiles128 = _cdiv(M, 128) * _cdiv(N, 128)
    one_full_row = 128 < M <= 256 and tiles128 > 256
    return 128 if (tiles256 <= 128 and not one_full_row) or (M <= 128 and tiles256 > 256) else 256


_SPLIT_RATE = (0, 305, 533, 680, 800)  # tile-steps per microsecond at 0, 64, 128, 192, 256 workgroups


def _split_rate(G: int) -> int:
    if G >= 256:
        waves = _cdiv(G, 256)
        return _SPLIT_RATE[4] * G // (waves * 256)
    i, f = divmod(G, 64)
    return _SPLIT_RATE[i] + (_SPLIT_RATE[i + 1] - _SPLIT_RATE[i]) * f // 64


def _split_cost_ns(tiles: int, M: int, N: int, K: int, S: int) -> int:
    ns = tiles * _cdiv(K, 32) * 1000 // max(1, _split_rate(tiles * S))
    if S > 1:
        ns += 3500 + S * M * (_cdiv(N, 4) * 4) * 8 // 6000
    return ns


def _split_plan_of(K: int, S: int) -> Tuple[int, int]:
    S = max(1, min(S, _cdiv(K, 64), 1024))
    kseg = _cdiv(_cdiv(K, S), 64) * 64
    return _cdiv(K, kseg), kseg


def gemm_split_plan(M: int, N: int, K: int, splits: int = 0, tile: int = 0) -> Tuple[int, int]:
    """(S, kseg) of gemm_pack.hip split_plan.  splits > 0: that many segments (at most one per
    64 k and at most 1024), each but the last of kseg k, a multiple of 64.  splits = 0: grids
    of 256x256 tiles (``tile``, or the automatic choice when it is 0) stay unsplit; for
    128x128 tiles, the S (segments of at least 512 k, at most 512 workgroups) of least
    estimated time: tile-steps over the measured rate at tiles x S workgroups, plus the reduce
    launch and the partials' round trip; ties go to the smaller S."""
    if K <= 0:
        return 1, K
    if splits > 0:
        return _split_plan_of(K, splits)
    if (tile or _gemm_tile_extent(M, N)) != 128:
        return 1, K
    tiles = _cdiv(M, 128) * _cdiv(N, 128)
    smax = max(1, min(K // 512, 1024, 512 // tiles))
    best, best_ns = (1, K), _split_cost_ns(tiles, M, N, K, 1)
    for s in range(2, smax + 1):
        p = _split_plan_of(K, s)
        ns = _split_cost_ns(tiles, M, N, K, p[0])
        if ns < best_ns:
            best, best_ns = p, ns
    return best


def _gemm_split_bytes(M: int, N: int, S: int) -> int:
    """f32 partials of a split: S planes of M rows of N rounded up to 4 floats."""
    return _al256(S * M * _cdiv(N, 4) * 4 * 4) if S > 1 else 0


def gemm_pack_bytes(M: int, N: int, K: int, ta: bool, tb: bool) -> int:
    """Workspace bytes of the packed copies: a K-contiguous copy, K rounded up to 8 and
    256-byte aligned, of each operand whose rows cannot start 16-byte aligned."""
    if M <= 0 or N <= 0 or K <= 0:
        return 0
    k8 = _cdiv(K, 8) * 8
    return ((_al256(M * k8 * 2) if _gemm_packs_a(M, K, ta) else 0)
            + (_al256(N * k8 * 2) if _gemm_packs_b(N, K, tb) else 0))


def gemm_workspace_bytes(M: int, N: int, K: int, ta: bool, tb: bool) -> int:
    """Workspace bytes of ihip_gemm_bf16_bias_relu_ws (gemm_pack.hip gemm_workspace_bytes): the
    packed copies, then the split-K partials of the split rule on K rounded up to 8; 0 when
    neither is needed."""
    if M <= 0 or N <= 0 or K <= 0:
        return 0
    return gemm_pack_bytes(M, N, K, ta, tb) + _gemm_split_bytes(M, N, gemm_split_plan(M, N, _cdiv(K, 8) * 8)[0])


def _match_reduce_any(c: _Ctx) -> Optional[HipLoweredKernel]:
    if len(c.outs) != 1:
        return None
    (oname, ov), = c.outs.items()
    if not (isinstance(ov.tree, tuple) and ov.tree[0] == "rany"):
        return None
    env = unify(ov.tree, ("rany", ("?in", "x"), ("?", "ax")), {})
    cmp = 0.0
    if env is None:
        env = unify(ov.tree, ("rany", ("ne", ("?in", "x"), ("?c", "c")), ("?", "ax")), {})
        if env is None:
            raise HipLoweringError("reduce_any over a computed operand is not lowered")
        cmp = env["c"][1]
    x = env["x"][1]
    rank = c.fn.tensors[x].rank
    if env["ax"] != (rank - 1,):
        raise HipLoweringError("reduce_any is lowered over the last axis only")
    if c.dtype(oname) not in ("bool", "i1"):
        raise HipLoweringError(f"reduce_any output {oname} must be bool")
    M, N = c.rows(x)
    dt = c.dtype(x)
    if dt == "f32":
        args = (("tensor", x), ("tensor", oname), ("i64", M), ("i64", N), ("f32", float(cmp)))
        kid = "ihip_reduce_any_rows_f32"
    elif dt in ("bool", "i1", "u8") and cmp == 0.0:
        args = (("tensor", x), ("tensor", oname), ("i64", M), ("i64", N))
        kid = "ihip_reduce_any_rows_u8"
    else:
        raise HipLoweringError(f"reduce_any input dtype {dt} is not lowered")
    # rows of at most 64 16-byte vectors: g lanes per row (about two vectors each; at least 2 lanes
    # for f32, 4 for bool), 256-thread workgroups; longer rows a one-wave workgroup each
    nvec = N // 4 if kid == "ihip_reduce_any_rows_f32" else N // 16
    if nvec <= 64:
        g = 2 if kid == "ihip_reduce_any_rows_f32" else 4
        while g < 32 and 2 * g < nvec:
            g *= 2
        launch = HipLaunch((max(1, _cdiv(M * g, 256)), 1, 1), (256, 1, 1), 0)
    else:
        launch = _row_launch(M, 1)
    return HipLoweredKernel(c.fn.name, kid, c.io([x, oname]), launch, [oname], dict(c.b), args)


def _softmax_templates(rank: int):
    last = rank - 1
    lead = tuple(range(last))
    X = ("?in", "x")
    E = ("exp", ("sub", X, ("bcast", ("rmax", X, (last,)), lead, rank)))
    return [("softmax", X, last), ("div", E, ("bcast", ("rsum", E, (last,)), lead, rank))]


def _softmax_stat_templates(rank: int):
    """The row statistics a softmax IR may also return (pipeline/cuda/core.py:453-493): the
    row maximum and the sum of exp(x - max)."""
    last = rank - 1
    lead = tuple(range(last))
    X = ("?in", "x")
    E = ("exp", ("sub", X, ("bcast", ("rmax", X, (last,)), lead, rank)))
    return (("max", ("rmax", X, (last,))), ("sum", ("rsum", E, (last,))))


def _match_softmax(c: _Ctx) -> Optional[HipLoweredKernel]:
    oname = env = None
    for name, v in c.outs.items():
        if v.rank < 1:
            continue
        for t in _softmax_templates(v.rank):
            env = unify(v.tree, t, {})
            if env is not None:
                oname = name
                break
        if oname is not None:
            break
    if oname is None:
        return None
    ov = c.outs[oname]
    stats: Dict[str, str] = {}  # "max" / "sum" -> output name
    for name, v in c.outs.items():
        if name == oname:
            continue
        for role, t in _softmax_stat_templates(ov.rank):
            if role not in stats and unify(v.tree, t, dict(env)) is not None:
                stats[role] = name
                break
        else:
            return None  # an output that is neither the softmax nor one of its statistics
    x = env["x"][1]
    if c.dtype(x) != "f32" or c.dtype(oname) != "f32" or any(c.dtype(n) != "f32" for n in stats.values()):
        raise HipLoweringError("HIP softmax takes f32 input and outputs")
    M, N = c.rows(x)
    if stats:
        if N == 0:
            raise HipLoweringError("softmax statistics of rows of length 0 (no maximum)")
        segs, _ = softmax_split_plan(M, N)
        st = lambda r: ("tensor", stats[r]) if r in stats else ("null", None)  # noqa: E731
        args = (("tensor", x), ("tensor", oname), st("max"), st("sum"), ("i64", M), ("i64", N))
        args += (("workspace", 8 * M * segs),) if segs else (("null", None), ("i64", 0))
        launch = HipLaunch((M * segs, 1, 1), (256, 1, 1), 32) if segs else _softmax_launch(M, N, 0)
        names = [x, oname] + [stats[r] for r in ("max", "sum") if r in stats]
        return HipLoweredKernel(c.fn.name, "ihip_softmax_rows_f32_stats", c.io(names), launch, list(c.fn.outputs),
                                dict(c.b), args)
    rows = c.knobs.rows_per_wg()
    if rows > 1 and not (N % 4 == 0 and N <= 4096):
        raise HipLoweringError(f"{rows} rows per workgroup needs the one-wave-per-row softmax (N % 4 == 0, "
                               f"N <= 4096); N = {N} runs one row per workgroup")
    launch = _softmax_launch(M, N, rows)
    args = (("tensor", x), ("tensor", oname), ("i64", M), ("i64", N))
    if rows:
        return HipLoweredKernel(c.fn.name, "ihip_softmax_rows_f32_ex", c.io([x, oname]), launch, [oname], dict(c.b),
                                args + (("i32", rows),))
    segs, _ = softmax_split_plan(M, N)
    if segs:  # rows longer than 65536 floats: S workgroups per row, two floats of partials each
        launch = HipLaunch((M * segs, 1, 1), (256, 1, 1), 32)
        return HipLoweredKernel(c.fn.name, "ihip_softmax_rows_f32_ws", c.io([x, oname]), launch, [oname], dict(c.b),
                                args + (("workspace", 8 * M * segs),))
    return HipLoweredKernel(c.fn.name, "ihip_softmax_rows_f32", c.io([x, oname]), launch, [oname], dict(c.b), args)


# Longest vector row (16-byte vectors) the workgroup-per-row softmax holds on the CU (rows.hip
# kResMaxVecs): 24 * 1024 in registers plus (160 KiB - 128 B) / 16 in LDS.
SOFTMAX_RESIDENT_MAX_VECS = 24 * 1024 + (160 * 1024 - 128) // 16


def _softmax_launch(M: int, N: int, rows: int) -> HipLaunch:
    """The unsplit launch rows.hip plans for 16-byte aligned x and y (rows: the rows-per-workgroup
    knob, 0 = automatic)."""
    if 0 < N <= 128 and N % 4 == 0 and not rows:  # short rows: g lanes per row (one vector each)
        g = 1
        while g < N // 4:
            g *= 2
        launch = HipLaunch((max(1, _cdiv(M * g, 256)), 1, 1), (256, 1, 1), 0)
    elif 0 < N <= 128 and not rows:  # short rows, N % 4 != 0: g lanes per row, up to 4 elements
        # each, 2 rows per group; the workgroup's rows staged in LDS (8 KiB + 144 B: the run's
        # offset in its 128-byte line and one vector of slack)
        g = 1
        while 4 * g < N:
            g *= 2
        launch = HipLaunch((max(1, _cdiv(M * g, 512)), 1, 1), (256, 1, 1), 4 * (2048 + 36))
    elif N % 4 == 0 and N <= 4096:  # a wave per row, or for N <= 1024 two rows per wave with 4 rows
        # per workgroup (two waves); automatic: N == 1024 four waves of two rows (8 per workgroup),
        # N <= 256 two waves of two rows, other N <= 1024 two waves of one row, longer rows four waves
        if not rows:
            rows = 8 if N == 1024 else 4 if N <= 256 else 2 if N <= 1024 else 4
        launch = _row_launch(M, rows)
        if rows == 8:
            launch = HipLaunch((max(1, _cdiv(M, 8)), 1, 1), (256, 1, 1), 0)
        elif N <= 1024 and rows == 4:
            launch = HipLaunch(launch.grid, (128, 1, 1), 0)
    elif N % 4 == 0 and N <= 65536:  # kW waves per row, one row per workgroup, partials in LDS
        kw = next(w for w in (2, 4, 8, 16) if N // 4 <= 1024 * w)
        launch = HipLaunch((max(1, M), 1, 1), (64 * kw, 1, 1), 8 * kw)
    elif N <= 65536:  # N % 4 != 0: the row in registers, kW waves per row; above 1024 a 4-byte
        # head and tail around a 16-byte aligned body (partials in LDS even for one wave)
        kw = next(w for w in (1, 2, 4, 8, 16) if N <= 4096 * w)
        launch = HipLaunch((max(1, M), 1, 1), (64 * kw, 1, 1), 8 * kw if (kw > 1 or N > 1024) else 0)
    elif N % 4 == 0 and N <= 4 * SOFTMAX_RESIDENT_MAX_VECS:  # vocabulary-width rows held on the CU:
        # 24 vectors per lane in registers, the rest of the row and the partials in 160 KiB of LDS
        launch = HipLaunch((max(1, M), 1, 1), (1024, 1, 1), 160 * 1024)
    else:  # two passes over x, one workgroup per row
        launch = HipLaunch((max(1, M), 1, 1), (1024, 1, 1), 128)
    return launch


def softmax_split_plan(M: int, N: int) -> Tuple[int, int]:
    """(S, vpl) of the split long-row softmax (rows.hip softmax_split_plan): rows longer than
    65536 floats are cut into S segments of 256 * vpl 16-byte vectors when a workgroup per row
    would leave CUs idle (fewer than 192 rows, or a last round of at most 160 rows after one or
    two full rounds of 256); vpl = 16 unless that leaves fewer than 4096 workgroups (then 8,
    then 4); (0, 0) = not split, also when S would exceed 2**20 or the grid 2**31 - 1 workgroups."""
    if M <= 0 or N <= 65536:
        return 0, 0
    if not (M < 192 or (256 < M < 640 and 0 < M % 256 <= 160)):
        return 0, 0
    n4 = N // 4
    vpl = 16
    s = _cdiv(n4, 256 * vpl)
    while vpl > 4 and M * s < 4096:
        vpl //= 2
        s = _cdiv(n4, 256 * vpl)
    if s > 1 << 20 or M * s > 0x7FFFFFFF:
        return 0, 0
    return s, vpl


def _match_gather(fn: IntentFunction, b: Dict[str, Any]) -> Optional[HipLoweredKernel]:
    """A lone gather(inp [M, N] f32, row [L] i32, col [L] i32) -> out [L] f32: the CUDA
    backend's gather2d (intentir_to_cuda.py:1779-1832), which it dispatches for a single-op IR
    (:2155-2156).  An index pair outside [0, M) x [0, N) gives attrs.other_value (default 0),
    as there (tests/backends/cuda/test_cuda_backend_smoke.py:292-336).  Any other use of gather
    is rejected."""
    gathers = [o for o in fn.ops if o.op == "gather"]
    if not gathers:
        return None
    form = ("HIP lowering unsupported gather form: gather is lowered as a lone op: "
            "gather(inp [M, N] f32, row [L] i32, col [L] i32) -> out [L] f32")
    if len(fn.ops) != 1 or len(gathers[0].inputs) != 3 or list(fn.outputs) != [gathers[0].output]:
        raise HipLoweringError(form)
    op = gathers[0]
    inp, row, col = op.inputs
    out = op.output
    t = fn.tensors
    if (t[inp].dtype, t[row].dtype, t[col].dtype, t[out].dtype) != ("f32", "i32", "i32", "f32"):
        raise HipLoweringError(form + f"; got {t[inp].dtype}, {t[row].dtype}, {t[col].dtype} -> {t[out].dtype}")
    try:
        shp = {n: resolve_shape(t[n], b) for n in (inp, row, col, out)}
    except KeyError as e:
        raise HipLoweringError(f"missing binding for gather: {e}") from e
    if len(shp[inp]) != 2 or len(shp[row]) != 1 or shp[col] != shp[row] or shp[out] != shp[row]:
        raise HipLoweringError(form + f"; got shapes {[list(shp[n]) for n in (inp, row, col, out)]}")
    (M, N), (L,) = shp[inp], shp[row]
    try:
        other = float((op.attrs or {}).get("other_value", 0.0))
    except (TypeError, ValueError) as e:
        raise HipLoweringError(f"gather other_value must be a number: {e}") from e
    io = {"arg_names": [inp, row, col, out], "scalars": {},
          "tensors": {n: {"dtype": t[n].dtype, "shape": t[n].dims()} for n in (inp, row, col, out)}}
    launch = HipLaunch((max(1, _cdiv(L, 1024)), 1, 1), (256, 1, 1), 0)  # 4 elements per thread
    return HipLoweredKernel(fn.name, "ihip_gather2d_f32", io, launch, [out], dict(b),
                            (("tensor", inp), ("tensor", row), ("tensor", col), ("tensor", out), ("i64", M),
                             ("i64", N), ("i64", L), ("f32", other)))


def _layernorm_templates():
    """(mean, var) written as sum / N (div{divisor}) or as reduce_sum{scale: 1/N} (a sum times
    a constant, interpreter.py:646-673), in the four combinations the reference builders use
    (pipeline/tilelang/core.py:1322-1384 divides, pipeline/cuda/core.py:496-546 scales)."""
    X = ("?in", "x")
    for mean_op in ("div", "mul"):
        for var_op in ("div", "mul"):
            MEAN = (mean_op, ("rsum", X, (1,)), ("?c", "n1"))
            D = ("sub", X, ("bcast", MEAN, (0,), 2))
            VAR = (var_op, ("rsum", ("mul", D, D), (1,)), ("?c", "n2"))
            R = ("rsqrt", ("add", VAR, ("?c", "eps")))
            Y = ("add", ("mul", ("mul", D, ("bcast", R, (0,), 2)), ("bcast", ("?in", "w"), (1,), 2)),
                 ("bcast", ("?in", "b"), (1,), 2))
            yield (mean_op, var_op), (("y", Y), ("mean", MEAN), ("rstd", R))


def _match_layernorm(c: _Ctx) -> Optional[HipLoweredKernel]:
    for forms, templates in _layernorm_templates():
        roles: Dict[str, str] = {}
        env: Dict[str, Any] = {}
        for name, v in c.outs.items():
            for role, t in templates:
                e = unify(v.tree, t, env)
                if e is not None and role not in roles.values():
                    env, roles[name] = e, role
                    break
            else:
                break
        else:
            if "y" in roles.values():
                break
    else:
        return None
    inv = {r: n for n, r in roles.items()}
    x, w, b = env["x"][1], env["w"][1], env["b"][1]
    y = inv["y"]
    M, N = c.rows(x)
    if c.fn.tensors[x].rank != 2:
        return None
    for key, op in zip(("n1", "n2"), forms):
        if not (close(env[key][1], N) if op == "div" else close(env[key][1] * N, 1.0)):
            raise HipLoweringError("LayerNorm chain takes its mean or variance over something other than the row "
                                   f"length ({'divides by' if op == 'div' else 'scales by'} {env[key][1]}, N = {N})")
    dt = {c.dtype(n) for n in (x, w, b, y)}
    if dt not in ({"f16"}, {"f32"}):
        raise HipLoweringError("HIP LayerNorm takes x, w, b, y all f16 or all f32; got "
                               + ", ".join(f"{n} {c.dtype(n)}" for n in (x, w, b, y)))
    for n in (w, b):  # the kernel reads N elements of each; a [1] weight would broadcast in numpy
        if c.shape(n) != (N,):
            raise HipLoweringError(f"HIP LayerNorm takes w and b of shape [{N}]; {n} is {list(c.shape(n))}")
    for role in ("mean", "rstd"):
        if role in inv and c.dtype(inv[role]) != "f32":
            raise HipLoweringError(f"LayerNorm {role} output must be f32")
    # statistics that are not outputs are not written (null pointers): no scratch memory
    stat = lambda r: ("tensor", inv[r]) if r in inv else ("null", None)  # noqa: E731
    args = (("tensor", x), ("tensor", w), ("tensor", b), ("tensor", y), stat("mean"), stat("rstd"), ("i64", M),
            ("i64", N), ("f32", float(env["eps"][1])))
    names = [x, w, b, y] + [inv[r] for r in ("mean", "rstd") if r in inv]
    if dt == {"f32"}:
        return HipLoweredKernel(c.fn.name, "ihip_layernorm_rows_f32", c.io(names), _layernorm_f32_launch(M, N),
                                list(c.fn.outputs), dict(c.b), args)
    if N % 8 == 0 and 0 < N <= 256:  # short rows: g lanes per row (one 16-byte vector each), 2 rows per group
        g = 1
        while g < N // 8:
            g *= 2
        launch = HipLaunch((max(1, _cdiv(M * g, 512)), 1, 1), (256, 1, 1), 0)
    elif N % 8 == 0 and 0 < N <= 4096:  # 16 rows per 1024-thread workgroup; w and b staged in LDS
        kvpl = next(v for v in (1, 2, 4, 8) if N // 8 <= 64 * v)
        launch = HipLaunch((max(1, _cdiv(M, 16)), 1, 1), (1024, 1, 1), 2 * kvpl * 64 * 16)
    elif N % 8 == 0 and N <= 8192:  # 2 waves per row, 8 rows per 1024-thread workgroup, partials in LDS
        launch = HipLaunch((max(1, _cdiv(M, 8)), 1, 1), (1024, 1, 1), 128)
    elif N % 8 == 0 and N <= 65536:  # kW waves per row, one row per workgroup
        kw = 2 if N <= 16384 else 4 if N <= 32768 else 8
        launch = HipLaunch((max(1, M), 1, 1), (64 * kw, 1, 1), 8 * kw)
    elif 0 < N <= 256:  # short rows, N % 8 != 0: g lanes per row, up to 5 (N <= 5g) or 8 elements
        # each, 4 rows per group; the workgroup's rows staged in LDS and w, b as f32 (8g each)
        g = 1
        while 8 * g < N:
            g *= 2
        slots = 5 if N <= 5 * g else 8
        launch = HipLaunch((max(1, _cdiv(M * g, 1024)), 1, 1), (256, 1, 1), 2 * (1024 * slots + 72) + 2 * 4 * 8 * g)
    elif 0 < N <= 4096 + 7:  # N % 8 != 0: 8 row classes x J workgroups of 4 waves, w and b per class in LDS
        J = min(128, _cdiv(_cdiv(M, 8), 4))
        launch = HipLaunch((8 * max(1, J), 1, 1), (256, 1, 1), 2 * 512 * 16)
    elif 0 < N <= 65536 + 7:  # N % 8 != 0: head / 16-byte body / tail, kW waves per row, one row per workgroup
        kw = next(k for k in (1, 2, 4, 8, 16) if N <= 4096 * k + 7)
        launch = HipLaunch((max(1, M), 1, 1), (64 * kw, 1, 1), 8 * kw)
    else:
        launch = HipLaunch((max(1, M), 1, 1), (256, 1, 1), 16)
    return HipLoweredKernel(c.fn.name, "ihip_layernorm_rows_f16", c.io(names), launch, list(c.fn.outputs),
                            dict(c.b), args)


def _layernorm_f32_launch(M: int, N: int) -> HipLaunch:
    """The launch ihip_layernorm_rows_f32 plans for 16-byte aligned tensors
    (layernorm_f32.hip): N % 4 == 0 and N <= 4096: a wave per row, 4 rows per 256-thread
    workgroup, w and b staged in LDS; N % 4 == 0 and N <= 65536: 2-16 waves per row, one row
    per workgroup; otherwise a 256-thread workgroup per row."""
    n4 = N // 4
    if N % 4 == 0 and 0 < N <= 4096:
        kvpl = next(v for v in (1, 2, 4, 8, 16) if n4 <= 64 * v)
        return HipLaunch((max(1, _cdiv(M, 4)), 1, 1), (256, 1, 1), 2 * 16 * 64 * kvpl)
    if N % 4 == 0 and 0 < N <= 65536:
        kw = next(w for w in (2, 4, 8, 16) if n4 <= 1024 * w)
        return HipLaunch((max(1, M), 1, 1), (64 * kw, 1, 1), 8 * kw)
    return HipLaunch((max(1, M), 1, 1), (256, 1, 1), 16)


def _match_gelu_axpy(c: _Ctx) -> Optional[HipLoweredKernel]:
    c.knobs.used.add("HIP_ELEMENTWISE_PROGRAM")
    if len(c.outs) != 1 or c.knobs.values.get("HIP_ELEMENTWISE_PROGRAM"):
        return None
    (oname, ov), = c.outs.items()
    X = ("?in", "x")
    Z = ("add", X, ("bcast", ("?in", "bias"), (1,), 2))
    U = ("add", Z, ("mul", ("mul", ("mul", Z, Z), Z), ("?c", "c0")))
    G = ("div", Z, ("add", ("exp", ("mul", U, ("?c", "c1"))), ("?c", "one")))
    env = unify(ov.tree, ("add", ("mul", G, ("?c", "alpha")), X), {})
    if env is None:
        return None
    if not (close(env["c0"][1], GELU_CUBIC) and close(env["c1"][1], GELU_NEG_2_SQRT_2_OVER_PI)
            and env["one"][1] == 1.0):
        return None
    x, bias = env["x"][1], env["bias"][1]
    # other dtypes and shapes run as a generic element-wise program (_match_elementwise)
    if any(c.dtype(n) != "bf16" for n in (x, bias, oname)):
        return None
    M, N = c.rows(x)
    if c.fn.tensors[x].rank != 2 or c.shape(bias) != (N,):
        return None
    if N % 8 == 0:  # lanes per row: 256, or N / 8 rounded up to a power of two, 256 / lanes rows per workgroup
        lanes = 1
        while lanes < 256 and lanes < N // 8:
            lanes *= 2
        launch = HipLaunch((max(1, _cdiv(N // 8, lanes)), max(1, min(65535, _cdiv(M, 8 * (256 // lanes)))), 1),
                           (256, 1, 1), 0)
    else:
        launch = HipLaunch((max(1, min(65536, _cdiv(M * N, 256))), 1, 1), (256, 1, 1), 0)
    return HipLoweredKernel(c.fn.name, "ihip_bias_gelu_tanh_axpy_bf16", c.io([x, bias, oname]), launch, [oname],
                            dict(c.b), (("tensor", x), ("tensor", bias), ("tensor", oname), ("i64", M), ("i64", N),
                                        ("f32", float(env["alpha"][1]))))


def _match_row_reduce(c: _Ctx) -> Optional[HipLoweredKernel]:
    if len(c.outs) != 1:
        return None
    (oname, ov), = c.outs.items()
    tree, scale = ov.tree, None
    # reduce_sum{scale}: the sum times a constant (interpreter.py:487, :646-673)
    env = unify(tree, ("mul", ("rsum", ("?", "x"), ("?", "ax")), ("?c", "s")), {})
    if env is not None:
        tree, scale = ("rsum", env["x"], env["ax"]), float(env["s"][1])
    kind = tree[0] if isinstance(tree, tuple) else None
    if kind not in ("rsum", "rmax"):
        return None
    env = unify(tree, (kind, ("?in", "x"), ("?", "ax")), {})
    if env is None:
        return None
    x = env["x"][1]
    if env["ax"] != (c.fn.tensors[x].rank - 1,):
        raise HipLoweringError(f"{kind} is lowered over the last axis only")
    if c.dtype(x) != "f32" or c.dtype(oname) != "f32":
        raise HipLoweringError("HIP row reductions take f32 input and output")
    M, N = c.rows(x)
    args = (("tensor", x), ("tensor", oname), ("i64", M), ("i64", N), ("i32", 0 if kind == "rsum" else 1))
    segs = reduce_rows_segments(M, N)
    kid = "ihip_reduce_rows_f32"
    if scale is not None:  # out = sum * scale: the _ex entry, with the split workspace when the rule splits
        kid = "ihip_reduce_rows_f32_ex"
        args += (("f32", scale),) + ((("workspace", 4 * M * segs),) if segs > 1 else (("null", None), ("i64", 0)))
    if segs > 1:  # rows too few for the CUs: S workgroups of 16 waves per row, partials in a workspace
        launch = HipLaunch((M * segs, 1, 1), (1024, 1, 1), 64)
        if scale is None:
            kid, args = "ihip_reduce_rows_f32_ws", args + (("workspace", 4 * M * segs),)
        return HipLoweredKernel(c.fn.name, kid, c.io([x, oname]), launch, [oname], dict(c.b), args)
    if 0 < N and N // 4 <= 128:  # short rows: g lanes per row (two to four vectors each), several per wave
        g = 1
        while g < 32 and 2 * g < N // 4:
            g *= 2
        launch = HipLaunch((max(1, _cdiv(M * g, 256)), 1, 1), (256, 1, 1), 0)
    elif N > 0:  # 16-byte body loads (a head and tail of < 4 elements around them when rows are
        # not 16-byte aligned): a wave per row, or 16 waves per row for few long rows
        few_long = M < 2048 and N // 4 > 256
        launch = HipLaunch((max(1, M), 1, 1), (1024 if few_long else 64, 1, 1), 64 if few_long else 0)
    else:
        launch = _row_launch(M)
    return HipLoweredKernel(c.fn.name, kid, c.io([x, oname]), launch, [oname], dict(c.b), args)


def reduce_rows_segments(M: int, N: int) -> int:
    """Segments per row of the split row reduction (rows.hip reduce_rows_segments): rows below
    256 are split so that about 512 workgroups run, at most 64 per row, each segment at least
    4096 16-byte vectors; 1 = no split."""
    if M <= 0 or M >= 256 or N <= 0:
        return 1
    n4 = N // 4
    s = min(64, _cdiv(512, M))
    while s > 1 and n4 // s < 4096:
        s -= 1
    return s


_EW_KINDS = frozenset({"in", "const", "bcast", "transpose", "iota", "cast", "where"}) | frozenset(EW_BINARY) | frozenset(
    EW_UNARY)


def _is_elementwise(tree: Any) -> bool:
    if not isinstance(tree, tuple) or not tree or tree[0] not in _EW_KINDS:
        return False
    k = tree[0]
    if k in ("in", "const", "iota"):
        return True
    if k in ("bcast", "transpose", "cast"):
        return _is_elementwise(tree[1])
    return all(_is_elementwise(t) for t in tree[1:])


def _leaves(tree: Any, out: List[str]) -> None:
    if isinstance(tree, tuple) and tree:
        if tree[0] == "in":
            if tree[1] not in out:
                out.append(tree[1])
            return
        for t in tree[1:]:
            _leaves(t, out)


def _match_elementwise(c: _Ctx) -> Optional[HipLoweredKernel]:
    """Any remaining chain of element-wise ops: one register program on ihip_elementwise_program
    (the reference's fused element-wise lowering, intentir_to_cuda.py:229-534, dispatched at :2170-2199)."""
    c.knobs.used.add("HIP_ELEMENTWISE_PROGRAM")
    outs = list(c.fn.outputs)
    if not all(_is_elementwise(c.outs[o].tree) for o in outs):
        return None
    shp = c.shape(outs[0])
    for o in outs:
        if c.shape(o) != shp:
            raise HipLoweringError(f"element-wise outputs of different shapes: {outs}")
    names: List[str] = []
    for o in outs:
        _leaves(c.outs[o].tree, names)
    for n in names + outs:
        if c.dtype(n) not in EW_DTYPE_CODE:
            raise HipLoweringError(f"element-wise program does not take {c.dtype(n)} ({n})")
    trees = [(o, c.outs[o].tree) for o in outs]
    decl, units = {n: c.shape(n) for n in names}, {n: c.eb.get(n).unit for n in names}
    try:
        try:
            prog = compile_elementwise(trees, shp, decl, units)
        except EwLimitError:  # beyond the interpreter kernel: the native form's limits
            prog = compile_elementwise(trees, shp, decl, units, native=True)
    except EwCompileError as e:
        raise HipLoweringError(f"element-wise chain of {c.fn.name}: {e}") from e
    used = []
    for n, _ in prog.inputs:
        if n not in used:
            used.append(n)
    launch = _ew_launch(prog, c.dtype)
    return HipLoweredKernel(c.fn.name, "ihip_elementwise_program", c.io(used + outs), launch, outs, dict(c.b),
                            (("ew_program", prog),))


def _ew_launch(prog, dtype_of) -> HipLaunch:
    """The launch ihip_elementwise_program plans (ewjit.hip plan_jit) for dense 16-byte aligned
    outputs: lanes own 8 elements when every operand is 16-bit or narrower, else 4.  Inputs read
    across their unit-stride axis (axis 2 contiguous, axis 3 strided; up to 4) select the
    LDS-tiled form: one workgroup per 64 x 64 tile, a 64 x 65 f32 tile each.  Otherwise up to
    16384 256-lane workgroups stride over groups of U rows and over vectors."""
    sh = [1] * (4 - len(prog.shape)) + [int(d) for d in prog.shape]
    narrow = all(dtype_of(n) in ("f16", "bf16", "bool", "i1", "u8") for n in [i for i, _ in prog.inputs] + list(prog.outputs))
    v = 8 if narrow else 4
    tiled = 0
    if sh[2] > 1 and sh[3] > 1:
        for _, st in prog.inputs:
            if tiled < 4 and st[2] == 1 and st[3] not in (0, 1):
                tiled += 1
    if tiled:
        tx, ty = _cdiv(sh[3], 64), sh[0] * sh[1] * _cdiv(sh[2], 64)
        return HipLaunch((max(1, min(tx, 65535)), max(1, min(ty, 65535)), 1), (256, 1, 1), tiled * 64 * 65 * 4)
    rows = sh[0] * sh[1] * sh[2]
    gx = max(1, min(1024, _cdiv(_cdiv(sh[3], v), 256)))
    # a lane takes U rows per trip, U = 64 // (row-varying loads x elements per lane) in 1..4
    # (ew_jit_rows_per_trip); inputs with zero stride or extent 1 on axes 0-2 do not count
    rowinv = [all(st[d] == 0 or sh[d] == 1 for d in range(3)) for _, st in prog.inputs]
    loads = sum(1 for ins in prog.code if ins[0] == 1 and not rowinv[ins[2]])
    U = 4 if loads == 0 else max(1, min(4, 64 // (loads * v)))
    return HipLaunch((gx, max(1, min(_cdiv(rows, U), 65535, _cdiv(16384, gx))), 1), (256, 1, 1), 0)


def call_args_to_json(call_args) -> List[Dict[str, Any]]:
    """The C argument plan as JSON (element-wise programs spelled out as tables)."""
    from .ewprogram import EwProgram  # noqa: PLC0415

    out = []
    for kind, v in call_args:
        if kind == "tensor":
            out.append({"kind": kind, "name": v})
        elif kind == "ew_program":
            assert isinstance(v, EwProgram)
            out.append({"kind": kind, "code": [list(ins) for ins in v.code],
                        "inputs": [{"name": n, "stride": list(st)} for n, st in v.inputs],
                        "outputs": list(v.outputs), "shape": list(v.shape), "listing": v.listing()})
        else:
            out.append({"kind": kind, "value": v})
    return out


def call_args_from_json(plan) -> Tuple[Tuple[str, Any], ...]:
    """Inverse of ``call_args_to_json``."""
    from .ewprogram import EwProgram  # noqa: PLC0415

    out: List[Tuple[str, Any]] = []
    for a in plan:
        kind = a["kind"]
        if kind == "tensor":
            out.append((kind, a["name"]))
        elif kind == "ew_program":
            code = tuple((int(op), int(d), int(x), int(y), int(z), float(imm)) for op, d, x, y, z, imm in a["code"])
            ins = tuple((i["name"], tuple(int(t) for t in i["stride"])) for i in a["inputs"])
            out.append((kind, EwProgram(code, ins, tuple(a["outputs"]), tuple(int(d) for d in a["shape"]))))
        else:
            out.append((kind, a["value"]))
    return tuple(out)


_MATCHERS = (_match_gemm, _match_reduce_any, _match_softmax, _match_layernorm, _match_gelu_axpy, _match_row_reduce,
             _match_elementwise)


def lower_intent_to_hip_kernel(intent, *, shape_bindings: Mapping[str, Any],
                               schedule_override: ScheduleSketch | Dict[str, Any] | None = None) -> HipLoweredKernel:
    """Lower one IntentIR function to a single gfx950 kernel call.

    ``intent`` may be an IntentIR JSON dict, an ``intent_ir_amd.ir.IntentFunction``
    or a reference ``IntentFunction`` (anything with ``to_json_dict()``).  Raises
    ``HipLoweringError`` when no kernel family matches."""
    bindings = _normalize_bindings(shape_bindings)
    _reference_knobs(shape_bindings, bindings)
    bindings.setdefault("HIP_RESPECT_SCHEDULE", 1 if schedule_override is not None else 0)
    fn = as_intent(intent)
    if schedule_override is not None:
        fn.schedule = (schedule_override if isinstance(schedule_override, ScheduleSketch)
                       else ScheduleSketch.from_json(schedule_override))
    fn = expand_macros(fn)
    unsupported = sorted({o.op for o in fn.ops} - HIP_SUPPORTED_OPS)
    if unsupported:
        raise HipLoweringError(f"HIP lowering unsupported ops {unsupported} in {fn.name}")
    k = _match_gather(fn, bindings)
    if k is not None:
        _Knobs(fn, bindings).check_used(k.kernel_id)
        k.io_spec["hip_call"] = call_args_to_json(k.call_args)
        return k
    try:
        ctx = _Ctx(fn, bindings)
    except PatternError as e:
        raise HipLoweringError(f"HIP lowering cannot read {fn.name}: {e}") from e
    for m in _MATCHERS:
        k = m(ctx)
        if k is not None:
            ctx.knobs.check_used(k.kernel_id)
            # the argument plan also travels in io_spec (as the reference's io_spec carries its
            # host_launch), so run_hip_kernel needs only the reference's arguments
            k.io_spec["hip_call"] = call_args_to_json(k.call_args)
            return k
    raise HipLoweringError(f"HIP lowering unsupported for intent: name={fn.name} ops={sorted({o.op for o in fn.ops})}")


__all__ = ["HipLoweringError", "HipLaunch", "HipLoweredKernel", "KNOBS", "call_args_from_json", "call_args_to_json",
           "lower_intent_to_hip_kernel", "reduce_rows_segments", "softmax_split_plan"]
