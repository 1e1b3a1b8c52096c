"""The reference's deterministic builder IRs, restated as JSON-form fixtures.

Each entry is the IntentIR the reference builds for one kernel (same tensor names, dtypes,
shapes, ops and attributes; schedules included where the builder sets them), written out by
hand from the cited builder.  Nothing here imports the reference.  Intermediates the builder
declares are declared here too, so the interpreter's name-based broadcasting sees the same
shapes.

``BUILDERS[name] = (citation, ir, kernel_id or None, reason)``: the C-ABI entry the HIP
lowering must pick, or None with the reason the IR is outside the backend (it then has to
raise HipLoweringError).
"""

from __future__ import annotations

import copy
from typing import Any, Dict, Optional, Tuple


def _t(dtype: str, *shape: Any) -> Dict[str, Any]:
    return {"dtype": dtype, "shape": list(shape), "layout": "row_major"}


def _op(op: str, inputs, output: str, **attrs) -> Dict[str, Any]:
    return {"op": op, "inputs": list(inputs), "output": output, "attrs": attrs}


def _ir(name, tensors, ops, outputs, schedule=None) -> Dict[str, Any]:
    d = {"name": name, "tensors": tensors, "ops": ops, "outputs": outputs}
    if schedule is not None:
        d["schedule"] = schedule
    return d


_S16 = {"tile_m": 16, "tile_n": 16, "tile_k": None, "vec_width": 1, "pipeline_depth": 1}
_S1 = {"tile_m": None, "tile_n": None, "tile_k": None, "vec_width": 1, "pipeline_depth": 1}
_SMM = {"tile_m": 32, "tile_n": 32, "tile_k": 16, "vec_width": 1, "pipeline_depth": 2}
MN = ("M", "N")


def _ew2(name, op, src):
    return _ir(name, {"A": _t("f32", *MN), "B": _t("f32", *MN), "C": _t("f32", *MN)}, [_op(op, ["A", "B"], "C")],
               ["C"], _S16)


def _ew1(name, op):
    return _ir(name, {"inp": _t("f32", *MN), "out": _t("f32", *MN)}, [_op(op, ["inp"], "out")], ["out"], _S16)


def _ln_tilelang(dt: str = "f32"):
    # pipeline/tilelang/core.py:1322-1384 (layer_norm_persistent)
    t = {"in_ptr": _t(dt, *MN), "weight_ptr": _t(dt, "N"), "bias_ptr": _t(dt, "N"), "out_ptr": _t(dt, *MN),
         "out_mean_ptr": _t("f32", "M"), "out_rstd_ptr": _t("f32", "M"),
         "sum_row": _t("f32", "M", 1), "mean_row": _t("f32", "M", 1), "diff": _t("f32", *MN), "sq": _t("f32", *MN),
         "var_sum": _t("f32", "M", 1), "var": _t("f32", "M", 1), "eps": _t("f32"), "var_eps": _t("f32", "M", 1),
         "rstd_row": _t("f32", "M", 1), "xhat": _t("f32", *MN), "w_b": _t("f32", *MN), "b_b": _t("f32", *MN),
         "scaled": _t("f32", *MN)}
    ops = [_op("reduce_sum", ["in_ptr"], "sum_row", dims=[1], keepdims=True),
           _op("div", ["sum_row"], "mean_row", divisor="N"),
           _op("sub", ["in_ptr", "mean_row"], "diff"),
           _op("mul", ["diff", "diff"], "sq"),
           _op("reduce_sum", ["sq"], "var_sum", dims=[1], keepdims=True),
           _op("div", ["var_sum"], "var", divisor="N"),
           _op("const", [], "eps", value=1e-5, dtype="f32"),
           _op("add", ["var", "eps"], "var_eps"),
           _op("rsqrt", ["var_eps"], "rstd_row"),
           _op("mul", ["diff", "rstd_row"], "xhat"),
           _op("broadcast_in_dim", ["weight_ptr"], "w_b", out_shape=["M", "N"], broadcast_dims=[1]),
           _op("broadcast_in_dim", ["bias_ptr"], "b_b", out_shape=["M", "N"], broadcast_dims=[1]),
           _op("mul", ["xhat", "w_b"], "scaled"),
           _op("add", ["scaled", "b_b"], "out_ptr"),
           _op("reshape", ["mean_row"], "out_mean_ptr", shape=["M"]),
           _op("reshape", ["rstd_row"], "out_rstd_ptr", shape=["M"])]
    return _ir("layer_norm_persistent", t, ops, ["out_ptr", "out_mean_ptr", "out_rstd_ptr"], _S16)


def _ln_cuda():
    # pipeline/cuda/core.py:496-546: reduce_sum{scale: "1.0/N"}, w and b broadcast by numpy
    t = {"in_ptr": _t("f32", *MN), "weight_ptr": _t("f32", "N"), "bias_ptr": _t("f32", "N"),
         "out_ptr": _t("f32", *MN), "out_mean_ptr": _t("f32", "M"), "out_rstd_ptr": _t("f32", "M")}
    ops = [_op("reduce_sum", ["in_ptr"], "out_mean_ptr", dims=[1], keepdims=False, scale="1.0/N"),
           _op("broadcast_in_dim", ["out_mean_ptr"], "mean_2d", out_shape=["M", "N"], broadcast_dims=[0]),
           _op("sub", ["in_ptr", "mean_2d"], "centered"),
           _op("mul", ["centered", "centered"], "sq"),
           _op("reduce_sum", ["sq"], "var", dims=[1], keepdims=False, scale="1.0/N"),
           _op("const", [], "eps", value=1e-5, dtype="f32"),
           _op("add", ["var", "eps"], "var_eps"),
           _op("rsqrt", ["var_eps"], "out_rstd_ptr"),
           _op("broadcast_in_dim", ["out_rstd_ptr"], "rstd_2d", out_shape=["M", "N"], broadcast_dims=[0]),
           _op("mul", ["centered", "rstd_2d"], "norm"),
           _op("mul", ["norm", "weight_ptr"], "scaled"),
           _op("add", ["scaled", "bias_ptr"], "out_ptr")]
    return _ir("layer_norm_persistent", t, ops, ["out_ptr", "out_mean_ptr", "out_rstd_ptr"], _S1)


def _softmax_cuda():
    # pipeline/cuda/core.py:453-493: the expanded chain, row max and row sum also returned
    t = {"input_ptr": _t("f32", *MN), "output_ptr": _t("f32", *MN), "row_max_ptr": _t("f32", "M"),
         "row_sum_ptr": _t("f32", "M")}
    ops = [_op("reduce_max", ["input_ptr"], "row_max_ptr", dims=[1], keepdims=False),
           _op("broadcast_in_dim", ["row_max_ptr"], "row_max_2d", out_shape=["M", "N"], broadcast_dims=[0]),
           _op("sub", ["input_ptr", "row_max_2d"], "x_shift"),
           _op("exp", ["x_shift"], "exp_scores"),
           _op("reduce_sum", ["exp_scores"], "row_sum_ptr", dims=[1], keepdims=False),
           _op("broadcast_in_dim", ["row_sum_ptr"], "row_sum_2d", out_shape=["M", "N"], broadcast_dims=[0]),
           _op("div", ["exp_scores", "row_sum_2d"], "output_ptr")]
    return _ir("softmax_inner", t, ops, ["output_ptr", "row_max_ptr", "row_sum_ptr"], _S1)


def _any(schedule):
    # pipeline/tilelang/core.py:115-130 and pipeline/cuda/core.py:409-426
    return _ir("any_kernel_dim", {"inp": _t("f32", *MN), "out": _t("bool", "M")},
               [_op("reduce_any", ["inp"], "out", dims=[1], keepdims=False)], ["out"], schedule)


def _clamp(schedule):
    # pipeline/tilelang/core.py:560-590 and pipeline/cuda/core.py:429-451: rank-0 lo / hi tensors
    return _ir("clamp2d", {"inp": _t("f32", *MN), "lo": _t("f32"), "hi": _t("f32"), "out": _t("f32", *MN),
                           **({"t0": _t("f32", *MN)} if schedule is _S16 else {})},
               [_op("max", ["inp", "lo"], "t0"), _op("min", ["t0", "hi"], "out")], ["out"], schedule)


def _mm(name, dt, ops, extra, outputs=("C",), schedule=_SMM):
    t = {"A": _t(dt, "M", "K"), "B": _t(dt, "K", "N"), "C": _t(dt, *MN), "mm": _t(dt, *MN), **extra}
    return _ir(name, t, ops, list(outputs), schedule)


BUILDERS: Dict[str, Tuple[str, Dict[str, Any], Optional[str], str]] = {
    # ---- reduce_any
    "tilelang.any_kernel_dim": ("pipeline/tilelang/core.py:115-130", _any(_S16), "ihip_reduce_any_rows_f32", ""),
    "cuda.any_kernel_dim": ("pipeline/cuda/core.py:409-426", _any(_S1), "ihip_reduce_any_rows_f32", ""),
    "cuda_smoke.any_ne": ("tests/backends/cuda/test_cuda_backend_smoke.py:249-267", _ir(
        "any_dim_cuda_smoke", {"A": _t("f32", *MN), "z": _t("f32"), "T": _t("i1", *MN), "Out": _t("i1", "M")},
        [_op("const", [], "z", value=0.0), _op("ne", ["A", "z"], "T"), _op("reduce_any", ["T"], "Out", dims=[1])],
        ["Out"], {"tile_n": 256, "parallel_axes": ["M"]}), "ihip_reduce_any_rows_f32", ""),
    # ---- softmax
    "tilelang.softmax_inner": ("pipeline/tilelang/core.py:259-274", _ir(
        "softmax_inner", {"input_ptr": _t("f32", *MN), "output_ptr": _t("f32", *MN)},
        [_op("softmax", ["input_ptr"], "output_ptr", axis=-1)], ["output_ptr"], _S16), "ihip_softmax_rows_f32", ""),
    "cuda.softmax_inner": ("pipeline/cuda/core.py:453-493", _softmax_cuda(), "ihip_softmax_rows_f32_stats", ""),
    # ---- LayerNorm
    "tilelang.layer_norm_persistent": ("pipeline/tilelang/core.py:1322-1384", _ln_tilelang(),
                                       "ihip_layernorm_rows_f32", ""),
    "cuda.layer_norm_persistent": ("pipeline/cuda/core.py:496-546", _ln_cuda(), "ihip_layernorm_rows_f32", ""),
    # ---- element-wise chains
    "tilelang.add2d": ("pipeline/tilelang/core.py:293-309", _ew2("add2d", "add", None), "ihip_elementwise_program", ""),
    "tilelang.transpose2d": ("pipeline/tilelang/core.py:323-338", _ir(
        "transpose2d", {"inp": _t("f32", *MN), "out": _t("f32", "N", "M")},
        [_op("transpose", ["inp"], "out", perm=[1, 0])], ["out"], _S16), "ihip_elementwise_program", ""),
    "tilelang.relu2d": ("pipeline/tilelang/core.py:352-367", _ew1("relu2d", "relu"), "ihip_elementwise_program", ""),
    "tilelang.add_bias2d": ("pipeline/tilelang/core.py:386-413", _ir(
        "add_bias2d", {"inp": _t("f32", *MN), "bias": _t("f32", "N"), "out": _t("f32", *MN), "bias2": _t("f32", *MN)},
        [_op("broadcast_in_dim", ["bias"], "bias2", out_shape=["M", "N"], broadcast_dims=[1]),
         _op("add", ["inp", "bias2"], "out")], ["out"], _S16), "ihip_elementwise_program", ""),
    "tilelang.where2d": ("pipeline/tilelang/core.py:431-451", _ir(
        "where2d", {"A": _t("f32", *MN), "B": _t("f32", *MN), "cond": _t("bool", *MN), "C": _t("f32", *MN)},
        [_op("gt", ["A", "B"], "cond"), _op("where", ["cond", "A", "B"], "C")], ["C"], _S16),
        "ihip_elementwise_program", ""),
    "tilelang.exp2d": ("pipeline/tilelang/core.py:494-509", _ew1("exp2d", "exp"), "ihip_elementwise_program", ""),
    "tilelang.floor2d": ("pipeline/tilelang/core.py:523-538", _ew1("floor2d", "floor"), "ihip_elementwise_program", ""),
    "tilelang.clamp2d": ("pipeline/tilelang/core.py:560-590", _clamp(_S16), "ihip_elementwise_program", ""),
    "cuda.clamp2d": ("pipeline/cuda/core.py:429-451", _clamp(_S1), "ihip_elementwise_program", ""),
    "tilelang.copy2d_divmod": ("pipeline/tilelang/core.py:623-638", _ew1("copy2d_divmod", "identity"),
                               "ihip_elementwise_program", ""),
    "tilelang.rowmask_where2d": ("pipeline/tilelang/core.py:1002-1024", _ir(
        "rowmask_where2d", {"inp": _t("f32", *MN), "row_mask": _t("bool", "M"), "out": _t("f32", *MN),
                            "m2": _t("bool", *MN), "z": _t("f32"), "z2": _t("f32", *MN)},
        [_op("broadcast_in_dim", ["row_mask"], "m2", out_shape=["M", "N"], broadcast_dims=[0]),
         _op("const", [], "z", value=0.0, dtype="f32"),
         _op("broadcast_in_dim", ["z"], "z2", out_shape=["M", "N"], broadcast_dims=[]),
         _op("where", ["m2", "inp", "z2"], "out")], ["out"], _S16), "ihip_elementwise_program", ""),
    "cuda_smoke.ew_bias_relu": ("tests/backends/cuda/test_cuda_backend_smoke.py:68-110", _ir(
        "ew_cuda_smoke", {"A": _t("f32", *MN), "B": _t("f32", "N"), "T": _t("f32", *MN), "Out": _t("f32", *MN)},
        [_op("add", ["A", "B"], "T"), _op("relu", ["T"], "Out")], ["Out"],
        {"tile_n": 256, "parallel_axes": ["M", "N"]}), "ihip_elementwise_program", ""),
    # ---- row reductions
    "tilelang.row_sum": ("pipeline/tilelang/core.py:465-480", _ir(
        "row_sum", {"inp": _t("f32", *MN), "out": _t("f32", "M")},
        [_op("reduce_sum", ["inp"], "out", dims=[1], keepdims=False)], ["out"], _S16), "ihip_reduce_rows_f32", ""),
    "tilelang.row_max": ("pipeline/tilelang/core.py:594-609", _ir(
        "row_max", {"inp": _t("f32", *MN), "out": _t("f32", "M")},
        [_op("reduce_max", ["inp"], "out", dims=[1], keepdims=False)], ["out"], _S16), "ihip_reduce_rows_f32", ""),
    # ---- matmul
    "cuda_smoke.matmul": ("tests/backends/cuda/test_cuda_backend_smoke.py:27-66", _ir(
        "mm_cuda_smoke", {"A": _t("f32", "M", "K"), "B": _t("f32", "K", "N"), "C": _t("f32", *MN)},
        [_op("matmul", ["A", "B"], "C")], ["C"], {"tile_m": 8, "tile_n": 16, "tile_k": 16, "parallel_axes": ["M", "N"]}),
        "ihip_gemm_f32_bias_relu", ""),
    "tilelang.matmul_relu2d": ("pipeline/tilelang/core.py:700-718", _mm(
        "matmul_relu2d", "f32", [_op("matmul", ["A", "B"], "mm"), _op("relu", ["mm"], "C")], {}),
        "ihip_gemm_f32_bias_relu", ""),
    "tilelang.matmul_bias_relu2d": ("pipeline/tilelang/core.py:886-910", _mm(
        "matmul_bias_relu2d", "f32",
        [_op("matmul", ["A", "B"], "mm"),
         _op("broadcast_in_dim", ["bias"], "b2", out_shape=["M", "N"], broadcast_dims=[1]),
         _op("add", ["mm", "b2"], "mm_b"), _op("relu", ["mm_b"], "C")],
        {"bias": _t("f32", "N"), "b2": _t("f32", *MN), "mm_b": _t("f32", *MN)}), "ihip_gemm_f32_bias_relu", ""),
}


def builder_ir(name: str) -> Dict[str, Any]:
    """A fresh copy of one builder's IR."""
    return copy.deepcopy(BUILDERS[name][1])


__all__ = ["BUILDERS", "builder_ir"]
