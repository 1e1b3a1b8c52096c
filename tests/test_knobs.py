"""Schedule knobs and the reference-shaped runtime call — CPU only (lowering, no launches).

The reference steers launch shapes with ``CUDA_RESPECT_SCHEDULE`` (a schedule override
is authoritative, a recovered schedule only a hint) and with knobs carried in the
bindings (backends/cuda/codegen/intentir_to_cuda.py:1012,1175-1200,2074-2097).  Here
each knob either selects one of the precompiled variants or raises HipLoweringError.
"""

from __future__ import annotations

import inspect
import json

import pytest

from intent_ir_amd import HipLoweringError, lower_intent_to_hip_kernel
from intent_ir_amd.configs import WORKLOADS
from intent_ir_amd.lowering import call_args_from_json
from intent_ir_amd.runtime import run_hip_kernel
from tests.ew_cases import CASES as EW_CASES

GEMM_B = {"M": 1024, "N": 1024, "K": 512}  # 16 tiles of 256x256: the automatic choice is 128x128


def test_gemm_tile_binding_knob():
    ir = WORKLOADS["matmul"].ir()
    auto = lower_intent_to_hip_kernel(ir, shape_bindings=GEMM_B)
    assert auto.kernel_id == "ihip_gemm_bf16_bias_relu" and auto.launch.grid[0] == 64
    k = lower_intent_to_hip_kernel(ir, shape_bindings={**GEMM_B, "HIP_GEMM_TILE": 256})
    assert k.kernel_id == "ihip_gemm_bf16_bias_relu_ex"
    assert k.call_args[-3:] == (("i32", 0), ("i32", 1), ("i32", 256))  # transpose_b, relu, tile
    assert k.launch.grid[0] == 16 and k.launch.lds_bytes == 163840
    k = lower_intent_to_hip_kernel(ir, shape_bindings={**GEMM_B, "HIP_GEMM_TILE": 128})
    assert k.call_args[-1] == ("i32", 128) and k.launch.grid[0] == 64 and k.launch.lds_bytes == 81920
    with pytest.raises(HipLoweringError, match="not available for the bf16 GEMM"):
        lower_intent_to_hip_kernel(ir, shape_bindings={**GEMM_B, "HIP_GEMM_TILE": 64})
    with pytest.raises(HipLoweringError, match="is not one of"):
        lower_intent_to_hip_kernel(ir, shape_bindings={**GEMM_B, "HIP_GEMM_TILE": 32})


def test_gemm_tile_from_an_authoritative_schedule():
    ir = WORKLOADS["matmul"].ir()
    k = lower_intent_to_hip_kernel(ir, shape_bindings=GEMM_B,
                                   schedule_override={"tile_m": 256, "tile_n": 256, "tile_k": 32, "pipeline_depth": 4})
    assert k.call_args[-1] == ("i32", 256) and k.bindings["HIP_RESPECT_SCHEDULE"] == 1
    k = lower_intent_to_hip_kernel(ir, shape_bindings={**GEMM_B, "T": 128}, schedule_override={"tile_m": "T"})
    assert k.call_args[-1] == ("i32", 128)
    # the binding knob overrides the schedule's tile, as the reference's tuning knobs do
    k = lower_intent_to_hip_kernel(ir, shape_bindings={**GEMM_B, "HIP_GEMM_TILE": 128},
                                   schedule_override={"tile_m": 256, "tile_n": 256})
    assert k.call_args[-1] == ("i32", 128)
    for sched, msg in (({"tile_m": 64}, "not available"), ({"tile_m": 128, "tile_n": 256}, "square"),
                       ({"tile_k": 64}, "not available"), ({"pipeline_depth": 2}, "not available"),
                       ({"tile_m": "NOPE"}, "names no integer binding")):
        with pytest.raises(HipLoweringError, match=msg):
            lower_intent_to_hip_kernel(ir, shape_bindings=GEMM_B, schedule_override=sched)


def test_recovered_schedule_is_a_hint_unless_respected():
    """The IR's own schedule (tile_m=32, ...) is ignored by default, authoritative on request."""
    ir = WORKLOADS["matmul"].ir()
    assert ir["schedule"]["tile_m"] == 32
    assert lower_intent_to_hip_kernel(ir, shape_bindings=GEMM_B).kernel_id == "ihip_gemm_bf16_bias_relu"
    with pytest.raises(HipLoweringError, match="not available"):
        lower_intent_to_hip_kernel(ir, shape_bindings={**GEMM_B, "HIP_RESPECT_SCHEDULE": 1})


def test_gemm_tile_knob_on_the_packed_path():
    ir = WORKLOADS["matmul"].ir()
    b = {"M": 64, "N": 263, "K": 64}  # N % 8 != 0 with B as [K, N]: B packed, then the tiled kernel
    k = lower_intent_to_hip_kernel(ir, shape_bindings={**b, "HIP_GEMM_TILE": 256})
    assert k.kernel_id == "ihip_gemm_bf16_bias_relu_ws" and k.call_args[-2] == ("i32", 256)
    assert k.call_args[-1] == ("workspace", 263 * 64 * 2 + 256 - 263 * 64 * 2 % 256)
    assert k.launch.lds_bytes == 163840 and k.launch.grid[0] == 2
    k = lower_intent_to_hip_kernel(ir, shape_bindings={**b, "HIP_GEMM_TILE": 128})
    assert k.launch.lds_bytes == 81920 and k.launch.grid[0] == 3
    auto = lower_intent_to_hip_kernel(ir, shape_bindings=b)  # 2 tiles of 256x256: 128x128 tiles
    assert auto.launch == k.launch and auto.call_args[-2] == ("i32", 0)


def test_gemm_tile_knob_on_the_guarded_kernel():
    ir = WORKLOADS["matmul"].ir()
    # a ragged K (K % 32 != 0) with operands above 2 GiB, whose rows are 16-byte aligned: the
    # guarded kernel (the tiled one points ragged k-chunks past every record)
    b = {"M": 65536, "N": 16384, "K": 40968}
    k = lower_intent_to_hip_kernel(ir, shape_bindings={**b, "HIP_GEMM_TILE": 256})
    assert k.kernel_id == "ihip_gemm_bf16_bias_relu_ex"
    assert k.launch.lds_bytes == 147456 and k.launch.grid[0] == 256 * 64
    k = lower_intent_to_hip_kernel(ir, shape_bindings={**b, "HIP_GEMM_TILE": 128})
    assert k.launch.lds_bytes == 73728 and k.launch.grid[0] == 512 * 128


@pytest.mark.parametrize("rows", [1, 2, 4])
def test_softmax_rows_per_workgroup_knob(rows):
    ir = WORKLOADS["softmax"].ir()
    k = lower_intent_to_hip_kernel(ir, shape_bindings={"M": 1000, "N": 1024, "HIP_ROWS_PER_WG": rows})
    assert k.kernel_id == "ihip_softmax_rows_f32_ex" and k.call_args[-1] == ("i32", rows)
    # four rows of 1024 floats run as two waves of two rows each
    assert k.launch.block[0] == (128 if rows == 4 else 64 * rows) and k.launch.grid[0] == -(-1000 // rows)
    k2 = lower_intent_to_hip_kernel(ir, shape_bindings={"M": 1000, "N": 1024}, schedule_override={"tile_m": rows})
    assert k2.call_args == k.call_args and k2.launch == k.launch


def test_softmax_rows_knob_outside_the_one_wave_form():
    ir = WORKLOADS["softmax"].ir()
    with pytest.raises(HipLoweringError, match="one-wave-per-row"):
        lower_intent_to_hip_kernel(ir, shape_bindings={"M": 8, "N": 8192, "HIP_ROWS_PER_WG": 2})
    k = lower_intent_to_hip_kernel(ir, shape_bindings={"M": 8, "N": 8192, "HIP_ROWS_PER_WG": 1})
    assert k.call_args[-1] == ("i32", 1)
    with pytest.raises(HipLoweringError, match="not available"):
        lower_intent_to_hip_kernel(ir, shape_bindings={"M": 8, "N": 1024}, schedule_override={"tile_m": 16})


@pytest.mark.parametrize("key,bindings,msg", [
    ("softmax", {"HIP_GEMM_TILE": 256}, "does not apply"),
    ("any", {"HIP_ROWS_PER_WG": 1}, "does not apply"),
    ("layernorm", {"HIP_GEMM_TILE": 128}, "does not apply"),
    ("gelu", {"HIP_FOO": 1}, "unknown HIP knob"),
    ("any", {"HIP_RESPECT_SCHEDULE": 2}, "is not one of"),
])
def test_knobs_that_do_not_apply_are_rejected(key, bindings, msg):
    w = WORKLOADS[key]
    b = {k: min(v, 64) for k, v in w.bindings.items()}
    with pytest.raises(HipLoweringError, match=msg):
        lower_intent_to_hip_kernel(w.ir(), shape_bindings={**b, **bindings})


@pytest.mark.parametrize("key", ["any", "layernorm", "gelu"])
def test_single_schedule_kernels_reject_authoritative_schedules(key):
    w = WORKLOADS[key]
    b = {k: min(v, 64) for k, v in w.bindings.items()}
    with pytest.raises(HipLoweringError, match="single launch schedule"):
        lower_intent_to_hip_kernel(w.ir(), shape_bindings=b, schedule_override={"tile_m": 16})
    # an override that sets no field asks for nothing
    lower_intent_to_hip_kernel(w.ir(), shape_bindings=b, schedule_override={})


def _all_lowerings():
    for key, w in WORKLOADS.items():
        yield key, lower_intent_to_hip_kernel(w.ir(), shape_bindings={k: min(v, 64) for k, v in w.bindings.items()})
    for name, ir, bindings, _ in EW_CASES[:6]:
        yield name, lower_intent_to_hip_kernel(ir, shape_bindings=bindings)


def test_call_plan_travels_in_io_spec_as_json():
    for name, k in _all_lowerings():
        spec = json.loads(json.dumps(k.io_spec))  # JSON-serialisable as is
        assert call_args_from_json(spec["hip_call"]) == k.call_args, name


def test_run_hip_kernel_takes_the_reference_arguments():
    """run_cuda_kernel(*, kernel_name, cuda_src, io_spec, launch, bindings, inputs_np, output_names,
    extra_cuda_cflags=None) (backends/cuda/runtime.py:22-45): the same keywords, cuda_src replaced
    by kernel_id, and nothing else required."""
    sig = inspect.signature(run_hip_kernel)
    required = {n for n, p in sig.parameters.items() if p.default is inspect.Parameter.empty}
    assert required == {"kernel_name", "kernel_id", "io_spec", "launch", "bindings", "inputs_np", "output_names"}
    assert all(p.kind is inspect.Parameter.KEYWORD_ONLY for p in sig.parameters.values())


def test_gelu_chain_in_other_dtypes_runs_as_a_program():
    """The bias + GELU + axpy kernel is bf16-only; the same chain in f32 or f16 is a generic program."""
    from intent_ir_amd.configs import bias_gelu_axpy_ir

    for dt in ("f32", "f16"):
        k = lower_intent_to_hip_kernel(bias_gelu_axpy_ir(dt), shape_bindings={"M": 8, "N": 64})
        assert k.kernel_id == "ihip_elementwise_program", dt


def test_elementwise_program_knob():
    w = WORKLOADS["gelu"]
    b = {"M": 8, "N": 64}
    assert lower_intent_to_hip_kernel(w.ir(), shape_bindings=b).kernel_id == "ihip_bias_gelu_tanh_axpy_bf16"
    k = lower_intent_to_hip_kernel(w.ir(), shape_bindings={**b, "HIP_ELEMENTWISE_PROGRAM": 1})
    assert k.kernel_id == "ihip_elementwise_program"
    with pytest.raises(HipLoweringError, match="does not apply"):
        lower_intent_to_hip_kernel(WORKLOADS["softmax"].ir(), shape_bindings={**b, "HIP_ELEMENTWISE_PROGRAM": 1})


def test_reference_cuda_knobs_are_honoured_or_rejected():
    """The reference's own binding knobs (intentir_to_cuda.py:577,1012,1175-1190 and the WMMA
    and launch knobs) either mean something here or raise: CUDA_RESPECT_SCHEDULE is
    HIP_RESPECT_SCHEDULE, ALLOW_TF32 only permits reduced precision (never used), a knob at the
    value where it requests nothing passes, any other request raises HipLoweringError."""
    ir = WORKLOADS["softmax"].ir()
    b = {"M": 64, "N": 1024}
    ir_s = dict(ir, schedule={"tile_m": 2})
    # CUDA_RESPECT_SCHEDULE=1 makes the IR's own schedule authoritative, as HIP_RESPECT_SCHEDULE=1 does
    k_cuda = lower_intent_to_hip_kernel(ir_s, shape_bindings={**b, "CUDA_RESPECT_SCHEDULE": 1})
    k_hip = lower_intent_to_hip_kernel(ir_s, shape_bindings={**b, "HIP_RESPECT_SCHEDULE": 1})
    assert k_cuda.call_args == k_hip.call_args and k_cuda.bindings["HIP_RESPECT_SCHEDULE"] == 1
    assert "CUDA_RESPECT_SCHEDULE" not in k_cuda.bindings
    k0 = lower_intent_to_hip_kernel(ir_s, shape_bindings={**b, "CUDA_RESPECT_SCHEDULE": 0})
    assert k0.call_args == lower_intent_to_hip_kernel(ir_s, shape_bindings=b).call_args
    with pytest.raises(HipLoweringError, match="disagree"):
        lower_intent_to_hip_kernel(ir, shape_bindings={**b, "CUDA_RESPECT_SCHEDULE": 1, "HIP_RESPECT_SCHEDULE": 0})
    with pytest.raises(HipLoweringError, match="is not one of"):
        lower_intent_to_hip_kernel(ir, shape_bindings={**b, "CUDA_RESPECT_SCHEDULE": 2})
    # launch-shape knobs: the no-request value passes, a request raises and names the HIP knob
    base = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    for idle in ({"SOFTMAX_THREADS": 0}, {"SOFTMAX_MAX_EPT": 16}, {"SOFTMAX_MAX_EPT": "16"}, {"WMMA_CP_A_POLICY": ""}):
        k = lower_intent_to_hip_kernel(ir, shape_bindings={**b, **idle})
        assert k.call_args == base.call_args and not set(idle) & set(k.bindings)
    with pytest.raises(HipLoweringError, match="SOFTMAX_THREADS=128 .*HIP_ROWS_PER_WG"):
        lower_intent_to_hip_kernel(ir, shape_bindings={**b, "SOFTMAX_THREADS": 128})
    with pytest.raises(HipLoweringError, match="SOFTMAX_MAX_EPT=8"):
        lower_intent_to_hip_kernel(ir, shape_bindings={**b, "SOFTMAX_MAX_EPT": 8})
    mm = WORKLOADS["matmul"].ir()
    with pytest.raises(HipLoweringError, match="WMMA_WARPS_M=2 .*HIP_GEMM_TILE"):
        lower_intent_to_hip_kernel(mm, shape_bindings={**GEMM_B, "WMMA_WARPS_M": 2})
    with pytest.raises(HipLoweringError, match="WMMA_CP_A_POLICY='cg'"):
        lower_intent_to_hip_kernel(mm, shape_bindings={**GEMM_B, "WMMA_CP_A_POLICY": "cg"})
    # ALLOW_TF32 permits a reduced-precision path; the exact f32 GEMM honours both values
    f32 = json.loads(json.dumps(mm))
    for t in ("A", "B", "C"):
        f32["tensors"][t]["dtype"] = "f32"
    for v in (0, 1):
        k = lower_intent_to_hip_kernel(f32, shape_bindings={**GEMM_B, "ALLOW_TF32": v})
        assert k.kernel_id == "ihip_gemm_f32_bias_relu" and "ALLOW_TF32" not in k.bindings
    with pytest.raises(HipLoweringError, match="ALLOW_TF32"):
        lower_intent_to_hip_kernel(f32, shape_bindings={**GEMM_B, "ALLOW_TF32": 3})


def test_gemm_split_rule_follows_the_forced_tile():
    """gemm_pack.hip split_plan sizes its segments for 128x128 tiles; with 256x256 tiles on
    request (the tile knob) the rule leaves the grid unsplit, and the lowering's workspace
    holds no partials for it."""
    from intent_ir_amd.lowering import gemm_split_plan

    M, N, K = 1024, 1024, 8192  # 64 tiles of 128x128: the rule splits into 4
    assert gemm_split_plan(M, N, K)[0] == 4 and gemm_split_plan(M, N, K, tile=128)[0] == 4
    assert gemm_split_plan(M, N, K, tile=256) == (1, K)
    assert gemm_split_plan(M, N, K, 3, tile=256)[0] == 3  # an explicit count is taken as asked
    ir = WORKLOADS["matmul"].ir()
    b = {"M": M, "N": N, "K": K}
    auto = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    assert auto.kernel_id == "ihip_gemm_bf16_bias_relu_ws" and auto.launch.grid[0] == 64 * 4
    big = lower_intent_to_hip_kernel(ir, shape_bindings={**b, "HIP_GEMM_TILE": 256})
    assert big.kernel_id == "ihip_gemm_bf16_bias_relu_ex" and big.launch.grid[0] == 16
