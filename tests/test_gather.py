"""gather lowering (CPU only): the CUDA backend's lone-op gather2d form and its rejections.

The reference dispatches a single-op gather(inp [M, N] f32, row [L] i32, col [L] i32) to
_kernel_gather2d_f32 (backends/cuda/codegen/intentir_to_cuda.py:1779-1832, :2155-2156);
here it lowers to ihip_gather2d_f32.  The IR below is the reference's own test case
(tests/backends/cuda/test_cuda_backend_smoke.py:292-310)."""

from __future__ import annotations

import copy
import ctypes

import pytest

from intent_ir_amd import HipLoweringError, lower_intent_to_hip_kernel
from intent_ir_amd.runtime import SIGNATURES, load_library

GATHER_IR = {
    "name": "gather2d_cuda_smoke",
    "tensors": {
        "A": {"dtype": "f32", "shape": ["M", "N"], "layout": "row_major"},
        "row": {"dtype": "i32", "shape": ["L"], "layout": "row_major"},
        "col": {"dtype": "i32", "shape": ["L"], "layout": "row_major"},
        "Out": {"dtype": "f32", "shape": ["L"], "layout": "row_major"},
    },
    "ops": [{"op": "gather", "inputs": ["A", "row", "col"], "output": "Out", "attrs": {"other_value": -1.0}}],
    "outputs": ["Out"],
    "parallel_axes": ["L"],
    "schedule": {"tile_n": 256, "parallel_axes": ["L"]},
}


def test_reference_gather_ir_lowers_to_the_gather_kernel():
    k = lower_intent_to_hip_kernel(GATHER_IR, shape_bindings={"M": 7, "N": 9, "L": 32})
    assert k.kernel_id == "ihip_gather2d_f32"
    assert k.call_args == (("tensor", "A"), ("tensor", "row"), ("tensor", "col"), ("tensor", "Out"), ("i64", 7),
                           ("i64", 9), ("i64", 32), ("f32", -1.0))
    assert len(k.call_args) + 1 == len(SIGNATURES[k.kernel_id][1])
    assert k.launch.grid == (1, 1, 1) and k.launch.block == (256, 1, 1)
    assert k.output_names == ["Out"] and set(k.io_spec["tensors"]) == {"A", "row", "col", "Out"}
    big = lower_intent_to_hip_kernel(GATHER_IR, shape_bindings={"M": 4096, "N": 8192, "L": 1 << 22})
    assert big.launch.grid == (4096, 1, 1)  # 4 elements per thread, 256 threads per workgroup
    ir = copy.deepcopy(GATHER_IR)
    del ir["ops"][0]["attrs"]
    assert lower_intent_to_hip_kernel(ir, shape_bindings={"M": 7, "N": 9, "L": 32}).call_args[-1] == ("f32", 0.0)


def _variant(mutate):
    ir = copy.deepcopy(GATHER_IR)
    mutate(ir)
    return ir


@pytest.mark.parametrize("mutate,msg", [
    (lambda ir: ir["tensors"]["A"].__setitem__("dtype", "f16"), "lone op"),
    (lambda ir: ir["tensors"]["row"].__setitem__("dtype", "i64"), "lone op"),
    (lambda ir: ir["tensors"]["A"].__setitem__("shape", ["M", "N", "L"]), "shapes"),
    (lambda ir: ir["tensors"]["col"].__setitem__("shape", ["M"]), "shapes"),
    (lambda ir: ir["ops"][0].__setitem__("inputs", ["A", "row"]), "lone op"),
    (lambda ir: ir["ops"][0]["attrs"].__setitem__("other_value", "x"), "number"),
    # gather feeding another op: not the lone-op form
    (lambda ir: (ir["tensors"].__setitem__("Y", {"dtype": "f32", "shape": ["L"]}),
                 ir["ops"].append({"op": "exp", "inputs": ["Out"], "output": "Y"}),
                 ir.__setitem__("outputs", ["Y"])), "lone op"),
])
def test_other_gather_forms_are_rejected(mutate, msg):
    with pytest.raises(HipLoweringError, match=msg):
        lower_intent_to_hip_kernel(_variant(mutate), shape_bindings={"M": 7, "N": 9, "L": 32})


def test_authoritative_schedule_fields_are_rejected():
    """The gather kernel has one launch shape: an authoritative tile_n is refused, not ignored."""
    with pytest.raises(HipLoweringError, match="not available for ihip_gather2d_f32"):
        lower_intent_to_hip_kernel(GATHER_IR, shape_bindings={"M": 7, "N": 9, "L": 32},
                                   schedule_override={"tile_n": 256})


def test_gather_argument_checks_without_a_device():
    lib = load_library()
    p = ctypes.c_void_p(256)  # never dereferenced: the checks return before any HIP call
    assert lib.ihip_gather2d_f32(p, p, p, p, 7, 9, -1, 0.0, None) == -1
    assert b"invalid shape" in lib.ihip_last_error()
    assert lib.ihip_gather2d_f32(p, None, p, p, 7, 9, 32, 0.0, None) == -1
    assert b"null pointer" in lib.ihip_last_error()
    assert lib.ihip_gather2d_f32(None, p, p, p, 7, 9, 32, 0.0, None) == -1
    assert b"inp is null" in lib.ihip_last_error()
    assert lib.ihip_gather2d_f32(p, p, p, p, 1 << 40, 1 << 40, 32, 0.0, None) == -1
    assert lib.ihip_gather2d_f32(None, None, None, None, 7, 9, 0, 0.0, None) == 0  # L = 0: nothing to do
