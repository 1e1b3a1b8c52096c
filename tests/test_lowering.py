"""IR loading, macro expansion and structural lowering — CPU only (no kernel launches)."""

from __future__ import annotations

import copy
import ctypes
import re
from pathlib import Path

import pytest

from intent_ir_amd import HipLoweringError, lower_intent_to_hip_kernel
from intent_ir_amd.configs import WORKLOADS, matmul_bias_relu2d_ir, softmax_inner_ir
from intent_ir_amd.lowering import gemm_workspace_bytes
from intent_ir_amd.ir import IntentFunction, IntentIRValidationError, as_intent
from intent_ir_amd.macros import expand_macros
from intent_ir_amd.runtime import LIB_PATH, SIGNATURES

ROOT = Path(__file__).resolve().parents[1]

EXPECTED_KERNEL = {
    "any": "ihip_reduce_any_rows_f32",
    "softmax": "ihip_softmax_rows_f32",
    "layernorm": "ihip_layernorm_rows_f16",
    "gelu": "ihip_bias_gelu_tanh_axpy_bf16",
    "matmul": "ihip_gemm_bf16_bias_relu",
}


@pytest.mark.parametrize("key", sorted(WORKLOADS))
def test_workloads_lower_to_their_kernel(key):
    w = WORKLOADS[key]
    k = lower_intent_to_hip_kernel(w.ir(), shape_bindings=w.bindings)
    assert k.kernel_id == EXPECTED_KERNEL[key]
    assert k.kernel_id in SIGNATURES
    # every tensor argument is declared in io_spec, and the arg count matches the C signature (+ stream)
    for kind, v in k.call_args:
        if kind == "tensor":
            assert v in k.io_spec["tensors"]
    assert len(k.call_args) + 1 == len(SIGNATURES[k.kernel_id][1])


def test_json_round_trip_and_reference_object_duck_typing():
    ir = WORKLOADS["layernorm"].ir()
    fn = IntentFunction.from_json_dict(ir)
    again = IntentFunction.from_json_dict(fn.to_json_dict())
    assert again.to_json_dict() == fn.to_json_dict()

    class RefLike:  # anything with to_json_dict(), like the reference IntentFunction
        def to_json_dict(self):
            return ir

    assert as_intent(RefLike()).to_json_dict() == fn.to_json_dict()
    k = lower_intent_to_hip_kernel(RefLike(), shape_bindings={"M": 8, "N": 64})
    assert k.kernel_id == "ihip_layernorm_rows_f16"


@pytest.mark.parametrize("mutate,msg", [
    (lambda ir: ir["ops"][0].__setitem__("inputs", ["nope"]), "undefined tensor"),
    (lambda ir: ir["ops"][0]["attrs"].__setitem__("dims", "1"), "dims must be list"),
    (lambda ir: ir.__setitem__("outputs", ["ghost"]), "not found"),
    (lambda ir: ir["tensors"]["inp"].__setitem__("dtype", "f8"), "dtype unsupported"),
    (lambda ir: ir["ops"][0].__setitem__("op", "frobnicate"), "unsupported"),
])
def test_validation_errors(mutate, msg):
    ir = copy.deepcopy(WORKLOADS["any"].ir())
    mutate(ir)
    with pytest.raises(IntentIRValidationError, match=msg):
        as_intent(ir)


def test_outputs_default_to_last_op():
    ir = softmax_inner_ir()
    del ir["outputs"]
    assert as_intent(ir).outputs == ["output_ptr"]


def test_gelu_macro_expands_to_interpreter_ops():
    fn = expand_macros(as_intent(WORKLOADS["gelu"].ir()))
    ops = {o.op for o in fn.ops}
    assert "gelu_tanh" not in ops
    assert ops <= {"broadcast_in_dim", "add", "mul", "const", "exp", "div"}
    assert all(o.attrs.get("dtype") == "f32" for o in fn.ops if o.op == "const")


def test_bindings_normalisation_and_knobs():
    w = WORKLOADS["softmax"]
    k = lower_intent_to_hip_kernel(w.ir(), shape_bindings={"M": 16.0, "N": "1024", "junk": object(), "flag": True})
    assert k.bindings["M"] == 16 and k.bindings["N"] == 1024 and k.bindings["flag"] == 1 and "junk" not in k.bindings
    assert k.bindings["HIP_RESPECT_SCHEDULE"] == 0
    k2 = lower_intent_to_hip_kernel(w.ir(), shape_bindings={"M": 16, "N": 1024}, schedule_override={"tile_m": 4})
    assert k2.bindings["HIP_RESPECT_SCHEDULE"] == 1


def test_softmax_expanded_chain_with_keepdims_forms():
    base = {"X": {"dtype": "f32", "shape": ["M", "N"]}, "Xc": {"dtype": "f32", "shape": ["M", "N"]},
            "E": {"dtype": "f32", "shape": ["M", "N"]}, "out": {"dtype": "f32", "shape": ["M", "N"]}}
    for keep, rshape in ((False, ["M"]), (True, ["M", 1])):
        ir = {"name": "sm", "tensors": dict(base, mx={"dtype": "f32", "shape": rshape}, sm={"dtype": "f32", "shape": rshape}),
              "ops": [{"op": "reduce_max", "inputs": ["X"], "output": "mx", "attrs": {"dims": [1], "keepdims": keep}},
                      {"op": "sub", "inputs": ["X", "mx"], "output": "Xc"},
                      {"op": "exp", "inputs": ["Xc"], "output": "E"},
                      {"op": "reduce_sum", "inputs": ["E"], "output": "sm", "attrs": {"dims": [1], "keepdims": keep}},
                      {"op": "div", "inputs": ["E", "sm"], "output": "out"}], "outputs": ["out"]}
        assert lower_intent_to_hip_kernel(ir, shape_bindings={"M": 4, "N": 8}).kernel_id == "ihip_softmax_rows_f32"


def test_softmax_over_wrong_axis_is_not_softmax():
    ir = softmax_inner_ir()
    ir["ops"][0]["attrs"]["axis"] = 0
    with pytest.raises(HipLoweringError):
        lower_intent_to_hip_kernel(ir, shape_bindings={"M": 4, "N": 8})


def test_trailing_alignment_is_not_mistaken_for_row_broadcast():
    """reduce_max keepdims=False declared [N] (not [M]) broadcasts along the trailing axis: not softmax."""
    ir = {"name": "notsm", "tensors": {"X": {"dtype": "f32", "shape": ["M", "N"]}, "mx": {"dtype": "f32", "shape": ["N"]},
                                       "Xc": {"dtype": "f32", "shape": ["M", "N"]}, "E": {"dtype": "f32", "shape": ["M", "N"]},
                                       "sm": {"dtype": "f32", "shape": ["N"]}, "out": {"dtype": "f32", "shape": ["M", "N"]}},
          "ops": [{"op": "reduce_max", "inputs": ["X"], "output": "mx", "attrs": {"dims": [1]}},
                  {"op": "sub", "inputs": ["X", "mx"], "output": "Xc"}, {"op": "exp", "inputs": ["Xc"], "output": "E"},
                  {"op": "reduce_sum", "inputs": ["E"], "output": "sm", "attrs": {"dims": [1]}},
                  {"op": "div", "inputs": ["E", "sm"], "output": "out"}], "outputs": ["out"]}
    with pytest.raises(HipLoweringError):
        lower_intent_to_hip_kernel(ir, shape_bindings={"M": 8, "N": 8})


def test_layernorm_chain_with_wrong_divisor_is_rejected():
    ir = WORKLOADS["layernorm"].ir()
    ir["ops"][1]["attrs"]["divisor"] = "M"
    with pytest.raises(HipLoweringError):
        lower_intent_to_hip_kernel(ir, shape_bindings={"M": 8, "N": 64})


def test_layernorm_without_stat_outputs_passes_null_statistics():
    """Statistics that are not outputs are not written: null pointers, no scratch buffers."""
    ir = WORKLOADS["layernorm"].ir()
    ir["outputs"] = ["out_ptr"]
    k = lower_intent_to_hip_kernel(ir, shape_bindings={"M": 8, "N": 64})
    assert k.call_args[4] == ("null", None) and k.call_args[5] == ("null", None)
    assert set(k.io_spec["tensors"]) == {"in_ptr", "weight_ptr", "bias_ptr", "out_ptr"}
    ir["outputs"] = ["out_ptr", "out_rstd_ptr"]
    k = lower_intent_to_hip_kernel(ir, shape_bindings={"M": 8, "N": 64})
    assert k.call_args[4] == ("null", None) and k.call_args[5] == ("tensor", "out_rstd_ptr")


def _layernorm_with_scalar_affine():
    """LN whose weight and bias are [1] tensors broadcast by numpy directly (no broadcast_in_dim)."""
    ir = WORKLOADS["layernorm"].ir()
    ir["tensors"]["weight_ptr"]["shape"] = [1]
    ir["tensors"]["bias_ptr"]["shape"] = [1]
    ops = [o for o in ir["ops"] if o["op"] != "broadcast_in_dim"]
    for o in ops:
        o["inputs"] = ["weight_ptr" if i == "w_b" else "bias_ptr" if i == "b_b" else i for i in o["inputs"]]
    ir["ops"] = ops
    for t in ("w_b", "b_b"):
        del ir["tensors"][t]
    return ir


def test_layernorm_with_scalar_weight_and_bias_is_not_the_row_kernel():
    """The kernel reads N elements of w and b; [1]-shaped ones would be read out of bounds."""
    import numpy as np

    from oracle.interpreter import execute_intent

    ir = _layernorm_with_scalar_affine()
    b = {"M": 4, "N": 64}
    rng = np.random.default_rng(0)
    inp = {"in_ptr": rng.standard_normal((4, 64)).astype(np.float32),
           "weight_ptr": np.array([1.5], np.float32), "bias_ptr": np.array([0.25], np.float32)}
    out = execute_intent(ir, inp, b)  # the IR is valid: numpy broadcasts the [1] operands
    assert out["out_ptr"].shape == (4, 64)
    with pytest.raises(HipLoweringError, match="w and b of shape"):
        lower_intent_to_hip_kernel(ir, shape_bindings=b)


def test_gelu_with_wrong_constant_is_not_gelu():
    """A chain that only looks like GELU is not given the GELU kernel; it runs as a generic program."""
    ir = WORKLOADS["gelu"].ir()
    fn = expand_macros(as_intent(ir)).to_json_dict()
    for op in fn["ops"]:
        if op["op"] == "const" and abs(op["attrs"]["value"] - 0.044715) < 1e-9:
            op["attrs"]["value"] = 0.05
    k = lower_intent_to_hip_kernel(fn, shape_bindings={"M": 4, "N": 64})
    assert k.kernel_id == "ihip_elementwise_program"
    assert any(c[0] == 2 and abs(c[5] - 0.05) < 1e-9 for c in k.call_args[0][1].code)  # the IMM carries 0.05


def test_gemm_forms_and_errors():
    b = {"M": 256, "N": 256, "K": 64}
    assert lower_intent_to_hip_kernel(matmul_bias_relu2d_ir(), shape_bindings=b).call_args[-1] == ("i32", 1)
    ir = matmul_bias_relu2d_ir()
    ir["ops"][0]["attrs"] = {"transpose_b": True}  # B declared [K, N] read as [N, K]: fine when N == K
    k = lower_intent_to_hip_kernel(ir, shape_bindings={"M": 256, "N": 64, "K": 64})
    assert k.kernel_id == "ihip_gemm_bf16_bias_relu_t" and k.call_args[-3:] == (("i32", 0), ("i32", 1), ("i32", 1))
    with pytest.raises(HipLoweringError, match="transpose_b=True"):
        lower_intent_to_hip_kernel(ir, shape_bindings=b | {"N": 128})
    f32 = matmul_bias_relu2d_ir("f32")  # the reference builder's own dtype: the fp32-MFMA kernel
    k = lower_intent_to_hip_kernel(f32, shape_bindings=b)
    assert k.kernel_id == "ihip_gemm_f32_bias_relu" and k.call_args[-4:] == (("i32", 0), ("i32", 0), ("i32", 1),
                                                                              ("i32", 0))
    mixed = matmul_bias_relu2d_ir()
    mixed["tensors"]["C"]["dtype"] = "f32"
    with pytest.raises(HipLoweringError, match="all bf16 or all f32"):
        lower_intent_to_hip_kernel(mixed, shape_bindings=b)
    # max(x, 0) is ReLU too
    ir = matmul_bias_relu2d_ir()
    ir["tensors"]["zero"] = {"dtype": "f32", "shape": []}
    ir["ops"][-1] = {"op": "max", "inputs": ["mm_b", "zero"], "output": "C"}
    ir["ops"].insert(0, {"op": "const", "inputs": [], "output": "zero", "attrs": {"value": 0.0, "dtype": "f32"}})
    assert lower_intent_to_hip_kernel(ir, shape_bindings=b).call_args[-1] == ("i32", 1)


@pytest.mark.parametrize("M,N,K,tile,path", [
    (256, 256, 64, 128, "fast"), (300, 264, 1000, 128, "fast"), (8, 8, 8, 128, "fast"), (4096, 4096, 64, 256, "fast"),
    (4096, 2048, 64, 128, "fast"), (4096, 2304, 64, 256, "fast"), (4100, 4104, 72, 256, "fast"),
    (256, 250, 64, 128, "packed"), (256, 256, 60, 128, "packed"), (65536, 16384, 40960, 256, "fast"),
    (65536, 16384, 40968, 256, "guarded"), (5000, 3001, 64, 256, "packed"), (7, 9, 3, 128, "packed"),
    (1024, 1024, 8192, 128, "split4"), (1000, 1000, 4100, 128, "packed+split4"), (128, 64, 65536, 128, "split128"),
    (1536, 1408, 8192, 128, "fast"), (1408, 1408, 1024, 128, "fast"), (64, 64, 4096, 128, "split8"),
    (512, 512, 16384, 128, "split16"), (1024, 1024, 2048, 128, "fast"),
    # skinny (M <= 128) with more than one round of 256x256 tiles: 128x128; with one round: 256x256
    (32, 131072, 4096, 128, "fast"), (128, 65792, 4096, 128, "fast"), (129, 131072, 4096, 256, "fast"),
    (64, 65536, 8192, 256, "fast"), (16, 50256, 4096, 256, "fast"),
    # one row of 256x256 tiles with 129-256 rows and more than a round of 128x128 tiles: 256x256
    (256, 32000, 4096, 256, "fast"), (200, 33024, 1024, 256, "fast"), (256, 16384, 8192, 128, "fast")])
def test_gemm_launch_descriptor_follows_the_fast_path(M, N, K, tile, path):
    """Rows 16-byte aligned (N % 8 == 0, K % 8 == 0) take the tiled kernel at any M and N (LDS:
    three paired-slice A regions and four B stages); other rows are packed into a workspace
    and then take the tiled kernel; the guarded kernel (a double-buffered pair of 64-k operand
    tiles) is left for shapes beyond the tiled kernel's limits, such as a ragged K with
    operands above 2 GiB.  All use 256x256 tiles, or 128x128 tiles when at most 128 tiles of
    256x256 (half the CUs) would be busy, or when M <= 128 and more than 256 such tiles run.  A grid of 128x128 tiles may be split along K into S
    segments (tiles x S workgroups), its f32 partials in the workspace, where the split rule
    estimates a gain: 64 tiles with K = 8192 take 4 segments, 16 tiles with K = 16384 take 16,
    one tile with K = 65536 takes 128 segments of 512; 132 tiles (1536 x 1408) would need a
    second wave to split, 121 tiles with K = 1024 and 64 tiles with K = 2048 gain too little
    over the partials' round trip.  256x256 tiles with N % 8 == 0 and K % 64 == 0 run the
    16x16x32 kernel on a persistent grid of at most one workgroup per CU (256)."""
    k = lower_intent_to_hip_kernel(matmul_bias_relu2d_ir(), shape_bindings={"M": M, "N": N, "K": K})
    S = int(path.split("split")[1]) if "split" in path else 1
    tiles = -(-M // tile) * -(-N // tile) * S
    m16 = (tile == 256 and path == "fast" and N % 8 == 0 and K % 64 == 0
           and K * 512 < 2 ** 32 and N * 128 < 2 ** 32)
    assert k.launch.grid == ((min(tiles, 256) if m16 else tiles), 1, 1)
    base = path.split("+")[0] if "+" in path else ("fast" if path.startswith("split") else path)
    assert k.launch.lds_bytes == {(256, "fast"): 163840, (128, "fast"): 81920, (256, "packed"): 163840,
                                  (128, "packed"): 81920, (256, "guarded"): 147456,
                                  (128, "guarded"): 73728}[(tile, base)]
    uses_ws = base == "packed" or S > 1
    assert (k.kernel_id == "ihip_gemm_bf16_bias_relu_ws") == uses_ws
    if uses_ws:
        assert k.call_args[-1] == ("workspace", gemm_workspace_bytes(M, N, K, False, False)) and k.call_args[-1][1] > 0
    if S > 1:
        partials = S * M * (-(-N // 4) * 4) * 4
        assert gemm_workspace_bytes(M, N, K, False, False) >= partials


@pytest.mark.parametrize("N,tb,lds,kid", [(50257, True, 163840, "ihip_gemm_bf16_bias_relu_t"),
                                          (263, True, 81920, "ihip_gemm_bf16_bias_relu_t"),
                                          (263, False, 81920, "ihip_gemm_bf16_bias_relu_ws"),
                                          (50257, False, 163840, "ihip_gemm_bf16_bias_relu_ws")])
def test_gemm_odd_n_takes_the_tiled_kernel_with_b_as_nk(N, tb, lds, kid):
    """With B given as [N, K] (transpose_b) the rows of A and B stay 16-byte aligned at any N,
    so the tiled kernel runs (C written with 2-byte stores); B as [K, N] with N % 8 != 0 is
    packed into a workspace as [N, K] first."""
    ir = matmul_bias_relu2d_ir()
    if tb:
        ir["tensors"]["B"]["shape"] = ["N", "K"]
        ir["ops"][0]["attrs"] = {"transpose_b": True}
    k = lower_intent_to_hip_kernel(ir, shape_bindings={"M": 300, "N": N, "K": 64})
    assert k.launch.lds_bytes == lds and k.kernel_id == kid


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_gemm_workspace_size_matches_the_library(ta, tb):
    """The lowering sizes the packed path's workspace by the library's rule
    (ihip_gemm_workspace_size), pinned here on shapes around every alignment case."""
    from intent_ir_amd.runtime import load_library

    lib = load_library()
    for M in (1, 7, 8, 9, 256, 1000, 4099):
        for N in (1, 8, 263, 264, 50257):
            for K in (1, 3, 8, 60, 64, 1000, 1024, 4095, 16383, 65536):
                want = lib.ihip_gemm_workspace_size(M, N, K, int(ta), int(tb))
                assert gemm_workspace_bytes(M, N, K, ta, tb) == want, (M, N, K, ta, tb)
    assert lib.ihip_gemm_workspace_size(0, 8, 3, 0, 0) == 0 == gemm_workspace_bytes(0, 8, 3, False, False)


def test_gemm_split_plan_matches_the_library():
    """The split rule and an explicit split count size the partials as the library does
    (ihip_gemm_splitk_workspace_size), and every plan covers K with segments of whole 64-k
    steps, the last one non-empty."""
    from intent_ir_amd.lowering import gemm_split_plan
    from intent_ir_amd.runtime import load_library

    lib = load_library()
    for M, N in ((1, 1), (128, 64), (1000, 1001), (1024, 1024), (1408, 1408), (1536, 1408), (4096, 4096)):
        for K in (8, 64, 520, 1024, 4100, 8192, 65536):
            for splits in (0, 1, 2, 3, 7, 64, 1025, 5000):
                S, kseg = gemm_split_plan(M, N, K, splits)
                assert (S == 1 or kseg % 64 == 0) and (S - 1) * kseg < K <= S * kseg, (M, N, K, splits, S, kseg)
                assert S <= max(1, splits) or splits == 0
                want = -(-S * M * (-(-N // 4) * 4) * 4 // 256) * 256 if S > 1 else 0
                assert lib.ihip_gemm_splitk_workspace_size(M, N, K, splits) == want, (M, N, K, splits)
    assert gemm_split_plan(1024, 1024, 8192) == (4, 2048)
    assert gemm_split_plan(4096, 4096, 8192) == (1, 8192)   # 256x256 tiles: never split
    assert gemm_split_plan(128, 64, 131072) == (256, 512)   # one tile: 256 segments fill the CUs
    assert gemm_split_plan(1000, 1000, 200) == (1, 200)     # K under two segments of 512


def test_unsupported_ops_raise():
    ir = {"name": "g", "tensors": {"x": {"dtype": "f32", "shape": ["N"]}, "i": {"dtype": "i32", "shape": ["N"]},
                                   "y": {"dtype": "f32", "shape": ["N"]}},
          "ops": [{"op": "gather", "inputs": ["x", "i"], "output": "y"}], "outputs": ["y"]}
    with pytest.raises(HipLoweringError, match="unsupported"):
        lower_intent_to_hip_kernel(ir, shape_bindings={"N": 4})


# ---------------------------------------------------------------- C-ABI library
def _header_symbols():
    text = (ROOT / "include" / "intentir_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(ihip_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_every_runtime_signature():
    assert _header_symbols() == sorted(SIGNATURES)


def test_library_exports_every_declared_symbol():
    if not LIB_PATH.exists():
        pytest.fail("libintentir_hip.so is not built: run python -m intent_ir_amd.build")
    lib = ctypes.CDLL(str(LIB_PATH))
    for sym in _header_symbols():
        assert hasattr(lib, sym), sym
    lib.ihip_abi_version.restype = ctypes.c_int
    assert lib.ihip_abi_version() == 3
    lib.ihip_last_error.restype = ctypes.c_char_p
    # the message is per thread and survives until the next call: other tests in this process
    # may have left one, and a successful call (an empty softmax needs no device) clears it
    lib.ihip_softmax_rows_f32.restype = ctypes.c_int
    lib.ihip_softmax_rows_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_void_p]
    assert lib.ihip_softmax_rows_f32(None, None, 0, 0, None) == 0
    assert lib.ihip_last_error() == b""


def test_library_rejects_bad_arguments_without_a_device():
    """Argument checks run on the host before any HIP call: no GPU needed to see them."""
    from intent_ir_amd.runtime import load_library

    lib = load_library()
    st = lib.ihip_softmax_rows_f32(None, None, -1, 4, None)
    assert st == -1 and b"invalid shape" in lib.ihip_last_error()
    st = lib.ihip_reduce_rows_f32(None, None, 4, 4, 7, None)
    assert st == -1 and b"unknown kind" in lib.ihip_last_error()
    st = lib.ihip_gemm_bf16_bias_relu(None, None, None, None, 2, 2, 2, 1, None)
    assert st == -1 and b"null" in lib.ihip_last_error()
    st = lib.ihip_reduce_any_rows_f32(None, None, 1 << 62, 1 << 62, 0.0, None)
    assert st == -1  # element count overflows int64
    st = lib.ihip_softmax_rows_f32_ex(None, None, 0, 8, 3, None)
    assert st == -1 and b"rows_per_wg 3" in lib.ihip_last_error()
    st = lib.ihip_gemm_bf16_bias_relu_ex(None, None, None, None, 0, 0, 0, 0, 0, 1, 64, None)
    assert st == -1 and b"tile 64" in lib.ihip_last_error()


@pytest.mark.parametrize("M,N,grid,block,lds", [
    (8192, 4099, 1024, 256, 16384), (3, 1029, 8, 256, 16384), (64, 7, 1, 256, 16592), (1000, 100, 16, 256, 17552), (1000, 33, 8, 256, 10896),
    (1000, 256, 63, 256, 0), (1000, 64, 16, 256, 0), (1000, 257, 256, 256, 16384),
    (8192, 4104, 1024, 1024, 128), (8192, 8191, 8192, 128, 16), (5, 65537, 5, 1024, 128), (5, 65545, 5, 256, 16)])
def test_layernorm_launch_descriptor(M, N, grid, block, lds):
    """Short rows (up to 256 halves) run several per wave: N / 8 lanes per row rounded up to a
    power of two and two rows per group for aligned rows; for the others one lane per 8 elements (5 when N <= 5 lanes' worth),
    four rows per group and the workgroup's rows staged in LDS (with w and b as f32).  Rows not 16-byte
    aligned up to N = 4096 + 7 run as 8 row classes of workgroups with w and b staged per class
    (grid 8 x min(128, ceil(ceil(M / 8) / 4))); longer ones one row per workgroup of 1-16
    waves; beyond 65536 + 7 a 256- or 1024-thread workgroup per row."""
    k = lower_intent_to_hip_kernel(WORKLOADS["layernorm"].ir(), shape_bindings={"M": M, "N": N})
    assert (k.launch.grid[0], k.launch.block[0], k.launch.lds_bytes) == (grid, block, lds)


@pytest.mark.parametrize("dt,M,N,grid,block", [
    ("f32", 1000, 4096, 1000, 64), ("f32", 1000, 16, 8, 256), ("f32", 1000, 256, 125, 256), ("f32", 1000, 260, 1000, 64),
    ("bool", 1000, 64, 16, 256), ("bool", 1000, 1025, 125, 256), ("bool", 1000, 2000, 1000, 64)])
def test_reduce_any_launch_descriptor(dt, M, N, grid, block):
    """Rows of at most 64 16-byte vectors run several per wave (g lanes per row, about two vectors
    each, at least 2 for f32 and 4 for bool, whose head and tail hold up to 15 bytes); longer rows a
    one-wave workgroup each."""
    ir = {"name": "any_rows", "tensors": {"x": {"dtype": dt, "shape": ["M", "N"]}, "out": {"dtype": "bool", "shape": ["M"]}},
          "ops": [{"op": "reduce_any", "inputs": ["x"], "output": "out", "attrs": {"dims": [1]}}], "outputs": ["out"]}
    k = lower_intent_to_hip_kernel(ir, shape_bindings={"M": M, "N": N})
    assert (k.launch.grid[0], k.launch.block[0]) == (grid, block)


@pytest.mark.parametrize("M,N,grid,block,lds", [
    (1000, 31, 16, 256, 8336), (1000, 127, 63, 256, 8336), (5, 1, 1, 256, 8336), (1000, 32, 32, 256, 0),
    (1000, 128, 125, 256, 0), (1000, 129, 1000, 64, 0),
    (1000, 200, 250, 128, 0), (1000, 256, 250, 128, 0), (1000, 512, 500, 128, 0), (1000, 768, 500, 128, 0),
    (1000, 1024, 125, 256, 0), (1000, 2048, 250, 256, 0), (1000, 4096, 250, 256, 0),
    (1024, 128256, 1024, 1024, 163840), (1000, 65540, 1000, 1024, 163840), (1000, 139232, 1000, 1024, 163840),
    (1000, 139236, 1000, 1024, 128), (1000, 128255, 1000, 1024, 128)])
def test_softmax_short_row_launch_descriptor(M, N, grid, block, lds):
    """Short rows (up to 128 floats) run several per wave: N / 4 lanes per row rounded up to a
    power of two for aligned rows; for the others one lane per 4 elements, two rows per group and
    the workgroup's rows staged in LDS (8 KiB + 144 B: the run's offset in its 128-byte line,
    one vector of slack).  Longer rows not 16-byte aligned take a
    wave per row.  Vector rows up to 4096 floats: two waves of two rows for N <= 256, two waves of
    one row up to 1020, four waves of two rows at 1024, four waves of one row beyond (the
    library's automatic choice, from kernel_runner --sweep softmax-rows).  Vector rows longer than 65536 floats, up to 139232, are held on the CU (all
    160 KiB of LDS); longer or unaligned ones run the two-pass kernel (128 B of partials)."""
    k = lower_intent_to_hip_kernel(WORKLOADS["softmax"].ir(), shape_bindings={"M": M, "N": N})
    assert (k.launch.grid[0], k.launch.block[0], k.launch.lds_bytes) == (grid, block, lds)
