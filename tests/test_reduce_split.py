"""Row-split reduce_sum / reduce_max: host-side plan and argument checks (CPU only).

Rows too few to fill the GPU (M < 256) and long enough are split over S workgroups per
row; partials go to a caller-owned workspace (ihip_reduce_rows_f32_ws).  The lowering
mirrors the library's split rule to size the workspace; these tests pin the two
together without a device."""

from __future__ import annotations

import ctypes

import pytest

from intent_ir_amd import lower_intent_to_hip_kernel
from intent_ir_amd.lowering import reduce_rows_segments
from intent_ir_amd.runtime import load_library

SHAPES = [(m, n) for m in (0, 1, 2, 3, 17, 63, 64, 100, 255, 256, 1000)
          for n in (0, 1, 7, 4096, 16384, 32767, 32768, 65536, 65537, 262144, 1 << 20, 1048573, 1 << 22)]


def _ir(op):
    return {"name": f"row_{op}", "tensors": {"x": {"dtype": "f32", "shape": ["M", "N"]},
                                             "out": {"dtype": "f32", "shape": ["M"]}},
            "ops": [{"op": op, "inputs": ["x"], "output": "out", "attrs": {"dims": [1]}}], "outputs": ["out"]}


def test_python_split_rule_matches_the_library():
    lib = load_library()
    for M, N in SHAPES:
        s = reduce_rows_segments(M, N)
        assert 1 <= s <= 64
        assert lib.ihip_reduce_rows_f32_workspace_size(M, N) == (4 * M * s if s > 1 else 0), (M, N)


@pytest.mark.parametrize("M,N,S", [(64, 1 << 20, 8), (1, 1 << 22, 64), (3, 1048573, 63), (255, 65536, 3),
                                   (17, 65536, 4), (256, 1 << 20, 1), (64, 4096, 1)])
def test_lowering_selects_the_split_form(M, N, S):
    for op in ("reduce_sum", "reduce_max"):
        k = lower_intent_to_hip_kernel(_ir(op), shape_bindings={"M": M, "N": N})
        assert reduce_rows_segments(M, N) == S
        if S > 1:
            assert k.kernel_id == "ihip_reduce_rows_f32_ws"
            assert k.call_args[-1] == ("workspace", 4 * M * S) and k.launch.grid[0] == M * S
        else:
            assert k.kernel_id == "ihip_reduce_rows_f32"


@pytest.mark.parametrize("M,N,grid", [(1000, 4, 4), (1000, 16, 8), (1000, 32, 16), (1000, 33, 16), (1000, 64, 32),
                                      (1000, 512, 125), (1000, 513, 125), (1000, 516, 1000)])
def test_short_row_launch_descriptor(M, N, grid):
    """Rows of at most 128 16-byte vectors run several per wave: about two vectors per lane (four
    at 65-128), g lanes per row a power of two up to 32, 256 threads per workgroup; longer rows a
    wave each."""
    for op in ("reduce_sum", "reduce_max"):
        k = lower_intent_to_hip_kernel(_ir(op), shape_bindings={"M": M, "N": N})
        assert k.launch.grid[0] == grid, (op, M, N)


def test_workspace_argument_checks_without_a_device():
    lib = load_library()
    p = ctypes.c_void_p(256)  # never dereferenced: the checks return before any HIP call
    st = lib.ihip_reduce_rows_f32_ws(p, p, 64, 1 << 20, 0, p, 8, None)
    assert st == -1 and b"needs 2048" in lib.ihip_last_error()
    st = lib.ihip_reduce_rows_f32_ws(p, p, 64, 1 << 20, 0, ctypes.c_void_p(258), 4096, None)
    assert st == -1 and b"aligned" in lib.ihip_last_error()
    st = lib.ihip_reduce_rows_f32_ws(p, p, 64, 1 << 20, 5, p, 4096, None)
    assert st == -1 and b"unknown kind" in lib.ihip_last_error()
