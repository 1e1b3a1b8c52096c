"""Split long-row softmax: host-side plan and argument checks (CPU only).

Rows longer than 65536 floats are split over S workgroups per row, with two floats of
partials per segment in a caller-owned workspace (ihip_softmax_rows_f32_ws).  The lowering
mirrors the library's plan to size the workspace; these tests pin the two together without a
device."""

from __future__ import annotations

import ctypes

import pytest

from intent_ir_amd import lower_intent_to_hip_kernel
from intent_ir_amd.configs import WORKLOADS
from intent_ir_amd.lowering import softmax_split_plan
from intent_ir_amd.runtime import load_library

SHAPES = [(m, n) for m in (0, 1, 2, 3, 17, 31, 32, 33, 64, 191, 192, 255, 256, 257, 300, 416, 417, 512, 513, 639,
                          640, 1000, 4096)
          for n in (0, 1, 4096, 65536, 65537, 65540, 100003, 128256, 151936, 262144, 1 << 20, 1048576 + 4, 1 << 22,
                    1 << 30)]


def test_python_split_plan_matches_the_library():
    lib = load_library()
    for M, N in SHAPES:
        s, vpl = softmax_split_plan(M, N)
        assert (s == 0) == (vpl == 0) and vpl in (0, 4, 8, 16) and 0 <= s <= 1 << 20
        if s:
            # the segments cover the longest body a row can have, and no segment is empty
            assert s * 256 * vpl >= N // 4 > (s - 1) * 256 * vpl
        assert lib.ihip_softmax_rows_f32_workspace_size(M, N) == 8 * M * s, (M, N)


@pytest.mark.parametrize("M,N,S,vpl", [(64, 128256, 32, 4), (1, 128256, 32, 4), (16, 151936, 38, 4),
                                       (32, 151936, 38, 4), (4096, 65540, 0, 0), (2, 1 << 20, 256, 4),
                                       (191, 128256, 32, 4), (192, 128256, 0, 0), (256, 128256, 0, 0),
                                       (257, 100000, 25, 4), (416, 128256, 16, 8), (417, 128256, 0, 0),
                                       (512, 128256, 0, 0), (639, 70000, 9, 8), (640, 70000, 0, 0),
                                       (300, 262144, 16, 16),
                                       (1, 1048580, 257, 4), (1, 1 << 26, 4096, 16), (100, 65536, 0, 0),
                                       (1 << 20, 1 << 30, 0, 0)])
def test_lowering_selects_the_split_form(M, N, S, vpl):
    assert softmax_split_plan(M, N) == (S, vpl)
    k = lower_intent_to_hip_kernel(WORKLOADS["softmax"].ir(), shape_bindings={"M": M, "N": N})
    if S:
        assert k.kernel_id == "ihip_softmax_rows_f32_ws"
        assert k.call_args[-1] == ("workspace", 8 * M * S) and k.launch.grid[0] == M * S
    else:
        assert k.kernel_id == "ihip_softmax_rows_f32"


def test_workspace_argument_checks_without_a_device():
    lib = load_library()
    p = ctypes.c_void_p(256)  # never dereferenced: the checks return before any HIP call
    need = lib.ihip_softmax_rows_f32_workspace_size(64, 128256)
    assert need == 8 * 64 * 32
    st = lib.ihip_softmax_rows_f32_ws(p, p, 64, 128256, p, need - 8, None)
    assert st == -1 and b"needs 16384" in lib.ihip_last_error()
    st = lib.ihip_softmax_rows_f32_ws(p, p, 64, 128256, ctypes.c_void_p(260), need, None)
    assert st == -1 and b"aligned" in lib.ihip_last_error()
    st = lib.ihip_softmax_rows_f32_ws(p, p, 64, 128256, None, 64, None)
    assert st == -1 and b"null pointer" in lib.ihip_last_error()
    st = lib.ihip_softmax_rows_f32_ws(p, p, -1, 128256, p, need, None)
    assert st == -1 and b"invalid shape" in lib.ihip_last_error()
    st = lib.ihip_softmax_rows_f32_ws(p, p, 64, 128256, p, -8, None)
    assert st == -1 and b"negative" in lib.ihip_last_error()
    assert lib.ihip_softmax_rows_f32_workspace_size(-1, 128256) == 0
    assert lib.ihip_softmax_rows_f32_workspace_size(1 << 40, 1 << 40) == 0
