"""Row-split reduce_sum / reduce_max on the GPU (ihip_reduce_rows_f32_ws).

Parity with the oracle (restated verify/interpreter.py:478-500): maxima bit-exact; sums
within an f32 summation bound, |out - sum64| <= 1e-6 * sum|x| + 1e-5 * |sum64| (the split
changes the f32 rounding order, not the value being computed).  Also: the split and unsplit
forms agree (maxima bit-identical), special values (NaN, inf, -0.0 rows) behave as numpy,
and rows at every 4-byte alignment (N % 4 != 0) split correctly around their head and tail.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from intent_ir_amd import lower_intent_to_hip_kernel, run_lowered
from intent_ir_amd.lowering import reduce_rows_segments
from oracle.interpreter import execute_intent

pytestmark = pytest.mark.gpu


def _ir(op):
    return {"name": f"row_{op}", "tensors": {"x": {"dtype": "f32", "shape": ["M", "N"]},
                                             "out": {"dtype": "f32", "shape": ["M"]}},
            "ops": [{"op": op, "inputs": ["x"], "output": "out", "attrs": {"dims": [1]}}], "outputs": ["out"]}


def _check_sum(out, x):
    ref = x.astype(np.float64).sum(axis=1)
    bound = 1e-6 * np.abs(x).astype(np.float64).sum(axis=1) + 1e-5 * np.abs(ref)
    err = np.abs(out.astype(np.float64) - ref)
    assert (err <= bound).all(), f"max err {err.max():.3g} over bound {bound[np.argmax(err - bound)]:.3g}"


@pytest.mark.parametrize("M,N", [(64, 1 << 20), (1, 1 << 22), (3, 1048573), (255, 65536), (17, 65537), (5, 262147)])
def test_split_reductions_match_the_oracle(hip, M, N):
    assert reduce_rows_segments(M, N) > 1
    x = np.random.default_rng(M * 13 + N).standard_normal((M, N)).astype(np.float32)
    for op in ("reduce_sum", "reduce_max"):
        k = lower_intent_to_hip_kernel(_ir(op), shape_bindings={"M": M, "N": N})
        print(f"[case] {k.kernel_id} {op} M={M} N={N} S={reduce_rows_segments(M, N)}", flush=True)
        assert k.kernel_id == "ihip_reduce_rows_f32_ws"
        out = run_lowered(k, {"x": x})["out"]
        if op == "reduce_max":
            np.testing.assert_array_equal(out, execute_intent(_ir(op), {"x": x}, {"M": M, "N": N})["out"])
        else:
            _check_sum(out, x)


@pytest.mark.parametrize("M,N", [(64, 1 << 20), (7, 1048577)])
def test_split_and_unsplit_forms_agree(hip, M, N):
    """Through the C-ABI: no workspace (rows unsplit) against a workspace (rows split)."""
    import torch

    x = torch.randn((M, N), device="cuda")
    x[0, N // 3] = float("nan")
    x[1, :] = -0.0
    x[2, 5] = float("inf")
    x[3, 7], x[3, N - 1] = float("inf"), float("-inf")
    ws_bytes = hip.ihip_reduce_rows_f32_workspace_size(M, N)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    xh = x.cpu().numpy()
    for kind in (0, 1):
        a = torch.empty(M, device="cuda")
        b = torch.empty(M, device="cuda")
        print(f"[case] reduce_rows_f32 kind={kind} M={M} N={N} ws={ws_bytes}", flush=True)
        assert hip.ihip_reduce_rows_f32(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(a.data_ptr()), M, N, kind, s) == 0
        assert hip.ihip_reduce_rows_f32_ws(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(b.data_ptr()), M, N, kind,
                                           ctypes.c_void_p(ws.data_ptr()), ws_bytes, s) == 0
        torch.cuda.synchronize()
        ah, bh = a.cpu().numpy(), b.cpu().numpy()
        ref = xh.sum(axis=1) if kind == 0 else xh.max(axis=1)
        np.testing.assert_array_equal(np.isnan(bh), np.isnan(ref))
        if kind == 1:
            np.testing.assert_array_equal(ah, bh)
            np.testing.assert_array_equal(bh, ref)
        else:
            assert bh[1] == 0.0 and not np.signbit(bh[1]), "a row of -0.0 sums to +0.0, as numpy"
            assert bh[2] == np.inf and np.isnan(bh[3])
            fin = np.isfinite(ref)
            _check_sum(bh[fin], xh[fin])
            _check_sum(ah[fin], xh[fin])
