"""Split long-row softmax on the GPU (ihip_softmax_rows_f32_ws).

Parity with the oracle (restated verify/interpreter.py:501-506) at the softmax contract,
rtol 1e-5 / atol 1e-7: the split changes only the rounding order of the row's sum (each
segment's sum is rescaled by exp(m_j - max) before the segments are added).  Also: the split
and the workgroup-per-row form (no workspace) agree within the same tolerance, results repeat
bit for bit, special values behave as numpy, and rows at every 4-byte alignment split around
their head and tail (or, with x and y at different offsets modulo 16 bytes, take the
workgroup-per-row kernel).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from intent_ir_amd import lower_intent_to_hip_kernel, run_lowered
from intent_ir_amd.configs import WORKLOADS
from intent_ir_amd.lowering import softmax_split_plan
from oracle.compare import compare_outputs
from oracle.interpreter import execute_intent

pytestmark = pytest.mark.gpu

TOL = {"atol": 1e-7, "rtol": 1e-5}


def _check(out, ref, what):
    d = compare_outputs({"y": out}, {"y": ref}, ["y"], TOL)
    assert d.ok, f"{what}: {d.summary}"


@pytest.mark.parametrize("M,N", [(1, 65540), (3, 128256), (64, 151936), (257, 100000), (5, 262144),
                                 (2, 1 << 20), (4, 65537), (3, 100003), (1, 1048580), (1, 1 << 24),
                                 (512, 65540), (448, 100003)])
def test_split_softmax_matches_the_oracle(hip, M, N):
    w = WORKLOADS["softmax"]
    b = {"M": M, "N": N}
    x = (np.random.default_rng(M * 7 + N).standard_normal((M, N)) * 3.0).astype(np.float32)
    k = lower_intent_to_hip_kernel(w.ir(), shape_bindings=b)
    print(f"[case] {k.kernel_id} M={M} N={N} plan={softmax_split_plan(M, N)}", flush=True)
    assert k.kernel_id == ("ihip_softmax_rows_f32_ws" if softmax_split_plan(M, N)[0] else "ihip_softmax_rows_f32")
    out = run_lowered(k, {"input_ptr": x})["output_ptr"]
    ref = execute_intent(w.ir(), {"input_ptr": x}, b)["output_ptr"]
    _check(out, ref, f"softmax M={M} N={N}")
    np.testing.assert_allclose(out.astype(np.float64).sum(axis=1), 1.0, rtol=0, atol=1e-5)


def _run(hip, x, y, M, N, ws=None, off=(0, 0)):
    import torch

    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    xp = ctypes.c_void_p(x.data_ptr() + 4 * off[0])
    yp = ctypes.c_void_p(y.data_ptr() + 4 * off[1])
    if ws is None:
        st = hip.ihip_softmax_rows_f32(xp, yp, M, N, s)
    else:
        st = hip.ihip_softmax_rows_f32_ws(xp, yp, M, N, ctypes.c_void_p(ws.data_ptr()), ws.numel(), s)
    assert st == 0, hip.ihip_last_error()
    torch.cuda.synchronize()
    return y.cpu().numpy()[off[1]:off[1] + M * N].reshape(M, N)


@pytest.mark.parametrize("M,N", [(8, 151936), (6, 131073)])
def test_split_and_unsplit_forms_agree(hip, M, N):
    """Through the C-ABI: no workspace (a workgroup per row, two passes; 16-byte loads, and
    4-byte loads with y one float off x's alignment) against the split, with special values
    in the rows; the split repeats bit for bit."""
    import torch

    rng = np.random.default_rng(N)
    xh = (rng.standard_normal((M, N)) * 4.0).astype(np.float32)
    xh[0, N // 3] = np.nan                 # NaN: the whole row NaN
    xh[1, 17] = np.inf                     # +inf: inf - inf, the whole row NaN
    xh[2, : 3 * N // 4] = -np.inf          # whole segments masked: they add 0
    xh[3, :] = -np.inf                     # everything masked: NaN, as numpy
    xh[4, N - 1] = 80.0                    # one dominant logit in the last segment
    x = torch.from_numpy(xh.ravel()).cuda()
    ws = torch.empty(hip.ihip_softmax_rows_f32_workspace_size(M, N), dtype=torch.uint8, device="cuda")
    assert ws.numel() > 0
    y = torch.empty(M * N, device="cuda")
    print(f"[case] softmax split vs unsplit M={M} N={N} ws={ws.numel()}", flush=True)
    a = _run(hip, x, y, M, N)
    a4 = _run(hip, x, torch.empty(M * N + 1, device="cuda"), M, N, off=(0, 1))
    b1 = _run(hip, x, y, M, N, ws)
    b2 = _run(hip, x, y, M, N, ws)
    np.testing.assert_array_equal(b1, b2)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = execute_intent(WORKLOADS["softmax"].ir(), {"input_ptr": xh}, {"M": M, "N": N})["output_ptr"]
    for got in (a, a4, b1):
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
        assert (got[2, : 3 * N // 4] == 0.0).all()
    assert np.isnan(b1[[0, 1, 3]]).all() and not np.isnan(b1[[2, 4, 5]]).any()
    assert (b1[2, : 3 * N // 4] == 0.0).all()
    fin = ~np.isnan(ref)
    _check(np.where(fin, b1, 0), np.where(fin, ref, 0), "split")
    _check(np.where(fin, b1, 0), np.where(fin, a, 0), "split against unsplit")
    _check(np.where(fin, a4, 0), np.where(fin, ref, 0), "unsplit, 4-byte loads")


@pytest.mark.parametrize("N", [65539, 100003, 131072])
@pytest.mark.parametrize("ox,oy", [(1, 1), (2, 2), (3, 3), (0, 0), (1, 2)])
def test_split_at_every_alignment(hip, N, ox, oy):
    """x and y at float offsets (ox, oy) from 256-byte aligned bases: equal offsets modulo 4
    split every row around its head and tail; others take the workgroup-per-row kernel."""
    import torch

    M = 5
    xh = np.random.default_rng(N + 10 * ox + oy).standard_normal(M * N + 8).astype(np.float32)
    x = torch.from_numpy(xh).cuda()
    y = torch.full((M * N + 8,), 7.0, device="cuda")
    ws = torch.empty(hip.ihip_softmax_rows_f32_workspace_size(M, N), dtype=torch.uint8, device="cuda")
    print(f"[case] softmax split N={N} offsets x={ox} y={oy}", flush=True)
    got = _run(hip, x, y, M, N, ws, (ox, oy))
    xs = xh[ox:ox + M * N].reshape(M, N)
    ref = execute_intent(WORKLOADS["softmax"].ir(), {"input_ptr": xs}, {"M": M, "N": N})["output_ptr"]
    _check(got, ref, f"offsets {ox},{oy}")
    yh = y.cpu().numpy()
    assert (yh[:oy] == 7.0).all() and (yh[oy + M * N:] == 7.0).all()  # nothing written outside y
