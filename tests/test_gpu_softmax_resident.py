"""Vocabulary-width softmax rows held on the CU (rows.hip softmax_rows_f32_resident).

Vector rows (N % 4 == 0, 16-byte aligned x and y) of 65536 < N <= 139232 floats run one
1024-thread workgroup per row with the row in registers (24 vectors per lane) and, past
98304 floats, the rest in LDS, filled by direct-to-LDS loads; x is read from HBM once.
These tests call the C-ABI without a workspace, so that every row count takes that kernel,
and check it against the oracle (restated verify/interpreter.py:501-506) at the softmax
contract, rtol 1e-5 / atol 1e-7, at the register/LDS boundaries (no LDS part, one LDS vector,
a partial last wave of copies, a full 160 KiB), with special values in either part, against
the two-pass kernel (y one float off x's alignment), and through the statistics entry.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from intent_ir_amd.configs import WORKLOADS
from intent_ir_amd.lowering import SOFTMAX_RESIDENT_MAX_VECS
from oracle.compare import compare_outputs
from oracle.interpreter import execute_intent

pytestmark = pytest.mark.gpu

TOL = {"atol": 1e-7, "rtol": 1e-5}
REG_FLOATS = 4 * 24 * 1024          # the register part of a row
MAX_FLOATS = 4 * SOFTMAX_RESIDENT_MAX_VECS


def _check(out, ref, what):
    fin = ~np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(out), np.isnan(ref), err_msg=what)
    d = compare_outputs({"y": np.where(fin, out, 0)}, {"y": np.where(fin, ref, 0)}, ["y"], TOL)
    assert d.ok, f"{what}: {d.summary}"


def _ref(x):
    M, N = x.shape
    with np.errstate(invalid="ignore", over="ignore"):
        return execute_intent(WORKLOADS["softmax"].ir(), {"input_ptr": x}, {"M": M, "N": N})["output_ptr"]


def _softmax(hip, xh, yoff=0):
    """ihip_softmax_rows_f32 (no workspace) on a copy of xh; y at a float offset `yoff` from a
    256-byte aligned base, guarded by sentinels on both sides."""
    import torch

    M, N = xh.shape
    x = torch.from_numpy(np.ascontiguousarray(xh).ravel()).cuda()
    y = torch.full((M * N + yoff + 8,), 7.0, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = hip.ihip_softmax_rows_f32(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr() + 4 * yoff), M, N, s)
    assert st == 0, hip.ihip_last_error()
    torch.cuda.synchronize()
    yh = y.cpu().numpy()
    assert (yh[:yoff] == 7.0).all() and (yh[yoff + M * N:] == 7.0).all()  # nothing written outside y
    return yh[yoff:yoff + M * N].reshape(M, N)


@pytest.mark.parametrize("N", [65540, REG_FLOATS - 4, REG_FLOATS, REG_FLOATS + 4, REG_FLOATS + 256, 128256, 131072,
                               MAX_FLOATS - 256, MAX_FLOATS])
def test_resident_softmax_matches_the_oracle(hip, N):
    M = 5
    x = (np.random.default_rng(N).standard_normal((M, N)) * 3.0).astype(np.float32)
    x[1, N - 1] = 40.0       # a dominant logit in the row's last vector (the LDS part when there is one)
    x[2, 3] = 40.0           # ... and in its first
    print(f"[case] softmax resident M={M} N={N} lds_vectors={max(0, N // 4 - REG_FLOATS // 4)}", flush=True)
    out = _softmax(hip, x)
    _check(out, _ref(x), f"N={N}")
    np.testing.assert_allclose(out.astype(np.float64).sum(axis=1), 1.0, rtol=0, atol=1e-5)


@pytest.mark.parametrize("N", [REG_FLOATS - 4, 128256, MAX_FLOATS])
def test_resident_softmax_special_values(hip, N):
    """NaN and +inf rows come out all NaN, an all -inf row NaN, masked entries exactly 0, in the
    register part and in the LDS part alike."""
    M = 8
    rng = np.random.default_rng(N + 1)
    x = (rng.standard_normal((M, N)) * 4.0).astype(np.float32)
    x[0, N // 5] = np.nan                  # NaN in the register part
    x[1, N - 3] = np.nan                   # NaN in the last vector
    x[2, N - 2] = np.inf                   # +inf: inf - inf, the whole row NaN
    x[3, :] = -np.inf                      # everything masked: NaN, as numpy
    x[4, : 3 * N // 4] = -np.inf           # the register part masked
    x[5, REG_FLOATS // 2:] = -np.inf       # the LDS part masked
    x[6, rng.random(N) < 0.3] = -np.inf    # scattered masks
    x[7, 7] = np.float32(-3.0e38)          # finite but beyond exp's range after the max shift
    print(f"[case] softmax resident special values N={N}", flush=True)
    out = _softmax(hip, x)
    ref = _ref(x)
    _check(out, ref, f"special N={N}")
    assert np.isnan(out[[0, 1, 2, 3]]).all() and not np.isnan(out[4:]).any()
    assert (out[np.isneginf(x) & ~np.isnan(ref)] == 0.0).all()


@pytest.mark.parametrize("M,N", [(300, 128256), (257, 100000), (64, MAX_FLOATS)])
def test_resident_softmax_many_rows_against_two_pass_kernel(hip, M, N):
    """Many workgroups: the resident kernel against the oracle and against the two-pass kernel
    (y one float off x's alignment takes it), which differs only in the sum's rounding order."""
    x = (np.random.default_rng(M + N).standard_normal((M, N)) * 2.0).astype(np.float32)
    x[np.random.default_rng(M).random((M, N)) < 0.01] = 30.0
    print(f"[case] softmax resident M={M} N={N} against the two-pass kernel", flush=True)
    a = _softmax(hip, x)
    b = _softmax(hip, x, yoff=1)
    _check(a, _ref(x), f"M={M} N={N}")
    _check(a, b, f"resident against two-pass M={M} N={N}")
    np.testing.assert_array_equal(a, _softmax(hip, x))  # repeats bit for bit


def test_resident_softmax_statistics(hip):
    """ihip_softmax_rows_f32_stats without a workspace: the row max exactly, the sum of
    exp(x - max) at the softmax tolerance."""
    import torch

    M, N = 7, 128256
    rng = np.random.default_rng(11)
    xh = (rng.standard_normal((M, N)) * 2.0).astype(np.float32)
    xh[3, N - 10] = 50.0
    x = torch.from_numpy(xh.ravel()).cuda()
    y = torch.empty(M * N, device="cuda")
    mx = torch.empty(M, device="cuda")
    sm = torch.empty(M, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"[case] softmax resident statistics M={M} N={N}", flush=True)
    st = hip.ihip_softmax_rows_f32_stats(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()),
                                         ctypes.c_void_p(mx.data_ptr()), ctypes.c_void_p(sm.data_ptr()), M, N,
                                         None, 0, s)
    assert st == 0, hip.ihip_last_error()
    torch.cuda.synchronize()
    ref_max = xh.max(axis=1)
    ref_sum = np.exp((xh - ref_max[:, None]).astype(np.float64)).sum(axis=1)
    np.testing.assert_array_equal(mx.cpu().numpy(), ref_max)
    np.testing.assert_allclose(sm.cpu().numpy(), ref_sum, rtol=1e-5)
    _check(y.cpu().numpy().reshape(M, N), _ref(xh), "stats entry")
