"""gather2d on the GPU (ihip_gather2d_f32), bit for bit.

In range, against the oracle's gather (numpy fancy indexing, restated verify/interpreter.py:284-291);
out of range (negative indices included), against the rule of the reference's own test
(tests/backends/cuda/test_cuda_backend_smoke.py:318-324): other_value.  Also: shapes that are
not a multiple of the 4-element vector, index and output arrays off 16-byte alignment (the
element-wise form), an empty inp, NaN and infinity carried through bitwise, and L = 0."""

from __future__ import annotations

import copy
import ctypes

import numpy as np
import pytest

from intent_ir_amd import lower_intent_to_hip_kernel, run_lowered
from oracle.interpreter import execute_intent

from test_gather import GATHER_IR

pytestmark = pytest.mark.gpu


def _rule(A, row, col, other):
    """The reference test's expectation, element by element (vectorised)."""
    M, N = A.shape
    ok = (row >= 0) & (row < M) & (col >= 0) & (col < N)
    out = np.full(row.shape, other, dtype=np.float32)
    out[ok] = A[row[ok], col[ok]]
    return out


def test_reference_case_mixed_in_and_out_of_range(hip):
    """The reference's test case: M, N, L = 7, 9, 32, indices in [-2, M + 2) and [-2, N + 2)."""
    M, N, L = 7, 9, 32
    rng = np.random.default_rng(0)
    A = rng.standard_normal((M, N), dtype=np.float32)
    row = rng.integers(-2, M + 2, size=(L,), dtype=np.int32)
    col = rng.integers(-2, N + 2, size=(L,), dtype=np.int32)
    k = lower_intent_to_hip_kernel(GATHER_IR, shape_bindings={"M": M, "N": N, "L": L})
    print(f"[case] {k.kernel_id} M={M} N={N} L={L}", flush=True)
    got = run_lowered(k, {"A": A, "row": row, "col": col})["Out"]
    np.testing.assert_array_equal(got, _rule(A, row, col, -1.0))


@pytest.mark.parametrize("M,N,L,frac_out", [(4096, 8192, 1 << 22, 0.0), (4096, 8192, (1 << 20) + 3, 0.1),
                                            (1, 1, 1001, 0.5), (300, 70000, 4099, 0.0)])
def test_gather_matches_the_oracle(hip, M, N, L, frac_out):
    rng = np.random.default_rng(M + N + L)
    A = rng.standard_normal((M, N), dtype=np.float32)
    row = rng.integers(0, M, size=(L,), dtype=np.int32)
    col = rng.integers(0, N, size=(L,), dtype=np.int32)
    bad = rng.random(L) < frac_out  # out of range: col = N or INT32_MAX, and half of those rows negative
    neg = bad & (rng.random(L) < 0.5)
    row[neg] = -rng.integers(1, 1 << 30, size=int(neg.sum()), dtype=np.int32)
    col[bad] = np.where(rng.random(int(bad.sum())) < 0.5, N, np.iinfo(np.int32).max)
    b = {"M": M, "N": N, "L": L}
    k = lower_intent_to_hip_kernel(GATHER_IR, shape_bindings=b)
    print(f"[case] {k.kernel_id} M={M} N={N} L={L} out-of-range {int(bad.sum())}", flush=True)
    got = run_lowered(k, {"A": A, "row": row, "col": col})["Out"]
    ok = ~bad
    ref = execute_intent(GATHER_IR, {"A": A, "row": row[ok], "col": col[ok]}, dict(b, L=int(ok.sum())))["Out"]
    np.testing.assert_array_equal(got[ok], ref)
    assert (got[bad] == -1.0).all()


@pytest.mark.parametrize("L", [1, 3, 4, 5, 1027])
@pytest.mark.parametrize("off", [0, 1, 2, 3])
def test_gather_at_every_alignment(hip, L, off):
    """Index and output arrays off (in elements) from 256-byte aligned bases: 0 takes the
    16-byte form (and a scalar tail when L % 4 != 0), the others the element-wise one; NaN,
    infinities and -0.0 in inp come out bit for bit; nothing is written outside out."""
    import torch

    M, N = 33, 65
    rng = np.random.default_rng(L * 4 + off)
    A = rng.standard_normal((M, N), dtype=np.float32)
    A[0, :4] = [np.nan, np.inf, -np.inf, -0.0]
    row = rng.integers(-3, M + 3, size=(L,), dtype=np.int32)
    col = rng.integers(-3, N + 3, size=(L,), dtype=np.int32)
    row[: min(L, 4)], col[: min(L, 4)] = 0, np.arange(min(L, 4))
    a = torch.from_numpy(A).cuda()
    r = torch.zeros(L + off, dtype=torch.int32, device="cuda")
    c = torch.zeros(L + off, dtype=torch.int32, device="cuda")
    r[off:], c[off:] = torch.from_numpy(row).cuda(), torch.from_numpy(col).cuda()
    o = torch.full((L + off + 4,), 123.0, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"[case] gather2d_f32 L={L} offset={off}", flush=True)
    st = hip.ihip_gather2d_f32(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(r.data_ptr() + 4 * off),
                               ctypes.c_void_p(c.data_ptr() + 4 * off), ctypes.c_void_p(o.data_ptr() + 4 * off),
                               M, N, L, 2.5, s)
    assert st == 0, hip.ihip_last_error()
    torch.cuda.synchronize()
    oh = o.cpu().numpy()
    np.testing.assert_array_equal(oh[off:off + L].view(np.uint32), _rule(A, row, col, 2.5).view(np.uint32))
    assert (oh[:off] == 123.0).all() and (oh[off + L:] == 123.0).all()


def test_gather_from_an_empty_tensor_and_of_nothing(hip):
    import torch

    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    row = torch.arange(8, dtype=torch.int32, device="cuda")
    o = torch.zeros(8, device="cuda")
    print("[case] gather2d_f32 M=0", flush=True)
    assert hip.ihip_gather2d_f32(None, ctypes.c_void_p(row.data_ptr()), ctypes.c_void_p(row.data_ptr()),
                                 ctypes.c_void_p(o.data_ptr()), 0, 5, 8, -7.0, s) == 0
    assert hip.ihip_gather2d_f32(None, None, None, None, 3, 5, 0, -7.0, s) == 0
    torch.cuda.synchronize()
    assert (o.cpu().numpy() == -7.0).all()
