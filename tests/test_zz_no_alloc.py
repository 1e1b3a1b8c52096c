"""ihip_reduce_rows_f32_noalloc: the entry point that allocates nothing, against
ihip_reduce_rows_f32_ws (the same kernels with a caller workspace).

Two calls in a row on one stream, the second with a smaller input (the scratch keeps
the first call's partials), each compared bit for bit with the workspace form; plus a
shape that does not split (no scratch used) and the size check."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run_pair(hip, torch, x, kind, s):
    M, N = x.shape
    a = torch.empty(M, device="cuda")
    b = torch.empty(M, device="cuda")
    need = hip.ihip_reduce_rows_f32_workspace_size(M, N)
    ws = torch.empty(max(1, need), dtype=torch.uint8, device="cuda")
    st = hip.ihip_reduce_rows_f32_noalloc(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(a.data_ptr()), M, N, kind, s)
    assert st == 0, hip.ihip_last_error()
    st = hip.ihip_reduce_rows_f32_ws(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(b.data_ptr()), M, N, kind,
                                     ctypes.c_void_p(ws.data_ptr()), need, s)
    assert st == 0, hip.ihip_last_error()
    torch.cuda.synchronize()
    return a.cpu().numpy(), b.cpu().numpy(), need


@pytest.mark.parametrize("kind", [0, 1])
def test_noalloc_matches_the_workspace_form_on_consecutive_calls(hip, kind):
    import torch

    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device="cuda")
    g.manual_seed(11 + kind)
    for M, N in ((64, 1 << 20), (5, 262147)):  # second call smaller: stale partials stay in scratch
        x = torch.randn((M, N), generator=g, device="cuda")
        print(f"[case] reduce_rows_f32_noalloc kind={kind} M={M} N={N}", flush=True)
        a, b, need = _run_pair(hip, torch, x, kind, s)
        assert need > 0
        np.testing.assert_array_equal(a, b)
        ref = x.double().sum(dim=1) if kind == 0 else x.max(dim=1).values.double()
        np.testing.assert_allclose(a, ref.cpu().numpy(), rtol=1e-5, atol=1e-2 if kind == 0 else 0)


def test_noalloc_without_a_split_and_the_size_check(hip):
    import torch

    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    x = torch.randn((300, 4096), device="cuda")  # 300 rows: no split, no scratch
    print("[case] reduce_rows_f32_noalloc unsplit M=300 N=4096", flush=True)
    a, b, need = _run_pair(hip, torch, x, 0, s)
    assert need == 0
    np.testing.assert_array_equal(a, b)
    p = ctypes.c_void_p(256)  # rejected on the host before any launch
    assert hip.ihip_reduce_rows_f32_noalloc(p, p, 64, 1 << 20, 9, None) == -1
    assert b"unknown kind" in hip.ihip_last_error()
