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


def _ws_reference(hip, torch, x, kind, s):
    M, N = x.shape
    out = torch.empty(M, device="cuda")
    need = hip.ihip_reduce_rows_f32_workspace_size(M, N)
    ws = torch.empty(max(1, need), dtype=torch.uint8, device="cuda")
    st = hip.ihip_reduce_rows_f32_ws(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()), M, N, kind,
                                     ctypes.c_void_p(ws.data_ptr()), need, s)
    assert st == 0, hip.ihip_last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _captured_noalloc_replays(hip, torch, kind):
    """Capture a split-shape noalloc call into a graph, replay it four times with new inputs and
    an eager noalloc call on a smaller shape (which rewrites the shared scratch) between the
    replays, and compare every result bit for bit with the workspace form."""
    g = torch.Generator(device="cuda")
    g.manual_seed(29 + kind)
    x = torch.randn((64, 1 << 20), generator=g, device="cuda")
    x2 = torch.randn((5, 262147), generator=g, device="cuda")
    a = torch.empty(64, device="cuda")
    c = torch.empty(5, device="cuda")
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    with torch.cuda.stream(cap):
        graph.capture_begin()
        st = hip.ihip_reduce_rows_f32_noalloc(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(a.data_ptr()), 64,
                                              1 << 20, kind, ctypes.c_void_p(cap.cuda_stream))
        graph.capture_end()
    assert st == 0, hip.ihip_last_error()
    torch.cuda.current_stream().wait_stream(cap)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for rep in range(4):
        x.copy_(torch.randn((64, 1 << 20), generator=g, device="cuda"))
        graph.replay()
        st = hip.ihip_reduce_rows_f32_noalloc(ctypes.c_void_p(x2.data_ptr()), ctypes.c_void_p(c.data_ptr()), 5,
                                              262147, kind, s)
        assert st == 0, hip.ihip_last_error()
        torch.cuda.synchronize()
        got, got2 = a.cpu().numpy(), c.cpu().numpy()
        np.testing.assert_array_equal(got, _ws_reference(hip, torch, x, kind, s), err_msg=f"replay {rep}")
        np.testing.assert_array_equal(got2, _ws_reference(hip, torch, x2, kind, s), err_msg=f"eager call {rep}")


@pytest.mark.parametrize("kind", [0, 1])
def test_noalloc_under_graph_capture(hip, kind):
    import torch

    print(f"[case] reduce_rows_f32_noalloc captured kind={kind}", flush=True)
    _captured_noalloc_replays(hip, torch, kind)


def test_noalloc_first_call_is_captured():
    """The first noalloc call of a process, inside a stream capture: it resolves the scratch's
    device address (hipGetSymbolAddress, not a stream operation) while capturing.  Runs in a
    fresh process, where no earlier call has resolved it."""
    import os
    import subprocess
    import sys

    from tests.conftest import hip_ready

    if not hip_ready():
        pytest.skip("no ROCm device")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import torch\n"
            "from intent_ir_amd.runtime import load_library\n"
            "from tests.test_zz_no_alloc import _captured_noalloc_replays\n"
            "_captured_noalloc_replays(load_library(), torch, 0)\n"
            "print('first-call capture ok', flush=True)\n")
    print("[case] reduce_rows_f32_noalloc first call under capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "first-call capture ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
