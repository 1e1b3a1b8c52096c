"""GPU checks of the f32 entry points: the fp32-MFMA GEMM, the f32 LayerNorm, softmax row
statistics, scaled row sums and element-wise programs past the interpreter kernel's limits.

* GEMM (ihip_gemm_f32_bias_relu): integer-valued operands in [-4, 4] give exact f32 products
  and partial sums, so every layout (transpose flags), tile (64 / 128), alignment and ragged
  edge must reproduce numpy bit for bit; N(0, 1) operands at large K are held to the fp32
  accumulation bound |C - C64| <= 2^-20 * sqrt(K) * (|A| @ |B|) against a float64 product, and
  the reference smoke test's rtol 1e-4 / atol 1e-4 at its own size.
* LayerNorm f32: y rtol 1e-5 / atol 1e-5, mean and rstd rtol 1e-5 / atol 1e-6 against the
  oracle, every kernel form (one wave per row, several waves, the any-shape form for odd N,
  unaligned views and rows past 65536).
* softmax statistics: row_max bit-exact, row_sum and y rtol 1e-5 / atol 1e-7, every form.
* reduce_sum{scale}: rtol 1e-5 / atol 1e-6, split and unsplit.
* element-wise programs with more than 8 inputs, 8 live values or 64 instructions: rtol 1e-5
  / atol 1e-6 against the oracle in AUTO mode, refused in INTERP mode.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from intent_ir_amd import HipRuntimeError, lower_intent_to_hip_kernel, run_lowered
from intent_ir_amd.runtime import EW_MODE_INTERP
from oracle.compare import compare_outputs
from oracle.interpreter import execute_intent
from tests.reference_builder_irs import builder_ir

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def _torch():
    import torch

    return torch


def _stream():
    return P(_torch().cuda.current_stream().cuda_stream)


def _ok(hip, st):
    assert st == 0, hip.ihip_last_error().decode()


def _dev(a: np.ndarray, pad: int = 0):
    """A device copy of a, starting `pad` floats into a larger allocation (an unaligned view)."""
    torch = _torch()
    flat = torch.zeros(a.size + pad + 4, dtype=torch.float32, device="cuda")
    flat[pad:pad + a.size] = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32).ravel()).cuda()
    return flat, flat[pad:pad + a.size]


def _gemm(hip, A, B, bias, M, N, K, ta, tb, relu, tile=0, pads=(0, 0, 0)):
    torch = _torch()
    _, a = _dev(A, pads[0])
    _, b = _dev(B, pads[1])
    bb = None if bias is None else _dev(bias)[1]
    cbuf, c = _dev(np.zeros(M * N, np.float32), pads[2])
    _ok(hip, hip.ihip_gemm_f32_bias_relu(P(a.data_ptr()), P(b.data_ptr()), P(None if bb is None else bb.data_ptr()),
                                         P(c.data_ptr()), M, N, K, int(ta), int(tb), int(relu), tile, _stream()))
    torch.cuda.synchronize()
    return c.cpu().numpy().reshape(M, N)


def _np_gemm(A, B, bias, ta, tb, relu):
    c = (A.T if ta else A) @ (B.T if tb else B)
    if bias is not None:
        c = c + bias[None, :]
    return np.maximum(c, 0) if relu else c


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (33, 65, 17), (64, 64, 32), (128, 128, 32), (129, 257, 95),
                                   (300, 200, 1000), (64, 4096, 64), (1000, 37, 300)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_f32_bit_exact_on_integer_operands(hip, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    A = rng.integers(-4, 5, size=(K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-4, 5, size=(N, K) if tb else (K, N)).astype(np.float32)
    bias = rng.integers(-8, 9, size=N).astype(np.float32)
    for relu, bs in ((False, None), (True, bias)):
        print(f"[case] gemm_f32 exact M={M} N={N} K={K} ta={ta} tb={tb} relu={relu}", flush=True)
        got = _gemm(hip, A, B, bs, M, N, K, ta, tb, relu)
        np.testing.assert_array_equal(got, _np_gemm(A, B, bs, ta, tb, relu).astype(np.float32))


@pytest.mark.parametrize("pads", [(1, 0, 0), (0, 3, 0), (0, 0, 1), (2, 1, 3)])
def test_gemm_f32_unaligned_operands_give_the_same_bits(hip, pads):
    """Operands and C at 4-byte offsets take element-wise copies and stores, with the same
    k order: bit-identical to the aligned call."""
    M, N, K = 130, 132, 68
    rng = np.random.default_rng(sum(pads))
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    print(f"[case] gemm_f32 pads={pads}", flush=True)
    ref = _gemm(hip, A, B, None, M, N, K, False, False, False)
    got = _gemm(hip, A, B, None, M, N, K, False, False, False, pads=pads)
    np.testing.assert_array_equal(got, ref)


def test_gemm_f32_tile_knob_gives_the_same_bits(hip):
    M, N, K = 520, 390, 250
    rng = np.random.default_rng(5)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    outs = [_gemm(hip, A, B, bias, M, N, K, False, False, True, tile=t) for t in (0, 64, 128)]
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(outs[0], outs[2])


def test_gemm_f32_k0_is_the_epilogue_of_zero(hip):
    bias = np.array([-1.0, 0.5, -0.0, 2.0, -3.0], np.float32)
    got = _gemm(hip, np.zeros((4, 0), np.float32), np.zeros((0, 5), np.float32), bias, 4, 5, 0, False, False, True)
    np.testing.assert_array_equal(got, np.broadcast_to(np.maximum(bias, 0), (4, 5)))


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (8192, 8192, 8192)])
def test_gemm_f32_large_within_the_accumulation_bound(hip, M, N, K):
    """Full-size products against a float64 evaluation on a row sample (64 rows): the fp32
    accumulation bound 2^-20 * sqrt(K) * (|A| @ |B|), 16x the expected 2^-24 * sqrt(K)."""
    torch = _torch()
    g = torch.Generator(device="cuda")
    g.manual_seed(M)
    a = torch.randn((M, K), device="cuda", generator=g)
    b = torch.randn((K, N), device="cuda", generator=g)
    bias = torch.randn((N,), device="cuda", generator=g)
    c = torch.empty((M, N), device="cuda")
    print(f"[case] gemm_f32 large {M}x{N}x{K}", flush=True)
    _ok(hip, hip.ihip_gemm_f32_bias_relu(P(a.data_ptr()), P(b.data_ptr()), P(bias.data_ptr()), P(c.data_ptr()), M, N,
                                         K, 0, 0, 1, 0, _stream()))
    torch.cuda.synchronize()
    rows = np.random.default_rng(0).choice(M, 64, replace=False)
    A = a[rows].double().cpu().numpy()
    B = b.double().cpu().numpy()
    ref = np.maximum(A @ B + bias.double().cpu().numpy()[None, :], 0)
    bound = 2.0 ** -20 * np.sqrt(K) * (np.abs(A) @ np.abs(B))
    got = c[rows].cpu().numpy().astype(np.float64)
    assert (np.abs(got - ref) <= bound).all(), np.max(np.abs(got - ref) / bound)


def test_gemm_f32_reference_smoke_tolerance(hip):
    """tests/backends/cuda/test_cuda_backend_smoke.py:27-66 as written: 32x48x16, rtol/atol 1e-4."""
    ir = builder_ir("cuda_smoke.matmul")
    b = {"M": 32, "N": 48, "K": 16}
    rng = np.random.default_rng(0)
    A = rng.standard_normal((32, 16), dtype=np.float32)
    B = rng.standard_normal((16, 48), dtype=np.float32)
    got = run_lowered(lower_intent_to_hip_kernel(ir, shape_bindings=b), {"A": A, "B": B})["C"]
    np.testing.assert_allclose(got, A @ B, rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------ LayerNorm f32
def _ln_check(got, ref, what):
    for o, tol in (("out_ptr", {"atol": 1e-5, "rtol": 1e-5}), ("out_mean_ptr", {"atol": 1e-6, "rtol": 1e-5}),
                   ("out_rstd_ptr", {"atol": 1e-6, "rtol": 1e-5})):
        d = compare_outputs({o: got[o]}, {o: np.asarray(ref[o]).reshape(got[o].shape)}, [o], tol)
        assert d.ok, f"{what}: {o} {d.summary} max_abs={d.max_abs_err:.3g} max_rel={d.max_rel_err:.3g}"


@pytest.mark.parametrize("N", [1, 2, 3, 7, 8, 17, 33, 64, 100, 256, 1000, 1024, 1027, 4096, 4100, 5000, 16384, 65536,
                               65540, 70000])
@pytest.mark.parametrize("form", ["tilelang.layer_norm_persistent", "cuda.layer_norm_persistent"])
def test_layernorm_f32_every_form(hip, N, form):
    M = 37
    b = {"M": M, "N": N}
    rng = np.random.default_rng(N)
    inp = {"in_ptr": (rng.standard_normal((M, N)) * 3 + 1).astype(np.float32),
           "weight_ptr": (1 + 0.1 * rng.standard_normal(N)).astype(np.float32),
           "bias_ptr": (0.1 * rng.standard_normal(N)).astype(np.float32)}
    ir = builder_ir(form)
    print(f"[case] layernorm f32 {form} N={N}", flush=True)
    got = run_lowered(lower_intent_to_hip_kernel(ir, shape_bindings=b), inp)
    _ln_check(got, execute_intent(ir, inp, b), f"{form} N={N}")


@pytest.mark.parametrize("N,pad", [(4096, 1), (1024, 2), (100, 3), (65536, 1)])
def test_layernorm_f32_unaligned_views(hip, N, pad):
    """Rows that start off a 16-byte boundary take the any-shape form; results as the oracle's."""
    torch = _torch()
    M = 19
    rng = np.random.default_rng(pad + N)
    x = rng.standard_normal((M, N)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(N)).astype(np.float32)
    bb = (0.1 * rng.standard_normal(N)).astype(np.float32)
    _, xd = _dev(x, pad)
    _, wd = _dev(w, pad)
    _, bd = _dev(bb)
    ybuf, yd = _dev(np.zeros(M * N, np.float32), pad)
    mean = torch.empty(M, device="cuda")
    rstd = torch.empty(M, device="cuda")
    print(f"[case] layernorm f32 unaligned N={N} pad={pad}", flush=True)
    _ok(hip, hip.ihip_layernorm_rows_f32(P(xd.data_ptr()), P(wd.data_ptr()), P(bd.data_ptr()), P(yd.data_ptr()),
                                         P(mean.data_ptr()), P(rstd.data_ptr()), M, N, ctypes.c_float(1e-5),
                                         _stream()))
    torch.cuda.synchronize()
    ir = builder_ir("tilelang.layer_norm_persistent")
    b = {"M": M, "N": N}
    ref = execute_intent(ir, {"in_ptr": x, "weight_ptr": w, "bias_ptr": bb}, b)
    got = {"out_ptr": yd.cpu().numpy().reshape(M, N), "out_mean_ptr": mean.cpu().numpy(),
           "out_rstd_ptr": rstd.cpu().numpy()}
    _ln_check(got, ref, f"unaligned N={N} pad={pad}")


def test_layernorm_f32_large(hip):
    """8192 x 4096 f32 (the LayerNorm config in f32) against the oracle in full."""
    M, N = 8192, 4096
    b = {"M": M, "N": N}
    rng = np.random.default_rng(3)
    inp = {"in_ptr": rng.standard_normal((M, N), dtype=np.float32),
           "weight_ptr": (1 + 0.1 * rng.standard_normal(N)).astype(np.float32),
           "bias_ptr": (0.1 * rng.standard_normal(N)).astype(np.float32)}
    ir = builder_ir("tilelang.layer_norm_persistent")
    got = run_lowered(lower_intent_to_hip_kernel(ir, shape_bindings=b), inp)
    _ln_check(got, execute_intent(ir, inp, b), "8192x4096")


# ------------------------------------------------------------------ softmax statistics
@pytest.mark.parametrize("N", [1, 4, 31, 64, 100, 128, 129, 1000, 1024, 1027, 4096, 4099, 5000, 16384, 65536, 65539,
                               70000, 131072])
@pytest.mark.parametrize("M", [3, 33])
def test_softmax_statistics_every_form(hip, M, N):
    ir = builder_ir("cuda.softmax_inner")
    b = {"M": M, "N": N}
    rng = np.random.default_rng(M * N)
    x = (rng.standard_normal((M, N)) * 2.0).astype(np.float32)
    x[rng.random((M, N)) < 0.01] = 30.0
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    print(f"[case] softmax stats {k.kernel_id} M={M} N={N} launch={k.launch}", flush=True)
    got = run_lowered(k, {"input_ptr": x})
    ref = execute_intent(ir, {"input_ptr": x}, b)
    assert np.array_equal(got["row_max_ptr"], ref["row_max_ptr"])
    for o, tol in (("output_ptr", {"atol": 1e-7, "rtol": 1e-5}), ("row_sum_ptr", {"atol": 1e-7, "rtol": 1e-5})):
        d = compare_outputs({o: got[o]}, {o: ref[o]}, [o], tol)
        assert d.ok, f"{o}: {d.summary} max_rel={d.max_rel_err:.3g}"


# ------------------------------------------------------------------ reduce_sum{scale}
@pytest.mark.parametrize("M,N", [(1, 1), (7, 33), (300, 100), (4096, 4096), (4, 1 << 20), (100, 65539)])
def test_scaled_row_sum(hip, M, N):
    ir = {"name": "row_mean", "tensors": {"x": {"dtype": "f32", "shape": ["M", "N"]},
                                          "m": {"dtype": "f32", "shape": ["M"]}},
          "ops": [{"op": "reduce_sum", "inputs": ["x"], "output": "m", "attrs": {"dims": [1], "scale": "1.0/N"}}],
          "outputs": ["m"]}
    b = {"M": M, "N": N}
    x = np.random.default_rng(N).standard_normal((M, N)).astype(np.float32) + 0.5
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    print(f"[case] scaled row sum {k.kernel_id} M={M} N={N}", flush=True)
    got = run_lowered(k, {"x": x})
    d = compare_outputs(got, execute_intent(ir, {"x": x}, b), ["m"], {"atol": 1e-6, "rtol": 1e-5})
    assert d.ok, d.summary


# ------------------------------------------------------------------ large element-wise programs
def _ew_sum_ir(n_in: int):
    t = {f"a{i}": {"dtype": "f32", "shape": ["M", "N"]} for i in range(n_in)}
    ops, acc = [], "a0"
    for i in range(1, n_in):
        out = f"s{i}" if i < n_in - 1 else "y"
        ops.append({"op": "add", "inputs": [acc, f"a{i}"], "output": out})
        acc = out
    t["y"] = {"dtype": "f32", "shape": ["M", "N"]}
    return {"name": f"sum{n_in}", "tensors": t, "ops": ops, "outputs": ["y"]}


def _ew_live_ir(n: int):
    """t_i = exp(x * c_i), y1 = sum t_i, y2 = product t_i: all n values live at once."""
    t = {"x": {"dtype": "f32", "shape": ["M", "N"]}, "y1": {"dtype": "f32", "shape": ["M", "N"]},
         "y2": {"dtype": "f32", "shape": ["M", "N"]}}
    ops = []
    for i in range(n):
        ops += [{"op": "const", "inputs": [], "output": f"c{i}", "attrs": {"value": 0.05 * (i + 1), "dtype": "f32"}},
                {"op": "mul", "inputs": ["x", f"c{i}"], "output": f"u{i}"},
                {"op": "exp", "inputs": [f"u{i}"], "output": f"t{i}"}]
    s, p = "t0", "t0"
    for i in range(1, n):
        ops += [{"op": "add", "inputs": [s, f"t{i}"], "output": f"s{i}" if i < n - 1 else "y1"},
                {"op": "mul", "inputs": [p, f"t{i}"], "output": f"p{i}" if i < n - 1 else "y2"}]
        s, p = (f"s{i}", f"p{i}") if i < n - 1 else ("y1", "y2")
    return {"name": f"live{n}", "tensors": t, "ops": ops, "outputs": ["y1", "y2"]}


def _ew_long_ir(n: int):
    """y = ((x * a + b) * a + b) ... n times: a chain of 2n dependent instructions."""
    t = {"x": {"dtype": "f32", "shape": ["M", "N"]}, "y": {"dtype": "f32", "shape": ["M", "N"]}}
    ops = [{"op": "const", "inputs": [], "output": "a", "attrs": {"value": 0.75, "dtype": "f32"}},
           {"op": "const", "inputs": [], "output": "b", "attrs": {"value": 0.125, "dtype": "f32"}}]
    v = "x"
    for i in range(n):
        ops += [{"op": "mul", "inputs": [v, "a"], "output": f"m{i}"},
                {"op": "add", "inputs": [f"m{i}", "b"], "output": f"v{i}" if i < n - 1 else "y"}]
        v = f"v{i}"
    return {"name": f"long{n}", "tensors": t, "ops": ops, "outputs": ["y"]}


@pytest.mark.parametrize("make,arg", [(_ew_sum_ir, 12), (_ew_sum_ir, 32), (_ew_live_ir, 12), (_ew_long_ir, 60)],
                         ids=["12-inputs", "32-inputs", "12-live", "120-instructions"])
def test_elementwise_programs_past_the_interpreter_limits(hip, make, arg):
    from intent_ir_amd.ewprogram import fits_interpreter

    ir = make(arg)
    b = {"M": 67, "N": 1000}
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    assert not fits_interpreter(k.call_args[0][1])
    rng = np.random.default_rng(arg)
    inp = {n: rng.standard_normal((67, 1000)).astype(np.float32) for n in ir["tensors"]
           if n not in {o["output"] for o in ir["ops"]}}
    print(f"[case] ew past limits {ir['name']}", flush=True)
    got = run_lowered(k, inp)
    ref = execute_intent(ir, inp, b)
    d = compare_outputs(got, ref, ir["outputs"], {"atol": 1e-6, "rtol": 1e-5})
    assert d.ok, f"{d.summary} max_rel={d.max_rel_err:.3g}"
    prev = hip.ihip_elementwise_mode(EW_MODE_INTERP)
    try:
        with pytest.raises(HipRuntimeError, match="interpreter kernel's limits"):
            run_lowered(k, inp)
    finally:
        hip.ihip_elementwise_mode(prev)


# ------------------------------------------------------------------ bf16 GEMM: 16x16x32 whole-tile kernel
@pytest.mark.parametrize("M,N,K", [(1000, 4096, 256), (4096, 1000, 320), (1000, 1000, 64), (8000, 8192, 512),
                                   (300, 264, 128), (257, 8, 64), (256, 264, 64), (513, 520, 192), (1, 2048, 128)])
@pytest.mark.parametrize("tb", [0, 1])
def test_gemm_m16_edge_tiles_match_the_ring_kernel_bit_for_bit(hip, M, N, K, tb):
    """M or N not a multiple of 256 (N % 8 == 0, K % 64 == 0) with 256x256 tiles: the 16x16x32
    kernel copies edge tiles through descriptors that end at the tensor and masks their stores.
    A C base 2 bytes off a 16-byte boundary sends the same product to the guarded kernel
    (gemm.hip), and tile knob 128 to the ring kernel; the three agree bit for bit, and nothing
    past C's last element is written."""
    torch = _torch()
    g = torch.Generator(device="cuda")
    g.manual_seed(M * 7 + N + K + tb)
    a = torch.randn((M, K), device="cuda", generator=g).bfloat16()
    b = torch.randn((N, K) if tb else (K, N), device="cuda", generator=g).bfloat16()
    bias = torch.randn((N,), device="cuda", generator=g)
    sentinel = -12345
    for relu in (1, 0):
        c1buf = torch.full((M * N + 64,), sentinel, device="cuda", dtype=torch.int16)
        c2buf = torch.full((M * N + 72,), sentinel, device="cuda", dtype=torch.int16)
        c3buf = torch.full((M * N + 64,), sentinel, device="cuda", dtype=torch.int16)
        c1, c2, c3 = c1buf[:M * N], c2buf[1:1 + M * N], c3buf[:M * N]
        print(f"[case] gemm m16 edge vs guarded and ring M={M} N={N} K={K} tb={tb} relu={relu}", flush=True)
        for c, tile in ((c1, 256), (c2, 256), (c3, 128)):
            _ok(hip, hip.ihip_gemm_bf16_bias_relu_ex(P(a.data_ptr()), P(b.data_ptr()), P(bias.data_ptr()),
                                                     P(c.data_ptr()), M, N, K, 0, tb, relu, tile, _stream()))
        torch.cuda.synchronize()
        assert torch.equal(c1, c2) and torch.equal(c1, c3)
        assert bool((c1buf[M * N:] == sentinel).all()) and bool((c2buf[1 + M * N:] == sentinel).all())
        assert int(c2buf[0]) == sentinel
        if M * N <= 1 << 22:  # and against a float32 evaluation (bf16 output rounding)
            ref = a.float() @ (b.float().t() if tb else b.float()) + bias
            ref = torch.relu(ref) if relu else ref
            got = c1.view(torch.bfloat16).reshape(M, N).float()
            assert torch.allclose(got, ref, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (256, 512, 128), (512, 768, 192), (1024, 1024, 1024),
                                   (2048, 1536, 4096), (256, 4096, 320), (4352, 4096, 128), (4096, 4352, 192),
                                   (8192, 8192, 64)])
@pytest.mark.parametrize("relu", [1, 0])
def test_gemm_m16_matches_the_ring_kernel_bit_for_bit(hip, M, N, K, relu):
    """Whole 256x256 tiles with K % 64 == 0 (tile knob 256) run gemm_m16.hip (16x16x32 MFMAs);
    tile knob 128 sends the same product to gemm_fast.hip's ring kernel (32x32x16 MFMAs), and a
    C base 2 bytes off a 16-byte boundary to the guarded kernel (gemm.hip, 2-byte stores).  The
    three agree bit for bit, with B given as [N, K] and as [K, N] (1, 2, 3 and more 64-k slices,
    so the prologue, the last two slices and the steady loop are all covered).  The 16x16x32
    grid is one workgroup per CU: 272 and 1024 tiles make workgroups take several tiles each, in
    uneven numbers for 272."""
    torch = _torch()
    g = torch.Generator(device="cuda")
    g.manual_seed(M + N + K)
    a = torch.randn((M, K), device="cuda", generator=g).bfloat16()
    bt = torch.randn((N, K), device="cuda", generator=g).bfloat16()
    b = bt.t().contiguous()  # the same product with B as [K, N]: the K-major form of the kernels
    bias = torch.randn((N,), device="cuda", generator=g)
    print(f"[case] gemm m16 vs ring vs guarded M={M} N={N} K={K} relu={relu}", flush=True)
    outs = []
    for tb, bx in ((1, bt), (0, b)):
        for tile, off in ((256, 0), (128, 0), (0, 1)):
            cbuf = torch.empty(M * N + 8, device="cuda", dtype=torch.bfloat16)
            c = cbuf[off:off + M * N]
            _ok(hip, hip.ihip_gemm_bf16_bias_relu_ex(P(a.data_ptr()), P(bx.data_ptr()), P(bias.data_ptr()),
                                                     P(c.data_ptr()), M, N, K, 0, tb, relu, tile, _stream()))
            outs.append(c)
    torch.cuda.synchronize()
    for c in outs[1:]:
        assert torch.equal(outs[0].view(torch.int16), c.view(torch.int16))
