"""GPU checks of masked softmax rows, stats-less LayerNorm, launch knobs and the
reference-shaped runtime call.

* Softmax rows holding -inf (masked logits): exp(-inf - max) is exactly 0, so those
  entries come out 0 and the rest is the softmax of the unmasked entries; a row that is
  all -inf is NaN (numpy: -inf - -inf = NaN).  Every kernel form is hit (one wave per
  row, several waves, 4-byte and head/body/tail rows).
* LayerNorm whose mean/rstd are not outputs writes no statistics: no scratch memory,
  no host synchronisation, so a launch can be captured in a graph.
* HIP_GEMM_TILE / HIP_ROWS_PER_WG select precompiled variants; the results must not
  change (every variant accumulates in the same order).
* run_hip_kernel called exactly like the reference's run_cuda_kernel
  (backends/cuda/runtime.py:22-45, cuda_src replaced by kernel_id).
"""

from __future__ import annotations

import numpy as np
import pytest

from intent_ir_amd import lower_intent_to_hip_kernel, run_lowered
from intent_ir_amd.configs import WORKLOADS
from intent_ir_amd.dtypes import to_compute_f32
from intent_ir_amd.ir import as_intent
from intent_ir_amd.runtime import launch_lowered, run_hip_kernel, tensor_shapes, to_device, torch_dtype
from oracle.compare import compare_outputs
from oracle.interpreter import execute_intent

pytestmark = pytest.mark.gpu


def _oracle(ir, inputs, b):
    fn = as_intent(ir)
    return execute_intent(ir, {n: to_compute_f32(v, fn.tensors[n].dtype) for n, v in inputs.items()}, b)


@pytest.mark.parametrize("N", [8, 31, 64, 100, 127, 128, 1000, 1029, 4096, 4099, 8192, 50257, 128256, 100003])
def test_softmax_rows_with_minus_inf(hip, N):
    w = WORKLOADS["softmax"]
    M = 6
    rng = np.random.default_rng(N)
    x = (rng.standard_normal((M, N)) * 2.0).astype(np.float32)
    x[0, rng.random(N) < 0.3] = -np.inf  # masked logits scattered over the row
    x[1, : N // 2] = -np.inf             # a masked prefix (head of the row)
    x[2, N - 5:] = -np.inf               # a masked tail
    x[3, :] = -np.inf                    # everything masked: NaN, as numpy
    x[4, 0] = -np.inf
    x[4, N - 1] = -np.inf
    x[5, 1] = -np.inf
    x[5, 2] = np.float32(-3.0e38)        # finite but beyond exp's range after the max shift
    b = {"M": M, "N": N}
    print(f"[case] softmax -inf rows N={N}", flush=True)
    out = run_lowered(lower_intent_to_hip_kernel(w.ir(), shape_bindings=b), {"input_ptr": x})["output_ptr"]
    with np.errstate(invalid="ignore"):
        ref = _oracle(w.ir(), {"input_ptr": x}, b)["output_ptr"]
    np.testing.assert_array_equal(np.isnan(out), np.isnan(ref))
    assert np.isnan(out[3]).all() and not np.isnan(out[[0, 1, 2, 4, 5]]).any()
    masked = np.isneginf(x)
    assert (out[masked & ~np.isnan(ref)] == 0.0).all()
    fin = ~np.isnan(ref)
    d = compare_outputs({"y": np.where(fin, out, 0)}, {"y": np.where(fin, ref, 0)}, ["y"],
                        {"atol": 1e-7, "rtol": 1e-5})
    assert d.ok, d.summary
    np.testing.assert_allclose(out[[0, 1, 2, 4, 5]].astype(np.float64).sum(axis=1), 1.0, rtol=1e-5)


def _ln_stats_less(M, N):
    ir = WORKLOADS["layernorm"].ir()
    ir["outputs"] = ["out_ptr"]
    return ir, {"M": M, "N": N}


@pytest.mark.parametrize("M,N", [(33, 4096), (16, 8192), (5, 4104), (3, 1000)])
def test_layernorm_without_statistics_matches_full_form(hip, M, N):
    import torch

    ir, b = _ln_stats_less(M, N)
    w = WORKLOADS["layernorm"]
    inp = w.gen(b)
    print(f"[case] layernorm stats-less M={M} N={N}", flush=True)
    y = run_lowered(lower_intent_to_hip_kernel(ir, shape_bindings=b), inp)["out_ptr"]
    full = run_lowered(lower_intent_to_hip_kernel(w.ir(), shape_bindings=b), inp)
    np.testing.assert_array_equal(y.view(np.uint16), full["out_ptr"].view(np.uint16))
    d = compare_outputs({"out_ptr": y}, _oracle(w.ir(), inp, b), ["out_ptr"], {"atol": 1e-3, "rtol": 1e-2})
    assert d.ok, d.summary
    torch.cuda.synchronize()


def test_layernorm_without_statistics_leaves_the_host_free_and_captures(hip):
    """launch_lowered returns while the stream is still busy (no host sync), and a stats-less
    launch captures into a HIP graph whose replays match the eager result."""
    import torch

    M, N = 8192, 4096
    ir, b = _ln_stats_less(M, N)
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    bufs = {"in_ptr": torch.randn((M, N), generator=g, device="cuda").half(),
            "weight_ptr": (1 + 0.1 * torch.randn(N, generator=g, device="cuda")).half(),
            "bias_ptr": (0.1 * torch.randn(N, generator=g, device="cuda")).half(),
            "out_ptr": torch.empty((M, N), dtype=torch.float16, device="cuda")}
    # keep the stream busy with a large GEMM so the LN launches queue behind it
    mk = lower_intent_to_hip_kernel(WORKLOADS["matmul"].ir(), shape_bindings={"M": 8192, "N": 8192, "K": 8192})
    ms = tensor_shapes(mk.io_spec, mk.bindings)
    mb = {n: torch.full(ms[n], 0.01, dtype=torch_dtype(s["dtype"]), device="cuda")
          for n, s in mk.io_spec["tensors"].items()}
    torch.cuda.synchronize()
    launch_lowered(mk, mb)
    launch_lowered(mk, mb)
    for _ in range(3):
        launch_lowered(k, bufs)
    busy = not torch.cuda.current_stream().query()
    torch.cuda.synchronize()
    assert busy, "the stream finished before launch_lowered returned: a host synchronisation is suspected"
    eager = bufs["out_ptr"].clone()
    bufs["out_ptr"].zero_()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        graph.capture_begin()
        launch_lowered(k, bufs, stream=s)
        graph.capture_end()
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):  # each replay checked against the eager result, with eager work between
        bufs["out_ptr"].fill_(float(i))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(bufs["out_ptr"], eager), f"replay {i} differs from the eager launch"
    del graph


@pytest.mark.parametrize("M,N,K,tb", [(1000, 1000, 512, False), (513, 264, 200, False), (300, 257, 96, True),
                                      (2048, 2048, 256, False)])
def test_gemm_tile_knob_gives_identical_results(hip, M, N, K, tb):
    ir = WORKLOADS["matmul"].ir()
    if tb:
        ir["tensors"]["B"]["shape"] = ["N", "K"]
        ir["ops"][0]["attrs"] = {"transpose_b": True}
    b = {"M": M, "N": N, "K": K}
    rng = np.random.default_rng(M + N + K)
    from intent_ir_amd.dtypes import f32_to_bf16_bits

    inp = {"A": f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32)),
           "B": f32_to_bf16_bits(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)),
           "bias": rng.standard_normal(N).astype(np.float32)}
    outs = []
    for knob in (None, 128, 256):
        bb = dict(b) if knob is None else {**b, "HIP_GEMM_TILE": knob}
        k = lower_intent_to_hip_kernel(ir, shape_bindings=bb)
        print(f"[case] gemm {b} tb={tb} tile={knob} -> {k.kernel_id} grid={k.launch.grid}", flush=True)
        outs.append(run_lowered(k, inp)["C"])
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(outs[0], outs[2])
    d = compare_outputs({"C": outs[1]}, _oracle(ir, inp, b), ["C"], {"atol": 2e-2, "rtol": 2e-2})
    assert d.ok, d.summary


@pytest.mark.parametrize("M,N", [(1000, 1024), (33, 64), (7, 4096), (4099, 100)])
def test_softmax_rows_per_workgroup_knob_gives_identical_results(hip, M, N):
    w = WORKLOADS["softmax"]
    inp = w.gen({"M": M, "N": N})
    outs = []
    for rows in (None, 1, 2, 4):
        bb = {"M": M, "N": N} if rows is None else {"M": M, "N": N, "HIP_ROWS_PER_WG": rows}
        k = lower_intent_to_hip_kernel(w.ir(), shape_bindings=bb)
        print(f"[case] softmax M={M} N={N} rows={rows} -> {k.kernel_id} block={k.launch.block}", flush=True)
        outs.append(run_lowered(k, inp)["output_ptr"])
    for o in outs[1:]:
        np.testing.assert_array_equal(outs[0], o)
    d = compare_outputs({"output_ptr": outs[2]}, _oracle(w.ir(), inp, {"M": M, "N": N}), ["output_ptr"],
                        {"atol": 1e-7, "rtol": 1e-5})
    assert d.ok, d.summary


@pytest.mark.parametrize("M", [1, 2, 3, 5, 6, 7, 9])
@pytest.mark.parametrize("N", [4, 64, 100, 512, 1000, 1024])
def test_softmax_two_rows_per_wave_at_every_row_count(hip, M, N):
    """Rows of at most 1024 floats run two rows per wave, two waves per workgroup: a wave whose
    second row is past the last re-reads the last row and must store nothing for it.  Every
    row count modulo 4 against the one-row-per-wave form (bit for bit) and the oracle; the
    output buffer's guard rows past M stay untouched."""
    import torch

    w = WORKLOADS["softmax"]
    b = {"M": M, "N": N}
    inp = w.gen(b)
    k2 = lower_intent_to_hip_kernel(w.ir(), shape_bindings=b)
    k1 = lower_intent_to_hip_kernel(w.ir(), shape_bindings={**b, "HIP_ROWS_PER_WG": 1})
    x = torch.from_numpy(inp["input_ptr"]).cuda()
    outs = []
    for k in (k2, k1):
        guard = torch.full((M + 4, N), 7.0, device="cuda")
        launch_lowered(k, {"input_ptr": x, "output_ptr": guard[:M]})
        torch.cuda.synchronize()
        assert torch.all(guard[M:] == 7.0), "a row past M was written"
        outs.append(guard[:M].cpu().numpy())
    np.testing.assert_array_equal(outs[0], outs[1])
    d = compare_outputs({"output_ptr": outs[0]}, _oracle(w.ir(), inp, b), ["output_ptr"], {"atol": 1e-7, "rtol": 1e-5})
    assert d.ok, d.summary


@pytest.mark.parametrize("key", sorted(WORKLOADS))
def test_run_hip_kernel_called_like_the_reference(hip, key):
    """The call site of the reference smoke test (tests/backends/cuda/test_cuda_backend_smoke.py:55-63),
    with cuda_src replaced by kernel_id: the argument plan travels in io_spec."""
    w = WORKLOADS[key]
    b = {"matmul": {"M": 64, "N": 96, "K": 128}}.get(key, {"M": 8, "N": 256})
    k = lower_intent_to_hip_kernel(w.ir(), shape_bindings=b)
    inp = w.gen(b)
    out = run_hip_kernel(kernel_name=k.kernel_name, kernel_id=k.kernel_id, io_spec=k.io_spec, launch=k.launch,
                         bindings=k.bindings, inputs_np=inp, output_names=k.output_names)
    ref = run_lowered(k, inp)
    for n in k.output_names:
        np.testing.assert_array_equal(out[n], ref[n])
    for n in inp:  # inputs come back too, as in the reference (frontends/cuda/runtime.py:1028-1031)
        np.testing.assert_array_equal(out[n], inp[n])


def test_run_hip_kernel_with_a_workspace_argument(hip):
    """A GEMM whose operands are packed carries a ("workspace", bytes) argument in its plan; the
    reference-shaped call allocates it from io_spec["hip_call"] alone."""
    w = WORKLOADS["matmul"]
    b = {"M": 64, "N": 97, "K": 100}
    k = lower_intent_to_hip_kernel(w.ir(), shape_bindings=b)
    assert k.kernel_id == "ihip_gemm_bf16_bias_relu_ws" and k.call_args[-1][0] == "workspace"
    inp = w.gen(b)
    out = run_hip_kernel(kernel_name=k.kernel_name, kernel_id=k.kernel_id, io_spec=k.io_spec, launch=k.launch,
                         bindings=k.bindings, inputs_np=inp, output_names=k.output_names)
    np.testing.assert_array_equal(out["C"], run_lowered(k, inp)["C"])
    d = compare_outputs({"C": out["C"]}, _oracle(w.ir(), inp, b), ["C"], {"atol": 2e-2, "rtol": 2e-2})
    assert d.ok, d.summary


def test_device_tensor_helpers_round_trip(hip):
    import torch

    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    t = to_device(x, "f32")
    assert t.device.type == "cuda" and torch.equal(t.cpu(), torch.from_numpy(x))


def test_gelu_workload_through_the_generic_program(hip):
    """HIP_ELEMENTWISE_PROGRAM=1: the bf16 GELU workload runs as an element-wise program (fused
    logistic step in its native code) and matches the oracle and the specialised kernel."""
    w = WORKLOADS["gelu"]
    b = {"M": 64, "N": 8192}
    inp = w.gen(b)
    prog = run_lowered(lower_intent_to_hip_kernel(w.ir(), shape_bindings={**b, "HIP_ELEMENTWISE_PROGRAM": 1}), inp)["y"]
    spec = run_lowered(lower_intent_to_hip_kernel(w.ir(), shape_bindings=b), inp)["y"]
    ref = _oracle(w.ir(), inp, b)
    for out in (prog, spec):
        d = compare_outputs({"y": out}, ref, ["y"], {"atol": 1e-3, "rtol": 1e-2})
        assert d.ok, d.summary
    # both round the same f32 value to bf16 unless it sits within a few ulps of a rounding tie
    assert np.mean(prog != spec) < 1e-3
