"""Randomised GEMM shapes and forms against the oracle (GPU).

Each seed draws M, N, K in [1, 700] (two thirds of them with N and K multiples of 8, so the
tiled kernel runs with ragged edge tiles; the rest take the guarded kernel), a layout
(transpose_a / transpose_b), bias or none and ReLU or none, and judges C against the oracle
restatement of verify/interpreter.py (matmul :507-520, then add / relu) with the GEMM
tolerances (rtol 2e-2) and the strict atol 1e-4 on unit-scale operands.  A second test plants
inf and NaN operands and checks the NaN / inf pattern of C exactly.
"""

from __future__ import annotations

import numpy as np
import pytest

from intent_ir_amd import lower_intent_to_hip_kernel, run_lowered
from intent_ir_amd.dtypes import f32_to_bf16_bits
from tests.test_gpu_parity import TOL, check, oracle_outputs

pytestmark = pytest.mark.gpu


def gemm_ir(ta: bool, tb: bool, bias: bool, relu: bool) -> dict:
    t = {"A": {"dtype": "bf16", "shape": ["K", "M"] if ta else ["M", "K"]},
         "B": {"dtype": "bf16", "shape": ["N", "K"] if tb else ["K", "N"]},
         "mm": {"dtype": "f32", "shape": ["M", "N"]}, "C": {"dtype": "bf16", "shape": ["M", "N"]}}
    ops = [{"op": "matmul", "inputs": ["A", "B"], "output": "mm", "attrs": {"transpose_a": ta, "transpose_b": tb}}]
    last = "mm"
    if bias:
        t["bias"] = {"dtype": "f32", "shape": ["N"]}
        t["mmb"] = {"dtype": "f32", "shape": ["M", "N"]}
        ops.append({"op": "add", "inputs": [last, "bias"], "output": "mmb"})
        last = "mmb"
    if relu:
        ops.append({"op": "relu", "inputs": [last], "output": "C"})
    else:
        ops[-1]["output"] = "C"
        if last == "mm":  # a lone matmul writes C directly
            del t["mm"]
        else:
            del t["mmb"]
    return {"name": "gemm_fuzz", "tensors": t, "ops": ops, "outputs": ["C"]}


@pytest.mark.parametrize("seed", range(48))
def test_random_gemm(hip, seed):
    rng = np.random.default_rng(1000 + seed)
    M, N, K = (int(v) for v in rng.integers(1, 701, size=3))
    if seed % 3:
        N, K = max(8, N // 8 * 8), max(8, K // 8 * 8)
    ta, tb, bias, relu = (bool(v) for v in rng.integers(0, 2, size=4))
    if ta and seed % 3:
        M = max(8, M // 8 * 8)
    ir = gemm_ir(ta, tb, bias, relu)
    b = {"M": M, "N": N, "K": K}
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    inp = {"A": f32_to_bf16_bits(A), "B": f32_to_bf16_bits(B)}
    if bias:
        inp["bias"] = rng.standard_normal(N).astype(np.float32)
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    print(f"[case] gemm fuzz seed={seed} M={M} N={N} K={K} ta={ta} tb={tb} bias={bias} relu={relu} "
          f"lds={k.launch.lds_bytes}", flush=True)
    out = run_lowered(k, inp)
    ref = oracle_outputs(ir, inp, b)
    check(out, ref, ["C"], TOL["matmul"], f"gemm fuzz {b} ta={ta} tb={tb}")
    check(out, ref, ["C"], TOL["matmul_strict"], f"gemm fuzz strict {b} ta={ta} tb={tb}")


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("M,N,K", [(67, 72, 40), (300, 263, 64), (520, 264, 96)])
def test_gemm_special_operands(hip, M, N, K, layout):
    """inf and NaN operands: C must hold NaN and +-inf where the oracle's float32 matmul does
    (a NaN or an inf times zero poisons its row or column; inf meeting -inf gives NaN), and
    ReLU keeps NaN (np.maximum).  Finite entries meet the GEMM tolerances."""
    tb = layout == "nt"
    rng = np.random.default_rng(M + N + K)
    ir = gemm_ir(False, tb, True, True)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    A[3, 5] = np.inf           # row 3: inf * B[5, :] -> +-inf, or NaN where B[5, n] == 0
    A[7, :] = 0.0
    A[7, 2] = np.nan           # row 7: NaN throughout
    Bk = B.T if tb else B      # [K, N] view for planting
    Bk[5, 11] = 0.0            # inf * 0 -> NaN at C[3, 11]
    Bk[9, 13] = -np.inf
    A[11, 9] = 1.0
    Bk[0, 13] = np.inf
    A[11, 0] = 1.0             # C[11, 13] = inf - inf = NaN
    inp = {"A": f32_to_bf16_bits(A), "B": f32_to_bf16_bits(B), "bias": rng.standard_normal(N).astype(np.float32)}
    b = {"M": M, "N": N, "K": K}
    k = lower_intent_to_hip_kernel(ir, shape_bindings=b)
    print(f"[case] gemm special operands M={M} N={N} K={K} layout={layout}", flush=True)
    out = run_lowered(k, inp)
    ref = oracle_outputs(ir, inp, b)
    c = np.asarray(out["C"], dtype=np.float64).reshape(M, N)
    r = np.asarray(ref["C"], dtype=np.float64)
    assert np.isnan(r).any() and np.isinf(r).any()
    np.testing.assert_array_equal(np.isnan(c), np.isnan(r), err_msg="NaN positions")
    np.testing.assert_array_equal(np.isinf(c) * np.sign(c), np.isinf(r) * np.sign(r), err_msg="inf positions")
    fin = np.isfinite(r)
    check({"C": c[fin]}, {"C": r[fin]}, ["C"], TOL["matmul"], f"gemm special {b} {layout}")
