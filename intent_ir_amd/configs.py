"""The five benchmark workloads: their IntentIR documents and seeded inputs.

Each IR is the form the reference's deterministic intent builders emit for the
corresponding kernel, with the dtypes the workload declares:

* ``any_kernel_dim``        pipeline/tilelang/core.py:115-130
* ``softmax_inner``         pipeline/tilelang/core.py:259-274
* ``layer_norm_persistent`` pipeline/tilelang/core.py:1322-1384 (x, w, b, y in f16)
* ``bias_gelu_axpy``        broadcast + add + ``gelu_tanh`` macro + axpy (bf16); the
                            add-bias prefix follows kernels/triton/ops/add_bias2d.py:6-21
* ``matmul_bias_relu2d``    pipeline/tilelang/core.py:886-910 (A, B, C in bf16)

Input distributions are those stated for the workloads.  bf16 inputs are
generated in float32 and rounded to bf16 (RNE); the oracle receives the exact
float32 widening of the stored bits.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, Mapping

import numpy as np

from .dtypes import f32_to_bf16_bits


def _t(dtype, shape):
    return {"dtype": dtype, "shape": list(shape), "layout": "row_major"}


def any_kernel_dim_ir() -> dict:
    return {
        "name": "any_kernel_dim",
        "tensors": {"inp": _t("f32", ["M", "N"]), "out": _t("bool", ["M"])},
        "ops": [{"op": "reduce_any", "inputs": ["inp"], "output": "out", "attrs": {"dims": [1], "keepdims": False}}],
        "outputs": ["out"],
        "schedule": {"tile_m": 16, "tile_n": 16, "vec_width": 1, "pipeline_depth": 1},
        "axis_roles": {"M": "spatial", "N": "reduction"},
    }


def softmax_inner_ir() -> dict:
    return {
        "name": "softmax_inner",
        "tensors": {"input_ptr": _t("f32", ["M", "N"]), "output_ptr": _t("f32", ["M", "N"])},
        "ops": [{"op": "softmax", "inputs": ["input_ptr"], "output": "output_ptr", "attrs": {"axis": -1}}],
        "outputs": ["output_ptr"],
        "schedule": {"tile_m": 16, "tile_n": 16, "vec_width": 1, "pipeline_depth": 1},
        "axis_roles": {"M": "spatial", "N": "channel"},
    }


def layer_norm_persistent_ir(io_dtype: str = "f16") -> dict:
    MN, M1 = ["M", "N"], ["M", 1]
    t = {
        "in_ptr": _t(io_dtype, MN), "weight_ptr": _t(io_dtype, ["N"]), "bias_ptr": _t(io_dtype, ["N"]),
        "out_ptr": _t(io_dtype, MN), "out_mean_ptr": _t("f32", ["M"]), "out_rstd_ptr": _t("f32", ["M"]),
        "sum_row": _t("f32", M1), "mean_row": _t("f32", M1), "diff": _t("f32", MN), "sq": _t("f32", MN),
        "var_sum": _t("f32", M1), "var": _t("f32", M1), "eps": _t("f32", []), "var_eps": _t("f32", M1),
        "rstd_row": _t("f32", M1), "xhat": _t("f32", MN), "w_b": _t("f32", MN), "b_b": _t("f32", MN),
        "scaled": _t("f32", MN),
    }
    ops = [
        {"op": "reduce_sum", "inputs": ["in_ptr"], "output": "sum_row", "attrs": {"dims": [1], "keepdims": True}},
        {"op": "div", "inputs": ["sum_row"], "output": "mean_row", "attrs": {"divisor": "N"}},
        {"op": "sub", "inputs": ["in_ptr", "mean_row"], "output": "diff"},
        {"op": "mul", "inputs": ["diff", "diff"], "output": "sq"},
        {"op": "reduce_sum", "inputs": ["sq"], "output": "var_sum", "attrs": {"dims": [1], "keepdims": True}},
        {"op": "div", "inputs": ["var_sum"], "output": "var", "attrs": {"divisor": "N"}},
        {"op": "const", "inputs": [], "output": "eps", "attrs": {"value": 1e-5, "dtype": "f32"}},
        {"op": "add", "inputs": ["var", "eps"], "output": "var_eps"},
        {"op": "rsqrt", "inputs": ["var_eps"], "output": "rstd_row"},
        {"op": "mul", "inputs": ["diff", "rstd_row"], "output": "xhat"},
        {"op": "broadcast_in_dim", "inputs": ["weight_ptr"], "output": "w_b",
         "attrs": {"out_shape": MN, "broadcast_dims": [1]}},
        {"op": "broadcast_in_dim", "inputs": ["bias_ptr"], "output": "b_b",
         "attrs": {"out_shape": MN, "broadcast_dims": [1]}},
        {"op": "mul", "inputs": ["xhat", "w_b"], "output": "scaled"},
        {"op": "add", "inputs": ["scaled", "b_b"], "output": "out_ptr"},
        {"op": "reshape", "inputs": ["mean_row"], "output": "out_mean_ptr", "attrs": {"shape": ["M"]}},
        {"op": "reshape", "inputs": ["rstd_row"], "output": "out_rstd_ptr", "attrs": {"shape": ["M"]}},
    ]
    return {
        "name": "layer_norm_persistent", "tensors": t, "ops": ops,
        "outputs": ["out_ptr", "out_mean_ptr", "out_rstd_ptr"],
        "schedule": {"tile_m": 16, "tile_n": 16, "vec_width": 1, "pipeline_depth": 1},
        "axis_roles": {"M": "spatial", "N": "channel"},
    }


def bias_gelu_axpy_ir(io_dtype: str = "bf16") -> dict:
    MN = ["M", "N"]
    return {
        "name": "bias_gelu_axpy",
        "tensors": {
            "x": _t(io_dtype, MN), "bias": _t(io_dtype, ["N"]), "y": _t(io_dtype, MN),
            "bias2d": _t("f32", MN), "z": _t("f32", MN), "g": _t("f32", MN), "half": _t("f32", []),
            "gh": _t("f32", MN),
        },
        "ops": [
            {"op": "broadcast_in_dim", "inputs": ["bias"], "output": "bias2d",
             "attrs": {"out_shape": MN, "broadcast_dims": [1]}},
            {"op": "add", "inputs": ["x", "bias2d"], "output": "z"},
            {"op": "gelu_tanh", "inputs": ["z"], "output": "g"},
            {"op": "const", "inputs": [], "output": "half", "attrs": {"value": 0.5, "dtype": "f32"}},
            {"op": "mul", "inputs": ["g", "half"], "output": "gh"},
            {"op": "add", "inputs": ["gh", "x"], "output": "y"},
        ],
        "outputs": ["y"],
        "schedule": {"tile_n": 256, "parallel_axes": ["M", "N"]},
        "parallel_axes": ["M", "N"],
        "axis_roles": {"M": "spatial", "N": "channel"},
    }


def matmul_bias_relu2d_ir(io_dtype: str = "bf16") -> dict:
    MN = ["M", "N"]
    return {
        "name": "matmul_bias_relu2d",
        "tensors": {
            "A": _t(io_dtype, ["M", "K"]), "B": _t(io_dtype, ["K", "N"]), "bias": _t("f32", ["N"]),
            "C": _t(io_dtype, MN), "mm": _t("f32", MN), "b2": _t("f32", MN), "mm_b": _t("f32", MN),
        },
        "ops": [
            {"op": "matmul", "inputs": ["A", "B"], "output": "mm", "attrs": {}},
            {"op": "broadcast_in_dim", "inputs": ["bias"], "output": "b2",
             "attrs": {"out_shape": MN, "broadcast_dims": [1]}},
            {"op": "add", "inputs": ["mm", "b2"], "output": "mm_b"},
            {"op": "relu", "inputs": ["mm_b"], "output": "C"},
        ],
        "outputs": ["C"],
        "schedule": {"tile_m": 32, "tile_n": 32, "tile_k": 16, "vec_width": 1, "pipeline_depth": 2},
        "axis_roles": {"M": "spatial", "N": "spatial", "K": "reduction"},
    }


# ----------------------------------------------------------------------------- inputs

def gen_any_kernel_dim(b: Mapping[str, int], seed: int = 1) -> Dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    m, n = int(b["M"]), int(b["N"])
    inp = np.zeros((m, n), dtype=np.float32)
    mask = rng.random((m, n)) < 1e-4
    inp[mask] = rng.standard_normal(int(mask.sum()), dtype=np.float32)
    return {"inp": inp}


def gen_softmax_inner(b: Mapping[str, int], seed: int = 2) -> Dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    m, n = int(b["M"]), int(b["N"])
    x = (rng.standard_normal((m, n), dtype=np.float32) * np.float32(2.0)).astype(np.float32)
    spike = rng.random((m, n)) < 0.01
    sign = np.where(rng.random(int(spike.sum())) < 0.5, -30.0, 30.0).astype(np.float32)
    x[spike] = sign
    return {"input_ptr": x}


def gen_layer_norm(b: Mapping[str, int], seed: int = 3) -> Dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    m, n = int(b["M"]), int(b["N"])
    return {
        "in_ptr": rng.standard_normal((m, n), dtype=np.float32).astype(np.float16),
        "weight_ptr": (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float16),
        "bias_ptr": (0.1 * rng.standard_normal(n)).astype(np.float16),
    }


def gen_bias_gelu_axpy(b: Mapping[str, int], seed: int = 4) -> Dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    m, n = int(b["M"]), int(b["N"])
    return {
        "x": f32_to_bf16_bits(rng.standard_normal((m, n), dtype=np.float32)),
        "bias": f32_to_bf16_bits((0.02 * rng.standard_normal(n)).astype(np.float32)),
    }


def gen_matmul_bias_relu(b: Mapping[str, int], seed: int = 5, sigma: float | None = None) -> Dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    m, n, k = int(b["M"]), int(b["N"]), int(b["K"])
    # Workload wording "N(0, 1/sqrt(8192))" read as a standard deviation of 1/sqrt(K).
    s = np.float32(1.0 / np.sqrt(k) if sigma is None else sigma)
    return {
        "A": f32_to_bf16_bits(rng.standard_normal((m, k), dtype=np.float32) * s),
        "B": f32_to_bf16_bits(rng.standard_normal((k, n), dtype=np.float32) * s),
        "bias": (0.1 * rng.standard_normal(n)).astype(np.float32),
    }


def gen_device(key: str, b: Mapping[str, int], torch, g) -> Dict[str, "object"]:
    """The workload's inputs with the same distributions, generated on the GPU (seeded
    torch generator ``g``), for benchmarking without host-side generation or copies."""
    dev = "cuda"
    M, N = int(b["M"]), int(b["N"])
    if key == "any":
        x = torch.zeros((M, N), dtype=torch.float32, device=dev)
        mask = torch.rand((M, N), generator=g, device=dev) < 1e-4
        x[mask] = torch.randn(int(mask.sum().item()), generator=g, device=dev)
        return {"inp": x}
    if key == "softmax":
        x = torch.randn((M, N), generator=g, device=dev) * 2.0
        spike = torch.rand((M, N), generator=g, device=dev) < 0.01
        sign = torch.where(torch.rand((M, N), generator=g, device=dev) < 0.5, -30.0, 30.0)
        return {"input_ptr": torch.where(spike, sign, x).contiguous()}
    if key == "layernorm":
        return {"in_ptr": torch.randn((M, N), generator=g, device=dev).half(),
                "weight_ptr": (1.0 + 0.1 * torch.randn(N, generator=g, device=dev)).half(),
                "bias_ptr": (0.1 * torch.randn(N, generator=g, device=dev)).half()}
    if key == "gelu":
        return {"x": torch.randn((M, N), generator=g, device=dev).bfloat16(),
                "bias": (0.02 * torch.randn(N, generator=g, device=dev)).bfloat16()}
    if key == "matmul":
        K = int(b["K"])
        s = 1.0 / float(np.sqrt(K))
        return {"A": (torch.randn((M, K), generator=g, device=dev) * s).bfloat16(),
                "B": (torch.randn((K, N), generator=g, device=dev) * s).bfloat16(),
                "bias": 0.1 * torch.randn(N, generator=g, device=dev)}
    raise KeyError(key)


@dataclass(frozen=True)
class Workload:
    key: str
    ir: Callable[[], dict]
    bindings: Dict[str, int]
    gen: Callable[..., Dict[str, np.ndarray]]
    bound: str              # "hbm" | "mfma"
    algo_units: str         # what one launch's algorithmic work counts
    description: str

    def algorithmic_bytes(self, b: Mapping[str, int] | None = None) -> int:
        return algorithmic_bytes(self.key, b or self.bindings)

    def algorithmic_flops(self, b: Mapping[str, int] | None = None) -> int:
        b = b or self.bindings
        return 2 * int(b["M"]) * int(b["N"]) * int(b["K"]) if self.key == "matmul" else 0


def algorithmic_bytes(key: str, b: Mapping[str, int]) -> int:
    """Bytes a launch must move at minimum: every input read once, every output written once."""
    M, N = int(b["M"]), int(b["N"])
    if key == "any":
        return 4 * M * N + M
    if key == "softmax":
        return 4 * M * N * 2
    if key == "layernorm":
        return 2 * M * N + 2 * 2 * N + 2 * M * N + 2 * 4 * M
    if key == "gelu":
        return 2 * M * N + 2 * N + 2 * M * N
    if key == "matmul":
        K = int(b["K"])
        return 2 * M * K + 2 * K * N + 4 * N + 2 * M * N
    raise KeyError(key)


WORKLOADS: Dict[str, Workload] = {
    "any": Workload("any", any_kernel_dim_ir, {"M": 8192, "N": 4096}, gen_any_kernel_dim, "hbm",
                    "one [8192,4096] f32 matrix -> bool[8192]", "any_kernel_dim reduce_any over dim=1"),
    "softmax": Workload("softmax", softmax_inner_ir, {"M": 16384, "N": 1024}, gen_softmax_inner, "hbm",
                        "one [16384,1024] f32 matrix", "row softmax f32"),
    "layernorm": Workload("layernorm", layer_norm_persistent_ir, {"M": 8192, "N": 4096}, gen_layer_norm, "hbm",
                          "one [8192,4096] f16 matrix + f32 stats", "LayerNorm forward f16"),
    "gelu": Workload("gelu", bias_gelu_axpy_ir, {"M": 32768, "N": 8192}, gen_bias_gelu_axpy, "hbm",
                     "one [32768,8192] bf16 matrix", "bias + GELU-tanh * 0.5 + x, bf16"),
    "matmul": Workload("matmul", matmul_bias_relu2d_ir, {"M": 8192, "N": 8192, "K": 8192}, gen_matmul_bias_relu,
                       "mfma", "one 8192^3 bf16 GEMM", "relu(A@B + bias) bf16 MFMA"),
}

__all__ = [
    "any_kernel_dim_ir", "softmax_inner_ir", "layer_norm_persistent_ir", "bias_gelu_axpy_ir",
    "matmul_bias_relu2d_ir", "gen_any_kernel_dim", "gen_softmax_inner", "gen_layer_norm", "gen_bias_gelu_axpy",
    "gen_matmul_bias_relu", "Workload", "WORKLOADS", "algorithmic_bytes",
]
