"""Op-name vocabulary of IntentIR and the subset the HIP backend lowers.

The op names are the IR's interface, so the CORE/EXPERIMENTAL/MACRO tiers keep
the reference's names (``intent_ir/ops/opset.py:19-78``).  ``gelu_tanh`` is a
macro op added by this backend's macro registry (``intent_ir_amd/macros.py``):
the reference has no GELU op, and its macro registry
(``intent_ir/macros/macro_lowering/registry.py:12-24``) is the extension point
it is registered through.

``HIP_SUPPORTED_OPS`` plays the role of ``CUDA_SUPPORTED_OPS``
(``backends/cuda/opset.py:10-31``): every op that may appear in an IR the HIP
lowering accepts (after macro expansion).
"""

from __future__ import annotations

CORE_OPS: frozenset = frozenset({
    "matmul", "softmax", "dropout", "correlation", "resize", "warp", "rope",
    "add", "sub", "mul", "div", "max", "min", "ne", "lt", "le", "gt", "ge", "and", "or", "not",
    "exp", "relu", "rsqrt", "abs", "floor", "cast", "where",
    "iota", "gather", "identity", "const", "reduce_sum", "reduce_any", "reduce_max",
    "broadcast_in_dim", "transpose", "reshape", "layout_cast",
})

EXPERIMENTAL_OPS: frozenset = frozenset({"conv2d"})

MACRO_OPS: frozenset = frozenset({"upsample_bicubic2d_aa", "gelu_tanh"})

SUPPORTED_OPS: frozenset = CORE_OPS | EXPERIMENTAL_OPS | MACRO_OPS

# Shape-only ops: no arithmetic, the backend folds them into index maps.
VIEW_OPS: frozenset = frozenset({"identity", "reshape", "layout_cast", "broadcast_in_dim", "transpose"})

# Element-wise ops the fused chain kernels evaluate.
ELEMENTWISE_OPS: frozenset = frozenset({
    "const", "add", "sub", "mul", "div", "max", "min", "exp", "relu", "rsqrt", "abs", "floor",
    "ne", "lt", "le", "gt", "ge", "and", "or", "not", "where", "cast", "iota",
}) | VIEW_OPS

HIP_SUPPORTED_OPS: frozenset = ELEMENTWISE_OPS | frozenset({
    "reduce_sum", "reduce_max", "reduce_any", "softmax", "matmul", "gather",
})

__all__ = ["CORE_OPS", "EXPERIMENTAL_OPS", "MACRO_OPS", "SUPPORTED_OPS", "VIEW_OPS", "ELEMENTWISE_OPS",
           "HIP_SUPPORTED_OPS"]
