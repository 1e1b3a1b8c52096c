"""intent_ir_amd — MI355X (gfx950) execution backend for IntentIR.

Drop-in counterpart of the reference GPU backend (backends/cuda): IntentIR JSON
in, one precompiled gfx950 kernel call plus its launch plan out.

    from intent_ir_amd import lower_intent_to_hip_kernel, run_hip_kernel
    k = lower_intent_to_hip_kernel(intent, shape_bindings={"M": 8192, "N": 4096})
    out = run_hip_kernel(kernel_name=k.kernel_name, kernel_id=k.kernel_id, io_spec=k.io_spec,
                         launch=k.launch, bindings=k.bindings, inputs_np={...},
                         output_names=k.output_names, call_args=k.call_args)
"""

from .ir import IntentFunction, IntentIRValidationError, as_intent  # noqa: F401
from .lowering import HipLaunch, HipLoweredKernel, HipLoweringError, lower_intent_to_hip_kernel  # noqa: F401
from .macros import expand_macros  # noqa: F401
from .opset import HIP_SUPPORTED_OPS  # noqa: F401
from .runtime import (HipRuntimeError, launch_lowered, load_library, make_hip_ref_fn, run_hip_kernel,  # noqa: F401
                      run_lowered)

__all__ = [
    "HIP_SUPPORTED_OPS", "HipLaunch", "HipLoweredKernel", "HipLoweringError", "HipRuntimeError", "IntentFunction",
    "IntentIRValidationError", "as_intent", "expand_macros", "launch_lowered", "load_library", "make_hip_ref_fn",
    "lower_intent_to_hip_kernel", "run_hip_kernel", "run_lowered",
]
