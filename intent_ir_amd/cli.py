"""JSON-in / JSON-out front door of the HIP lowering, for callers outside Python.

Same shape as the reference's C++ codegen tool (backends/cuda/cpp_codegen/
intentir_cuda_codegen.cpp:5876-5905, driven by backends/cuda/codegen/cpp_driver.py:212-232):

    python -m intent_ir_amd.cli --intent intent.json --bindings bindings.json

prints one JSON object: kernel_name, kernel_id (the C-ABI symbol), io_spec, launch,
output_names, bindings and call_args (the C argument list, element-wise programs
spelled out as instruction and operand tables).  Exit status 0 on success, 2 for
bad usage, 3 when the IR cannot be lowered or run (message on stderr), as the
reference tool does.

With ``--run inputs.npz --out outputs.npz`` the kernel is also launched on the
GPU (inputs by IR tensor name; bf16 as uint16 bit patterns or float values) and
the outputs are written, bf16 widened to float32.

``lower_from_json_str(intent_json, bindings_json) -> str`` is the in-process form,
like the reference's pybind ``lower_from_json_str`` (intentir_cuda_codegen.cpp:5858-5862).
"""

from __future__ import annotations

import argparse
import json
import sys
from typing import Any, Dict, List, Optional

from .ir import IntentIRValidationError
from .lowering import HipLoweredKernel, HipLoweringError, call_args_to_json, lower_intent_to_hip_kernel


def lowered_to_json(k: HipLoweredKernel) -> Dict[str, Any]:
    return {
        "kernel_name": k.kernel_name,
        "kernel_id": k.kernel_id,
        "io_spec": k.io_spec,
        "launch": {"grid": list(k.launch.grid), "block": list(k.launch.block), "lds_bytes": k.launch.lds_bytes},
        "output_names": list(k.output_names),
        "bindings": k.bindings,
        "call_args": call_args_to_json(k.call_args),
    }


def lower_from_json_str(intent_json: str, bindings_json: str) -> str:
    k = lower_intent_to_hip_kernel(json.loads(intent_json), shape_bindings=json.loads(bindings_json))
    return json.dumps(lowered_to_json(k))


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m intent_ir_amd.cli", description=__doc__.split("\n\n")[0])
    ap.add_argument("--intent", help="IntentIR JSON file")
    ap.add_argument("--bindings", "--shapes", dest="bindings", help="JSON object of shape bindings")
    ap.add_argument("--run", metavar="INPUTS_NPZ", help="also launch the kernel on these inputs (needs a GPU)")
    ap.add_argument("--out", metavar="OUTPUTS_NPZ", help="where --run writes the outputs")
    try:
        args = ap.parse_args(argv)
    except SystemExit as e:
        return 0 if e.code == 0 else 2
    if not args.intent or not args.bindings:
        print("missing --intent/--bindings (use --help)", file=sys.stderr)
        return 2
    if args.run and not args.out:
        print("--run needs --out", file=sys.stderr)
        return 2
    try:
        with open(args.intent) as f:
            intent = json.load(f)
        with open(args.bindings) as f:
            bindings = json.load(f)
        k = lower_intent_to_hip_kernel(intent, shape_bindings=bindings)
        print(json.dumps(lowered_to_json(k)))
        if args.run:
            import numpy as np  # noqa: PLC0415

            from .runtime import run_lowered  # noqa: PLC0415

            with np.load(args.run, allow_pickle=False) as z:
                inputs = {n: z[n] for n in z.files}
            out = run_lowered(k, inputs)
            np.savez(args.out, **{n: out[n] for n in k.output_names})
        return 0
    except (HipLoweringError, IntentIRValidationError, ValueError, KeyError, OSError, RuntimeError) as e:
        print(f"intent_ir_amd.cli error: {e}", file=sys.stderr)
        return 3


if __name__ == "__main__":
    sys.exit(main())
