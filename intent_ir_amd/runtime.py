"""ctypes runtime of the HIP backend: load libintentir_hip.so and launch kernels.

Mirrors the reference runtime entry ``run_cuda_kernel(*, kernel_name,
cuda_src, io_spec, launch, bindings, inputs_np, output_names, ...)``
(backends/cuda/runtime.py:22-45 -> frontends/cuda/runtime.py:926-1031):
allocate every tensor of ``io_spec``, copy the numpy inputs in, launch, wait,
and return inputs plus outputs as numpy arrays (the reference returns both,
frontends/cuda/runtime.py:1028-1031).  bf16 outputs come back as their exact
float32 widening (numpy has no bfloat16).

PyTorch-ROCm is used only for device memory and the current stream; every
kernel runs through the C-ABI.  There is no CPU fallback: without the built
library or a ROCm device, calls raise ``HipRuntimeError``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Any, Dict, Iterable, Mapping, Optional, Sequence, Tuple

import numpy as np

from .dtypes import bf16_bits_to_f32, to_storage
from .ir import resolve_dim

LIB_PATH = Path(__file__).resolve().parent / "libintentir_hip.so"


class HipRuntimeError(RuntimeError):
    """Library missing, no device, rejected arguments or a failed launch."""


_P, _I64, _I32, _F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

# Signatures of every entry point declared in include/intentir_hip.h.
SIGNATURES: Dict[str, Tuple[Any, Tuple[Any, ...]]] = {
    "ihip_abi_version": (ctypes.c_int, ()),
    "ihip_last_error": (ctypes.c_char_p, ()),
    "ihip_reduce_any_rows_f32": (_I32, (_P, _P, _I64, _I64, _F32, _P)),
    "ihip_reduce_any_rows_u8": (_I32, (_P, _P, _I64, _I64, _P)),
    "ihip_reduce_rows_f32": (_I32, (_P, _P, _I64, _I64, _I32, _P)),
    "ihip_reduce_rows_f32_workspace_size": (_I64, (_I64, _I64)),
    "ihip_reduce_rows_f32_ws": (_I32, (_P, _P, _I64, _I64, _I32, _P, _I64, _P)),
    "ihip_reduce_rows_f32_ex": (_I32, (_P, _P, _I64, _I64, _I32, _F32, _P, _I64, _P)),
    "ihip_reduce_rows_f32_noalloc": (_I32, (_P, _P, _I64, _I64, _I32, _P)),
    "ihip_softmax_rows_f32": (_I32, (_P, _P, _I64, _I64, _P)),
    "ihip_softmax_rows_f32_ex": (_I32, (_P, _P, _I64, _I64, _I32, _P)),
    "ihip_softmax_rows_f32_workspace_size": (_I64, (_I64, _I64)),
    "ihip_softmax_rows_f32_ws": (_I32, (_P, _P, _I64, _I64, _P, _I64, _P)),
    "ihip_softmax_rows_f32_stats": (_I32, (_P, _P, _P, _P, _I64, _I64, _P, _I64, _P)),
    "ihip_layernorm_rows_f16": (_I32, (_P, _P, _P, _P, _P, _P, _I64, _I64, _F32, _P)),
    "ihip_layernorm_rows_f32": (_I32, (_P, _P, _P, _P, _P, _P, _I64, _I64, _F32, _P)),
    "ihip_bias_gelu_tanh_axpy_bf16": (_I32, (_P, _P, _P, _I64, _I64, _F32, _P)),
    "ihip_gather2d_f32": (_I32, (_P, _P, _P, _P, _I64, _I64, _I64, _F32, _P)),
    "ihip_gemm_bf16_bias_relu": (_I32, (_P, _P, _P, _P, _I64, _I64, _I64, _I32, _P)),
    "ihip_gemm_bf16_bias_relu_t": (_I32, (_P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _P)),
    "ihip_gemm_bf16_bias_relu_ex": (_I32, (_P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P)),
    "ihip_gemm_f32_bias_relu": (_I32, (_P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P)),
    "ihip_gemm_workspace_size": (_I64, (_I64, _I64, _I64, _I32, _I32)),
    "ihip_gemm_bf16_bias_relu_ws": (_I32, (_P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P, _I64, _P)),
    "ihip_gemm_splitk_workspace_size": (_I64, (_I64, _I64, _I64, _I32)),
    "ihip_gemm_bf16_bias_relu_splitk": (_I32, (_P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P,
                                                _I64, _P)),
    "ihip_elementwise_program": (_I32, (_P, _I32, _P, _I32, _P, _I32, _P, _I32, _P)),
    "ihip_elementwise_mode": (_I32, (_I32,)),
    "ihip_elementwise_prepare": (_I32, (_P, _I32, _P, _I32, _P, _I32)),
    "ihip_elementwise_prepare_operands": (_I32, (_P, _I32, _P, _I32, _P, _I32, _P, _I32)),
    "ihip_elementwise_source": (_I32, (_P, _I32, _P, _I32, _P, _I32, _P, _I32, _P, _I64, _P)),
}
EW_MODE_AUTO, EW_MODE_INTERP, EW_MODE_NATIVE = 0, 1, 2


class EwInstr(ctypes.Structure):
    """ihip_ew_instr (include/intentir_hip.h)."""
    _fields_ = [("op", ctypes.c_uint8), ("dst", ctypes.c_uint8), ("a", ctypes.c_uint8), ("b", ctypes.c_uint8),
                ("c", ctypes.c_uint8), ("reserved", ctypes.c_uint8 * 3), ("imm", ctypes.c_float)]


class EwOperand(ctypes.Structure):
    """ihip_ew_operand (include/intentir_hip.h)."""
    _fields_ = [("ptr", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("stride", ctypes.c_int64 * 4)]


def elementwise_source(prog, ptrs: Mapping[str, int], dtypes: Mapping[str, str]) -> str:
    """The HIP source ihip_elementwise_program compiles for an EwProgram with operands at ``ptrs``
    (only their alignment matters; no device needed)."""
    lib = load_library()
    args = ew_program_args(prog, ptrs, dtypes)
    keep = args.pop()
    n = ctypes.c_int64(0)
    st = lib.ihip_elementwise_source(*args, None, 0, ctypes.byref(n))
    if st != 0:
        raise HipRuntimeError(f"ihip_elementwise_source failed (status {st}): {lib.ihip_last_error().decode()}")
    buf = ctypes.create_string_buffer(n.value + 1)
    st = lib.ihip_elementwise_source(*args, buf, n.value + 1, None)
    del keep
    if st != 0:
        raise HipRuntimeError(f"ihip_elementwise_source failed (status {st}): {lib.ihip_last_error().decode()}")
    return buf.value.decode()


def ew_program_args(prog, ptrs: Mapping[str, int], dtypes: Mapping[str, str]) -> list:
    """ctypes arguments of ihip_elementwise_program (minus the stream) for an EwProgram."""
    from .ewprogram import DTYPE_CODE  # noqa: PLC0415

    code = (EwInstr * len(prog.code))()
    for i, (op, d, a, b, c, imm) in enumerate(prog.code):
        code[i].op, code[i].dst, code[i].a, code[i].b, code[i].c, code[i].imm = op, d, a, b, c, imm
    ins = (EwOperand * max(1, len(prog.inputs)))()
    for i, (name, st) in enumerate(prog.inputs):
        ins[i].ptr, ins[i].dtype = ptrs[name], DTYPE_CODE[dtypes[name]]
        for j in range(4):
            ins[i].stride[j] = int(st[j])
    outs = (EwOperand * len(prog.outputs))()
    for i, name in enumerate(prog.outputs):
        outs[i].ptr, outs[i].dtype = ptrs[name], DTYPE_CODE[dtypes[name]]
    shape = (ctypes.c_int64 * max(1, len(prog.shape)))(*[int(d) for d in prog.shape])
    return [ctypes.cast(code, _P), _I32(len(prog.code)), ctypes.cast(ins, _P), _I32(len(prog.inputs)),
            ctypes.cast(outs, _P), _I32(len(prog.outputs)), ctypes.cast(shape, _P), _I32(len(prog.shape)),
            (code, ins, outs, shape)]


ABI_VERSION = 3

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def load_library(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load (once) the in-tree library and bind every signature; raise if absent."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise HipRuntimeError(f"{p} is not built: run __graft_entry__.build() or python -m intent_ir_amd.build")
        try:
            lib = ctypes.CDLL(str(p))
        except OSError as e:
            raise HipRuntimeError(f"cannot load {p}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, list(args)
        if lib.ihip_abi_version() != ABI_VERSION:
            raise HipRuntimeError(f"{p} has ABI {lib.ihip_abi_version()}, expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def call(name: str, *args: Any) -> None:
    """Call an entry point; raise HipRuntimeError with the library's message on failure."""
    lib = load_library()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.ihip_last_error().decode(errors="replace")
        raise HipRuntimeError(f"{name} failed (status {status}): {msg}")


# ---------------------------------------------------------------- torch plumbing
def _torch():
    try:
        import torch  # noqa: PLC0415
    except ImportError as e:  # pragma: no cover - torch is part of the image
        raise HipRuntimeError("PyTorch-ROCm is required for device memory") from e
    if not torch.cuda.is_available():
        raise HipRuntimeError("no ROCm device is visible")
    return torch


def torch_dtype(dtype: str):
    import torch  # noqa: PLC0415
    return {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32, "f64": torch.float64,
            "i8": torch.int8, "i16": torch.int16, "u8": torch.uint8, "bool": torch.bool, "i1": torch.bool,
            "i32": torch.int32, "i64": torch.int64}[dtype]


def to_device(arr: np.ndarray, dtype: str, device: str = "cuda"):
    """numpy -> device tensor in the storage the kernel reads (bf16 from uint16 bits or values)."""
    torch = _torch()
    st = to_storage(arr, dtype)
    if dtype == "bf16":
        return torch.from_numpy(st.view(np.int16)).to(device).view(torch.bfloat16)
    return torch.from_numpy(st).to(device)


def to_host(t, dtype: str) -> np.ndarray:
    """device tensor -> numpy (bf16 widened exactly to float32)."""
    torch = _torch()
    if dtype == "bf16":
        return bf16_bits_to_f32(t.detach().view(torch.int16).cpu().numpy().view(np.uint16))
    return t.detach().cpu().numpy()


def _check_buffer(name: str, t, dtype: str, shape: Sequence[int]) -> None:
    """Host-side guard: the buffer must be exactly what the kernel will index."""
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise HipRuntimeError(f"{name}: expected a torch tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise HipRuntimeError(f"{name}: tensor is on {t.device}, not a ROCm device")
    if t.dtype != torch_dtype(dtype):
        raise HipRuntimeError(f"{name}: dtype {t.dtype} but the IR declares {dtype}")
    if tuple(t.shape) != tuple(shape) and t.numel() != int(np.prod(shape, dtype=np.int64)):
        raise HipRuntimeError(f"{name}: shape {tuple(t.shape)} but the IR binds {tuple(shape)}")
    if not t.is_contiguous():
        raise HipRuntimeError(f"{name}: tensor must be contiguous")


def _ctype_args(call_args: Iterable[Tuple[str, Any]], buffers: Mapping[str, Any], keep: list,
                dtypes: Optional[Mapping[str, str]] = None, stream=None):
    """ctypes arguments of a lowered call.  A workspace is a fresh torch allocation marked as used
    by ``stream`` (record_stream), so the caching allocator does not hand it out again before the
    kernels reading it have run: no host synchronisation is needed."""
    out = []
    for kind, v in call_args:
        if kind == "ew_program":
            args = ew_program_args(v, {n: buffers[n].data_ptr() for n in buffers}, dtypes or {})
            keep.append(args.pop())  # keep the ctypes arrays alive through the call
            out.extend(args)
        elif kind == "tensor":
            out.append(_P(buffers[v].data_ptr()))
        elif kind == "i64":
            out.append(_I64(int(v)))
        elif kind == "i32":
            out.append(_I32(int(v)))
        elif kind == "f32":
            out.append(_F32(float(v)))
        elif kind == "null":
            out.append(_P(None))
        elif kind == "workspace":
            torch = _torch()
            t = torch.empty(max(1, int(v)), dtype=torch.uint8, device="cuda")
            if stream is not None:
                t.record_stream(stream)
            keep.append(t)
            out.extend([_P(t.data_ptr()), _I64(int(v))])
        else:
            raise HipRuntimeError(f"unknown call argument kind {kind}")
    return out


def tensor_shapes(io_spec: Mapping[str, Any], bindings: Mapping[str, Any]) -> Dict[str, Tuple[int, ...]]:
    return {n: tuple(resolve_dim(d, bindings) for d in spec["shape"]) for n, spec in io_spec["tensors"].items()}


def launch_lowered(lowered, buffers: Mapping[str, Any], stream=None) -> None:
    """Launch a lowered kernel on device-resident torch tensors (no copies, no sync).

    ``buffers`` maps every tensor of ``lowered.io_spec`` to a contiguous device
    tensor of the declared dtype and bound shape; ``stream`` is a torch stream or
    None for torch's current stream."""
    torch = _torch()
    shapes = tensor_shapes(lowered.io_spec, lowered.bindings)
    for n, spec in lowered.io_spec["tensors"].items():
        if n not in buffers:
            raise HipRuntimeError(f"missing buffer for {n}")
        _check_buffer(n, buffers[n], spec["dtype"], shapes[n])
    s = stream if stream is not None else torch.cuda.current_stream()
    keep: list = []  # host-side ctypes arrays of an element-wise program (copied at launch)
    dtypes = {n: spec["dtype"] for n, spec in lowered.io_spec["tensors"].items()}
    args = _ctype_args(lowered.call_args, buffers, keep, dtypes, s)
    call(lowered.kernel_id, *args, _P(s.cuda_stream))


def run_hip_kernel(*, kernel_name: str, kernel_id: str, io_spec: Mapping[str, Any], launch: Any,
                   bindings: Mapping[str, Any], inputs_np: Mapping[str, np.ndarray], output_names: Iterable[str],
                   call_args: Optional[Sequence[Tuple[str, Any]]] = None) -> Dict[str, np.ndarray]:
    """Allocate, copy inputs, launch, synchronise, and return inputs + outputs as numpy.

    Called like the reference's ``run_cuda_kernel`` (its ``cuda_src`` replaced by
    ``kernel_id``).  The argument plan comes from ``io_spec["hip_call"]``, which the
    lowering writes; ``call_args`` (``HipLoweredKernel.call_args``) overrides it."""
    torch = _torch()
    if call_args is None:
        if "hip_call" not in io_spec:
            raise HipRuntimeError(f"io_spec of {kernel_name} carries no hip_call plan and no call_args were given")
        from .lowering import call_args_from_json  # noqa: PLC0415

        call_args = call_args_from_json(io_spec["hip_call"])
    shapes = tensor_shapes(io_spec, bindings)
    outs = list(output_names)
    buffers: Dict[str, Any] = {}
    for n, spec in io_spec["tensors"].items():
        dt = spec["dtype"]
        if n in inputs_np:
            arr = np.asarray(inputs_np[n])
            if arr.size != int(np.prod(shapes[n], dtype=np.int64)):
                raise HipRuntimeError(f"input {n} has shape {arr.shape}, the IR binds {shapes[n]}")
            buffers[n] = to_device(arr.reshape(shapes[n]), dt)
        elif n in outs:
            buffers[n] = torch.empty(shapes[n], dtype=torch_dtype(dt), device="cuda")
        else:
            raise HipRuntimeError(f"missing input {n} for kernel {kernel_name}")

    class _L:  # the lowered-kernel fields launch_lowered reads
        pass

    lk = _L()
    lk.io_spec, lk.bindings, lk.call_args, lk.kernel_id = io_spec, bindings, tuple(call_args), kernel_id
    launch_lowered(lk, buffers)
    torch.cuda.synchronize()
    result: Dict[str, np.ndarray] = {n: np.asarray(v) for n, v in inputs_np.items()}
    for n in outs:
        result[n] = to_host(buffers[n], io_spec["tensors"][n]["dtype"]).reshape(shapes[n])
    return result


def make_hip_ref_fn(intent, make_inputs):
    """``run_ref_fn`` for the reference's ``run_diff(intent, run_ref_fn, cases)``
    (verify/diff_runner.py:37-44): per case, lower ``intent`` for ``case.shapes``, run it
    through the C-ABI on ``case.inputs`` (or ``make_inputs(case)``) and return every
    external input and every output under its IR name, 16-bit floats widened to float32
    so the interpreter computes in float32 (inputs are exact widenings of what the
    kernel read)."""
    from .dtypes import to_compute_f32  # noqa: PLC0415
    from .ir import as_intent  # noqa: PLC0415
    from .lowering import lower_intent_to_hip_kernel  # noqa: PLC0415

    fn = as_intent(intent)

    def run_ref_fn(case):
        k = lower_intent_to_hip_kernel(intent, shape_bindings=dict(case.shapes))
        inputs = dict(case.inputs) if case.inputs else make_inputs(case)
        out = run_lowered(k, inputs)
        return {n: (to_compute_f32(v, fn.tensors[n].dtype) if n in fn.tensors else v) for n, v in out.items()}

    return run_ref_fn


def run_lowered(lowered, inputs_np: Mapping[str, np.ndarray]) -> Dict[str, np.ndarray]:
    return run_hip_kernel(kernel_name=lowered.kernel_name, kernel_id=lowered.kernel_id, io_spec=lowered.io_spec,
                          launch=lowered.launch, bindings=lowered.bindings, inputs_np=inputs_np,
                          output_names=lowered.output_names, call_args=lowered.call_args)


__all__ = ["HipRuntimeError", "SIGNATURES", "EwInstr", "EwOperand", "elementwise_source", "ew_program_args", "make_hip_ref_fn", "LIB_PATH", "load_library", "call", "launch_lowered", "run_hip_kernel",
           "run_lowered", "to_device", "to_host", "torch_dtype", "tensor_shapes"]
