"""Host-side dtype plumbing for IntentIR tensors.

numpy has no bfloat16, so bf16 tensors travel as ``uint16`` bit patterns and are
widened to float32 exactly (a bf16 value is the top half of a float32).  The
narrowing conversion is round-to-nearest-even, NaN kept quiet — the same rule
the device kernels apply when they store bf16.
"""

from __future__ import annotations

import numpy as np

# Bytes per element of each IntentIR dtype as stored in device memory.
ITEMSIZE = {"f16": 2, "bf16": 2, "f32": 4, "f64": 8, "i8": 1, "i16": 2, "u8": 1, "i1": 1,
            "bool": 1, "i32": 4, "i64": 8}

# numpy storage dtype used for each IntentIR dtype on the host.
STORAGE = {"f16": np.float16, "bf16": np.uint16, "f32": np.float32, "f64": np.float64, "i8": np.int8,
           "i16": np.int16, "u8": np.uint8, "i1": np.bool_, "bool": np.bool_, "i32": np.int32,
           "i64": np.int64}


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit pattern (uint16), round-to-nearest-even, NaN stays NaN."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    rounded = ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        rounded = rounded.copy()
        rounded[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x0040)).astype(np.uint16)
    return rounded


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bit pattern (uint16) -> float32 (exact)."""
    u = np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return u.view(np.float32)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16 value, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def to_storage(arr: np.ndarray, dtype: str) -> np.ndarray:
    """Host array -> the contiguous storage the device kernel reads for ``dtype``.

    bf16 accepts either uint16 bit patterns or real values (rounded RNE)."""
    a = np.asarray(arr)
    if dtype == "bf16":
        if a.dtype == np.uint16:
            return np.ascontiguousarray(a)
        return f32_to_bf16_bits(a.astype(np.float32))
    if dtype in ("bool", "i1"):
        return np.ascontiguousarray(a != 0, dtype=np.bool_) if a.dtype != np.bool_ else np.ascontiguousarray(a)
    return np.ascontiguousarray(a, dtype=STORAGE[dtype])


def to_compute_f32(arr: np.ndarray, dtype: str) -> np.ndarray:
    """Storage -> the float32 values the oracle computes on (exact widening)."""
    a = np.asarray(arr)
    if dtype == "bf16" and a.dtype == np.uint16:
        return bf16_bits_to_f32(a)
    if dtype in ("f16", "bf16", "f32"):
        return a.astype(np.float32)
    return a


__all__ = ["ITEMSIZE", "STORAGE", "f32_to_bf16_bits", "bf16_bits_to_f32", "round_to_bf16", "to_storage",
           "to_compute_f32"]
