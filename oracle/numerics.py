"""Storage-type conversions for the oracle (NumPy has no bfloat16 here).

bfloat16 values are carried as raw uint16 bit patterns.  Rounding from
float32 is round-to-nearest-even on the bit pattern; NaN becomes the quiet
NaN 0x7FC0 with the input's sign.
"""

from __future__ import annotations

import numpy as np

DTYPES = ("float32", "float16", "bfloat16")


def f32_to_bf16_bits(x) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    bias = np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    out = ((u + bias) >> np.uint32(16)).astype(np.uint16)
    if nan.any():
        out[nan] = (((u[nan] >> np.uint32(16)) & np.uint32(0x8000)) | np.uint32(0x7FC0)).astype(np.uint16)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    """Round float values to ``dtype`` and return them as float32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "float32":
        return x.copy()
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    raise ValueError(dtype)


def to_storage(x, dtype: str) -> np.ndarray:
    """float values -> storage array (float32, float16, or uint16 bf16 bits)."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "float32":
        return np.ascontiguousarray(x)
    if dtype == "float16":
        return x.astype(np.float16)
    if dtype == "bfloat16":
        return f32_to_bf16_bits(x)
    raise ValueError(dtype)


def from_storage(a, dtype: str) -> np.ndarray:
    """storage array -> float32 values."""
    if dtype == "float32":
        return np.asarray(a, dtype=np.float32)
    if dtype == "float16":
        return np.asarray(a, dtype=np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return bf16_bits_to_f32(a)
    raise ValueError(dtype)


def nan_storage(dtype: str):
    """The storage value used to poison never-read cache positions."""
    if dtype == "float32":
        return np.float32(np.nan)
    if dtype == "float16":
        return np.float16(np.nan)
    return np.uint16(0x7FC0)


def storage_dtype(dtype: str):
    return {"float32": np.float32, "float16": np.float16, "bfloat16": np.uint16}[dtype]
