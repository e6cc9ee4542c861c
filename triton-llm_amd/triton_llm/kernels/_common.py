"""Shared host-side helpers for the kernel wrappers (no GPU work on import)."""

from __future__ import annotations

import ctypes
import math

import numpy as np

from triton_llm import gpu
from triton_llm import _lib

LOG2E = 1.4426950408889634


def contiguous_strides(shape) -> tuple[int, ...]:
    """Element strides of a C-contiguous array of ``shape``."""
    out = []
    acc = 1
    for s in reversed(shape):
        out.append(acc)
        acc *= int(s)
    return tuple(reversed(out))


def check_status(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"GPU runtime error (hip): {status} ({_lib.error_string(status)}) in {what}")


def same_dtype(*tensors) -> int:
    """Dtype code shared by all tensors; ValueError if they differ."""
    names = {gpu.dtype_name(t.dtype) for t in tensors}
    if len(names) != 1:
        raise ValueError(f"inputs must share one dtype, got {sorted(names)}")
    return gpu.dtype_code(tensors[0].dtype)


def is_pow2(n: int) -> bool:
    return n > 0 and (n & (n - 1)) == 0


def default_scale(d_k: int) -> float:
    return 1.0 / math.sqrt(d_k)


def vp(t) -> ctypes.c_void_p:
    """Raw pointer argument of a DeviceTensor (NULL for None)."""
    if t is None:
        return ctypes.c_void_p(None)
    return t.ptr if isinstance(t.ptr, ctypes.c_void_p) else ctypes.c_void_p(t.ptr)


def scratch(nbytes: int, workspace=None):
    """Return a workspace of at least ``nbytes`` (the caller's if big enough)."""
    if nbytes == 0:
        return None
    if workspace is not None:
        if workspace.nbytes < nbytes:
            raise ValueError(f"workspace holds {workspace.nbytes} bytes, {nbytes} required")
        return workspace
    return gpu.allocate((nbytes,), np.uint8)
