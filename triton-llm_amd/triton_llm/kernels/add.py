"""Elementwise add on the HIP library: ``add(x_dev, y_dev, out_dev=None)``
with the reference's signature and asserts (triton_llm/kernels/add.py:54-104).
float32, float16 and bfloat16, fp32 arithmetic."""

from __future__ import annotations

import numpy as np

from triton_llm import gpu
from ._common import check_status, same_dtype, vp


def add(x_dev: "gpu.DeviceTensor", y_dev: "gpu.DeviceTensor",
        out_dev: "gpu.DeviceTensor | None" = None) -> "gpu.DeviceTensor":
    """GPU-resident element-wise addition. No sync, no host copies."""
    assert x_dev.shape == y_dev.shape, f"Shape mismatch: {x_dev.shape} vs {y_dev.shape}"
    if out_dev is not None:
        assert out_dev.shape == x_dev.shape, f"out_dev shape mismatch: expected {x_dev.shape}, got {out_dev.shape}"
    N = int(np.prod(x_dev.shape))
    if out_dev is None:
        out_dev = gpu.allocate(x_dev.shape, x_dev.dtype)
    if N == 0:
        return out_dev
    code = same_dtype(x_dev, y_dev, out_dev)
    check_status(gpu.runtime().tl_add(vp(x_dev), vp(y_dev), vp(out_dev), N, code, None), "add")
    return out_dev
