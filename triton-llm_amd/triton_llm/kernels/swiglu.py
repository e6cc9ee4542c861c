"""SwiGLU on the HIP library: ``swiglu(gate_dev, up_dev, out_dev=None)`` with
the reference's signature, errors and stable sigmoid
(triton_llm/kernels/swiglu.py:21-125): ``silu(gate) * up`` elementwise,
``ValueError`` on mismatched shapes, empty input returns an (allocated)
output.  float32, float16 and bfloat16, fp32 arithmetic."""

from __future__ import annotations

import numpy as np

from triton_llm import gpu
from ._common import check_status, same_dtype, vp


def swiglu(gate_dev: "gpu.DeviceTensor", up_dev: "gpu.DeviceTensor",
           out_dev: "gpu.DeviceTensor | None" = None) -> "gpu.DeviceTensor":
    """GPU-resident SwiGLU activation. No sync, no host copies."""
    if gate_dev.shape != up_dev.shape:
        raise ValueError(f"gate_dev shape {gate_dev.shape} does not match up_dev shape {up_dev.shape}")
    N = int(np.prod(gate_dev.shape))
    if out_dev is not None:
        assert out_dev.shape == gate_dev.shape, f"out_dev shape mismatch: expected {gate_dev.shape}, got {out_dev.shape}"
    if out_dev is None:
        out_dev = gpu.allocate(gate_dev.shape, gate_dev.dtype)
    if N == 0:
        return out_dev
    code = same_dtype(gate_dev, up_dev, out_dev)
    check_status(gpu.runtime().tl_swiglu(vp(gate_dev), vp(up_dev), vp(out_dev), N, code, None), "swiglu")
    return out_dev
