"""RMSNorm (and the fused residual add + RMSNorm) on the HIP library.

``rms_norm(x_dev, w_dev, out_dev, eps)`` keeps the reference's signature,
asserts and errors (triton_llm/kernels/rms_norm.py:68-116): x ``(M, N)``, w
``(N,)``, out ``(M, N)``; ``M == 0`` returns at once, ``N == 0`` raises
``ValueError``.  ``add_rms_norm`` is additive: ``h = a + b`` (written to
``h_dev``) and ``out = rms_norm(h)`` in one pass, the model's residual add
followed by the next norm (smollm2_triton/model.py:352-357).  float32, float16
and bfloat16, fp32 arithmetic.
"""

from __future__ import annotations

from triton_llm import gpu
from ._common import check_status, same_dtype, vp


def rms_norm(x_dev: "gpu.DeviceTensor", w_dev: "gpu.DeviceTensor", out_dev: "gpu.DeviceTensor",
             eps: float = 1e-5) -> "gpu.DeviceTensor":
    """GPU-resident RMSNorm. No sync, no host copies."""
    M, N = x_dev.shape
    assert w_dev.shape == (N,), f"w_dev shape mismatch: expected ({N},), got {w_dev.shape}"
    assert out_dev.shape == (M, N), f"out_dev shape mismatch: expected ({M},{N}), got {out_dev.shape}"
    if M == 0:
        return out_dev
    if N == 0:
        raise ValueError("RMSNorm requires the last dimension N > 0")
    code = same_dtype(x_dev, w_dev, out_dev)
    check_status(gpu.runtime().tl_rms_norm(vp(x_dev), vp(w_dev), vp(out_dev), M, N, float(eps), code, None),
                 "rms_norm")
    return out_dev


def add_rms_norm(a_dev, b_dev, h_dev, w_dev, out_dev, eps: float = 1e-5):
    """``h = a + b`` and ``out = rms_norm(h, w)`` in one pass; returns (h, out)."""
    M, N = a_dev.shape
    assert b_dev.shape == (M, N) and h_dev.shape == (M, N), f"shape mismatch: {a_dev.shape}, {b_dev.shape}, {h_dev.shape}"
    assert w_dev.shape == (N,), f"w_dev shape mismatch: expected ({N},), got {w_dev.shape}"
    assert out_dev.shape == (M, N), f"out_dev shape mismatch: expected ({M},{N}), got {out_dev.shape}"
    if M == 0:
        return h_dev, out_dev
    if N == 0:
        raise ValueError("RMSNorm requires the last dimension N > 0")
    code = same_dtype(a_dev, b_dev, h_dev, w_dev, out_dev)
    check_status(gpu.runtime().tl_add_rms_norm(vp(a_dev), vp(b_dev), vp(h_dev), vp(w_dev), vp(out_dev), M, N,
                                               float(eps), code, None), "add_rms_norm")
    return h_dev, out_dev
