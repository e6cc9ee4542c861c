"""
RoPE (rotary position embedding) on the gfx950 HIP library.

Same entry points, arguments, validation order and error types as the
reference (triton_llm/kernels/rope.py of ziliangpeng/triton-llm):
``precompute_cos_sin`` (:73-123), ``precompute_cos_sin_device`` (:126-150),
``apply_rope`` (:153-222).  Pairing is the half-split one the reference code
uses (element i with i + d_k/2, rope.py:51-66); the position of row r is
``r % seq_len + position_offset`` (rope.py:49).

``apply_rope`` runs ``tl_rope_inplace``: fp32 rotation with separately
rounded products and sums, so fp32 results equal NumPy's bit for bit; 16-bit
inputs (float16 / gpu.bfloat16) are rotated in fp32 and rounded once.
"""

from __future__ import annotations

import numpy as np

from triton_llm import gpu
from triton_llm import _lib
from ._common import launch, check_status, vp


def precompute_cos_sin(
    max_seq_len: int,
    d_k: int,
    theta: float = 100000.0,
) -> tuple[np.ndarray, np.ndarray]:
    """Half-packed cos/sin tables, each ``(max_seq_len, d_k // 2)`` float32.

    ``cos[p, i] = cos(p * theta ** (-2 i / d_k))``, evaluated with the same
    float32 NumPy operations as the reference (rope.py:110-123), so the tables
    are identical to the reference's on the same host.
    """
    if max_seq_len < 1:
        raise ValueError(f"max_seq_len must be >= 1, got {max_seq_len}")
    if d_k < 2 or d_k % 2 != 0:
        raise ValueError(f"d_k must be even and >= 2, got {d_k}")
    if theta <= 0:
        raise ValueError(f"theta must be > 0, got {theta}")

    half = d_k // 2
    positions = np.arange(max_seq_len, dtype=np.float32)
    indices = np.arange(half, dtype=np.float32)
    freqs = 1.0 / (theta ** (2 * indices / d_k))
    angles = np.outer(positions, freqs)
    cos = np.cos(angles).astype(np.float32)
    sin = np.sin(angles).astype(np.float32)
    return cos, sin


def precompute_cos_sin_device(
    max_seq_len: int,
    d_k: int,
    theta: float = 100000.0,
) -> tuple["gpu.DeviceTensor", "gpu.DeviceTensor"]:
    """``precompute_cos_sin`` uploaded to the GPU (float32)."""
    cos_np, sin_np = precompute_cos_sin(max_seq_len, d_k, theta)
    return gpu.to_device(cos_np), gpu.to_device(sin_np)


def apply_rope(
    x_dev: "gpu.DeviceTensor",
    cos_dev: "gpu.DeviceTensor",
    sin_dev: "gpu.DeviceTensor",
    seq_len: int,
    position_offset: int = 0,
) -> "gpu.DeviceTensor":
    """GPU-resident RoPE, in place on ``x_dev`` (n_rows, d_k). No sync.

    Validation mirrors rope.py:179-203 (ValueError for each case, same order).
    """
    if len(x_dev.shape) != 2:
        raise ValueError(f"x_dev must be 2D (n_rows, d_k), got shape {x_dev.shape}")
    n_rows, d_k = x_dev.shape
    if d_k < 2 or d_k % 2 != 0:
        raise ValueError(f"d_k must be even and >= 2, got {d_k}")
    half = d_k // 2
    if len(cos_dev.shape) != 2 or len(sin_dev.shape) != 2:
        raise ValueError("cos_dev and sin_dev must be 2D tensors")
    if cos_dev.shape != sin_dev.shape:
        raise ValueError(f"cos_dev and sin_dev shape mismatch: {cos_dev.shape} vs {sin_dev.shape}")
    if cos_dev.shape[1] != half:
        raise ValueError(f"cos_dev last dim must be d_k // 2 ({half}), got {cos_dev.shape[1]}")
    if n_rows == 0:
        return x_dev
    if seq_len < 1:
        raise ValueError(f"seq_len must be >= 1, got {seq_len}")
    if position_offset < 0:
        raise ValueError(f"position_offset must be >= 0, got {position_offset}")
    if position_offset + seq_len > cos_dev.shape[0]:
        raise ValueError(
            f"position_offset ({position_offset}) + seq_len ({seq_len}) "
            f"exceeds cos/sin table size ({cos_dev.shape[0]})"
        )
    if n_rows % seq_len != 0:
        raise ValueError(
            f"Total rows ({n_rows}) must be a multiple of seq_len ({seq_len})"
        )
    if gpu.dtype_name(cos_dev.dtype) != "float32" or gpu.dtype_name(sin_dev.dtype) != "float32":
        raise ValueError("cos_dev and sin_dev must be float32 tables")
    code = gpu.dtype_code(x_dev.dtype)

    lib = gpu.runtime()
    launch(lib.tl_rope_inplace, vp(x_dev), vp(cos_dev), vp(sin_dev),
        n_rows, d_k, d_k, seq_len, position_offset, code, None,
        what="apply_rope")
    return x_dev
