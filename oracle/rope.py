"""RoPE restatement (test infrastructure only).

Follows triton_llm/kernels/rope.py of the reference:
  * table construction op for op (rope.py:110-123), float32 throughout;
  * half-split pairing (i, i + d/2) (rope.py:51-66) and the row position
    rule pos = row % seq_len + offset (rope.py:49);
  * each product and the sum/difference rounded separately in float32, as
    NumPy evaluates ``x_e * c - x_o * s``.
"""

from __future__ import annotations

import numpy as np

from .numerics import from_storage, round_to, to_storage


def precompute_cos_sin(max_seq_len: int, d_k: int, theta: float = 100000.0):
    """rope.py:73-123 -- half-packed (max_seq_len, d_k // 2) float32 tables."""
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
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


def rotate(x, cos_rows, sin_rows):
    """Rotate rows of x (..., d) by per-row cos/sin (..., d/2), float32."""
    x = np.asarray(x, dtype=np.float32)
    half = x.shape[-1] // 2
    xe = x[..., :half]
    xo = x[..., half:]
    c = np.asarray(cos_rows, dtype=np.float32)
    s = np.asarray(sin_rows, dtype=np.float32)
    out = np.empty_like(x)
    out[..., :half] = xe * c - xo * s
    out[..., half:] = xe * s + xo * c
    return out


def apply_rope(x, cos, sin, seq_len: int, position_offset: int = 0):
    """rope.py:25-70 on a 2-D float32 (n_rows, d_k) array; returns a new array."""
    x = np.asarray(x, dtype=np.float32)
    n_rows = x.shape[0]
    pos = (np.arange(n_rows) % seq_len) + position_offset
    return rotate(x, cos[pos], sin[pos])


def apply_rope_storage(x_storage, cos, sin, positions, dtype: str):
    """RoPE on storage-typed rows (..., d) at ``positions`` (broadcast over rows),
    rotated in float32 and rounded once to ``dtype`` -- what the HIP kernels store."""
    xf = from_storage(x_storage, dtype)
    out = rotate(xf, cos[positions], sin[positions])
    return to_storage(round_to(out, dtype), dtype)
