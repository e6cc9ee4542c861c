"""GEMM restatement (test infrastructure only).

* :func:`gemm_ref` -- triton_llm/kernels/gemm.py:53-108: C = A @ B for
  row-major A (M, K), B (K, N); the reference kernel accumulates in fp32
  over 32-wide K blocks (:39-46).  Here the sum is taken in float64 and
  rounded once, so it is the exact product up to one rounding, and the GPU
  result is compared against it within a tolerance that scales with K.

Pinned in tests/test_oracle.py by the identity, a rank-one product and
associativity against a vector, which a transposed operand or a dropped
term would fail.
"""

from __future__ import annotations

import numpy as np


def gemm_ref(a, b) -> np.ndarray:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    assert a.ndim == 2 and b.ndim == 2 and a.shape[1] == b.shape[0], (a.shape, b.shape)
    if a.shape[1] == 0:
        return np.zeros((a.shape[0], b.shape[1]), np.float32)
    return (a @ b).astype(np.float32)
