"""
Fused (optionally causal) self-attention for one head, host arrays in/out.

Same entry point, arguments, assertions and return type as the reference's
``attention`` (triton_llm/kernels/attention.py:141-216 of
ziliangpeng/triton-llm):

    attention(Q, K, V) = softmax(Q @ K^T / sqrt(d_k)) @ V

causal=True masks key j > i (top-left; requires seq_q == seq_k), causal=False
applies no mask and allows seq_q != seq_k (single-query decode against a
cache, as gpt2_triton/model.py:346-348 calls it).  Inputs are upcast to
C-contiguous float32 and the result is a float32 NumPy array; the call
synchronises, like the reference (attention.py:215-216).

The work runs on the gfx950 HIP library: seq_q == 1 with d_k in (64, 128)
uses the split-K decode kernel, everything else the flash kernel.
"""

from __future__ import annotations

import numpy as np

from triton_llm import gpu
from .attention_gqa import attention_gqa


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool = True) -> np.ndarray:
    """O = softmax(Q @ K^T / sqrt(d_k)) @ V for 2-D float32 Q (seq_q, d_k), K/V (seq_k, d_k)."""
    assert q.ndim == 2 and k.ndim == 2 and v.ndim == 2
    d_k = q.shape[1]
    seq_q = q.shape[0]
    seq_k = k.shape[0]
    assert k.shape == (seq_k, d_k), f"K shape {k.shape} != {({seq_k}, {d_k})}"
    assert v.shape == (seq_k, d_k), f"V shape {v.shape} != {({seq_k}, {d_k})}"
    if not causal:
        assert q.shape[1] == k.shape[1] == d_k, \
            f"d_k mismatch: q={q.shape[1]}, k={k.shape[1]}, v={v.shape[1]}"
    else:
        assert seq_q == seq_k, \
            f"causal requires seq_q == seq_k, got {seq_q} vs {seq_k}"
    assert d_k > 0 and (d_k & (d_k - 1)) == 0, \
        f"d_k ({d_k}) must be a positive power of 2"

    if seq_q == 0 or seq_k == 0:
        return np.empty((seq_q, d_k), dtype=np.float32)

    q = np.require(q, dtype=np.float32, requirements=["C_CONTIGUOUS"])
    k = np.require(k, dtype=np.float32, requirements=["C_CONTIGUOUS"])
    v = np.require(v, dtype=np.float32, requirements=["C_CONTIGUOUS"])

    q_dev = gpu.to_device(q)
    k_dev = gpu.to_device(k)
    v_dev = gpu.to_device(v)
    # One head: the GQA entry with n_head = n_kv_head = 1.  With seq_q == seq_k
    # its bottom-right causal mask is the reference's top-left mask.
    o_dev = attention_gqa(q_dev, k_dev, v_dev, 1, 1, causal=causal)
    gpu.synchronize()
    return gpu.to_host(o_dev)
